"""CPU oracle (test infrastructure, not product code).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, always as the checker or the CPU baseline, never as a path that
produces operator results.
"""
