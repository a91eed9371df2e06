"""CPU checks of bench.py's driver contract that need no GPU: more than one GPU
is refused with a message (this build measures one), and the traffic figure the
roofline object carries is read from the committed rocprof counter summary."""

from __future__ import annotations

import importlib.util
import json
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120, cwd=ROOT)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert line["n_gpus"] == 2 and "one GPU" in line["error"]


def test_bench_reads_the_committed_traffic_figure():
    spec = importlib.util.spec_from_file_location("bench_main", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    traffic = mod.pmc_traffic()
    # the fused gate/up at M=1 moves its 234,926,080 algorithmic bytes within 1%
    assert traffic is not None and abs(traffic / 234_926_080 - 1.0) < 0.01
