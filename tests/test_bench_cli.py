"""CPU checks of bench.py's driver contract that need no GPU: more than one GPU
is refused with a message (this build measures one), the traffic figure the
roofline object carries is read from the committed rocprof counter summary,
and the headline line, built by the same code from a full-size synthetic ops
block, stays short enough to survive a reader that keeps the last 8 KB of
stdout, and parses."""

from __future__ import annotations

import importlib.util
import json
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "fused-decode_amd"))


def _bench_module():
    spec = importlib.util.spec_from_file_location("bench_main", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120, cwd=ROOT)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert line["n_gpus"] == 2 and "one GPU" in line["error"]


def test_bench_reads_the_committed_traffic_figure():
    traffic = _bench_module().pmc_traffic()
    # the fused gate/up at M=1 moves its 234,926,080 algorithmic bytes within 1%
    assert traffic is not None and abs(traffic / 234_926_080 - 1.0) < 0.01


def _synthetic_rows():
    """One row per ops-block configuration, every figure at its longest form."""
    from fused_decode import bench as B

    rows = []
    for op, shape, dt, kind in B.ops_configs():
        extra = {"same_size_kind": "read", "same_size_us": 1234.5678}
        if kind is not None:
            extra.update(kind=kind, hipblaslt_dev_us=1234.56789)
        rows.append(B._compact(op, shape, dt, 123_456_789_012, 1234.56789, 1234.56789, 6543.21, 0.012345678901,
                               **extra))
    return rows


def test_ops_configs_cover_every_benchmark_config():
    from fused_decode import bench as B

    cfg = B.ops_configs()
    gemv = [c for c in cfg if c[0] == "linear_decode"]
    # 4 weight shapes x M in {1,2,4,8,16} x kinds {dot, simt} x dtypes {fp16, bf16}
    assert len(gemv) == 4 * 5 * 2 * 2
    assert {(c[2], c[3]) for c in gemv} == {(d, k) for d in B.OPS_DTYPES for k in ("dot", "simt")}
    assert sum(c[0] == "swiglu" for c in cfg) == 4 and sum(c[0] == "rope" for c in cfg) == 4
    assert sum(c[0] in ("rms_norm", "add_rms_norm") for c in cfg) == 4


def test_headline_line_fits_and_parses():
    mod = _bench_module()
    rows = _synthetic_rows()
    mlp = {dt: {m: {"eager_us": 12345.678, "graph_us": 12345.678, "graph_per_call_us": 12345.678}
                for m in (1, 8)} for dt in ("f16", "bf16")}
    decode = {"workload": "x" * 260}
    for m in (1, 8):
        for key in (f"m{m}", f"m{m}_unfused", f"m{m}_fp8"):
            decode.update({f"{key}_us": 12345.6, f"{key}_gbs": 12345.6, f"{key}_launches": 7,
                           f"{key}_states": [12345.6, 30, 12345.6, 30]})
    cpu = {"value": 12345.6, "unit": "us", "cores": 128, "kind": "port", "sample": "s" * 200,
           "cpu_model": "m" * 60, "cpus_visible": 256, "torch_threads": 128}
    line = mod.headline(steps=200, warmup=20, kind="dot", mlp=mlp, gate_us=35.123456, roof=6543.21,
                        read_roof=6789.01, traffic=235_298_221, decode=decode, ops_rows=rows,
                        ops_path="gpurun_out/bench_ops.json", cpu=cpu)
    text = mod.render(line)
    assert "\n" not in text
    assert len(text.encode()) <= mod.LINE_LIMIT < 8000, len(text)
    back = json.loads(text)
    for key in ("metric", "value", "unit", "ms_per_step", "config", "roofline", "cpu_baseline", "ops", "mlp"):
        assert key in back
    assert back["config"]["workload"] and back["roofline"]["frac"] > 0
    # every GEMV (dtype, kind, shape) is summarised with one value per row count
    groups = [k for k in back["ops"] if k.startswith("gemv ")]
    assert len(groups) == 16 and all(len(back["ops"][k][0]) == 5 for k in groups)
    assert {"f16", "bf16"} <= set(back["mlp"]) and set(back["mlp"]["bf16"]) == {"m1", "m8"}
