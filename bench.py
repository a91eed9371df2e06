#!/usr/bin/env python
"""Headline benchmark: Llama-3-8B post-attention MLP (post_attn_mlp) on one MI355X.

Workload: hidden [M, 4096], norm_w [4096], w_gate_up [28672, 4096],
w_down [4096, 14336], fp16, eps 1e-5, residual fused; M = 1 (the `value`) and
M = 8 (reported beside it). Weights are random-init with the configured
distributions (no checkpoints); four independent weight sets (1.41 GB) are
rotated so every step streams its 352 MB of weights from HBM, not from the
256 MB Infinity Cache.

A step is one post_attn_mlp call launched eagerly (the reference's method,
bench.py:42-56: back-to-back calls between events); W untimed warmup steps,
then exactly K timed steps between HIP events, bracketed by synchronisation.
`value` is microseconds per step at M=1 (lower is better). The same steps
replayed from a HIP graph holding 100 steps (`graph_us`), from one graph
per call (`graph_per_call_us`, the reference's _graph_time), and the 32-layer decode step
minus attention, graph-captured (`decode_step`: the fused form with
pre_attn_qkv, and the reference's operators composed), are reported beside it.

roofline: the dominant kernel, the fused RMSNorm + gate/up GEMV + SwiGLU
launch, timed alone with HIP events on the stream it is launched on;
achieved = its algorithmic bytes / its average duration.

mlp: the same post_attn_mlp timings in fp16 and bf16 at M = 1 and 8.

ops: every norm, SwiGLU, RoPE and decode-GEMV benchmark configuration (device
and eager microseconds, GB/s, % of the copy roof and of 8 TB/s, and the
largest deviation from the reference's float32 formulas), one full row each,
is written to --ops-out; the headline line carries a summary of them (device
microseconds, % of the copy roof and of the same-size roof kernel, max error)
and stays under LINE_LIMIT bytes, so a reader that keeps only the last 8 KB of
stdout still sees all of it.

cpu_baseline: the reference's eager formula of the same block
(src/fused_decode/bench.py:395-398: F.rms_norm, F.linear, F.silu, F.linear + residual)
run by PyTorch on the host CPU in fp16 at M=1, over a bounded sample of calls,
with the thread count and CPU model.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "fused-decode_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

H, I = 4096, 14336
EPS = 1e-5
N_SETS = 4
GRAPH_ROTATIONS = 25  # the graph_us graph holds 25 rotations of the 4 weight sets: 100 steps per launch
HBM_PEAK_GBS = 8000.0


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="bound on the CPU baseline sample")
    ap.add_argument("--no-decode-step", action="store_true", help="skip the 32-layer decode step")
    ap.add_argument("--no-ops", action="store_true", help="skip the per-op block")
    ap.add_argument("--ops-out", default="gpurun_out/bench_ops.json",
                    help="file for the full per-op rows (the headline line carries their summary)")
    return ap.parse_args()


def make_sets(torch, m: int, dtype, dev):
    g = torch.Generator(device=dev).manual_seed(1234)
    sets = []
    for _ in range(N_SETS):
        hidden = torch.randn(m, H, generator=g, device=dev, dtype=torch.float32).to(dtype)
        norm_w = (1 + 0.1 * torch.randn(H, generator=g, device=dev, dtype=torch.float32)).to(dtype)
        w_gu = (torch.randn(2 * I, H, generator=g, device=dev, dtype=torch.float32) * H ** -0.5).to(dtype)
        w_d = (torch.randn(H, I, generator=g, device=dev, dtype=torch.float32) * I ** -0.5).to(dtype)
        sets.append((hidden, norm_w, w_gu, w_d))
    return sets


def time_graph_steps(torch, fd, sets, steps: int, warmup: int, kind: str | None) -> tuple[float, float]:
    """Microseconds per step of the same rotation replayed from HIP graphs, two ways:
    one graph holding GRAPH_ROTATIONS rotations of the N_SETS steps (what a decode
    loop that captures its whole step does), and one graph per call (the
    reference's _graph_time, bench.py:451-472). Every hipGraphLaunch leaves the
    GPU idle for about 4 us before its first kernel (measured: one step per graph
    +4.2 us/step, four steps +0.4, twenty steps none), so the second pays that
    once per step."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for st in sets:
            fd.post_attn_mlp(*st, EPS, kind=kind)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    whole = torch.cuda.CUDAGraph()
    with torch.cuda.graph(whole):
        for st in sets * GRAPH_ROTATIONS:
            fd.post_attn_mlp(*st, EPS, kind=kind)
    per_call = []
    for st in sets:
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            fd.post_attn_mlp(*st, EPS, kind=kind)
        per_call.append(gr)

    def timed(run, n):
        for s in range(max(2, warmup // per_replay)):
            run(s)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for s in range(n):
            run(s)
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) * 1000.0

    per_replay = N_SETS * GRAPH_ROTATIONS
    reps = max(1, steps // per_replay)
    rotation_us = timed(lambda s: whole.replay(), reps) / (reps * per_replay)
    per_call_us = timed(lambda s: per_call[s % N_SETS].replay(), steps) / steps
    return rotation_us, per_call_us


def time_eager_steps(torch, fd, sets, steps: int, warmup: int, kind: str | None) -> float:
    for s in range(warmup):
        fd.post_attn_mlp(*sets[s % N_SETS], EPS, kind=kind)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for s in range(steps):
        fd.post_attn_mlp(*sets[s % N_SETS], EPS, kind=kind)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1000.0 / steps


def time_gate_up_kernel(torch, lib, sets, m: int, iters: int, kind_code: int) -> float:
    """Average duration (us) of the fused norm + gate/up + SwiGLU launch alone."""
    from fused_decode._lib import DTYPE_CODE, check

    mids = [torch.empty(m, I, device=sets[0][0].device, dtype=sets[0][0].dtype) for _ in sets]
    stream = torch.cuda.current_stream().cuda_stream

    def launch(s):
        hid, nw, wgu, _ = sets[s % N_SETS]
        check("fd_mlp_gate_up", lib.fd_mlp_gate_up(
            mids[s % N_SETS].data_ptr(), None, hid.data_ptr(), nw.data_ptr(), DTYPE_CODE[nw.dtype],
            wgu.data_ptr(), m, H, I, EPS, kind_code, DTYPE_CODE[hid.dtype], stream))

    for s in range(10):
        launch(s)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for s in range(iters):
        launch(s)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1000.0 / iters


def copy_roof_gbs(torch) -> float:
    from fused_decode.kernels import launch_copy

    n = 1 << 30  # 1 GiB source and destination: far above the Infinity Cache
    src = torch.empty(n, dtype=torch.uint8, device="cuda")
    src.fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        launch_copy(dst, src)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    iters = 20
    start.record()
    for _ in range(iters):
        launch_copy(dst, src)
    end.record()
    torch.cuda.synchronize()
    us = start.elapsed_time(end) * 1000.0 / iters
    del src, dst
    return 2 * n / (us * 1e-6) / 1e9


def read_roof_gbs(torch) -> float:
    """The read roof: fd_read streaming 1 GiB (the copy's load pattern, no stores)."""
    from fused_decode.kernels import launch_read

    n = 1 << 30
    src = torch.zeros(n, dtype=torch.uint8, device="cuda")
    hit = torch.zeros(1, dtype=torch.int32, device="cuda")
    for _ in range(3):
        launch_read(src, hit)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    iters = 20
    start.record()
    for _ in range(iters):
        launch_read(src, hit)
    end.record()
    torch.cuda.synchronize()
    us = start.elapsed_time(end) * 1000.0 / iters
    del src, hit
    return n / (us * 1e-6) / 1e9


OPS_NOTE = ("dev_us: one HIP graph over rotated buffer sets (HBM reads); eager_us: allocating calls back to "
            "back; gbs and pct_* from dev_us and the reference's useful bytes; same_size_us: the roof kernel "
            "moving the op's bytes the same way (fd_copy of half each way for the norms and RoPE, fd_triad for "
            "SwiGLU, fd_read of all for the GEMVs) timed like dev_us, pct_same_size = same_size_us / dev_us; "
            "max_abs_vs_fp32 against the reference's formulas in float32, rounded once")


def pmc_traffic() -> int | None:
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3
    FETCH_SIZE/WRITE_SIZE passes (profiles/mlp_gate_up_m1_pmc.md), or None."""
    path = ROOT / "profiles" / "mlp_gate_up_m1_pmc.md"
    try:
        text = path.read_text()
        block = text.split("```json", 1)[1].split("```", 1)[0]
        return int(json.loads(block)["traffic_bytes"])
    except Exception:
        return None


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(torch, seconds: float) -> dict:
    """The reference's eager MLP block (bench.py:395-398) on the host CPU, fp16,
    M=1, Llama-3-8B widths, random weights of the benchmark's distributions:
    microseconds per call over a bounded sample. Threads: the job's share of the
    host (OMP_NUM_THREADS when set, else the CPUs this process may run on)."""
    import torch.nn.functional as F

    allowed = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    threads = min(allowed, int(os.environ.get("OMP_NUM_THREADS") or allowed))
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(7)
    dt = torch.float16
    hid = torch.randn(1, H, generator=g).to(dt)
    nw = (1 + 0.1 * torch.randn(H, generator=g)).to(dt)
    wgu = (torch.randn(2 * I, H, generator=g) * H ** -0.5).to(dt)
    wd = (torch.randn(H, I, generator=g) * I ** -0.5).to(dt)

    def block():
        h = F.rms_norm(hid, (H,), nw, EPS)
        gate, up = F.linear(h, wgu).split(I, dim=-1)
        return F.linear(F.silu(gate) * up, wd) + hid

    block()  # warm
    calls, t0 = 0, time.perf_counter()
    while True:
        block()
        calls += 1
        el = time.perf_counter() - t0
        if el >= seconds or calls >= 20000:
            break
    return {
        "value": round(el / calls * 1e6, 1),
        "unit": "us",
        "cores": threads,
        "kind": "port",
        "sample": f"{calls} calls of the reference's eager post_attn_mlp block (bench.py:395-398) on torch "
                  f"{torch.__version__} CPU, fp16, M=1, H=4096, I=14336, {el:.1f} s",
        "cpu_model": _cpu_model(),
        "cpus_visible": os.cpu_count(),
        "torch_threads": torch.get_num_threads(),
    }


def progress(msg: str) -> None:
    """One line per finished stage on stderr (stdout carries only the JSON line)."""
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


LINE_LIMIT = 6000  # bytes: the headline line stays well inside an 8 KB stdout window
_DT = {"float16": "f16", "bfloat16": "bf16"}


def headline(*, steps: int, warmup: int, kind: str, mlp: dict, gate_us: float, roof: float, read_roof: float,
             traffic: int | None, decode: dict | None = None, ops_rows: list | None = None,
             ops_path: str | None = None, cpu: dict | None = None) -> dict:
    """The one JSON object bench.py prints last. ``mlp[dtype][m]`` holds the
    post_attn_mlp timings (eager_us, graph_us, graph_per_call_us) for dtype
    "f16"/"bf16" and m 1/8; ``value`` is fp16 M=1 eager. The full per-op rows go
    to ``ops_path``; the line carries their summary (fused_decode.bench.summarize_ops)."""
    us1 = mlp["f16"][1]["eager_us"]
    weights = 3 * H * I * 2
    mlp_bytes = (3 * H * I + 2 * 1 * H + H) * 2
    gate_bytes = (2 * I * H + 1 * H + H + 1 * I) * 2  # weights, hidden, norm_w, mid write
    gate_gbs = gate_bytes / (gate_us * 1e-6) / 1e9
    line = {
        "metric": "post_attn_mlp us @M=1 (Llama-3-8B widths); M=8 in m8_us",
        "value": round(us1, 3),
        "unit": "us",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(us1 / 1000.0, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic: random-init weights ~N(0,1/sqrt(K)), hidden ~N(0,1), 4 rotating weight sets",
        "config": {
            "workload": "post_attn_mlp Llama-3-8B H=4096 I=14336 M=1, fp16, cold weights (4 rotating sets)",
            "kind": kind,
            "m": 1,
        },
        "m8_us": round(mlp["f16"][8]["eager_us"], 3),
        "mlp": {
            "cols": "[eager_us, graph_us (one graph of 100 steps), graph_per_call_us (one graph per call)]",
            **{dt: {f"m{m}": [round(r["eager_us"], 2), round(r["graph_us"], 2), round(r["graph_per_call_us"], 2)]
                    for m, r in sorted(per_m.items())} for dt, per_m in mlp.items()},
        },
        "mlp_gbs": round(mlp_bytes / (us1 * 1e-6) / 1e9, 1),
        "copy_roof_gbs": round(roof, 1),
        "read_roof_gbs": round(read_roof, 1),
        "pct_copy_roof": round(100.0 * mlp_bytes / (us1 * 1e-6) / 1e9 / roof, 1),
        "target_us": round(1.25 * weights / (roof * 1e9) * 1e6, 2),
        "roofline": {
            "bound": "hbm",
            "kernel": "mlp_gate_up (RMSNorm + gate/up GEMV + SwiGLU), M=1",
            "achieved": round(gate_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gate_gbs / HBM_PEAK_GBS, 4),
            "avg_us": round(gate_us, 3),
            "algorithmic_bytes": gate_bytes,
            "traffic": traffic,
            "traffic_source": "profiles/mlp_gate_up_m1_pmc.md (FETCH_SIZE x2.0 + WRITE_SIZE, copy-calibrated)",
        },
    }
    if decode is not None:
        line["decode_step"] = decode
    if ops_rows is not None:
        from fused_decode.bench import summarize_ops

        line["ops"] = summarize_ops(ops_rows)
        line["ops_file"] = ops_path
    if cpu is not None:
        line["cpu_baseline"] = cpu
    return line


def render(line: dict) -> str:
    """The headline as one compact JSON line."""
    return json.dumps(line, separators=(",", ":"))


def main() -> None:
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark runs on one GPU only; --gpus must be 1 "
                          "(the operator set has no multi-GPU path)", "n_gpus": args.gpus}))
        sys.exit(2)
    import torch

    import fused_decode as fd
    from fused_decode._lib import KIND_CODE, lib
    from fused_decode.kernels import resolve_kind

    torch.cuda.set_device(0)
    dev = torch.device("cuda:0")
    kind = resolve_kind(None)
    roof = copy_roof_gbs(torch)

    mlp: dict = {}
    gate_us = None
    for dtype in (torch.float16, torch.bfloat16):
        dt = _DT[str(dtype).replace("torch.", "")]
        mlp[dt] = {}
        for m in (1, 8):
            sets = make_sets(torch, m, dtype, dev)
            graph_us, graph_per_call_us = time_graph_steps(torch, fd, sets, args.steps, args.warmup, None)
            r = mlp[dt][m] = {
                "graph_us": graph_us,
                "graph_per_call_us": graph_per_call_us,
                "eager_us": time_eager_steps(torch, fd, sets, args.steps, args.warmup, None),
            }
            if m == 1 and dtype == torch.float16:
                gate_us = time_gate_up_kernel(torch, lib(), sets, m, max(args.steps, 50), KIND_CODE[kind])
            progress(f"post_attn_mlp {dt} M={m}: eager {r['eager_us']:.2f} us, graph {r['graph_us']:.2f} us, "
                     f"one graph per call {r['graph_per_call_us']:.2f} us")
            del sets
            torch.cuda.empty_cache()

    decode = None
    if not args.no_decode_step:
        from fused_decode.decode_step import DecodeStep, time_replays, two_states

        decode = {"workload": "32-layer Llama-3-8B decode step minus attention, hipGraph, fp16 (fp8: E4M3 "
                              "weights; unfused: the reference's operators); us: median of 30 replays; states: "
                              "[fast us, n, slow us, n] when replays split into two rates"}
        for m in (1, 8):
            for form in ("fused", "unfused", "fp8"):
                ds = DecodeStep(m=m, layers=32, dtype=torch.float16, fused=form != "unfused",
                                weights="fp8" if form == "fp8" else "fp16")
                summ = two_states([r["us"] for r in time_replays(ds, 30, 2)])
                g_us = summ["all"]["median_us"]
                key = f"m{m}" if form == "fused" else f"m{m}_{form}"
                decode[f"{key}_us"] = round(g_us, 1)
                decode[f"{key}_gbs"] = round(ds.weight_bytes / (g_us * 1e-6) / 1e9, 1)
                decode[f"{key}_launches"] = ds.launches_per_layer
                if "fast" in summ:
                    decode[f"{key}_states"] = [summ["fast"]["median_us"], summ["fast"]["n"],
                                               summ["slow"]["median_us"], summ["slow"]["n"]]
                progress(f"decode step {key}: {g_us:.1f} us {summ}")
                del ds
                torch.cuda.empty_cache()
    ops_rows = None
    if not args.no_ops:
        from fused_decode.bench import ops_block

        ops_rows = ops_block(roof, log=lambda row: progress(
            f"{row['op']} {row['shape']} {row['dtype']} {row.get('kind', '')}: dev {row['dev_us']} us, "
            f"eager {row['eager_us']} us, {row['pct_copy_roof']}% of copy roof, max_abs {row['max_abs_vs_fp32']:.3g}"))
        out = Path(args.ops_out)
        out.parent.mkdir(parents=True, exist_ok=True)
        out.write_text(json.dumps({"note": OPS_NOTE, "copy_roof_gbs": roof, "rows": ops_rows}, indent=1))
        progress(f"{len(ops_rows)} op rows written to {out}")
        torch.cuda.empty_cache()
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(torch, args.cpu_seconds)
        progress("cpu baseline done")
    line = headline(steps=args.steps, warmup=args.warmup, kind=kind, mlp=mlp, gate_us=gate_us, roof=roof,
                    read_roof=read_roof_gbs(torch), traffic=pmc_traffic(), decode=decode, ops_rows=ops_rows,
                    ops_path=args.ops_out if ops_rows is not None else None, cpu=cpu)
    text = render(line)
    if len(text) > LINE_LIMIT:
        progress(f"headline line is {len(text)} bytes (limit {LINE_LIMIT}): the ops summary is left out")
        line.pop("ops", None)
        text = render(line)
    print(text, flush=True)


if __name__ == "__main__":
    main()
