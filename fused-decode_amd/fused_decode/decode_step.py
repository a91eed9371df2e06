"""A random-init Llama-3-8B decode step minus attention, captured in a HIP graph.

    python -m fused_decode.decode_step [--m 1] [--layers 32] [--dtype fp16] [--steps 20] [--unfused]

Per layer (widths of Llama-3-8B: H=4096, 32 query / 8 KV heads of 128, I=14336),
fused form (the default):

    qkv = pre_attn_qkv(x, attn_norm_w, w_qkv, cos, sin)   # RMSNorm + [M, 6144] GEMV + RoPE of q, k
    attn = stand-in attention output                     # seeded random [M, 4096] per layer
    h    = linear_decode(attn, w_o, row_add=x)           # O-proj with the residual fused
    x    = post_attn_mlp(h, mlp_norm_w, w_gate_up, w_down)

That is four launches per layer. From 5 rows with kind "dot" the projections
run on MFMA and the layer hands row sums of squares along (rowsq.py): the O-proj
writes them for h, the MLP's gate/up normalises h from them inside its kernel,
its down projection writes them for the next x, and the next layer's QKV takes
its norm from those. With rowsq=False each norm derives its sums from its own
input (from 9 rows the MLP's RMSNorm runs as a row kernel, five launches). The
unfused form composes the reference's operators instead, six launches per layer
(seven from 9 rows):

    normed, stream = add_rms_norm(x, zero, attn_norm_w)   # stream <- x, normed <- rms(x)
    qkv  = linear_decode(normed, w_qkv)                  # [M, 6144]
    q, k = rope(qkv[:, :5120] as [M, 40, 128])           # q and k heads in one launch, position 1024
    h    = linear_decode(attn, w_o, row_add=stream)
    x    = post_attn_mlp(h, mlp_norm_w, w_gate_up, w_down)

post_attn_mlp returns the whole residual stream (its residual add is fused into
the down projection). Both forms compute the same values with the same rounding
points. The whole step is captured once and replayed.

With weights="fp8" the four projections hold E4M3 codes with per-row scales
(quantize_fp8) and the layer runs as pre_attn_qkv_fp8, linear_decode_fp8 (O-proj
with the residual) and post_attn_mlp_fp8: four launches per layer, with the same
row-sum handoff from 5 rows.

Weights per layer: 436,207,616 bytes in fp16 (13.96 GB for 32 layers), half that
plus the scales in fp8, random with the benchmark distributions (no checkpoint
is loaded).
"""

from __future__ import annotations

import argparse
import json

import torch

from .kernels import _MFMA_MIN_M
from .fp8 import linear_decode_fp8, post_attn_mlp_fp8, pre_attn_qkv_fp8, quantize_fp8
from .ops import add_rms_norm, linear_decode, post_attn_mlp, pre_attn_qkv, rope
from .rowsq import (linear_fp8_sumsq, linear_sumsq, post_attn_mlp_fp8_sumsq, post_attn_mlp_sumsq,
                    pre_attn_qkv_fp8_sumsq, pre_attn_qkv_sumsq, sumsq_buffer)

H, I, HEADS, KV_HEADS, HEAD_DIM = 4096, 14336, 32, 8, 128
QKV = (HEADS + 2 * KV_HEADS) * HEAD_DIM  # 6144


def llama3_angles(position: int, dim: int = HEAD_DIM, theta: float = 500000.0, device="cuda"):
    """cos/sin rows [1, 1, dim] for one position (rotate-half layout)."""
    inv = 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float64, device=device) / dim))
    ang = position * inv
    emb = torch.cat((ang, ang))
    return emb.cos().view(1, 1, dim), emb.sin().view(1, 1, dim)


class DecodeStep:
    """Weights and buffers of an L-layer decode step; `step()` runs it eagerly,
    `capture()` records it into a HIP graph and `replay()` runs that."""

    def __init__(self, m: int = 1, layers: int = 32, dtype=torch.float16, device="cuda",
                 seed: int = 0, h: int = H, i: int = I, kind: str | None = None, position: int = 1024,
                 fused: bool = True, weights: str = "fp16", rowsq: bool = True):
        if weights not in ("fp16", "fp8"):
            raise ValueError("weights must be 'fp16' (the activation dtype) or 'fp8'")
        self.m, self.layers, self.dtype, self.kind, self.fused = m, layers, dtype, kind, fused
        self.fp8 = weights == "fp8"
        # the row-sum handoff needs the MFMA kernels (the fp8 forms take them from
        # 5 rows whatever the kind)
        mfma = m >= _MFMA_MIN_M and (self.fp8 or (kind or "dot") == "dot")
        self.rowsq = rowsq and fused and mfma
        self.h, self.i = h, i
        heads = h // HEAD_DIM
        kv = max(1, heads // 4)
        self.qk_heads = heads + kv
        self.qkv_n = (heads + 2 * kv) * HEAD_DIM
        g = torch.Generator(device=device).manual_seed(seed)

        def rnd(*shape, scale=1.0, mean=0.0):
            t = torch.randn(*shape, generator=g, device=device, dtype=torch.float32)
            return (t * scale + mean).to(dtype)

        # projections as activation-dtype weights, or as E4M3 codes + per-row scales
        proj = (lambda *shape, scale: quantize_fp8(rnd(*shape, scale=scale))) if self.fp8 else rnd
        self.w = []
        for _ in range(layers):
            self.w.append({
                "attn_norm": rnd(h, scale=0.1, mean=1.0),
                "qkv": proj(self.qkv_n, h, scale=h ** -0.5),
                "o": proj(h, h, scale=h ** -0.5),
                "mlp_norm": rnd(h, scale=0.1, mean=1.0),
                "gate_up": proj(2 * i, h, scale=h ** -0.5),
                "down": proj(h, i, scale=i ** -0.5),
                "attn_out": rnd(m, h),  # stand-in for the attention output of this layer
            })
        cos, sin = llama3_angles(position, device=device)
        self.cos, self.sin = cos.to(dtype), sin.to(dtype)
        self.x_in = rnd(m, h)
        self.zero = torch.zeros(m, h, device=device, dtype=dtype)
        self.stream = torch.empty(m, h, device=device, dtype=dtype)
        self.normed = torch.empty(m, h, device=device, dtype=dtype)
        self.qkv = torch.empty(m, self.qkv_n, device=device, dtype=dtype)
        self.hbuf = torch.empty(m, h, device=device, dtype=dtype)
        self.out = torch.empty(m, h, device=device, dtype=dtype)
        if self.rowsq:
            self.xbuf = torch.empty(m, h, device=device, dtype=dtype)
            self.mid = torch.empty(m, i, device=device, dtype=dtype)
            self.ss_h, self.ss_x = sumsq_buffer(h, device), sumsq_buffer(h, device)
        self.graph = None

    @property
    def weight_bytes(self) -> int:
        e = torch.empty((), dtype=self.dtype).element_size()
        proj = self.qkv_n * self.h + self.h * self.h + 3 * self.h * self.i
        if self.fp8:  # one byte per weight plus a float32 scale per row
            per = proj + 4 * (self.qkv_n + self.h + 2 * self.i + self.h) + 2 * self.h * e
        else:
            per = proj * e + 2 * self.h * e
        return per * self.layers

    def step(self) -> torch.Tensor:
        if self.rowsq:
            return self._step_rowsq()
        if self.fp8:
            return self._step_fp8()
        return self._step_fused() if self.fused else self._step_composed()

    def _step_rowsq(self) -> torch.Tensor:
        """The fused layer with row sums of squares handed to each RMSNorm (the
        first layer's QKV, whose input no launch of the step wrote, normalises
        itself)."""
        x = self.x_in
        rope_cols = self.qk_heads * HEAD_DIM
        for li, w in enumerate(self.w):
            if self.fp8:
                if li == 0:
                    pre_attn_qkv_fp8(x, w["attn_norm"], *w["qkv"], self.cos, self.sin, 1e-5,
                                     rope_cols=rope_cols, out=self.qkv)
                else:
                    pre_attn_qkv_fp8_sumsq(x, w["attn_norm"], *w["qkv"], self.cos, self.sin, 1e-5,
                                           rope_cols=rope_cols, ss_in=self.ss_x, out=self.qkv)
                linear_fp8_sumsq(w["attn_out"], *w["o"], row_add=x, out=self.hbuf, ss_out=self.ss_h)
                post_attn_mlp_fp8_sumsq(self.hbuf, w["mlp_norm"], *w["gate_up"], *w["down"], 1e-5, out=self.xbuf,
                                        ss_in=self.ss_h, ss_out=self.ss_x, mid=self.mid)
            else:
                if li == 0:
                    pre_attn_qkv(x, w["attn_norm"], w["qkv"], self.cos, self.sin, 1e-5, rope_cols=rope_cols,
                                 out=self.qkv, kind=self.kind)
                else:
                    pre_attn_qkv_sumsq(x, w["attn_norm"], w["qkv"], self.cos, self.sin, 1e-5,
                                       rope_cols=rope_cols, ss_in=self.ss_x, out=self.qkv)
                linear_sumsq(w["attn_out"], w["o"], row_add=x, out=self.hbuf, ss_out=self.ss_h)
                post_attn_mlp_sumsq(self.hbuf, w["mlp_norm"], w["gate_up"], w["down"], 1e-5, out=self.xbuf,
                                    ss_in=self.ss_h, ss_out=self.ss_x, mid=self.mid)
            x = self.xbuf
        self.out.copy_(x)
        return self.out

    def _step_fp8(self) -> torch.Tensor:
        """The fused layer with E4M3 projections: pre_attn_qkv_fp8, fp8 O-proj with
        the residual, post_attn_mlp_fp8."""
        x = self.x_in
        rope_cols = self.qk_heads * HEAD_DIM
        for w in self.w:
            pre_attn_qkv_fp8(x, w["attn_norm"], *w["qkv"], self.cos, self.sin, 1e-5, rope_cols=rope_cols,
                             out=self.qkv)
            linear_decode_fp8(w["attn_out"], *w["o"], row_add=x, out=self.hbuf)
            x = post_attn_mlp_fp8(self.hbuf, w["mlp_norm"], *w["gate_up"], *w["down"], 1e-5)
        self.out.copy_(x)
        return self.out

    def _step_fused(self) -> torch.Tensor:
        x = self.x_in
        rope_cols = self.qk_heads * HEAD_DIM
        for w in self.w:
            pre_attn_qkv(x, w["attn_norm"], w["qkv"], self.cos, self.sin, 1e-5, rope_cols=rope_cols,
                         out=self.qkv, kind=self.kind)
            linear_decode(w["attn_out"], w["o"], row_add=x, out=self.hbuf, kind=self.kind)
            x = post_attn_mlp(self.hbuf, w["mlp_norm"], w["gate_up"], w["down"], 1e-5, kind=self.kind)
        self.out.copy_(x)
        return self.out

    def _step_composed(self) -> torch.Tensor:
        x = self.x_in
        qk = self.qkv[:, : self.qk_heads * HEAD_DIM].view(self.m, self.qk_heads, HEAD_DIM)
        for w in self.w:
            add_rms_norm(x, self.zero, w["attn_norm"], 1e-5, out=self.normed, residual_out=self.stream)
            linear_decode(self.normed, w["qkv"], out=self.qkv, kind=self.kind)
            rope(qk, self.cos, self.sin, out=qk)
            linear_decode(w["attn_out"], w["o"], row_add=self.stream, out=self.hbuf, kind=self.kind)
            x = post_attn_mlp(self.hbuf, w["mlp_norm"], w["gate_up"], w["down"], 1e-5, kind=self.kind)
        self.out.copy_(x)
        return self.out

    @property
    def launches_per_layer(self) -> int:
        """HIP launches one layer issues (the fused QKV folds its norm in at every M;
        the MLP is two launches, three where its fp16/bf16 MFMA form from 9 rows runs
        a row kernel for its RMSNorm)."""
        row_kernel = (self.kind or "dot") == "dot" and self.m > 8 and not self.fp8 and not self.rowsq
        mlp = 3 if row_kernel else 2
        if self.fp8 or self.fused:
            return 1 + 1 + mlp
        return 4 + mlp

    def capture(self) -> None:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            self.step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.step()

    def replay(self) -> torch.Tensor:
        if self.graph is None:
            self.capture()
        self.graph.replay()
        return self.out


def time_step(ds: DecodeStep, steps: int, warmup: int, graph: bool) -> float:
    run = ds.replay if graph else ds.step
    if graph and ds.graph is None:
        ds.capture()
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        run()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1000.0 / steps


# A child process (no torch, no GPU work) that samples the current clock of the
# gfx, memory, data-fabric and SoC domains with amdsmi every PERIOD seconds and
# appends one JSON line per sample (time.monotonic stamps, shared with the parent)
# to PATH, until the parent removes the STOP file.
_CLOCK_SAMPLER = """
import json, os, sys, time
import amdsmi
path, stop, period, index = sys.argv[1], sys.argv[2], float(sys.argv[3]), int(sys.argv[4])
amdsmi.amdsmi_init()
dev = amdsmi.amdsmi_get_processor_handles()[index]
kinds = {"gfx": amdsmi.AmdSmiClkType.GFX, "mem": amdsmi.AmdSmiClkType.MEM, "df": amdsmi.AmdSmiClkType.DF,
         "soc": amdsmi.AmdSmiClkType.SOC}
with open(path, "w") as out:
    while os.path.exists(stop):
        t0 = time.monotonic()
        row = {}
        for name, kind in kinds.items():
            try:
                row[name] = amdsmi.amdsmi_get_clock_info(dev, kind).get("clk")
            except Exception as exc:
                row[name] = None
        row["t0"], row["t1"] = t0, time.monotonic()
        out.write(json.dumps(row) + "\\n")
        out.flush()
        time.sleep(period)
amdsmi.amdsmi_shut_down()
"""


class ClockSampler:
    """Runs _CLOCK_SAMPLER in a child process for the duration of a with block;
    ``samples`` then holds its rows (clock MHz per domain, monotonic t0/t1)."""

    def __init__(self, path: str, period: float = 0.005):
        self.path, self.period, self.samples = path, period, []

    def __enter__(self):
        import subprocess
        import sys
        import time

        self.stop = self.path + ".run"
        open(self.stop, "w").close()
        self.proc = subprocess.Popen([sys.executable, "-c", _CLOCK_SAMPLER, self.path, self.stop, str(self.period),
                                      str(torch.cuda.current_device())])
        time.sleep(1.0)  # the child's amdsmi_init
        return self

    def __exit__(self, *exc):
        import os

        os.remove(self.stop)
        self.proc.wait(timeout=30)
        with open(self.path) as f:
            self.samples = [json.loads(line) for line in f if line.strip()]
        return False

    def between(self, t0: float, t1: float) -> list[dict]:
        """Samples whose reading overlapped the window [t0, t1]."""
        return [s for s in self.samples if s["t0"] <= t1 and s["t1"] >= t0]


def counter_rates(pa: list, pb: list) -> dict:
    """Per XCD, the median over its CUs of each CU's shader-counter advance over
    the wall clock's between two clock-probe results (kernels.clock_probe rows:
    [XCD << 8 | CU position, counter, wall]); a CU seen by only one probe is
    skipped."""
    import statistics

    first_a, first_b = {}, {}
    for key, t, w in pa:
        first_a.setdefault(key, (t, w))
    for key, t, w in pb:
        first_b.setdefault(key, (t, w))
    per_xcd: dict = {}
    for key in first_a.keys() & first_b.keys():
        dt, dw = first_b[key][0] - first_a[key][0], first_b[key][1] - first_a[key][1]
        if dw > 0 and dt > 0:
            per_xcd.setdefault(key >> 8, []).append(dt / dw)
    return {x: round(statistics.median(v), 2) for x, v in sorted(per_xcd.items())}


def time_replays(ds: DecodeStep, replays: int, warmup: int, probe_wgs: int = 4096) -> list[dict]:
    """Each graph replay timed on its own (HIP events around it, synchronised
    after it) between two clock probes on the same stream (kernels.clock_probe,
    enough workgroups to land on every CU): per XCD, the median over its CUs of
    the shader counter's advance over the wall clock's across the replay
    (``counter_rate``, counter ticks per wall-clock tick), which is
    proportional to the XCD's average gfx clock during the replay."""
    from .kernels import clock_probe

    if ds.graph is None:
        ds.capture()
    for _ in range(warmup):
        ds.replay()
    torch.cuda.synchronize()
    pa = torch.zeros(probe_wgs, 3, dtype=torch.int64, device="cuda")
    pb = torch.zeros_like(pa)
    out = []
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    import time

    for i in range(replays):
        t0 = time.monotonic()
        khz = clock_probe(pa)
        start.record()
        ds.replay()
        end.record()
        clock_probe(pb)
        torch.cuda.synchronize()
        out.append({"replay": i, "us": round(start.elapsed_time(end) * 1000.0, 1),
                    "counter_rate_per_xcd": counter_rates(pa.cpu().tolist(), pb.cpu().tolist()), "wall_khz": khz,
                    "t0": t0, "t1": time.monotonic()})
    return out


def two_states(times: list[float]) -> dict:
    """Split replay times at the widest gap in their sorted order (the boundary
    between two steady rates, when there are two) and summarise each side and
    the whole: count, median, spread."""
    import statistics

    st = sorted(times)
    gaps = [(b - a, i) for i, (a, b) in enumerate(zip(st, st[1:]))]
    widest, at = max(gaps) if gaps else (0.0, 0)
    summary = {"all": {"n": len(st), "median_us": round(statistics.median(st), 1),
                       "min_us": st[0], "max_us": st[-1]}}
    # two states only when the widest gap exceeds 1% of the median and both sides hold >= 3 replays
    if widest > 0.01 * statistics.median(st) and 3 <= at + 1 <= len(st) - 3:
        lo, hi = st[:at + 1], st[at + 1:]
        summary["fast"] = {"n": len(lo), "median_us": round(statistics.median(lo), 1), "max_us": lo[-1]}
        summary["slow"] = {"n": len(hi), "median_us": round(statistics.median(hi), 1), "min_us": hi[0]}
    return summary


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--m", type=int, nargs="+", default=[1, 8])
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--dtype", choices=["fp16", "bf16"], default="fp16")
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--unfused", action="store_true", help="compose the reference's operators (6 launches/layer at M < 5)")
    ap.add_argument("--weights", choices=["fp16", "fp8"], default="fp16", help="projection weights (fp8: E4M3 + row scales)")
    ap.add_argument("--no-rowsq", action="store_true", help="no row-sum handoff (each RMSNorm derives its sums from its own input)")
    ap.add_argument("--replays", type=int, default=0,
                    help="time this many graph replays one by one, each between two clock probes")
    ap.add_argument("--fresh", type=int, default=1, help="with --replays: step objects built and timed in turn")
    ap.add_argument("--churn", type=float, default=0.0,
                    help="with --replays: allocate, touch and free this many GB before building each step object")
    ap.add_argument("--smi", default=None, metavar="JSONL",
                    help="with --replays: sample the gfx, memory, fabric and SoC clocks (amdsmi, a child process) "
                         "into this file and report each replay's")
    ap.add_argument("--keep", action="store_true",
                    help="with --replays: keep every step object alive (each takes new memory) instead of freeing it")
    args = ap.parse_args()
    dtype = torch.float16 if args.dtype == "fp16" else torch.bfloat16
    if args.replays:
        replay_report(args, dtype)
        return
    for m in args.m:
        ds = DecodeStep(m=m, layers=args.layers, dtype=dtype, fused=not args.unfused, weights=args.weights,
                        rowsq=not args.no_rowsq)
        eager = time_step(ds, args.steps, args.warmup, graph=False)
        graph = time_step(ds, args.steps, args.warmup, graph=True)
        wb = ds.weight_bytes
        print(json.dumps({
            "workload": f"decode step minus attention, {args.layers} layers, Llama-3-8B widths, M={m}, {args.dtype}, "
                        f"{'unfused' if args.unfused else 'fused'}, {args.weights} weights",
            "eager_us": round(eager, 2),
            "graph_us": round(graph, 2),
            "weight_bytes": wb,
            "graph_gbs": round(wb / (graph * 1e-6) / 1e9, 1),
            "launches_per_step": ds.launches_per_layer * args.layers + 1,
            "finite": bool(torch.isfinite(ds.out.float()).all().item()),
        }), flush=True)
        del ds
        torch.cuda.empty_cache()


def replay_report(args, dtype) -> None:
    """--replays: per M and fresh step object, one JSON line per replay (its time
    and each XCD's shader-counter rate during it; with --smi the clock levels
    the sampler saw inside it), and a summary line: the replay times split into
    their steady states, each with its median rate."""
    import contextlib
    import statistics

    kept = []
    sampler = ClockSampler(args.smi) if args.smi else None
    with sampler if sampler else contextlib.nullcontext():
        runs = _replay_runs(args, dtype, kept, sampler)
    if not sampler:
        return
    for m, f, rows in runs:
        for r in rows:
            smp = sampler.between(r["t0"], r["t1"])
            for dom in ("gfx", "mem", "df", "soc"):
                vals = [s[dom] for s in smp if isinstance(s.get(dom), (int, float))]
                r[f"{dom}_mhz"] = sorted(set(vals)) if vals else None
            r["smi_samples"] = len(smp)
            print(json.dumps(r), flush=True)
    print(json.dumps({"smi_samples_total": len(sampler.samples),
                      "smi_call_ms_median": round(1e3 * statistics.median(s["t1"] - s["t0"] for s in sampler.samples), 2)
                      if sampler.samples else None}), flush=True)


def _replay_runs(args, dtype, kept, sampler) -> list:
    """The replays of replay_report: (m, fresh, rows) per step object; rows are
    printed here unless a sampler's samples are to be attached first."""
    import statistics

    runs = []
    for m in args.m:
        for f in range(args.fresh):
            if args.churn > 0:  # memory the step's weights may then be placed in after it was freed
                blocks = [torch.ones(1 << 30, dtype=torch.uint8, device="cuda") for _ in range(int(args.churn))]
                torch.cuda.synchronize()
                del blocks
                torch.cuda.empty_cache()
            ds = DecodeStep(m=m, layers=args.layers, dtype=dtype, fused=not args.unfused, weights=args.weights,
                            rowsq=not args.no_rowsq)
            rows = time_replays(ds, args.replays, args.warmup)
            for r in rows:
                clk = list(r["counter_rate_per_xcd"].values())
                r.update(m=m, fresh=f, counter_rate_median=round(statistics.median(clk), 2) if clk else None)
            runs.append((m, f, rows))
            if not sampler:
                for r in rows:
                    print(json.dumps(r), flush=True)
            summ = two_states([r["us"] for r in rows])
            for state in ("fast", "slow"):
                if state in summ:
                    sel = [r["counter_rate_median"] for r in rows if r["counter_rate_median"] is not None
                           and (r["us"] <= summ["fast"]["max_us"]) == (state == "fast")]
                    summ[state]["counter_rate_median"] = round(statistics.median(sel), 2) if sel else None
            clk_all = [r["counter_rate_median"] for r in rows if r["counter_rate_median"] is not None]
            summ["all"]["counter_rate_median"] = round(statistics.median(clk_all), 2) if clk_all else None
            print(json.dumps({"summary": True, "m": m, "fresh": f, "weights": args.weights, "churn_gb": args.churn,
                              "kept": args.keep, **summ}), flush=True)
            if args.keep:
                kept.append(ds)
            del ds
            torch.cuda.empty_cache()
    return runs


if __name__ == "__main__":
    main()
