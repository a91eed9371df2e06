"""Per-operator roofline and latency bench on one MI355X.

    python -m fused_decode.bench [--out results.json] [--quick] [--dtype fp16|bf16|both] [--tune [--tune-out tiles.json]]

Mirrors the reference's bench (src/fused_decode/bench.py): an in-process copy
roof, HIP-event medians (10 warmup calls, then `rounds` rounds of back-to-back
calls, median of per-call microseconds; reference bench.py:42-56), useful
bytes counted as in the reference README (README.md:33-43), PyTorch eager on
the GPU beside each op, and graph replay of the MLP. Added for MI355X:

* cold-cache numbers: every op rotates through enough distinct input/weight
  sets that the rotation exceeds 2x the 256 MB Infinity Cache, so each call
  reads HBM; warm (same buffers every call) numbers are reported beside them;
* the copy roof moves >= 1 GiB, and a read-only roof is reported as well;
* % of the 8 TB/s datasheet peak next to % of the copy roof;
* PyTorch eager on the host CPU (same dtype, same shapes, thread count stated)
  as the CPU baseline.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import time

import torch
import torch.nn.functional as F

from . import _lib, kernels
from .kernels import launch_copy, launch_copy_persistent, launch_read, launch_triad
from .ops import add_rms_norm, linear_decode, post_attn_mlp, pre_attn_qkv, rms_norm, rope, swiglu

LLAMA_H = 4096
LLAMA_I = 14336
DATASHEET_GBS = 8000.0
MALL_BYTES = 256 * 1024 * 1024
ROTATE_TARGET = 2 * MALL_BYTES + 64 * 1024 * 1024


def _sync() -> None:
    torch.cuda.synchronize()


def _cus() -> int:
    return torch.cuda.get_device_properties(0).multi_processor_count


def time_us(fn, iters: int, warmup: int = 10, rounds: int = 5) -> float:
    """Median over rounds of per-call microseconds; fn(i) gets the call index."""
    for i in range(warmup):
        fn(i)
    _sync()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    samples = []
    for _ in range(rounds):
        start.record()
        for i in range(iters):
            fn(i)
        end.record()
        _sync()
        samples.append(start.elapsed_time(end) / iters * 1000.0)
    return statistics.median(samples)


def cpu_time_us(fn, budget_s: float = 2.0, max_iters: int = 50) -> float:
    fn()
    t0 = time.perf_counter()
    n = 0
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= max_iters:
            return el / n * 1e6


def copies_for(working_set: int) -> int:
    """Number of distinct buffer sets so a rotation exceeds 2x the Infinity Cache
    (capped at 64: below ~10 MB per call an op is launch-bound, not HBM-bound)."""
    return min(64, max(1, math.ceil(ROTATE_TARGET / max(1, working_set))))


def graph_us(fn, k: int, replays: int = 20) -> float | None:
    """Device time per call: one HIP graph holding fn(0..k-1) (every buffer set
    once), replayed; excludes the Python launch path."""
    try:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for i in range(k):
                fn(i)
        torch.cuda.current_stream().wait_stream(side)
        _sync()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(k):
                fn(i)
        reps = max(replays, math.ceil(200 / k))
        us = time_us(lambda i: g.replay(), iters=reps, warmup=3, rounds=3) / k
        del g
        return us
    except Exception as exc:  # pragma: no cover
        print("graph capture failed:", exc)
        return None


def bench_roofline() -> dict:
    n = 1 << 30
    a = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    c = torch.empty_like(a)
    copy_us = time_us(lambda i: launch_copy(c, a), iters=10, warmup=3)
    del a, c
    e = (1 << 30) // 2
    x = torch.randn(e, device="cuda", dtype=torch.float16)
    y = torch.randn(e, device="cuda", dtype=torch.float16)
    z = torch.empty_like(x)
    triad_us = time_us(lambda i: launch_triad(x, y, z, 1.25), iters=10, warmup=3)
    del x, y, z
    torch.cuda.empty_cache()
    return {
        "copy_bytes_each_way": n,
        "copy_us": copy_us,
        "copy_gbs": 2 * n / (copy_us * 1e-6) / 1e9,
        "triad_us": triad_us,
        "triad_gbs": 3 * e * 2 / (triad_us * 1e-6) / 1e9,
        "datasheet_gbs": DATASHEET_GBS,
    }


def _row(name, nbytes, cold_us, warm_us, roof, dev_us=None, **extra) -> dict:
    """`us`: eager launches back to back (the reference's method); `dev_us`: the
    same calls replayed from a HIP graph (device time). GB/s and % of roof use
    the device time when there is one."""
    t = dev_us if dev_us else cold_us
    gbs = nbytes / (t * 1e-6) / 1e9
    row = {
        "name": name,
        "bytes": nbytes,
        "us": cold_us,
        "dev_us": dev_us,
        "us_warm": warm_us,
        "gbs": gbs,
        "gbs_eager": nbytes / (cold_us * 1e-6) / 1e9,
        "gbs_warm": nbytes / (warm_us * 1e-6) / 1e9,
        "pct_copy_roof": 100.0 * gbs / roof,
        "pct_datasheet": 100.0 * gbs / DATASHEET_GBS,
    }
    row.update(extra)
    return row


def _print(row: dict) -> None:
    dev = f"dev {row['dev_us']:8.2f}" if row.get("dev_us") else "dev      n/a"
    parts = [f"{row['name']:<44}", f"{row['us']:9.2f} us", dev, f"{row['gbs']:8.1f} GB/s",
             f"{row['pct_copy_roof']:5.1f}% copy", f"warm {row['us_warm']:8.2f}"]
    for k in ("eager_us", "cpu_eager_us", "graph_us", "hipblas_us", "composed_dev_us"):
        if row.get(k) is not None:
            parts.append(f"{k} {row[k]:.2f}")
    print("  ".join(parts), flush=True)


def _gen(shape, dtype, g, scale=1.0, mean=0.0):
    return (torch.randn(*shape, generator=g, device="cuda", dtype=torch.float32) * scale + mean).to(dtype)


def bench_pointwise(dtype, roof, quick, cpu) -> list[dict]:
    rows = []
    e = torch.empty((), dtype=dtype).element_size()
    g = torch.Generator(device="cuda").manual_seed(0)
    norm_shapes = [(8192, LLAMA_H), (1, LLAMA_H)]
    for r, h in norm_shapes:
        ws = 4 * r * h * e
        k = copies_for(ws)
        xs = [_gen((r, h), dtype, g) for _ in range(k)]
        rs = [_gen((r, h), dtype, g) for _ in range(k)]
        w = _gen((h,), dtype, g, 0.1, 1.0)
        outs = [torch.empty_like(xs[0]) for _ in range(k)]
        cold = time_us(lambda i: rms_norm(xs[i % k], w, 1e-5, out=outs[i % k]), iters=max(20, 2 * k))
        dev = graph_us(lambda i: rms_norm(xs[i % k], w, 1e-5, out=outs[i % k]), k)
        warm = time_us(lambda i: rms_norm(xs[0], w, 1e-5, out=outs[0]), iters=50)
        eager = time_us(lambda i: F.rms_norm(xs[i % k], (h,), w, 1e-5), iters=max(20, 2 * k))
        cpu_us = None
        if cpu:
            xc, wc = xs[0].cpu(), w.cpu()
            cpu_us = cpu_time_us(lambda: F.rms_norm(xc, (h,), wc, 1e-5))
        rows.append(_row(f"rms_norm {r}x{h} {dtype}", (2 * r * h + h) * e, cold, warm, roof, dev,
                         eager_us=eager, cpu_eager_us=cpu_us))
        _print(rows[-1])
        cold = time_us(lambda i: add_rms_norm(xs[i % k], rs[i % k], w, 1e-5, out=outs[i % k], residual_out=rs[i % k]),
                       iters=max(20, 2 * k))
        dev = graph_us(lambda i: add_rms_norm(xs[i % k], rs[i % k], w, 1e-5, out=outs[i % k], residual_out=rs[i % k]), k)
        warm = time_us(lambda i: add_rms_norm(xs[0], rs[0], w, 1e-5, out=outs[0], residual_out=rs[0]), iters=50)
        eager = time_us(lambda i: F.rms_norm(xs[i % k] + rs[i % k], (h,), w, 1e-5), iters=max(20, 2 * k))
        cpu_us = None
        if cpu:
            xc, rc, wc = xs[0].cpu(), rs[0].cpu(), w.cpu()
            cpu_us = cpu_time_us(lambda: F.rms_norm(xc + rc, (h,), wc, 1e-5))
        rows.append(_row(f"add_rms_norm {r}x{h} {dtype}", (4 * r * h + h) * e, cold, warm, roof, dev,
                         eager_us=eager, cpu_eager_us=cpu_us))
        _print(rows[-1])
        del xs, rs, outs
    for r in ([2048, 1] if not quick else [2048]):
        n = LLAMA_I
        k = copies_for(3 * r * n * e)
        gs = [_gen((r, n), dtype, g, 2.0) for _ in range(k)]
        us_ = [_gen((r, n), dtype, g, 2.0) for _ in range(k)]
        outs = [torch.empty_like(gs[0]) for _ in range(k)]
        cold = time_us(lambda i: swiglu(gs[i % k], us_[i % k], out=outs[i % k]), iters=max(20, 2 * k))
        dev = graph_us(lambda i: swiglu(gs[i % k], us_[i % k], out=outs[i % k]), k)
        warm = time_us(lambda i: swiglu(gs[0], us_[0], out=outs[0]), iters=50)
        eager = time_us(lambda i: F.silu(gs[i % k]) * us_[i % k], iters=max(20, 2 * k))
        cpu_us = None
        if cpu:
            gc, uc = gs[0].cpu(), us_[0].cpu()
            cpu_us = cpu_time_us(lambda: F.silu(gc) * uc)
        rows.append(_row(f"swiglu {r}x{n} {dtype}", 3 * r * n * e, cold, warm, roof, dev, eager_us=eager, cpu_eager_us=cpu_us))
        _print(rows[-1])
        del gs, us_, outs
    # RoPE with Llama-3 tables (theta 500000) viewed [S, 1, 128]
    inv = 1.0 / (500000.0 ** (torch.arange(0, 128, 2, dtype=torch.float64, device="cuda") / 128))
    pos = torch.arange(2048, dtype=torch.float64, device="cuda")
    emb = torch.cat([torch.outer(pos, inv)] * 2, -1)
    cos_t, sin_t = emb.cos().to(dtype), emb.sin().to(dtype)
    for xshape, cs in (((1, 2048, 32, 128), (cos_t.view(2048, 1, 128), sin_t.view(2048, 1, 128))),
                       ((1, 1, 32, 128), (cos_t[1024].view(1, 1, 128), sin_t[1024].view(1, 1, 128)))):
        numel = math.prod(xshape)
        nbytes = 2 * numel * e + 2 * cs[0].numel() * e
        k = copies_for(nbytes)
        xs = [_gen(xshape, dtype, g) for _ in range(k)]
        outs = [torch.empty_like(xs[0]) for _ in range(k)]
        c, s = cs

        def eager_rope(x, c=c, s=s):
            cb, sb = c.expand_as(x), s.expand_as(x)
            h = x.shape[-1] // 2
            return torch.cat((x[..., :h] * cb[..., :h] - x[..., h:] * sb[..., :h],
                              x[..., h:] * cb[..., h:] + x[..., :h] * sb[..., h:]), -1)

        cold = time_us(lambda i: rope(xs[i % k], c, s, out=outs[i % k]), iters=max(20, 2 * k))
        dev = graph_us(lambda i: rope(xs[i % k], c, s, out=outs[i % k]), k)
        warm = time_us(lambda i: rope(xs[0], c, s, out=outs[0]), iters=50)
        eager = time_us(lambda i: eager_rope(xs[i % k]), iters=max(20, 2 * k))
        cpu_us = None
        if cpu:
            xc, cc, sc = xs[0].cpu(), c.cpu(), s.cpu()
            cpu_us = cpu_time_us(lambda: eager_rope(xc, cc, sc))
        rows.append(_row(f"rope {xshape} {dtype}", nbytes, cold, warm, roof, dev, eager_us=eager, cpu_eager_us=cpu_us))
        _print(rows[-1])
        del xs, outs
    torch.cuda.empty_cache()
    return rows


def bench_linear(dtype, roof, quick, cpu) -> list[dict]:
    rows = []
    e = torch.empty((), dtype=dtype).element_size()
    g = torch.Generator(device="cuda").manual_seed(1)
    shapes = [(4096, 4096), (4096, 14336), (28672, 4096), (6144, 4096)]
    ms = [1, 8] if quick else [1, 2, 4, 8, 16]
    for n, kk in shapes:
        wbytes = n * kk * e
        k = copies_for(wbytes)
        ws = [_gen((n, kk), dtype, g, kk ** -0.5) for _ in range(k)]
        for m in ms:
            x = _gen((m, kk), dtype, g)
            out = torch.empty(m, n, device="cuda", dtype=dtype)
            nbytes = (m * kk + n * kk + m * n) * e
            hip = time_us(lambda i: F.linear(x, ws[i % k]), iters=max(30, 2 * k))
            hip_dev = graph_us(lambda i: F.linear(x, ws[i % k]), k)
            cpu_us = None
            if cpu and m in (1, 8):
                xc, wc = x.cpu(), ws[0].cpu()
                cpu_us = cpu_time_us(lambda: F.linear(xc, wc), budget_s=1.0, max_iters=10)
            for kind in ("simt", "dot"):
                cold = time_us(lambda i: linear_decode(x, ws[i % k], out=out, kind=kind), iters=max(30, 2 * k))
                dev = graph_us(lambda i: linear_decode(x, ws[i % k], out=out, kind=kind), k)
                warm = time_us(lambda i: linear_decode(x, ws[0], out=out, kind=kind), iters=50)
                rows.append(_row(f"linear M={m} N={n} K={kk} {kind} {dtype}", nbytes, cold, warm, roof, dev,
                                 hipblas_us=hip, hipblas_dev_us=hip_dev, cpu_eager_us=cpu_us))
                _print(rows[-1])
        del ws
        torch.cuda.empty_cache()
    return rows


def one_gemv(m: int, n: int, kk: int, kind: str, dtype, replays: int = 20, fp8: bool = False) -> dict:
    """One decode GEMV alone: device time per call from a HIP graph over rotated
    weights (the ops block's `dev_us`), beside a read of the same bytes timed the
    same way. A profiler run over it sees only this kernel and the read. With
    `fp8` the weights are E4M3 codes with float32 row scales (`linear_decode_fp8`)."""
    e = torch.empty((), dtype=dtype).element_size()
    g = torch.Generator(device="cuda").manual_seed(1)
    if fp8:
        from .fp8 import linear_decode_fp8, quantize_fp8

        k = copies_for(n * kk)
        ws = [quantize_fp8(_gen((n, kk), dtype, g, kk ** -0.5)) for _ in range(k)]
        x = _gen((m, kk), dtype, g)
        out = torch.empty(m, n, device="cuda", dtype=dtype)
        dev = graph_us(lambda i: linear_decode_fp8(x, *ws[i % k], out=out), k, replays)
        wbytes = n * kk + 4 * n
    else:
        k = copies_for(n * kk * e)
        ws = [_gen((n, kk), dtype, g, kk ** -0.5) for _ in range(k)]
        x = _gen((m, kk), dtype, g)
        out = torch.empty(m, n, device="cuda", dtype=dtype)
        dev = graph_us(lambda i: linear_decode(x, ws[i % k], out=out, kind=kind), k, replays)
        wbytes = n * kk * e
    del ws
    torch.cuda.empty_cache()
    nbytes = wbytes + (m * kk + m * n) * e
    kr = copies_for(nbytes)
    srcs = [torch.zeros(nbytes // 16 * 16, dtype=torch.uint8, device="cuda") for _ in range(kr)]
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    read = graph_us(lambda i: launch_read(srcs[i % kr], flag), kr, replays)
    row = {"op": "linear_decode_fp8" if fp8 else "linear_decode", "shape": [m, n, kk],
           "dtype": str(dtype).replace("torch.", ""), "kind": "e4m3" if fp8 else kind,
           "bytes": nbytes, "dev_us": round(dev, 3), "gbs": round(nbytes / dev / 1e3, 1),
           "same_size_read_us": round(read, 3), "pct_same_size": round(100 * read / dev, 1)}
    print(json.dumps(row), flush=True)
    return row


def bench_mlp(dtype, roof, quick, cpu) -> list[dict]:
    rows = []
    e = torch.empty((), dtype=dtype).element_size()
    g = torch.Generator(device="cuda").manual_seed(2)
    h, i_ = LLAMA_H, LLAMA_I
    k = copies_for(3 * h * i_ * e)
    sets = []
    for _ in range(k):
        sets.append((_gen((h,), dtype, g, 0.1, 1.0), _gen((2 * i_, h), dtype, g, h ** -0.5), _gen((h, i_), dtype, g, i_ ** -0.5)))
    for m in ([1, 8] if not quick else [1]):
        hid = _gen((m, h), dtype, g)

        def eager(j, m=m):
            nw, wgu, wd = sets[j % k]
            hn = F.rms_norm(hid, (h,), nw, 1e-5)
            gate, up = F.linear(hn, wgu).split(i_, dim=-1)
            return F.linear(F.silu(gate) * up, wd) + hid

        for kind in ("dot", "simt"):
            cold = time_us(lambda j: post_attn_mlp(hid, *sets[j % k], 1e-5, kind=kind), iters=max(30, 2 * k))
            warm = time_us(lambda j: post_attn_mlp(hid, *sets[0], 1e-5, kind=kind), iters=30)
            g_us = graph_us(lambda j: post_attn_mlp(hid, *sets[j % k], 1e-5, kind=kind), k)
            eager_us = time_us(eager, iters=max(30, 2 * k))
            cpu_us = None
            if cpu and kind == "dot":
                nw, wgu, wd = (t.cpu() for t in sets[0])
                hc = hid.cpu()

                def cpu_mlp():
                    hn = F.rms_norm(hc, (h,), nw, 1e-5)
                    gate, up = F.linear(hn, wgu).split(i_, dim=-1)
                    return F.linear(F.silu(gate) * up, wd) + hc

                cpu_us = cpu_time_us(cpu_mlp, budget_s=3.0, max_iters=10)
            nbytes = (3 * h * i_ + 2 * m * h + h) * e
            rows.append(_row(f"post_attn_mlp M={m} {kind} {dtype}", nbytes, cold, warm, roof, g_us,
                             eager_us=eager_us, cpu_eager_us=cpu_us,
                             target_us=1.25 * 3 * h * i_ * e / (roof * 1e9) * 1e6))
            _print(rows[-1])
    del sets
    torch.cuda.empty_cache()
    return rows


def bench_qkv(dtype, roof, quick, cpu) -> list[dict]:
    """pre_attn_qkv at Llama-3-8B widths (H=4096, N=6144, q+k heads 40 x 128 rotated),
    beside the same work as three launches of this library (rms_norm,
    linear_decode, rope) and PyTorch eager."""
    rows = []
    e = torch.empty((), dtype=dtype).element_size()
    g = torch.Generator(device="cuda").manual_seed(3)
    h, d = LLAMA_H, 128
    n, rc = 48 * d, 40 * d
    k = copies_for(n * h * e)
    sets = [(_gen((h,), dtype, g, 0.1, 1.0), _gen((n, h), dtype, g, h ** -0.5)) for _ in range(k)]
    ang = 1024 * (1.0 / (500000.0 ** (torch.arange(0, d, 2, device="cuda", dtype=torch.float64) / d)))
    cos = torch.cat([ang, ang]).cos().to(dtype).view(1, d)
    sin = torch.cat([ang, ang]).sin().to(dtype).view(1, d)
    for m in ([1, 8] if not quick else [1]):
        hid = _gen((m, h), dtype, g)
        out = torch.empty(m, n, device="cuda", dtype=dtype)

        def fused(j, m=m):
            nw, w = sets[j % k]
            return pre_attn_qkv(hid, nw, w, cos, sin, 1e-5, rope_cols=rc, out=out)

        def composed(j, m=m):
            nw, w = sets[j % k]
            y = linear_decode(rms_norm(hid, nw, 1e-5), w, out=out)
            heads = y[:, :rc].view(m, rc // d, d)
            rope(heads, cos, sin, out=heads)
            return y

        def eager(j, m=m):
            nw, w = sets[j % k]
            y = F.linear(F.rms_norm(hid, (h,), nw, 1e-5), w)
            x = y[:, :rc].view(m, rc // d, d).float()
            x1, x2 = x[..., : d // 2], x[..., d // 2:]
            c, s_ = cos.float(), sin.float()
            rot = torch.cat([x1 * c[..., : d // 2] - x2 * s_[..., : d // 2], x2 * c[..., d // 2:] + x1 * s_[..., d // 2:]], -1)
            return torch.cat([rot.to(dtype).view(m, rc), y[:, rc:]], -1)

        cold = time_us(fused, iters=max(30, 2 * k))
        warm = time_us(lambda j: fused(0), iters=30)
        g_us = graph_us(fused, k)
        comp_us = graph_us(composed, k)
        eager_us = time_us(eager, iters=max(30, 2 * k))
        nbytes = (n * h + m * h + h + m * n) * e + 2 * d * e
        rows.append(_row(f"pre_attn_qkv M={m} {dtype}", nbytes, cold, warm, roof, g_us,
                         composed_dev_us=comp_us, eager_us=eager_us))
        _print(rows[-1])
    del sets
    torch.cuda.empty_cache()
    return rows


def bench_fp8(dtype, roof, quick, cpu) -> list[dict]:
    """FP8-weight GEMV (the four decode shapes, M = 1 and 8), MLP and fused QKV
    (M = 1 and 8); bytes count one byte per weight plus the float32 scales."""
    from .fp8 import linear_decode_fp8, post_attn_mlp_fp8, pre_attn_qkv_fp8, quantize_fp8

    rows = []
    e = torch.empty((), dtype=dtype).element_size()
    g = torch.Generator(device="cuda").manual_seed(5)
    shapes = [(4096, 4096), (4096, 14336), (28672, 4096), (6144, 4096)]
    for n, kk in shapes:
        k = copies_for(n * kk)
        ws = [quantize_fp8(_gen((n, kk), dtype, g, kk ** -0.5)) for _ in range(k)]
        for m in ([1] if quick else [1, 8]):
            x = _gen((m, kk), dtype, g)
            out = torch.empty(m, n, device="cuda", dtype=dtype)
            fn = lambda i: linear_decode_fp8(x, *ws[i % k], out=out)  # noqa: E731
            cold = time_us(fn, iters=max(30, 2 * k))
            dev = graph_us(fn, k)
            warm = time_us(lambda i: linear_decode_fp8(x, *ws[0], out=out), iters=50)
            nbytes = n * kk + 4 * n + (m * kk + m * n) * e
            rows.append(_row(f"linear_fp8 M={m} N={n} K={kk} {dtype}", nbytes, cold, warm, roof, dev))
            _print(rows[-1])
        del ws
        torch.cuda.empty_cache()
    h, i_ = LLAMA_H, LLAMA_I
    k = copies_for(3 * h * i_)
    sets = [(_gen((h,), dtype, g, 0.1, 1.0),) + quantize_fp8(_gen((2 * i_, h), dtype, g, h ** -0.5))
            + quantize_fp8(_gen((h, i_), dtype, g, i_ ** -0.5)) for _ in range(k)]
    for m in ([1] if quick else [1, 8]):
        hid = _gen((m, h), dtype, g)
        fn = lambda j: post_attn_mlp_fp8(hid, *sets[j % k], 1e-5)  # noqa: E731
        cold = time_us(fn, iters=max(30, 2 * k))
        dev = graph_us(fn, k)
        warm = time_us(lambda j: post_attn_mlp_fp8(hid, *sets[0], 1e-5), iters=30)
        nbytes = 3 * h * i_ + 4 * (2 * i_ + h) + (2 * m * h + h) * e
        rows.append(_row(f"post_attn_mlp_fp8 M={m} {dtype}", nbytes, cold, warm, roof, dev))
        _print(rows[-1])
    del sets
    torch.cuda.empty_cache()
    d = 128
    n, rc = 48 * d, 40 * d
    k = copies_for(n * h)
    qsets = [(_gen((h,), dtype, g, 0.1, 1.0),) + quantize_fp8(_gen((n, h), dtype, g, h ** -0.5))
             for _ in range(k)]
    ang = 1024 * (1.0 / (500000.0 ** (torch.arange(0, d, 2, device="cuda", dtype=torch.float64) / d)))
    cos = torch.cat([ang, ang]).cos().to(dtype).view(1, d)
    sin = torch.cat([ang, ang]).sin().to(dtype).view(1, d)
    for m in ([1] if quick else [1, 8]):
        hid = _gen((m, h), dtype, g)
        out = torch.empty(m, n, device="cuda", dtype=dtype)
        fn = lambda j: pre_attn_qkv_fp8(hid, *qsets[j % k], cos, sin, 1e-5, rope_cols=rc, out=out)  # noqa: E731
        cold = time_us(fn, iters=max(30, 2 * k))
        dev = graph_us(fn, k)
        warm = time_us(lambda j: fn(0), iters=30)
        nbytes = n * h + 4 * n + (m * h + h + m * n) * e + 2 * d * e
        rows.append(_row(f"pre_attn_qkv_fp8 M={m} {dtype}", nbytes, cold, warm, roof, dev))
        _print(rows[-1])
    del qsets
    torch.cuda.empty_cache()
    return rows


# ------------------------------------------------------------------ ops block
#
# One compact row per benchmark configuration of the norms, SwiGLU, RoPE and the
# decode GEMV, for the headline bench line. `max_abs_vs_fp32` compares each op
# with the reference's PyTorch formulas (reference.py:14-63) evaluated in float32
# on the GPU and rounded once, as the reference's bench does (bench.py:224-227,
# :373-374).


def fp32_rms(x, w, eps, residual=None):
    """(y, residual_out) of the reference's rms_norm / add_rms_norm formula."""
    s = x.float() if residual is None else x.float() + residual.float()
    y = s * torch.rsqrt(s.pow(2).mean(-1, keepdim=True) + eps) * w.float()
    return y.to(x.dtype), s.to(x.dtype)


def fp32_swiglu(gate, up):
    return (F.silu(gate.float()) * up.float()).to(gate.dtype)


def fp32_rope(x, cos, sin):
    h = x.shape[-1] // 2
    xf, c, s = x.float(), cos.float().expand(x.shape), sin.float().expand(x.shape)
    return torch.cat((xf[..., :h] * c[..., :h] - xf[..., h:] * s[..., :h],
                      xf[..., h:] * c[..., h:] + xf[..., :h] * s[..., h:]), -1).to(x.dtype)


def fp32_linear(x, w, bias=None, row_add=None):
    y = x.float() @ w.float().t()
    if bias is not None:
        y = y + bias.float()
    if row_add is not None:
        y = y + row_add.float()
    return y.to(x.dtype)


def _max_abs(a, b) -> float:
    return float((a.float() - b.float()).abs().max().item())


# The benchmark configurations of the ops block (the norms at one width in fp16;
# SwiGLU, RoPE and the GEMVs in both activation dtypes; the GEMV at every decode
# weight shape, row count and kind).
NORM_ROWS = (8192, 1)
SWIGLU_ROWS = (2048, 1)
ROPE_X_SHAPES = ((1, 2048, 32, 128), (1, 1, 32, 128))
GEMV_SHAPES = ((4096, 4096), (4096, 14336), (28672, 4096), (6144, 4096))
GEMV_MS = (1, 2, 4, 8, 16)
GEMV_KINDS = ("dot", "simt")
OPS_DTYPES = (torch.float16, torch.bfloat16)


def ops_configs() -> list[tuple]:
    """(op, shape, dtype, kind) of every row ``ops_block`` produces, in its order."""
    cfg = []
    for r in NORM_ROWS:
        cfg += [("rms_norm", (r, LLAMA_H), torch.float16, None), ("add_rms_norm", (r, LLAMA_H), torch.float16, None)]
    cfg += [("swiglu", (r, LLAMA_I), dt, None) for dt in OPS_DTYPES for r in SWIGLU_ROWS]
    cfg += [("rope", s, dt, None) for dt in OPS_DTYPES for s in ROPE_X_SHAPES]
    cfg += [("linear_decode", (m, n, k), dt, kind) for dt in OPS_DTYPES for n, k in GEMV_SHAPES for m in GEMV_MS
            for kind in GEMV_KINDS]
    return cfg


_SHORT = {"float16": "f16", "bfloat16": "bf16"}


def _g3(v: float) -> float:
    """Three significant digits (error columns)."""
    return float(f"{v:.3g}")


OPS_SUMMARY_COLS = ("[dev_us, pct_copy_roof, pct_same_size, max_abs]; gemv: those per M=1,2,4,8,16, "
                    "one max_abs; F.linear: hipBLASLt dev_us per M")


def summarize_ops(rows: list[dict]) -> dict:
    """The ops rows in a few KB for the headline line: one entry per norm, SwiGLU
    and RoPE configuration, one per GEMV (dtype, kind, N x K) with a value per
    row count, and F.linear's device time per (dtype, N x K) beside them."""
    out: dict = {"cols": OPS_SUMMARY_COLS}
    for r in rows:
        dt = _SHORT.get(r["dtype"], r["dtype"])
        same = r.get("pct_same_size")
        if r["op"] == "linear_decode":
            _, n, k = r["shape"]
            grp = out.setdefault(f"gemv {dt} {r['kind']} {n}x{k}", [[], [], [], 0.0])
            grp[0].append(r["dev_us"])
            grp[1].append(round(r["pct_copy_roof"]))
            grp[2].append(round(same) if same else None)
            grp[3] = max(grp[3], _g3(r["max_abs_vs_fp32"]))
            if r.get("hipblaslt_dev_us") and r["kind"] == GEMV_KINDS[0]:
                out.setdefault(f"F.linear {dt} {n}x{k}", []).append(round(r["hipblaslt_dev_us"], 2))
        else:
            key = f"{r['op']} {'x'.join(str(v) for v in r['shape'])} {dt}"
            out[key] = [r["dev_us"], r["pct_copy_roof"], same, _g3(r["max_abs_vs_fp32"])]
    return out


def _compact(op, shape, dtype, nbytes, dev_us, eager_us, roof, max_abs, **extra) -> dict:
    gbs = nbytes / (dev_us * 1e-6) / 1e9
    row = {"op": op, "shape": list(shape), "dtype": str(dtype).replace("torch.", ""), "bytes": nbytes,
           "dev_us": round(dev_us, 2), "eager_us": round(eager_us, 2), "gbs": round(gbs, 1),
           "eager_gbs": round(nbytes / (eager_us * 1e-6) / 1e9, 1),
           "pct_copy_roof": round(100.0 * gbs / roof, 1), "pct_8tbs": round(100.0 * gbs / DATASHEET_GBS, 1),
           "max_abs_vs_fp32": max_abs}
    row.update({k: (round(v, 2) if isinstance(v, float) else v) for k, v in extra.items()})
    if extra.get("same_size_us"):
        row["pct_same_size"] = round(100.0 * extra["same_size_us"] / dev_us, 1)
    return row


def ops_block(roof: float, log=print) -> list[dict]:
    """Every norm, SwiGLU, RoPE and GEMV benchmark configuration: device time (one
    HIP graph over rotated buffer sets, so each call reads HBM), eager time (back
    to back allocating calls over the same rotation, the reference's method),
    GB/s of the device time, % of the copy roof and of 8 TB/s, and the largest
    deviation from the float32 formula."""
    rows = []
    g = torch.Generator(device="cuda").manual_seed(11)
    eps = 1e-5

    def timed(call, k, iters=None):
        dev = graph_us(call, k)
        eager = time_us(call, iters=iters or max(30, 2 * k), warmup=5, rounds=3)
        return dev, eager

    roofs: dict = {}

    def same_size(kind: str, nbytes: int) -> dict:
        """The roof kernel moving an op's bytes the same way, timed like its
        dev_us (a HIP graph over rotated buffers): a copy of half each way for
        ops that read and write as much (the faster of fd_copy's one-pass grid
        and its persistent form at 4 and 8 workgroups per CU), a triad for two
        reads and a write, a read of all of them for the GEMVs."""
        key = (kind, nbytes)
        if key not in roofs:
            if kind == "triad":  # two reads and one write, fp16
                n = max(8, nbytes // 6 // 8 * 8)
                k = copies_for(6 * n)
                src = [torch.zeros(n, dtype=torch.float16, device="cuda") for _ in range(3 * k)]
                roofs[key] = graph_us(lambda i: launch_triad(src[3 * (i % k)], src[3 * (i % k) + 1],
                                                             src[3 * (i % k) + 2], 1.0), k)
            elif kind == "copy":  # the faster of fd_copy and its persistent form
                half = max(16, nbytes // 2 // 16 * 16)
                k = copies_for(2 * half)
                src = [torch.zeros(half, dtype=torch.uint8, device="cuda") for _ in range(k)]
                dst = [torch.empty(half, dtype=torch.uint8, device="cuda") for _ in range(k)]
                times = [graph_us(lambda i: launch_copy(dst[i % k], src[i % k]), k)]
                for per_cu in (4, 8):
                    wg = per_cu * _cus()
                    times.append(graph_us(lambda i: launch_copy_persistent(dst[i % k], src[i % k], wg), k))
                roofs[key] = min(t for t in times if t is not None)
            else:
                n = max(16, nbytes // 16 * 16)
                k = copies_for(n)
                src = [torch.zeros(n, dtype=torch.uint8, device="cuda") for _ in range(k)]
                hit = torch.zeros(1, dtype=torch.int32, device="cuda")
                roofs[key] = graph_us(lambda i: launch_read(src[i % k], hit), k)
            del src
            torch.cuda.empty_cache()
        return {"same_size_kind": kind, "same_size_us": roofs[key]}

    # norms: x, residual ~N(0,1), weight ~N(1, 0.1), eps 1e-5, residual_out in place
    for r in NORM_ROWS:
        dt, h = torch.float16, LLAMA_H
        e = 2
        k = copies_for(4 * r * h * e)
        xs = [_gen((r, h), dt, g) for _ in range(k)]
        rs = [_gen((r, h), dt, g) for _ in range(k)]
        w = _gen((h,), dt, g, 0.1, 1.0)
        err = _max_abs(rms_norm(xs[0], w, eps), fp32_rms(xs[0], w, eps)[0])
        dev, eager = timed(lambda i: rms_norm(xs[i % k], w, eps), k)
        rows.append(_compact("rms_norm", (r, h), dt, (2 * r * h + h) * e, dev, eager, roof, err,
                             **same_size("copy", (2 * r * h + h) * e)))
        y_ref, ro_ref = fp32_rms(xs[0], w, eps, rs[0])
        r0 = rs[0].clone()
        y, ro = add_rms_norm(xs[0], r0, w, eps, residual_out=r0)
        err = max(_max_abs(y, y_ref), _max_abs(ro, ro_ref))
        dev, eager = timed(lambda i: add_rms_norm(xs[i % k], rs[i % k], w, eps, residual_out=rs[i % k]), k)
        rows.append(_compact("add_rms_norm", (r, h), dt, (4 * r * h + h) * e, dev, eager, roof, err,
                             **same_size("copy", (4 * r * h + h) * e)))
        log(rows[-2]), log(rows[-1])
        del xs, rs
    # SwiGLU: gate, up ~N(0, 2)
    for dt in OPS_DTYPES:
        for r in SWIGLU_ROWS:
            n = LLAMA_I
            k = copies_for(3 * r * n * 2)
            gs = [_gen((r, n), dt, g, 2.0) for _ in range(k)]
            us_ = [_gen((r, n), dt, g, 2.0) for _ in range(k)]
            err = _max_abs(swiglu(gs[0], us_[0]), fp32_swiglu(gs[0], us_[0]))
            dev, eager = timed(lambda i: swiglu(gs[i % k], us_[i % k]), k)
            rows.append(_compact("swiglu", (r, n), dt, 3 * r * n * 2, dev, eager, roof, err,
                                 **same_size("triad", 3 * r * n * 2)))
            log(rows[-1])
            del gs, us_
    # RoPE with Llama-3 tables (theta 500000), cos/sin [2048, 128] viewed [2048, 1, 128]
    inv = 1.0 / (500000.0 ** (torch.arange(0, 128, 2, dtype=torch.float64, device="cuda") / 128))
    emb = torch.cat([torch.outer(torch.arange(2048, dtype=torch.float64, device="cuda"), inv)] * 2, -1)
    for dt in OPS_DTYPES:
        cos_t, sin_t = emb.cos().to(dt), emb.sin().to(dt)
        for xshape in ROPE_X_SHAPES:
            t = xshape[1]  # all 2048 positions, or the one token at position 1024
            pos = slice(0, t) if t > 1 else slice(1024, 1025)
            c, s_ = cos_t[pos].view(t, 1, 128), sin_t[pos].view(t, 1, 128)
            nbytes = 2 * math.prod(xshape) * 2 + 2 * c.numel() * 2
            k = copies_for(nbytes)
            xs = [_gen(xshape, dt, g) for _ in range(k)]
            err = _max_abs(rope(xs[0], c, s_), fp32_rope(xs[0], c, s_))
            dev, eager = timed(lambda i: rope(xs[i % k], c, s_), k)
            rows.append(_compact("rope", xshape, dt, nbytes, dev, eager, roof, err, **same_size("copy", nbytes)))
            log(rows[-1])
            del xs
    # decode GEMV: x ~N(0,1), W ~N(0, 1/sqrt(K)), bias and row_add in the error check
    for dt in OPS_DTYPES:
        for n, kk in GEMV_SHAPES:
            k = copies_for(n * kk * 2)
            ws = [_gen((n, kk), dt, g, kk ** -0.5) for _ in range(k)]
            bias, wf = _gen((n,), dt, g), ws[0]
            for m in GEMV_MS:
                x = _gen((m, kk), dt, g)
                ra = _gen((m, n), dt, g)
                ref = fp32_linear(x, wf, bias, ra)
                hip = graph_us(lambda i: F.linear(x, ws[i % k]), k)
                for kind in GEMV_KINDS:
                    err = _max_abs(linear_decode(x, wf, bias, row_add=ra, kind=kind), ref)
                    dev, eager = timed(lambda i: linear_decode(x, ws[i % k], kind=kind), k)
                    extra = {"kind": kind, **same_size("read", (m * kk + n * kk + m * n) * 2)}
                    if hip is not None:
                        extra["hipblaslt_dev_us"] = hip
                    rows.append(_compact("linear_decode", (m, n, kk), dt, (m * kk + n * kk + m * n) * 2, dev, eager,
                                         roof, err, **extra))
                    log(rows[-1])
            del ws
            torch.cuda.empty_cache()
    torch.cuda.empty_cache()
    return rows


def bench_graph_modes(dtype) -> list[dict]:
    """post_attn_mlp at Llama-3-8B widths, M = 1 and 8, over a rotation of 4 weight
    sets: per-step time launched eagerly, and replayed from HIP graphs holding 1,
    4 or 20 steps. Each hipGraphLaunch leaves the GPU idle before its first
    kernel (a kernel trace of this function shows the gaps), so the per-step cost
    of graph replay depends on how many steps one graph holds."""
    g = torch.Generator(device="cuda").manual_seed(6)
    h, i_, ns = LLAMA_H, LLAMA_I, 4
    rows = []
    for m in (1, 8):
        sets = [(_gen((m, h), dtype, g), _gen((h,), dtype, g, 0.1, 1.0), _gen((2 * i_, h), dtype, g, h ** -0.5),
                 _gen((h, i_), dtype, g, i_ ** -0.5)) for _ in range(ns)]
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for st in sets:
                post_attn_mlp(*st, 1e-5)
        torch.cuda.current_stream().wait_stream(side)
        _sync()
        row = {"name": f"post_attn_mlp M={m} {dtype} graph modes"}
        marker_a = torch.zeros(16, dtype=torch.uint8, device="cuda")
        marker_b = torch.empty_like(marker_a)
        launch_copy(marker_b, marker_a)  # phase marker in a kernel trace (copy_vec_kernel)
        row["eager_us"] = time_us(lambda j: post_attn_mlp(*sets[j % ns], 1e-5), iters=120, warmup=8, rounds=3)
        for per in (1, 4, 20):
            launch_copy(marker_b, marker_a)
            graphs = []
            for first in range(0, ns if per == 1 else 1):
                gr = torch.cuda.CUDAGraph()
                with torch.cuda.graph(gr):
                    for j in range(per):
                        post_attn_mlp(*sets[(first + j) % ns], 1e-5)
                graphs.append(gr)
            us = time_us(lambda j: graphs[j % len(graphs)].replay(), iters=max(6, 120 // per), warmup=2, rounds=3)
            row[f"graph_{per}_steps_us"] = us / per
            del graphs
        rows.append(row)
        print(json.dumps({k: (round(v, 2) if isinstance(v, float) else v) for k, v in row.items()}), flush=True)
        del sets
        torch.cuda.empty_cache()
    return rows


def trace_gaps(csv_path: str) -> None:
    """Summarise a rocprofv3 kernel-trace CSV of ``--only graph``: per phase
    (between copy_vec_kernel markers), the kernels' mean durations and the idle
    gaps between one kernel's end and the next one's start."""
    import csv

    with open(csv_path) as f:
        rows = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))
    phases, cur = [], []
    for r in rows:
        if "copy_vec_kernel" in r["Kernel_Name"]:
            phases.append(cur)
            cur = []
        else:
            cur.append(r)
    phases.append(cur)
    names = [f"M={m} {mode}" for m in (1, 8) for mode in ("eager", "graph of 1 step", "graph of 4 steps",
                                                            "graph of 20 steps")]
    for name, ph in zip(names, [p for p in phases if p][-8:]):
        gaps = [(int(b["Start_Timestamp"]) - int(a["End_Timestamp"])) / 1e3 for a, b in zip(ph, ph[1:])]
        busy = sum(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in ph) / 1e3
        big = [g for g in gaps if g > 1.0]
        print(f"{name:22s} {len(ph):4d} kernels  busy {busy / max(1, len(ph)):7.2f} us/kernel  "
              f"idle gaps > 1 us: {len(big):3d} (mean {statistics.mean(big) if big else 0.0:5.2f} us)  "
              f"all gaps mean {statistics.mean(gaps) if gaps else 0.0:5.2f} us")


# Byte counts of the benchmark configurations whose same-size ceilings matter:
# the 4096^2 and 6144x4096 GEMVs at M=1, RoPE over 2048 tokens, the K=14336 GEMV,
# rms_norm 8192x4096, SwiGLU 2048x14336, the N=28672 GEMV, add_rms_norm, 1 GiB.
CEILING_SIZES = (33_570_816, 34_603_008, 50_352_128, 117_477_376, 134_225_920, 176_160_768, 234_946_560,
                 268_443_648, 1 << 30)


def ceilings() -> list[dict]:
    """Device time (one HIP graph over rotated buffers, as every dev_us) of the
    read roof (fd_read), the copy roof (fd_copy, half the bytes each way) and
    the copy's persistent form at 2, 4 and 8 workgroups per CU, at each size of
    CEILING_SIZES; prints a markdown table (GB/s over the bytes moved)."""
    cus = _cus()
    rows = []
    print("| Bytes | fd_read us | GB/s | fd_copy us | GB/s | persistent 2/CU | 4/CU | 8/CU | best copy GB/s |")
    print("|---|---|---|---|---|---|---|---|---|")
    for nbytes in CEILING_SIZES:
        n = nbytes // 16 * 16
        k = copies_for(n)
        src = [torch.zeros(n, dtype=torch.uint8, device="cuda") for _ in range(k)]
        hit = torch.zeros(1, dtype=torch.int32, device="cuda")
        read = graph_us(lambda i: launch_read(src[i % k], hit), k)
        del src
        torch.cuda.empty_cache()
        half = n // 2 // 16 * 16
        k = copies_for(2 * half)
        a = [torch.zeros(half, dtype=torch.uint8, device="cuda") for _ in range(k)]
        b = [torch.empty(half, dtype=torch.uint8, device="cuda") for _ in range(k)]
        copy = graph_us(lambda i: launch_copy(b[i % k], a[i % k]), k)
        pers = {p: graph_us(lambda i, p=p: launch_copy_persistent(b[i % k], a[i % k], p * cus), k) for p in (2, 4, 8)}
        del a, b
        torch.cuda.empty_cache()
        best = min([copy, *pers.values()])
        row = {"bytes": n, "read_us": read, "copy_us": copy, **{f"persistent_{p}_us": v for p, v in pers.items()}}
        rows.append(row)
        print(f"| {n:,} | {read:.2f} | {n / read / 1e3:.0f} | {copy:.2f} | {2 * half / copy / 1e3:.0f} | "
              f"{pers[2]:.2f} | {pers[4]:.2f} | {pers[8]:.2f} | {2 * half / best / 1e3:.0f} |", flush=True)
    return rows


TIE_BAND = 1.05  # per-shape slack of the cutoff rule


def tune(dtype, out_path: str | None = None) -> dict:
    """Tile search for the HIP GEMV on this GPU (replaces the reference's Triton
    tile sweep, bench.py:475-517): for every decode weight shape and M = 1..16,
    each kind is timed over the tiles of the kernels it may run (kind "simt":
    SIMT; kind "dot": SIMT and MFMA; graph-replayed device time,
    cold weights) next to F.linear. Returns and optionally writes the table
    ``linear_config`` reads: the best tile per (kind, N, K, M) where it beats
    the default by 3% or more (its row count names the kernel), and
    the value for DECODE_LINEAR_MAX_M: the largest M up to which, at every row
    count, the default kind's best tiles run a decode layer's four GEMVs faster
    in sum than F.linear with no shape more than 5% slower (``strict_max_m``:
    every shape faster), and the same cutoff for kind "simt"
    (``simt_decode_linear_max_m``, SIMT_DECODE_LINEAR_MAX_M)."""
    g = torch.Generator(device="cuda").manual_seed(4)
    e = torch.empty((), dtype=dtype).element_size()
    shapes = [(4096, 4096), (4096, 14336), (28672, 4096), (6144, 4096)]
    entries, best_us, default_us, hip_us = {}, {}, {}, {}
    for n, kk in shapes:
        k = copies_for(n * kk * e)
        ws = [_gen((n, kk), dtype, g, kk ** -0.5) for _ in range(k)]
        for m in range(1, 17):
            x = _gen((m, kk), dtype, g)
            out = torch.empty(m, n, device="cuda", dtype=dtype)
            hip_us[f"{n}x{kk}:m{m}"] = graph_us(lambda i: F.linear(x, ws[i % k]), k)
            for kind in ("simt", "dot"):
                dflt = kernels.default_tile(kernels._kernel_of(kind, m), n, kk)
                # SIMT: the per-tile kernel over rows and waves, the persistent one over
                # rows and waves (its waves set 1, 2 or 4 K chunks per lane)
                cands = {(r, w, 1) for r in (2, 4, 8) if r * m <= 64 for w in (4, 8, dflt[1])}
                chunks = -(-kk // 512)
                for cpl in (1, 2, 4):
                    w = -(-chunks // cpl)
                    if w <= 8:
                        cands |= {(r, w, 2) for r in (2, 4, 8) if r * m <= 64 and r * cpl <= 8}
                if kind == "dot":  # the DMA MFMA GEMV: waves x units in flight within a CU's LDS
                    br = 4 if m <= 4 else 8 if m <= 8 else 16
                    cands |= {(16, w, st) for w in (2, 4, 8) for st in (1, 2, 3)
                              if w * st * (256 + 16 * br) * 16 + w * 1024 <= 160 * 1024}
                cands.add(dflt)
                times = {}
                for t in sorted(cands):
                    us = graph_us(lambda i, t=t: kernels.linear_out(x, ws[i % k], out, kind=kind, tile=t), k)
                    if us is not None:
                        times[t] = us
                key = kernels.tile_key(kind, n, kk, m)
                best = min(times, key=times.get)
                best_us[key], default_us[key] = times[best], times[dflt]
                if best != dflt and times[best] <= 0.97 * times[dflt]:
                    entries[key] = list(best)
                print(f"{key:<24} default {dflt} {times[dflt]:8.2f} us  best {best} {times[best]:8.2f} us  "
                      f"F.linear {hip_us[f'{n}x{kk}:m{m}']:8.2f} us", flush=True)
        del ws
        torch.cuda.empty_cache()
    def cutoffs(kind: str) -> tuple[int, int]:
        max_m = strict_m = 0
        for m in range(1, 17):
            ours = [best_us[kernels.tile_key(kind, n, kk, m)] for n, kk in shapes]
            theirs = [hip_us[f"{n}x{kk}:m{m}"] for n, kk in shapes]
            if strict_m == m - 1 and all(a <= b for a, b in zip(ours, theirs)):
                strict_m = m
            if max_m == m - 1 and sum(ours) < sum(theirs) and all(a <= TIE_BAND * b for a, b in zip(ours, theirs)):
                max_m = m
        return max_m, strict_m

    max_m, strict_m = cutoffs("dot")
    simt_max_m, simt_strict_m = cutoffs("simt")
    table = {"arch": torch.cuda.get_device_properties(0).gcnArchName.split(":")[0],
             "dtype": str(dtype).replace("torch.", ""), "entries": entries,
             "best_us": best_us, "default_us": default_us, "hipblas_us": hip_us,
             "decode_linear_max_m": max_m, "strict_max_m": strict_m,
             "simt_decode_linear_max_m": simt_max_m, "simt_strict_max_m": simt_strict_m}
    print(f"DECODE_LINEAR_MAX_M: {max_m} (a layer's four GEMVs faster in sum, none more than "
          f"{100 * (TIE_BAND - 1):.0f}% slower than F.linear); every shape faster up to M={strict_m}; "
          f"kind simt: {simt_max_m} (every shape faster up to M={simt_strict_m}); "
          f"{len(entries)} tiles beat the default by >= 3%", flush=True)
    if out_path:
        with open(out_path, "w") as f:
            json.dump(table, f, indent=1, sort_keys=True)
    return table


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--out", default=None)
    ap.add_argument("--quick", action="store_true")
    ap.add_argument("--dtype", choices=["fp16", "bf16", "both"], default="fp16")
    ap.add_argument("--no-cpu", action="store_true", help="skip PyTorch-eager-on-CPU timings")
    ap.add_argument("--only", choices=["pointwise", "linear", "mlp", "qkv", "fp8", "graph"], default=None)
    ap.add_argument("--tune", action="store_true", help="GEMV tile search (writes --tune-out if given)")
    ap.add_argument("--tune-out", default=None)
    ap.add_argument("--ceilings", action="store_true",
                    help="time the read and copy roof patterns at the decode ops' sizes and exit")
    ap.add_argument("--gemv", default=None, metavar="M,N,K",
                    help="time one GEMV (with --kind, --dtype, --replays) beside a same-size read and exit")
    ap.add_argument("--kind", choices=["dot", "simt"], default="dot")
    ap.add_argument("--fp8", action="store_true", help="with --gemv: E4M3 weights (linear_decode_fp8)")
    ap.add_argument("--replays", type=int, default=20)
    ap.add_argument("--trace-gaps", default=None, metavar="CSV",
                    help="summarise a rocprofv3 kernel trace of --only graph and exit")
    args = ap.parse_args()
    if args.trace_gaps:
        trace_gaps(args.trace_gaps)
        return
    if args.ceilings:
        _lib.lib()
        torch.cuda.set_device(0)
        ceilings()
        return
    _lib.lib()
    torch.cuda.set_device(0)
    if args.gemv:
        m, n, kk = (int(v) for v in args.gemv.split(","))
        one_gemv(m, n, kk, args.kind, torch.bfloat16 if args.dtype == "bf16" else torch.float16, args.replays,
                 args.fp8)
        return
    if args.tune:
        tune(torch.float16 if args.dtype != "bf16" else torch.bfloat16, args.tune_out)
        return
    payload = {
        "gpu": torch.cuda.get_device_name(0),
        "torch": torch.__version__,
        "hip_runtime": _lib.runtime_version(),
        "cpu": platform.processor() or platform.machine(),
        "cpu_threads": torch.get_num_threads(),
        "os_cpu_count": os.cpu_count(),
        "cache_note": f"cold = rotation over >= {ROTATE_TARGET >> 20} MiB of distinct buffers; warm = same buffers",
    }
    if args.only == "graph":
        bench_graph_modes(torch.float16)
        return
    roof = bench_roofline()
    payload["roofline"] = roof
    print(f"copy roof {roof['copy_gbs']:.1f} GB/s  triad {roof['triad_gbs']:.1f} GB/s  (datasheet {DATASHEET_GBS:.0f})", flush=True)
    dtypes = {"fp16": [torch.float16], "bf16": [torch.bfloat16], "both": [torch.float16, torch.bfloat16]}[args.dtype]
    payload["rows"] = []
    for dt in dtypes:
        if args.only in (None, "pointwise"):
            payload["rows"] += bench_pointwise(dt, roof["copy_gbs"], args.quick, not args.no_cpu)
        if args.only in (None, "linear"):
            payload["rows"] += bench_linear(dt, roof["copy_gbs"], args.quick, not args.no_cpu)
        if args.only in (None, "mlp"):
            payload["rows"] += bench_mlp(dt, roof["copy_gbs"], args.quick, not args.no_cpu)
        if args.only in (None, "qkv"):
            payload["rows"] += bench_qkv(dt, roof["copy_gbs"], args.quick, not args.no_cpu)
        if args.only in (None, "fp8"):
            payload["rows"] += bench_fp8(dt, roof["copy_gbs"], args.quick, not args.no_cpu)
        if args.out:
            with open(args.out, "w") as f:
                json.dump(payload, f, indent=1)


if __name__ == "__main__":
    main()
