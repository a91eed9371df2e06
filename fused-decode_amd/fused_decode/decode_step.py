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
    args = ap.parse_args()
    dtype = torch.float16 if args.dtype == "fp16" else torch.bfloat16
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


if __name__ == "__main__":
    main()
