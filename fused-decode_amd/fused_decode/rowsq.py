"""Row sums of squares handed from a producer launch to the next RMSNorm.

In a decode step every RMSNorm reads a hidden state that a GEMV with the
residual fused in has just written (the O projection before the MLP, the MLP's
down projection before the next layer's QKV). From 5 rows with kind "dot"
those GEMVs run on the MFMA kernel, which can also write, per 16-column tile
``t`` of its [M, N] output, the float32 sums of the squares of its rounded
outputs: ``ss[t, m]`` for ``m < 16`` (rows past M hold 0). The consumer then
derives each row's inverse RMS from ``ceil(N / 16)`` partial sums instead of
re-reading the rows, and normalises inside its own kernel:

    ss_h = sumsq_buffer(H, device)                     # float32 [ceil(H/16), 16]
    linear_sumsq(attn, w_o, row_add=x, out=h, ss_out=ss_h)
    post_attn_mlp_sumsq(h, mlp_norm, w_gu, w_d, eps, out=x, ss_in=ss_h, ss_out=ss_x)
    pre_attn_qkv_sumsq(x, attn_norm, w_qkv, cos, sin, eps, rope_cols=c, out=qkv, ss_in=ss_x)

The MLP's RMSNorm then needs no row kernel of its own (one launch fewer per
layer) and the QKV kernel no pass over its input before its first MFMA. The
results are the operators' results: the norm's sum of squares is the same
float32 sum, added in another order. ``ss_in`` must be the sums of exactly the
``hidden`` passed beside it, written by the launch that wrote ``hidden``.

No reference counterpart: the reference's operators each normalise their own
input (ops.py:72-88 inside the composition at ops.py:312-315).
"""

from __future__ import annotations

import ctypes

import torch

from . import _checks
from ._checks import SUMSQ_MIN_ROWS as MIN_ROWS
from ._lib import DTYPE_CODE, KIND_CODE, check, lib, stream_of
from .ops import _qkv_args


def sumsq_buffer(width: int, device) -> torch.Tensor:
    """Float32 ``[ceil(width / 16), 16]`` tile sums for an activation of ``width``
    columns (torch allocations are 16-byte aligned, as the kernels need)."""
    return torch.empty((width + 15) // 16, 16, device=device, dtype=torch.float32)


def _p(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def linear_sumsq(x: torch.Tensor, weight: torch.Tensor, *, out: torch.Tensor, ss_out: torch.Tensor,
                 bias: torch.Tensor | None = None, row_add: torch.Tensor | None = None,
                 kind: str = "dot") -> torch.Tensor:
    """``out = round(x @ weight.T + bias + row_add)`` (``linear_decode``) for a
    contiguous ``x [M, K]``, ``weight [N, K]``, ``out [M, N]`` and ``row_add``
    ``[M, N]``, also writing ``ss_out`` (``sumsq_buffer(N)``) for the norm that reads
    ``out`` next."""
    _checks.check("linear_sumsq", x=x, weight=weight, bias=bias, row_add=row_add, kind=kind, out=out,
                  ss_out=ss_out)
    (m, k), n = x.shape, weight.shape[0]
    code = DTYPE_CODE[x.dtype]
    check("fd_linear_sumsq", lib().fd_linear_sumsq(
        _p(out), _p(x), _p(weight), _p(bias), DTYPE_CODE[bias.dtype] if bias is not None else code,
        _p(row_add), DTYPE_CODE[row_add.dtype] if row_add is not None else code, m, n, k, k, 1,
        int(weight.stride(0)), int(weight.stride(1)), int(bias.stride(0)) if bias is not None else 0,
        n if row_add is not None else 0, 1 if row_add is not None else 0, n, 1, KIND_CODE[kind], code,
        _p(ss_out), ctypes.c_void_p(stream_of(x))))
    return out


def post_attn_mlp_sumsq(hidden: torch.Tensor, norm_weight: torch.Tensor, w_gate_up: torch.Tensor,
                        w_down: torch.Tensor, eps: float, *, out: torch.Tensor, ss_in: torch.Tensor | None = None,
                        ss_out: torch.Tensor | None = None, mid: torch.Tensor | None = None,
                        kind: str = "dot") -> torch.Tensor:
    """``post_attn_mlp`` for a contiguous ``hidden [M, H]``: with ``ss_in`` (the sums
    of ``hidden``) the RMSNorm runs inside the gate/up kernel; with ``ss_out`` the
    down projection writes the sums of ``out`` for the next norm."""
    a = _checks.check("post_attn_mlp_sumsq", hidden=hidden, norm_weight=norm_weight, w_gate_up=w_gate_up,
                      w_down=w_down, eps=eps, kind=kind, out=out, mid=mid, ss_in=ss_in, ss_out=ss_out)
    (m, h), i, eps = hidden.shape, w_down.shape[1], a["eps"]
    if mid is None:
        mid = torch.empty(m, i, device=hidden.device, dtype=hidden.dtype)
    check("fd_post_attn_mlp_sumsq", lib().fd_post_attn_mlp_sumsq(
        _p(out), _p(mid), _p(hidden), _p(norm_weight), DTYPE_CODE[norm_weight.dtype], _p(w_gate_up), _p(w_down),
        m, h, i, float(eps), KIND_CODE[kind], DTYPE_CODE[hidden.dtype], _p(ss_in),
        (h + 15) // 16 if ss_in is not None else 0, _p(ss_out), ctypes.c_void_p(stream_of(hidden))))
    return out


def pre_attn_qkv_sumsq(hidden: torch.Tensor, norm_weight: torch.Tensor, w_qkv: torch.Tensor, cos: torch.Tensor,
                       sin: torch.Tensor, eps: float, *, rope_cols: int, ss_in: torch.Tensor, out: torch.Tensor,
                       bias: torch.Tensor | None = None, kind: str = "dot") -> torch.Tensor:
    """``pre_attn_qkv`` for a contiguous ``hidden [M, H]`` whose RMSNorm takes its
    row sums from ``ss_in`` (written by the launch that wrote ``hidden``)."""
    a0 = _checks.check("pre_attn_qkv_sumsq", hidden=hidden, norm_weight=norm_weight, w_qkv=w_qkv, eps=eps,
                       kind=kind, bias=bias, ss_in=ss_in, out=out)
    (m, h), n = hidden.shape, w_qkv.shape[0]
    a = _qkv_args(hidden, norm_weight, n, h, cos, sin, a0["eps"], rope_cols, bias, out)
    code = DTYPE_CODE[hidden.dtype]
    check("fd_pre_attn_qkv_sumsq", lib().fd_pre_attn_qkv_sumsq(
        _p(a.out), _p(hidden), _p(norm_weight), DTYPE_CODE[norm_weight.dtype], _p(w_qkv), _p(bias),
        DTYPE_CODE[bias.dtype] if bias is not None else code, _p(a.cos), _p(a.sin), DTYPE_CODE[a.cos.dtype],
        a.cs_row_stride, m, h, n, a.rope_cols, a.d, a.eps, KIND_CODE[kind], code, _p(ss_in), (h + 15) // 16,
        ctypes.c_void_p(stream_of(hidden))))
    return a.out


def linear_fp8_sumsq(x: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor, *, out: torch.Tensor,
                     ss_out: torch.Tensor, bias: torch.Tensor | None = None,
                     row_add: torch.Tensor | None = None) -> torch.Tensor:
    """``linear_decode_fp8`` (E4M3 ``weight [N, K]``, float32 ``scale [N]``) for a
    contiguous ``x [M, K]``, also writing ``ss_out`` for the next norm."""
    _checks.check("linear_fp8_sumsq", x=x, weight=weight, scale=scale, bias=bias, row_add=row_add, out=out,
                  ss_out=ss_out)
    (m, k), n = x.shape, weight.shape[0]
    code = DTYPE_CODE[x.dtype]
    check("fd_linear_fp8_sumsq", lib().fd_linear_fp8_sumsq(
        _p(out), _p(x), _p(weight), _p(scale), _p(bias), DTYPE_CODE[bias.dtype] if bias is not None else code,
        _p(row_add), DTYPE_CODE[row_add.dtype] if row_add is not None else code, m, n, k, k,
        int(weight.stride(0)), int(bias.stride(0)) if bias is not None else 0, n if row_add is not None else 0,
        1 if row_add is not None else 0, n, 1, code, _p(ss_out), ctypes.c_void_p(stream_of(x))))
    return out


def post_attn_mlp_fp8_sumsq(hidden: torch.Tensor, norm_weight: torch.Tensor, w_gate_up: torch.Tensor,
                            gate_up_scale: torch.Tensor, w_down: torch.Tensor, down_scale: torch.Tensor, eps: float,
                            *, out: torch.Tensor, ss_in: torch.Tensor | None = None,
                            ss_out: torch.Tensor | None = None, mid: torch.Tensor | None = None) -> torch.Tensor:
    """``post_attn_mlp_fp8`` for a contiguous ``hidden [M, H]`` with the row sums
    of ``post_attn_mlp_sumsq``."""
    a = _checks.check("post_attn_mlp_fp8_sumsq", hidden=hidden, norm_weight=norm_weight, w_gate_up=w_gate_up,
                      gate_up_scale=gate_up_scale, w_down=w_down, down_scale=down_scale, eps=eps, out=out,
                      mid=mid, ss_in=ss_in, ss_out=ss_out)
    (m, h), i, eps = hidden.shape, w_down.shape[1], a["eps"]
    if mid is None:
        mid = torch.empty(m, i, device=hidden.device, dtype=hidden.dtype)
    check("fd_post_attn_mlp_fp8_sumsq", lib().fd_post_attn_mlp_fp8_sumsq(
        _p(out), _p(mid), _p(hidden), _p(norm_weight), DTYPE_CODE[norm_weight.dtype], _p(w_gate_up),
        _p(gate_up_scale), _p(w_down), _p(down_scale), m, h, i, float(eps), DTYPE_CODE[hidden.dtype], _p(ss_in),
        (h + 15) // 16 if ss_in is not None else 0, _p(ss_out), ctypes.c_void_p(stream_of(hidden))))
    return out


def pre_attn_qkv_fp8_sumsq(hidden: torch.Tensor, norm_weight: torch.Tensor, w_qkv: torch.Tensor,
                           scale: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, eps: float, *,
                           rope_cols: int, ss_in: torch.Tensor, out: torch.Tensor,
                           bias: torch.Tensor | None = None) -> torch.Tensor:
    """``pre_attn_qkv_fp8`` for a contiguous ``hidden [M, H]`` whose RMSNorm takes
    its row sums from ``ss_in``."""
    a0 = _checks.check("pre_attn_qkv_fp8_sumsq", hidden=hidden, norm_weight=norm_weight, w_qkv=w_qkv,
                       scale=scale, eps=eps, bias=bias, ss_in=ss_in, out=out)
    (m, h), n = hidden.shape, w_qkv.shape[0]
    a = _qkv_args(hidden, norm_weight, n, h, cos, sin, a0["eps"], rope_cols, bias, out)
    code = DTYPE_CODE[hidden.dtype]
    check("fd_pre_attn_qkv_fp8_sumsq", lib().fd_pre_attn_qkv_fp8_sumsq(
        _p(a.out), _p(hidden), _p(norm_weight), DTYPE_CODE[norm_weight.dtype], _p(w_qkv), _p(scale), _p(bias),
        DTYPE_CODE[bias.dtype] if bias is not None else code, _p(a.cos), _p(a.sin), DTYPE_CODE[a.cos.dtype],
        a.cs_row_stride, m, h, n, a.rope_cols, a.d, a.eps, code, _p(ss_in), (h + 15) // 16,
        ctypes.c_void_p(stream_of(hidden))))
    return a.out
