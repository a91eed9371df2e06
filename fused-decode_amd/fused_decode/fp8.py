"""FP8 (OCP E4M3) weights for the decode GEMV and the post-attention MLP.

    q, scale = quantize_fp8(w)                        # [N, K] -> e4m3 codes + float32 [N]
    y = linear_decode_fp8(x, q, scale, bias, row_add=r)
    y = post_attn_mlp_fp8(hidden, norm_w, q_gu, s_gu, q_d, s_d, eps)
    y = pre_attn_qkv_fp8(hidden, norm_w, q_qkv, s_qkv, cos, sin, eps, rope_cols=c)

Per-output-channel quantisation: scale[n] = max|w[n, :]| * (1/448) and the codes are
w / scale rounded to nearest-even E4M3 (torch's float8_e4m3fn cast). The HIP
kernels decode the codes exactly and compute in float32 with fp16/bf16
activations, so the only approximation is the weight quantisation itself:

    y[m, n] = round(scale[n] * sum_k e4m3(q[n, k]) * x[m, k] + bias[n] + row_add[m, n])

A decode GEMV at M <= 16 streams one byte per weight instead of two. There is no
reference counterpart (the reference has fp16/bf16 weights only); this is the
low-precision weight format its roadmap leaves for last.
"""

from __future__ import annotations

import torch

from . import _lib
from ._lib import DTYPE_CODE, check, lib, stream_of
from .ops import (
    _as_mk,
    _as_row_add,
    _check_activation,
    _check_eps,
    _check_norm_weight,
    _qkv_args,
    _rope_qkv_heads,
    rms_norm,
    swiglu,
)

FP8_MAX = 448.0
FP8_DTYPE = torch.float8_e4m3fn
_HAND_LIMIT = 16
_FP8_MFMA_MIN_M = 5  # rows from which the fp8 kernels run on MFMA (fp8.hip)


def quantize_fp8(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """``[N, K]`` float weight -> (E4M3 codes ``[N, K]`` as ``torch.float8_e4m3fn``,
    float32 per-row scales ``[N]``). An all-zero row gets scale 1."""
    if not isinstance(weight, torch.Tensor) or weight.ndim != 2:
        raise ValueError("weight must be a rank-2 tensor [N, K]")
    if not weight.is_floating_point():
        raise TypeError("weight must be a floating-point tensor")
    w = weight.float()
    amax = w.abs().amax(dim=1)
    # a multiply by the float32 reciprocal, which every device rounds the same way
    # (torch divides by a scalar as a multiply on GPUs but exactly on CPUs)
    scale = torch.where(amax > 0, amax * (1.0 / FP8_MAX), torch.ones_like(amax))
    codes = (w / scale[:, None]).clamp(-FP8_MAX, FP8_MAX).to(FP8_DTYPE)
    return codes.contiguous(), scale.contiguous()


def dequantize_fp8(codes: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """float32 ``scale[n] * e4m3(codes[n, k])``."""
    return codes.float() * scale.float()[:, None]


def _check_fp8_weight(weight: torch.Tensor, scale: torch.Tensor, like: torch.Tensor, name: str) -> None:
    if weight.dtype != FP8_DTYPE:
        raise TypeError(f"{name} must be torch.float8_e4m3fn codes (see quantize_fp8)")
    if weight.ndim != 2:
        raise ValueError(f"{name} must have shape [N, K], got {tuple(weight.shape)}")
    if scale.dtype != torch.float32 or scale.ndim != 1 or scale.shape[0] != weight.shape[0]:
        raise ValueError(f"{name} scale must be float32 of shape ({weight.shape[0]},)")
    if weight.device != like.device or scale.device != like.device:
        raise ValueError(f"{name} and its scale must be on {like.device}")


def _fp8_rows_ok(weight: torch.Tensor) -> bool:
    return weight.stride(1) == 1 and (weight.shape[0] == 1 or weight.stride(0) % 16 == 0) \
        and weight.shape[1] % 16 == 0 and weight.data_ptr() % 16 == 0


def _decoded_product(x2, weight, scale, bias, ra, dtype):
    """float32 product of the decoded weights, for shapes the HIP kernel does not take."""
    y = (x2.float() @ weight.float().t()) * scale
    if bias is not None:
        y = y + bias.float()
    if ra is not None:
        y = y + ra.float()
    return y.to(dtype)


def linear_decode_fp8(
    x: torch.Tensor,
    weight: torch.Tensor,
    scale: torch.Tensor,
    bias: torch.Tensor | None = None,
    *,
    row_add: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """``y = (x @ dequantize(weight, scale).T) (+ bias) (+ row_add)`` with E4M3
    ``weight [N, K]`` and float32 ``scale [N]``; argument rules as
    ``linear_decode`` (ops.py:212-280 of the reference). Up to 16 rows with
    ``K % 16 == 0`` this is the HIP fp8 GEMV; otherwise a float32 product of the
    decoded weights (same values, slower)."""
    _check_activation(x, "x")
    _check_fp8_weight(weight, scale, x, "weight")
    n, k = weight.shape
    if x.shape[-1] != k:
        raise ValueError(f"x last dim {x.shape[-1]} != weight K {k}")
    x2, leading = _as_mk(x)
    m = x2.shape[0]
    expected = (n,) if leading is None else (*leading, n)
    if bias is not None:
        if bias.ndim != 1 or bias.shape[0] != n:
            raise ValueError(f"bias must have shape ({n},), got {tuple(bias.shape)}")
        if bias.device != x.device:
            raise ValueError("bias must be on the same device as x")
        if bias.dtype not in (x.dtype, torch.float32):
            raise TypeError("bias must match x or be float32")
    ra = None
    if row_add is not None:
        if row_add.device != x.device:
            raise ValueError("row_add must be on the same device as x")
        ra = _as_row_add(row_add, m, n, expected)
    if out is None:
        out = torch.empty(expected, device=x.device, dtype=x.dtype)
    elif tuple(out.shape) != expected or out.dtype != x.dtype or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous {expected} tensor of dtype {x.dtype}")
    y2 = out.view(m, n)
    if m == 0 or n == 0:
        return out
    if m > _HAND_LIMIT or not _fp8_rows_ok(weight) or x2.stride(1) != 1 or \
            (m > 1 and x2.stride(0) % 8 != 0) or x2.data_ptr() % 16 != 0:
        y2.copy_(_decoded_product(x2, weight, scale, bias, ra, x.dtype))
        return out
    bias_ptr, bias_code, sb = None, DTYPE_CODE[x.dtype], 0
    if bias is not None:
        bias_ptr, bias_code, sb = bias.data_ptr(), DTYPE_CODE[bias.dtype], int(bias.stride(0))
    row_ptr, row_code, srm, srn = None, DTYPE_CODE[x.dtype], 0, 0
    if ra is not None:
        row_ptr, row_code = ra.data_ptr(), DTYPE_CODE[ra.dtype]
        srm = 0 if ra.shape[0] == 1 else int(ra.stride(0))
        srn = 0 if ra.shape[1] == 1 else int(ra.stride(1))
    sc = scale if scale.is_contiguous() else scale.contiguous()
    status = lib().fd_linear_fp8(
        y2.data_ptr(), x2.data_ptr(), weight.data_ptr(), sc.data_ptr(), bias_ptr, bias_code,
        row_ptr, row_code, m, n, k, int(x2.stride(0)), int(weight.stride(0)), sb, srm, srn,
        int(y2.stride(0)), int(y2.stride(1)), DTYPE_CODE[x.dtype], stream_of(x),
    )
    check("fd_linear_fp8", status)
    return out


def post_attn_mlp_fp8(
    hidden: torch.Tensor,
    norm_weight: torch.Tensor,
    w_gate_up: torch.Tensor,
    gate_up_scale: torch.Tensor,
    w_down: torch.Tensor,
    down_scale: torch.Tensor,
    eps: float = 1e-6,
) -> torch.Tensor:
    """``post_attn_mlp`` with E4M3 weights (``w_gate_up [2I, H]``, ``w_down [H, I]``)
    and their float32 per-row scales: the same four rounding points (reference
    reference.py:66-79), each projection as ``linear_decode_fp8``. Two HIP launches
    up to 16 rows; otherwise composed from the operators."""
    _check_activation(hidden, "hidden")
    _check_fp8_weight(w_gate_up, gate_up_scale, hidden, "w_gate_up")
    _check_fp8_weight(w_down, down_scale, hidden, "w_down")
    two_i, h = w_gate_up.shape
    h_down, i = w_down.shape
    if two_i != 2 * i or h != h_down or hidden.shape[-1] != h:
        raise ValueError(
            f"expected w_gate_up [2I, H] and w_down [H, I] with hidden [..., H], "
            f"got {tuple(w_gate_up.shape)}, {tuple(w_down.shape)}, {tuple(hidden.shape)}"
        )
    _check_norm_weight(norm_weight, hidden)
    eps = _check_eps(eps)
    m = hidden.numel() // h if h else 0
    if 0 < m <= _HAND_LIMIT and w_gate_up.is_contiguous() and w_down.is_contiguous() \
            and h % 16 == 0 and i % 16 == 0:
        h2 = hidden.reshape(m, h)
        if not h2.is_contiguous():
            h2 = h2.contiguous()
        nw = norm_weight if norm_weight.is_contiguous() else norm_weight.contiguous()
        y = torch.empty((m, h), device=hidden.device, dtype=hidden.dtype)
        mid = torch.empty((m, i), device=hidden.device, dtype=hidden.dtype)
        status = lib().fd_post_attn_mlp_fp8(
            y.data_ptr(), mid.data_ptr(), h2.data_ptr(), nw.data_ptr(), DTYPE_CODE[nw.dtype],
            w_gate_up.data_ptr(), gate_up_scale.contiguous().data_ptr(), w_down.data_ptr(),
            down_scale.contiguous().data_ptr(), m, h, i, float(eps), DTYPE_CODE[hidden.dtype],
            stream_of(hidden),
        )
        if status != _lib.FD_EUNSUPPORTED:
            check("fd_post_attn_mlp_fp8", status)
            return y.view(hidden.shape)
    normed = rms_norm(hidden, norm_weight, eps=eps)
    gate_up = linear_decode_fp8(normed, w_gate_up, gate_up_scale)
    gate, up = gate_up.split(i, dim=-1)
    return linear_decode_fp8(swiglu(gate, up), w_down, down_scale, row_add=hidden)


def pre_attn_qkv_fp8(
    hidden: torch.Tensor,
    norm_weight: torch.Tensor,
    w_qkv: torch.Tensor,
    scale: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    eps: float = 1e-6,
    *,
    rope_cols: int,
    bias: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """``pre_attn_qkv`` with E4M3 ``w_qkv [N, H]`` and its float32 per-row
    ``scale [N]``: RMSNorm, the projection as ``linear_decode_fp8``'s product (plus
    ``bias``), rounding, then RoPE of the first ``rope_cols`` columns, with the
    argument rules of ``pre_attn_qkv``. One HIP launch up to 4 rows, two up to 16
    (the norm runs as a row kernel ahead of the MFMA form); otherwise, or for
    shapes the kernels do not take, composed from the operators."""
    _check_activation(hidden, "hidden")
    _check_fp8_weight(w_qkv, scale, hidden, "w_qkv")
    n, h = w_qkv.shape
    a = _qkv_args(hidden, norm_weight, n, h, cos, sin, eps, rope_cols, bias, out)
    out, m = a.out, a.m
    if m == 0 or n == 0:
        return out
    if m <= _HAND_LIMIT and w_qkv.is_contiguous() and h % 16 == 0:
        h2 = hidden.reshape(m, h)
        if not h2.is_contiguous():
            h2 = h2.contiguous()
        nw = norm_weight if norm_weight.is_contiguous() else norm_weight.contiguous()
        b = bias if bias is None or bias.is_contiguous() else bias.contiguous()
        normed = None
        if m >= _FP8_MFMA_MIN_M:
            normed = torch.empty((m, h), device=hidden.device, dtype=hidden.dtype)
        status = lib().fd_pre_attn_qkv_fp8(
            out.data_ptr(), normed.data_ptr() if normed is not None else None, h2.data_ptr(),
            nw.data_ptr(), DTYPE_CODE[nw.dtype], w_qkv.data_ptr(), scale.contiguous().data_ptr(),
            b.data_ptr() if b is not None else None,
            DTYPE_CODE[b.dtype] if b is not None else DTYPE_CODE[hidden.dtype],
            a.cos.data_ptr(), a.sin.data_ptr(), DTYPE_CODE[a.cos.dtype], a.cs_row_stride, m, h, n,
            a.rope_cols, a.d, float(a.eps), DTYPE_CODE[hidden.dtype], stream_of(hidden),
        )
        if status != _lib.FD_EUNSUPPORTED:
            check("fd_pre_attn_qkv_fp8", status)
            return out
    normed = rms_norm(hidden, norm_weight, eps=a.eps)
    linear_decode_fp8(normed, w_qkv, scale, bias, out=out)
    _rope_qkv_heads(a)
    return out


__all__ = ["FP8_MAX", "dequantize_fp8", "linear_decode_fp8", "post_attn_mlp_fp8", "pre_attn_qkv_fp8",
           "quantize_fp8"]
