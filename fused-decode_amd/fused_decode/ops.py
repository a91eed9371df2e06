"""Public operators (drop-in for the reference's src/fused_decode/ops.py).

Inference only: these launches record no backward. Signatures, argument
checks, exception types and message keywords follow the reference
(ops.py:34-69 validation, :72-315 operators); the device work is the gfx950 HIP
library behind ``kernels``. ``linear_decode`` uses the hand-written GEMV up to
``DECODE_LINEAR_MAX_M`` rows by default and ``F.linear`` (hipBLASLt) above it;
passing ``kind`` forces the GEMV up to 16 rows, as in the reference.
"""

from __future__ import annotations

import math
from typing import NamedTuple

import torch
import torch.nn.functional as F

from . import _lib
from .kernels import (
    _MFMA_MIN_M,
    linear_out,
    post_attn_mlp_out,
    pre_attn_qkv_out,
    resolve_kind,
    rms_out,
    rope_out,
    swiglu_out,
)

# Largest flattened batch the default dispatcher sends to the HIP GEMV. The
# reference sets this per GPU from measurement (its RTX 4070 Laptop value is 1,
# ops.py:16-19); for MI355X it is the `decode_linear_max_m` of the tile search
# (python -m fused_decode.bench --tune, table in tiles_gfx950.json): at every row
# count up to 16 the four GEMVs of a Llama-3-8B layer run faster in sum than
# hipBLASLt's F.linear, none of them more than 5% slower (each strictly faster
# up to 14 rows), so the HIP GEMV is the default over the whole hand range.
DECODE_LINEAR_MAX_M = 16
_HAND_LIMIT = 16
_ACTIVATION = (torch.float16, torch.bfloat16)
_NORM_WEIGHT = (torch.float16, torch.bfloat16, torch.float32)

__all__ = [
    "DECODE_LINEAR_MAX_M",
    "add_rms_norm",
    "linear_decode",
    "post_attn_mlp",
    "pre_attn_qkv",
    "rms_norm",
    "rope",
    "swiglu",
]


def _check_activation(t: torch.Tensor, name: str) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a CUDA tensor")
    if t.dtype not in _ACTIVATION:
        raise TypeError(f"{name} must be float16 or bfloat16, got {t.dtype}")


def _check_same(t: torch.Tensor, like: torch.Tensor, name: str) -> None:
    if t.shape != like.shape:
        raise ValueError(f"{name} shape {tuple(t.shape)} != {tuple(like.shape)}")
    if t.dtype != like.dtype:
        raise TypeError(f"{name} dtype {t.dtype} != {like.dtype}")
    if t.device != like.device:
        raise ValueError(f"{name} is on {t.device}, expected {like.device}")


def _check_norm_weight(weight: torch.Tensor, x: torch.Tensor) -> None:
    if weight.device != x.device:
        raise ValueError(f"weight is on {weight.device}, expected {x.device}")
    if weight.dtype not in _NORM_WEIGHT:
        raise TypeError("weight must be float16, bfloat16, or float32")
    if weight.ndim != 1 or weight.shape[0] != x.shape[-1]:
        raise ValueError(f"weight must have shape ({x.shape[-1]},), got {tuple(weight.shape)}")


def _check_eps(eps: float) -> float:
    eps = float(eps)
    if not math.isfinite(eps) or eps < 0:
        raise ValueError("eps must be a finite value >= 0")
    return eps


def _check_out(out: torch.Tensor, like: torch.Tensor) -> None:
    _check_same(out, like, "out")


def rms_norm(
    x: torch.Tensor,
    weight: torch.Tensor,
    eps: float = 1e-6,
    *,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """RMSNorm over the last dimension with a float32 reduction. ``weight`` is ``(N,)``
    (float16, bfloat16 or float32). Reference: ops.py:72-88."""
    _check_activation(x, "x")
    _check_norm_weight(weight, x)
    eps = _check_eps(eps)
    if out is None:
        out = torch.empty(x.shape, device=x.device, dtype=x.dtype)
    else:
        _check_out(out, x)
    rms_out(x, weight, eps, out)
    return out


def add_rms_norm(
    x: torch.Tensor,
    residual: torch.Tensor,
    weight: torch.Tensor,
    eps: float = 1e-6,
    *,
    out: torch.Tensor | None = None,
    residual_out: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """``residual_out = x + residual``, then RMSNorm of the float32 sum (not of the
    rounded stored residual). ``residual_out=residual`` updates the residual
    stream in place. Reference: ops.py:91-119."""
    _check_activation(x, "x")
    _check_activation(residual, "residual")
    _check_same(residual, x, "residual")
    _check_norm_weight(weight, x)
    eps = _check_eps(eps)
    if out is None:
        out = torch.empty(x.shape, device=x.device, dtype=x.dtype)
    else:
        _check_out(out, x)
    if residual_out is None:
        residual_out = torch.empty(x.shape, device=x.device, dtype=x.dtype)
    else:
        _check_same(residual_out, x, "residual_out")
    rms_out(x, weight, eps, out, residual=residual, residual_out=residual_out)
    return out, residual_out


def _broadcast_angles(src: torch.Tensor, like: torch.Tensor, name: str) -> torch.Tensor:
    """Broadcast like PyTorch (shapes align on the right). Reference: ops.py:122-135."""
    if src.device != like.device:
        raise ValueError(f"{name} is on {src.device}, expected {like.device}")
    if src.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise TypeError(f"{name} must be float16, bfloat16, or float32")
    if src.shape[-1] != like.shape[-1]:
        raise ValueError(f"{name} last dim {src.shape[-1]} != x last dim {like.shape[-1]}")
    try:
        return src.expand(like.shape)
    except RuntimeError as exc:
        raise ValueError(
            f"cannot broadcast {name} shape {tuple(src.shape)} to {tuple(like.shape)}"
        ) from exc


def rope(
    x: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    *,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Llama rotate-half RoPE on the last dimension (GPT-NeoX pairing, not GPT-J
    interleaved pairs). ``cos``/``sin`` broadcast over leading dims.
    Reference: ops.py:138-160."""
    _check_activation(x, "x")
    if x.shape[-1] % 2 != 0:
        raise ValueError("rope last dimension must be even")
    cos_b = _broadcast_angles(cos, x, "cos")
    sin_b = _broadcast_angles(sin, x, "sin")
    if out is None:
        out = torch.empty(x.shape, device=x.device, dtype=x.dtype)
    else:
        _check_out(out, x)
    rope_out(x, cos_b, sin_b, out)
    return out


def swiglu(
    gate: torch.Tensor,
    up: torch.Tensor,
    *,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """``silu(gate) * up`` in float32, stored in ``gate.dtype``. Reference: ops.py:163-178."""
    _check_activation(gate, "gate")
    _check_activation(up, "up")
    _check_same(up, gate, "up")
    if out is None:
        out = torch.empty(gate.shape, device=gate.device, dtype=gate.dtype)
    else:
        _check_out(out, gate)
    swiglu_out(gate, up, out)
    return out


def _as_mk(x: torch.Tensor) -> tuple[torch.Tensor, tuple[int, ...] | None]:
    """Flatten x to ``[M, K]``; 2-D strided x passes through. Reference: ops.py:181-192."""
    k = x.shape[-1]
    if x.ndim == 1:
        if not x.is_contiguous():
            x = x.contiguous()
        return x.view(1, k), None
    leading = tuple(x.shape[:-1])
    if x.ndim == 2 and x.stride(0) >= 0 and x.stride(1) >= 0:
        return x, leading
    if not x.is_contiguous():
        x = x.contiguous()
    return x.view(-1, k), leading


def _as_row_add(row_add: torch.Tensor, m: int, n: int, expected: tuple[int, ...]) -> torch.Tensor:
    """row_add as ``[M, N]``-indexable (size-1 dims broadcast). Reference: ops.py:195-209."""
    if row_add.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise TypeError("row_add must be float16, bfloat16, or float32")
    if row_add.ndim == 1 and row_add.numel() == n:
        return row_add.view(1, n)
    if row_add.shape == torch.Size(expected) and row_add.is_contiguous():
        return row_add.view(m, n)
    if row_add.ndim == 2 and row_add.shape[0] in (1, m) and row_add.shape[1] in (1, n):
        return row_add
    try:
        return row_add.expand(expected).contiguous().view(m, n)
    except RuntimeError as exc:
        raise ValueError(
            f"row_add shape {tuple(row_add.shape)} is not broadcastable to {expected}"
        ) from exc


def linear_decode(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None = None,
    *,
    row_add: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    kind: str | None = None,
) -> torch.Tensor:
    """``y = x @ weight.T + bias (+ row_add)``, weight ``[N, K]`` like ``F.linear``.

    The HIP GEMV runs for a flattened batch up to ``DECODE_LINEAR_MAX_M`` rows,
    or up to 16 when ``kind`` ("dot" or "simt") is given; wider batches call
    ``F.linear`` (bit-identical to it), with row_add added in float32.
    Reference: ops.py:212-280.
    """
    _check_activation(x, "x")
    if weight.ndim != 2:
        raise ValueError(f"weight must have shape [N, K], got {tuple(weight.shape)}")
    if weight.device != x.device or weight.dtype != x.dtype:
        raise ValueError("weight device and dtype must match x")
    n, k = weight.shape
    if x.shape[-1] != k:
        raise ValueError(f"x last dim {x.shape[-1]} != weight K {k}")
    hand_limit = _HAND_LIMIT if kind is not None else DECODE_LINEAR_MAX_M
    kind = resolve_kind(kind)
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
    if m > hand_limit and out is None:
        produced = F.linear(x2, weight, bias)
        if ra is not None:
            produced = (produced.float() + ra.float()).to(dtype=x.dtype)
        if x.ndim == 1:
            return produced.view(n)
        return produced.view(expected)
    if out is None:
        y_full = torch.empty(expected, device=x.device, dtype=x.dtype)
    else:
        if tuple(out.shape) != expected or out.dtype != x.dtype or out.device != x.device:
            raise ValueError(f"out must be a contiguous {expected} tensor of dtype {x.dtype}")
        if not out.is_contiguous():
            raise ValueError("out must be contiguous")
        y_full = out
    y2 = y_full.view(m, n)
    if m == 0 or n == 0:
        return y_full
    if m > hand_limit:
        produced = F.linear(x2, weight, bias)
        if ra is not None:
            produced = (produced.float() + ra.float()).to(dtype=x.dtype)
        y2.copy_(produced)
        return y_full
    linear_out(x2, weight, y2, bias=bias, row_add=ra, kind=kind)
    return y_full


def post_attn_mlp(
    hidden: torch.Tensor,
    norm_weight: torch.Tensor,
    w_gate_up: torch.Tensor,
    w_down: torch.Tensor,
    eps: float = 1e-6,
    *,
    kind: str | None = None,
) -> torch.Tensor:
    """Llama post-attention block without the attention.

    ``hidden`` is ``[..., H]``, ``w_gate_up`` is ``[2I, H]`` (gate rows above up
    rows), ``w_down`` is ``[H, I]``. Returns ``down(swiglu(gate_up(rms(hidden)))) +
    hidden``, each intermediate rounded to the activation dtype. Up to the GEMV
    row limit this is two HIP launches: norm + gate/up GEMV + SwiGLU fused, then
    the down GEMV with the residual fused. Reference: ops.py:283-315.
    """
    _check_activation(hidden, "hidden")
    if w_gate_up.ndim != 2 or w_down.ndim != 2:
        raise ValueError("w_gate_up and w_down must be rank-2")
    two_i, h = w_gate_up.shape
    h_down, i = w_down.shape
    if two_i != 2 * i or h != h_down or hidden.shape[-1] != h:
        raise ValueError(
            f"expected w_gate_up [2I, H] and w_down [H, I] with hidden [..., H], "
            f"got {tuple(w_gate_up.shape)}, {tuple(w_down.shape)}, {tuple(hidden.shape)}"
        )
    if w_gate_up.dtype != hidden.dtype or w_down.dtype != hidden.dtype:
        raise TypeError("MLP weights must match hidden dtype")
    if w_gate_up.device != hidden.device or w_down.device != hidden.device:
        raise ValueError("MLP weights must be on the same device as hidden")
    _check_norm_weight(norm_weight, hidden)
    eps = _check_eps(eps)
    hand_limit = _HAND_LIMIT if kind is not None else DECODE_LINEAR_MAX_M
    kind_r = resolve_kind(kind)
    m = hidden.numel() // h if h else 0
    if 0 < m <= hand_limit and w_gate_up.is_contiguous() and w_down.is_contiguous():
        h2 = hidden.reshape(m, h)
        if not h2.is_contiguous():
            h2 = h2.contiguous()
        nw = norm_weight if norm_weight.is_contiguous() else norm_weight.contiguous()
        y = torch.empty((m, h), device=hidden.device, dtype=hidden.dtype)
        mid = torch.empty((m, i), device=hidden.device, dtype=hidden.dtype)
        status = post_attn_mlp_out(h2, nw, w_gate_up, w_down, eps, y, mid, kind_r)
        if status == _lib.FD_OK:
            return y.view(hidden.shape)
    normed = rms_norm(hidden, norm_weight, eps=eps)
    gate_up = linear_decode(normed, w_gate_up, kind=kind)
    gate, up = gate_up.split(i, dim=-1)
    return linear_decode(swiglu(gate, up), w_down, row_add=hidden, kind=kind)


def _token_angles(src: torch.Tensor, lead: tuple, name: str) -> torch.Tensor:
    """cos/sin of ``pre_attn_qkv`` as ``[1 or M, D]`` contiguous rows: ``src``
    broadcasts to ``[*lead, D]`` (a size-1 heads axis before D is allowed)."""
    if not isinstance(src, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if src.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise TypeError(f"{name} must be float16, bfloat16, or float32")
    d = src.shape[-1]
    if src.ndim == len(lead) + 2 and src.shape[-2] == 1:
        src = src.squeeze(-2)
    if src.numel() == d:
        return src.reshape(1, d).contiguous()
    try:
        full = src.expand(*lead, d)
    except RuntimeError as exc:
        raise ValueError(
            f"cannot broadcast {name} shape {tuple(src.shape)} to {(*lead, d)}"
        ) from exc
    return full.reshape(-1, d).contiguous()


class _QkvArgs(NamedTuple):
    m: int
    n: int
    h: int
    d: int
    rope_cols: int
    eps: float
    cos: torch.Tensor  # [1 or m, d] contiguous rows
    sin: torch.Tensor
    cs_row_stride: int
    out: torch.Tensor


def _qkv_args(hidden, norm_weight, n, h, cos, sin, eps, rope_cols, bias, out) -> _QkvArgs:
    """Checks and operands shared by ``pre_attn_qkv`` and its fp8 form, for a
    projection of ``n`` rows over ``h`` (``hidden [..., h]``)."""
    if hidden.shape[-1] != h:
        raise ValueError(f"hidden last dim {hidden.shape[-1]} != w_qkv H {h}")
    _check_norm_weight(norm_weight, hidden)
    eps = _check_eps(eps)
    for name, t in (("cos", cos), ("sin", sin)):
        if isinstance(t, torch.Tensor) and t.device != hidden.device:
            raise ValueError(f"{name} is on {t.device}, expected {hidden.device}")
    rope_cols = int(rope_cols)
    d = cos.shape[-1]
    if sin.shape[-1] != d:
        raise ValueError(f"sin last dim {sin.shape[-1]} != cos last dim {d}")
    if d % 2 != 0:
        raise ValueError("rope head dimension must be even")
    if rope_cols < 0 or rope_cols > n or rope_cols % d != 0:
        raise ValueError(f"rope_cols must be a multiple of {d} in [0, {n}], got {rope_cols}")
    if bias is not None:
        if bias.ndim != 1 or bias.shape[0] != n:
            raise ValueError(f"bias must have shape ({n},), got {tuple(bias.shape)}")
        if bias.device != hidden.device:
            raise ValueError("bias must be on the same device as hidden")
        if bias.dtype not in (hidden.dtype, torch.float32):
            raise TypeError("bias must match hidden or be float32")
    lead = tuple(hidden.shape[:-1])
    cos_r = _token_angles(cos, lead, "cos")
    sin_r = _token_angles(sin, lead, "sin")
    if cos_r.dtype != sin_r.dtype:
        cos_r, sin_r = cos_r.float(), sin_r.float()
    expected = (*lead, n)
    if out is None:
        out = torch.empty(expected, device=hidden.device, dtype=hidden.dtype)
    else:
        if tuple(out.shape) != expected or out.dtype != hidden.dtype or out.device != hidden.device:
            raise ValueError(f"out must be a contiguous {expected} tensor of dtype {hidden.dtype}")
        if not out.is_contiguous():
            raise ValueError("out must be contiguous")
    m = hidden.numel() // h if h else 0
    if m and n and cos_r.shape[0] not in (1, m):
        raise ValueError(f"cos/sin need 1 or {m} rows, got {cos_r.shape[0]}")
    rs = 0 if cos_r.shape[0] == 1 else d
    return _QkvArgs(m, n, h, d, rope_cols, eps, cos_r, sin_r, rs, out)


def _rope_qkv_heads(a: _QkvArgs) -> None:
    """RoPE of the first ``rope_cols`` columns of ``a.out`` in place (the composed path)."""
    if a.rope_cols:
        heads = a.out.view(a.m, a.n)[:, : a.rope_cols].unflatten(-1, (a.rope_cols // a.d, a.d))
        rope(heads, a.cos.unsqueeze(1), a.sin.unsqueeze(1), out=heads)


def pre_attn_qkv(
    hidden: torch.Tensor,
    norm_weight: torch.Tensor,
    w_qkv: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    eps: float = 1e-6,
    *,
    rope_cols: int,
    bias: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    kind: str | None = None,
) -> torch.Tensor:
    """Pre-attention half of a Llama decode layer: RMSNorm, the fused QKV
    projection and RoPE of the q and k heads.

    ``hidden`` is ``[..., H]``, ``w_qkv`` is ``[N, H]`` (q, k, v rows stacked),
    ``bias`` is ``[N]`` (hidden's dtype or float32) or None. The first
    ``rope_cols`` output columns, viewed as heads of ``D = cos.shape[-1]``, get the
    rotate-half RoPE of ``rope`` with one cos/sin row per token: ``cos``/``sin``
    broadcast to ``[..., D]`` (``[D]`` or ``[1, D]`` for one position, ``[..., D]``
    or ``[..., 1, D]`` per token). Returns ``[..., N]`` equal to
    ``rope(linear_decode(rms_norm(hidden), w_qkv, bias)[..., :rope_cols])`` with
    the reference's rounding after each step. Up to the GEMV row limit this is one
    HIP launch (two for kind "dot" from 5 rows: the norm runs as a row kernel).
    No reference counterpart as one call; it composes ops.py:72-88, :212-280 and
    :138-160.
    """
    _check_activation(hidden, "hidden")
    if w_qkv.ndim != 2:
        raise ValueError(f"w_qkv must have shape [N, H], got {tuple(w_qkv.shape)}")
    n, h = w_qkv.shape
    if w_qkv.dtype != hidden.dtype:
        raise TypeError("w_qkv must match hidden dtype")
    if w_qkv.device != hidden.device:
        raise ValueError("w_qkv must be on the same device as hidden")
    a = _qkv_args(hidden, norm_weight, n, h, cos, sin, eps, rope_cols, bias, out)
    out, m, eps = a.out, a.m, a.eps
    if m == 0 or n == 0:
        return out
    hand_limit = _HAND_LIMIT if kind is not None else DECODE_LINEAR_MAX_M
    kind_r = resolve_kind(kind)
    if m <= hand_limit and w_qkv.is_contiguous():
        h2 = hidden.reshape(m, h)
        if not h2.is_contiguous():
            h2 = h2.contiguous()
        nw = norm_weight if norm_weight.is_contiguous() else norm_weight.contiguous()
        b = bias if bias is None or bias.is_contiguous() else bias.contiguous()
        normed = None
        if kind_r == "dot" and m >= _MFMA_MIN_M:
            normed = torch.empty((m, h), device=hidden.device, dtype=hidden.dtype)
        status = pre_attn_qkv_out(h2, nw, w_qkv, b, a.cos, a.sin, a.cs_row_stride, a.rope_cols,
                                  a.d, eps, out.view(m, n), normed, kind_r)
        if status == _lib.FD_OK:
            return out
    normed = rms_norm(hidden, norm_weight, eps=eps)
    linear_decode(normed, w_qkv, bias, out=out, kind=kind)
    _rope_qkv_heads(a)
    return out
