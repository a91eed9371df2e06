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

import math
import warnings

import torch

from . import _lib
from ._checks import check
from ._lib import DTYPE_CODE, fail, native
from .ops import (_FP8_ROWS, _PLANS, _check_out, _dense, _empty, _plan_qkv, _raw_stream, _remember, _row_add_rows,
                  _sig, rms_norm, swiglu)

FP8_MAX = 448.0
FP8_DTYPE = torch.float8_e4m3fn
_HAND_LIMIT = _FP8_ROWS
_FP8_MFMA_MIN_M = 5  # rows from which the fp8 kernels run on MFMA (fp8.hip)
_warned: set[str] = set()


def _slow_path(why: str) -> None:
    """The decoded float32 product streams 4x the code bytes: say so, once per reason."""
    if why not in _warned:
        _warned.add(why)
        warnings.warn(f"linear_decode_fp8: {why}; computing a float32 product of the decoded weights "
                      "(same values, about 4x the weight traffic of the fp8 kernels)", RuntimeWarning,
                      stacklevel=5)  # _slow_path, the plan's helper, the plan, linear_decode_fp8, its caller


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
    ``K % 16 == 0`` this is the HIP fp8 GEMV; other shapes compute a float32
    product of the decoded weights (same values, several times the traffic: a
    RuntimeWarning says so once per reason)."""
    try:
        key = ("linear_fp8", _sig(x), _sig(weight), _sig(scale), _sig(bias), _sig(row_add), _sig(out))
        plan = _PLANS.get(key)
    except AttributeError:  # a non-tensor argument: checked below
        key, plan = None, None
    if plan is None:
        plan = _remember(key, _plan_linear_fp8(x, weight, scale, bias, row_add, out))
    return plan(x, weight, scale, bias, row_add, out)


def _plan_linear_fp8(x, weight, scale, bias, row_add, out):
    """Launch plan of ``linear_decode_fp8`` for one argument signature: the
    contract's checks and the shape rules of the kernel run once; each call
    checks only the two pointers whose alignment the signature leaves open."""
    check("linear_decode_fp8", x=x, weight=weight, scale=scale, bias=bias, row_add=row_add)
    n, k = (int(d) for d in weight.shape)
    m = 1 if x.ndim == 1 else math.prod(x.shape[:-1])
    expected = (n,) if x.ndim == 1 else (*x.shape[:-1], n)
    ra = None if row_add is None else _row_add_rows(row_add, m, n, expected)
    if out is not None:
        _check_out(out, expected, x)
    alloc = _empty(expected, x)
    if m == 0 or n == 0:
        return lambda x, w, sc, b, r, o: alloc(x) if o is None else o

    def slow(x2, w, sc, b, r, y, why):
        _slow_path(why)
        p = (x2.float() @ w.float().t()) * sc
        if b is not None:
            p = p + b.float()
        if r is not None:
            p = p + r.expand(expected).reshape(m, n).float()
        y.view(m, n).copy_(p.to(x2.dtype))
        return y

    x2p = x.reshape(m, k)
    x_copy = x2p.stride(1) != 1  # gathered per call into contiguous rows
    why = None
    if m > _HAND_LIMIT:
        why = f"{m} rows is above the kernels' {_HAND_LIMIT}"
    elif not (weight.stride(1) == 1 and (n == 1 or weight.stride(0) % 16 == 0) and k % 16 == 0):
        why = "the codes are not 16-byte rows with K % 16 == 0"
    elif not x_copy and m > 1 and x2p.stride(0) % 8 != 0:
        why = "x rows are not 16-byte aligned with unit stride"
    if why is not None:
        def fallback(x, w, sc, b, r, o):
            x2 = x.reshape(m, k)
            return slow(x2.contiguous() if x_copy else x2, w, sc, b, r, alloc(x) if o is None else o, why)
        return fallback

    act, dev = DTYPE_CODE[x.dtype], x.device.index
    bcode = act if bias is None else DTYPE_CODE[bias.dtype]
    sb = 0 if bias is None else int(bias.stride(0))
    rcode = act if row_add is None else DTYPE_CODE[row_add.dtype]
    srm, srn, r_flat = ra if ra is not None else (0, 0, False)
    dense_sc = _dense(scale)
    sxm = k if x_copy else int(x2p.stride(0))
    call = native().linear_fp8

    def run(x, w, sc, b, r, o):
        y = alloc(x) if o is None else o
        x2 = x.reshape(m, k)
        if x_copy:
            x2 = x2.contiguous()
        if w.data_ptr() % 16:
            return slow(x2, w, sc, b, r, y, "the codes are not 16-byte rows with K % 16 == 0")
        if x2.data_ptr() % 16:
            return slow(x2, w, sc, b, r, y, "x rows are not 16-byte aligned with unit stride")
        if r is not None and r_flat:  # indexed in place through (srm, srn), or copied when its dims do not merge
            r = r.expand(expected).reshape(m, n)
        status = call(y.data_ptr(), x2.data_ptr(), w.data_ptr(), (sc if dense_sc else sc.contiguous()).data_ptr(),
                      None if b is None else b.data_ptr(), bcode, None if r is None else r.data_ptr(), rcode,
                      m, n, k, sxm, int(w.stride(0)), sb, srm, srn, n, 1, act, _raw_stream(dev))
        if status:
            fail("fd_linear_fp8", status)
        return y
    return run


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
    up to 16 rows (from 5 the MFMA gate/up normalises inside its kernel);
    otherwise composed from the operators."""
    try:
        key = ("mlp_fp8", _sig(hidden), _sig(norm_weight), _sig(w_gate_up), _sig(gate_up_scale), _sig(w_down),
               _sig(down_scale), eps)
        plan = _PLANS.get(key)
    except (AttributeError, TypeError):  # a non-tensor or unhashable argument: checked below
        key, plan = None, None
    if plan is None:
        plan = _remember(key, _plan_mlp_fp8(hidden, norm_weight, w_gate_up, gate_up_scale, w_down, down_scale, eps))
    return plan(hidden, norm_weight, w_gate_up, gate_up_scale, w_down, down_scale)


def _plan_mlp_fp8(hidden, norm_weight, w_gate_up, gate_up_scale, w_down, down_scale, eps):
    """Launch plan of ``post_attn_mlp_fp8`` for one argument signature."""
    a = check("post_attn_mlp_fp8", hidden=hidden, norm_weight=norm_weight, w_gate_up=w_gate_up,
              gate_up_scale=gate_up_scale, w_down=w_down, down_scale=down_scale, eps=eps)
    eps = a["eps"]
    h, i = int(w_gate_up.shape[1]), int(w_down.shape[1])
    m = hidden.numel() // h if h else 0

    def composed(x, nw, wgu, sgu, wd, sd):
        normed = rms_norm(x, nw, eps=eps)
        gate, up = linear_decode_fp8(normed, wgu, sgu).split(i, dim=-1)
        return linear_decode_fp8(swiglu(gate, up), wd, sd, row_add=x)

    if not (0 < m <= _HAND_LIMIT and w_gate_up.is_contiguous() and w_down.is_contiguous()
            and h % 16 == 0 and i % 16 == 0):
        return composed
    shape = tuple(hidden.shape)
    dense_h, dense_nw, dense_s = _dense(hidden), _dense(norm_weight), _dense(gate_up_scale) and _dense(down_scale)
    call, act, nwc, dev = (native().post_attn_mlp_fp8, DTYPE_CODE[hidden.dtype], DTYPE_CODE[norm_weight.dtype],
                           hidden.device.index)

    def fused(x, nw, wgu, sgu, wd, sd):
        x2 = x if dense_h else x.contiguous()
        nw2 = nw if dense_nw else nw.contiguous()
        if not dense_s:
            sgu, sd = sgu.contiguous(), sd.contiguous()
        y = x2.new_empty((m, h))
        mid = x2.new_empty((m, i))
        status = call(y.data_ptr(), mid.data_ptr(), x2.data_ptr(), nw2.data_ptr(), nwc, wgu.data_ptr(),
                      sgu.data_ptr(), wd.data_ptr(), sd.data_ptr(), m, h, i, eps, act, _raw_stream(dev))
        if status == _lib.FD_EUNSUPPORTED:  # e.g. an unaligned operand or a hidden width beyond the LDS
            return composed(x, nw, wgu, sgu, wd, sd)
        if status:
            fail("fd_post_attn_mlp_fp8", status)
        return y.view(shape)
    return fused


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
    argument rules of ``pre_attn_qkv``. One HIP launch up to 16 rows (from 5 the
    MFMA form with the norm folded in); otherwise, or for shapes the kernels do
    not take, composed from the operators."""
    try:
        key = ("qkv_fp8", _sig(hidden), _sig(norm_weight), _sig(w_qkv), _sig(scale), _sig(cos), _sig(sin), eps,
               rope_cols, _sig(bias), _sig(out))
        plan = _PLANS.get(key)
    except (AttributeError, TypeError):  # a non-tensor or unhashable argument: checked below
        key, plan = None, None
    if plan is None:
        plan = _remember(key, _plan_qkv(hidden, norm_weight, w_qkv, scale, cos, sin, eps, rope_cols, bias, out,
                                        None))
    return plan(hidden, norm_weight, w_qkv, scale, cos, sin, bias, out)


__all__ = ["FP8_MAX", "dequantize_fp8", "linear_decode_fp8", "post_attn_mlp_fp8", "pre_attn_qkv_fp8",
           "quantize_fp8"]
