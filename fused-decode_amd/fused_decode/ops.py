"""Public operators (drop-in for the reference's src/fused_decode/ops.py).

Inference only: these launches record no backward. The signatures, defaults,
exception types and message keywords are the reference's (ops.py:72-315); the
argument rules live in ``_checks.CONTRACT`` and the device work in the gfx950
HIP library, reached through its CPython binding (``_lib.native()``).

Launch plans. At one token a kernel runs for 2-7 us, and a HIP launch alone
costs about 2.4 us of host time, so the rest of a call's host work has to stay
near a microsecond or the host, not the GPU, sets the pace of an eager decode
loop. Each call is therefore keyed by its argument signature: every tensor's
shape, strides, dtype and device, the scalars, and the environment variables
that steer dispatch (the reference reads them on every call, kernels.py:92,
:103, :583, :595, and so does the key). The first call with a signature checks
the arguments against the contract, resolves the kernel, tile, row layouts and
dtype codes, and stores a plan: a closure that allocates the outputs, reads the
data pointers and torch's current stream, and calls the library. Later calls
with that signature run the plan directly. Nothing in a plan depends on data
pointers (the library checks alignment and picks its vector or generic kernels
itself on every call).

``linear_decode`` uses the hand-written GEMV up to ``DECODE_LINEAR_MAX_M`` rows
by default (``SIMT_DECODE_LINEAR_MAX_M`` for kind "simt" chosen through the
environment) and ``F.linear`` (hipBLASLt) above it; passing ``kind`` forces the
GEMV up to 16 rows, as in the reference.
"""

from __future__ import annotations

import math
import os
from typing import Callable, NamedTuple

import torch
import torch.nn.functional as F

from . import _lib
from ._checks import check
from ._layout import contiguous_strides, plan_rows
from ._lib import DTYPE_CODE, FD_EUNSUPPORTED, KIND_CODE, FdTile, fail, native
from .kernels import (
    _rms_env,
    linear_config,
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
# hipBLASLt's F.linear, each of them strictly faster, so the HIP GEMV is the
# default over the whole hand range.
DECODE_LINEAR_MAX_M = 16
# The same cutoff for the SIMT kernel, which the default dispatcher runs when
# FUSED_DECODE_LINEAR_KIND selects kind "simt", by the same rule: from 9 rows its
# v_dot2 work on the down projection (K = 14336, whose activations the
# persistent kernel then holds in two phases) makes it no faster than F.linear
# (M = 9: 26.07 against 26.06 us, M = 10: 26.99 against 26.06, within the 5%
# band; M = 11: 28.12 against 26.16, beyond it), so the default stops at 10. A
# caller that names the kind still gets the SIMT kernel up to 16 rows, as in the
# reference.
SIMT_DECODE_LINEAR_MAX_M = 10
_FORCED_LIMIT = 16  # rows the GEMV takes when the caller names a kind
_FP8_ROWS = 16  # rows the E4M3 kernels take

__all__ = [
    "DECODE_LINEAR_MAX_M",
    "SIMT_DECODE_LINEAR_MAX_M",
    "add_rms_norm",
    "linear_decode",
    "post_attn_mlp",
    "pre_attn_qkv",
    "rms_norm",
    "rope",
    "swiglu",
]

# ------------------------------------------------------------------ plans

Plan = Callable[..., object]
_PLANS: dict[tuple, Plan] = {}
_PLAN_LIMIT = 4096
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None) or _lib.stream_of_device


def _remember(key, plan: Plan) -> Plan:
    if key is not None:
        if len(_PLANS) >= _PLAN_LIMIT:
            _PLANS.clear()
        _PLANS[key] = plan
    return plan


def clear_plans() -> None:
    """Forget every cached launch plan (the next call per signature re-checks)."""
    _PLANS.clear()


def _sig(t):
    """Signature of an optional tensor argument (the device as its index: -1 is the CPU)."""
    return None if t is None else (t.shape, t.stride(), t.dtype, t.get_device())


# os.environ keeps its values in a bytes-keyed dict on POSIX; reading that dict
# costs a dict lookup where os.environ.get costs an encode and, for an unset
# variable, a raised KeyError.
_ENV_DATA = getattr(os.environ, "_data", None)


def _env(name: str, _keys: dict = {}):  # noqa: B006 (a per-process key cache)
    if _ENV_DATA is None:
        return os.environ.get(name)
    key = _keys.get(name)
    if key is None:
        key = _keys[name] = os.environ.encodekey(name)
    return _ENV_DATA.get(key)


def _dense(t: torch.Tensor) -> bool:
    return t.is_contiguous()


def _empty(shape, like: torch.Tensor) -> Callable[[torch.Tensor], torch.Tensor]:
    """Allocator of a contiguous output of ``shape`` in ``like``'s dtype/device:
    ``empty_like`` when that is the same thing (the cheapest torch allocation)."""
    shape = tuple(shape)
    if _dense(like) and tuple(like.shape) == shape:
        return torch.empty_like
    dtype, device = like.dtype, like.device
    return lambda _ref: torch.empty(shape, dtype=dtype, device=device)


# ------------------------------------------------------------------ norms


def rms_norm(
    x: torch.Tensor,
    weight: torch.Tensor,
    eps: float = 1e-6,
    *,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """RMSNorm over the last dimension with a float32 reduction. ``weight`` is ``(N,)``
    (float16, bfloat16 or float32). Reference: ops.py:72-88."""
    try:
        key = ("rms", x.shape, x.stride(), x.dtype, x.get_device(), weight.shape, weight.stride(), weight.dtype,
               weight.get_device(), eps, None if out is None else _sig(out), _env("FUSED_DECODE_RMS_BLOCK"),
               _env("FUSED_DECODE_RMS_WARPS"))
        plan = _PLANS.get(key)
    except AttributeError:  # not a tensor: let the contract say so
        key, plan = None, None
    if plan is None:
        plan = _remember(key, _plan_norm(False, x, weight, eps, out, None, None))
    return plan(x, weight, out, None, None)


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
    try:
        key = ("add_rms", x.shape, x.stride(), x.dtype, x.get_device(), residual.shape, residual.stride(),
               residual.dtype, residual.get_device(), weight.shape, weight.stride(), weight.dtype, weight.get_device(),
               eps, None if out is None else _sig(out), None if residual_out is None else _sig(residual_out),
               _env("FUSED_DECODE_RMS_BLOCK"), _env("FUSED_DECODE_RMS_WARPS"))
        plan = _PLANS.get(key)
    except AttributeError:
        key, plan = None, None
    if plan is None:
        plan = _remember(key, _plan_norm(True, x, weight, eps, out, residual, residual_out))
    return plan(x, weight, out, residual, residual_out)


def _plan_norm(add: bool, x, weight, eps, out, residual, residual_out) -> Plan:
    if add:
        a = check("add_rms_norm", x=x, residual=residual, weight=weight, eps=eps, out=out,
                  residual_out=residual_out)
    else:
        a = check("rms_norm", x=x, weight=weight, eps=eps, out=out)
    eps = a["eps"]
    _rms_env()
    shape = tuple(x.shape)
    alloc = _empty(shape, x)
    if x.numel() == 0:
        def empty(x, w, out, r, ro):
            y = alloc(x) if out is None else out
            if add:
                return y, alloc(x) if ro is None else ro
            return y
        return empty

    dense = contiguous_strides(shape)
    strides = [tuple(x.stride())] + ([tuple(residual.stride())] if add else [])
    strides += [dense if out is None else tuple(out.stride())]
    if add:
        strides.append(dense if residual_out is None else tuple(residual_out.stride()))
    rows = plan_rows(shape, strides)
    if rows is None:  # more than three unmergeable leading dims: the staging launcher
        def staged(x, w, out, r, ro):
            y = alloc(x) if out is None else out
            if add:
                ro = alloc(x) if ro is None else ro
                rms_out(x, w, eps, y, residual=r, residual_out=ro)
                return y, ro
            rms_out(x, w, eps, y)
            return y
        return staged

    call = native().add_rms_norm if add else native().rms_norm
    act, wcode, wstride, dev = DTYPE_CODE[x.dtype], DTYPE_CODE[weight.dtype], int(weight.stride(0)), x.device.index
    if add:
        rx, rr, ry, rro = rows

        def run_add(x, w, out, r, ro):
            y = alloc(x) if out is None else out
            ro = alloc(x) if ro is None else ro
            status = call(y.data_ptr(), ro.data_ptr(), x.data_ptr(), r.data_ptr(), w.data_ptr(), wcode, wstride,
                          rx, rr, ry, rro, eps, act, _raw_stream(dev))
            if status:
                fail("fd_add_rms_norm", status)
            return y, ro
        return run_add

    rx, ry = rows

    def run(x, w, out, r, ro):
        y = alloc(x) if out is None else out
        status = call(y.data_ptr(), x.data_ptr(), w.data_ptr(), wcode, wstride, rx, ry, eps, act,
                      _raw_stream(dev))
        if status:
            fail("fd_rms_norm", status)
        return y
    return run


# ------------------------------------------------------------------ pointwise


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
    try:
        key = ("rope", x.shape, x.stride(), x.dtype, x.get_device(), cos.shape, cos.stride(), cos.dtype, cos.get_device(),
               sin.shape, sin.stride(), sin.dtype, sin.get_device(), None if out is None else _sig(out))
        plan = _PLANS.get(key)
    except AttributeError:
        key, plan = None, None
    if plan is None:
        plan = _remember(key, _plan_rope(x, cos, sin, out))
    return plan(x, cos, sin, out)


def _plan_rope(x, cos, sin, out) -> Plan:
    check("rope", x=x, cos=cos, sin=sin, out=out)
    shape = tuple(x.shape)
    alloc = _empty(shape, x)
    mixed = cos.dtype != sin.dtype  # one dtype code per launch: widen both (exact)
    if x.numel() == 0 or mixed:
        def general(x, c, s, out):
            y = alloc(x) if out is None else out
            if x.numel():
                rope_out(x, c.expand(x.shape), s.expand(x.shape), y)
            return y
        return general
    cb, sb = cos.expand(shape), sin.expand(shape)  # stride-0 broadcast dims, never copied
    strides = [tuple(x.stride()), tuple(cb.stride()), tuple(sb.stride()),
               contiguous_strides(shape) if out is None else tuple(out.stride())]
    rows = plan_rows(shape, strides)
    if rows is None:
        def staged(x, c, s, out):
            y = alloc(x) if out is None else out
            rope_out(x, c.expand(x.shape), s.expand(x.shape), y)
            return y
        return staged
    rx, rc, rs, ry = rows
    call, cs, act, dev = native().rope, DTYPE_CODE[cos.dtype], DTYPE_CODE[x.dtype], x.device.index

    def run(x, c, s, out):
        y = alloc(x) if out is None else out
        status = call(y.data_ptr(), x.data_ptr(), c.data_ptr(), s.data_ptr(), cs, rx, rc, rs, ry, act,
                      _raw_stream(dev))
        if status:
            fail("fd_rope", status)
        return y
    return run


def swiglu(
    gate: torch.Tensor,
    up: torch.Tensor,
    *,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """``silu(gate) * up`` in float32, stored in ``gate.dtype``. Reference: ops.py:163-178."""
    try:
        key = ("swiglu", gate.shape, gate.stride(), gate.dtype, gate.get_device(), up.shape, up.stride(), up.dtype,
               up.get_device(), None if out is None else _sig(out))
        plan = _PLANS.get(key)
    except AttributeError:
        key, plan = None, None
    if plan is None:
        plan = _remember(key, _plan_swiglu(gate, up, out))
    return plan(gate, up, out)


def _plan_swiglu(gate, up, out) -> Plan:
    check("swiglu", gate=gate, up=up, out=out)
    shape = tuple(gate.shape)
    alloc = _empty(shape, gate)
    strides = [tuple(gate.stride()), tuple(up.stride()),
               contiguous_strides(shape) if out is None else tuple(out.stride())]
    rows = plan_rows(shape, strides) if gate.numel() else None
    if rows is None:
        def general(g, u, out):
            y = alloc(g) if out is None else out
            swiglu_out(g, u, y)
            return y
        return general
    rg, ru, ry = rows
    call, act, dev = native().swiglu, DTYPE_CODE[gate.dtype], gate.device.index

    def run(g, u, out):
        y = alloc(g) if out is None else out
        status = call(y.data_ptr(), g.data_ptr(), u.data_ptr(), rg, ru, ry, act, _raw_stream(dev))
        if status:
            fail("fd_swiglu", status)
        return y
    return run


# ------------------------------------------------------------------ GEMV


class _Rows(NamedTuple):
    """How an operand is addressed as ``[M, X]`` rows: element (m, j) at
    ``m * row + j * col``; ``flat`` re-derives the view per call when the
    leading dims do not merge into one stride (a copy)."""

    row: int
    col: int
    flat: bool


def _as_rows(t: torch.Tensor, m: int) -> _Rows:
    """``t [..., X]`` as ``m`` rows of X (1-D: one row), without a copy when the
    leading dims merge into one stride."""
    if t.ndim == 1:
        return _Rows(0, int(t.stride(0)), False)
    lead = [(s, st) for s, st in zip(t.shape[:-1], t.stride()[:-1]) if s != 1]
    row = lead[-1][1] if lead else 0
    for (s0, st0), (s1, st1) in zip(lead, lead[1:]):
        if st0 != st1 * s1:
            return _Rows(int(t.shape[-1]), 1, True)  # per-call contiguous copy
    return _Rows(int(row), int(t.stride(-1)), False)


def _row_add_rows(row_add: torch.Tensor, m: int, n: int, expected: tuple) -> tuple[int, int, bool]:
    """Strides (srm, srn) that index ``row_add`` as the ``[M, N]`` output (0 for a
    broadcast dim), or flat=True for a per-call contiguous copy. Legal shapes:
    ``[N]``; 2-D with dims 1 or M and 1 or N; anything that broadcasts to the
    output's shape (the set the reference accepts, ops.py:195-209)."""
    shp = tuple(row_add.shape)
    if row_add.ndim == 1 and shp[0] == n:
        return 0, int(row_add.stride(0)), False
    if row_add.ndim == 2 and shp[0] in (1, m) and shp[1] in (1, n):
        return (0 if shp[0] == 1 else int(row_add.stride(0)),
                0 if shp[1] == 1 else int(row_add.stride(1)), False)
    try:
        view = row_add.expand(expected)
    except RuntimeError as exc:
        raise ValueError(f"row_add shape {shp} is not broadcastable to {expected}") from exc
    r = _as_rows(view, m)
    if r.flat:
        return n, 1, True
    return r.row, r.col, False


def _check_out(out, expected: tuple, like: torch.Tensor) -> None:
    if tuple(out.shape) != expected or out.dtype != like.dtype or out.device != like.device:
        raise ValueError(f"out must be a contiguous {expected} tensor of dtype {like.dtype} on {like.device}")
    if not out.is_contiguous():
        raise ValueError("out must be contiguous")


def _default_limit(kind: str) -> int:
    """Rows up to which the default dispatcher runs the HIP GEMV of `kind`."""
    return DECODE_LINEAR_MAX_M if kind == "dot" else SIMT_DECODE_LINEAR_MAX_M


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

    The HIP GEMV runs for a flattened batch up to ``DECODE_LINEAR_MAX_M`` rows
    (``SIMT_DECODE_LINEAR_MAX_M`` when FUSED_DECODE_LINEAR_KIND selects "simt"),
    or up to 16 when ``kind`` ("dot" or "simt") is given; wider batches call
    ``F.linear`` (bit-identical to it), with row_add added in float32.
    Reference: ops.py:212-280.
    """
    try:
        key = ("linear", x.shape, x.stride(), x.dtype, x.get_device(), weight.shape, weight.stride(), weight.dtype,
               weight.get_device(), _sig(bias), _sig(row_add), _sig(out), kind,
               _env("FUSED_DECODE_LINEAR_KIND"), _env("FUSED_DECODE_LINEAR"))
        plan = _PLANS.get(key)
    except AttributeError:
        key, plan = None, None
    if plan is None:
        plan = _remember(key, _plan_linear(x, weight, bias, row_add, out, kind))
    return plan(x, weight, bias, row_add, out)


def _plan_linear(x, weight, bias, row_add, out, kind) -> Plan:
    check("linear_decode", x=x, weight=weight, bias=bias, row_add=row_add, kind=kind)
    kind_r = resolve_kind(kind)
    limit = _FORCED_LIMIT if kind is not None else _default_limit(kind_r)
    n, k = (int(d) for d in weight.shape)
    m = 1 if x.ndim == 1 else math.prod(x.shape[:-1])
    expected = (n,) if x.ndim == 1 else (*x.shape[:-1], n)
    ra = None if row_add is None else _row_add_rows(row_add, m, n, expected)
    if out is not None:
        _check_out(out, expected, x)
    alloc = _empty(expected, x)
    if m == 0 or n == 0:
        return lambda x, w, b, r, out: alloc(x) if out is None else out
    xr = _as_rows(x, m)

    def operands(x, r):
        """x as [M, K] and row_add as [M, N]-indexable tensors for F.linear."""
        x2 = x.reshape(m, k)
        if r is None:
            return x2, None
        if r.ndim == 1 or (r.ndim == 2 and r.shape[0] in (1, m) and r.shape[1] in (1, n)):
            return x2, r
        return x2, r.expand(expected).reshape(m, n)

    if m > limit:  # hipBLASLt, bit-identical to F.linear; row_add in float32, one rounding
        def fallback(x, w, b, r, out):
            x2, r2 = operands(x, r)
            y = F.linear(x2, w, b)
            if r2 is not None:
                y = (y.float() + r2.float()).to(x.dtype)
            if out is None:
                return y.view(expected)
            out.view(m, n).copy_(y)
            return out
        return fallback

    rows, _, waves, stages = linear_config(kind_r, n, k, m)
    tile = bytes(FdTile(rows, waves, stages))
    call, act, kcode, dev = native().linear_tiled, DTYPE_CODE[x.dtype], KIND_CODE[kind_r], x.device.index
    swn, swk = int(weight.stride(0)), int(weight.stride(1))
    bcode = DTYPE_CODE[bias.dtype] if bias is not None else act
    sb = int(bias.stride(0)) if bias is not None else 0
    rcode = DTYPE_CODE[row_add.dtype] if row_add is not None else act
    srm, srn, r_flat = ra if ra is not None else (0, 0, False)

    def run(x, w, b, r, out):
        y = alloc(x) if out is None else out
        if xr.flat:
            x = x.reshape(m, k)
        if r_flat:
            r = r.expand(expected).reshape(m, n)
        status = call(y.data_ptr(), x.data_ptr(), w.data_ptr(), None if b is None else b.data_ptr(), bcode,
                      None if r is None else r.data_ptr(), rcode, m, n, k, xr.row, xr.col, swn, swk, sb, srm,
                      srn, n, 1, tile, kcode, act, _raw_stream(dev))
        if status:
            fail("fd_linear_tiled", status)
        return y
    return run


# ------------------------------------------------------------------ fused blocks


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
    try:
        key = ("mlp", _sig(hidden), _sig(norm_weight), _sig(w_gate_up), _sig(w_down), eps, kind,
               _env("FUSED_DECODE_LINEAR_KIND"))
        plan = _PLANS.get(key)
    except AttributeError:
        key, plan = None, None
    if plan is None:
        plan = _remember(key, _plan_mlp(hidden, norm_weight, w_gate_up, w_down, eps, kind))
    return plan(hidden, norm_weight, w_gate_up, w_down)


def _plan_mlp(hidden, norm_weight, w_gate_up, w_down, eps, kind) -> Plan:
    a = check("post_attn_mlp", hidden=hidden, norm_weight=norm_weight, w_gate_up=w_gate_up, w_down=w_down,
              eps=eps, kind=kind)
    eps = a["eps"]
    limit = _FORCED_LIMIT if kind is not None else DECODE_LINEAR_MAX_M
    kind_r = resolve_kind(kind)
    h, i = int(w_gate_up.shape[1]), int(w_down.shape[1])
    m = hidden.numel() // h if h else 0

    def composed(x, nw, wgu, wd):
        normed = rms_norm(x, nw, eps=eps)
        gate, up = linear_decode(normed, wgu, kind=kind).split(i, dim=-1)
        return linear_decode(swiglu(gate, up), wd, row_add=x, kind=kind)

    if not (0 < m <= limit and w_gate_up.is_contiguous() and w_down.is_contiguous()):
        return composed
    shape = tuple(hidden.shape)
    dense_h, dense_nw = _dense(hidden), _dense(norm_weight)
    call, act, nwc, kcode, dev = (native().post_attn_mlp, DTYPE_CODE[hidden.dtype], DTYPE_CODE[norm_weight.dtype],
                                  KIND_CODE[kind_r], hidden.device.index)

    def fused(x, nw, wgu, wd):
        x2 = x if dense_h else x.contiguous()
        nw = nw if dense_nw else nw.contiguous()
        y = x2.new_empty((m, h))
        mid = x2.new_empty((m, i))
        status = call(y.data_ptr(), mid.data_ptr(), x2.data_ptr(), nw.data_ptr(), nwc, wgu.data_ptr(),
                      wd.data_ptr(), m, h, i, eps, kcode, act, _raw_stream(dev))
        if status == FD_EUNSUPPORTED:  # e.g. H % 8 or an unaligned operand: the composed operators
            return composed(x, nw, wgu, wd)
        if status:
            fail("fd_post_attn_mlp", status)
        return y.view(shape)
    return fused


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
    """Operands shared by ``pre_attn_qkv`` and its fp8 form, for a projection of
    ``n`` rows over ``h`` (``hidden [..., h]``), after the contract's checks."""
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
    lead = tuple(hidden.shape[:-1])
    cos_r = _token_angles(cos, lead, "cos")
    sin_r = _token_angles(sin, lead, "sin")
    if cos_r.dtype != sin_r.dtype:
        cos_r, sin_r = cos_r.float(), sin_r.float()
    expected = (*lead, n)
    if out is None:
        out = torch.empty(expected, device=hidden.device, dtype=hidden.dtype)
    else:
        _check_out(out, expected, hidden)
    m = hidden.numel() // h if h else 0
    if m and n and cos_r.shape[0] not in (1, m):
        raise ValueError(f"cos/sin need 1 or {m} rows, got {cos_r.shape[0]}")
    rs = 0 if cos_r.shape[0] == 1 else d
    return _QkvArgs(m, n, h, d, rope_cols, float(eps), cos_r, sin_r, rs, out)


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
    HIP launch (from 5 rows with kind "dot" an MFMA kernel with the norm folded in).
    No reference counterpart as one call; it composes ops.py:72-88, :212-280 and
    :138-160.
    """
    try:
        key = ("qkv", _sig(hidden), _sig(norm_weight), _sig(w_qkv), _sig(cos), _sig(sin), eps, rope_cols,
               _sig(bias), _sig(out), kind, _env("FUSED_DECODE_LINEAR_KIND"))
        plan = _PLANS.get(key)
    except (AttributeError, TypeError):  # a non-tensor or unhashable argument: checked below
        key, plan = None, None
    if plan is None:
        plan = _remember(key, _plan_qkv(hidden, norm_weight, w_qkv, None, cos, sin, eps, rope_cols, bias, out,
                                        kind))
    return plan(hidden, norm_weight, w_qkv, None, cos, sin, bias, out)


def _plan_qkv(hidden, norm_weight, w_qkv, scale, cos, sin, eps, rope_cols, bias, out, kind) -> Plan:
    """Launch plan of ``pre_attn_qkv`` (``scale`` None) or ``pre_attn_qkv_fp8``
    for one argument signature: every check runs here once; the plan's calls
    only take the pointers. cos/sin already in the kernel's ``[1 or M, D]``
    contiguous rows of one dtype are passed as they are, others are gathered
    per call."""
    fp8 = scale is not None
    if fp8:
        a0 = check("pre_attn_qkv_fp8", hidden=hidden, norm_weight=norm_weight, w_qkv=w_qkv, scale=scale,
                   eps=eps, bias=bias)
    else:
        a0 = check("pre_attn_qkv", hidden=hidden, norm_weight=norm_weight, w_qkv=w_qkv, eps=eps, kind=kind,
                   bias=bias)
    n, h = (int(v) for v in w_qkv.shape)
    a = _qkv_args(hidden, norm_weight, n, h, cos, sin, a0["eps"], rope_cols, bias, out)
    m, d, rc, rs, eps = a.m, a.d, a.rope_cols, a.cs_row_stride, a.eps
    lead, expected = tuple(hidden.shape[:-1]), tuple(a.out.shape)

    def angles(c, s):
        cr, sr = _token_angles(c, lead, "cos"), _token_angles(s, lead, "sin")
        return (cr, sr) if cr.dtype == sr.dtype else (cr.float(), sr.float())

    def composed(x, nw, w, sc, c, s, b, o):
        y = o if o is not None else x.new_empty(expected)
        cr, sr = angles(c, s)
        normed = rms_norm(x, nw, eps=eps)
        if fp8:
            from .fp8 import linear_decode_fp8

            linear_decode_fp8(normed, w, sc, b, out=y)
        else:
            linear_decode(normed, w, b, out=y, kind=kind)
        _rope_qkv_heads(_QkvArgs(m, n, h, d, rc, eps, cr, sr, rs, y))
        return y

    if m == 0 or n == 0:
        return lambda x, nw, w, sc, c, s, b, o: o if o is not None else x.new_empty(expected)
    if fp8:
        fits = m <= _FP8_ROWS and w_qkv.is_contiguous() and h % 16 == 0
    else:
        fits = m <= (_FORCED_LIMIT if kind is not None else DECODE_LINEAR_MAX_M) and w_qkv.is_contiguous()
    if not fits:
        return composed
    direct = (a.cos.data_ptr() == cos.data_ptr() and a.sin.data_ptr() == sin.data_ptr()
              and cos.dtype == sin.dtype)
    dense_h, dense_nw = _dense(hidden), _dense(norm_weight)
    dense_b = bias is None or _dense(bias)
    dense_sc = not fp8 or _dense(scale)
    act, nwc, csc, dev = (DTYPE_CODE[hidden.dtype], DTYPE_CODE[norm_weight.dtype], DTYPE_CODE[a.cos.dtype],
                          hidden.device.index)
    bc = DTYPE_CODE[bias.dtype] if bias is not None else act
    call = native().pre_attn_qkv_fp8 if fp8 else native().pre_attn_qkv
    kcode = None if fp8 else KIND_CODE[resolve_kind(kind)]
    name = "fd_pre_attn_qkv_fp8" if fp8 else "fd_pre_attn_qkv"

    def fused(x, nw, w, sc, c, s, b, o):
        y = o if o is not None else x.new_empty(expected)
        cr, sr = (c, s) if direct else angles(c, s)
        x2 = x if dense_h else x.contiguous()
        nw2 = nw if dense_nw else nw.contiguous()
        bp = None if b is None else (b if dense_b else b.contiguous()).data_ptr()
        if fp8:
            sp = (sc if dense_sc else sc.contiguous()).data_ptr()
            status = call(y.data_ptr(), None, x2.data_ptr(), nw2.data_ptr(), nwc, w.data_ptr(), sp, bp, bc,
                          cr.data_ptr(), sr.data_ptr(), csc, rs, m, h, n, rc, d, eps, act, _raw_stream(dev))
        else:
            status = call(y.data_ptr(), None, x2.data_ptr(), nw2.data_ptr(), nwc, w.data_ptr(), bp, bc,
                          cr.data_ptr(), sr.data_ptr(), csc, rs, m, h, n, rc, d, eps, kcode, act,
                          _raw_stream(dev))
        if status == FD_EUNSUPPORTED:  # a shape the fused kernels do not take: the operators
            return composed(x, nw, w, sc, c, s, b, y)
        if status:
            fail(name, status)
        return y
    return fused
