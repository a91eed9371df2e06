"""CPU oracle for the decode operator set: test infrastructure only.

A NumPy restatement of the reference's fp32 semantics
(src/fused_decode/reference.py) used as the checker for the HIP kernels. It is
imported only by tests/, by __graft_entry__.smoke() and by bench.py's
cpu_baseline leg; the product path never calls it.

Conventions: every array is float32 and holds values exactly representable in
the activation dtype ("f16" or "bf16"); results are rounded to that dtype with
round-to-nearest-even (what torch's ``.to(dtype)`` does) and returned as
float32. Arithmetic is float32 with the rounding points of the reference.

Pinning (tests/test_oracle.py): every function is checked against closed forms,
invariants, float64 brute force and independent library routines (torch CPU
``F.rms_norm``, ``F.silu``, ``F.linear``, complex rotation for RoPE), so a
dropped term, a wrong sign or index, or a transposed operand fails a check.
"""

from __future__ import annotations

import numpy as np

F32 = np.float32


def round_to(a: np.ndarray, dtype: str) -> np.ndarray:
    """Round float32 values to fp16 or bf16 (nearest-even), returned as float32."""
    a = np.asarray(a, dtype=F32)
    if dtype == "f16":
        with np.errstate(over="ignore"):  # out-of-range values become inf, as in torch
            return a.astype(np.float16).astype(F32)
    if dtype == "bf16":
        bits = a.view(np.uint32).astype(np.uint64)
        # round-to-nearest-even on the upper 16 bits; NaN stays NaN
        lsb = (bits >> 16) & 1
        rounded = ((bits + 0x7FFF + lsb) >> 16) << 16
        out = rounded.astype(np.uint32).view(F32)
        nan = np.isnan(a)
        if nan.any():
            out = out.copy()
            out[nan] = np.float32("nan")
        return out
    if dtype == "f32":
        return a
    raise ValueError(f"unknown dtype {dtype}")


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float, dtype: str) -> np.ndarray:
    """y = round(x * rsqrt(mean(x^2) + eps) * w). Reference: reference.py:14-18."""
    x = np.asarray(x, F32)
    var = np.mean(x * x, axis=-1, keepdims=True, dtype=F32)
    inv = F32(1.0) / np.sqrt(var + F32(eps), dtype=F32)
    return round_to(x * inv * np.asarray(w, F32), dtype)


def add_rms_norm(x, residual, w, eps: float, dtype: str):
    """s = x + r in fp32; (round(s * rsqrt(mean(s^2)+eps) * w), round(s)).
    The norm uses the fp32 sum, not the rounded residual. Reference: reference.py:21-30."""
    s = np.asarray(x, F32) + np.asarray(residual, F32)
    var = np.mean(s * s, axis=-1, keepdims=True, dtype=F32)
    inv = F32(1.0) / np.sqrt(var + F32(eps), dtype=F32)
    return round_to(s * inv * np.asarray(w, F32), dtype), round_to(s, dtype)


def silu(g: np.ndarray) -> np.ndarray:
    """g * sigmoid(g) in fp32 with the overflow-free sigmoid (kernels.py:448-451)."""
    g = np.asarray(g, F32)
    e = np.exp(-np.abs(g), dtype=F32)
    sig = np.where(g >= 0, F32(1.0) / (F32(1.0) + e), e / (F32(1.0) + e)).astype(F32)
    return g * sig


def swiglu(gate, up, dtype: str) -> np.ndarray:
    """round(silu(gate) * up). Reference: reference.py:33-35."""
    return round_to(silu(gate) * np.asarray(up, F32), dtype)


def rope(x, cos, sin, dtype: str) -> np.ndarray:
    """Rotate-half RoPE, cos/sin broadcast to x. Reference: reference.py:38-47."""
    x = np.asarray(x, F32)
    c = np.broadcast_to(np.asarray(cos, F32), x.shape)
    s = np.broadcast_to(np.asarray(sin, F32), x.shape)
    h = x.shape[-1] // 2
    x1, x2 = x[..., :h], x[..., h:]
    out = np.concatenate((x1 * c[..., :h] - x2 * s[..., :h], x2 * c[..., h:] + x1 * s[..., h:]), axis=-1)
    return round_to(out, dtype)


def linear(x, w, bias=None, row_add=None, dtype: str = "f16") -> np.ndarray:
    """round(x @ w.T + bias + row_add) with one fp32 accumulation and a single
    rounding. Reference: reference.py:50-63 (fp32 CPU F.linear, then row_add)."""
    x = np.asarray(x, F32)
    w = np.asarray(w, F32)
    y = x @ w.T
    if bias is not None:
        y = y + np.asarray(bias, F32)
    if row_add is not None:
        ra = np.asarray(row_add, F32)
        if ra.size == y.size:  # same elements, possibly another leading shape
            ra = ra.reshape(y.shape)
        y = y + ra  # otherwise size-1 dims broadcast
    return round_to(y.astype(F32), dtype)


def post_attn_mlp(hidden, norm_w, w_gate_up, w_down, eps: float, dtype: str) -> np.ndarray:
    """Composition with the reference's four rounding points (reference.py:66-79):
    h = round(rms(hidden)); gu = round(h @ Wgu.T); mid = round(silu(g) * u);
    y = round(mid @ Wd.T + hidden)."""
    i = np.shape(w_down)[1]
    h = rms_norm(hidden, norm_w, eps, dtype)
    gu = linear(h, w_gate_up, dtype=dtype)
    mid = swiglu(gu[..., :i], gu[..., i:], dtype)
    return linear(mid, w_down, row_add=hidden, dtype=dtype)


def pre_attn_qkv(hidden, norm_w, w_qkv, cos, sin, eps: float, rope_cols: int, bias=None,
                 dtype: str = "f16") -> np.ndarray:
    """The pre-attention composition a caller of the reference writes from its
    operators: h = round(rms(hidden)) (reference.py:14-18), y = round(h @ Wqkv.T +
    bias) (reference.py:50-63), then rotate-half RoPE (reference.py:38-47) of the
    first rope_cols columns viewed as heads of D = cos.shape[-1], each row m with
    cos/sin row m (one row broadcasts to all)."""
    h = rms_norm(np.asarray(hidden, F32), norm_w, eps, dtype)
    return _rope_leading_cols(linear(h, w_qkv, bias=bias, dtype=dtype), cos, sin, rope_cols, dtype)


def _rope_leading_cols(y, cos, sin, rope_cols: int, dtype: str) -> np.ndarray:
    """Rotate-half RoPE of y[:, :rope_cols] viewed as heads of D = cos.shape[-1]."""
    if not rope_cols:
        return y
    m = y.shape[0]
    d = np.shape(cos)[-1]
    c = np.asarray(cos, F32).reshape(-1, 1, d)
    s = np.asarray(sin, F32).reshape(-1, 1, d)
    heads = y[:, :rope_cols].reshape(m, rope_cols // d, d)
    y = y.copy()
    y[:, :rope_cols] = rope(heads, c, s, dtype).reshape(m, rope_cols)
    return y


def bytes_qkv(m: int, h: int, n: int, head_dim: int, cs_rows: int, e: int = 2, ce: int = 2) -> int:
    """Weights + hidden read + norm weight + output write + cos/sin rows."""
    return (n * h + m * h + h + m * n) * e + 2 * cs_rows * head_dim * ce


# ---------------------------------------------------------------- fp8 weights
# OCP FP8 E4M3 ("e4m3fn"): 1 sign, 4 exponent bits (bias 7), 3 mantissa bits;
# no infinities, 0x7f/0xff are NaN, largest finite 448, subnormals m * 2^-9.
FP8_MAX = 448.0


def fp8_decode(codes) -> np.ndarray:
    """E4M3 byte codes -> float32 values (exact), from the format's definition."""
    b = np.asarray(codes, np.uint8).astype(np.int32)
    sign = np.where(b & 0x80, -1.0, 1.0)
    e = (b >> 3) & 0xF
    m = b & 0x7
    val = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * 2.0 ** (e - 7))
    val = np.where((b & 0x7F) == 0x7F, np.nan, val)
    return (sign * val).astype(F32)


def fp8_encode(values) -> np.ndarray:
    """float32 -> E4M3 codes, round to nearest even, |v| > 448 saturated to 448
    (the quantizer never produces NaN)."""
    v = np.clip(np.asarray(values, np.float64), -FP8_MAX, FP8_MAX)
    grid = fp8_decode(np.arange(0x7F, dtype=np.uint8)).astype(np.float64)  # 0 .. 448, ascending
    mag = np.abs(v)
    hi = np.clip(np.searchsorted(grid, mag, side="left"), 1, 0x7E)
    lo = hi - 1
    d_lo, d_hi = mag - grid[lo], grid[hi] - mag
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (hi % 2 == 0))
    code = np.where(pick_hi, hi, lo)
    code = np.where(mag <= grid[0], 0, code)
    code = np.where(mag >= grid[0x7E], 0x7E, code)
    return (code | np.where(v < 0, 0x80, 0)).astype(np.uint8)


def fp8_quantize(w) -> tuple:
    """Per-output-channel scaling: scale[n] = max|w[n,:]| * float32(1/448) (1 for an
    all-zero row), codes = encode(w / scale)."""
    w = np.asarray(w, F32)
    amax = np.max(np.abs(w), axis=1)
    scale = np.where(amax > 0, amax * F32(1.0 / FP8_MAX), F32(1.0)).astype(F32)
    return fp8_encode(w / scale[:, None]), scale


def linear_fp8(x, codes, scale, bias=None, row_add=None, dtype: str = "f16") -> np.ndarray:
    """round(scale[n] * sum_k decode(codes[n,k]) * x[m,k] + bias[n] + row_add[m,n]):
    fp32 accumulation of the exact decoded weights, the channel scale applied to
    the sum, then the reference's epilogue order (kernels.py:657-672)."""
    acc = np.asarray(x, F32) @ fp8_decode(codes).T
    y = acc * np.asarray(scale, F32)
    if bias is not None:
        y = y + np.asarray(bias, F32)
    if row_add is not None:
        ra = np.asarray(row_add, F32)
        y = y + (ra.reshape(y.shape) if ra.size == y.size else ra)
    return round_to(y.astype(F32), dtype)


def post_attn_mlp_fp8(hidden, norm_w, gu_codes, gu_scale, d_codes, d_scale, eps: float,
                      dtype: str) -> np.ndarray:
    """post_attn_mlp (reference.py:66-79) with fp8 weights: the same four rounding
    points, each projection as linear_fp8."""
    i = np.shape(d_codes)[1]
    h = rms_norm(hidden, norm_w, eps, dtype)
    gu = linear_fp8(h, gu_codes, gu_scale, dtype=dtype)
    mid = swiglu(gu[..., :i], gu[..., i:], dtype)
    return linear_fp8(mid, d_codes, d_scale, row_add=hidden, dtype=dtype)


def pre_attn_qkv_fp8(hidden, norm_w, codes, scale, cos, sin, eps: float, rope_cols: int,
                     bias=None, dtype: str = "f16") -> np.ndarray:
    """pre_attn_qkv with fp8 weights: the same rounding points, the projection as
    linear_fp8."""
    h = rms_norm(np.asarray(hidden, F32), norm_w, eps, dtype)
    y = linear_fp8(h, codes, scale, bias=bias, dtype=dtype)
    return _rope_leading_cols(y, cos, sin, rope_cols, dtype)


def bytes_qkv_fp8(m: int, h: int, n: int, head_dim: int, cs_rows: int, e: int = 2, ce: int = 2) -> int:
    """fp8 weights + fp32 scales + hidden read + norm weight + output write + cos/sin rows."""
    return n * h + 4 * n + (m * h + h + m * n) * e + 2 * cs_rows * head_dim * ce


def bytes_linear_fp8(m: int, n: int, k: int, e: int = 2) -> int:
    """fp8 weights (1 byte each) + fp32 scales + activations in and out."""
    return n * k + 4 * n + (m * k + m * n) * e


def bytes_mlp_fp8(m: int, h: int, i: int, e: int = 2) -> int:
    return 3 * h * i + 4 * (2 * i + h) + (2 * m * h + h) * e


# Useful-byte accounting (reference README.md:33-43, bench.py:215-216, :247,
# :274, :303-305): weights counted once, no cache reuse, e bytes per element.
def bytes_rms(rows: int, n: int, e: int = 2) -> int:
    return (2 * rows * n + n) * e


def bytes_add_rms(rows: int, n: int, e: int = 2) -> int:
    return (4 * rows * n + n) * e


def bytes_swiglu(rows: int, n: int, e: int = 2) -> int:
    return 3 * rows * n * e


def bytes_rope(x_elems: int, cos_elems: int, sin_elems: int, e: int = 2, ce: int = 2) -> int:
    return 2 * x_elems * e + (cos_elems + sin_elems) * ce


def bytes_linear(m: int, n: int, k: int, bias: bool = False, e: int = 2) -> int:
    return (m * k + n * k + m * n + (n if bias else 0)) * e


def bytes_mlp(m: int, h: int, i: int, e: int = 2) -> int:
    """Weights (3*H*I) + hidden read + norm weight + output write."""
    return (3 * h * i + 2 * m * h + h) * e
