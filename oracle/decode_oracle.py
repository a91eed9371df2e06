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
    hidden = np.asarray(hidden, F32)
    m = hidden.shape[0]
    h = rms_norm(hidden, norm_w, eps, dtype)
    y = linear(h, w_qkv, bias=bias, dtype=dtype)
    if rope_cols:
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
