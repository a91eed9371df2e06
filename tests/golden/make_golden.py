"""Writes the golden fixtures of this directory: seeded inputs at small shapes
and the oracle's outputs for them, one compressed .npz per operator family.

    python tests/golden/make_golden.py          (from the repository root)

Inputs are drawn with NumPy's seeded generator and rounded to the case's storage
type (fp16, or bf16 by round-to-nearest-even), so every stored float32 value is
exactly representable in that type; fp8 weights are the oracle quantiser's
codes and scales. Outputs are the oracle's (oracle/decode_oracle.py), already
rounded to the storage type. Keys are "<case>/<name>": per case the inputs, the
outputs ("out", and "residual_out" for add_rms_norm), "dtype" ("f16"/"bf16")
and the scalar parameters. Everything is a plain numeric or string array, so
the files load with numpy.load(..., allow_pickle=False).

The reference ships no golden vectors (its tests recompute reference.py live):
these fixtures freeze the oracle's outputs, whose functions are pinned in
tests/test_oracle.py, so that tests/test_golden.py notices any change to the
oracle and tests/test_golden_gpu.py checks the HIP path against fixed vectors.
"""

from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import decode_oracle as O  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
DTYPES = ("f16", "bf16")
EPS = 1e-5


def _draw(rng, shape, dtype, scale=1.0, mean=0.0):
    return O.round_to((rng.standard_normal(shape) * scale + mean).astype(np.float32), dtype)


def _angles(rows: int, d: int, first_pos: int):
    """Llama-3 rotate-half tables (theta = 500000) for positions first_pos.. ."""
    inv = 1.0 / (500000.0 ** (np.arange(0, d, 2, dtype=np.float64) / d))
    pos = np.arange(first_pos, first_pos + rows, dtype=np.float64)
    emb = np.concatenate([pos[:, None] * inv[None], pos[:, None] * inv[None]], axis=1)
    return np.cos(emb).astype(np.float32), np.sin(emb).astype(np.float32)


def norms():
    out = {}
    for i, dt in enumerate(DTYPES):
        rng = np.random.default_rng(100 + i)
        x = _draw(rng, (5, 96), dt)
        r = _draw(rng, (5, 96), dt)
        w = _draw(rng, (96,), dt, 0.1, 1.0)
        out[f"rms_{dt}/x"], out[f"rms_{dt}/w"] = x, w
        out[f"rms_{dt}/out"] = O.rms_norm(x, w, EPS, dt)
        y, ro = O.add_rms_norm(x, r, w, EPS, dt)
        out[f"add_rms_{dt}/x"], out[f"add_rms_{dt}/residual"], out[f"add_rms_{dt}/w"] = x, r, w
        out[f"add_rms_{dt}/out"], out[f"add_rms_{dt}/residual_out"] = y, ro
        for c in (f"rms_{dt}", f"add_rms_{dt}"):
            out[f"{c}/dtype"], out[f"{c}/eps"] = np.array(dt), np.array(EPS, np.float32)
    return out


def pointwise():
    out = {}
    for i, dt in enumerate(DTYPES):
        rng = np.random.default_rng(200 + i)
        g = _draw(rng, (3, 80), dt, 2.0)
        u = _draw(rng, (3, 80), dt, 2.0)
        out[f"swiglu_{dt}/gate"], out[f"swiglu_{dt}/up"] = g, u
        out[f"swiglu_{dt}/out"] = O.swiglu(g, u, dt)
        x = _draw(rng, (1, 3, 4, 32), dt)
        cos, sin = _angles(3, 32, 0)
        cos, sin = cos.reshape(3, 1, 32), sin.reshape(3, 1, 32)
        out[f"rope_{dt}/x"], out[f"rope_{dt}/cos"], out[f"rope_{dt}/sin"] = x, cos, sin
        out[f"rope_{dt}/out"] = O.rope(x, cos, sin, dt)
        out[f"swiglu_{dt}/dtype"] = out[f"rope_{dt}/dtype"] = np.array(dt)
    return out


def linear():
    out = {}
    for i, dt in enumerate(DTYPES):
        for m in (1, 6):
            rng = np.random.default_rng(300 + 10 * i + m)
            n, k = 24, 64
            c = f"linear_{dt}_m{m}"
            x = _draw(rng, (m, k), dt)
            w = _draw(rng, (n, k), dt, k ** -0.5)
            b = rng.standard_normal(n).astype(np.float32)
            ra = _draw(rng, (m, n), dt)
            out[f"{c}/x"], out[f"{c}/w"], out[f"{c}/bias"], out[f"{c}/row_add"] = x, w, b, ra
            out[f"{c}/out"] = O.linear(x, w, bias=b, row_add=ra, dtype=dt)
            out[f"{c}/dtype"] = np.array(dt)
    return out


def mlp():
    out = {}
    for i, dt in enumerate(DTYPES):
        for m in (1, 6):
            rng = np.random.default_rng(400 + 10 * i + m)
            h, inter = 64, 48
            c = f"mlp_{dt}_m{m}"
            hid = _draw(rng, (m, h), dt)
            nw = _draw(rng, (h,), dt, 0.1, 1.0)
            wgu = _draw(rng, (2 * inter, h), dt, h ** -0.5)
            wd = _draw(rng, (h, inter), dt, inter ** -0.5)
            out[f"{c}/hidden"], out[f"{c}/norm_w"], out[f"{c}/w_gate_up"], out[f"{c}/w_down"] = hid, nw, wgu, wd
            out[f"{c}/out"] = O.post_attn_mlp(hid, nw, wgu, wd, EPS, dt)
            out[f"{c}/dtype"], out[f"{c}/eps"] = np.array(dt), np.array(EPS, np.float32)
    return out


def qkv():
    out = {}
    for i, dt in enumerate(DTYPES):
        for m in (1, 6):
            rng = np.random.default_rng(500 + 10 * i + m)
            h, heads, kv, d = 64, 2, 1, 32
            n, rc = (heads + 2 * kv) * d, (heads + kv) * d
            c = f"qkv_{dt}_m{m}"
            hid = _draw(rng, (m, h), dt)
            nw = _draw(rng, (h,), dt, 0.1, 1.0)
            w = _draw(rng, (n, h), dt, h ** -0.5)
            b = (rng.standard_normal(n) * 0.5).astype(np.float32)
            cos, sin = _angles(m, d, 1000 + m)
            out[f"{c}/hidden"], out[f"{c}/norm_w"], out[f"{c}/w_qkv"], out[f"{c}/bias"] = hid, nw, w, b
            out[f"{c}/cos"], out[f"{c}/sin"] = cos, sin
            out[f"{c}/out"] = O.pre_attn_qkv(hid, nw, w, cos, sin, EPS, rc, bias=b, dtype=dt)
            out[f"{c}/dtype"], out[f"{c}/eps"] = np.array(dt), np.array(EPS, np.float32)
            out[f"{c}/rope_cols"] = np.array(rc, np.int64)
    return out


def fp8():
    out = {}
    for i, dt in enumerate(DTYPES):
        for m in (1, 6):
            rng = np.random.default_rng(600 + 10 * i + m)
            c = f"linear_fp8_{dt}_m{m}"
            n, k = 24, 64
            x = _draw(rng, (m, k), dt)
            q, s = O.fp8_quantize(rng.standard_normal((n, k)).astype(np.float32) * k ** -0.5)
            b = rng.standard_normal(n).astype(np.float32)
            ra = _draw(rng, (m, n), dt)
            out[f"{c}/x"], out[f"{c}/codes"], out[f"{c}/scale"] = x, q, s
            out[f"{c}/bias"], out[f"{c}/row_add"] = b, ra
            out[f"{c}/out"] = O.linear_fp8(x, q, s, bias=b, row_add=ra, dtype=dt)
            out[f"{c}/dtype"] = np.array(dt)

            c = f"mlp_fp8_{dt}_m{m}"
            h, inter = 64, 48
            hid = _draw(rng, (m, h), dt)
            nw = _draw(rng, (h,), dt, 0.1, 1.0)
            qgu, sgu = O.fp8_quantize(rng.standard_normal((2 * inter, h)).astype(np.float32) * h ** -0.5)
            qd, sd = O.fp8_quantize(rng.standard_normal((h, inter)).astype(np.float32) * inter ** -0.5)
            out[f"{c}/hidden"], out[f"{c}/norm_w"] = hid, nw
            out[f"{c}/gu_codes"], out[f"{c}/gu_scale"], out[f"{c}/d_codes"], out[f"{c}/d_scale"] = qgu, sgu, qd, sd
            out[f"{c}/out"] = O.post_attn_mlp_fp8(hid, nw, qgu, sgu, qd, sd, EPS, dt)
            out[f"{c}/dtype"], out[f"{c}/eps"] = np.array(dt), np.array(EPS, np.float32)

            c = f"qkv_fp8_{dt}_m{m}"
            h, heads, kv, d = 64, 2, 1, 32
            n, rc = (heads + 2 * kv) * d, (heads + kv) * d
            hid = _draw(rng, (m, h), dt)
            nw = _draw(rng, (h,), dt, 0.1, 1.0)
            q, s = O.fp8_quantize(rng.standard_normal((n, h)).astype(np.float32) * h ** -0.5)
            b = (rng.standard_normal(n) * 0.5).astype(np.float32)
            cos, sin = _angles(m, d, 2000 + m)
            out[f"{c}/hidden"], out[f"{c}/norm_w"], out[f"{c}/codes"], out[f"{c}/scale"] = hid, nw, q, s
            out[f"{c}/bias"], out[f"{c}/cos"], out[f"{c}/sin"] = b, cos, sin
            out[f"{c}/out"] = O.pre_attn_qkv_fp8(hid, nw, q, s, cos, sin, EPS, rc, bias=b, dtype=dt)
            out[f"{c}/dtype"], out[f"{c}/eps"] = np.array(dt), np.array(EPS, np.float32)
            out[f"{c}/rope_cols"] = np.array(rc, np.int64)
    return out


FAMILIES = {"norms": norms, "pointwise": pointwise, "linear": linear, "mlp": mlp, "qkv": qkv,
            "fp8": fp8}


def main() -> None:
    for name, make in FAMILIES.items():
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **make())
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
