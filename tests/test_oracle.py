"""Pins the CPU oracle (CPU only).

Each oracle function is checked against something that does not restate its
formula: closed forms, invariants, float64 brute force, and independent
library routines (torch CPU F.rms_norm / F.silu / F.linear, complex rotation
for RoPE). Planted mistakes (tests at the bottom) show the checks bite.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import decode_oracle as O

RNG = np.random.default_rng(1234)


def as_dtype(a: np.ndarray, dtype: str) -> np.ndarray:
    return O.round_to(np.asarray(a, np.float32), dtype)


def torch_round(a: np.ndarray, dtype: str) -> np.ndarray:
    td = torch.float16 if dtype == "f16" else torch.bfloat16
    return torch.from_numpy(np.asarray(a, np.float32)).to(td).float().numpy()


# ---------------------------------------------------------------- rounding


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_round_to_matches_torch_cast(dtype):
    a = np.concatenate([
        RNG.standard_normal(20000).astype(np.float32) * 10,
        np.array([0.0, -0.0, 1.0, 65504.0, 1e-8, -1e-8, 3.0e38, 1.00390625, 1.01171875], np.float32),
    ])
    np.testing.assert_array_equal(O.round_to(a, dtype), torch_round(a, dtype))


def test_round_bf16_ties_to_even():
    # 1 + 2^-8 is exactly halfway between bf16 neighbours 1 and 1 + 2^-7: ties to 1.0
    assert O.round_to(np.float32(1.0 + 2**-8), "bf16") == np.float32(1.0)
    # 1 + 3*2^-8 is halfway between 1+2^-7 and 1+2^-6: ties to even (1 + 2^-6)
    assert O.round_to(np.float32(1.0 + 3 * 2**-8), "bf16") == np.float32(1.0 + 2**-6)


# ---------------------------------------------------------------- rms


def test_rms_constant_row_closed_form():
    c, eps = 3.0, 1e-5
    x = np.full((1, 64), c, np.float32)
    w = as_dtype(RNG.standard_normal(64), "f16")
    y = O.rms_norm(x, w, eps, "f32")
    np.testing.assert_allclose(y, (c * w / np.sqrt(c * c + eps))[None], rtol=1e-6)
    assert np.all(O.rms_norm(np.zeros((2, 8), np.float32), np.ones(8, np.float32), 1e-6, "f16") == 0)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_rms_matches_torch_rms_norm(dtype):
    x = as_dtype(RNG.standard_normal((7, 300)), dtype)
    w = as_dtype(1 + 0.1 * RNG.standard_normal(300), dtype)
    ours = O.rms_norm(x, w, 1e-5, "f32")
    lib = F.rms_norm(torch.from_numpy(x), (300,), torch.from_numpy(w), 1e-5).numpy()
    np.testing.assert_allclose(ours, lib, rtol=2e-6, atol=1e-6)


def test_rms_float64_brute_force():
    x = as_dtype(RNG.standard_normal((3, 5)), "f16")
    w = as_dtype(RNG.standard_normal(5), "f16")
    eps = 1e-6
    exp = np.empty((3, 5))
    for r in range(3):
        ss = sum(float(v) ** 2 for v in x[r])
        inv = 1.0 / np.sqrt(ss / 5 + eps)
        for c in range(5):
            exp[r, c] = float(x[r, c]) * inv * float(w[c])
    np.testing.assert_allclose(O.rms_norm(x, w, eps, "f32"), exp, rtol=1e-6, atol=1e-7)


def test_add_rms_uses_float32_sum_and_reduces_to_rms():
    x = as_dtype(RNG.standard_normal((4, 256)), "f16")
    r = as_dtype(RNG.standard_normal((4, 256)), "f16")
    w = as_dtype(RNG.standard_normal(256), "f16")
    y, ro = O.add_rms_norm(x, r, w, 1e-6, "f16")
    np.testing.assert_array_equal(ro, torch_round(x + r, "f16"))
    # residual = 0 reduces to plain rms
    y0, _ = O.add_rms_norm(x, np.zeros_like(x), w, 1e-6, "f16")
    np.testing.assert_array_equal(y0, O.rms_norm(x, w, 1e-6, "f16"))
    # the norm sees the fp32 sum: equals rms of the unrounded sum
    np.testing.assert_array_equal(y, O.rms_norm(x + r, w, 1e-6, "f16"))
    lib = F.rms_norm(torch.from_numpy(x + r), (256,), torch.from_numpy(w), 1e-6).to(torch.float16).float().numpy()
    np.testing.assert_allclose(y, lib, rtol=1e-3, atol=1e-3)


# ---------------------------------------------------------------- swiglu


def test_silu_special_values_and_library():
    g = np.array([-1e4, -100.0, -20.0, -1.0, 0.0, 1.0, 20.0, 100.0, 6e4], np.float32)
    s = O.silu(g)
    assert np.all(np.isfinite(s))
    assert s[4] == 0.0
    np.testing.assert_allclose(s[-2:], g[-2:], rtol=1e-6)  # large g: silu(g) ~ g
    assert abs(s[0]) < 1e-30  # large negative: ~0, no NaN
    gg = RNG.standard_normal(5000).astype(np.float32) * 4
    np.testing.assert_allclose(O.silu(gg), F.silu(torch.from_numpy(gg)).numpy(), rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_swiglu_matches_library(dtype):
    g = as_dtype(2 * RNG.standard_normal((3, 1000)), dtype)
    u = as_dtype(2 * RNG.standard_normal((3, 1000)), dtype)
    lib = (F.silu(torch.from_numpy(g)) * torch.from_numpy(u)).numpy()
    ulp = 2.0**-10 if dtype == "f16" else 2.0**-7  # one unit in the last place, relative
    np.testing.assert_allclose(O.swiglu(g, u, dtype), torch_round(lib, dtype), rtol=ulp, atol=1e-6)
    assert np.all(O.swiglu(np.zeros_like(g), u, dtype) == 0)


# ---------------------------------------------------------------- rope


def test_rope_identity_and_quarter_turn():
    x = as_dtype(RNG.standard_normal((2, 3, 16)), "f16")
    one, zero = np.ones(16, np.float32), np.zeros(16, np.float32)
    np.testing.assert_array_equal(O.rope(x, one, zero, "f16"), x)
    q = O.rope(x, zero, one, "f16")
    np.testing.assert_array_equal(q, np.concatenate([-x[..., 8:], x[..., :8]], -1))


def _tables(pos, dim=128, theta=500000.0):
    inv = 1.0 / theta ** (np.arange(0, dim, 2, dtype=np.float64) / dim)
    ang = np.outer(np.asarray(pos, np.float64), inv)
    emb = np.concatenate([ang, ang], -1)
    return np.cos(emb), np.sin(emb), ang


def test_rope_equals_complex_rotation():
    """Rotate-half RoPE is multiplication of (x[j] + i x[j+h]) by exp(i*angle_j)."""
    pos = np.arange(6)
    cos, sin, ang = _tables(pos)
    x = RNG.standard_normal((6, 4, 128)).astype(np.float32)
    y = O.rope(x, cos[:, None, :].astype(np.float32), sin[:, None, :].astype(np.float32), "f32")
    z = (x[..., :64] + 1j * x[..., 64:]) * np.exp(1j * ang)[:, None, :]
    np.testing.assert_allclose(y, np.concatenate([z.real, z.imag], -1), rtol=1e-5, atol=1e-5)


def test_rope_composition_is_addition_of_positions():
    p, q = 700, 324
    cp, sp, _ = _tables([p])
    cq, sq, _ = _tables([q])
    cpq, spq, _ = _tables([p + q])
    x = RNG.standard_normal((1, 128))
    twice = O.rope(O.rope(x, cp, sp, "f32"), cq, sq, "f32")
    once = O.rope(x, cpq, spq, "f32")
    np.testing.assert_allclose(twice, once, rtol=1e-4, atol=1e-4)


# ---------------------------------------------------------------- linear


def test_linear_identity_and_float64():
    x = as_dtype(RNG.standard_normal((3, 32)), "f16")
    np.testing.assert_array_equal(O.linear(x, np.eye(32, dtype=np.float32), dtype="f16"), x)
    w = as_dtype(RNG.standard_normal((48, 32)) / 6, "f16")
    b = as_dtype(RNG.standard_normal(48), "f16")
    r = as_dtype(RNG.standard_normal((3, 48)), "f16")
    exp = x.astype(np.float64) @ w.T.astype(np.float64) + b + r
    np.testing.assert_allclose(O.linear(x, w, b, r, dtype="f32"), exp, rtol=1e-5, atol=1e-5)
    lib = F.linear(torch.from_numpy(x), torch.from_numpy(w), torch.from_numpy(b)).numpy() + r
    np.testing.assert_allclose(O.linear(x, w, b, r, dtype="f32"), lib, rtol=1e-6, atol=1e-6)


def test_linear_row_add_broadcast():
    x = as_dtype(RNG.standard_normal((4, 8)), "f16")
    w = as_dtype(RNG.standard_normal((5, 8)), "f16")
    r = as_dtype(RNG.standard_normal((4, 1)), "f16")
    np.testing.assert_allclose(O.linear(x, w, None, r, "f32"), x @ w.T + r, rtol=1e-6)


# ---------------------------------------------------------------- mlp


def test_post_attn_mlp_known_answer():
    """Gate rows select normed coordinates, up rows are constants: the answer is
    computable by hand from rms, silu and the residual."""
    h, i = 8, 4
    hidden = np.array([[1, -2, 3, 0.5, 0, 2, -1, 1]], np.float32)
    norm_w = np.ones(h, np.float32)
    w_gu = np.zeros((2 * i, h), np.float32)
    for j in range(i):
        w_gu[j, j] = 1.0          # gate_j = normed[j]
        w_gu[i + j, :] = 0.0
        w_gu[i + j, 7] = 2.0      # up_j = 2 * normed[7]
    w_down = np.zeros((h, i), np.float32)
    w_down[0, :] = 1.0            # out[0] = sum_j mid_j
    rms = np.sqrt(np.mean(hidden.astype(np.float64) ** 2) + 1e-6)
    normed = hidden[0] / rms
    mids = [normed[j] / (1 + np.exp(-normed[j])) * 2 * normed[7] for j in range(i)]
    exp = hidden.astype(np.float64).copy()
    exp[0, 0] += sum(mids)
    y = O.post_attn_mlp(hidden, norm_w, w_gu, w_down, 1e-6, "f32")
    np.testing.assert_allclose(y, exp, rtol=1e-5, atol=1e-5)


def test_post_attn_mlp_matches_torch_formula():
    h, i, m = 64, 96, 3
    hid = as_dtype(RNG.standard_normal((m, h)), "f16")
    nw = as_dtype(1 + 0.1 * RNG.standard_normal(h), "f16")
    wgu = as_dtype(RNG.standard_normal((2 * i, h)) / 8, "f16")
    wd = as_dtype(RNG.standard_normal((h, i)) / 10, "f16")
    T = lambda a: torch.from_numpy(a)  # noqa: E731
    hn = F.rms_norm(T(hid), (h,), T(nw), 1e-6).half().float()
    gu = F.linear(hn, T(wgu)).half().float()
    mid = (F.silu(gu[:, :i]) * gu[:, i:]).half().float()
    lib = (F.linear(mid, T(wd)) + T(hid)).half().float().numpy()
    np.testing.assert_allclose(O.post_attn_mlp(hid, nw, wgu, wd, 1e-6, "f16"), lib, rtol=2e-3, atol=2e-3)


# ---------------------------------------------------------------- pre-attention QKV


def _qkv_case(m=3, h=32, d=16, heads=3, kv=1, seed=0):
    r = np.random.default_rng(seed)
    n = (heads + 2 * kv) * d
    hid = r.standard_normal((m, h)).astype(np.float32)
    nw = (1 + 0.1 * r.standard_normal(h)).astype(np.float32)
    w = (r.standard_normal((n, h)) / np.sqrt(h)).astype(np.float32)
    return hid, nw, w, (heads + kv) * d, d


def test_pre_attn_qkv_quarter_turn_swaps_head_halves():
    """cos = 0, sin = 1 turns every rotated head (x1, x2) into (-x2, x1) exactly and
    leaves the v columns alone: pins the head split at D, the partner column
    d + D/2 and the signs, against the same call with no rotation."""
    hid, nw, w, rc, d = _qkv_case()
    plain = O.pre_attn_qkv(hid, nw, w, np.ones(d), np.zeros(d), 1e-6, 0, dtype="f32")
    turned = O.pre_attn_qkv(hid, nw, w, np.zeros(d), np.ones(d), 1e-6, rc, dtype="f32")
    for head in range(rc // d):
        a, b = plain[:, head * d: head * d + d // 2], plain[:, head * d + d // 2: (head + 1) * d]
        np.testing.assert_array_equal(turned[:, head * d: head * d + d // 2], -b)
        np.testing.assert_array_equal(turned[:, head * d + d // 2: (head + 1) * d], a)
    np.testing.assert_array_equal(turned[:, rc:], plain[:, rc:])
    # no rotation at all equals a zero rope_cols call
    same = O.pre_attn_qkv(hid, nw, w, np.ones(d), np.zeros(d), 1e-6, rc, dtype="f32")
    np.testing.assert_array_equal(same, plain)


def test_pre_attn_qkv_matches_torch_composition_and_per_row_angles():
    """Against torch CPU library routines (F.rms_norm, F.linear, complex rotation),
    with one position per row: row m uses angle row m."""
    hid, nw, w, rc, d = _qkv_case(m=4, seed=3)
    pos = np.array([3.0, 17.0, 250.0, 1024.0])
    inv = 500000.0 ** (-np.arange(0, d, 2) / d)
    ang = pos[:, None] * inv[None]
    cos = np.concatenate([np.cos(ang), np.cos(ang)], 1).astype(np.float32)
    sin = np.concatenate([np.sin(ang), np.sin(ang)], 1).astype(np.float32)
    bias = np.linspace(-1, 1, w.shape[0]).astype(np.float32)
    got = O.pre_attn_qkv(hid, nw, w, cos, sin, 1e-5, rc, bias=bias, dtype="f32")
    T = lambda a: torch.from_numpy(a).double()  # noqa: E731
    hn = F.rms_norm(T(hid), (hid.shape[1],), T(nw), 1e-5)
    y = F.linear(hn, T(w), T(bias)).numpy()
    exp = y.copy()
    for head in range(rc // d):
        x1 = y[:, head * d: head * d + d // 2]
        x2 = y[:, head * d + d // 2: (head + 1) * d]
        z = (x1 + 1j * x2) * np.exp(1j * ang)
        exp[:, head * d: head * d + d // 2] = z.real
        exp[:, head * d + d // 2: (head + 1) * d] = z.imag
    np.testing.assert_allclose(got, exp, rtol=1e-4, atol=1e-4)
    # a per-row call equals four single-row calls with that row's angles (to the
    # last bit of a float32 matmul, whose summation order depends on the row count)
    for r in range(4):
        one = O.pre_attn_qkv(hid[r:r + 1], nw, w, cos[r], sin[r], 1e-5, rc, bias=bias, dtype="f32")
        np.testing.assert_allclose(one[0], got[r], rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------- fp8 weights


def test_fp8_decode_matches_torch_for_every_code():
    codes = np.arange(256, dtype=np.uint8)
    ours = O.fp8_decode(codes)
    lib = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(np.isnan(ours), np.isnan(lib))
    assert np.array_equal(ours[~np.isnan(ours)], lib[~np.isnan(lib)])
    assert ours[0x7E] == 448.0 and ours[0x01] == 2.0 ** -9 and ours[0x08] == 2.0 ** -6


def test_fp8_encode_matches_torch_rounding_and_saturates():
    grid = O.fp8_decode(np.arange(0x7F, dtype=np.uint8))
    ties = (grid[:-1] + grid[1:]) / 2  # every midpoint: round half to even
    v = np.concatenate([RNG.standard_normal(20000).astype(np.float32) * 60, grid, ties, -ties]).astype(np.float32)
    lib = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(O.fp8_encode(v), lib)
    assert O.fp8_encode(np.array([1000.0, -1e9], np.float32)).tolist() == [0x7E, 0xFE]  # saturation, not NaN


def test_fp8_quantize_scale_and_error_bound():
    w = RNG.standard_normal((16, 256)).astype(np.float32) * np.linspace(0.01, 3, 16, dtype=np.float32)[:, None]
    w[3] = 0.0
    codes, scale = O.fp8_quantize(w)
    deq = O.fp8_decode(codes) * scale[:, None]
    assert scale[3] == 1.0 and not deq[3].any()
    rows = [r for r in range(16) if r != 3]
    assert np.allclose(np.abs(deq[rows]).max(1), np.abs(w[rows]).max(1), rtol=1e-6)  # amax maps to 448
    # E4M3 keeps 3 mantissa bits: relative error <= 2^-4 in the normal range,
    # absolute <= 2^-10 * scale in the subnormal range
    err = np.abs(deq - w)
    bound = np.maximum(np.abs(w) * 2.0 ** -4, scale[:, None] * 2.0 ** -10) * (1 + 1e-6)
    assert (err <= bound).all()


def test_linear_fp8_against_float64_and_the_dequantized_product():
    x = as_dtype(RNG.standard_normal((3, 96)), "f16")
    codes, scale = O.fp8_quantize(RNG.standard_normal((40, 96)).astype(np.float32) / 10)
    bias = RNG.standard_normal(40).astype(np.float32)
    got = O.linear_fp8(x, codes, scale, bias=bias, dtype="f32")
    exp = (x.astype(np.float64) @ O.fp8_decode(codes).astype(np.float64).T) * scale + bias
    np.testing.assert_allclose(got, exp, rtol=1e-5, atol=1e-5)
    deq = O.fp8_decode(codes) * scale[:, None]
    np.testing.assert_allclose(got, O.linear(x, deq, bias=bias, dtype="f32"), rtol=1e-5, atol=1e-5)
    # a planted mistake: scaling the weights' rows by the wrong channel's scale
    bad = (x @ O.fp8_decode(codes).T) * scale[::-1] + bias
    assert not np.allclose(bad, exp, rtol=1e-3)


def test_post_attn_mlp_fp8_equals_mlp_of_dequantized_weights():
    h, i, m = 64, 96, 2
    hid = as_dtype(RNG.standard_normal((m, h)), "f16")
    nw = as_dtype(1 + 0.1 * RNG.standard_normal(h), "f16")
    gq, gs = O.fp8_quantize(RNG.standard_normal((2 * i, h)).astype(np.float32) / 8)
    dq, ds = O.fp8_quantize(RNG.standard_normal((h, i)).astype(np.float32) / 10)
    got = O.post_attn_mlp_fp8(hid, nw, gq, gs, dq, ds, 1e-6, "f16")
    ref = O.post_attn_mlp(hid, nw, O.fp8_decode(gq) * gs[:, None], O.fp8_decode(dq) * ds[:, None], 1e-6, "f16")
    np.testing.assert_allclose(got, ref, rtol=2e-3, atol=2e-3)


def test_pre_attn_qkv_fp8_equals_qkv_of_dequantized_weights_and_rotates():
    """The fp8 QKV is the fp16 composition over the decoded weights (to float32
    rounding of where the scale is applied), and its RoPE is the same rotation:
    a quarter turn swaps head halves exactly. Reversed scales are caught."""
    hid, nw, w, rc, d = _qkv_case(m=3, seed=5)
    codes, scale = O.fp8_quantize(w)
    deq = O.fp8_decode(codes) * scale[:, None]
    bias = np.linspace(-0.5, 0.5, w.shape[0]).astype(np.float32)
    cos = RNG.standard_normal(d).astype(np.float32)
    sin = RNG.standard_normal(d).astype(np.float32)
    got = O.pre_attn_qkv_fp8(hid, nw, codes, scale, cos, sin, 1e-5, rc, bias=bias, dtype="f32")
    ref = O.pre_attn_qkv(hid, nw, deq, cos, sin, 1e-5, rc, bias=bias, dtype="f32")
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)
    bad = O.pre_attn_qkv_fp8(hid, nw, codes, scale[::-1].copy(), cos, sin, 1e-5, rc, bias=bias, dtype="f32")
    assert not np.allclose(bad, ref, rtol=1e-3, atol=1e-3)
    plain = O.pre_attn_qkv_fp8(hid, nw, codes, scale, np.ones(d), np.zeros(d), 1e-5, 0, dtype="f32")
    turned = O.pre_attn_qkv_fp8(hid, nw, codes, scale, np.zeros(d), np.ones(d), 1e-5, rc, dtype="f32")
    for head in range(rc // d):
        a, b = plain[:, head * d: head * d + d // 2], plain[:, head * d + d // 2: (head + 1) * d]
        np.testing.assert_array_equal(turned[:, head * d: head * d + d // 2], -b)
        np.testing.assert_array_equal(turned[:, head * d + d // 2: (head + 1) * d], a)
    np.testing.assert_array_equal(turned[:, rc:], plain[:, rc:])


# ---------------------------------------------------------------- bytes


def test_useful_bytes_match_the_readme_byte_rules():
    assert O.bytes_add_rms(8192, 4096) == 268_443_648
    assert O.bytes_rms(8192, 4096) == 134_225_920
    assert O.bytes_swiglu(2048, 14336) == 176_160_768
    assert O.bytes_rope(2048 * 32 * 128, 2048 * 128, 2048 * 128) == 34_603_008
    assert O.bytes_linear(1, 4096, 4096) == 33_570_816
    assert O.bytes_linear(1, 4096, 14336) == 117_477_376
    assert O.bytes_linear(1, 28672, 4096) == 234_946_560
    assert O.bytes_mlp(1, 4096, 14336) == 352_346_112
    assert O.bytes_mlp(8, 4096, 14336) == 352_460_800


# ---------------------------------------------------------------- planted mistakes


def test_planted_mistakes_are_caught():
    """Plausible slips in the oracle fail the checks above."""
    x = as_dtype(RNG.standard_normal((2, 64)), "f16")
    w = as_dtype(RNG.standard_normal(64), "f16")
    lib = F.rms_norm(torch.from_numpy(x), (64,), torch.from_numpy(w), 1e-5).numpy()
    # variance with a dropped 1/N
    bad = x / np.sqrt(np.sum(x * x, -1, keepdims=True) + 1e-5) * w
    assert not np.allclose(bad, lib, rtol=1e-3)
    # rope with the sign of the sine term flipped
    cos, sin, ang = _tables([5])
    xr = RNG.standard_normal((1, 128)).astype(np.float32)
    h = 64
    wrong = np.concatenate([xr[:, :h] * cos[:, :h] + xr[:, h:] * sin[:, :h], xr[:, h:] * cos[:, h:] - xr[:, :h] * sin[:, h:]], -1)
    z = (xr[:, :h] + 1j * xr[:, h:]) * np.exp(1j * ang)
    assert not np.allclose(wrong, np.concatenate([z.real, z.imag], -1), atol=1e-3)
    # linear with a transposed weight (square case)
    wsq = as_dtype(RNG.standard_normal((16, 16)), "f16")
    xs = as_dtype(RNG.standard_normal((2, 16)), "f16")
    assert not np.allclose(xs @ wsq, F.linear(torch.from_numpy(xs), torch.from_numpy(wsq)).numpy(), atol=1e-3)
