"""GPU parity tests: the HIP operators against the CPU oracle on identical seeded
inputs (generated on the CPU, then copied to the GPU).

Tolerances are the reference's (tests/test_ops.py:27-35): GEMV outputs fp16
rtol=atol=2e-2, bf16 4e-2; pointwise fp16 rtol 1e-2 / atol 5e-3, bf16 2e-2.
The cases mirror the reference's tests (tests/test_ops.py:42-187) and add the
benchmark configurations at full size, every M in 1..16, and graph capture.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import decode_oracle as O

pytestmark = pytest.mark.gpu

DTYPES = [torch.float16, torch.bfloat16]
DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _lib_loaded():
    import fused_decode._lib as L

    L.lib()  # raises if the HIP library is missing: no silent fallback


def fd():
    import fused_decode

    return fused_decode


def tag(dtype) -> str:
    return "f16" if dtype == torch.float16 else "bf16"


def tol(dtype, kind="pointwise"):
    if kind == "linear":
        return {"rtol": 2e-2, "atol": 2e-2} if dtype == torch.float16 else {"rtol": 4e-2, "atol": 4e-2}
    return {"rtol": 1e-2, "atol": 5e-3} if dtype == torch.float16 else {"rtol": 2e-2, "atol": 2e-2}


def randn(*shape, dtype=torch.float16, seed=0, scale=1.0, mean=0.0, gen=None):
    g = gen or torch.Generator().manual_seed(seed)
    t = torch.randn(*shape, generator=g, dtype=torch.float32) * scale + mean
    return t.to(dtype)


def npf(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def check(actual: torch.Tensor, expected: np.ndarray, dtype, kind="pointwise"):
    assert actual.is_cuda
    torch.testing.assert_close(actual.float().cpu(), torch.from_numpy(np.ascontiguousarray(expected)), **tol(dtype, kind))


# ---------------------------------------------------------------- norms


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(4, 128), (1, 4096), (3, 3072), (5, 100), (2, 8, 64)])
def test_rms_norm(dtype, shape):
    x = randn(*shape, dtype=dtype, seed=0)
    w = randn(shape[-1], dtype=dtype, seed=100)
    y = fd().rms_norm(x.to(DEV), w.to(DEV))
    check(y, O.rms_norm(npf(x), npf(w), 1e-6, tag(dtype)), dtype)


@pytest.mark.parametrize("dtype", DTYPES)
def test_rms_norm_strided_and_fp32_weight(dtype):
    base = randn(32, 48, dtype=dtype, seed=1).to(DEV)
    x = base.t()
    assert x.stride(-1) != 1
    w = randn(x.shape[-1], dtype=torch.float32, seed=2).to(DEV)
    check(fd().rms_norm(x, w), O.rms_norm(npf(x), npf(w), 1e-6, tag(dtype)), dtype)

    y = randn(7, 9, 32, dtype=dtype, seed=3).to(DEV).transpose(0, 1)
    assert not y.is_contiguous()
    wy = torch.ones(y.shape[-1], device=DEV, dtype=dtype)
    check(fd().rms_norm(y, wy), O.rms_norm(npf(y), npf(wy), 1e-6, tag(dtype)), dtype)


@pytest.mark.parametrize("dtype", DTYPES)
def test_add_rms_norm_inplace(dtype):
    x = randn(6, 256, dtype=dtype, seed=2).to(DEV)
    residual = randn(6, 256, dtype=dtype, seed=3).to(DEV)
    w = randn(256, dtype=dtype, seed=4).to(DEV)
    y_ref, r_ref = O.add_rms_norm(npf(x), npf(residual), npf(w), 1e-6, tag(dtype))
    y, residual_out = fd().add_rms_norm(x, residual, w)
    check(y, y_ref, dtype)
    check(residual_out, r_ref, dtype)

    residual2 = residual.clone()
    y2, residual_back = fd().add_rms_norm(x, residual2, w, residual_out=residual2)
    assert residual_back.data_ptr() == residual2.data_ptr()
    check(y2, y_ref, dtype)
    check(residual2, r_ref, dtype)


def test_rms_two_pass():
    x = randn(2, 9000, dtype=torch.float16, seed=3).to(DEV)
    w = randn(9000, dtype=torch.float16, seed=5).to(DEV)
    check(fd().rms_norm(x, w), O.rms_norm(npf(x), npf(w), 1e-6, "f16"), torch.float16)


def test_rms_norm_in_place_and_out_param():
    x = randn(3, 512, seed=6).to(DEV)
    w = randn(512, seed=7, scale=0.1, mean=1.0).to(DEV)
    expected = O.rms_norm(npf(x), npf(w), 1e-5, "f16")
    out = torch.empty_like(x)
    r = fd().rms_norm(x, w, 1e-5, out=out)
    assert r.data_ptr() == out.data_ptr()
    check(out, expected, torch.float16)
    fd().rms_norm(x, w, 1e-5, out=x)  # out aliases x
    check(x, expected, torch.float16)


def test_rms_norm_unexpressible_out_is_written():
    x = randn(2, 3, 4, 5, 64, seed=8).to(DEV)
    w = randn(64, seed=9).to(DEV)
    out = torch.zeros(5, 4, 3, 2, 64, device=DEV, dtype=torch.float16).permute(3, 2, 1, 0, 4)
    fd().rms_norm(x, w, out=out)
    check(out, O.rms_norm(npf(x), npf(w), 1e-6, "f16"), torch.float16)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows", [8192, 1])
def test_add_rms_norm_config(dtype, rows):
    """Benchmark configuration: [rows, 4096], eps 1e-5, residual updated in place."""
    g = torch.Generator().manual_seed(11)
    x = randn(rows, 4096, dtype=dtype, gen=g)
    r = randn(rows, 4096, dtype=dtype, gen=g)
    w = randn(4096, dtype=dtype, gen=g, scale=0.1, mean=1.0)
    y_ref, r_ref = O.add_rms_norm(npf(x), npf(r), npf(w), 1e-5, tag(dtype))
    rd = r.to(DEV)
    y, ro = fd().add_rms_norm(x.to(DEV), rd, w.to(DEV), 1e-5, residual_out=rd)
    assert ro.data_ptr() == rd.data_ptr()
    check(y, y_ref, dtype)
    check(rd, r_ref, dtype)
    y1 = fd().rms_norm(x.to(DEV), w.to(DEV), 1e-5)
    check(y1, O.rms_norm(npf(x), npf(w), 1e-5, tag(dtype)), dtype)


# ---------------------------------------------------------------- rope


@pytest.mark.parametrize("dtype", DTYPES)
def test_rope_broadcast_and_transpose(dtype):
    x = randn(2, 8, 4, 128, dtype=dtype, seed=4).to(DEV)
    cos = randn(8, 1, 128, dtype=dtype, seed=5).to(DEV)
    sin = randn(8, 1, 128, dtype=dtype, seed=6).to(DEV)
    check(fd().rope(x, cos, sin), O.rope(npf(x), npf(cos), npf(sin), tag(dtype)), dtype)

    transposed = randn(2, 4, 8, 64, dtype=dtype, seed=7).to(DEV).transpose(1, 2)
    assert not transposed.is_contiguous()
    cos_t = randn(1, 8, 1, 64, dtype=torch.float32, seed=8).to(DEV)
    sin_t = randn(1, 8, 1, 64, dtype=torch.float32, seed=9).to(DEV)
    check(fd().rope(transposed, cos_t, sin_t), O.rope(npf(transposed), npf(cos_t), npf(sin_t), tag(dtype)), dtype)


def llama3_tables(positions: int, dim: int = 128, theta: float = 500000.0):
    inv_freq = 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float64) / dim))
    pos = torch.arange(positions, dtype=torch.float64)
    freqs = torch.outer(pos, inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos(), emb.sin()


@pytest.mark.parametrize("dtype", DTYPES)
def test_rope_config(dtype):
    """[1, 2048, 32, 128] with Llama-3 tables viewed [2048, 1, 128]; one token at position 1024."""
    cos, sin = llama3_tables(2048)
    cos, sin = cos.to(dtype), sin.to(dtype)
    x = randn(1, 2048, 32, 128, dtype=dtype, seed=12)
    c3, s3 = cos.view(2048, 1, 128), sin.view(2048, 1, 128)
    y = fd().rope(x.to(DEV), c3.to(DEV), s3.to(DEV))
    check(y, O.rope(npf(x), npf(c3), npf(s3), tag(dtype)), dtype)
    x1 = randn(1, 1, 32, 128, dtype=dtype, seed=13)
    c1, s1 = cos[1024].view(1, 1, 128), sin[1024].view(1, 1, 128)
    y1 = fd().rope(x1.to(DEV), c1.to(DEV), s1.to(DEV))
    check(y1, O.rope(npf(x1), npf(c1), npf(s1), tag(dtype)), dtype)


def test_rope_mixed_angle_dtypes_and_odd_half():
    x = randn(3, 5, 12, seed=14).to(DEV)  # half = 6: not a multiple of 8 -> generic kernel
    cos = randn(5, 12, dtype=torch.float32, seed=15).to(DEV)
    sin = randn(5, 12, dtype=torch.float16, seed=16).to(DEV)
    check(fd().rope(x, cos, sin), O.rope(npf(x), npf(cos), npf(sin), "f16"), torch.float16)


# ---------------------------------------------------------------- swiglu


@pytest.mark.parametrize("dtype", DTYPES)
def test_swiglu_strided_halves(dtype):
    packed = randn(3, 256, dtype=dtype, seed=5).to(DEV)
    gate, up = packed.split(128, dim=-1)
    assert not gate.is_contiguous()
    check(fd().swiglu(gate, up), O.swiglu(npf(gate), npf(up), tag(dtype)), dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows", [2048, 1])
def test_swiglu_config(dtype, rows):
    g = torch.Generator().manual_seed(17)
    gate = randn(rows, 14336, dtype=dtype, gen=g, scale=2.0)
    up = randn(rows, 14336, dtype=dtype, gen=g, scale=2.0)
    check(fd().swiglu(gate.to(DEV), up.to(DEV)), O.swiglu(npf(gate), npf(up), tag(dtype)), dtype)


def test_swiglu_extremes_no_nan():
    gate = torch.tensor([[-60000.0, -80.0, -1.0, 0.0, 1.0, 80.0, 300.0, 60000.0]], dtype=torch.float16)
    up = torch.ones_like(gate) * 0.5
    y = fd().swiglu(gate.to(DEV), up.to(DEV))
    assert torch.isfinite(y.float()).all()
    check(y, O.swiglu(npf(gate), npf(up), "f16"), torch.float16)


# ---------------------------------------------------------------- linear


def _linear_case(m, n, k, dtype, seed, bias=False):
    g = torch.Generator().manual_seed(seed)
    x = randn(m, k, dtype=dtype, gen=g, scale=k ** -0.5)
    w = randn(n, k, dtype=dtype, gen=g, scale=k ** -0.5)
    b = randn(n, dtype=dtype, gen=g) if bias else None
    return x, w, b


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("kind", ["dot", "simt"])
@pytest.mark.parametrize("m,n,k", [(1, 64, 100), (3, 128, 128), (8, 256, 64), (6, 48, 8), (5, 40, 24),
                                   (1, 40, 8)])
def test_linear_small(dtype, kind, m, n, k):
    """Small and ragged shapes, including K below one MFMA unit (128) and one B
    fragment group (32), where most lanes of a unit lie past K."""
    x, w, b = _linear_case(m, n, k, dtype, 6, bias=True)
    y = fd().linear_decode(x.to(DEV), w.to(DEV), b.to(DEV), kind=kind)
    check(y, O.linear(npf(x), npf(w), npf(b), dtype=tag(dtype)), dtype, "linear")


@pytest.mark.parametrize("kind", ["dot", "simt"])
def test_linear_decode_shape_and_strided_weight(kind):
    dtype = torch.float16
    x, w, _ = _linear_case(1, 1024, 4096, dtype, 7)
    check(fd().linear_decode(x.to(DEV), w.to(DEV), kind=kind), O.linear(npf(x), npf(w), dtype="f16"), dtype, "linear")

    raw = randn(128, 64, seed=70).to(DEV)
    w_t = raw.t()
    assert not w_t.is_contiguous()
    x2 = randn(4, 128, seed=71, scale=128 ** -0.5).to(DEV)
    row = randn(4, 64, seed=72).to(DEV)
    y = fd().linear_decode(x2, w_t, row_add=row, kind=kind)
    check(y, O.linear(npf(x2), npf(w_t), row_add=npf(row), dtype="f16"), dtype, "linear")


def test_linear_fallback_matches_hipblas():
    """Above the GEMV row limit the result is F.linear itself (bit-exact)."""
    g = torch.Generator().manual_seed(8)
    x = randn(20, 32, gen=g).to(DEV)
    w = randn(48, 32, gen=g).to(DEV)
    bias = randn(48, gen=g).to(DEV)
    y = fd().linear_decode(x, w, bias)
    torch.testing.assert_close(y, F.linear(x, w, bias), rtol=0, atol=0)
    row = randn(20, 48, gen=g).to(DEV)
    fused = fd().linear_decode(x, w, row_add=row)
    manual = F.linear(x, w) + row
    torch.testing.assert_close(fused, manual, rtol=1e-3, atol=1e-3)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("kind", ["dot", "simt"])
def test_linear_every_m(dtype, kind):
    """M = 1..16 through both kinds (MFMA for dot from 5 rows), with bias and row_add."""
    for m in range(1, 17):
        x, w, b = _linear_case(m, 200, 1536, dtype, 100 + m, bias=True)
        ra = randn(m, 200, dtype=dtype, seed=200 + m)
        y = fd().linear_decode(x.to(DEV), w.to(DEV), b.to(DEV), row_add=ra.to(DEV), kind=kind)
        check(y, O.linear(npf(x), npf(w), npf(b), npf(ra), dtype=tag(dtype)), dtype, "linear")


@pytest.mark.parametrize("kind", ["dot", "simt"])
def test_linear_epilogue_dtypes_and_broadcast(kind):
    """fp32 bias, fp32 row_add broadcast [1, N] and [M, 1], 3-D x, out= param."""
    m, n, k = 8, 96, 512
    x, w, _ = _linear_case(m, n, k, torch.bfloat16, 31)
    b32 = randn(n, dtype=torch.float32, seed=32)
    r1n = randn(1, n, dtype=torch.float32, seed=33)
    rm1 = randn(m, 1, dtype=torch.float16, seed=34)
    xd, wd = x.to(DEV), w.to(DEV)
    y = fd().linear_decode(xd, wd, b32.to(DEV), row_add=r1n.to(DEV), kind=kind)
    check(y, O.linear(npf(x), npf(w), npf(b32), npf(r1n), dtype="bf16"), torch.bfloat16, "linear")
    y = fd().linear_decode(xd, wd, row_add=rm1.to(DEV), kind=kind)
    check(y, O.linear(npf(x), npf(w), None, npf(rm1), dtype="bf16"), torch.bfloat16, "linear")
    x3 = xd.view(2, 4, k)
    out = torch.empty(2, 4, n, device=DEV, dtype=torch.bfloat16)
    y3 = fd().linear_decode(x3, wd, out=out, kind=kind)
    assert y3.data_ptr() == out.data_ptr()
    check(out.view(m, n), O.linear(npf(x), npf(w), dtype="bf16"), torch.bfloat16, "linear")


def test_linear_unaligned_and_empty():
    # x offset by one element: not 16-byte aligned -> generic kernel
    big = randn(1, 4097, seed=40, scale=4096 ** -0.5).to(DEV)
    x = big[:, 1:]
    w = randn(64, 4096, seed=41, scale=4096 ** -0.5).to(DEV)
    check(fd().linear_decode(x, w, kind="simt"), O.linear(npf(x), npf(w), dtype="f16"), torch.float16, "linear")
    e = fd().linear_decode(torch.empty(0, 64, device=DEV, dtype=torch.float16), torch.empty(8, 64, device=DEV, dtype=torch.float16), kind="dot")
    assert e.shape == (0, 8)
    z = fd().linear_decode(torch.empty(2, 64, device=DEV, dtype=torch.float16), torch.empty(0, 64, device=DEV, dtype=torch.float16), kind="dot")
    assert z.shape == (2, 0)


def test_linear_k0_is_the_epilogue():
    """K = 0: y = round(bias + row_add) with x and the weights never read (x is
    null through the C entry point), for the SIMT (M < 5) and MFMA forms."""
    from fused_decode import _lib as L

    n = 40
    w = torch.zeros(n, 8, device=DEV, dtype=torch.float16)  # aligned, never read at K = 0
    st = torch.cuda.current_stream().cuda_stream
    for m in (1, 3, 6):
        bias = randn(n, seed=50 + m).to(DEV)
        ra = randn(m, n, seed=60 + m).to(DEV)
        exp = O.linear(np.zeros((m, 0), np.float32), np.zeros((n, 0), np.float32), bias=npf(bias),
                       row_add=npf(ra), dtype="f16")
        for kind in (L.FD_KIND_DOT, L.FD_KIND_SIMT):
            y = torch.full((m, n), float("nan"), device=DEV, dtype=torch.float16)
            L.check("fd_linear", L.lib().fd_linear(
                y.data_ptr(), None, w.data_ptr(), bias.data_ptr(), L.FD_F16, ra.data_ptr(), L.FD_F16,
                m, n, 0, 8, 1, 8, 1, 1, n, 1, n, 1, kind, L.FD_F16, st))
            torch.testing.assert_close(y.float().cpu(), torch.from_numpy(exp), rtol=0, atol=0)
    b1 = randn(1, seed=70).to(DEV)
    y1 = fd().linear_decode(torch.empty(2, 0, device=DEV, dtype=torch.float16),
                            torch.empty(1, 0, device=DEV, dtype=torch.float16), b1, kind="simt")
    torch.testing.assert_close(y1, b1.expand(2, 1), rtol=0, atol=0)


LINEAR_CONFIGS = [(4096, 4096), (4096, 14336), (28672, 4096), (6144, 4096)]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("nk", LINEAR_CONFIGS, ids=lambda nk: f"N{nk[0]}K{nk[1]}")
def test_linear_config_shapes(dtype, nk):
    """Benchmark GEMV shapes, M in {1,2,4,8,16}, both kinds, bias and row_add."""
    n, k = nk
    g = torch.Generator().manual_seed(50 + n + k)
    w = randn(n, k, dtype=dtype, gen=g, scale=k ** -0.5)
    b = randn(n, dtype=dtype, gen=g)
    wd, bd = w.to(DEV), b.to(DEV)
    wn, bn = npf(w), npf(b)
    for m in (1, 2, 4, 8, 16):
        x = randn(m, k, dtype=dtype, gen=g)
        ra = randn(m, n, dtype=dtype, gen=g)
        xd, rd = x.to(DEV), ra.to(DEV)
        exp_plain = O.linear(npf(x), wn, dtype=tag(dtype))
        exp_epi = O.linear(npf(x), wn, bn, npf(ra), dtype=tag(dtype))
        for kind in ("dot", "simt"):
            check(fd().linear_decode(xd, wd, kind=kind), exp_plain, dtype, "linear")
            check(fd().linear_decode(xd, wd, bd, row_add=rd, kind=kind), exp_epi, dtype, "linear")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m,n,k", [(9, 4096, 14336), (16, 4096, 14336), (12, 300, 14336), (16, 70, 9000),
                                   (2, 130, 16408), (4, 1000, 20480)])
def test_linear_simt_phases(dtype, m, n, k):
    """The persistent SIMT GEMV where K is past eight waves of the chunks per
    lane its registers hold: two or three phases, even and ragged K (the last
    phase's chunks partly or wholly past K), tiles past N and workgroups with
    no tile; bias and row_add."""
    x, w, b = _linear_case(m, n, k, dtype, 300 + m + n, bias=True)
    ra = randn(m, n, dtype=dtype, seed=400 + m)
    exp = O.linear(npf(x), npf(w), npf(b), npf(ra), dtype=tag(dtype))
    y = fd().linear_decode(x.to(DEV), w.to(DEV), b.to(DEV), row_add=ra.to(DEV), kind="simt")
    check(y, exp, dtype, "linear")


# ---------------------------------------------------------------- post_attn_mlp


def test_post_attn_mlp():
    g = torch.Generator().manual_seed(9)
    dtype = torch.float16
    x = randn(4, 64, gen=g)
    norm_w = randn(64, gen=g)
    w_gu = randn(256, 64, gen=g, scale=64 ** -0.5)
    w_down = randn(64, 128, gen=g, scale=128 ** -0.5)
    ref = O.post_attn_mlp(npf(x), npf(norm_w), npf(w_gu), npf(w_down), 1e-6, "f16")
    for kind in ("dot", "simt", None):
        y = fd().post_attn_mlp(x.to(DEV), norm_w.to(DEV), w_gu.to(DEV), w_down.to(DEV), kind=kind)
        check(y, ref, dtype, "linear")


@pytest.mark.parametrize("m", [5, 8])
def test_post_attn_mlp_wide_hidden_row_kernel_form(m):
    """H = 36864: the norm weight's float32 LDS stage no longer fits beside the
    gate/up kernel's tiles, so from 5 rows the MLP runs its norm as a row kernel
    first (three launches) instead of inside the gate/up kernel."""
    h, i = 36864, 64
    g = torch.Generator().manual_seed(95 + m)
    x = randn(m, h, gen=g)
    nw = randn(h, gen=g, scale=0.1, mean=1.0)
    w_gu = randn(2 * i, h, gen=g, scale=h ** -0.5)
    w_d = randn(h, i, gen=g, scale=i ** -0.5)
    y = fd().post_attn_mlp(x.to(DEV), nw.to(DEV), w_gu.to(DEV), w_d.to(DEV), 1e-5, kind="dot")
    check(y, O.post_attn_mlp(npf(x), npf(nw), npf(w_gu), npf(w_d), 1e-5, "f16"), torch.float16, "linear")


@pytest.mark.parametrize("m", [5, 8, 12, 16])
@pytest.mark.parametrize("i", [4096, 4104, 14336])
def test_post_attn_mlp_gate_up_tile_forms(m, i):
    """The MFMA gate/up with tiles of 16 gate + 16 up rows only (I = 4096: 256
    tiles, one round over the CUs) and with the rows past the last whole round
    in tiles of 8 + 8 (I = 4104: one such tile, 8 rows; I = 14336: 768 + 256
    tiles); the norm inside the kernel up to 8 rows, a row kernel's normalised
    rows from 9; bf16 at 8 rows."""
    h = 1024
    dtype = torch.bfloat16 if m == 8 and i == 14336 else torch.float16
    g = torch.Generator().manual_seed(i + m)
    x = randn(m, h, dtype=dtype, gen=g)
    nw = randn(h, dtype=dtype, gen=g, scale=0.1, mean=1.0)
    w_gu = randn(2 * i, h, dtype=dtype, gen=g, scale=h ** -0.5)
    w_d = randn(h, i, dtype=dtype, gen=g, scale=i ** -0.5)
    y = fd().post_attn_mlp(x.to(DEV), nw.to(DEV), w_gu.to(DEV), w_d.to(DEV), 1e-5, kind="dot")
    check(y, O.post_attn_mlp(npf(x), npf(nw), npf(w_gu), npf(w_d), 1e-5, tag(dtype)), dtype, "linear")


@pytest.mark.parametrize("dtype", DTYPES)
def test_post_attn_mlp_every_m_and_fp32_norm_weight(dtype):
    h, i = 256, 384
    g = torch.Generator().manual_seed(90)
    w_gu = randn(2 * i, h, dtype=dtype, gen=g, scale=h ** -0.5)
    w_down = randn(h, i, dtype=dtype, gen=g, scale=i ** -0.5)
    norm_w = randn(h, dtype=torch.float32, gen=g, scale=0.1, mean=1.0)
    wgd, wdd, nwd = w_gu.to(DEV), w_down.to(DEV), norm_w.to(DEV)
    for m in range(1, 17):
        x = randn(m, h, dtype=dtype, gen=g)
        ref = O.post_attn_mlp(npf(x), npf(norm_w), npf(w_gu), npf(w_down), 1e-5, tag(dtype))
        for kind in ("dot", "simt"):
            y = fd().post_attn_mlp(x.to(DEV), nwd, wgd, wdd, 1e-5, kind=kind)
            check(y, ref, dtype, "linear")


@pytest.mark.parametrize("m", [1, 2, 3, 4])
def test_post_attn_mlp_several_tiles_per_workgroup(m):
    """I = 6144 with 4-row SIMT tiles: 1536 tiles over at most two 8-wave
    workgroups per CU, so each workgroup streams several tiles (epilogues on
    alternating halves of the partial-sum buffer)."""
    h, i = 256, 6144
    g = torch.Generator().manual_seed(92 + m)
    w_gu = randn(2 * i, h, gen=g, scale=h ** -0.5)
    w_down = randn(h, i, gen=g, scale=i ** -0.5)
    norm_w = randn(h, gen=g, scale=0.1, mean=1.0)
    x = randn(m, h, gen=g)
    y = fd().post_attn_mlp(x.to(DEV), norm_w.to(DEV), w_gu.to(DEV), w_down.to(DEV), 1e-5, kind="simt")
    check(y, O.post_attn_mlp(npf(x), npf(norm_w), npf(w_gu), npf(w_down), 1e-5, "f16"), torch.float16, "linear")


@pytest.mark.parametrize("dtype", DTYPES)
def test_post_attn_mlp_strided_batched_and_composed_forms(dtype):
    """The block on inputs the fused launch does not take as they are, each
    against the oracle: a column-strided hidden (copied into place), a 3-D hidden
    [2, 3, H] (flattened rows), row-strided weight views (the composed path of
    the reference's own operators), and M = 20 above the row cutoff (the
    F.linear fallback inside linear_decode)."""
    h, i = 256, 384
    g = torch.Generator().manual_seed(91)
    w_gu = randn(2 * i, h, dtype=dtype, gen=g, scale=h ** -0.5)
    w_down = randn(h, i, dtype=dtype, gen=g, scale=i ** -0.5)
    norm_w = randn(h, dtype=dtype, gen=g, scale=0.1, mean=1.0)
    wgd, wdd, nwd = w_gu.to(DEV), w_down.to(DEV), norm_w.to(DEV)

    def ref(x):
        return O.post_attn_mlp(npf(x).reshape(-1, h), npf(norm_w), npf(w_gu), npf(w_down), 1e-5,
                               tag(dtype)).reshape(tuple(x.shape))

    wide = randn(3, 2 * h, dtype=dtype, gen=g).to(DEV)
    strided = wide[:, ::2]  # column stride 2
    assert not strided.is_contiguous()
    batched = randn(2, 3, h, dtype=dtype, gen=g).to(DEV)
    many = randn(20, h, dtype=dtype, gen=g).to(DEV)
    # row-strided views of the same weights: rows 0, 2, 4, ... of a padded copy
    pad_gu = torch.zeros(4 * i, h, dtype=dtype, device=DEV)
    pad_gu[::2] = wgd
    pad_d = torch.zeros(2 * h, i, dtype=dtype, device=DEV)
    pad_d[::2] = wdd
    for kind in ("dot", "simt"):
        for x in (strided, batched, many):
            y = fd().post_attn_mlp(x, nwd, wgd, wdd, 1e-5, kind=kind)
            assert y.shape == x.shape
            check(y, ref(x), dtype, "linear")
        y = fd().post_attn_mlp(batched, nwd, pad_gu[::2], pad_d[::2], 1e-5, kind=kind)
        check(y, ref(batched), dtype, "linear")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m", [1, 8])
def test_post_attn_mlp_llama3_8b(dtype, m):
    """Benchmark configuration: H=4096, I=14336, residual fused, both kinds."""
    h, i = 4096, 14336
    g = torch.Generator().manual_seed(1000 + m)
    hidden = randn(m, h, dtype=dtype, gen=g)
    norm_w = randn(h, dtype=dtype, gen=g, scale=0.1, mean=1.0)
    w_gu = randn(2 * i, h, dtype=dtype, gen=g, scale=h ** -0.5)
    w_down = randn(h, i, dtype=dtype, gen=g, scale=i ** -0.5)
    ref = O.post_attn_mlp(npf(hidden), npf(norm_w), npf(w_gu), npf(w_down), 1e-5, tag(dtype))
    args = (hidden.to(DEV), norm_w.to(DEV), w_gu.to(DEV), w_down.to(DEV), 1e-5)
    for kind in ("dot", "simt"):
        check(fd().post_attn_mlp(*args, kind=kind), ref, dtype, "linear")


def test_post_attn_mlp_graph_replays_match_eager():
    """Capture the block in a HIP graph; every replay equals the eager result."""
    h, i, m = 512, 1024, 2
    g = torch.Generator().manual_seed(77)
    hidden = randn(m, h, gen=g).to(DEV)
    norm_w = randn(h, gen=g, scale=0.1, mean=1.0).to(DEV)
    w_gu = randn(2 * i, h, gen=g, scale=h ** -0.5).to(DEV)
    w_down = randn(h, i, gen=g, scale=i ** -0.5).to(DEV)
    eager = fd().post_attn_mlp(hidden, norm_w, w_gu, w_down, kind="simt")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fd().post_attn_mlp(hidden, norm_w, w_gu, w_down, kind="simt")
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fd().post_attn_mlp(hidden, norm_w, w_gu, w_down, kind="simt")
    for _ in range(4):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        torch.testing.assert_close(out, eager, rtol=0, atol=0)
        _ = (hidden * 2).sum().item()  # unrelated eager work between replays


# ---------------------------------------------------------------- errors


def test_rejected_inputs():
    x = torch.randn(4, 16)
    w = torch.randn(16)
    with pytest.raises(ValueError, match="CUDA"):
        fd().rms_norm(x, w)
    cuda = torch.randn(4, 16, device=DEV, dtype=torch.float16)
    with pytest.raises(ValueError, match="weight"):
        fd().rms_norm(cuda, torch.randn(8, device=DEV, dtype=torch.float16))
    with pytest.raises(ValueError, match="even"):
        fd().rope(
            torch.randn(2, 3, device=DEV, dtype=torch.float16),
            torch.randn(2, 3, device=DEV, dtype=torch.float16),
            torch.randn(2, 3, device=DEV, dtype=torch.float16),
        )
    with pytest.raises(ValueError, match="kind"):
        fd().linear_decode(cuda, torch.randn(8, 16, device=DEV, dtype=torch.float16), kind="mfma")
    with pytest.raises(TypeError, match="bias"):
        fd().linear_decode(cuda, torch.randn(8, 16, device=DEV, dtype=torch.float16),
                           torch.randn(8, device=DEV, dtype=torch.bfloat16), kind="simt")


def test_library_runtime_is_torchs():
    import fused_decode._lib as L

    assert L.runtime_version() // 10_000_000 == int(torch.version.hip.split(".")[0])
    assert math.isfinite(float(L.runtime_version()))


# ---------------------------------------------------------------- decode step


def _oracle_decode_step(ds, tagd):
    """The harness's layer sequence restated with the oracle's operators."""
    n = lambda t: t.detach().float().cpu().numpy()  # noqa: E731
    x = n(ds.x_in)
    cos, sin = n(ds.cos), n(ds.sin)
    qk = ds.qk_heads * 128
    for w in ds.w:
        normed, stream = O.add_rms_norm(x, np.zeros_like(x), n(w["attn_norm"]), 1e-5, tagd)
        qkv = O.linear(normed, n(w["qkv"]), dtype=tagd)
        q = qkv[:, :qk].reshape(ds.m, ds.qk_heads, 128)
        qkv[:, :qk] = O.rope(q, cos, sin, tagd).reshape(ds.m, qk)
        h = O.linear(n(w["attn_out"]), n(w["o"]), row_add=stream, dtype=tagd)
        x = O.post_attn_mlp(h, n(w["mlp_norm"]), n(w["gate_up"]), n(w["down"]), 1e-5, tagd)
    return x, qkv


@pytest.mark.parametrize("fused", [True, False], ids=["fused", "composed"])
@pytest.mark.parametrize("m", [1, 3, 5, 8, 16])
def test_decode_step_small_matches_oracle_and_graph(m, fused):
    """Both forms of the layer, below and above the MFMA switch at 5 rows (where
    the fused form hands row sums of squares to each norm and the composed one
    runs the MLP's norm inside its gate/up, or as a row kernel from 9 rows),
    against the oracle, then graph replays."""
    from fused_decode.decode_step import DecodeStep

    ds = DecodeStep(m=m, layers=2, h=256, i=512, seed=5, fused=fused)
    eager = ds.step().clone()
    ref, ref_qkv = _oracle_decode_step(ds, "f16")
    check(eager, ref, torch.float16, "linear")
    check(ds.qkv, ref_qkv, torch.float16, "linear")  # last layer's q/k after RoPE, and v
    ds.capture()
    for _ in range(3):
        ds.out.zero_()
        out = ds.replay()
        torch.cuda.synchronize()
        torch.testing.assert_close(out, eager, rtol=0, atol=0)
        _ = (ds.x_in.float() * 2).sum().item()  # unrelated eager work between replays


@pytest.mark.parametrize("m", [1, 5, 8, 16])
def test_decode_step_small_bf16_matches_oracle(m):
    """The fused layer in bfloat16 (the norm weights bfloat16 too, so from 5 rows
    the QKV streams its norm weight and adds the producer's row sums per wave, and
    the gate/up normalises from them) against the oracle, then a graph replay."""
    from fused_decode.decode_step import DecodeStep

    ds = DecodeStep(m=m, layers=2, h=256, i=512, seed=9, dtype=torch.bfloat16)
    eager = ds.step().clone()
    qkv = ds.qkv.clone()
    ref, ref_qkv = _oracle_decode_step(ds, "bf16")
    check(eager, ref, torch.bfloat16, "linear")
    check(qkv, ref_qkv, torch.bfloat16, "linear")
    ds.capture()
    ds.out.zero_()
    torch.testing.assert_close(ds.replay(), eager, rtol=0, atol=0)


@pytest.mark.parametrize("m,dtype", [(1, torch.float16), (8, torch.float16), (1, torch.bfloat16),
                                     (8, torch.bfloat16), (16, torch.float16)])
def test_decode_step_llama3_8b_matches_oracle(m, dtype):
    """Two layers at full Llama-3-8B widths (H=4096, 32 q + 8 kv heads of 128,
    I=14336), the shapes the 32-layer benchmark step runs, against the oracle:
    the step's output and the last layer's q/k/v, then a graph replay."""
    from fused_decode.decode_step import DecodeStep

    print(f"[decode step llama3-8b m={m} {dtype}]", flush=True)
    ds = DecodeStep(m=m, layers=2, seed=6, dtype=dtype)
    assert ds.weight_bytes == 2 * 436_207_616 + 2 * 2 * 4096 * 2
    eager = ds.step().clone()
    qkv = ds.qkv.clone()
    ref, ref_qkv = _oracle_decode_step(ds, tag(dtype))
    check(eager, ref, dtype, "linear")
    check(qkv, ref_qkv, dtype, "linear")
    ds.out.zero_()
    torch.testing.assert_close(ds.replay(), eager, rtol=0, atol=0)


@pytest.mark.parametrize("m,kind", [(1, "simt"), (3, "dot"), (8, "dot"), (16, "dot"), (8, "simt")])
def test_mlp_gate_up_entry_point(m, kind):
    """fd_mlp_gate_up through the C ABI: mid = round(silu(g) * u) of the normed input."""
    from fused_decode import _lib as L

    h, i = 512, 768
    g = torch.Generator().manual_seed(300 + m)
    hidden = randn(m, h, gen=g)
    norm_w = randn(h, gen=g, scale=0.1, mean=1.0)
    w_gu = randn(2 * i, h, gen=g, scale=h ** -0.5)
    hn = O.rms_norm(npf(hidden), npf(norm_w), 1e-5, "f16")
    gu = O.linear(hn, npf(w_gu), dtype="f16")
    ref = O.swiglu(gu[:, :i], gu[:, i:], "f16")
    hd, nwd, wgd = hidden.to(DEV), norm_w.to(DEV), w_gu.to(DEV)
    mid = torch.empty(m, i, device=DEV, dtype=torch.float16)
    normed = torch.empty(m, h, device=DEV, dtype=torch.float16)
    st = torch.cuda.current_stream().cuda_stream
    L.check("fd_mlp_gate_up", L.lib().fd_mlp_gate_up(
        mid.data_ptr(), normed.data_ptr(), hd.data_ptr(), nwd.data_ptr(), L.FD_F16, wgd.data_ptr(),
        m, h, i, 1e-5, L.KIND_CODE[kind], L.FD_F16, st))
    check(mid, ref, torch.float16, "linear")
    if kind == "dot" and m >= 9:
        check(normed, hn, torch.float16)  # the row kernel's output is the staged input
        assert L.lib().fd_mlp_gate_up(mid.data_ptr(), None, hd.data_ptr(), nwd.data_ptr(), L.FD_F16,
                                      wgd.data_ptr(), m, h, i, 1e-5, L.FD_KIND_DOT, L.FD_F16, st) == L.FD_EINVAL
