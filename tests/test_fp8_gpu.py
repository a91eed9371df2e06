"""GPU parity of the FP8-weight GEMV, MLP and fused QKV against the oracle's E4M3
products (oracle.linear_fp8 / post_attn_mlp_fp8 / pre_attn_qkv_fp8 on the same
codes and scales), at the
reference's GEMV tolerance (tests/test_ops.py:27-35: fp16 2e-2, bf16 4e-2): the
codes are decoded exactly on both sides, so only summation order differs."""

from __future__ import annotations

import warnings

import numpy as np
import pytest
import torch

from oracle import decode_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = [torch.float16, torch.bfloat16]


@pytest.fixture(scope="module", autouse=True)
def _lib_loaded():
    import fused_decode._lib as L

    L.lib()


def tag(dtype):
    return "f16" if dtype == torch.float16 else "bf16"


def tol(dtype):
    return {"rtol": 2e-2, "atol": 2e-2} if dtype == torch.float16 else {"rtol": 4e-2, "atol": 4e-2}


def rnd(*shape, seed, dtype=torch.float16, scale=1.0, mean=0.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale + mean).to(dtype)


def quant(w):
    import fused_decode as fd

    q, s = fd.quantize_fp8(w.to(DEV))
    return q, s, q.cpu().view(torch.uint8).numpy(), s.cpu().numpy()


def npf(t):
    return t.detach().float().cpu().numpy()


def test_quantizer_matches_oracle():
    w = rnd(64, 160, seed=1, scale=0.05)
    w[5] = 0
    q, s, qn, sn = quant(w)
    oq, os_ = O.fp8_quantize(npf(w))
    assert np.array_equal(qn, oq) and np.array_equal(sn, os_)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 13, 16])
def test_linear_fp8_matches_oracle(dtype, m):
    import fused_decode as fd

    n, k = 200, 1152  # ragged N, K not a multiple of the 1024-element step
    x = rnd(m, k, seed=m, dtype=dtype)
    q, s, qn, sn = quant(rnd(n, k, seed=40 + m, scale=k ** -0.5))
    bias = rnd(n, seed=2, dtype=torch.float32)
    row = rnd(m, n, seed=3, dtype=dtype)
    y = fd.linear_decode_fp8(x.to(DEV), q, s, bias.to(DEV), row_add=row.to(DEV))
    ref = O.linear_fp8(npf(x), qn, sn, npf(bias), npf(row), tag(dtype))
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(dtype))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("nk", [(28672, 4096), (4096, 14336)], ids=["gate_up", "down"])
def test_linear_fp8_llama_shapes(dtype, nk):
    import fused_decode as fd

    n, k = nk
    x = rnd(8, k, seed=7, dtype=dtype)
    q, s, qn, sn = quant(rnd(n, k, seed=8, scale=k ** -0.5))
    y = fd.linear_decode_fp8(x.to(DEV), q, s)
    ref = O.linear_fp8(npf(x[:2]), qn, sn, dtype=tag(dtype))  # two rows of the oracle
    torch.testing.assert_close(y[:2].float().cpu(), torch.from_numpy(ref), **tol(dtype))
    y1 = fd.linear_decode_fp8(x[:1].to(DEV), q, s)  # the M = 1 kernel gives the same row
    torch.testing.assert_close(y1.float().cpu(), torch.from_numpy(ref[:1]), **tol(dtype))
    y4 = fd.linear_decode_fp8(x[:4].to(DEV), q, s)  # and the persistent SIMT kernel (2-4 rows)
    torch.testing.assert_close(y4[:2].float().cpu(), torch.from_numpy(ref), **tol(dtype))


def test_linear_fp8_fallback_shapes():
    import fused_decode as fd

    from fused_decode import fp8 as F8

    x = rnd(24, 200, seed=9)  # 24 rows > 16 and K % 16 != 0: the float32 path
    q, s, qn, sn = quant(rnd(48, 200, seed=10, scale=0.1))
    F8._warned.clear()
    with pytest.warns(RuntimeWarning, match="float32 product"):
        y = fd.linear_decode_fp8(x.to(DEV), q, s)
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(O.linear_fp8(npf(x), qn, sn, dtype="f16")),
                               **tol(torch.float16))
    # codes at an address that is not 16-byte aligned, after a call that cached the
    # plan of the same signature on aligned codes: the float32 path, same values
    x = rnd(4, 256, seed=11)
    q, s, qn, sn = quant(rnd(32, 256, seed=12, scale=0.1))
    raw = torch.empty(32 * 256 + 8, dtype=torch.uint8, device=DEV)
    mis = raw[8:].view(32, 256)
    mis.copy_(q.view(torch.uint8))
    qm = mis.view(q.dtype)
    assert qm.stride() == q.stride() and qm.data_ptr() % 16 == 8
    ref = torch.from_numpy(O.linear_fp8(npf(x), qn, sn, dtype="f16"))
    y = fd.linear_decode_fp8(x.to(DEV), q, s)
    torch.testing.assert_close(y.float().cpu(), ref, **tol(torch.float16))
    with pytest.warns(RuntimeWarning, match="16-byte rows"):
        y1 = fd.linear_decode_fp8(x.to(DEV), qm, s)
    torch.testing.assert_close(y1.float().cpu(), ref, **tol(torch.float16))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m", [1, 3, 8, 16])
def test_post_attn_mlp_fp8_matches_oracle(dtype, m):
    import fused_decode as fd

    h, i = 256, 512
    hid = rnd(m, h, seed=20 + m, dtype=dtype)
    nw = rnd(h, seed=30, dtype=dtype, scale=0.1, mean=1.0)
    gq, gs, gqn, gsn = quant(rnd(2 * i, h, seed=31, scale=h ** -0.5))
    dq, ds, dqn, dsn = quant(rnd(h, i, seed=32, scale=i ** -0.5))
    y = fd.post_attn_mlp_fp8(hid.to(DEV), nw.to(DEV), gq, gs, dq, ds, 1e-5)
    ref = O.post_attn_mlp_fp8(npf(hid), npf(nw), gqn, gsn, dqn, dsn, 1e-5, tag(dtype))
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(dtype))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m", [1, 8])
def test_post_attn_mlp_fp8_norm_weight_in_other_dtypes(dtype, m):
    import fused_decode as fd

    h, i = 256, 512
    other = torch.bfloat16 if dtype == torch.float16 else torch.float16
    gq, gs, gqn, gsn = quant(rnd(2 * i, h, seed=33, scale=h ** -0.5))
    dq, ds, dqn, dsn = quant(rnd(h, i, seed=34, scale=i ** -0.5))
    for j, nw_dtype in enumerate((torch.float32, other)):
        hid = rnd(m, h, seed=35 + m + j, dtype=dtype)
        nw = rnd(h, seed=37 + j, dtype=nw_dtype, scale=0.3, mean=1.0)
        y = fd.post_attn_mlp_fp8(hid.to(DEV), nw.to(DEV), gq, gs, dq, ds, 1e-5)
        ref = O.post_attn_mlp_fp8(npf(hid), npf(nw), gqn, gsn, dqn, dsn, 1e-5, tag(dtype))
        torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(dtype))


@pytest.mark.parametrize("m,h", [(8, 1040), (9, 1024), (16, 1024)])
@pytest.mark.parametrize("i", [4096, 4112, 14336])
def test_post_attn_mlp_fp8_relayout_tile_forms(m, h, i):
    """The E4M3 relayout gate/up (from 9 rows, and at 5-8 rows where H is not a
    multiple of 512) with tiles of 16 gate + 16 up rows only (I = 4096: one
    round over the CUs) and with the rows past the last whole round in tiles of
    8 + 8 (I = 4112: two such tiles; I = 14336: 768 + 256 tiles). The MLP's two
    HIP launches run (H and I multiples of 16): no composed fallback, no warning."""
    import fused_decode as fd

    dtype = torch.bfloat16 if m == 16 and i == 14336 else torch.float16
    hid = rnd(m, h, seed=80 + m, dtype=dtype)
    nw = rnd(h, seed=81, dtype=dtype, scale=0.1, mean=1.0)
    gq, gs, gqn, gsn = quant(rnd(2 * i, h, seed=82 + i, scale=h ** -0.5))
    dq, ds, dqn, dsn = quant(rnd(h, i, seed=83 + i, scale=i ** -0.5))
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        y = fd.post_attn_mlp_fp8(hid.to(DEV), nw.to(DEV), gq, gs, dq, ds, 1e-5)
    ref = O.post_attn_mlp_fp8(npf(hid), npf(nw), gqn, gsn, dqn, dsn, 1e-5, tag(dtype))
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(dtype))


def test_post_attn_mlp_fp8_wide_hidden_composes():
    """H = 39936 at M = 8: beyond the width the MFMA gate/up's norm-weight LDS
    stage takes, the library declines (FD_EUNSUPPORTED) and the operator
    composes rms_norm, the fp8 GEMVs and swiglu; same result."""
    import fused_decode as fd
    from fused_decode import _lib as L

    h, i, m = 39936, 64, 8
    hid = rnd(m, h, seed=70)
    nw = rnd(h, seed=71, scale=0.1, mean=1.0)
    gq, gs, gqn, gsn = quant(rnd(2 * i, h, seed=72, scale=h ** -0.5))
    dq, ds, dqn, dsn = quant(rnd(h, i, seed=73, scale=i ** -0.5))
    hd, nwd = hid.to(DEV), nw.to(DEV)
    y_c = torch.empty(m, h, device=DEV, dtype=torch.float16)
    mid = torch.empty(m, i, device=DEV, dtype=torch.float16)
    st = torch.cuda.current_stream().cuda_stream
    assert L.lib().fd_post_attn_mlp_fp8(y_c.data_ptr(), mid.data_ptr(), hd.data_ptr(), nwd.data_ptr(), L.FD_F16,
                                        gq.data_ptr(), gs.data_ptr(), dq.data_ptr(), ds.data_ptr(), m, h, i, 1e-5,
                                        L.FD_F16, st) == L.FD_EUNSUPPORTED
    y = fd.post_attn_mlp_fp8(hd, nwd, gq, gs, dq, ds, 1e-5)
    ref = O.post_attn_mlp_fp8(npf(hid), npf(nw), gqn, gsn, dqn, dsn, 1e-5, "f16")
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(torch.float16))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("i_", [64, 2064, 4096])
def test_post_attn_mlp_fp8_resident_rows_form(dtype, i_):
    """H a multiple of 512 and 5-8 rows: the E4M3 gate/up runs its persistent
    form (row scales staged per tile iteration, the normalised rows resident
    in LDS); I = 64 has fewer tiles (8) than CUs, I = 2064 splits the tiles
    unevenly, I = 4096 gives every workgroup two."""
    import fused_decode as fd

    h = 512
    gq, gs, gqn, gsn = quant(rnd(2 * i_, h, seed=70, scale=h ** -0.5))
    dq, ds, dqn, dsn = quant(rnd(h, i_, seed=71, scale=i_ ** -0.5))
    for m in (5, 6, 7, 8):
        for nw_dtype in (torch.float32, dtype):
            hid = rnd(m, h, seed=72 + m, dtype=dtype)
            nw = rnd(h, seed=80 + m, dtype=nw_dtype, scale=0.1, mean=1.0)
            y = fd.post_attn_mlp_fp8(hid.to(DEV), nw.to(DEV), gq, gs, dq, ds, 1e-5)
            ref = O.post_attn_mlp_fp8(npf(hid), npf(nw), gqn, gsn, dqn, dsn, 1e-5, tag(dtype))
            torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(dtype))


@pytest.mark.parametrize("m", [1, 2, 3, 4])
def test_post_attn_mlp_fp8_several_tiles_per_workgroup(m):
    """I = 6144 with 4-row tiles: 1536 tiles over two workgroups per CU, so each
    workgroup streams several tiles of the persistent fp8 gate/up."""
    import fused_decode as fd

    h, i = 256, 6144
    hid = rnd(m, h, seed=60 + m)
    nw = rnd(h, seed=61, scale=0.1, mean=1.0)
    gq, gs, gqn, gsn = quant(rnd(2 * i, h, seed=62, scale=h ** -0.5))
    dq, ds, dqn, dsn = quant(rnd(h, i, seed=63, scale=i ** -0.5))
    y = fd.post_attn_mlp_fp8(hid.to(DEV), nw.to(DEV), gq, gs, dq, ds, 1e-5)
    ref = O.post_attn_mlp_fp8(npf(hid), npf(nw), gqn, gsn, dqn, dsn, 1e-5, "f16")
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(torch.float16))


@pytest.mark.parametrize("m", [1, 8])
def test_post_attn_mlp_fp8_llama3_8b(m):
    """Llama-3-8B widths: the fused two-launch path against the composed fp8
    operators on the GPU, and row 0 against the oracle."""
    import fused_decode as fd

    h, i = 4096, 14336
    hid = rnd(m, h, seed=40).to(DEV)
    nw = rnd(h, seed=41, scale=0.1, mean=1.0).to(DEV)
    gq, gs, gqn, gsn = quant(rnd(2 * i, h, seed=42, scale=h ** -0.5))
    dq, ds, dqn, dsn = quant(rnd(h, i, seed=43, scale=i ** -0.5))
    y = fd.post_attn_mlp_fp8(hid, nw, gq, gs, dq, ds, 1e-5)
    normed = fd.rms_norm(hid, nw, eps=1e-5)
    g, u = fd.linear_decode_fp8(normed, gq, gs).split(i, dim=-1)
    comp = fd.linear_decode_fp8(fd.swiglu(g, u), dq, ds, row_add=hid)
    torch.testing.assert_close(y, comp, **tol(torch.float16))
    ref = O.post_attn_mlp_fp8(npf(hid[:1]), npf(nw), gqn, gsn, dqn, dsn, 1e-5, "f16")
    torch.testing.assert_close(y[:1].float().cpu(), torch.from_numpy(ref), **tol(torch.float16))


def test_post_attn_mlp_fp8_graph_replays_match_eager():
    import fused_decode as fd

    h, i = 256, 512
    hid = rnd(2, h, seed=50).to(DEV)
    nw = rnd(h, seed=51, scale=0.1, mean=1.0).to(DEV)
    gq, gs, _, _ = quant(rnd(2 * i, h, seed=52, scale=h ** -0.5))
    dq, ds, _, _ = quant(rnd(h, i, seed=53, scale=i ** -0.5))
    eager = fd.post_attn_mlp_fp8(hid, nw, gq, gs, dq, ds, 1e-5).clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fd.post_attn_mlp_fp8(hid, nw, gq, gs, dq, ds, 1e-5)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fd.post_attn_mlp_fp8(hid, nw, gq, gs, dq, ds, 1e-5)
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        torch.testing.assert_close(out, eager, rtol=0, atol=0)


@pytest.mark.parametrize("m", [1, 6])
@pytest.mark.parametrize("k", [16, 48])
def test_linear_fp8_k_below_one_unit(m, k):
    """K below one 128-element MFMA unit (and one 1024-code SIMT step)."""
    import fused_decode as fd

    n = 40
    x = rnd(m, k, seed=100 + k + m)
    q, s, qn, sn = quant(rnd(n, k, seed=110 + k, scale=k ** -0.5))
    y = fd.linear_decode_fp8(x.to(DEV), q, s)
    ref = O.linear_fp8(npf(x), qn, sn, dtype="f16")
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(torch.float16))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m", [1, 8])
def test_linear_fp8_nan_codes_decode_as_nan(dtype, m):
    """E4M3FN codes 0x7f and 0xff are NaN, as torch's float8_e4m3fn casts and the
    oracle's decode have them: a row holding one gives NaN outputs and every
    other row the oracle's values, on the SIMT (M = 1) and MFMA (M = 8) forms."""
    import fused_decode as fd

    n, k = 64, 512
    x = rnd(m, k, seed=3, dtype=dtype)
    _, s, qn, sn = quant(rnd(n, k, seed=4, scale=k ** -0.5))
    qn = qn.copy()
    qn[5, 17] = 0x7F
    qn[40, 300] = 0xFF
    q = torch.from_numpy(qn).view(torch.float8_e4m3fn).to(DEV)
    y = fd.linear_decode_fp8(x.to(DEV), q, s).float().cpu()
    ref = O.linear_fp8(npf(x), qn, sn, dtype=tag(dtype))
    assert np.isnan(ref[:, [5, 40]]).all()
    assert torch.isnan(y[:, [5, 40]]).all()
    keep = [j for j in range(n) if j not in (5, 40)]
    torch.testing.assert_close(y[:, keep], torch.from_numpy(ref)[:, keep], **tol(dtype))


def test_linear_fp8_k0_is_the_epilogue():
    """K = 0 through the C entry point: y = round(scale-free bias + row_add), with
    x null and no code read, for the SIMT (M = 1) and MFMA (M = 6) forms."""
    from fused_decode import _lib as L

    n = 48
    codes = torch.zeros(n, 16, device=DEV, dtype=torch.uint8)  # aligned, never read at K = 0
    scale = torch.ones(n, device=DEV)
    st = torch.cuda.current_stream().cuda_stream
    for m in (1, 6):
        bias = rnd(n, seed=80 + m).to(DEV)
        ra = rnd(m, n, seed=90 + m).to(DEV)
        exp = O.linear(np.zeros((m, 0), np.float32), np.zeros((n, 0), np.float32), bias=npf(bias),
                       row_add=npf(ra), dtype="f16")
        y = torch.full((m, n), float("nan"), device=DEV, dtype=torch.float16)
        L.check("fd_linear_fp8", L.lib().fd_linear_fp8(
            y.data_ptr(), None, codes.data_ptr(), scale.data_ptr(), bias.data_ptr(), L.FD_F16,
            ra.data_ptr(), L.FD_F16, m, n, 0, 16, 16, 1, n, 1, n, 1, L.FD_F16, st))
        torch.testing.assert_close(y.float().cpu(), torch.from_numpy(exp), rtol=0, atol=0)


def test_fp8_rejects():
    import fused_decode as fd

    x = rnd(2, 64, seed=60).to(DEV)
    q, s, _, _ = quant(rnd(32, 64, seed=61))
    with pytest.raises(TypeError, match="float8_e4m3fn"):
        fd.linear_decode_fp8(x, q.float(), s)
    with pytest.raises(ValueError, match="scale"):
        fd.linear_decode_fp8(x, q, s[:5])
    with pytest.raises(ValueError, match="CUDA"):
        fd.linear_decode_fp8(x.cpu(), q, s)
    with pytest.raises(ValueError, match="K"):
        fd.linear_decode_fp8(x[:, :32], q, s)


@pytest.mark.parametrize("m", [2, 8, 16])
def test_decode_step_fp8_matches_oracle_and_graph(m):
    """The fp8 layer below and above the MFMA switch at 5 rows."""
    from fused_decode.decode_step import HEAD_DIM, DecodeStep

    ds = DecodeStep(m=m, layers=2, h=256, i=512, seed=5, weights="fp8")
    eager = ds.step().clone()
    codes = lambda q: q.cpu().view(torch.uint8).numpy()  # noqa: E731
    x = npf(ds.x_in)
    cos, sin = npf(ds.cos), npf(ds.sin)
    qk = ds.qk_heads * HEAD_DIM
    for w in ds.w:
        qkv = O.pre_attn_qkv_fp8(x, npf(w["attn_norm"]), codes(w["qkv"][0]), npf(w["qkv"][1]), cos, sin,
                                 1e-5, qk, dtype="f16")
        h = O.linear_fp8(npf(w["attn_out"]), codes(w["o"][0]), npf(w["o"][1]), row_add=x, dtype="f16")
        x = O.post_attn_mlp_fp8(h, npf(w["mlp_norm"]), codes(w["gate_up"][0]), npf(w["gate_up"][1]),
                                codes(w["down"][0]), npf(w["down"][1]), 1e-5, "f16")
    torch.testing.assert_close(eager.float().cpu(), torch.from_numpy(x), **tol(torch.float16))
    torch.testing.assert_close(ds.qkv.float().cpu(), torch.from_numpy(qkv), **tol(torch.float16))
    ds.capture()
    for _ in range(3):
        ds.out.zero_()
        out = ds.replay()
        torch.cuda.synchronize()
        torch.testing.assert_close(out, eager, rtol=0, atol=0)
    assert ds.launches_per_layer == 4  # from 5 rows the MLP's norm runs inside its gate/up (row sums)


@pytest.mark.parametrize("m", [1, 4, 8])
def test_decode_step_fp8_llama3_8b_matches_oracle(m):
    """Two E4M3 layers at full Llama-3-8B widths, the shapes of the 32-layer
    benchmark step: one row (the one-row kernels), four (the persistent SIMT
    forms) and eight (the resident gate/up, the QKV from the producer's row sums
    in eight-wave workgroups, the O and down projections writing row sums with
    four units in flight), against the oracle, then a graph replay."""
    from fused_decode.decode_step import HEAD_DIM, DecodeStep

    print(f"[fp8 decode step llama3-8b m={m}]", flush=True)
    ds = DecodeStep(m=m, layers=2, seed=7, weights="fp8")
    eager = ds.step().clone()
    codes = lambda q: q.cpu().view(torch.uint8).numpy()  # noqa: E731
    x = npf(ds.x_in)
    cos, sin = npf(ds.cos), npf(ds.sin)
    qk = ds.qk_heads * HEAD_DIM
    for w in ds.w:
        qkv = O.pre_attn_qkv_fp8(x, npf(w["attn_norm"]), codes(w["qkv"][0]), npf(w["qkv"][1]), cos, sin,
                                 1e-5, qk, dtype="f16")
        h = O.linear_fp8(npf(w["attn_out"]), codes(w["o"][0]), npf(w["o"][1]), row_add=x, dtype="f16")
        x = O.post_attn_mlp_fp8(h, npf(w["mlp_norm"]), codes(w["gate_up"][0]), npf(w["gate_up"][1]),
                                codes(w["down"][0]), npf(w["down"][1]), 1e-5, "f16")
    torch.testing.assert_close(eager.float().cpu(), torch.from_numpy(x), **tol(torch.float16))
    torch.testing.assert_close(ds.qkv.float().cpu(), torch.from_numpy(qkv), **tol(torch.float16))
    ds.out.zero_()
    torch.testing.assert_close(ds.replay(), eager, rtol=0, atol=0)


# ---------------------------------------------------------------- fused QKV


def qkv_case(m, h, heads, kv, d, dtype, seed, bias=False, per_row=True, cs_dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    n = (heads + 2 * kv) * d
    hidden = (torch.randn(m, h, generator=g)).to(dtype)
    norm_w = (torch.randn(h, generator=g) * 0.1 + 1.0).to(dtype)
    w = torch.randn(n, h, generator=g) * h ** -0.5
    b = torch.randn(n, generator=g) * 0.5 if bias else None
    rows = m if per_row else 1
    inv = 1.0 / (500000.0 ** (torch.arange(0, d, 2, dtype=torch.float64) / d))
    pos = torch.arange(900 + seed, 900 + seed + rows, dtype=torch.float64)
    emb = torch.cat([pos[:, None] * inv[None], pos[:, None] * inv[None]], dim=1)
    q, s, qn, sn = quant(w)
    return (hidden, norm_w, q, s, qn, sn, b, emb.cos().to(cs_dtype), emb.sin().to(cs_dtype),
            (heads + kv) * d)


def qkv_run(hidden, norm_w, q, s, b, cos, sin, rc, eps=1e-5, out=None):
    import fused_decode as fd

    dev = lambda t: None if t is None else t.to(DEV)  # noqa: E731
    return fd.pre_attn_qkv_fp8(dev(hidden), dev(norm_w), q, s, dev(cos), dev(sin), eps, rope_cols=rc,
                               bias=dev(b), out=out)


def qkv_oracle(hidden, norm_w, qn, sn, b, cos, sin, rc, dtype, eps=1e-5):
    return O.pre_attn_qkv_fp8(npf(hidden), npf(norm_w), qn, sn, npf(cos), npf(sin), eps, rc,
                              bias=None if b is None else npf(b), dtype=tag(dtype))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 13, 16])
def test_pre_attn_qkv_fp8_matches_oracle(dtype, m):
    hidden, nw, q, s, qn, sn, b, cos, sin, rc = qkv_case(m, 512, 4, 2, 64, dtype, seed=m, bias=m % 2 == 1)
    y = qkv_run(hidden, nw, q, s, b, cos, sin, rc)
    ref = qkv_oracle(hidden, nw, qn, sn, b, cos, sin, rc, dtype)
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(dtype))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m", [1, 3, 5, 8, 16])
def test_pre_attn_qkv_fp8_norm_weight_in_other_dtypes(dtype, m):
    """A float32 or other-half-type norm weight: the folded MFMA path (5+ rows)
    converts it while staging each K chunk, the SIMT path per element."""
    other = torch.bfloat16 if dtype == torch.float16 else torch.float16
    for j, nw_dtype in enumerate((torch.float32, other)):
        hidden, _, q, s, qn, sn, b, cos, sin, rc = qkv_case(m, 512, 4, 2, 64, dtype, seed=80 + m, bias=j == 0)
        nw = rnd(512, seed=95 + m + j, dtype=nw_dtype, scale=0.3, mean=1.0)
        y = qkv_run(hidden, nw, q, s, b, cos, sin, rc)
        ref = qkv_oracle(hidden, nw, qn, sn, b, cos, sin, rc, dtype)
        torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(dtype))


@pytest.mark.parametrize("m", [1, 3])
def test_pre_attn_qkv_fp8_several_tiles_per_workgroup(m):
    """128 q + 8 kv heads of 128 (N = 18432): more tiles than the 8 resident
    workgroups per CU take, so each workgroup streams 2 (M = 1, 8-row tiles) or
    3 (M = 3, 4-row tiles) tiles and its epilogues alternate the two halves of
    the partial-sum buffer."""
    hidden, nw, q, s, qn, sn, b, cos, sin, rc = qkv_case(m, 256, 128, 8, 128, torch.float16, seed=60 + m,
                                                          bias=True)
    y = qkv_run(hidden, nw, q, s, b, cos, sin, rc)
    ref = qkv_oracle(hidden, nw, qn, sn, b, cos, sin, rc, torch.float16)
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(torch.float16))


@pytest.mark.parametrize("m", [1, 4, 8])
def test_pre_attn_qkv_fp8_shared_angles_and_rope_cols_edges(m):
    """One cos/sin row for every token in each angle dtype; rope_cols 0 (norm +
    GEMV only) and N (every column rotated)."""
    for cs_dtype in (torch.float16, torch.bfloat16, torch.float32):
        hidden, nw, q, s, qn, sn, b, cos, sin, rc = qkv_case(m, 256, 2, 1, 128, torch.float16, seed=30 + m,
                                                             bias=True, per_row=False, cs_dtype=cs_dtype)
        y = qkv_run(hidden, nw, q, s, b, cos, sin, rc)
        ref = qkv_oracle(hidden, nw, qn, sn, b, cos, sin, rc, torch.float16)
        torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(torch.float16))
    n = q.shape[0]
    for rc in (0, n):
        y = qkv_run(hidden, nw, q, s, b, cos, sin, rc)
        ref = qkv_oracle(hidden, nw, qn, sn, b, cos, sin, rc, torch.float16)
        torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(torch.float16))


def test_pre_attn_qkv_fp8_composes_where_the_kernel_declines():
    """head_dim 72 and 24 rows: composed from rms_norm, linear_decode_fp8 and rope,
    same values."""
    hidden, nw, q, s, qn, sn, b, cos, sin, rc = qkv_case(2, 256, 2, 1, 72, torch.float16, seed=9)
    y = qkv_run(hidden, nw, q, s, b, cos, sin, rc)
    ref = qkv_oracle(hidden, nw, qn, sn, b, cos, sin, rc, torch.float16)
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(torch.float16))
    hidden, nw, q, s, qn, sn, b, cos, sin, rc = qkv_case(24, 256, 2, 1, 64, torch.bfloat16, seed=10)
    y = qkv_run(hidden, nw, q, s, b, cos, sin, rc)
    ref = qkv_oracle(hidden, nw, qn, sn, b, cos, sin, rc, torch.bfloat16)
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(torch.bfloat16))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m", [1, 8])
def test_pre_attn_qkv_fp8_llama3_8b(dtype, m):
    """H=4096, 32 q + 8 kv heads of 128: the fused call against the library's own
    composition (rms_norm, linear_decode_fp8, rope) and row 0 of the oracle."""
    import fused_decode as fd

    hidden, nw, q, s, qn, sn, b, cos, sin, rc = qkv_case(m, 4096, 32, 8, 128, dtype, seed=20 + m)
    hd, nwd, cd, sd = (t.to(DEV) for t in (hidden, nw, cos, sin))
    y = fd.pre_attn_qkv_fp8(hd, nwd, q, s, cd, sd, 1e-5, rope_cols=rc)
    comp = fd.linear_decode_fp8(fd.rms_norm(hd, nwd, eps=1e-5), q, s)
    heads = comp[:, :rc].unflatten(-1, (rc // 128, 128))
    fd.rope(heads, cd[:, None], sd[:, None], out=heads)
    torch.testing.assert_close(y, comp, **tol(dtype))
    ref = qkv_oracle(hidden[:1], nw, qn, sn, b, cos[:1], sin[:1], rc, dtype)
    torch.testing.assert_close(y[:1].float().cpu(), torch.from_numpy(ref), **tol(dtype))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m", [5, 8, 12])
@pytest.mark.parametrize("nw_dtype", ["act", torch.float32])
def test_pre_attn_qkv_fp8_ragged_hidden(dtype, m, nw_dtype):
    """E4M3 QKV over a hidden width with a partial last K unit (272), the norm
    weight streamed (activations' dtype) or staged (float32)."""
    hidden, nw, q, s, qn, sn, b, cos, sin, rc = qkv_case(m, 272, 4, 2, 64, dtype, seed=95 + m, bias=True)
    if nw_dtype != "act":
        nw = nw.to(nw_dtype)
    y = qkv_run(hidden, nw, q, s, b, cos, sin, rc)
    ref = qkv_oracle(hidden, nw, qn, sn, b, cos, sin, rc, dtype)
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(dtype))


@pytest.mark.parametrize("m", [2, 8])
def test_pre_attn_qkv_fp8_plan_reuse(m):
    """A second call with the same argument signature (the cached plan) on new
    operands, and angles gathered per call ([M, 1, D] views), match the oracle."""
    from fused_decode import ops

    ops.clear_plans()
    for seed in (41, 42):
        hidden, nw, q, s, qn, sn, b, cos, sin, rc = qkv_case(m, 256, 4, 2, 64, torch.float16, seed=seed, bias=True)
        y = qkv_run(hidden, nw, q, s, b, cos, sin, rc)
        ref = qkv_oracle(hidden, nw, qn, sn, b, cos, sin, rc, torch.float16)
        torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(torch.float16))
    for seed in (43, 44):
        hidden, nw, q, s, qn, sn, b, cos, sin, rc = qkv_case(m, 256, 4, 2, 64, torch.float16, seed=seed)
        y = qkv_run(hidden, nw, q, s, None, cos.unsqueeze(1), sin.unsqueeze(1), rc)
        ref = qkv_oracle(hidden, nw, qn, sn, None, cos, sin, rc, torch.float16)
        torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(torch.float16))


def test_pre_attn_qkv_fp8_entry_point_and_rejects():
    """fd_pre_attn_qkv_fp8 through the C ABI: from 5 rows the MFMA form folds the
    RMSNorm in (`normed` may be null and is left untouched), H not a multiple of 16
    is FD_EUNSUPPORTED; the Python checks of pre_attn_qkv hold."""
    import fused_decode as fd
    from fused_decode import _lib as L

    hidden, nw, q, s, qn, sn, b, cos, sin, rc = qkv_case(8, 256, 2, 1, 64, torch.float16, seed=12)
    hd, nwd, cd, sd = (t.to(DEV) for t in (hidden, nw, cos, sin))
    n = q.shape[0]
    y = torch.empty(8, n, device=DEV, dtype=torch.float16)
    normed = torch.empty(8, 256, device=DEV, dtype=torch.float16)
    st = torch.cuda.current_stream().cuda_stream
    args = lambda nrm, hh: (  # noqa: E731
        y.data_ptr(), nrm, hd.data_ptr(), nwd.data_ptr(), L.FD_F16, q.data_ptr(), s.data_ptr(), None,
        L.FD_F16, cd.data_ptr(), sd.data_ptr(), L.FD_F32, 64, 8, hh, n, rc, 64, 1e-5, L.FD_F16, st)
    assert L.lib().fd_pre_attn_qkv_fp8(*args(normed.data_ptr(), 248)) == L.FD_EUNSUPPORTED
    ref = qkv_oracle(hidden, nw, qn, sn, b, cos, sin, rc, torch.float16)
    L.check("fd_pre_attn_qkv_fp8", L.lib().fd_pre_attn_qkv_fp8(*args(None, 256)))
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(torch.float16))
    normed.fill_(7.0)
    y.zero_()
    L.check("fd_pre_attn_qkv_fp8", L.lib().fd_pre_attn_qkv_fp8(*args(normed.data_ptr(), 256)))
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(torch.float16))
    assert bool((normed == 7.0).all()), "normed must be left untouched"
    with pytest.raises(TypeError, match="float8_e4m3fn"):
        fd.pre_attn_qkv_fp8(hd, nwd, q.float(), s, cd, sd, rope_cols=rc)
    with pytest.raises(ValueError, match="scale"):
        fd.pre_attn_qkv_fp8(hd, nwd, q, s[:3], cd, sd, rope_cols=rc)
    with pytest.raises(ValueError, match="rope_cols"):
        fd.pre_attn_qkv_fp8(hd, nwd, q, s, cd, sd, rope_cols=rc + 3)
    with pytest.raises(ValueError, match="CUDA"):
        fd.pre_attn_qkv_fp8(hidden, nwd, q, s, cd, sd, rope_cols=rc)
