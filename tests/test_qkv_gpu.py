"""GPU parity tests of the fused pre-attention QKV (RMSNorm + QKV GEMV + RoPE of
the q and k heads) against the oracle's composition of the reference operators,
and of the fused decode step against the composed one.

Tolerances are the reference's GEMV ones (tests/test_ops.py:27-35): fp16
rtol=atol=2e-2, bf16 4e-2.
"""

from __future__ import annotations

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

    L.lib()  # raises if the HIP library is missing: no silent fallback


def tag(dtype) -> str:
    return "f16" if dtype == torch.float16 else "bf16"


def tol(dtype):
    return {"rtol": 2e-2, "atol": 2e-2} if dtype == torch.float16 else {"rtol": 4e-2, "atol": 4e-2}


def randn(*shape, gen, dtype=torch.float16, scale=1.0, mean=0.0):
    return (torch.randn(*shape, generator=gen, dtype=torch.float32) * scale + mean).to(dtype)


def npf(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def angles(rows: int, d: int, first_pos: int, dtype=torch.float32):
    """Llama-3 cos/sin rows for positions first_pos .. first_pos+rows-1."""
    inv = 1.0 / (500000.0 ** (torch.arange(0, d, 2, dtype=torch.float64) / d))
    pos = torch.arange(first_pos, first_pos + rows, dtype=torch.float64)
    emb = torch.cat([pos[:, None] * inv[None], pos[:, None] * inv[None]], dim=1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def case(m, h, heads, kv, d, dtype, seed, bias=False, per_row=True, cs_dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    n = (heads + 2 * kv) * d
    hidden = randn(m, h, gen=g, dtype=dtype)
    norm_w = randn(h, gen=g, dtype=dtype, scale=0.1, mean=1.0)
    w = randn(n, h, gen=g, dtype=dtype, scale=h ** -0.5)
    b = randn(n, gen=g, dtype=torch.float32, scale=0.5) if bias else None
    cos, sin = angles(m if per_row else 1, d, 1000 + seed)
    return hidden, norm_w, w, b, cos.to(cs_dtype), sin.to(cs_dtype), (heads + kv) * d


def run(hidden, norm_w, w, b, cos, sin, rope_cols, kind, eps=1e-5, out=None):
    import fused_decode as fd

    dev = lambda t: None if t is None else t.to(DEV)  # noqa: E731
    return fd.pre_attn_qkv(dev(hidden), dev(norm_w), dev(w), dev(cos), dev(sin), eps,
                           rope_cols=rope_cols, bias=dev(b), out=out, kind=kind)


def oracle(hidden, norm_w, w, b, cos, sin, rope_cols, dtype, eps=1e-5):
    return O.pre_attn_qkv(npf(hidden), npf(norm_w), npf(w), npf(cos), npf(sin), eps, rope_cols,
                          bias=None if b is None else npf(b), dtype=tag(dtype))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("kind", ["dot", "simt"])
@pytest.mark.parametrize("m", [1, 2, 4, 5, 6, 7, 8, 11, 16])
def test_pre_attn_qkv_matches_oracle(dtype, kind, m):
    hidden, nw, w, b, cos, sin, rc = case(m, 512, 4, 2, 64, dtype, seed=m)
    y = run(hidden, nw, w, b, cos, sin, rc, kind)
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(oracle(hidden, nw, w, b, cos, sin, rc, dtype)),
                               **tol(dtype))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("kind", ["dot", "simt"])
@pytest.mark.parametrize("m", [1, 5, 8, 16])
def test_pre_attn_qkv_norm_weight_in_other_dtypes(dtype, kind, m):
    """The norm weight may be float32 or the other half type; the folded MFMA
    path (kind "dot", 5+ rows) converts it while staging each K chunk, the
    others per element. A float32 weight carries bits no half type holds."""
    other = torch.bfloat16 if dtype == torch.float16 else torch.float16
    for j, nw_dtype in enumerate((torch.float32, other)):
        hidden, _, w, b, cos, sin, rc = case(m, 512, 4, 2, 64, dtype, seed=70 + m, bias=j == 1)
        nw = randn(512, gen=torch.Generator().manual_seed(90 + m + j), dtype=nw_dtype, scale=0.3, mean=1.0)
        y = run(hidden, nw, w, b, cos, sin, rc, kind)
        ref = oracle(hidden, nw, w, b, cos, sin, rc, dtype)
        torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(dtype))


@pytest.mark.parametrize("kind", ["dot", "simt"])
@pytest.mark.parametrize("m", [1, 8])
def test_pre_attn_qkv_bias_shared_angles_half_precision_angles(kind, m):
    for cs_dtype in (torch.float16, torch.bfloat16, torch.float32):
        hidden, nw, w, b, cos, sin, rc = case(m, 256, 2, 1, 128, torch.float16, seed=40 + m, bias=True,
                                              per_row=False, cs_dtype=cs_dtype)
        y = run(hidden, nw, w, b, cos, sin, rc, kind)
        ref = oracle(hidden, nw, w, b, cos, sin, rc, torch.float16)
        torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(torch.float16))


@pytest.mark.parametrize("kind", ["dot", "simt"])
def test_pre_attn_qkv_rope_cols_zero_and_all(kind):
    """rope_cols = 0 is norm + GEMV only; rope_cols = N rotates every column."""
    hidden, nw, w, b, cos, sin, _ = case(3, 256, 2, 1, 64, torch.float16, seed=7)
    n = w.shape[0]
    for rc in (0, n):
        y = run(hidden, nw, w, b, cos, sin, rc, kind)
        ref = oracle(hidden, nw, w, b, cos, sin, rc, torch.float16)
        torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(torch.float16))


def test_pre_attn_qkv_unsupported_head_dim_composes():
    """head_dim 72 (not a multiple of 16): the library declines and the operator
    composes rms_norm, linear_decode and rope; same result either way."""
    hidden, nw, w, b, cos, sin, rc = case(2, 256, 2, 1, 72, torch.float16, seed=9)
    y = run(hidden, nw, w, b, cos, sin, rc, None)
    ref = oracle(hidden, nw, w, b, cos, sin, rc, torch.float16)
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(torch.float16))


def test_pre_attn_qkv_above_row_limit_and_leading_dims():
    import fused_decode as fd

    hidden, nw, w, b, cos, sin, rc = case(24, 256, 2, 1, 64, torch.bfloat16, seed=11)
    y = run(hidden, nw, w, b, cos, sin, rc, None)  # 24 rows > 8: F.linear path, composed
    ref = oracle(hidden, nw, w, b, cos, sin, rc, torch.bfloat16)
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(torch.bfloat16))
    # [2, 3, H] hidden with per-token angles [2, 3, 1, D]
    h3 = hidden[:6].reshape(2, 3, 256).to(DEV)
    c3, s3 = cos[:6].reshape(2, 3, 1, 64).to(DEV), sin[:6].reshape(2, 3, 1, 64).to(DEV)
    y3 = fd.pre_attn_qkv(h3, nw.to(DEV), w.to(DEV), c3, s3, 1e-5, rope_cols=rc)
    assert y3.shape == (2, 3, w.shape[0])
    ref6 = oracle(hidden[:6], nw, w, b, cos[:6], sin[:6], rc, torch.bfloat16)
    torch.testing.assert_close(y3.reshape(6, -1).float().cpu(), torch.from_numpy(ref6), **tol(torch.bfloat16))
    c1, s1 = cos[:1].to(DEV), sin[:1].to(DEV)
    assert fd.pre_attn_qkv(h3[:0], nw.to(DEV), w.to(DEV), c1, s1, rope_cols=rc).shape == (0, 3, w.shape[0])


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m", [1, 3])
def test_pre_attn_qkv_several_tiles_per_workgroup(dtype, m):
    """128 q + 8 kv heads of 128 (N = 18432): more tiles than the 8 resident
    workgroups per CU take, so each workgroup streams 2 (M = 1, 8-row tiles) or
    3 (M = 3, 4-row tiles) tiles and its epilogues alternate the two halves of
    the partial-sum buffer."""
    hidden, nw, w, b, cos, sin, rc = case(m, 256, 128, 8, 128, dtype, seed=70 + m, bias=True)
    y = run(hidden, nw, w, b, cos, sin, rc, "simt")
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(oracle(hidden, nw, w, b, cos, sin, rc, dtype)),
                               **tol(dtype))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m", [1, 8])
def test_pre_attn_qkv_llama3_8b_matches_composed_ops(dtype, m):
    """Llama-3-8B widths (H=4096, 32 q + 8 kv heads of 128): every row of the
    fused call against the oracle, and against the library's own composition of
    rms_norm, linear_decode and rope."""
    import fused_decode as fd

    hidden, nw, w, b, cos, sin, rc = case(m, 4096, 32, 8, 128, dtype, seed=20 + m)
    hd, nwd, wd, cd, sd = (t.to(DEV) for t in (hidden, nw, w, cos, sin))
    y = fd.pre_attn_qkv(hd, nwd, wd, cd, sd, 1e-5, rope_cols=rc)
    ref = oracle(hidden, nw, w, b, cos, sin, rc, dtype)
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(dtype))
    normed = fd.rms_norm(hd, nwd, eps=1e-5)
    comp = fd.linear_decode(normed, wd)
    heads = comp[:, :rc].unflatten(-1, (rc // 128, 128))
    fd.rope(heads, cd[:, None], sd[:, None], out=heads)
    torch.testing.assert_close(y, comp, **tol(dtype))


def test_pre_attn_qkv_rejects():
    import fused_decode as fd

    hidden, nw, w, b, cos, sin, rc = case(2, 256, 2, 1, 64, torch.float16, seed=3)
    hd, nwd, wd, cd, sd = (t.to(DEV) for t in (hidden, nw, w, cos, sin))
    with pytest.raises(ValueError, match="CUDA"):
        fd.pre_attn_qkv(hidden, nwd, wd, cd, sd, rope_cols=rc)
    with pytest.raises(ValueError, match="rope_cols"):
        fd.pre_attn_qkv(hd, nwd, wd, cd, sd, rope_cols=rc + 3)
    with pytest.raises(ValueError, match="even"):
        fd.pre_attn_qkv(hd, nwd, wd, cd[:, :63], sd[:, :63], rope_cols=0)
    with pytest.raises(ValueError, match="weight"):
        fd.pre_attn_qkv(hd, nwd[:100], wd, cd, sd, rope_cols=rc)
    with pytest.raises(TypeError):
        fd.pre_attn_qkv(hd, nwd, wd.bfloat16(), cd, sd, rope_cols=rc)
    with pytest.raises(ValueError, match="bias"):
        fd.pre_attn_qkv(hd, nwd, wd, cd, sd, rope_cols=rc, bias=torch.zeros(5, device=DEV))
    with pytest.raises(ValueError, match="broadcast|rows"):
        fd.pre_attn_qkv(hd, nwd, wd, cd.repeat(3, 1), sd.repeat(3, 1), rope_cols=rc)
    with pytest.raises(ValueError):
        fd.pre_attn_qkv(hd, nwd, wd, cd, sd, rope_cols=rc, kind="mfma")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m", [5, 8, 12])
@pytest.mark.parametrize("nw_dtype", ["act", torch.float32])
def test_pre_attn_qkv_ragged_hidden(dtype, m, nw_dtype):
    """A hidden width that is not a whole number of 128-wide K units (264): the
    last unit's activations and norm weights past H read as zero, whether the
    norm weight streams with the units (the activations' dtype) or is staged as
    float32."""
    hidden, nw, w, b, cos, sin, rc = case(m, 264, 4, 2, 64, dtype, seed=90 + m, bias=True)
    if nw_dtype != "act":
        nw = nw.to(nw_dtype)
    y = run(hidden, nw, w, b, cos, sin, rc, kind="dot")
    ref = oracle(hidden, nw, w, b, cos, sin, rc, dtype)
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(dtype))


@pytest.mark.parametrize("m", [2, 8])
def test_pre_attn_qkv_plan_reuse(m):
    """Calls that share an argument signature reuse one cached launch plan: new
    operands of that signature give their own results, and angles that need
    gathering ([M, 1, D] float16 cos beside float32 sin) are gathered on every
    call, also when the plan is reused."""
    import fused_decode as fd
    from fused_decode import ops

    ops.clear_plans()
    for seed in (31, 32):
        hidden, nw, w, b, cos, sin, rc = case(m, 256, 4, 2, 64, torch.float16, seed=seed, bias=True)
        y = run(hidden, nw, w, b, cos, sin, rc, kind="dot")
        ref = oracle(hidden, nw, w, b, cos, sin, rc, torch.float16)
        torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(torch.float16))
    for seed in (33, 34):
        hidden, nw, w, b, cos, sin, rc = case(m, 256, 4, 2, 64, torch.float16, seed=seed)
        c16 = cos.half()
        y = fd.pre_attn_qkv(hidden.to(DEV), nw.to(DEV), w.to(DEV), c16.unsqueeze(1).to(DEV),
                            sin.unsqueeze(1).to(DEV), 1e-5, rope_cols=rc)
        ref = oracle(hidden, nw, w, None, c16.float(), sin, rc, torch.float16)
        torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(torch.float16))


def test_pre_attn_qkv_entry_point_normed_and_status():
    """fd_pre_attn_qkv through the C ABI at 8 rows (the MFMA form): `normed` may
    be NULL; an unsupported head_dim is FD_EUNSUPPORTED, not a launch."""
    from fused_decode import _lib as L

    hidden, nw, w, b, cos, sin, rc = case(8, 256, 2, 1, 64, torch.float16, seed=12)
    hd, nwd, wd, cd, sd = (t.to(DEV) for t in (hidden, nw, w, cos, sin))
    n = w.shape[0]
    y = torch.empty(8, n, device=DEV, dtype=torch.float16)
    normed = torch.empty(8, 256, device=DEV, dtype=torch.float16)
    st = torch.cuda.current_stream().cuda_stream
    args = lambda nrm, hdim, kind: (  # noqa: E731
        y.data_ptr(), nrm, hd.data_ptr(), nwd.data_ptr(), L.FD_F16, wd.data_ptr(), None, L.FD_F16,
        cd.data_ptr(), sd.data_ptr(), L.FD_F32, 64, 8, 256, n, rc, hdim, 1e-5, kind, L.FD_F16, st)
    assert L.lib().fd_pre_attn_qkv(*args(normed.data_ptr(), 72, L.FD_KIND_DOT)) in (L.FD_EINVAL, L.FD_EUNSUPPORTED)
    ref = oracle(hidden, nw, w, b, cos, sin, rc, torch.float16)
    # the MFMA form folds the RMSNorm in: `normed` is optional and left untouched
    normed.fill_(7.0)
    for buf in (None, normed.data_ptr()):
        y.zero_()
        L.check("fd_pre_attn_qkv", L.lib().fd_pre_attn_qkv(*args(buf, 64, L.FD_KIND_DOT)))
        torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(torch.float16))
    assert bool((normed == 7.0).all())


def test_pre_attn_qkv_wide_hidden_streams_the_norm_weight():
    """H = 32768 at 8 rows: a norm weight in the activations' dtype streams with
    the weight tiles (one launch at any H), a float32 one is staged in LDS and
    does not fit (FD_EUNSUPPORTED, so the Python operator composes); both match
    the oracle."""
    import fused_decode as fd
    from fused_decode import _lib as L

    h = 32768
    hidden, nw, w, b, cos, sin, rc = case(8, h, 2, 1, 64, torch.float16, seed=14)
    hd, wd, cd, sd = (t.to(DEV) for t in (hidden, w, cos, sin))
    n = w.shape[0]
    st = torch.cuda.current_stream().cuda_stream
    for nw_t, code, want in ((nw, L.FD_F16, L.FD_OK), (nw.float(), L.FD_F32, L.FD_EUNSUPPORTED)):
        nwd = nw_t.to(DEV)
        y = torch.zeros(8, n, device=DEV, dtype=torch.float16)
        status = L.lib().fd_pre_attn_qkv(y.data_ptr(), None, hd.data_ptr(), nwd.data_ptr(), code, wd.data_ptr(),
                                         None, L.FD_F16, cd.data_ptr(), sd.data_ptr(), L.FD_F32, 64, 8, h, n, rc,
                                         64, 1e-5, L.FD_KIND_DOT, L.FD_F16, st)
        assert status == want
        ref = torch.from_numpy(oracle(hidden, nw_t, w, b, cos, sin, rc, torch.float16))
        if status == L.FD_OK:
            torch.testing.assert_close(y.float().cpu(), ref, **tol(torch.float16))
        out = fd.pre_attn_qkv(hd, nwd, wd, cd, sd, 1e-5, rope_cols=rc, kind="dot")
        torch.testing.assert_close(out.float().cpu(), ref, **tol(torch.float16))


@pytest.mark.parametrize("m", [1, 3, 8])
def test_decode_step_fused_matches_composed_and_graph(m):
    from fused_decode.decode_step import DecodeStep

    fused = DecodeStep(m=m, layers=2, h=256, i=512, seed=15, fused=True)
    comp = DecodeStep(m=m, layers=2, h=256, i=512, seed=15, fused=False)
    a = fused.step().clone()
    c = comp.step().clone()
    torch.testing.assert_close(a, c, **tol(torch.float16))
    torch.testing.assert_close(fused.qkv, comp.qkv, **tol(torch.float16))
    fused.capture()
    for _ in range(3):
        fused.out.zero_()
        out = fused.replay()
        torch.cuda.synchronize()
        torch.testing.assert_close(out, a, rtol=0, atol=0)
    assert fused.launches_per_layer == 4  # from 5 rows with the row-sum handoff
    assert comp.launches_per_layer == 6  # the MLP is two launches up to 8 rows
