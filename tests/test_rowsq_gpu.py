"""GPU tests of the row-sum-of-squares handoff (fused_decode.rowsq): the
producer GEMVs' per-tile sums against sums of their own rounded outputs, and
each consumer (MLP gate/up normalising inside its kernel, the QKV kernel's
norm) against the oracle's composition, fp16/bf16 weights and E4M3 weights.

Tolerances are the reference's GEMV ones (tests/test_ops.py:27-35): fp16
rtol=atol=2e-2, bf16 4e-2. The tile sums are float32 sums of 16 squares,
checked to float32 rounding.
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


def rnd(*shape, seed, dtype=torch.float16, scale=1.0, mean=0.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale + mean).to(dtype)


def npf(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def tile_sums(y: torch.Tensor) -> torch.Tensor:
    """[ceil(N/16), 16] float32: sums of the squared outputs per 16-column tile
    and row (rows past M zero), in float64 then rounded."""
    m, n = y.shape
    t = (n + 15) // 16
    sq = torch.zeros(16, t * 16, dtype=torch.float64)
    sq[:m, :n] = y.double().cpu() ** 2
    return sq.view(16, t, 16).sum(-1).t().float()


def quant(w):
    import fused_decode as fd

    q, s = fd.quantize_fp8(w.to(DEV))
    return q, s, q.cpu().view(torch.uint8).numpy(), s.cpu().numpy()


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m,n", [(5, 256), (8, 264), (16, 512), (8, 4096)])
def test_linear_sumsq_tiles_and_output(dtype, m, n):
    """The output is linear_decode's, bit for bit; the tile sums are those of it
    (N = 264: a last tile of 8 columns)."""
    import fused_decode as fd
    from fused_decode.rowsq import linear_sumsq, sumsq_buffer

    k = 384
    x, w = rnd(m, k, seed=1, dtype=dtype).to(DEV), rnd(n, k, seed=2, dtype=dtype, scale=k ** -0.5).to(DEV)
    r = rnd(m, n, seed=3, dtype=dtype).to(DEV)
    ss = sumsq_buffer(n, DEV).fill_(float("nan"))
    y = torch.empty(m, n, device=DEV, dtype=dtype)
    linear_sumsq(x, w, row_add=r, out=y, ss_out=ss)
    ref = fd.linear_decode(x, w, row_add=r, kind="dot")
    torch.testing.assert_close(y, ref, rtol=0, atol=0)
    torch.testing.assert_close(ss.cpu(), tile_sums(y), rtol=2e-6, atol=1e-6)
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(O.linear(npf(x), npf(w), row_add=npf(r),
                                                                             dtype=tag(dtype))), **tol(dtype))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m", [5, 8, 16])
@pytest.mark.parametrize("nw_dtype", [None, torch.float32], ids=["nw-act", "nw-f32"])
def test_post_attn_mlp_sumsq_chain_matches_oracle(dtype, m, nw_dtype):
    """O-proj (writes the sums of h) -> MLP normalising h from them inside its
    gate/up kernel, its down projection writing the sums of the result; against
    the oracle, and the result's sums against the result."""
    from fused_decode.rowsq import linear_sumsq, post_attn_mlp_sumsq, sumsq_buffer

    h, i = 256, 512
    nw_dtype = nw_dtype or dtype
    attn, x = rnd(m, h, seed=10 + m, dtype=dtype), rnd(m, h, seed=20 + m, dtype=dtype)
    wo = rnd(h, h, seed=11, dtype=dtype, scale=h ** -0.5)
    nw = rnd(h, seed=12, dtype=nw_dtype, scale=0.3, mean=1.0)
    wgu = rnd(2 * i, h, seed=13, dtype=dtype, scale=h ** -0.5)
    wd = rnd(h, i, seed=14, dtype=dtype, scale=i ** -0.5)
    dev = [t.to(DEV) for t in (attn, x, wo, nw, wgu, wd)]
    hbuf = torch.empty(m, h, device=DEV, dtype=dtype)
    out = torch.empty(m, h, device=DEV, dtype=dtype)
    ss_h, ss_x = sumsq_buffer(h, DEV), sumsq_buffer(h, DEV)
    linear_sumsq(dev[0], dev[2], row_add=dev[1], out=hbuf, ss_out=ss_h)
    post_attn_mlp_sumsq(hbuf, dev[3], dev[4], dev[5], 1e-5, out=out, ss_in=ss_h, ss_out=ss_x)
    href = O.linear(npf(attn), npf(wo), row_add=npf(x), dtype=tag(dtype))
    ref = O.post_attn_mlp(npf(hbuf), npf(nw), npf(wgu), npf(wd), 1e-5, tag(dtype))
    torch.testing.assert_close(hbuf.float().cpu(), torch.from_numpy(href), **tol(dtype))
    torch.testing.assert_close(out.float().cpu(), torch.from_numpy(ref), **tol(dtype))
    torch.testing.assert_close(ss_x.cpu(), tile_sums(out), rtol=2e-6, atol=1e-6)


@pytest.mark.parametrize("weights", ["fp16", "fp8"])
@pytest.mark.parametrize("m", [5, 8])
def test_post_attn_mlp_sumsq_ragged_widths(weights, m):
    """H not a whole number of 128-element units (its last tile of sums half
    full, the norm weight's LDS stage zero-padded) and I not a whole tile."""
    from fused_decode.rowsq import (linear_fp8_sumsq, linear_sumsq, post_attn_mlp_fp8_sumsq,
                                    post_attn_mlp_sumsq, sumsq_buffer)

    fp8 = weights == "fp8"
    h, i = (272, 528) if fp8 else (264, 520)
    attn, x = rnd(m, h, seed=60 + m), rnd(m, h, seed=61 + m)
    nw = rnd(h, seed=62, dtype=torch.float32, scale=0.3, mean=1.0)
    wo = rnd(h, h, seed=63, scale=h ** -0.5)
    wgu, wd = rnd(2 * i, h, seed=64, scale=h ** -0.5), rnd(h, i, seed=65, scale=i ** -0.5)
    hbuf, out = (torch.empty(m, h, device=DEV, dtype=torch.float16) for _ in range(2))
    ss_h, ss_x = sumsq_buffer(h, DEV), sumsq_buffer(h, DEV)
    if fp8:
        (oq, os_, _, _), (gq, gs, gqn, gsn), (dq, ds, dqn, dsn) = quant(wo), quant(wgu), quant(wd)
        linear_fp8_sumsq(attn.to(DEV), oq, os_, row_add=x.to(DEV), out=hbuf, ss_out=ss_h)
        post_attn_mlp_fp8_sumsq(hbuf, nw.to(DEV), gq, gs, dq, ds, 1e-5, out=out, ss_in=ss_h, ss_out=ss_x)
        ref = O.post_attn_mlp_fp8(npf(hbuf), npf(nw), gqn, gsn, dqn, dsn, 1e-5, "f16")
    else:
        linear_sumsq(attn.to(DEV), wo.to(DEV), row_add=x.to(DEV), out=hbuf, ss_out=ss_h)
        post_attn_mlp_sumsq(hbuf, nw.to(DEV), wgu.to(DEV), wd.to(DEV), 1e-5, out=out, ss_in=ss_h, ss_out=ss_x)
        ref = O.post_attn_mlp(npf(hbuf), npf(nw), npf(wgu), npf(wd), 1e-5, "f16")
    torch.testing.assert_close(ss_h.cpu(), tile_sums(hbuf), rtol=2e-6, atol=1e-6)
    torch.testing.assert_close(out.float().cpu(), torch.from_numpy(ref), **tol(torch.float16))
    torch.testing.assert_close(ss_x.cpu(), tile_sums(out), rtol=2e-6, atol=1e-6)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m", [5, 8, 16])
@pytest.mark.parametrize("nw_kind", ["other", "act"])
def test_pre_attn_qkv_sumsq_matches_oracle(dtype, m, nw_kind):
    """The QKV kernel's norm from a producer's sums (MLP down projection), with
    a norm weight of the other 16-bit dtype (staged in LDS, the workgroup adds
    the sums) and of the activations' dtype (streamed with the units, each wave
    adds the sums)."""
    from fused_decode.rowsq import post_attn_mlp_sumsq, pre_attn_qkv_sumsq, sumsq_buffer

    h, i, d, heads, kv = 256, 512, 64, 4, 2
    n = (heads + 2 * kv) * d
    x = rnd(m, h, seed=30 + m, dtype=dtype)
    nw_mlp = rnd(h, seed=31, dtype=dtype, scale=0.1, mean=1.0)
    wgu, wd = rnd(2 * i, h, seed=32, dtype=dtype, scale=h ** -0.5), rnd(h, i, seed=33, dtype=dtype, scale=i ** -0.5)
    other = torch.bfloat16 if dtype == torch.float16 else torch.float16
    nw = rnd(h, seed=34, dtype=other if nw_kind == "other" else dtype, scale=0.3, mean=1.0)
    w = rnd(n, h, seed=35, dtype=dtype, scale=h ** -0.5)
    b = rnd(n, seed=36, dtype=torch.float32, scale=0.5)
    pos = torch.arange(700, 700 + m, dtype=torch.float64)
    inv = 1.0 / (500000.0 ** (torch.arange(0, d, 2, dtype=torch.float64) / d))
    emb = torch.cat([pos[:, None] * inv[None]] * 2, dim=1)
    cos, sin = emb.cos().float(), emb.sin().float()
    xd = torch.empty(m, h, device=DEV, dtype=dtype)
    ss = sumsq_buffer(h, DEV)
    post_attn_mlp_sumsq(x.to(DEV), nw_mlp.to(DEV), wgu.to(DEV), wd.to(DEV), 1e-5, out=xd, ss_out=ss)
    y = torch.empty(m, n, device=DEV, dtype=dtype)
    pre_attn_qkv_sumsq(xd, nw.to(DEV), w.to(DEV), cos.to(DEV), sin.to(DEV), 1e-5, rope_cols=(heads + kv) * d,
                       ss_in=ss, out=y, bias=b.to(DEV))
    ref = O.pre_attn_qkv(npf(xd), npf(nw), npf(w), npf(cos), npf(sin), 1e-5, (heads + kv) * d, bias=npf(b),
                         dtype=tag(dtype))
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(dtype))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m", [5, 8, 16])
def test_fp8_sumsq_chain_matches_oracle(dtype, m):
    """The E4M3 forms: O-proj writing sums -> MLP from them, writing sums -> QKV
    from those, each against the oracle on the previous stage's actual output."""
    from fused_decode.rowsq import linear_fp8_sumsq, post_attn_mlp_fp8_sumsq, pre_attn_qkv_fp8_sumsq, sumsq_buffer

    h, i, d, heads, kv = 256, 512, 64, 4, 2
    n = (heads + 2 * kv) * d
    attn, x = rnd(m, h, seed=40 + m, dtype=dtype), rnd(m, h, seed=50 + m, dtype=dtype)
    oq, os_, oqn, osn = quant(rnd(h, h, seed=41, scale=h ** -0.5))
    gq, gs, gqn, gsn = quant(rnd(2 * i, h, seed=42, scale=h ** -0.5))
    dq, ds, dqn, dsn = quant(rnd(h, i, seed=43, scale=i ** -0.5))
    qq, qs, qqn, qsn = quant(rnd(n, h, seed=44, scale=h ** -0.5))
    nw1 = rnd(h, seed=45, dtype=torch.float32, scale=0.3, mean=1.0)
    nw2 = rnd(h, seed=46, dtype=dtype, scale=0.3, mean=1.0)
    cos = torch.cos(torch.arange(d, dtype=torch.float32) * 0.37 + 1.0)
    sin = torch.sin(torch.arange(d, dtype=torch.float32) * 0.37 + 1.0)
    hbuf, xbuf = (torch.empty(m, h, device=DEV, dtype=dtype) for _ in range(2))
    y = torch.empty(m, n, device=DEV, dtype=dtype)
    ss_h, ss_x = sumsq_buffer(h, DEV), sumsq_buffer(h, DEV)
    linear_fp8_sumsq(attn.to(DEV), oq, os_, row_add=x.to(DEV), out=hbuf, ss_out=ss_h)
    post_attn_mlp_fp8_sumsq(hbuf, nw1.to(DEV), gq, gs, dq, ds, 1e-5, out=xbuf, ss_in=ss_h, ss_out=ss_x)
    pre_attn_qkv_fp8_sumsq(xbuf, nw2.to(DEV), qq, qs, cos.to(DEV), sin.to(DEV), 1e-5, rope_cols=(heads + kv) * d,
                           ss_in=ss_x, out=y)
    t = tag(dtype)
    torch.testing.assert_close(hbuf.float().cpu(), torch.from_numpy(
        O.linear_fp8(npf(attn), oqn, osn, row_add=npf(x), dtype=t)), **tol(dtype))
    torch.testing.assert_close(ss_h.cpu(), tile_sums(hbuf), rtol=2e-6, atol=1e-6)
    torch.testing.assert_close(xbuf.float().cpu(), torch.from_numpy(
        O.post_attn_mlp_fp8(npf(hbuf), npf(nw1), gqn, gsn, dqn, dsn, 1e-5, t)), **tol(dtype))
    torch.testing.assert_close(ss_x.cpu(), tile_sums(xbuf), rtol=2e-6, atol=1e-6)
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(
        O.pre_attn_qkv_fp8(npf(xbuf), npf(nw2), qqn, qsn, npf(cos), npf(sin), 1e-5, (heads + kv) * d,
                           dtype=t)), **tol(dtype))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m", [5, 8, 16])
@pytest.mark.parametrize("h", [2048, 2064])
def test_fp8_sumsq_wide_launch_shapes(dtype, m, h):
    """The E4M3 row-sum launches at widths where their wide shapes run: the
    O-proj-like GEMV writing sums (one tile per CU and 16 or more K units: four
    waves with four units in flight each; H = 2064 ends in a partial unit), the
    QKV taking its norm from those sums (from 8 K units at up to 8 rows: eight
    waves), and the down projection at Llama-3-8B size (N = 4096, K = 14336)."""
    from fused_decode.rowsq import linear_fp8_sumsq, pre_attn_qkv_fp8_sumsq, sumsq_buffer

    d, heads, kv = 128, 16, 4
    n = (heads + 2 * kv) * d
    attn, x = rnd(m, h, seed=60 + m, dtype=dtype), rnd(m, h, seed=70 + m, dtype=dtype)
    oq, os_, oqn, osn = quant(rnd(h, h, seed=61, scale=h ** -0.5))
    qq, qs, qqn, qsn = quant(rnd(n, h, seed=62, scale=h ** -0.5))
    nw = rnd(h, seed=63, dtype=dtype, scale=0.3, mean=1.0)
    ang = torch.arange(d, dtype=torch.float32) * 0.37 + 1.0
    cos, sin = torch.cos(ang), torch.sin(ang)
    hbuf = torch.empty(m, h, device=DEV, dtype=dtype)
    y = torch.empty(m, n, device=DEV, dtype=dtype)
    ss_h = sumsq_buffer(h, DEV)
    linear_fp8_sumsq(attn.to(DEV), oq, os_, row_add=x.to(DEV), out=hbuf, ss_out=ss_h)
    pre_attn_qkv_fp8_sumsq(hbuf, nw.to(DEV), qq, qs, cos.to(DEV), sin.to(DEV), 1e-5, rope_cols=(heads + kv) * d,
                           ss_in=ss_h, out=y)
    t = tag(dtype)
    torch.testing.assert_close(hbuf.float().cpu(), torch.from_numpy(
        O.linear_fp8(npf(attn), oqn, osn, row_add=npf(x), dtype=t)), **tol(dtype))
    torch.testing.assert_close(ss_h.cpu(), tile_sums(hbuf), rtol=2e-6, atol=1e-6)
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(
        O.pre_attn_qkv_fp8(npf(hbuf), npf(nw), qqn, qsn, npf(cos), npf(sin), 1e-5, (heads + kv) * d,
                           dtype=t)), **tol(dtype))
    if h == 2048:  # the down projection's shape, its residual as row_add
        k_d, n_d = 14336, 4096
        mid, res = rnd(m, k_d, seed=64 + m, dtype=dtype), rnd(m, n_d, seed=65 + m, dtype=dtype)
        dq, ds, dqn, dsn = quant(rnd(n_d, k_d, seed=66, scale=k_d ** -0.5))
        out = torch.empty(m, n_d, device=DEV, dtype=dtype)
        ss = sumsq_buffer(n_d, DEV)
        linear_fp8_sumsq(mid.to(DEV), dq, ds, row_add=res.to(DEV), out=out, ss_out=ss)
        torch.testing.assert_close(out.float().cpu(), torch.from_numpy(
            O.linear_fp8(npf(mid), dqn, dsn, row_add=npf(res), dtype=t)), **tol(dtype))
        torch.testing.assert_close(ss.cpu(), tile_sums(out), rtol=2e-6, atol=1e-6)


@pytest.mark.parametrize("weights", ["fp16", "fp8"])
@pytest.mark.parametrize("m", [5, 8, 16])
def test_decode_step_rowsq_matches_row_kernel_form(weights, m):
    """The decode step with and without the handoff (four launches per layer;
    five without it where the fp16 MLP from 9 rows runs its norm as a row
    kernel), the same values within the GEMV tolerance (the norms' sums are
    added in another order), graph replays identical to eager."""
    from fused_decode.decode_step import DecodeStep

    a = DecodeStep(m=m, layers=3, h=256, i=512, seed=25, weights=weights)
    b = DecodeStep(m=m, layers=3, h=256, i=512, seed=25, weights=weights, rowsq=False)
    assert a.rowsq and not b.rowsq
    assert (a.launches_per_layer, b.launches_per_layer) == (4, 5 if weights == "fp16" and m > 8 else 4)
    ya, yb = a.step().clone(), b.step().clone()
    torch.testing.assert_close(ya, yb, **tol(torch.float16))
    torch.testing.assert_close(a.qkv, b.qkv, **tol(torch.float16))
    a.capture()
    for _ in range(3):
        a.out.zero_()
        out = a.replay()
        torch.cuda.synchronize()
        torch.testing.assert_close(out, ya, rtol=0, atol=0)
        _ = (a.x_in.float() * 3).sum().item()
