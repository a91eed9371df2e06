"""GPU parity of the FP8-weight GEMV and MLP against the oracle's E4M3 products
(oracle.linear_fp8 / post_attn_mlp_fp8 on the same codes and scales), at the
reference's GEMV tolerance (tests/test_ops.py:27-35: fp16 2e-2, bf16 4e-2): the
codes are decoded exactly on both sides, so only summation order differs."""

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
@pytest.mark.parametrize("m", [1, 2, 5, 8, 13, 16])
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


def test_linear_fp8_fallback_shapes():
    import fused_decode as fd

    x = rnd(24, 200, seed=9)  # 24 rows > 16 and K % 16 != 0: the float32 path
    q, s, qn, sn = quant(rnd(48, 200, seed=10, scale=0.1))
    y = fd.linear_decode_fp8(x.to(DEV), q, s)
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(O.linear_fp8(npf(x), qn, sn, dtype="f16")),
                               **tol(torch.float16))


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


def test_decode_step_fp8_matches_oracle_and_graph():
    from fused_decode.decode_step import HEAD_DIM, DecodeStep

    m = 2
    ds = DecodeStep(m=m, layers=2, h=256, i=512, seed=5, weights="fp8")
    eager = ds.step().clone()
    codes = lambda q: q.cpu().view(torch.uint8).numpy()  # noqa: E731
    x = npf(ds.x_in)
    cos, sin = npf(ds.cos), npf(ds.sin)
    qk = ds.qk_heads * HEAD_DIM
    for w in ds.w:
        normed = O.rms_norm(x, npf(w["attn_norm"]), 1e-5, "f16")
        qkv = O.linear_fp8(normed, codes(w["qkv"][0]), npf(w["qkv"][1]), dtype="f16")
        q = qkv[:, :qk].reshape(m, ds.qk_heads, HEAD_DIM)
        qkv[:, :qk] = O.rope(q, cos, sin, "f16").reshape(m, qk)
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
    assert ds.launches_per_layer == 6
