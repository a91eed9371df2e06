"""GPU parity on ragged shapes for the pipelined GEMV-family kernels: K not a
multiple of the SIMT step (512 fp16 / 1024 fp8 elements per wave) or of one MFMA
unit (128), K below one unit, N not a multiple of any tile, and the fused MLP
and QKV on odd widths, for both kinds, the SIMT and MFMA row ranges and both
weight formats. These are the lanes and rows whose loads read a clamped
in-bounds address and are masked where used. Tolerances as the other GEMV
tests (the reference's, tests/test_ops.py:27-35)."""

from __future__ import annotations

import pytest
import torch

from oracle import decode_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _lib_loaded():
    import fused_decode._lib as L

    L.lib()  # raises if the HIP library is missing


def tag(dtype):
    return "f16" if dtype == torch.float16 else "bf16"


def tol(dtype):
    return {"rtol": 2e-2, "atol": 2e-2} if dtype == torch.float16 else {"rtol": 4e-2, "atol": 4e-2}


def rnd(*shape, g, dtype=torch.float16, scale=1.0, mean=0.0):
    return (torch.randn(*shape, generator=g) * scale + mean).to(dtype)


def npf(t):
    return t.detach().float().cpu().numpy()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("k", [8, 24, 136, 520, 1000, 4104])
def test_linear_ragged_k(dtype, k):
    import fused_decode as fd

    g = torch.Generator().manual_seed(k)
    for n in (1, 17, 200):
        w = rnd(n, k, g=g, dtype=dtype, scale=k ** -0.5)
        b = rnd(n, g=g, dtype=torch.float32)
        wd, bd = w.to(DEV), b.to(DEV)
        for m in (1, 2, 5, 16):
            x = rnd(m, k, g=g, dtype=dtype)
            ref = O.linear(npf(x), npf(w), npf(b), dtype=tag(dtype))
            for kind in ("dot", "simt"):
                y = fd.linear_decode(x.to(DEV), wd, bd, kind=kind)
                torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(dtype),
                                           msg=lambda s: f"n={n} m={m} kind={kind}: {s}")


@pytest.mark.parametrize("h,i", [(72, 40), (520, 104), (1032, 200)])
def test_post_attn_mlp_ragged(h, i):
    import fused_decode as fd

    g = torch.Generator().manual_seed(h + i)
    norm_w = rnd(h, g=g, scale=0.1, mean=1.0)
    w_gu = rnd(2 * i, h, g=g, scale=h ** -0.5)
    w_down = rnd(h, i, g=g, scale=i ** -0.5)
    args = (norm_w.to(DEV), w_gu.to(DEV), w_down.to(DEV), 1e-5)
    for m in (1, 3, 5, 9):
        x = rnd(m, h, g=g)
        ref = O.post_attn_mlp(npf(x), npf(norm_w), npf(w_gu), npf(w_down), 1e-5, "f16")
        for kind in ("dot", "simt"):
            y = fd.post_attn_mlp(x.to(DEV), *args, kind=kind)
            torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(torch.float16),
                                       msg=lambda s: f"m={m} kind={kind}: {s}")


@pytest.mark.parametrize("h", [136, 1040])
def test_pre_attn_qkv_ragged_tail(h):
    """Rotated columns then a v block whose width is no multiple of any tile."""
    import fused_decode as fd

    g = torch.Generator().manual_seed(h)
    d = 32
    rc = 3 * d
    n = rc + 21
    norm_w = rnd(h, g=g, scale=0.1, mean=1.0)
    w = rnd(n, h, g=g, scale=h ** -0.5)
    b = rnd(n, g=g, dtype=torch.float32)
    pos = torch.arange(5, dtype=torch.float64)[:, None] * (1e4 ** (-torch.arange(0, d, 2) / d))[None]
    cos = torch.cat([pos.cos(), pos.cos()], 1).float()
    sin = torch.cat([pos.sin(), pos.sin()], 1).float()
    for m in (1, 2, 5):
        x = rnd(m, h, g=g)
        ref = O.pre_attn_qkv(npf(x), npf(norm_w), npf(w), npf(cos[:m]), npf(sin[:m]), 1e-5, rc,
                             bias=npf(b), dtype="f16")
        for kind in ("dot", "simt"):
            y = fd.pre_attn_qkv(x.to(DEV), norm_w.to(DEV), w.to(DEV), cos[:m].to(DEV), sin[:m].to(DEV),
                                1e-5, rope_cols=rc, bias=b.to(DEV), kind=kind)
            torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(torch.float16),
                                       msg=lambda s: f"m={m} kind={kind}: {s}")


def _quant(w):
    import fused_decode as fd

    q, s = fd.quantize_fp8(w.to(DEV))
    return q, s, q.cpu().view(torch.uint8).numpy(), s.cpu().numpy()


@pytest.mark.parametrize("k", [16, 48, 144, 1040, 2064])
def test_linear_fp8_ragged_k(k):
    import fused_decode as fd

    g = torch.Generator().manual_seed(500 + k)
    for n in (1, 17, 200):
        q, s, qn, sn = _quant(rnd(n, k, g=g, scale=k ** -0.5))
        for m in (1, 3, 6, 16):
            x = rnd(m, k, g=g)
            ref = O.linear_fp8(npf(x), qn, sn, dtype="f16")
            y = fd.linear_decode_fp8(x.to(DEV), q, s)
            torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(torch.float16),
                                       msg=lambda t: f"n={n} m={m}: {t}")


@pytest.mark.parametrize("h,i", [(144, 48), (1040, 208)])
def test_post_attn_mlp_fp8_ragged(h, i):
    import fused_decode as fd

    g = torch.Generator().manual_seed(600 + h)
    norm_w = rnd(h, g=g, scale=0.1, mean=1.0)
    gq, gs, gqn, gsn = _quant(rnd(2 * i, h, g=g, scale=h ** -0.5))
    dq, ds, dqn, dsn = _quant(rnd(h, i, g=g, scale=i ** -0.5))
    for m in (1, 3, 5, 9):
        x = rnd(m, h, g=g)
        ref = O.post_attn_mlp_fp8(npf(x), npf(norm_w), gqn, gsn, dqn, dsn, 1e-5, "f16")
        y = fd.post_attn_mlp_fp8(x.to(DEV), norm_w.to(DEV), gq, gs, dq, ds, 1e-5)
        torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(torch.float16),
                                   msg=lambda t: f"m={m}: {t}")


def test_pre_attn_qkv_fp8_ragged_tail():
    import fused_decode as fd

    g = torch.Generator().manual_seed(700)
    h, d = 1040, 32
    rc = 3 * d
    n = rc + 21
    norm_w = rnd(h, g=g, scale=0.1, mean=1.0)
    q, s, qn, sn = _quant(rnd(n, h, g=g, scale=h ** -0.5))
    pos = torch.arange(6, dtype=torch.float64)[:, None] * (1e4 ** (-torch.arange(0, d, 2) / d))[None]
    cos = torch.cat([pos.cos(), pos.cos()], 1).float()
    sin = torch.cat([pos.sin(), pos.sin()], 1).float()
    for m in (1, 2, 6):
        x = rnd(m, h, g=g)
        ref = O.pre_attn_qkv_fp8(npf(x), npf(norm_w), qn, sn, npf(cos[:m]), npf(sin[:m]), 1e-5, rc,
                                 dtype="f16")
        y = fd.pre_attn_qkv_fp8(x.to(DEV), norm_w.to(DEV), q, s, cos[:m].to(DEV), sin[:m].to(DEV), 1e-5,
                                rope_cols=rc)
        torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), **tol(torch.float16),
                                   msg=lambda t: f"m={m}: {t}")
