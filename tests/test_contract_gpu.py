"""The operators' argument contract and their per-signature launch plans.

Every rule of fused_decode._checks.CONTRACT is broken once and must raise the
reference's exception type with a message naming the argument (the reference
tests match "CUDA", "weight", "even", tests/test_ops.py:174-187). Then the plan
cache: repeated calls with one signature and new values, signatures that differ
only in strides, environment variables that change between calls with an
unchanged signature, and the row_add / flattening forms linear_decode accepts,
all against the oracle (fp16 GEMV tolerance rtol=atol=2e-2, pointwise rtol
1e-2 / atol 5e-3: the reference's tests/test_ops.py:27-35).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import decode_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
F16 = torch.float16


@pytest.fixture(scope="module", autouse=True)
def _lib_loaded():
    import fused_decode._lib as L

    L.native()  # raises if the library or its binding is missing


def fd():
    import fused_decode

    return fused_decode


def r(*shape, seed=0, dtype=F16, scale=1.0, mean=0.0, dev=DEV):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale + mean).to(dtype).to(dev)


def npf(t):
    return t.detach().float().cpu().numpy()


def close(a, e, kind="pointwise"):
    tol = {"rtol": 2e-2, "atol": 2e-2} if kind == "linear" else {"rtol": 1e-2, "atol": 5e-3}
    torch.testing.assert_close(a.float().cpu(), torch.from_numpy(np.ascontiguousarray(e)), **tol)


def _tensors():
    x, w, res = r(4, 64), r(64, seed=1), r(4, 64, seed=2)
    W, q, cs = r(32, 64, seed=3), r(1, 2, 4, 64, seed=4), r(2, 1, 64, seed=5)
    q8, s8 = fd().quantize_fp8(W)
    return dict(x=x, w=w, res=res, W=W, q=q, cs=cs, wgu=r(256, 64, seed=6), wd=r(64, 128, seed=7), q8=q8, s8=s8)


# (case, call on the fused_decode module f and the tensors t, exception, keyword)
BAD = [
    ("x not a tensor", lambda f, t: f.rms_norm([1.0], t["w"]), TypeError, "tensor"),
    ("x on the CPU", lambda f, t: f.rms_norm(t["x"].cpu(), t["w"]), ValueError, "CUDA"),
    ("x float32", lambda f, t: f.rms_norm(t["x"].float(), t["w"]), TypeError, "float16"),
    ("weight length", lambda f, t: f.rms_norm(t["x"], t["w"][:32]), ValueError, "weight"),
    ("weight dtype", lambda f, t: f.rms_norm(t["x"], t["w"].double()), TypeError, "weight"),
    ("weight device", lambda f, t: f.rms_norm(t["x"], t["w"].cpu()), ValueError, "weight"),
    ("eps nan", lambda f, t: f.rms_norm(t["x"], t["w"], float("nan")), ValueError, "eps"),
    ("eps negative", lambda f, t: f.rms_norm(t["x"], t["w"], -1.0), ValueError, "eps"),
    ("out shape", lambda f, t: f.rms_norm(t["x"], t["w"], out=r(2, 64)), ValueError, "out"),
    ("out dtype", lambda f, t: f.rms_norm(t["x"], t["w"], out=t["x"].bfloat16()), TypeError, "out"),
    ("residual shape", lambda f, t: f.add_rms_norm(t["x"], t["res"][:2], t["w"]), ValueError, "residual"),
    ("residual dtype", lambda f, t: f.add_rms_norm(t["x"], t["res"].bfloat16(), t["w"]), TypeError, "residual"),
    ("residual None", lambda f, t: f.add_rms_norm(t["x"], None, t["w"]), TypeError, "residual"),
    ("residual_out shape", lambda f, t: f.add_rms_norm(t["x"], t["res"], t["w"], residual_out=r(3, 64)),
     ValueError, "residual_out"),
    ("rope odd", lambda f, t: f.rope(r(2, 3), r(2, 3), r(2, 3)), ValueError, "even"),
    ("rope cos dtype", lambda f, t: f.rope(t["q"], t["cs"].double(), t["cs"]), TypeError, "cos"),
    ("rope cos last dim", lambda f, t: f.rope(t["q"], t["cs"][..., :32], t["cs"]), ValueError, "cos"),
    ("rope cos broadcast", lambda f, t: f.rope(t["q"], r(3, 1, 64), t["cs"]), ValueError, "broadcast"),
    ("rope sin device", lambda f, t: f.rope(t["q"], t["cs"], t["cs"].cpu()), ValueError, "sin"),
    ("swiglu up shape", lambda f, t: f.swiglu(t["x"], t["res"][:1]), ValueError, "up"),
    ("linear weight rank", lambda f, t: f.linear_decode(t["x"], t["w"]), ValueError, "weight"),
    ("linear weight dtype", lambda f, t: f.linear_decode(t["x"], t["W"].bfloat16()), ValueError, "weight"),
    ("linear K", lambda f, t: f.linear_decode(t["x"][:, :32], t["W"]), ValueError, "K"),
    ("linear kind", lambda f, t: f.linear_decode(t["x"], t["W"], kind="mfma"), ValueError, "kind"),
    ("linear bias shape", lambda f, t: f.linear_decode(t["x"], t["W"], r(31)), ValueError, "bias"),
    ("linear bias dtype", lambda f, t: f.linear_decode(t["x"], t["W"], r(32, dtype=torch.bfloat16)), TypeError,
     "bias"),
    ("linear row_add dtype", lambda f, t: f.linear_decode(t["x"], t["W"], row_add=r(4, 32).double()), TypeError,
     "row_add"),
    ("linear row_add shape", lambda f, t: f.linear_decode(t["x"], t["W"], row_add=r(3, 32)), ValueError,
     "row_add"),
    ("linear out", lambda f, t: f.linear_decode(t["x"], t["W"], out=r(4, 32).t()), ValueError, "out"),
    ("mlp rank", lambda f, t: f.post_attn_mlp(t["x"], t["w"], t["wgu"].flatten(), t["wd"]), ValueError,
     "rank-2"),
    ("mlp widths", lambda f, t: f.post_attn_mlp(t["x"], t["w"], t["wgu"][:200], t["wd"]), ValueError,
     "w_gate_up"),
    ("mlp dtype", lambda f, t: f.post_attn_mlp(t["x"], t["w"], t["wgu"].bfloat16(), t["wd"]), TypeError,
     "MLP weights"),
    ("mlp norm weight", lambda f, t: f.post_attn_mlp(t["x"], t["w"][:8], t["wgu"], t["wd"]), ValueError,
     "weight"),
    ("qkv weight dtype", lambda f, t: f.pre_attn_qkv(t["x"], t["w"], t["W"].bfloat16(), t["cs"][0], t["cs"][0],
                                                       rope_cols=0), TypeError, "w_qkv"),
    ("fp8 codes", lambda f, t: f.linear_decode_fp8(t["x"], t["W"], t["s8"]), TypeError, "float8_e4m3fn"),
    ("fp8 scale", lambda f, t: f.linear_decode_fp8(t["x"], t["q8"], t["s8"][:3]), ValueError, "scale"),
]


@pytest.mark.parametrize("case", [c[0] for c in BAD])
def test_every_rule_rejects_with_its_keyword(case):
    _, call, exc, word = next(c for c in BAD if c[0] == case)
    with pytest.raises(exc, match=word):
        call(fd(), _tensors())


def test_cached_plans_follow_new_values_and_strides():
    f = fd()
    w = r(256, seed=10, scale=0.1, mean=1.0)
    for seed in (1, 2, 3):  # one signature, new values each call
        x = r(8, 256, seed=seed)
        close(f.rms_norm(x, w, 1e-5), O.rms_norm(npf(x), npf(w), 1e-5, "f16"))
    xt = r(256, 8, seed=4).t()  # same shape, transposed strides: its own plan
    close(f.rms_norm(xt, w, 1e-5), O.rms_norm(npf(xt), npf(w), 1e-5, "f16"))
    out = torch.empty(256, 8, device=DEV, dtype=F16).t()  # a strided out
    y = f.rms_norm(xt, w, 1e-5, out=out)
    assert y.data_ptr() == out.data_ptr()
    close(out, O.rms_norm(npf(xt), npf(w), 1e-5, "f16"))
    # in place, twice, through one plan
    x = r(8, 256, seed=5)
    ref = O.rms_norm(O.rms_norm(npf(x), npf(w), 1e-5, "f16"), npf(w), 1e-5, "f16")
    f.rms_norm(x, w, 1e-5, out=x)
    f.rms_norm(x, w, 1e-5, out=x)
    close(x, ref)


def test_environment_changes_reach_cached_signatures(monkeypatch):
    f = fd()
    x, W = r(1, 64), r(32, 64, seed=1, scale=0.125)
    ref = O.linear(npf(x), npf(W), dtype="f16")
    monkeypatch.delenv("FUSED_DECODE_LINEAR", raising=False)
    monkeypatch.delenv("FUSED_DECODE_LINEAR_KIND", raising=False)
    close(f.linear_decode(x, W), ref, "linear")
    monkeypatch.setenv("FUSED_DECODE_LINEAR_KIND", "bogus")
    with pytest.raises(ValueError, match="kind"):
        f.linear_decode(x, W)
    monkeypatch.setenv("FUSED_DECODE_LINEAR_KIND", "simt")
    close(f.linear_decode(x, W), ref, "linear")
    monkeypatch.setenv("FUSED_DECODE_LINEAR", "64,64,4")
    with pytest.raises(ValueError, match="block_n,block_k,warps,stages"):
        f.linear_decode(x, W)
    monkeypatch.delenv("FUSED_DECODE_LINEAR")
    xs, w = r(2, 64, seed=3), r(64, seed=4)
    f.rms_norm(xs, w)
    monkeypatch.setenv("FUSED_DECODE_RMS_BLOCK", "1000")
    with pytest.raises(ValueError, match="power of 2"):
        f.rms_norm(xs, w)


@pytest.mark.parametrize("form", ["vector", "row", "column", "full", "full_strided", "scalar", "lead3",
                                  "flat_mn", "permuted"])
def test_linear_row_add_and_flattening_forms(form):
    """Each row_add shape linear_decode accepts (the set of the reference's
    ops.py:195-209) and x flattening with and without a copy, against the oracle."""
    f = fd()
    n, k = 48, 64
    W, b = r(n, k, seed=20, scale=k ** -0.5), r(n, seed=21, dtype=torch.float32)
    x = r(6, k, seed=22)
    ra = {
        "vector": r(n, seed=23),
        "row": r(1, n, seed=23),
        "column": r(6, 1, seed=23),
        "full": r(6, n, seed=23),
        "full_strided": r(n, 6, seed=23).t(),
        "scalar": r(1, seed=23, dtype=torch.float32),
    }.get(form)
    if form in ("lead3", "flat_mn", "permuted"):
        x = r(2, 3, k, seed=22) if form != "permuted" else r(3, 2, k, seed=22).transpose(0, 1)
        ra = r(2, 3, n, seed=23) if form == "lead3" else r(6, n, seed=23)
        if form == "permuted":
            ra = r(1, 3, n, seed=23)
    y = f.linear_decode(x, W, b, row_add=ra, kind="simt")
    x2 = npf(x).reshape(-1, k)
    ra_np = npf(ra)
    if form == "lead3":
        ra_np = ra_np.reshape(6, n)
    elif form == "permuted":
        ra_np = np.broadcast_to(ra_np, (2, 3, n)).reshape(6, n)
    ref = O.linear(x2, npf(W), bias=npf(b), row_add=ra_np, dtype="f16")
    close(y.reshape(-1, n), ref, "linear")
    assert y.shape == (*x.shape[:-1], n)
