"""The operators' argument contract and their per-signature launch plans.

Every rule of fused_decode._checks.CONTRACT is broken once and must raise the
reference's exception type with a message naming the argument (the reference
tests match "CUDA", "weight", "even", tests/test_ops.py:174-187); the row-sum
forms (fused_decode.rowsq), whose C entry points see no tensor extents, break
each of their rules too and must raise before anything is launched. Then the plan
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


def _sumsq_tensors():
    """M=8 rows (the row-sum kernels run from 5), H=64, I=128, a 32-row linear
    weight and a 3x16-column QKV with 16-wide heads; every argument valid."""
    from fused_decode import rowsq

    m, h, i = 8, 64, 128
    t = dict(x=r(m, h, seed=30), hidden=r(m, h, seed=31), nw=r(h, seed=32, scale=0.1, mean=1.0),
             W=r(32, h, seed=33, scale=h ** -0.5), wgu=r(2 * i, h, seed=34, scale=h ** -0.5),
             wd=r(h, i, seed=35, scale=i ** -0.5), wqkv=r(48, h, seed=36, scale=h ** -0.5),
             cs=r(1, 16, seed=37), out32=torch.zeros(m, 32, device=DEV, dtype=F16),
             outh=torch.zeros(m, h, device=DEV, dtype=F16), out48=torch.zeros(m, 48, device=DEV, dtype=F16),
             ss32=rowsq.sumsq_buffer(32, DEV).zero_(), ssh=rowsq.sumsq_buffer(h, DEV).fill_(float(h)),
             ssh2=rowsq.sumsq_buffer(h, DEV).zero_())
    t["q8"], t["s8"] = fd().quantize_fp8(t["W"])
    t["q8gu"], t["s8gu"] = fd().quantize_fp8(t["wgu"])
    t["q8d"], t["s8d"] = fd().quantize_fp8(t["wd"])
    t["q8qkv"], t["s8qkv"] = fd().quantize_fp8(t["wqkv"])
    return t


def _rs():
    from fused_decode import rowsq

    return rowsq


def _lin(t, **kw):
    a = dict(out=t["out32"], ss_out=t["ss32"])
    a.update(kw)
    return _rs().linear_sumsq(a.pop("x", t["x"]), a.pop("weight", t["W"]), **a)


def _mlp(t, **kw):
    a = dict(hidden=t["hidden"], norm_weight=t["nw"], w_gate_up=t["wgu"], w_down=t["wd"], eps=1e-5,
             out=t["outh"], ss_in=t["ssh"], ss_out=t["ssh2"])
    a.update(kw)
    return _rs().post_attn_mlp_sumsq(a.pop("hidden"), a.pop("norm_weight"), a.pop("w_gate_up"), a.pop("w_down"),
                                     a.pop("eps"), **a)


def _qkv(t, **kw):
    a = dict(hidden=t["hidden"], norm_weight=t["nw"], w_qkv=t["wqkv"], cos=t["cs"], sin=t["cs"], eps=1e-5,
             rope_cols=32, ss_in=t["ssh"], out=t["out48"])
    a.update(kw)
    return _rs().pre_attn_qkv_sumsq(a.pop("hidden"), a.pop("norm_weight"), a.pop("w_qkv"), a.pop("cos"),
                                    a.pop("sin"), a.pop("eps"), **a)


def _lin8(t, **kw):
    a = dict(weight=t["q8"], scale=t["s8"], out=t["out32"], ss_out=t["ss32"])
    a.update(kw)
    return _rs().linear_fp8_sumsq(a.pop("x", t["x"]), a.pop("weight"), a.pop("scale"), **a)


def _mlp8(t, **kw):
    a = dict(hidden=t["hidden"], norm_weight=t["nw"], w_gate_up=t["q8gu"], gate_up_scale=t["s8gu"],
             w_down=t["q8d"], down_scale=t["s8d"], eps=1e-5, out=t["outh"], ss_in=t["ssh"], ss_out=t["ssh2"])
    a.update(kw)
    return _rs().post_attn_mlp_fp8_sumsq(a.pop("hidden"), a.pop("norm_weight"), a.pop("w_gate_up"),
                                         a.pop("gate_up_scale"), a.pop("w_down"), a.pop("down_scale"),
                                         a.pop("eps"), **a)


def _qkv8(t, **kw):
    a = dict(hidden=t["hidden"], norm_weight=t["nw"], w_qkv=t["q8qkv"], scale=t["s8qkv"], cos=t["cs"],
             sin=t["cs"], eps=1e-5, rope_cols=32, ss_in=t["ssh"], out=t["out48"])
    a.update(kw)
    return _rs().pre_attn_qkv_fp8_sumsq(a.pop("hidden"), a.pop("norm_weight"), a.pop("w_qkv"), a.pop("scale"),
                                        a.pop("cos"), a.pop("sin"), a.pop("eps"), **a)


def _strided_k(w):
    """``w``'s values with K stride 2 (every other column of a twice-wide copy)."""
    wide = torch.zeros(w.shape[0], 2 * w.shape[1], device=w.device, dtype=w.dtype)
    wide[:, ::2] = w
    return wide[:, ::2]


def _transposed(w):
    """``w``'s values in a non-contiguous (column-major) layout."""
    return w.t().contiguous().t()


# (case, call on the tensors t, exception, keyword): one case per rule of the
# six row-sum forms' contracts, each raised before any launch
BAD_SUMSQ = [
    # linear_sumsq
    ("lin x on the CPU", lambda t: _lin(t, x=t["x"].cpu()), ValueError, "CUDA"),
    ("lin weight dtype", lambda t: _lin(t, weight=t["W"].bfloat16()), ValueError, "weight"),
    ("lin K", lambda t: _lin(t, x=t["x"][:, :32].contiguous()), ValueError, "K"),
    ("lin kind name", lambda t: _lin(t, kind="mfma"), ValueError, "kind"),
    ("lin kind simt", lambda t: _lin(t, kind="simt"), ValueError, "'dot'"),
    ("lin bias shape", lambda t: _lin(t, bias=r(31)), ValueError, "bias"),
    ("lin row_add dtype", lambda t: _lin(t, row_add=r(8, 32).double()), TypeError, "row_add"),
    ("lin row_add shape", lambda t: _lin(t, row_add=r(1, 32)), ValueError, "row_add"),
    ("lin row_add strided", lambda t: _lin(t, row_add=r(32, 8).t()), ValueError, "row_add"),
    ("lin rows", lambda t: _lin(t, x=t["x"][:4], out=t["out32"][:4]), ValueError, "5 to 16 rows"),
    ("lin x strided", lambda t: _lin(t, x=_transposed(t["x"])), ValueError, "contiguous"),
    ("lin K stride", lambda t: _lin(t, weight=_strided_k(t["W"])), ValueError, "unit stride"),
    ("lin out shape", lambda t: _lin(t, out=t["out32"][:, :16]), ValueError, "out"),
    ("lin out dtype", lambda t: _lin(t, out=t["out32"].bfloat16()), TypeError, "out"),
    ("lin out device", lambda t: _lin(t, out=t["out32"].cpu()), ValueError, "out"),
    ("lin ss_out size", lambda t: _lin(t, ss_out=t["ssh"]), ValueError, "ss_out"),
    ("lin ss_out dtype", lambda t: _lin(t, ss_out=t["ss32"].half()), ValueError, "ss_out"),
    ("lin ss_out missing", lambda t: _lin(t, ss_out=None), ValueError, "ss_out"),
    # post_attn_mlp_sumsq
    ("mlp hidden dtype", lambda t: _mlp(t, hidden=t["hidden"].float()), TypeError, "float16"),
    ("mlp widths", lambda t: _mlp(t, w_gate_up=t["wgu"][:200]), ValueError, "w_gate_up"),
    ("mlp weight dtype", lambda t: _mlp(t, w_down=t["wd"].bfloat16()), TypeError, "MLP weights"),
    ("mlp norm weight", lambda t: _mlp(t, norm_weight=t["nw"][:8]), ValueError, "weight"),
    ("mlp eps", lambda t: _mlp(t, eps=float("inf")), ValueError, "eps"),
    ("mlp kind simt", lambda t: _mlp(t, kind="simt"), ValueError, "'dot'"),
    ("mlp rows", lambda t: _mlp(t, hidden=t["hidden"][:4], out=t["outh"][:4]), ValueError, "5 to 16 rows"),
    ("mlp w_gate_up strided", lambda t: _mlp(t, w_gate_up=_transposed(t["wgu"])), ValueError, "w_gate_up"),
    ("mlp w_down strided", lambda t: _mlp(t, w_down=_transposed(t["wd"])), ValueError, "w_down"),
    ("mlp out shape", lambda t: _mlp(t, out=t["out32"]), ValueError, "out"),
    ("mlp mid shape", lambda t: _mlp(t, mid=t["out32"]), ValueError, "mid"),
    ("mlp ss_in size", lambda t: _mlp(t, ss_in=t["ss32"]), ValueError, "ss_in"),
    ("mlp ss_out device", lambda t: _mlp(t, ss_out=t["ssh2"].cpu()), ValueError, "ss_out"),
    # pre_attn_qkv_sumsq
    ("qkv K", lambda t: _qkv(t, w_qkv=t["wqkv"][:, :32].contiguous()), ValueError, "K"),
    ("qkv weight dtype", lambda t: _qkv(t, w_qkv=t["wqkv"].bfloat16()), TypeError, "w_qkv"),
    ("qkv bias dtype", lambda t: _qkv(t, bias=r(48, dtype=torch.bfloat16)), TypeError, "bias"),
    ("qkv kind simt", lambda t: _qkv(t, kind="simt"), ValueError, "'dot'"),
    ("qkv w strided", lambda t: _qkv(t, w_qkv=_transposed(t["wqkv"])), ValueError, "w_qkv"),
    ("qkv ss_in missing", lambda t: _qkv(t, ss_in=None), ValueError, "ss_in"),
    ("qkv ss_in size", lambda t: _qkv(t, ss_in=t["ss32"]), ValueError, "ss_in"),
    ("qkv out shape", lambda t: _qkv(t, out=t["out32"]), ValueError, "out"),
    ("qkv rope_cols", lambda t: _qkv(t, rope_cols=40), ValueError, "rope_cols"),
    # linear_fp8_sumsq
    ("lin8 codes", lambda t: _lin8(t, weight=t["W"]), TypeError, "float8_e4m3fn"),
    ("lin8 scale", lambda t: _lin8(t, scale=t["s8"][:3]), ValueError, "scale"),
    ("lin8 K", lambda t: _lin8(t, x=t["x"][:, :32].contiguous()), ValueError, "K"),
    ("lin8 rows", lambda t: _lin8(t, x=t["x"][:4], out=t["out32"][:4]), ValueError, "5 to 16 rows"),
    ("lin8 out shape", lambda t: _lin8(t, out=t["outh"]), ValueError, "out"),
    ("lin8 ss_out size", lambda t: _lin8(t, ss_out=t["ssh"]), ValueError, "ss_out"),
    # post_attn_mlp_fp8_sumsq
    ("mlp8 codes", lambda t: _mlp8(t, w_gate_up=t["wgu"]), TypeError, "float8_e4m3fn"),
    ("mlp8 gate_up scale", lambda t: _mlp8(t, gate_up_scale=t["s8gu"][:5]), ValueError, "scale"),
    ("mlp8 down scale", lambda t: _mlp8(t, down_scale=t["s8d"].half()), ValueError, "scale"),
    ("mlp8 out shape", lambda t: _mlp8(t, out=t["out32"]), ValueError, "out"),
    ("mlp8 mid dtype", lambda t: _mlp8(t, mid=torch.empty(8, 128, device=DEV, dtype=torch.bfloat16)),
     TypeError, "mid"),
    ("mlp8 ss_in dtype", lambda t: _mlp8(t, ss_in=t["ssh"].half()), ValueError, "ss_in"),
    # pre_attn_qkv_fp8_sumsq
    ("qkv8 scale", lambda t: _qkv8(t, scale=t["s8qkv"][:7]), ValueError, "scale"),
    ("qkv8 K", lambda t: _qkv8(t, hidden=r(8, 32, seed=3)), ValueError, "K"),
    ("qkv8 ss_in missing", lambda t: _qkv8(t, ss_in=None), ValueError, "ss_in"),
    ("qkv8 out shape", lambda t: _qkv8(t, out=t["outh"]), ValueError, "out"),
]


@pytest.fixture(scope="module")
def sumsq_tensors():
    return _sumsq_tensors()


@pytest.mark.parametrize("case", [c[0] for c in BAD_SUMSQ])
def test_every_row_sum_rule_rejects_before_launch(case, sumsq_tensors):
    _, call, exc, word = next(c for c in BAD_SUMSQ if c[0] == case)
    t = sumsq_tensors
    before = {k: v.clone() for k, v in t.items() if k.startswith(("out", "ss"))}
    with pytest.raises(exc, match=word):
        call(t)
    torch.cuda.synchronize()
    for k, v in before.items():  # nothing was launched: outputs and sums untouched
        assert torch.equal(t[k], v), k


def test_row_sum_forms_accept_the_valid_arguments(sumsq_tensors):
    """The same tensors with nothing broken pass every rule and run."""
    t = sumsq_tensors
    for call in (_lin, _mlp, _qkv, _lin8, _mlp8, _qkv8):
        call(t)
    torch.cuda.synchronize()


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


def test_simt_kind_from_the_environment_stops_at_its_own_cutoff(monkeypatch):
    """With kind "simt" chosen through FUSED_DECODE_LINEAR_KIND the default
    dispatcher runs the HIP GEMV up to SIMT_DECODE_LINEAR_MAX_M rows and F.linear
    (bit-identical) above; naming the kind still runs the HIP GEMV up to 16 rows
    (reference ops.py:247-249)."""
    import torch.nn.functional as F

    f = fd()
    from fused_decode import ops

    monkeypatch.delenv("FUSED_DECODE_LINEAR", raising=False)
    monkeypatch.setenv("FUSED_DECODE_LINEAR_KIND", "simt")
    W = r(96, 512, seed=5, scale=0.05)
    for m in (ops.SIMT_DECODE_LINEAR_MAX_M, ops.SIMT_DECODE_LINEAR_MAX_M + 1, 16):
        x = r(m, 512, seed=m)
        ref = O.linear(npf(x), npf(W), dtype="f16")
        y = f.linear_decode(x, W)
        close(y, ref, "linear")
        if m > ops.SIMT_DECODE_LINEAR_MAX_M:
            assert torch.equal(y, F.linear(x, W))
        close(f.linear_decode(x, W, kind="simt"), ref, "linear")
    monkeypatch.setenv("FUSED_DECODE_LINEAR_KIND", "dot")
    x = r(16, 512, seed=16)
    close(f.linear_decode(x, W), O.linear(npf(x), npf(W), dtype="f16"), "linear")


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
