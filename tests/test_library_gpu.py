"""torch.library registration on the GPU: torch.library.opcheck of every custom op,
a torch.compile(fullgraph) trace of a decode layer built from them against the
eager operators (bit-exact: the same HIP launches run), and HIP-graph capture."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module")
def fdl():
    import fused_decode._lib as L
    import fused_decode  # noqa: F401

    L.lib()  # raises if the HIP library is missing
    return torch.ops.fused_decode


def rnd(*shape, seed, scale=1.0, mean=0.0, dtype=torch.float16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale + mean).to(dtype).to(DEV)


def layer_inputs(m=2, h=256, i=512, heads=2, kv=1, d=64):
    n = (heads + 2 * kv) * d
    return dict(
        x=rnd(m, h, seed=1), nw1=rnd(h, seed=2, scale=0.1, mean=1.0), wqkv=rnd(n, h, seed=3, scale=h ** -0.5),
        cos=rnd(1, d, seed=4), sin=rnd(1, d, seed=5), attn=rnd(m, h, seed=6), wo=rnd(h, h, seed=7, scale=h ** -0.5),
        nw2=rnd(h, seed=8, scale=0.1, mean=1.0), wgu=rnd(2 * i, h, seed=9, scale=h ** -0.5),
        wd=rnd(h, i, seed=10, scale=i ** -0.5), rc=(heads + kv) * d)


def test_opcheck_every_op(fdl):
    t = layer_inputs()
    x, nw = t["x"], t["nw1"]
    q = rnd(1, 3, 4, 64, seed=11)
    cs, sn = rnd(3, 1, 64, seed=12), rnd(3, 1, 64, seed=13)
    cases = [
        (fdl.rms_norm, (x, nw, 1e-5)),
        (fdl.add_rms_norm, (x, t["attn"], nw, 1e-5)),
        (fdl.rope, (q, cs, sn)),
        (fdl.swiglu, (x, t["attn"])),
        (fdl.linear_decode, (x, t["wo"], None, t["attn"], "simt")),
        (fdl.post_attn_mlp, (x, nw, t["wgu"], t["wd"], 1e-5, None)),
        (fdl.pre_attn_qkv, (x, nw, t["wqkv"], t["cos"], t["sin"], 1e-5, t["rc"], None, "dot")),
    ]
    import fused_decode as fd

    q8, s8 = fd.quantize_fp8(t["wqkv"])
    g8, sg = fd.quantize_fp8(t["wgu"])
    d8, sd = fd.quantize_fp8(t["wd"])
    o8, so = fd.quantize_fp8(t["wo"])
    for op, args in cases:
        torch.library.opcheck(op, args)
    # The schema check compares inputs before and after with arithmetic torch does
    # not implement for float8_e4m3fn tensors, so the fp8 ops run the other checks.
    fp8_cases = [
        (fdl.linear_decode_fp8, (t["attn"], o8, so, None, x)),
        (fdl.post_attn_mlp_fp8, (x, nw, g8, sg, d8, sd, 1e-5)),
        (fdl.pre_attn_qkv_fp8, (x, nw, q8, s8, t["cos"], t["sin"], 1e-5, t["rc"], None)),
    ]
    for op, args in fp8_cases:
        torch.library.opcheck(op, args, test_utils=("test_faketensor", "test_aot_dispatch_dynamic"))


def test_compiled_layer_matches_eager_operators(fdl):
    import fused_decode as fd

    t = layer_inputs()

    def layer_ops(x):
        qkv = fdl.pre_attn_qkv(x, t["nw1"], t["wqkv"], t["cos"], t["sin"], 1e-5, t["rc"])
        h = fdl.linear_decode(t["attn"], t["wo"], None, x)
        return fdl.post_attn_mlp(h, t["nw2"], t["wgu"], t["wd"], 1e-5), qkv

    def layer_eager(x):
        qkv = fd.pre_attn_qkv(x, t["nw1"], t["wqkv"], t["cos"], t["sin"], 1e-5, rope_cols=t["rc"])
        h = fd.linear_decode(t["attn"], t["wo"], row_add=x)
        return fd.post_attn_mlp(h, t["nw2"], t["wgu"], t["wd"], 1e-5), qkv

    compiled = torch.compile(layer_ops, backend="aot_eager", fullgraph=True)
    y_c, qkv_c = compiled(t["x"])
    y_e, qkv_e = layer_eager(t["x"])
    torch.testing.assert_close(y_c, y_e, rtol=0, atol=0)
    torch.testing.assert_close(qkv_c, qkv_e, rtol=0, atol=0)


def test_custom_ops_capture_in_a_hip_graph(fdl):
    t = layer_inputs(m=1)
    x = t["x"]
    ref = fdl.post_attn_mlp(x, t["nw2"], t["wgu"], t["wd"], 1e-5).clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fdl.post_attn_mlp(x, t["nw2"], t["wgu"], t["wd"], 1e-5)
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fdl.post_attn_mlp(x, t["nw2"], t["wgu"], t["wd"], 1e-5)
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        torch.testing.assert_close(out, ref, rtol=0, atol=0)


# ------------------------------------------------ custom ops against the oracle
#
# Tolerances follow the reference's tests/test_ops.py:27-38: GEMV-shaped outputs
# fp16 rtol=atol=2e-2 (bf16 4e-2), pointwise fp16 rtol 1e-2 / atol 5e-3 (bf16 2e-2).


def _tol(dtype, kind):
    if kind == "linear":
        return {"rtol": 2e-2, "atol": 2e-2} if dtype == torch.float16 else {"rtol": 4e-2, "atol": 4e-2}
    return {"rtol": 1e-2, "atol": 5e-3} if dtype == torch.float16 else {"rtol": 2e-2, "atol": 2e-2}


def _np(t):
    return t.detach().float().cpu().numpy()


def _close(actual, expected, dtype, kind):
    torch.testing.assert_close(actual.float().cpu(), torch.from_numpy(expected), **_tol(dtype, kind))


def _oracle_cases(dtype, m):
    """(op name, args for torch.ops.fused_decode, oracle output(s), tolerance kind)."""
    from oracle import decode_oracle as O

    tg = "f16" if dtype == torch.float16 else "bf16"
    h, i, d, heads, kv = 256, 384, 64, 2, 1
    n = (heads + 2 * kv) * d
    g = torch.Generator().manual_seed(70 + m)

    def r(*shape, scale=1.0, mean=0.0, dt=dtype):
        return (torch.randn(*shape, generator=g) * scale + mean).to(dt).to(DEV)

    x, res, nw = r(m, h), r(m, h), r(h, scale=0.1, mean=1.0)
    gate, up = r(m, i, scale=2.0), r(m, i, scale=2.0)
    q = r(1, m, 4, d)
    cos3, sin3 = r(m, 1, d, dt=torch.float32), r(m, 1, d, dt=torch.float32)
    w, bias, row = r(n, h, scale=h ** -0.5), r(n, dt=torch.float32), r(m, n)
    wgu, wd = r(2 * i, h, scale=h ** -0.5), r(h, i, scale=i ** -0.5)
    ang = torch.arange(d // 2, dtype=torch.float64) * 0.21
    cos = torch.cat([ang.cos(), ang.cos()]).float().view(1, d).to(DEV)
    sin = torch.cat([ang.sin(), ang.sin()]).float().view(1, d).to(DEV)
    rc = (heads + kv) * d
    import fused_decode as fd

    q8, s8 = fd.quantize_fp8(w)
    g8, sg = fd.quantize_fp8(wgu)
    d8, sdn = fd.quantize_fp8(wd)
    c = lambda t: t.cpu().view(torch.uint8).numpy()  # noqa: E731
    return [
        ("rms_norm", (x, nw, 1e-5), O.rms_norm(_np(x), _np(nw), 1e-5, tg), "pointwise"),
        ("add_rms_norm", (x, res, nw, 1e-5), O.add_rms_norm(_np(x), _np(res), _np(nw), 1e-5, tg), "pointwise"),
        ("rope", (q, cos3, sin3), O.rope(_np(q), _np(cos3), _np(sin3), tg), "pointwise"),
        ("swiglu", (gate, up), O.swiglu(_np(gate), _np(up), tg), "pointwise"),
        ("linear_decode", (x, w, bias, row, "dot"),
         O.linear(_np(x), _np(w), bias=_np(bias), row_add=_np(row), dtype=tg), "linear"),
        ("linear_decode", (x, w, bias, row, "simt"),
         O.linear(_np(x), _np(w), bias=_np(bias), row_add=_np(row), dtype=tg), "linear"),
        ("post_attn_mlp", (x, nw, wgu, wd, 1e-5, None),
         O.post_attn_mlp(_np(x), _np(nw), _np(wgu), _np(wd), 1e-5, tg), "linear"),
        ("pre_attn_qkv", (x, nw, w, cos, sin, 1e-5, rc, bias, None),
         O.pre_attn_qkv(_np(x), _np(nw), _np(w), _np(cos), _np(sin), 1e-5, rc, bias=_np(bias), dtype=tg),
         "linear"),
        ("linear_decode_fp8", (x, q8, s8, bias, row),
         O.linear_fp8(_np(x), c(q8), _np(s8), bias=_np(bias), row_add=_np(row), dtype=tg), "linear"),
        ("post_attn_mlp_fp8", (x, nw, g8, sg, d8, sdn, 1e-5),
         O.post_attn_mlp_fp8(_np(x), _np(nw), c(g8), _np(sg), c(d8), _np(sdn), 1e-5, tg), "linear"),
        ("pre_attn_qkv_fp8", (x, nw, q8, s8, cos, sin, 1e-5, rc, bias),
         O.pre_attn_qkv_fp8(_np(x), _np(nw), c(q8), _np(s8), _np(cos), _np(sin), 1e-5, rc,
                            bias=_np(bias), dtype=tg), "linear"),
    ]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m", [1, 6])
def test_custom_ops_match_the_oracle(fdl, dtype, m):
    """Every torch.ops.fused_decode op, called eagerly and (at 6 rows) through a
    torch.compile(fullgraph) graph, against the oracle on the same inputs."""
    seen = set()
    for name, args, expected, kind in _oracle_cases(dtype, m):
        op = getattr(fdl, name)
        outs = [op(*args)]
        if m == 6:
            torch.compiler.reset()  # one wrapper code object serves every op: start each afresh
            compiled = torch.compile(lambda *a, op=op: op(*a), backend="aot_eager", fullgraph=True)
            outs.append(compiled(*args))
        for got in outs:
            if isinstance(expected, tuple):  # add_rms_norm: (out, residual_out)
                for a, e in zip(got, expected):
                    _close(a, e, dtype, kind)
            else:
                _close(got, expected, dtype, kind)
        seen.add(name)
    from fused_decode.library import OPS

    assert seen == set(OPS)
