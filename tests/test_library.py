"""torch.library registration (CPU): the ops exist under torch.ops.fused_decode with
the expected schemas, their fake kernels give the real result shapes on fake CUDA
tensors, and real CPU inputs hit the operators' own validation."""

from __future__ import annotations

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode


@pytest.fixture(scope="module")
def fdl():
    import fused_decode  # noqa: F401  (registers the ops)

    return torch.ops.fused_decode


def test_every_operator_is_registered(fdl):
    from fused_decode.library import OPS

    for name in OPS:
        op = getattr(fdl, name)
        assert op.default._schema.name == f"fused_decode::{name}"
    schema = str(fdl.pre_attn_qkv.default._schema)
    assert "SymInt rope_cols" in schema and "str? kind=None" in schema
    assert "(Tensor, Tensor)" in str(fdl.add_rms_norm.default._schema)


def test_fake_kernels_give_result_shapes(fdl):
    h, i, n = 64, 96, 48
    with FakeTensorMode():
        f16 = dict(device="cuda", dtype=torch.float16)
        x = torch.empty(2, 3, h, **f16)
        w = torch.empty(h, **f16)
        assert fdl.rms_norm(x, w, 1e-5).shape == (2, 3, h)
        out, res = fdl.add_rms_norm(x, x, w, 1e-5)
        assert out.shape == res.shape == (2, 3, h) and out.dtype == torch.float16
        q = torch.empty(1, 5, 4, 32, **f16)
        assert fdl.rope(q, torch.empty(5, 1, 32, **f16), torch.empty(5, 1, 32, **f16)).shape == q.shape
        assert fdl.swiglu(x, x).shape == x.shape
        wl = torch.empty(n, h, **f16)
        assert fdl.linear_decode(x, wl).shape == (2, 3, n)
        assert fdl.linear_decode(torch.empty(h, **f16), wl, None, None, "simt").shape == (n,)
        wgu, wd = torch.empty(2 * i, h, **f16), torch.empty(h, i, **f16)
        assert fdl.post_attn_mlp(x, w, wgu, wd, 1e-5).shape == x.shape
        cs = torch.empty(1, 16, **f16)
        assert fdl.pre_attn_qkv(x, w, wl, cs, cs, 1e-5, 32).shape == (2, 3, n)
        q8 = torch.empty(n, h, device="cuda", dtype=torch.float8_e4m3fn)
        s8 = torch.empty(n, device="cuda", dtype=torch.float32)
        assert fdl.linear_decode_fp8(x, q8, s8).shape == (2, 3, n)
        g8 = torch.empty(2 * i, h, device="cuda", dtype=torch.float8_e4m3fn)
        d8 = torch.empty(h, i, device="cuda", dtype=torch.float8_e4m3fn)
        sg, sd = torch.empty(2 * i, device="cuda"), torch.empty(h, device="cuda")
        assert fdl.post_attn_mlp_fp8(x, w, g8, sg, d8, sd, 1e-5).shape == x.shape
        assert fdl.pre_attn_qkv_fp8(x, w, q8, s8, cs, cs, 1e-5, 32).shape == (2, 3, n)


def test_real_cpu_inputs_reach_the_operator_checks(fdl):
    x = torch.randn(2, 8, dtype=torch.float16)
    with pytest.raises(ValueError, match="CUDA"):
        fdl.rms_norm(x, torch.ones(8, dtype=torch.float16), 1e-6)
    with pytest.raises(ValueError, match="CUDA"):
        fdl.linear_decode(x, torch.ones(4, 8, dtype=torch.float16))
