"""Host logic on the CPU: joint row layouts, kind resolution, env knobs and the
reference's input validation (the checks that run before any device work)."""

from __future__ import annotations

import pytest
import torch

from fused_decode import _layout, kernels, ops


def rows_tuple(r):
    return (r.a, r.b, r.c, r.sa, r.sb, r.sc, r.col, r.n)


def test_contiguous_collapses_to_one_dim():
    x = torch.empty(2, 8, 64)
    (li,), (lo,) = _layout.joint_layout([x], [torch.empty(2, 8, 64)])
    assert rows_tuple(li.rows) == (1, 1, 16, 0, 0, 64, 1, 64)
    assert lo.target is None


def test_transposed_keeps_two_dims_for_all_operands():
    x = torch.empty(7, 9, 32).transpose(0, 1)  # [9, 7, 32]
    out = torch.empty(9, 7, 32)
    (li,), (lo,) = _layout.joint_layout([x], [out])
    assert rows_tuple(li.rows) == (1, 9, 7, 0, 32, 9 * 32, 1, 32)
    assert rows_tuple(lo.rows) == (1, 9, 7, 0, 7 * 32, 32, 1, 32)


def test_broadcast_angles_get_zero_strides():
    x = torch.empty(1, 2048, 32, 128)
    cos = torch.empty(2048, 1, 128).expand(x.shape)
    (lx, lc), _ = _layout.joint_layout([x, cos], [torch.empty_like(x)])
    assert (lx.rows.b, lx.rows.c) == (2048, 32)
    assert (lc.rows.sb, lc.rows.sc) == (128, 0)


def test_column_stride_is_kept():
    base = torch.empty(32, 48)
    (li,), _ = _layout.joint_layout([base.t()], [torch.empty(48, 32)])
    assert li.rows.col == 48 and li.rows.c == 48 and li.rows.sc == 1


def test_unexpressible_output_is_written_back():
    """A non-contiguous output whose layout needs more than three leading dims is
    computed into a temporary and copied back (never silently dropped)."""
    x = torch.arange(2 * 3 * 4 * 5 * 8.0).view(2, 3, 4, 5, 8)
    out = torch.zeros(5, 4, 3, 2, 8).permute(3, 2, 1, 0, 4)  # [2,3,4,5,8], 4 unmergeable dims
    _, (lo,) = _layout.joint_layout([x], [out])
    assert lo.target is out and lo.tensor is not out
    lo.tensor.copy_(x)
    _layout.finish([lo])
    assert torch.equal(out, x)


def test_five_unmergeable_dims_fall_back_to_contiguous():
    x = torch.empty(2, 3, 4, 5, 6, 8).permute(4, 3, 2, 1, 0, 5)
    out = torch.empty(x.shape).permute(1, 0, 2, 3, 4, 5).contiguous().permute(1, 0, 2, 3, 4, 5)
    (li,), (lo,) = _layout.joint_layout([x], [out])
    assert li.tensor.is_contiguous() and lo.tensor.is_contiguous()
    assert li.rows.c * li.rows.b * li.rows.a == 6 * 5 * 4 * 3 * 2
    assert lo.target is out


def test_resolve_kind(monkeypatch):
    monkeypatch.delenv("FUSED_DECODE_LINEAR_KIND", raising=False)
    assert kernels.resolve_kind(None) == "dot"
    monkeypatch.setenv("FUSED_DECODE_LINEAR_KIND", "simt")
    assert kernels.resolve_kind(None) == "simt"
    assert kernels.resolve_kind("dot") == "dot"
    with pytest.raises(ValueError, match="kind"):
        kernels.resolve_kind("mfma")
    monkeypatch.setenv("FUSED_DECODE_LINEAR_KIND", "bogus")
    with pytest.raises(ValueError):
        kernels.resolve_kind(None)


def test_rms_block_env_validation(monkeypatch):
    monkeypatch.setenv("FUSED_DECODE_RMS_BLOCK", "1000")
    with pytest.raises(ValueError, match="power of 2"):
        kernels._rms_env()


def test_linear_config_tiling(monkeypatch):
    monkeypatch.delenv("FUSED_DECODE_LINEAR", raising=False)
    monkeypatch.setattr(kernels, "_TILE_TABLE", {})
    assert kernels.linear_config("dot", 4096, 4096) == (16, 128, 4, 2)        # MFMA kernel, 2 units in flight
    assert kernels.linear_config("dot", 28672, 4096, 8) == (16, 128, 4, 2)
    assert kernels.linear_config("dot", 64, 256, 8) == (16, 128, 2, 2)        # two K units: two waves
    # dot below 5 rows: SIMT, rows and form left to the library (0 rows, stages 0)
    assert kernels.linear_config("dot", 4096, 4096, 1) == (0, 512, 8, 0)
    monkeypatch.setattr(kernels, "_TILE_TABLE", {"dot:4096x4096:m4": [16, 8, 1]})
    assert kernels.linear_config("dot", 4096, 4096, 4) == (16, 128, 8, 1)     # the table picks MFMA
    monkeypatch.setattr(kernels, "_TILE_TABLE", {})
    assert kernels.linear_config("simt", 4096, 14336) == (0, 512, 8, 0)
    assert kernels.linear_config("simt", 64, 100) == (0, 512, 1, 0)
    # a measured table entry wins for its exact shape and row count
    monkeypatch.setattr(kernels, "_TILE_TABLE", {"simt:4096x4096:m1": [2, 8, 1]})
    assert kernels.linear_config("simt", 4096, 4096, 1) == (2, 512, 8, 1)
    assert kernels.linear_config("simt", 4096, 4096, 2) == (0, 512, 8, 0)
    # the reference's override variable, with this build's meaning of the fields
    monkeypatch.setenv("FUSED_DECODE_LINEAR", "8,512,4,1")
    assert kernels.linear_config("simt", 4096, 4096, 1) == (8, 512, 4, 1)
    with pytest.raises(ValueError, match="block_k must be 128"):
        monkeypatch.setenv("FUSED_DECODE_LINEAR", "16,512,8,1")
        kernels.linear_config("dot", 4096, 4096, 8)
    monkeypatch.setenv("FUSED_DECODE_LINEAR", "16,128,8,1")
    with pytest.raises(ValueError, match="kind 'dot'"):
        kernels.linear_config("simt", 4096, 4096, 8)
    monkeypatch.setenv("FUSED_DECODE_LINEAR", "64,64,4")
    with pytest.raises(ValueError, match="block_n,block_k,warps,stages"):
        kernels.linear_config("simt", 4096, 4096, 1)


def test_cpu_tensors_are_rejected_like_the_reference():
    with pytest.raises(ValueError, match="CUDA"):
        ops.rms_norm(torch.randn(4, 16), torch.randn(16))
    with pytest.raises(ValueError, match="CUDA"):
        ops.linear_decode(torch.randn(1, 16, dtype=torch.float16), torch.randn(8, 16, dtype=torch.float16))
    with pytest.raises(ValueError, match="CUDA"):
        ops.post_attn_mlp(torch.randn(1, 8, dtype=torch.float16), torch.ones(8), torch.randn(16, 8), torch.randn(8, 8))
    with pytest.raises(TypeError, match="tensor"):
        ops.swiglu([1.0], torch.randn(1))


def test_exports_match_reference_surface():
    import fused_decode

    for name in ("DECODE_LINEAR_MAX_M", "add_rms_norm", "linear_decode", "post_attn_mlp",
                 "rms_norm", "rope", "swiglu"):
        assert hasattr(fused_decode, name)
    assert 1 <= fused_decode.DECODE_LINEAR_MAX_M <= 16


def test_tile_table_matches_the_dispatch_constants():
    """The committed gfx950 tile table: its cutoffs are DECODE_LINEAR_MAX_M and
    SIMT_DECODE_LINEAR_MAX_M, and every entry is a tile the library accepts for
    its kernel and row count."""
    import json

    with open(kernels.TILE_TABLE_FILE) as f:
        table = json.load(f)
    assert table["arch"] == "gfx950"
    assert table["decode_linear_max_m"] == ops.DECODE_LINEAR_MAX_M
    assert 1 <= table["strict_max_m"] <= table["decode_linear_max_m"]
    assert table["simt_decode_linear_max_m"] == ops.SIMT_DECODE_LINEAR_MAX_M
    assert 1 <= table["simt_strict_max_m"] <= table["simt_decode_linear_max_m"]
    for key, (rows, waves, stages) in table["entries"].items():
        kind, shape, m = key.split(":")
        m = int(m[1:])
        assert kind in ("dot", "simt") and 0 <= waves <= 8
        if rows == 16:
            assert kind == "dot" and stages in (1, 2, 3) and waves in (2, 4, 8)
        else:  # SIMT: the per-tile kernel (stages 1, 1-8 waves) or the persistent one
            # (stages 2; its waves spread the K chunks 1, 2 or 4 per lane over at most eight)
            assert rows in (2, 4, 8) and rows * m <= 64 and stages in (1, 2)
            chunks = -(-int(shape.split("x")[1]) // 512)
            assert (stages == 1 and waves >= 1) or (stages == 2 and chunks <= 8 * 4)


def test_quantize_fp8_on_cpu_matches_the_oracle():
    import numpy as np

    from fused_decode.fp8 import quantize_fp8
    from oracle import decode_oracle as O

    w = torch.randn(24, 96, generator=torch.Generator().manual_seed(3)) * 0.02
    w[4] = 0
    q, s = quantize_fp8(w)
    oq, os_ = O.fp8_quantize(w.numpy())
    assert q.dtype == torch.float8_e4m3fn and s.dtype == torch.float32
    assert np.array_equal(q.view(torch.uint8).numpy(), oq) and np.array_equal(s.numpy(), os_)
