"""Every GEMV tiling the library accepts computes the same product: forced tiles
(fd_linear_tiled through linear_out, and the FUSED_DECODE_LINEAR override) against
the oracle at the GEMV tolerance (tests/test_ops.py:27-35: fp16 2e-2)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import decode_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def rnd(*shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.float16)


# (rows, waves, stages): SIMT rows 2/4/8, the per-tile kernel (stages 1) with 1-8
# waves and the persistent one (stages 2; at K = 1152, 3 chunks, waves 0, 2 and 1
# give 1, 2 and 4 chunks per lane); MFMA (16 rows) with 2, 4 or 8 waves and 1-3
# K units in flight per wave
TILES = [(2, 4, 1), (2, 8, 1), (4, 3, 1), (8, 8, 1), (2, 0, 2), (4, 0, 2), (8, 0, 2), (2, 2, 2), (2, 1, 2),
         (16, 8, 1), (16, 4, 2), (16, 2, 3), (16, 4, 3), (16, 8, 2), (0, 0, 0)]


# 8 SIMT rows per workgroup take M <= 8 (the library rejects more); four K chunks
# per lane take M <= 8 too (the persistent kernel's registers)
CASES = [(m, t) for t in TILES for m in (1, 3, 8, 13) if not (t[0] == 8 and m > 8) and not (t == (2, 1, 2) and m > 8)]


@pytest.mark.parametrize("m,tile", CASES, ids=lambda v: "r%d_w%d_s%d" % v if isinstance(v, tuple) else "m%d" % v)
def test_forced_tiles_match_oracle(m, tile):
    from fused_decode import kernels

    n, k = 200, 1152  # ragged N (not a multiple of 16), K of 9 MFMA units / 2.25 SIMT chunks
    x, w = rnd(m, k, seed=m), rnd(n, k, seed=50 + m, scale=k ** -0.5)
    bias = rnd(n, seed=90)
    row = rnd(m, n, seed=91)
    y = torch.empty(m, n, device=DEV, dtype=torch.float16)
    kernels.linear_out(x.to(DEV), w.to(DEV), y, bias=bias.to(DEV), row_add=row.to(DEV), kind="dot", tile=tile)
    ref = O.linear(x.float().numpy(), w.float().numpy(), bias.float().numpy(), row.float().numpy(), "f16")
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(np.ascontiguousarray(ref)), rtol=2e-2, atol=2e-2)


def test_env_override_runs_the_named_kernel(monkeypatch):
    import fused_decode as fd

    x, w = rnd(3, 512, seed=1), rnd(64, 512, seed=2, scale=512 ** -0.5)
    ref = O.linear(x.float().numpy(), w.float().numpy(), dtype="f16")
    for env in ("16,128,8,2", "2,512,4,1", "8,512,8,1"):
        monkeypatch.setenv("FUSED_DECODE_LINEAR", env)
        y = fd.linear_decode(x.to(DEV), w.to(DEV), kind="dot")
        torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), rtol=2e-2, atol=2e-2)
