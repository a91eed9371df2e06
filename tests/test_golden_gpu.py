"""The HIP operators on the golden fixtures' inputs (tests/golden/*.npz) against
the stored oracle outputs, at the reference's tolerances (tests/test_ops.py:27-35:
pointwise fp16 rtol 1e-2 / atol 5e-3, bf16 2e-2; GEMV fp16 2e-2, bf16 4e-2).
The GEMV, MLP and QKV cases run both kinds; M = 6 takes the MFMA forms."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from test_golden import FAMILIES, cases, load

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _lib_loaded():
    import fused_decode._lib as L

    L.lib()  # raises if the HIP library is missing: no silent fallback


def tol(dt: str, kind: str):
    if kind == "gemv":
        return {"rtol": 2e-2, "atol": 2e-2} if dt == "f16" else {"rtol": 4e-2, "atol": 4e-2}
    return {"rtol": 1e-2, "atol": 5e-3} if dt == "f16" else {"rtol": 2e-2, "atol": 2e-2}


def act(a: np.ndarray, dt: str) -> torch.Tensor:
    """An exactly representable float32 array as a device tensor of the storage type."""
    return torch.from_numpy(np.ascontiguousarray(a)).to(torch.float16 if dt == "f16" else torch.bfloat16).to(DEV)


def f32(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def codes(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).view(torch.float8_e4m3fn).to(DEV)


def run(case: str, g: dict, kind: str) -> dict:
    import fused_decode as fd

    dt = str(g["dtype"])
    eps = float(g["eps"]) if "eps" in g else None
    rc = int(g["rope_cols"]) if "rope_cols" in g else None
    if case.startswith("rms_"):
        return {"out": fd.rms_norm(act(g["x"], dt), act(g["w"], dt), eps)}
    if case.startswith("add_rms_"):
        y, ro = fd.add_rms_norm(act(g["x"], dt), act(g["residual"], dt), act(g["w"], dt), eps)
        return {"out": y, "residual_out": ro}
    if case.startswith("swiglu_"):
        return {"out": fd.swiglu(act(g["gate"], dt), act(g["up"], dt))}
    if case.startswith("rope_"):
        return {"out": fd.rope(act(g["x"], dt), f32(g["cos"]), f32(g["sin"]))}
    if case.startswith("linear_fp8_"):
        return {"out": fd.linear_decode_fp8(act(g["x"], dt), codes(g["codes"]), f32(g["scale"]), f32(g["bias"]),
                                            row_add=act(g["row_add"], dt))}
    if case.startswith("linear_"):
        return {"out": fd.linear_decode(act(g["x"], dt), act(g["w"], dt), f32(g["bias"]),
                                        row_add=act(g["row_add"], dt), kind=kind)}
    if case.startswith("mlp_fp8_"):
        return {"out": fd.post_attn_mlp_fp8(act(g["hidden"], dt), act(g["norm_w"], dt), codes(g["gu_codes"]),
                                            f32(g["gu_scale"]), codes(g["d_codes"]), f32(g["d_scale"]), eps)}
    if case.startswith("mlp_"):
        return {"out": fd.post_attn_mlp(act(g["hidden"], dt), act(g["norm_w"], dt), act(g["w_gate_up"], dt),
                                        act(g["w_down"], dt), eps, kind=kind)}
    if case.startswith("qkv_fp8_"):
        return {"out": fd.pre_attn_qkv_fp8(act(g["hidden"], dt), act(g["norm_w"], dt), codes(g["codes"]),
                                           f32(g["scale"]), f32(g["cos"]), f32(g["sin"]), eps, rope_cols=rc,
                                           bias=f32(g["bias"]))}
    if case.startswith("qkv_"):
        return {"out": fd.pre_attn_qkv(act(g["hidden"], dt), act(g["norm_w"], dt), act(g["w_qkv"], dt),
                                       f32(g["cos"]), f32(g["sin"]), eps, rope_cols=rc, bias=f32(g["bias"]),
                                       kind=kind)}
    raise AssertionError(f"no recipe for fixture case {case}")


# the pointwise and fp8 entry points take no kind
PARAMS = [(f, k) for f in FAMILIES for k in (("dot", "simt") if f in ("linear", "mlp", "qkv") else (None,))]


@pytest.mark.parametrize("family,kind", PARAMS)
def test_hip_matches_the_golden_outputs(family, kind):
    pointwise = family in ("norms", "pointwise")
    for case, g in cases(load(family)).items():
        dt = str(g["dtype"])
        for name, y in run(case, g, kind).items():
            assert y.is_cuda
            torch.testing.assert_close(y.float().cpu(), torch.from_numpy(g[name]),
                                       **tol(dt, "pointwise" if pointwise else "gemv"), msg=f"{case}/{name}")
