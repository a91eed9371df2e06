"""The golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py):
they load without pickle, their half-precision inputs are exactly representable
in the case's storage type, and the oracle reproduces every stored output bit
for bit, so any change to the oracle's arithmetic shows up here."""

from __future__ import annotations

import os

import numpy as np
import pytest

from oracle import decode_oracle as O

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FAMILIES = ["norms", "pointwise", "linear", "mlp", "qkv", "fp8"]
# inputs drawn in the storage type (bias, cos/sin and fp8 scales are float32)
ROUNDED = {"x", "w", "residual", "gate", "up", "row_add", "hidden", "norm_w", "w_gate_up",
           "w_down", "w_qkv"}


def load(family: str):
    return np.load(os.path.join(HERE, f"{family}.npz"), allow_pickle=False)


def cases(d) -> dict:
    out: dict = {}
    for key in d.files:
        case, name = key.split("/")
        out.setdefault(case, {})[name] = d[key]
    return out


def recompute(case: str, g: dict) -> dict:
    dt = str(g["dtype"])
    eps = float(g["eps"]) if "eps" in g else None
    rc = int(g["rope_cols"]) if "rope_cols" in g else None
    if case.startswith("rms_"):
        return {"out": O.rms_norm(g["x"], g["w"], eps, dt)}
    if case.startswith("add_rms_"):
        y, ro = O.add_rms_norm(g["x"], g["residual"], g["w"], eps, dt)
        return {"out": y, "residual_out": ro}
    if case.startswith("swiglu_"):
        return {"out": O.swiglu(g["gate"], g["up"], dt)}
    if case.startswith("rope_"):
        return {"out": O.rope(g["x"], g["cos"], g["sin"], dt)}
    if case.startswith("linear_fp8_"):
        return {"out": O.linear_fp8(g["x"], g["codes"], g["scale"], bias=g["bias"], row_add=g["row_add"], dtype=dt)}
    if case.startswith("linear_"):
        return {"out": O.linear(g["x"], g["w"], bias=g["bias"], row_add=g["row_add"], dtype=dt)}
    if case.startswith("mlp_fp8_"):
        return {"out": O.post_attn_mlp_fp8(g["hidden"], g["norm_w"], g["gu_codes"], g["gu_scale"], g["d_codes"],
                                           g["d_scale"], eps, dt)}
    if case.startswith("mlp_"):
        return {"out": O.post_attn_mlp(g["hidden"], g["norm_w"], g["w_gate_up"], g["w_down"], eps, dt)}
    if case.startswith("qkv_fp8_"):
        return {"out": O.pre_attn_qkv_fp8(g["hidden"], g["norm_w"], g["codes"], g["scale"], g["cos"], g["sin"], eps,
                                          rc, bias=g["bias"], dtype=dt)}
    if case.startswith("qkv_"):
        return {"out": O.pre_attn_qkv(g["hidden"], g["norm_w"], g["w_qkv"], g["cos"], g["sin"], eps, rc,
                                      bias=g["bias"], dtype=dt)}
    raise AssertionError(f"no recipe for fixture case {case}")


def test_every_family_is_present_and_loads_without_pickle():
    for family in FAMILIES:
        d = load(family)
        assert d.files, family
        for key in d.files:
            assert d[key].dtype != object, key


@pytest.mark.parametrize("family", FAMILIES)
def test_inputs_are_exact_in_their_storage_type(family):
    for case, g in cases(load(family)).items():
        dt = str(g["dtype"])
        for name, a in g.items():
            if name in ROUNDED:
                assert np.array_equal(O.round_to(a, dt).view(np.uint32), a.view(np.uint32)), (case, name)


@pytest.mark.parametrize("family", FAMILIES)
def test_oracle_reproduces_the_fixtures_bit_for_bit(family):
    for case, g in cases(load(family)).items():
        for name, want in recompute(case, g).items():
            got = np.ascontiguousarray(want, dtype=np.float32)
            stored = g[name]
            assert got.shape == stored.shape, (case, name)
            assert np.array_equal(got.view(np.uint32), stored.view(np.uint32)), (case, name)
            assert np.isfinite(stored).all(), (case, name)


def test_a_planted_oracle_change_fails(monkeypatch):
    """A 0.1% error planted in the oracle's SiLU no longer reproduces the MLP fixture."""
    g = cases(load("mlp"))["mlp_f16_m1"]
    silu = O.silu
    monkeypatch.setattr(O, "silu", lambda v: silu(v) * np.float32(1.001))
    got = np.ascontiguousarray(recompute("mlp_f16_m1", g)["out"], dtype=np.float32)
    assert not np.array_equal(got.view(np.uint32), g["out"].view(np.uint32))
