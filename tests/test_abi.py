"""The C ABI library loads, exports every entry point include/fused_decode.h
declares, and rejects bad arguments before any HIP call (CPU only)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "fused_decode.h"


def declared() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(fd_\w+)\(", text, re.M)))


@pytest.fixture(scope="module")
def L():
    from fused_decode import _lib

    return _lib


def test_header_declares_the_operator_set():
    names = declared()
    for n in ("fd_rms_norm", "fd_add_rms_norm", "fd_swiglu", "fd_rope", "fd_linear",
              "fd_post_attn_mlp", "fd_pre_attn_qkv", "fd_copy", "fd_triad", "fd_last_error",
              "fd_version"):
        assert n in names


def test_library_exports_every_declared_symbol(L):
    lib = L.lib()
    for name in declared():
        assert hasattr(lib, name), name
    assert set(declared()) - {"fd_last_error"} == set(L.SIGNATURES)


def test_version_and_error_string(L):
    lib = L.lib()
    assert lib.fd_version() == 100
    assert lib.fd_copy(None, None, -1, None) == L.FD_EINVAL
    assert b"bytes" in lib.fd_last_error()
    assert lib.fd_copy(None, None, 0, None) == L.FD_OK  # empty copy: nothing to do
    assert lib.fd_copy_persistent(None, None, -16, 8, None) == L.FD_EINVAL
    assert lib.fd_copy_persistent(None, None, 16, 0, None) == L.FD_EINVAL and b"workgroups" in lib.fd_last_error()
    assert lib.fd_copy_persistent(None, None, 0, 8, None) == L.FD_OK
    khz = ctypes.c_int(0)
    assert lib.fd_clock_probe(None, 8, ctypes.byref(khz), None) == L.FD_EINVAL
    assert lib.fd_clock_probe(FAKE, 0, ctypes.byref(khz), None) == L.FD_EINVAL and b"workgroups" in lib.fd_last_error()
    assert lib.fd_clock_probe(FAKE + 4, 8, ctypes.byref(khz), None) == L.FD_EINVAL


@pytest.mark.skipif(torch.cuda.is_available(), reason="host-only argument checks")
def test_read_rejects(L):
    lib = L.lib()
    assert lib.fd_copy_persistent(0x1008, 0x2000, 16, 8, None) == L.FD_EUNSUPPORTED  # misaligned destination
    assert lib.fd_copy_persistent(0x1000, 0x2000, 24, 8, None) == L.FD_EUNSUPPORTED  # not whole vectors
    assert lib.fd_copy_persistent(None, 0x2000, 16, 8, None) == L.FD_EINVAL
    assert lib.fd_read(0x1000, -16, 0, 0x2000, None) == L.FD_EINVAL
    assert lib.fd_read(None, 0, 0, None, None) == L.FD_OK        # nothing to read
    assert lib.fd_read(None, 16, 0, 0x2000, None) == L.FD_EINVAL
    assert lib.fd_read(0x1000, 16, 0, None, None) == L.FD_EINVAL
    assert lib.fd_read(0x1008, 16, 0, 0x2000, None) == L.FD_EUNSUPPORTED  # misaligned source
    assert lib.fd_read(0x1000, 24, 0, 0x2000, None) == L.FD_EUNSUPPORTED  # not whole vectors
    assert lib.fd_read(0x1000, 16, 0, 0x2002, None) == L.FD_EINVAL        # misaligned flag


# Argument checks below return before any HIP call; the pointers are never
# dereferenced. Skipped where a GPU is present so no launch can ever see them.
nogpu = pytest.mark.skipif(torch.cuda.is_available(), reason="host-only argument checks")
FAKE = 0x1000


def rows(a=1, b=1, c=4, n=64, col=1, L=None):
    from fused_decode._lib import FdRows

    return FdRows(a, b, c, 0, 0, n, col, n)


@nogpu
def test_linear_rejects(L):
    lib = L.lib()
    args = dict(bias=None, bd=0, row=None, rd=0, M=4, N=8, K=16, sxm=16, sxk=1, swn=16, swk=1,
                sb=0, srm=0, srn=0, sym=8, syn=1, kind=0, act=0)

    def call(**kw):
        a = {**args, **kw}
        return lib.fd_linear(FAKE, FAKE, FAKE, a["bias"], a["bd"], a["row"], a["rd"], a["M"], a["N"],
                             a["K"], a["sxm"], a["sxk"], a["swn"], a["swk"], a["sb"], a["srm"], a["srn"],
                             a["sym"], a["syn"], a["kind"], a["act"], None)

    assert call(M=17) == L.FD_EINVAL and b"M <= 16" in lib.fd_last_error()
    assert call(kind=7) == L.FD_EINVAL and b"kind" in lib.fd_last_error()
    assert call(act=2) == L.FD_EINVAL and b"act_dtype" in lib.fd_last_error()
    assert call(bias=FAKE, bd=1) == L.FD_EINVAL and b"bias" in lib.fd_last_error()
    assert call(sxm=-1) == L.FD_EINVAL and b"stride" in lib.fd_last_error()
    assert call(M=0) == L.FD_OK  # empty: no launch


@nogpu
def test_row_ops_reject(L):
    lib = L.lib()
    r = rows()
    odd = rows(n=63)
    assert lib.fd_rope(FAKE, FAKE, FAKE, FAKE, 0, odd, odd, odd, odd, 0, None) == L.FD_EINVAL
    assert b"even" in lib.fd_last_error()
    assert lib.fd_rms_norm(FAKE, FAKE, FAKE, 5, 1, r, r, 1e-6, 0, None) == L.FD_EINVAL
    assert lib.fd_rms_norm(FAKE, FAKE, FAKE, 0, 1, r, rows(n=32), 1e-6, 0, None) == L.FD_EINVAL
    assert b"row grid" in lib.fd_last_error()
    assert lib.fd_rms_norm(FAKE, FAKE, FAKE, 0, 1, r, r, float("nan"), 0, None) == L.FD_EINVAL
    assert lib.fd_swiglu(FAKE, FAKE, FAKE, r, r, rows(c=5), 1, None) == L.FD_EINVAL
    assert lib.fd_swiglu(None, FAKE, FAKE, r, r, r, 1, None) == L.FD_EINVAL


@nogpu
def test_mlp_rejects(L):
    lib = L.lib()
    assert lib.fd_post_attn_mlp(FAKE, FAKE, FAKE, FAKE, 0, FAKE, FAKE, 17, 64, 128, 1e-6, 0, 0, None) == L.FD_EINVAL
    assert lib.fd_post_attn_mlp(FAKE, FAKE, FAKE, FAKE, 0, FAKE, FAKE, 2, 0, 128, 1e-6, 0, 0, None) == L.FD_EINVAL
    assert lib.fd_post_attn_mlp(FAKE, FAKE, FAKE, FAKE, 0, FAKE, FAKE, 2, 60, 128, 1e-6, 0, 0, None) == L.FD_EUNSUPPORTED
    assert lib.fd_post_attn_mlp(FAKE, FAKE, FAKE, FAKE, 0, FAKE, FAKE, 0, 64, 128, 1e-6, 0, 0, None) == L.FD_OK
    # kind=dot from 9 rows runs the RMSNorm as a row kernel into `normed`
    assert lib.fd_mlp_gate_up(FAKE, None, FAKE, FAKE, 0, FAKE, 9, 64, 128, 1e-6, 0, 0, None) == L.FD_EINVAL


@nogpu
def test_qkv_rejects(L):
    lib = L.lib()

    def call(m=2, h=64, n=96, rope_cols=64, head_dim=32, eps=1e-6, kind=0, normed=None, cs_rs=0):
        return lib.fd_pre_attn_qkv(FAKE, normed, FAKE, FAKE, 0, FAKE, None, 0, FAKE, FAKE, 2, cs_rs,
                                   m, h, n, rope_cols, head_dim, eps, kind, 0, None)

    assert call(m=17) == L.FD_EINVAL
    assert call(rope_cols=100) == L.FD_EINVAL            # above N
    assert call(rope_cols=48) == L.FD_EINVAL             # not a multiple of head_dim
    assert call(head_dim=31, rope_cols=62) == L.FD_EINVAL  # odd head_dim
    assert call(head_dim=24, rope_cols=48) == L.FD_EUNSUPPORTED  # head_dim % 16
    assert call(h=60) == L.FD_EUNSUPPORTED
    assert call(eps=float("nan")) == L.FD_EINVAL
    assert call(kind=5) == L.FD_EINVAL
    assert call(cs_rs=-1) == L.FD_EINVAL
    assert call(m=0) == L.FD_OK


@nogpu
def test_tiled_linear_rejects_tiles_the_kernel_cannot_run(L):
    lib = L.lib()

    def call(m, kind, rows=0, waves=0, stages=0):
        t = L.FdTile(rows, waves, stages)
        return lib.fd_linear_tiled(FAKE, FAKE, FAKE, None, 0, None, 0, m, 64, 64, 64, 1, 64, 1, 0, 0, 0,
                                   64, 1, ctypes.byref(t), kind, 0, None)

    assert call(1, 1, rows=3) == L.FD_EINVAL          # SIMT rows are 2, 4 or 8
    assert call(9, 1, rows=8) == L.FD_EINVAL          # 8 rows only up to M = 8
    assert call(1, 1, stages=3) == L.FD_EINVAL        # SIMT forms: 1 per-tile, 2 persistent
    assert call(1, 1, rows=16) == L.FD_EINVAL         # 16 rows = the MFMA kernel, kind dot only
    assert call(8, 0, rows=5) == L.FD_EINVAL
    assert call(8, 0, stages=4) == L.FD_EINVAL        # MFMA: 1-3 units in flight
    assert call(8, 0, waves=3) == L.FD_EINVAL         # MFMA: 2, 4 or 8 waves
    assert call(16, 0, rows=16, waves=8, stages=3) == L.FD_EINVAL  # ring beyond a CU's LDS
    assert call(1, 0, waves=9) == L.FD_EINVAL
    assert lib.fd_linear_tiled(FAKE, FAKE, FAKE, None, 0, None, 0, 0, 64, 64, 64, 1, 64, 1, 0, 0, 0,
                               64, 1, None, 1, 0, None) == L.FD_OK   # M = 0, default tile


@nogpu
def test_fp8_entry_points_reject(L):
    lib = L.lib()

    def lin(m=1, k=64, swn=64, x=FAKE):
        return lib.fd_linear_fp8(FAKE, x, FAKE, FAKE, None, 0, None, 0, m, 32, k, k, swn, 0, 0, 0, 32, 1, 0, None)

    assert lin(m=17) == L.FD_EINVAL
    assert lin(k=40, swn=40) == L.FD_EUNSUPPORTED     # K % 16
    assert lin(x=FAKE + 2) == L.FD_EUNSUPPORTED       # misaligned activations
    assert lib.fd_linear_fp8(FAKE, FAKE, FAKE, None, None, 0, None, 0, 1, 32, 64, 64, 64, 0, 0, 0, 32, 1, 0,
                             None) == L.FD_EINVAL      # scale is required
    mlp = lambda m, h, i: lib.fd_post_attn_mlp_fp8(0x300000, 0x200000, 0x100000, FAKE, 0, FAKE, FAKE, FAKE,  # noqa: E731
                                                   FAKE, m, h, i, 1e-6, 0, None)
    assert mlp(17, 64, 128) == L.FD_EINVAL
    assert mlp(2, 72, 128) == L.FD_EUNSUPPORTED
    assert mlp(0, 64, 128) == L.FD_OK

    def qkv(m=2, h=64, rope_cols=64, head_dim=32, scale=FAKE, normed=None):
        return lib.fd_pre_attn_qkv_fp8(FAKE, normed, FAKE, FAKE, 0, FAKE, scale, None, 0, FAKE, FAKE, 2, 0,
                                       m, h, 96, rope_cols, head_dim, 1e-6, 0, None)

    assert qkv(m=17) == L.FD_EINVAL
    assert qkv(scale=None) == L.FD_EINVAL                  # scale is required
    assert qkv(h=72) == L.FD_EUNSUPPORTED                  # H % 16
    assert qkv(head_dim=24, rope_cols=48) == L.FD_EUNSUPPORTED
    assert qkv(rope_cols=48) == L.FD_EINVAL                # not a multiple of head_dim
    # the MFMA form (from 5 rows) folds the norm in: a null `normed` passes the
    # checks (without a GPU only the launch fails)
    assert qkv(m=5) not in (L.FD_EINVAL, L.FD_EUNSUPPORTED)
    assert qkv(m=0) == L.FD_OK


@nogpu
def test_mlp_rejects_overlapping_buffers(L):
    """y, mid and hidden of the MLP entry points must not share memory: from 5
    rows y first holds the normalised rows while hidden is still to be added."""
    lib = L.lib()
    m, h, i = 8, 64, 128
    hid = 0x100000
    mid = 0x200000
    y_ok = 0x300000

    def mlp(y, mid_p, kind=0):
        return lib.fd_post_attn_mlp(y, mid_p, hid, FAKE, 0, FAKE, FAKE, m, h, i, 1e-6, kind, 0, None)

    def mlp8(y, mid_p):
        return lib.fd_post_attn_mlp_fp8(y, mid_p, hid, FAKE, 0, FAKE, FAKE, FAKE, FAKE, m, h, i, 1e-6, 0, None)

    for call in (mlp, mlp8):
        assert call(hid, mid) == L.FD_EINVAL and b"hidden" in lib.fd_last_error()
        assert call(hid + 2 * h, mid) == L.FD_EINVAL          # y starts inside hidden's rows
        assert call(y_ok, hid + 16) == L.FD_EINVAL and b"mid" in lib.fd_last_error()
        assert call(y_ok, y_ok) == L.FD_EINVAL


def _header_signatures() -> dict[str, str]:
    """Argument codes of every entry point the header declares (p pointer, s stream,
    i int, l int64_t, f float, r fd_rows*, t fd_tile*)."""
    sigs = {}
    for m in re.finditer(r"^(?:int|const char\*)\s+(fd_\w+)\(([^;]*?)\);", HEADER.read_text(), re.M | re.S):
        codes = []
        for p in (q.strip() for q in m.group(2).replace("\n", " ").split(",")):
            if not p or p == "void":
                continue
            if "fd_rows*" in p:
                codes.append("r")
            elif "fd_tile*" in p:
                codes.append("t")
            elif p.startswith("void* stream"):
                codes.append("s")
            elif "*" in p:
                codes.append("p")
            else:
                codes.append({"int64_t": "l", "int": "i", "float": "f"}[p.split()[0]])
        sigs[m.group(1)] = "".join(codes)
    return sigs


def test_python_binding_matches_the_header():
    """fdcall.c converts each entry point's arguments by a code string: it must
    match the declaration in include/fused_decode.h argument for argument."""
    src = (ROOT / "fused-decode_amd" / "csrc" / "fdcall.c").read_text()
    sigs = _header_signatures()
    wrapped = dict(re.findall(r'WRAP\((\w+), "(\w+)"', src))
    assert wrapped, "no wrappers found"
    for name, fmt in wrapped.items():
        assert sigs["fd_" + name] == fmt, name


def test_ctypes_signatures_match_the_header(L):
    """Every ctypes argtypes list has the header's argument count and kinds."""
    import ctypes

    kinds = {ctypes.c_void_p: "p", ctypes.c_int: "i", ctypes.c_int64: "l", ctypes.c_float: "f"}
    for name, fmt in _header_signatures().items():
        if name not in L.SIGNATURES:
            continue
        got = "".join(kinds.get(t, "r" if "FdRows" in str(t) else "t" if "FdTile" in str(t) else "p")
                      for t in L.SIGNATURES[name])
        assert got == fmt.replace("s", "p"), name


@nogpu
def test_sumsq_entry_points_reject(L):
    """The row-sum handoff runs on the MFMA kernels only (kind=dot, 5..16 rows),
    with ceil(H/16) tiles and 16-byte aligned sums; every check returns before a
    launch."""
    lib = L.lib()
    F, ss = FAKE, 0x4000
    lin = lambda m, kind, out: lib.fd_linear_sumsq(F, F, F, None, 0, None, 0, m, 64, 64, 64, 1, 64, 1, 0, 0,  # noqa: E731
                                                   0, 64, 1, kind, 0, out, None)
    assert lin(4, 0, ss) == L.FD_EUNSUPPORTED and b"MFMA" in lib.fd_last_error()
    assert lin(8, 1, ss) == L.FD_EUNSUPPORTED
    assert lin(8, 0, None) == L.FD_EINVAL
    assert lin(8, 0, ss + 8) == L.FD_EUNSUPPORTED
    mlp = lambda m, tiles, sin, sout: lib.fd_post_attn_mlp_sumsq(  # noqa: E731
        F, 0x10000, 0x20000, F, 0, F, F, m, 256, 512, 1e-5, 0, 0, sin, tiles, sout, None)
    assert mlp(4, 16, ss, None) == L.FD_EUNSUPPORTED
    assert mlp(8, 15, ss, None) == L.FD_EINVAL and b"ss_tiles" in lib.fd_last_error()
    assert mlp(8, 16, ss + 4, None) == L.FD_EUNSUPPORTED
    assert mlp(8, 16, ss, ss + 4) == L.FD_EUNSUPPORTED
    qkv = lambda m, sin, tiles: lib.fd_pre_attn_qkv_sumsq(  # noqa: E731
        F, F, F, 0, F, None, 0, F, F, 2, 0, m, 256, 256, 128, 64, 1e-5, 0, 0, sin, tiles, None)
    assert qkv(8, None, 16) == L.FD_EINVAL
    assert qkv(3, ss, 16) == L.FD_EUNSUPPORTED
    assert qkv(8, ss, 17) == L.FD_EINVAL
    assert lib.fd_linear_fp8_sumsq(F, F, F, F, None, 0, None, 0, 2, 64, 64, 64, 64, 0, 0, 0, 64, 1, 0, ss,
                                   None) == L.FD_EUNSUPPORTED
    assert lib.fd_post_attn_mlp_fp8_sumsq(F, 0x10000, 0x20000, F, 0, F, F, F, F, 8, 256, 512, 1e-5, 0, ss, 3,
                                          None, None) == L.FD_EINVAL
    assert lib.fd_pre_attn_qkv_fp8_sumsq(F, F, F, 0, F, F, None, 0, F, F, 2, 0, 4, 256, 256, 128, 64, 1e-5, 0,
                                         ss, 16, None) == L.FD_EUNSUPPORTED
