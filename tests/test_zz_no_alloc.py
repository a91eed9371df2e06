"""fd_post_attn_mlp_noalloc, the MLP entry point that allocates nothing (its
`mid` rows live in a library-owned device array), against fd_post_attn_mlp
with a caller-owned `mid`: the same kernels, so the outputs must be identical,
and both within the GEMV tolerance of the oracle (fp16 rtol=atol=2e-2, the
reference's tests/test_ops.py:27-35). Two calls in a row, the second smaller,
since every call on a GPU reuses that GPU's array; then a graph capture, and a
fresh process whose very first call is made under capture."""

from __future__ import annotations

import subprocess
import sys
import textwrap
from pathlib import Path

import pytest
import torch

from oracle import decode_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module")
def L():
    import fused_decode._lib as lib

    lib.lib()  # raises if the HIP library is missing
    return lib


def _case(m, h, i, seed, dtype=torch.float16):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s, scale=1.0, mean=0.0: (torch.randn(*s, generator=g) * scale + mean).to(dtype)  # noqa: E731
    return r(m, h), r(h, scale=0.1, mean=1.0), r(2 * i, h, scale=h ** -0.5), r(h, i, scale=i ** -0.5)


def _run_both(L, m, h, i, kind, seed, dtype=torch.float16):
    hidden, nw, wgu, wd = _case(m, h, i, seed, dtype)
    hd, nwd, wgud, wdd = (t.to(DEV) for t in (hidden, nw, wgu, wd))
    code = L.DTYPE_CODE[dtype]
    st = torch.cuda.current_stream().cuda_stream
    y_ref = torch.empty(m, h, device=DEV, dtype=dtype)
    mid = torch.empty(m, i, device=DEV, dtype=dtype)
    L.check("fd_post_attn_mlp", L.lib().fd_post_attn_mlp(
        y_ref.data_ptr(), mid.data_ptr(), hd.data_ptr(), nwd.data_ptr(), code, wgud.data_ptr(),
        wdd.data_ptr(), m, h, i, 1e-5, kind, code, st))
    y = torch.full((m, h), float("nan"), device=DEV, dtype=dtype)
    L.check("fd_post_attn_mlp_noalloc", L.lib().fd_post_attn_mlp_noalloc(
        y.data_ptr(), hd.data_ptr(), nwd.data_ptr(), code, wgud.data_ptr(), wdd.data_ptr(),
        m, h, i, 1e-5, kind, code, st))
    torch.cuda.synchronize()
    f = lambda t: t.float().numpy()  # noqa: E731
    ref = O.post_attn_mlp(f(hidden), f(nw), f(wgu), f(wd), 1e-5, "f16" if dtype == torch.float16 else "bf16")
    return y, y_ref, ref, (hd, nwd, wgud, wdd)


def test_noalloc_matches_the_allocating_entry_point(L):
    # first call: 16 rows on the MFMA route (kind dot), 256 KiB of the scratch
    print("[noalloc] m=16 h=1024 i=8192 dot", flush=True)
    y, y_ref, ref, _ = _run_both(L, 16, 1024, 8192, L.FD_KIND_DOT, seed=1)
    torch.testing.assert_close(y, y_ref, rtol=0, atol=0)
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), rtol=2e-2, atol=2e-2)
    # second call, smaller: 3 rows on the fused SIMT route, over the first call's contents
    print("[noalloc] m=3 h=256 i=512 simt", flush=True)
    y, y_ref, ref, _ = _run_both(L, 3, 256, 512, L.FD_KIND_SIMT, seed=2)
    torch.testing.assert_close(y, y_ref, rtol=0, atol=0)
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), rtol=2e-2, atol=2e-2)


def test_noalloc_bfloat16(L):
    """bfloat16 activations and weights, two calls in a row (8 rows on the MFMA
    route, then 2 rows on the SIMT route), against the allocating entry point;
    oracle tolerance for bfloat16 GEMVs rtol=atol=4e-2 (tests/test_ops.py:27-35)."""
    print("[noalloc] bf16 m=8 h=512 i=2048 dot", flush=True)
    y, y_ref, ref, _ = _run_both(L, 8, 512, 2048, L.FD_KIND_DOT, seed=4, dtype=torch.bfloat16)
    torch.testing.assert_close(y, y_ref, rtol=0, atol=0)
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), rtol=4e-2, atol=4e-2)
    print("[noalloc] bf16 m=2 h=256 i=384 simt", flush=True)
    y, y_ref, ref, _ = _run_both(L, 2, 256, 384, L.FD_KIND_SIMT, seed=5, dtype=torch.bfloat16)
    torch.testing.assert_close(y, y_ref, rtol=0, atol=0)
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), rtol=4e-2, atol=4e-2)


def test_noalloc_llama3_8b_widths_and_graph_capture(L):
    """Llama-3-8B widths at M = 8 (229,376 bytes of scratch), eagerly and replayed
    from a HIP graph, against the allocating entry point."""
    print("[noalloc] m=8 h=4096 i=14336 dot, graph", flush=True)
    m, h, i = 8, 4096, 14336
    y, y_ref, ref, (hd, nwd, wgud, wdd) = _run_both(L, m, h, i, L.FD_KIND_DOT, seed=3)
    torch.testing.assert_close(y, y_ref, rtol=0, atol=0)
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(ref), rtol=2e-2, atol=2e-2)
    out = torch.empty(m, h, device=DEV, dtype=torch.float16)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        L.check("fd_post_attn_mlp_noalloc", L.lib().fd_post_attn_mlp_noalloc(
            out.data_ptr(), hd.data_ptr(), nwd.data_ptr(), L.FD_F16, wgud.data_ptr(), wdd.data_ptr(),
            m, h, i, 1e-5, L.FD_KIND_DOT, L.FD_F16, side.cuda_stream))
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        torch.testing.assert_close(out, y_ref, rtol=0, atol=0)
        _ = (hd.float() * 2).sum().item()  # unrelated eager work between replays


# A fresh process whose first fd_post_attn_mlp_noalloc call is inside a graph
# capture: the library's set-up (fd_init, run by the loader) has resolved the
# array's address before the capture, so the captured call performs no lookup.
_FIRST_CALL_CAPTURED = textwrap.dedent("""
    import sys
    sys.path[:0] = [{root!r}, {pkg!r}]
    import torch
    import fused_decode._lib as L

    L.lib()  # loads the library; its set-up runs here, outside any capture
    m, h, i = 8, 512, 2048
    g = torch.Generator().manual_seed(7)
    r = lambda *s, scale=1.0, mean=0.0: (torch.randn(*s, generator=g) * scale + mean).half().cuda()
    hid, nw, wgu, wd = r(m, h), r(h, scale=0.1, mean=1.0), r(2 * i, h, scale=h ** -0.5), r(h, i, scale=i ** -0.5)
    out = torch.zeros(m, h, device="cuda", dtype=torch.float16)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    print("[noalloc subprocess] capturing the first call", flush=True)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        L.check("fd_post_attn_mlp_noalloc", L.lib().fd_post_attn_mlp_noalloc(
            out.data_ptr(), hid.data_ptr(), nw.data_ptr(), L.FD_F16, wgu.data_ptr(), wd.data_ptr(),
            m, h, i, 1e-5, L.FD_KIND_DOT, L.FD_F16, side.cuda_stream))
    y_ref = torch.empty(m, h, device="cuda", dtype=torch.float16)
    mid = torch.empty(m, i, device="cuda", dtype=torch.float16)
    L.check("fd_post_attn_mlp", L.lib().fd_post_attn_mlp(
        y_ref.data_ptr(), mid.data_ptr(), hid.data_ptr(), nw.data_ptr(), L.FD_F16, wgu.data_ptr(),
        wd.data_ptr(), m, h, i, 1e-5, L.FD_KIND_DOT, L.FD_F16, torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    for rep in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, y_ref), f"replay {{rep}} differs from fd_post_attn_mlp"
        _ = (hid.float() * 2).sum().item()  # unrelated eager work between replays
    print("[noalloc subprocess] ok", flush=True)
""")


def test_noalloc_first_call_under_capture_in_a_fresh_process():
    root = Path(__file__).resolve().parents[1]
    code = _FIRST_CALL_CAPTURED.format(root=str(root), pkg=str(root / "fused-decode_amd"))
    print("[noalloc] fresh process, first call captured, m=8 h=512 i=2048", flush=True)
    proc = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=110)
    print(proc.stdout[-2000:], proc.stderr[-2000:], flush=True)
    assert proc.returncode == 0 and "[noalloc subprocess] ok" in proc.stdout


def test_noalloc_rejects_sizes_beyond_the_scratch(L):
    st = torch.cuda.current_stream().cuda_stream
    # 16 rows x 40,000 x 2 bytes = 1,280,000 > 1 MiB: rejected before any launch
    assert L.lib().fd_post_attn_mlp_noalloc(0x1000, 0x2000, 0x3000, L.FD_F16, 0x4000, 0x5000,
                                            16, 4096, 40000, 1e-5, L.FD_KIND_DOT, L.FD_F16, st) == L.FD_EINVAL
    assert b"scratch" in L.lib().fd_last_error()
    assert L.lib().fd_post_attn_mlp_noalloc(0x1000, 0x2000, 0x3000, L.FD_F16, 0x4000, 0x5000,
                                            17, 64, 64, 1e-5, L.FD_KIND_DOT, L.FD_F16, st) == L.FD_EINVAL
    assert L.lib().fd_post_attn_mlp_noalloc(0x1000, 0x2000, 0x3000, L.FD_F16, 0x4000, 0x5000,
                                            0, 64, 64, 1e-5, L.FD_KIND_DOT, L.FD_F16, st) == L.FD_OK
