"""The bandwidth roofs every "% of copy roof" figure divides by: fd_copy must
copy exactly the bytes it is given (vector path for 16-byte aligned sizes and
pointers, byte path otherwise) and touch nothing past them; fd_triad must
compute c = a + b * scale in float32 with one rounding to the element type;
fd_read must read every word it is given (its flag follows the xor of each
wave's words) and nothing past them.
The launchers of the reference's kernels.py:833-858 (launch_copy,
launch_triad) are exercised through the same calls."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module")
def L():
    import fused_decode._lib as lib

    lib.lib()  # raises if the HIP library is missing
    return lib


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


@pytest.mark.parametrize("nbytes", [1, 15, 16, 17, 4096, 4096 + 48, (1 << 20) + 3, 64 << 20])
@pytest.mark.parametrize("src_off", [0, 1])
def test_copy_is_exact_and_stays_in_bounds(L, nbytes, src_off):
    g = torch.Generator(device=DEV).manual_seed(nbytes)
    src = torch.randint(0, 256, (nbytes + 64,), generator=g, device=DEV, dtype=torch.uint8)
    dst = torch.full((nbytes + 64,), 0xA5, device=DEV, dtype=torch.uint8)
    s = src[src_off: src_off + nbytes]
    L.check("fd_copy", L.lib().fd_copy(dst.data_ptr(), s.data_ptr(), nbytes, _stream()))
    torch.cuda.synchronize()
    assert torch.equal(dst[:nbytes], s)
    assert bool((dst[nbytes:] == 0xA5).all())  # nothing written past the copy


@pytest.mark.parametrize("nbytes", [16, 4096 + 48, (1 << 20) + 32, 64 << 20])
@pytest.mark.parametrize("workgroups", [1, 7, 2048])
def test_persistent_copy_is_exact_and_stays_in_bounds(L, nbytes, workgroups):
    """fd_copy_persistent: grids smaller than the data (several grid-stride
    passes) and larger (idle workgroups), guard bytes past the end untouched."""
    print(f"[roof] persistent copy {nbytes} bytes, {workgroups} workgroups", flush=True)
    g = torch.Generator(device=DEV).manual_seed(nbytes + workgroups)
    src = torch.randint(0, 256, (nbytes + 64,), generator=g, device=DEV, dtype=torch.uint8)
    dst = torch.full((nbytes + 64,), 0xA5, device=DEV, dtype=torch.uint8)
    L.check("fd_copy_persistent", L.lib().fd_copy_persistent(dst.data_ptr(), src.data_ptr(), nbytes, workgroups,
                                                             _stream()))
    torch.cuda.synchronize()
    assert torch.equal(dst[:nbytes], src[:nbytes])
    assert bool((dst[nbytes:] == 0xA5).all())


def test_launch_copy_wrapper(L):
    from fused_decode.kernels import launch_copy

    src = torch.randn(3, 1000, device=DEV, dtype=torch.float16)
    dst = torch.empty_like(src)
    launch_copy(dst, src)
    torch.cuda.synchronize()
    assert torch.equal(dst, src)
    with pytest.raises(ValueError, match="byte"):
        launch_copy(dst[:2], src)


def _triad_expected(a: torch.Tensor, b: torch.Tensor, scale: float) -> torch.Tensor:
    """a + b*scale from the stored values, in float64, rounded once to the dtype."""
    return (a.double().cpu() + b.double().cpu() * scale).to(a.dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("n", [1, 7, 8, 1000, (1 << 20) + 5])
@pytest.mark.parametrize("off", [0, 1])
def test_triad_matches_a_plus_b_scale(L, dtype, n, off):
    g = torch.Generator(device=DEV).manual_seed(n + off)
    a = torch.randn(n + off, generator=g, device=DEV, dtype=torch.float32).to(dtype)[off:]
    b = torch.randn(n + off, generator=g, device=DEV, dtype=torch.float32).to(dtype)[off:]
    c = torch.full((n + off + 8,), 7.0, device=DEV, dtype=dtype)
    cv = c[off: off + n]
    code = L.DTYPE_CODE[dtype]
    L.check("fd_triad", L.lib().fd_triad(cv.data_ptr(), a.data_ptr(), b.data_ptr(), 1.25, n, code,
                                         _stream()))
    torch.cuda.synchronize()
    # float32 math (the product may be fused into an FMA), then one rounding:
    # within one unit in the last place of the stored type
    rtol = {torch.float16: 1e-3, torch.bfloat16: 8e-3, torch.float32: 2.4e-7}[dtype]
    torch.testing.assert_close(cv.cpu(), _triad_expected(a, b, 1.25), rtol=rtol, atol=1e-6)
    assert bool((c[off + n:] == 7.0).all())
    if off:
        assert float(c[0]) == 7.0


def test_launch_triad_wrapper(L):
    from fused_decode.kernels import launch_triad

    a = torch.randn(4096, device=DEV, dtype=torch.bfloat16)
    b = torch.randn(4096, device=DEV, dtype=torch.bfloat16)
    c = torch.empty_like(a)
    launch_triad(a, b, c, -0.5)
    torch.cuda.synchronize()
    torch.testing.assert_close(c.cpu(), _triad_expected(a, b, -0.5), rtol=8e-3, atol=1e-6)


def _wave_xors(words: torch.Tensor) -> list[int]:
    """The xor of the 32-bit words each wave of fd_read's kernel reads: wave w of
    block b takes 16-byte vectors b*1024 + 64w + j + 256i (j < 64, i < 4)."""
    nvec = words.numel() // 4
    vec = words.view(nvec, 4).cpu().numpy().astype("uint32")
    out = []
    blocks = (nvec + 1023) // 1024
    for b in range(blocks):
        for w in range(4):
            acc = 0
            for i in range(4):
                lo = b * 1024 + 256 * i + 64 * w
                for row in vec[lo: min(lo + 64, nvec)]:
                    for x in row:
                        acc ^= int(x)
            out.append(acc)
    return out


@pytest.mark.parametrize("nvec", [1, 64, 1024, 1024 + 320, 5000])
def test_read_flags_exactly_the_matching_wave(L, nvec):
    g = torch.Generator().manual_seed(nvec)
    words = torch.zeros(nvec * 4 + 64, dtype=torch.int32)  # 64 trailing words, never read
    words[nvec * 4:] = 0x5A5A5A5A
    pos = int(torch.randint(0, nvec * 4, (1,), generator=g))
    words[pos] = 0x1234567
    src = words.to(DEV)
    xors = _wave_xors(words[: nvec * 4])
    hit = torch.zeros(1, dtype=torch.int32, device=DEV)
    for key, expect in ((0x1234567, 1), (0x7777777, 0), (0x5A5A5A5A, 0)):
        hit.zero_()
        L.check("fd_read", L.lib().fd_read(src.data_ptr(), nvec * 16, key, hit.data_ptr(), _stream()))
        torch.cuda.synchronize()
        assert int(hit.item()) == expect, (key, expect)
        assert (key in xors) == bool(expect)  # the model of the waves agrees
    # all-zero data: every wave's xor is 0
    zero = torch.zeros(nvec * 4, dtype=torch.int32, device=DEV)
    hit.zero_()
    L.check("fd_read", L.lib().fd_read(zero.data_ptr(), nvec * 16, 0, hit.data_ptr(), _stream()))
    torch.cuda.synchronize()
    assert int(hit.item()) == 1


def test_read_launcher(L):
    from fused_decode.kernels import launch_read

    src = torch.zeros(1 << 16, dtype=torch.float16, device=DEV)
    hit = torch.zeros(1, dtype=torch.int32, device=DEV)
    launch_read(src, hit, key=0)
    torch.cuda.synchronize()
    assert int(hit.item()) == 1


def test_clock_probe_brackets_work(L):
    """Two clock probes (4096 workgroups, so every CU is seen by both) around a
    1 GiB copy: the wall span of every CU is no shorter than the copy the events
    timed, and each XCD's median counter rate (its CUs' shader-counter advance
    per wall-clock tick) is positive and within 30% of every other XCD's."""
    from fused_decode.decode_step import counter_rates
    from fused_decode.kernels import clock_probe, launch_copy

    print("[roof] clock probe around a 1 GiB copy", flush=True)
    src = torch.ones(1 << 30, dtype=torch.uint8, device=DEV)
    dst = torch.empty_like(src)
    pa = torch.zeros(4096, 3, dtype=torch.int64, device=DEV)
    pb = torch.zeros_like(pa)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    khz = clock_probe(pa)
    start.record()
    launch_copy(dst, src)
    end.record()
    clock_probe(pb)
    torch.cuda.synchronize()
    copy_us = start.elapsed_time(end) * 1000.0
    assert khz > 0
    a, b = pa.cpu().tolist(), pb.cpu().tolist()
    wall_first = {}
    for key, _, w in a:
        wall_first.setdefault(key, w)
    for key, _, w in b:
        if key in wall_first:
            assert (w - wall_first[key]) / khz * 1000.0 >= 0.9 * copy_us
    rates = counter_rates(a, b)
    print(f"[roof] counter rate per XCD {rates}, wall {khz} kHz, copy {copy_us:.1f} us", flush=True)
    assert len(rates) >= 1
    assert min(rates.values()) > 0 and max(rates.values()) <= 1.3 * min(rates.values())
