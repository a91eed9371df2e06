"""Bindings of libfused_decode_hip.so (the C ABI in include/fused_decode.h).

Two bindings of the same library: ``native()`` is the CPython extension
``_fdcall`` (csrc/fdcall.c) that the operators launch through, a few tens of
nanoseconds per argument; ``lib()`` is a ctypes handle with every entry
point's argument types declared, for tests and tools that call the C ABI the
way a foreign host would. Both load the one shared library, after torch, so
its dependency on ``libamdhip64.so.7`` resolves to the HIP runtime torch
already loaded: streams and graph captures are shared with torch. There is no
fallback: if the library or the binding is missing, every operator raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (loads torch's HIP runtime before ours)

LIB_NAME = "libfused_decode_hip.so"
LIB_PATH = Path(os.environ.get("FUSED_DECODE_LIB", Path(__file__).with_name(LIB_NAME)))

FD_F16, FD_BF16, FD_F32 = 0, 1, 2
FD_KIND_DOT, FD_KIND_SIMT = 0, 1
FD_OK, FD_EINVAL, FD_EUNSUPPORTED, FD_ELAUNCH = 0, 1, 2, 3

DTYPE_CODE = {torch.float16: FD_F16, torch.bfloat16: FD_BF16, torch.float32: FD_F32}
KIND_CODE = {"dot": FD_KIND_DOT, "simt": FD_KIND_SIMT}


class FdTile(ctypes.Structure):
    """``fd_tile``: weight rows per workgroup, waves per workgroup, MFMA K units in
    flight per wave (0 = the library default for that field)."""

    _fields_ = [("rows", ctypes.c_int), ("waves", ctypes.c_int), ("stages", ctypes.c_int)]


class FdRows(ctypes.Structure):
    """``fd_rows``: a*b*c rows of n elements; row (i,j,l) at i*sa+j*sb+l*sc."""

    _fields_ = [
        ("a", ctypes.c_int64),
        ("b", ctypes.c_int64),
        ("c", ctypes.c_int64),
        ("sa", ctypes.c_int64),
        ("sb", ctypes.c_int64),
        ("sc", ctypes.c_int64),
        ("col", ctypes.c_int64),
        ("n", ctypes.c_int64),
    ]


_p = ctypes.c_void_p
_i = ctypes.c_int
_l = ctypes.c_int64
_f = ctypes.c_float
_rows = ctypes.POINTER(FdRows)

# name -> argument types; every entry point returns an int status.
SIGNATURES: dict[str, list] = {
    "fd_version": [],
    "fd_init": [],
    "fd_runtime_version": [ctypes.POINTER(ctypes.c_int)],
    "fd_rms_norm": [_p, _p, _p, _i, _l, _rows, _rows, _f, _i, _p],
    "fd_add_rms_norm": [_p, _p, _p, _p, _p, _i, _l, _rows, _rows, _rows, _rows, _f, _i, _p],
    "fd_swiglu": [_p, _p, _p, _rows, _rows, _rows, _i, _p],
    "fd_rope": [_p, _p, _p, _p, _i, _rows, _rows, _rows, _rows, _i, _p],
    "fd_linear": [_p, _p, _p, _p, _i, _p, _i, _l, _l, _l, _l, _l, _l, _l, _l, _l, _l, _l, _l, _i, _i, _p],
    "fd_linear_fp8": [_p, _p, _p, _p, _p, _i, _p, _i, _l, _l, _l, _l, _l, _l, _l, _l, _l, _l, _i, _p],
    "fd_post_attn_mlp_fp8": [_p, _p, _p, _p, _i, _p, _p, _p, _p, _l, _l, _l, _f, _i, _p],
    "fd_linear_tiled": [_p, _p, _p, _p, _i, _p, _i, _l, _l, _l, _l, _l, _l, _l, _l, _l, _l, _l, _l,
                        ctypes.POINTER(FdTile), _i, _i, _p],
    "fd_post_attn_mlp": [_p, _p, _p, _p, _i, _p, _p, _l, _l, _l, _f, _i, _i, _p],
    "fd_post_attn_mlp_noalloc": [_p, _p, _p, _i, _p, _p, _l, _l, _l, _f, _i, _i, _p],
    "fd_mlp_gate_up": [_p, _p, _p, _p, _i, _p, _l, _l, _l, _f, _i, _i, _p],
    "fd_pre_attn_qkv": [_p, _p, _p, _p, _i, _p, _p, _i, _p, _p, _i, _l, _l, _l, _l, _l, _l, _f, _i,
                        _i, _p],
    "fd_pre_attn_qkv_fp8": [_p, _p, _p, _p, _i, _p, _p, _p, _i, _p, _p, _i, _l, _l, _l, _l, _l,
                            _l, _f, _i, _p],
    "fd_linear_sumsq": [_p, _p, _p, _p, _i, _p, _i, _l, _l, _l, _l, _l, _l, _l, _l, _l, _l, _l, _l, _i, _i,
                        _p, _p],
    "fd_post_attn_mlp_sumsq": [_p, _p, _p, _p, _i, _p, _p, _l, _l, _l, _f, _i, _i, _p, _l, _p, _p],
    "fd_pre_attn_qkv_sumsq": [_p, _p, _p, _i, _p, _p, _i, _p, _p, _i, _l, _l, _l, _l, _l, _l, _f, _i, _i, _p,
                              _l, _p],
    "fd_linear_fp8_sumsq": [_p, _p, _p, _p, _p, _i, _p, _i, _l, _l, _l, _l, _l, _l, _l, _l, _l, _l, _i, _p, _p],
    "fd_post_attn_mlp_fp8_sumsq": [_p, _p, _p, _p, _i, _p, _p, _p, _p, _l, _l, _l, _f, _i, _p, _l, _p, _p],
    "fd_pre_attn_qkv_fp8_sumsq": [_p, _p, _p, _i, _p, _p, _p, _i, _p, _p, _i, _l, _l, _l, _l, _l, _l, _f, _i,
                                  _p, _l, _p],
    "fd_copy": [_p, _p, _l, _p],
    "fd_copy_persistent": [_p, _p, _l, _i, _p],
    "fd_clock_probe": [_p, _i, ctypes.POINTER(ctypes.c_int), _p],
    "fd_triad": [_p, _p, _p, _f, _l, _i, _p],
    "fd_read": [_p, _l, _i, _p, _p],
}

_LIB: ctypes.CDLL | None = None


class FusedDecodeError(RuntimeError):
    """A non-OK status from the HIP library."""

    def __init__(self, func: str, status: int, message: str):
        super().__init__(f"{func} failed (status {status}): {message}")
        self.status = status


def lib() -> ctypes.CDLL:
    """Load the library once; raise if it has not been built."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is not built: run `python fused-decode_amd/build.py` "
                "(or __graft_entry__.build()) first"
            )
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_int
        handle.fd_last_error.argtypes = []
        handle.fd_last_error.restype = ctypes.c_char_p
        _LIB = handle
        _init()
    return _LIB


_INITIALISED = False


def _init() -> None:
    """fd_init once per process where a GPU is visible (the library's per-device
    set-up, done before any caller can be capturing a graph)."""
    global _INITIALISED
    if _INITIALISED or not torch.cuda.is_available():
        return
    _INITIALISED = True
    check("fd_init", lib().fd_init())


def check(func: str, status: int) -> None:
    if status != FD_OK:
        msg = lib().fd_last_error().decode(errors="replace")
        raise FusedDecodeError(func, status, msg)


_NATIVE = None


def native():
    """The ``_fdcall`` extension, bound to the library (loaded once)."""
    global _NATIVE
    if _NATIVE is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is not built: run `python fused-decode_amd/build.py` "
                "(or __graft_entry__.build()) first"
            )
        try:
            from . import _fdcall
        except ImportError as exc:
            raise RuntimeError(
                "the Python binding fused_decode._fdcall is not built: run "
                "`python fused-decode_amd/build.py` (or __graft_entry__.build()) first"
            ) from exc
        _fdcall.bind(str(LIB_PATH))
        _NATIVE = _fdcall
        _init()
    return _NATIVE


def fail(func: str, status: int) -> None:
    """Raise the library's error for a non-OK ``status`` of ``func``."""
    raise FusedDecodeError(func, status, native().last_error())


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t: torch.Tensor) -> int:
    """Handle of torch's current stream on the tensor's device."""
    if _raw_stream is not None:
        return _raw_stream(t.device.index if t.device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(t.device).cuda_stream


def stream_of_device(index: int) -> int:
    """Handle of torch's current stream on device ``index``."""
    return torch.cuda.current_stream(index).cuda_stream


def runtime_version() -> int:
    v = ctypes.c_int(0)
    check("fd_runtime_version", lib().fd_runtime_version(ctypes.byref(v)))
    return v.value
