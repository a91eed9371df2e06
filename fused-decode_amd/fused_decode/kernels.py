"""Launchers: Python-side calls into the gfx950 HIP library.

Same launcher boundary as the reference's src/fused_decode/kernels.py
(``rms_out``, ``swiglu_out``, ``rope_out``, ``linear_out``, ``resolve_kind``,
``linear_config``, ``launch_copy``, ``launch_triad``), but every launch goes
through the C ABI of libfused_decode_hip.so (its ``_fdcall`` binding) on
torch's current stream. The launchers write into caller-provided tensors and
never synchronise, so they can be captured into a HIP graph. They plan row
layouts on every call; the public operators (``ops``) cache that planning per
argument signature and call the binding directly.
"""

from __future__ import annotations

import json
import os
import warnings

import torch

from . import _lib
from ._layout import finish, joint_layout
from ._lib import DTYPE_CODE, KIND_CODE, FdTile, fail, native, stream_of

_warned: set[str] = set()


def _warn_once(key: str, msg: str) -> None:
    if key not in _warned:
        _warned.add(key)
        warnings.warn(msg, RuntimeWarning, stacklevel=3)


def _rms_env() -> None:
    """The reference's Triton tile knobs (kernels.py:91-108) have no meaning for
    the HIP kernels. FUSED_DECODE_RMS_BLOCK keeps its power-of-two validation;
    both are otherwise ignored with a one-time warning."""
    block = os.environ.get("FUSED_DECODE_RMS_BLOCK")
    if block:
        b = int(block)
        if b & (b - 1):
            raise ValueError("FUSED_DECODE_RMS_BLOCK must be a power of 2")
        _warn_once("rms_block", "FUSED_DECODE_RMS_BLOCK is a Triton tile knob; the HIP RMSNorm ignores it")
    if os.environ.get("FUSED_DECODE_RMS_WARPS"):
        _warn_once("rms_warps", "FUSED_DECODE_RMS_WARPS is a Triton knob; the HIP RMSNorm ignores it")


def rms_out(
    x: torch.Tensor,
    weight: torch.Tensor,
    eps: float,
    out: torch.Tensor,
    residual: torch.Tensor | None = None,
    residual_out: torch.Tensor | None = None,
) -> None:
    """RMSNorm (and fused residual add) into ``out``; mirrors kernels.py:343-414."""
    _rms_env()
    add = residual is not None
    if add and residual_out is None:
        raise ValueError("residual requires residual_out")
    ins = [x, residual] if add else [x]
    outs = [out, residual_out] if add else [out]
    for t, what in zip(ins[1:] + outs, (["residual"] if add else []) + ["out"] + (["residual_out"] if add else [])):
        if tuple(t.shape) != tuple(x.shape):
            raise ValueError(f"{what} cannot be indexed with the same row grid as the input")
    if x.numel() == 0:
        return
    li, lo = joint_layout(ins, outs)
    act = DTYPE_CODE[x.dtype]
    w_code = DTYPE_CODE[weight.dtype]
    st = stream_of(x)
    rows = [bytes(op.rows) for op in li + lo]
    if add:
        status = native().add_rms_norm(
            lo[0].tensor.data_ptr(), lo[1].tensor.data_ptr(), li[0].tensor.data_ptr(),
            li[1].tensor.data_ptr(), weight.data_ptr(), w_code, int(weight.stride(0)),
            rows[0], rows[1], rows[2], rows[3], float(eps), act, st,
        )
        if status:
            fail("fd_add_rms_norm", status)
    else:
        status = native().rms_norm(
            lo[0].tensor.data_ptr(), li[0].tensor.data_ptr(), weight.data_ptr(), w_code,
            int(weight.stride(0)), rows[0], rows[1], float(eps), act, st,
        )
        if status:
            fail("fd_rms_norm", status)
    finish(lo)


def swiglu_out(gate: torch.Tensor, up: torch.Tensor, out: torch.Tensor) -> None:
    """``out = silu(gate) * up``; mirrors kernels.py:456-487."""
    if gate.numel() == 0:
        return
    li, lo = joint_layout([gate, up], [out])
    status = native().swiglu(
        lo[0].tensor.data_ptr(), li[0].tensor.data_ptr(), li[1].tensor.data_ptr(),
        bytes(li[0].rows), bytes(li[1].rows), bytes(lo[0].rows), DTYPE_CODE[gate.dtype], stream_of(gate),
    )
    if status:
        fail("fd_swiglu", status)
    finish(lo)


def rope_out(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, out: torch.Tensor) -> None:
    """Rotate-half RoPE; ``cos``/``sin`` already expanded to ``x.shape``
    (stride-0 broadcast dims). Mirrors kernels.py:541-578."""
    if x.numel() == 0:
        return
    if cos.dtype != sin.dtype:
        # one dtype code per launch: widen both (exact for fp16/bf16 -> fp32)
        cos, sin = cos.float(), sin.float()
    li, lo = joint_layout([x, cos, sin], [out])
    status = native().rope(
        lo[0].tensor.data_ptr(), li[0].tensor.data_ptr(), li[1].tensor.data_ptr(),
        li[2].tensor.data_ptr(), DTYPE_CODE[cos.dtype], bytes(li[0].rows), bytes(li[1].rows),
        bytes(li[2].rows), bytes(lo[0].rows), DTYPE_CODE[x.dtype], stream_of(x),
    )
    if status:
        fail("fd_rope", status)
    finish(lo)


def resolve_kind(kind: str | None) -> str:
    """``kind`` or ``FUSED_DECODE_LINEAR_KIND`` (default "dot"); mirrors kernels.py:581-586."""
    if kind is None:
        kind = os.environ.get("FUSED_DECODE_LINEAR_KIND", "dot")
    if kind not in ("dot", "simt"):
        raise ValueError("kind must be 'dot' or 'simt'")
    return kind


# K elements per wave step of each GEMV kernel (a fixed property of the kernel).
_BLOCK_K = {"simt": 512, "dot": 128}
_MFMA_MIN_M = 5  # kind "dot" runs the MFMA kernel from this many rows on (kMfmaMinM in gemv.hip)
_TILE_TABLE: dict | None = None
TILE_TABLE_FILE = os.path.join(os.path.dirname(__file__), "tiles_gfx950.json")


def _tile_table() -> dict:
    """Measured tiles per (kind, N, K, M), written by ``python -m fused_decode.bench
    --tune``; empty when the file is absent."""
    global _TILE_TABLE
    if _TILE_TABLE is None:
        try:
            with open(TILE_TABLE_FILE) as f:
                _TILE_TABLE = json.load(f).get("entries", {})
        except (OSError, ValueError):
            _TILE_TABLE = {}
    return _TILE_TABLE


def _kernel_of(kind: str, m: int | None) -> str:
    """The kernel the library runs by default: MFMA ("dot") for kind "dot" from
    5 rows (or when m is None), SIMT otherwise."""
    return "dot" if kind == "dot" and (m is None or m >= _MFMA_MIN_M) else "simt"


def tile_key(kind: str, n: int, k: int, m: int) -> str:
    return f"{kind}:{n}x{k}:m{m}"


def linear_config(kind: str, n: int, k: int, m: int | None = None) -> tuple[int, int, int, int]:
    """Tiling of the HIP GEMV for ``[N, K]`` weights and ``m`` rows: (rows per
    workgroup, K elements per wave step, waves per workgroup, MFMA K units in
    flight per wave). 16 rows is the MFMA kernel (kind "dot" only), 2/4/8 the
    SIMT kernel.

    ``FUSED_DECODE_LINEAR=block_n,block_k,warps,stages`` overrides it as in the
    reference (kernels.py:589-603): block_n = rows per workgroup, block_k the
    kernel's step (SIMT 512, MFMA 128), warps = waves (SIMT 1-8, MFMA 2, 4 or
    8), stages = MFMA K units in flight per wave (1-3) or the SIMT form (0 the
    library's choice, 1 per-tile, 2 persistent, whose waves then set the K chunks
    each lane keeps). Otherwise the measured table
    (``tiles_gfx950.json``, per kind, N, K and M) decides for its shapes, and
    the library's defaults (MFMA for "dot" from 5 rows) for the rest."""
    forced = os.environ.get("FUSED_DECODE_LINEAR")
    if forced:
        try:
            block_n, block_k, warps, stages = (int(part) for part in forced.split(","))
        except ValueError as exc:
            raise ValueError("FUSED_DECODE_LINEAR must be block_n,block_k,warps,stages") from exc
        kern = "dot" if block_n == 16 else "simt"
        if kern == "dot" and kind != "dot":
            raise ValueError("FUSED_DECODE_LINEAR block_n 16 is the MFMA GEMV, which needs kind 'dot'")
        if block_k != _BLOCK_K[kern]:
            raise ValueError(f"FUSED_DECODE_LINEAR block_k must be {_BLOCK_K[kern]} for block_n {block_n}")
        return block_n, block_k, warps, stages
    if m is not None:
        hit = _tile_table().get(tile_key(kind, n, k, m))
        if hit:
            rows, waves, stages = hit
            return rows, _BLOCK_K["dot" if rows == 16 else "simt"], waves, stages
    kern = _kernel_of(kind, m)
    rows, waves, stages = default_tile(kern, n, k)
    return rows, _BLOCK_K[kern], waves, stages


def default_tile(kern: str, n: int, k: int) -> tuple[int, int, int]:
    """The library's own choice (rows, waves, stages) for a kernel ("simt" or "dot"):
    the MFMA GEMV runs four waves (two below four K units) with two units in
    flight each; for the SIMT GEMV (0, waves, 0) leaves rows and form to the
    library: the persistent kernel (stages 2; its waves set 1, 2 or 4 K chunks
    per lane) from 2 rows where its registers hold them, else the per-tile one
    (stages 1), with one wave per chunk up to eight."""
    if kern == "dot":
        return 16, (4 if -(-k // 128) >= 4 else 2), 2
    return 0, _waves(-(-k // 512)), 0


def _waves(items: int) -> int:
    """pick_waves of fd_gemv.h: one wave per work item, up to eight."""
    return max(1, min(8, items))


def linear_out(
    x: torch.Tensor,
    weight: torch.Tensor,
    y: torch.Tensor,
    *,
    bias: torch.Tensor | None = None,
    row_add: torch.Tensor | None = None,
    kind: str | None = None,
    tile: tuple[int, int, int] | None = None,
) -> None:
    """``y = x @ weight.T [+ bias] [+ row_add]`` for x ``[M, K]``, M <= 16.
    ``row_add`` is ``[M, N]``, ``[1, N]``, ``[M, 1]`` or ``[1, 1]`` (size-1 dims
    broadcast). ``tile`` = (rows, waves, stages) overrides ``linear_config``.
    Mirrors kernels.py:741-830."""
    kind = resolve_kind(kind)
    m, k = x.shape
    n, k_w = weight.shape
    if k != k_w:
        raise ValueError(f"K mismatch: x has {k}, weight has {k_w}")
    if tuple(y.shape) != (m, n):
        raise ValueError(f"y shape {tuple(y.shape)} != {(m, n)}")
    if m > 16:
        raise ValueError("linear_out only covers M <= 16")
    if m == 0 or n == 0:
        return
    if any(s < 0 for s in x.stride()):
        x = x.contiguous()
    if any(s < 0 for s in weight.stride()):
        weight = weight.contiguous()
    bias_ptr, bias_code, sb = None, DTYPE_CODE[x.dtype], 0
    if bias is not None:
        if bias.stride(0) < 0:
            bias = bias.contiguous()
        bias_ptr, bias_code, sb = bias.data_ptr(), DTYPE_CODE[bias.dtype], int(bias.stride(0))
    row_ptr, row_code, srm, srn = None, DTYPE_CODE[x.dtype], 0, 0
    if row_add is not None:
        if any(s < 0 for s in row_add.stride()):
            row_add = row_add.contiguous()
        row_ptr, row_code = row_add.data_ptr(), DTYPE_CODE[row_add.dtype]
        srm = 0 if row_add.shape[0] == 1 else int(row_add.stride(0))
        srn = 0 if row_add.shape[1] == 1 else int(row_add.stride(1))
    if tile is None:
        rows, _, waves, stages = linear_config(kind, n, k, m)
        tile = (rows, waves, stages)
    status = native().linear_tiled(
        y.data_ptr(), x.data_ptr(), weight.data_ptr(), bias_ptr, bias_code, row_ptr, row_code,
        m, n, k, int(x.stride(0)), int(x.stride(1)), int(weight.stride(0)), int(weight.stride(1)),
        sb, srm, srn, int(y.stride(0)), int(y.stride(1)), bytes(FdTile(*tile)),
        KIND_CODE[kind], DTYPE_CODE[x.dtype], stream_of(x),
    )
    if status:
        fail("fd_linear_tiled", status)


def post_attn_mlp_out(
    hidden: torch.Tensor,
    norm_weight: torch.Tensor,
    w_gate_up: torch.Tensor,
    w_down: torch.Tensor,
    eps: float,
    out: torch.Tensor,
    mid: torch.Tensor,
    kind: str,
) -> int:
    """Fused MLP for contiguous ``hidden [M, H]`` (M <= 16): two launches. ``mid``
    is ``[M, I]`` scratch. Returns the library status (FD_EUNSUPPORTED lets the
    caller fall back to the composed operators)."""
    m, h = hidden.shape
    i = w_down.shape[1]
    status = native().post_attn_mlp(
        out.data_ptr(), mid.data_ptr(), hidden.data_ptr(), norm_weight.data_ptr(),
        DTYPE_CODE[norm_weight.dtype], w_gate_up.data_ptr(), w_down.data_ptr(), m, h, i,
        float(eps), KIND_CODE[kind], DTYPE_CODE[hidden.dtype], stream_of(hidden),
    )
    if status not in (_lib.FD_OK, _lib.FD_EUNSUPPORTED):
        fail("fd_post_attn_mlp", status)
    return status


def pre_attn_qkv_out(
    hidden: torch.Tensor,
    norm_weight: torch.Tensor,
    w_qkv: torch.Tensor,
    bias: torch.Tensor | None,
    cos: torch.Tensor | None,
    sin: torch.Tensor | None,
    cs_row_stride: int,
    rope_cols: int,
    head_dim: int,
    eps: float,
    out: torch.Tensor,
    normed: torch.Tensor | None,
    kind: str,
) -> int:
    """Fused RMSNorm + QKV GEMV + RoPE for contiguous ``hidden [M, H]`` (M <= 16)
    into contiguous ``out [M, N]``; ``cos``/``sin`` are contiguous rows of
    ``head_dim`` (row stride ``cs_row_stride``, 0 = shared). ``normed`` is unused
    (the MFMA form folds the norm in) and may be None. Returns the library status (FD_EUNSUPPORTED
    lets the caller compose the operators instead)."""
    m, h = hidden.shape
    n = w_qkv.shape[0]
    status = native().pre_attn_qkv(
        out.data_ptr(), normed.data_ptr() if normed is not None else None, hidden.data_ptr(),
        norm_weight.data_ptr(), DTYPE_CODE[norm_weight.dtype], w_qkv.data_ptr(),
        bias.data_ptr() if bias is not None else None,
        DTYPE_CODE[bias.dtype] if bias is not None else DTYPE_CODE[hidden.dtype],
        cos.data_ptr() if cos is not None else None, sin.data_ptr() if sin is not None else None,
        DTYPE_CODE[cos.dtype] if cos is not None else DTYPE_CODE[torch.float32],
        cs_row_stride, m, h, n, rope_cols, head_dim, float(eps), KIND_CODE[kind],
        DTYPE_CODE[hidden.dtype], stream_of(hidden),
    )
    if status not in (_lib.FD_OK, _lib.FD_EUNSUPPORTED):
        fail("fd_pre_attn_qkv", status)
    return status


def launch_copy(dst: torch.Tensor, src: torch.Tensor) -> None:
    """Bandwidth-roof copy of ``src`` into ``dst`` (same byte size, contiguous)."""
    nbytes = src.numel() * src.element_size()
    if dst.numel() * dst.element_size() != nbytes:
        raise ValueError("copy needs equal byte sizes")
    status = native().copy(dst.data_ptr(), src.data_ptr(), nbytes, stream_of(src))
    if status:
        fail("fd_copy", status)


def launch_copy_persistent(dst: torch.Tensor, src: torch.Tensor, workgroups: int) -> None:
    """The copy roof's persistent form (``fd_copy_persistent``): ``workgroups``
    workgroups walk the 16-byte vectors grid-stride; same contract as
    ``launch_copy`` plus 16-byte aligned tensors of a 16-byte multiple."""
    nbytes = src.numel() * src.element_size()
    if dst.numel() * dst.element_size() != nbytes:
        raise ValueError("copy needs equal byte sizes")
    _lib.check("fd_copy_persistent", _lib.lib().fd_copy_persistent(
        dst.data_ptr(), src.data_ptr(), nbytes, int(workgroups), stream_of(src)))


def clock_probe(out: torch.Tensor) -> int:
    """``fd_clock_probe`` into ``out`` (int64 ``[W, 3]`` on the GPU, W workgroups:
    XCD id, shader clock counter, wall clock counter per row) on the current
    stream; returns the wall clock's rate in kHz."""
    import ctypes

    if out.dtype != torch.int64 or out.ndim != 2 or out.shape[1] != 3 or not out.is_contiguous():
        raise ValueError("out must be a contiguous int64 [W, 3] tensor")
    khz = ctypes.c_int(0)
    _lib.check("fd_clock_probe", _lib.lib().fd_clock_probe(out.data_ptr(), int(out.shape[0]), ctypes.byref(khz),
                                                           stream_of(out)))
    return khz.value


def launch_read(src: torch.Tensor, hit: torch.Tensor, key: int = 0x2545F491) -> None:
    """Read roof: stream ``src`` (contiguous, 16-byte multiple) and set bit 0 of
    the int32 ``hit`` where the xor of a wave's words equals ``key``."""
    nbytes = src.numel() * src.element_size()
    status = native().read(src.data_ptr(), nbytes, int(key), hit.data_ptr(), stream_of(src))
    if status:
        fail("fd_read", status)


def launch_triad(a: torch.Tensor, b: torch.Tensor, c: torch.Tensor, scale: float = 1.0) -> None:
    """``c = a + b * scale`` over contiguous tensors of one dtype."""
    status = native().triad(
        c.data_ptr(), a.data_ptr(), b.data_ptr(), float(scale), a.numel(), DTYPE_CODE[a.dtype],
        stream_of(a),
    )
    if status:
        fail("fd_triad", status)
