"""Argument contract of the public operators, written as data.

Every operator names its checks in ``CONTRACT``: an ordered tuple of rules over
the call's named arguments. ``check(op, **args)`` applies them in order and the
first failure raises ``TypeError`` (wrong kind of object or dtype) or
``ValueError`` (device, shape, value). The operators run this once per distinct
argument signature (``ops`` caches the resulting launch plan), so the rules
can afford clear messages.

What a rule accepts is the drop-in contract of the reference's operators
(src/fused_decode/ops.py:34-69 for the shared checks, :72-315 for each
operator): activations are CUDA float16/bfloat16 tensors, norm weights and
RoPE angles may also be float32, bias is the activation dtype or float32,
row_add is any float dtype broadcastable to the output, eps is finite and
non-negative, and the messages carry the words the reference's tests match
("CUDA", "weight", "even"). fp8 weights (``float8_e4m3fn`` codes with float32
row scales) have rules of their own.
"""

from __future__ import annotations

import math
from typing import Callable

import torch

ACTIVATION = (torch.float16, torch.bfloat16)
FLOAT = (torch.float16, torch.bfloat16, torch.float32)
FP8 = torch.float8_e4m3fn

Rule = Callable[[dict], None]


def _names(dtypes) -> str:
    return " or ".join(str(d).replace("torch.", "") for d in dtypes)


# ------------------------------------------------------------------ rules


def tensor_on_gpu(name: str, dtypes=ACTIVATION) -> Rule:
    """A CUDA (HIP) tensor of one of ``dtypes``."""

    def rule(a: dict) -> None:
        t = a[name]
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name} must be a tensor, got {type(t).__name__}")
        if not t.is_cuda:
            raise ValueError(f"{name} must be a CUDA tensor (a HIP device), got device {t.device}")
        if t.dtype not in dtypes:
            raise TypeError(f"{name} must be {_names(dtypes)}, got {t.dtype}")

    return rule


def like(name: str, ref: str, *, optional: bool = False) -> Rule:
    """Same shape, dtype and device as ``ref``."""

    def rule(a: dict) -> None:
        t, r = a[name], a[ref]
        if t is None and optional:
            return
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name} must be a tensor, got {type(t).__name__}")
        if t.device != r.device:
            raise ValueError(f"{name} is on {t.device} but {ref} is on {r.device}")
        if t.shape != r.shape:
            raise ValueError(f"{name} has shape {tuple(t.shape)}, {ref} has {tuple(r.shape)}")
        if t.dtype != r.dtype:
            raise TypeError(f"{name} is {t.dtype}, {ref} is {r.dtype}")

    return rule


def vector_for(name: str, ref: str, *, label: str | None = None, dtypes=FLOAT) -> Rule:
    """A 1-D tensor with one element per column of ``ref`` (its last dim), on
    ``ref``'s device, of one of ``dtypes``. ``label`` names it in messages
    (the norm weight is "weight" whatever the argument is called)."""
    label = label or name

    def rule(a: dict) -> None:
        t, r = a[name], a[ref]
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{label} must be a tensor, got {type(t).__name__}")
        if t.device != r.device:
            raise ValueError(f"{label} is on {t.device} but {ref} is on {r.device}")
        if t.dtype not in dtypes:
            raise TypeError(f"{label} must be {_names(dtypes)}, got {t.dtype}")
        if t.ndim != 1 or t.shape[0] != r.shape[-1]:
            raise ValueError(f"{label} must have shape ({r.shape[-1]},), got {tuple(t.shape)}")

    return rule


def finite_eps(name: str = "eps") -> Rule:
    def rule(a: dict) -> None:
        try:
            v = float(a[name])
        except (TypeError, ValueError) as exc:
            raise ValueError(f"{name} must be a finite value >= 0, got {a[name]!r}") from exc
        if not (math.isfinite(v) and v >= 0):
            raise ValueError(f"{name} must be a finite value >= 0, got {v}")
        a[name] = v

    return rule


def even_last(name: str, what: str = "rope last dimension") -> Rule:
    def rule(a: dict) -> None:
        n = a[name].shape[-1] if a[name].ndim else 0
        if n % 2:
            raise ValueError(f"{what} must be even, got {n}")

    return rule


def broadcast_angles(name: str, ref: str) -> Rule:
    """cos/sin of RoPE: a float tensor on ``ref``'s device whose last dim equals
    ``ref``'s and that broadcasts to ``ref``'s shape (shapes align on the right)."""

    def rule(a: dict) -> None:
        t, r = a[name], a[ref]
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name} must be a tensor, got {type(t).__name__}")
        if t.device != r.device:
            raise ValueError(f"{name} is on {t.device} but {ref} is on {r.device}")
        if t.dtype not in FLOAT:
            raise TypeError(f"{name} must be {_names(FLOAT)}, got {t.dtype}")
        if t.ndim == 0 or t.shape[-1] != r.shape[-1]:
            raise ValueError(f"{name} last dim {tuple(t.shape)[-1:]} must equal {ref}'s {r.shape[-1]}")
        if not _broadcasts(t.shape, r.shape):
            raise ValueError(f"cannot broadcast {name} shape {tuple(t.shape)} to {tuple(r.shape)}")

    return rule


def _broadcasts(src, dst) -> bool:
    """``src`` expands to ``dst``: no more dims, and each (right-aligned) is 1 or equal."""
    if len(src) > len(dst):
        return False
    return all(s in (1, d) for s, d in zip(reversed(src), reversed(dst)))


def weight_matrix(name: str, ref: str, *, label: str | None = None, fp8: bool = False,
                  dtype_error: type = ValueError) -> Rule:
    """A rank-2 ``[N, K]`` weight on ``ref``'s device: the activation dtype, or
    float8_e4m3fn codes with ``fp8``. A dtype mismatch of a plain weight raises
    ``dtype_error``: ValueError in linear_decode's contract ("weight device and
    dtype must match x"), TypeError for the fused QKV."""
    label = label or name

    def rule(a: dict) -> None:
        w, r = a[name], a[ref]
        if not isinstance(w, torch.Tensor):
            raise TypeError(f"{label} must be a tensor, got {type(w).__name__}")
        if fp8:
            if w.dtype != FP8:
                raise TypeError(f"{label} must hold torch.float8_e4m3fn codes (see quantize_fp8), got {w.dtype}")
            if w.device != r.device:
                raise ValueError(f"{label} is on {w.device} but {ref} is on {r.device}")
        elif w.device != r.device or w.dtype != r.dtype:
            err = dtype_error if w.device == r.device else ValueError
            raise err(f"{label} device and dtype must match {ref}: got {w.device}/{w.dtype}, "
                      f"{ref} is {r.device}/{r.dtype}")
        if w.ndim != 2:
            raise ValueError(f"{label} must have shape [N, K], got {tuple(w.shape)}")

    return rule


def row_scales(name: str, weight: str) -> Rule:
    """float32 per-row scales ``[N]`` of an fp8 weight, on its device."""

    def rule(a: dict) -> None:
        s, w = a[name], a[weight]
        if not isinstance(s, torch.Tensor) or s.dtype != torch.float32 or s.ndim != 1 \
                or s.shape[0] != w.shape[0]:
            got = tuple(s.shape) if isinstance(s, torch.Tensor) else type(s).__name__
            raise ValueError(f"{weight} scale must be float32 of shape ({w.shape[0]},), got {got}")
        if s.device != w.device:
            raise ValueError(f"{weight} scale is on {s.device}, {weight} on {w.device}")

    return rule


def inner_dim(ref: str, weight: str) -> Rule:
    """``ref``'s last dim is the weight's K."""

    def rule(a: dict) -> None:
        k = a[weight].shape[1]
        if a[ref].shape[-1] != k:
            raise ValueError(f"{ref} last dim {a[ref].shape[-1]} != {weight} K {k}")

    return rule


def bias_for(name: str, ref: str, weight: str) -> Rule:
    """Optional ``[N]`` bias in the activation dtype or float32."""

    def rule(a: dict) -> None:
        b = a.get(name)
        if b is None:
            return
        n, r = a[weight].shape[0], a[ref]
        if not isinstance(b, torch.Tensor):
            raise TypeError(f"{name} must be a tensor or None, got {type(b).__name__}")
        if b.ndim != 1 or b.shape[0] != n:
            raise ValueError(f"{name} must have shape ({n},), got {tuple(b.shape)}")
        if b.device != r.device:
            raise ValueError(f"{name} must be on {ref}'s device {r.device}, got {b.device}")
        if b.dtype not in (r.dtype, torch.float32):
            raise TypeError(f"{name} must match {ref} ({r.dtype}) or be float32, got {b.dtype}")

    return rule


def row_add_for(name: str, ref: str, weight: str) -> Rule:
    """Optional epilogue addend: any float dtype, on ``ref``'s device, shaped so
    it indexes the ``[M, N]`` output (``ops`` resolves the broadcast)."""

    def rule(a: dict) -> None:
        t = a.get(name)
        if t is None:
            return
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name} must be a tensor or None, got {type(t).__name__}")
        if t.device != a[ref].device:
            raise ValueError(f"{name} must be on {ref}'s device {a[ref].device}, got {t.device}")
        if t.dtype not in FLOAT:
            raise TypeError(f"{name} must be {_names(FLOAT)}, got {t.dtype}")

    return rule


def mlp_weights(gate_up: str, down: str, ref: str, *, fp8: bool = False) -> Rule:
    """``gate_up [2I, H]`` and ``down [H, I]`` for ``ref [..., H]``: rank 2,
    consistent widths, on ``ref``'s device, in its dtype (or fp8 codes)."""

    def rule(a: dict) -> None:
        wgu, wd, r = a[gate_up], a[down], a[ref]
        for nm, w in ((gate_up, wgu), (down, wd)):
            if not isinstance(w, torch.Tensor):
                raise TypeError(f"{nm} must be a tensor, got {type(w).__name__}")
        if fp8:
            for nm, w in ((gate_up, wgu), (down, wd)):
                if w.dtype != FP8:
                    raise TypeError(f"{nm} must hold torch.float8_e4m3fn codes (see quantize_fp8), got {w.dtype}")
        if wgu.ndim != 2 or wd.ndim != 2:
            raise ValueError(f"{gate_up} and {down} must be rank-2, got {wgu.ndim} and {wd.ndim} dims")
        (two_i, h), (h_d, i) = wgu.shape, wd.shape
        if two_i != 2 * i or h != h_d or r.shape[-1] != h:
            raise ValueError(
                f"expected {gate_up} [2I, H] and {down} [H, I] with {ref} [..., H], got "
                f"{tuple(wgu.shape)}, {tuple(wd.shape)}, {tuple(r.shape)}")
        if not fp8 and (wgu.dtype != r.dtype or wd.dtype != r.dtype):
            raise TypeError(f"MLP weights must be {ref}'s dtype {r.dtype}, got {wgu.dtype} and {wd.dtype}")
        if wgu.device != r.device or wd.device != r.device:
            raise ValueError(f"MLP weights must be on {ref}'s device {r.device}")

    return rule


def kind_name(name: str = "kind") -> Rule:
    def rule(a: dict) -> None:
        k = a[name]
        if k is not None and k not in ("dot", "simt"):
            raise ValueError(f"kind must be 'dot' or 'simt' (or None for FUSED_DECODE_LINEAR_KIND), got {k!r}")

    return rule


def output_like(name: str, ref: str) -> Rule:
    """``out`` of a row-wise operator: same shape, dtype and device as the input
    (any strides)."""
    return like(name, ref, optional=True)


# ------------------------------------------------- row-sum (sumsq) entry points
#
# The row-sum forms call C entry points that take bare pointers with no extents
# and, for the MLP and QKV weights, no strides: every operand's layout is fixed
# here, before any launch, so a mis-shaped tensor raises instead of becoming an
# out-of-bounds read or write on the GPU.

SUMSQ_MIN_ROWS = 5  # the MFMA kernels that write and read the sums run from this many rows


def decode_rows(name: str, lo: int = SUMSQ_MIN_ROWS, hi: int = 16) -> Rule:
    """A contiguous rank-2 ``[M, K]`` activation with ``lo <= M <= hi``."""

    def rule(a: dict) -> None:
        t = a[name]
        if t.ndim != 2 or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous [M, K] tensor, got shape {tuple(t.shape)} "
                             f"strides {t.stride()}")
        if not lo <= t.shape[0] <= hi:
            raise ValueError(f"row sums of squares run on the MFMA kernels: {name} needs {lo} to {hi} rows, "
                             f"got {t.shape[0]}")

    return rule


def unit_k_stride(name: str) -> Rule:
    """A weight whose K (last) dim is dense: element stride 1."""

    def rule(a: dict) -> None:
        w = a[name]
        if w.shape[-1] > 1 and w.stride(-1) != 1:
            raise ValueError(f"{name} must have unit stride along K, got strides {w.stride()}")

    return rule


def dense(*names: str) -> Rule:
    """Contiguous tensors (kernels that take no strides for them)."""

    def rule(a: dict) -> None:
        for name in names:
            t = a.get(name)
            if isinstance(t, torch.Tensor) and not t.is_contiguous():
                raise ValueError(f"{name} must be contiguous, got shape {tuple(t.shape)} strides {t.stride()}")

    return rule


def matrix_for(name: str, ref: str, rows: Callable[[dict], int], cols: Callable[[dict], int], *,
               optional: bool = False, dtypes=None) -> Rule:
    """A contiguous ``[rows, cols]`` tensor on ``ref``'s device, in ``ref``'s dtype
    (or one of ``dtypes``): an output, scratch or addend the kernel indexes as
    dense rows."""

    def rule(a: dict) -> None:
        t, r = a.get(name), a[ref]
        if t is None:
            if optional:
                return
            raise ValueError(f"{name} is required")
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name} must be a tensor, got {type(t).__name__}")
        if t.device != r.device:
            raise ValueError(f"{name} is on {t.device} but {ref} is on {r.device}")
        ok = (r.dtype,) if dtypes is None else dtypes
        if t.dtype not in ok:
            raise TypeError(f"{name} must be {_names(ok)}, got {t.dtype}")
        shape = (rows(a), cols(a))
        if tuple(t.shape) != shape or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous {list(shape)} tensor, got shape {tuple(t.shape)} "
                             f"strides {t.stride()}")

    return rule


def sums_buffer(name: str, ref: str, width: Callable[[dict], int], *, optional: bool = False) -> Rule:
    """Float32 tile sums of squares for a ``width``-column activation: a
    contiguous buffer of ``ceil(width / 16) * 16`` values on ``ref``'s device
    (``sumsq_buffer``)."""

    def rule(a: dict) -> None:
        t = a.get(name)
        if t is None:
            if optional:
                return
            raise ValueError(f"{name} is required")
        w = width(a)
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name} must be a tensor, got {type(t).__name__}")
        if t.device != a[ref].device:
            raise ValueError(f"{name} is on {t.device} but {ref} is on {a[ref].device}")
        if t.dtype != torch.float32 or not t.is_contiguous() or t.numel() != (w + 15) // 16 * 16:
            raise ValueError(f"{name} must be a contiguous float32 tensor of ceil({w}/16)*16 values "
                             f"(sumsq_buffer), got {t.dtype} shape {tuple(t.shape)}")

    return rule


def _m(ref: str) -> Callable[[dict], int]:
    return lambda a: a[ref].shape[0]


def _rows_of(weight: str) -> Callable[[dict], int]:
    return lambda a: a[weight].shape[0]


def _cols_of(weight: str) -> Callable[[dict], int]:
    return lambda a: a[weight].shape[1]


# ------------------------------------------------------------------ contract

CONTRACT: dict[str, tuple[Rule, ...]] = {
    "rms_norm": (tensor_on_gpu("x"), vector_for("weight", "x"), finite_eps(), output_like("out", "x")),
    "add_rms_norm": (tensor_on_gpu("x"), tensor_on_gpu("residual"), like("residual", "x"),
                     vector_for("weight", "x"), finite_eps(), output_like("out", "x"),
                     output_like("residual_out", "x")),
    "rope": (tensor_on_gpu("x"), even_last("x"), broadcast_angles("cos", "x"),
             broadcast_angles("sin", "x"), output_like("out", "x")),
    "swiglu": (tensor_on_gpu("gate"), tensor_on_gpu("up"), like("up", "gate"), output_like("out", "gate")),
    "linear_decode": (tensor_on_gpu("x"), weight_matrix("weight", "x"), inner_dim("x", "weight"),
                      kind_name(), bias_for("bias", "x", "weight"), row_add_for("row_add", "x", "weight")),
    "post_attn_mlp": (tensor_on_gpu("hidden"), mlp_weights("w_gate_up", "w_down", "hidden"),
                      vector_for("norm_weight", "hidden", label="weight"), finite_eps(), kind_name()),
    "pre_attn_qkv": (tensor_on_gpu("hidden"), weight_matrix("w_qkv", "hidden", dtype_error=TypeError),
                     inner_dim("hidden", "w_qkv"),
                     vector_for("norm_weight", "hidden", label="weight"), finite_eps(), kind_name(),
                     bias_for("bias", "hidden", "w_qkv")),
    "linear_decode_fp8": (tensor_on_gpu("x"), weight_matrix("weight", "x", fp8=True),
                          row_scales("scale", "weight"), inner_dim("x", "weight"),
                          bias_for("bias", "x", "weight"), row_add_for("row_add", "x", "weight")),
    "post_attn_mlp_fp8": (tensor_on_gpu("hidden"), mlp_weights("w_gate_up", "w_down", "hidden", fp8=True),
                          row_scales("gate_up_scale", "w_gate_up"), row_scales("down_scale", "w_down"),
                          vector_for("norm_weight", "hidden", label="weight"), finite_eps()),
    "pre_attn_qkv_fp8": (tensor_on_gpu("hidden"), weight_matrix("w_qkv", "hidden", fp8=True),
                         row_scales("scale", "w_qkv"), inner_dim("hidden", "w_qkv"),
                         vector_for("norm_weight", "hidden", label="weight"), finite_eps(),
                         bias_for("bias", "hidden", "w_qkv")),
}



def dot_kind_if(*sums: str, name: str = "kind") -> Rule:
    """The row sums come from the MFMA kernel, which kind "dot" selects: required
    when any of the ``sums`` buffers is passed."""

    def rule(a: dict) -> None:
        if any(a.get(s) is not None for s in sums) and a[name] != "dot":
            raise ValueError(f"row sums of squares come from the MFMA GEMV: kind must be 'dot', got {a[name]!r}")

    return rule


def _h(a: dict) -> int:
    return a["hidden"].shape[1]


_SUMSQ_LINEAR = (decode_rows("x"), unit_k_stride("weight"),
                 matrix_for("out", "x", _m("x"), _rows_of("weight")),
                 matrix_for("row_add", "x", _m("x"), _rows_of("weight"), optional=True, dtypes=FLOAT),
                 sums_buffer("ss_out", "x", _rows_of("weight")))
_SUMSQ_MLP = (decode_rows("hidden"), dense("norm_weight", "w_gate_up", "w_down"),
              matrix_for("out", "hidden", _m("hidden"), _h),
              matrix_for("mid", "hidden", _m("hidden"), _cols_of("w_down"), optional=True),
              sums_buffer("ss_in", "hidden", _h, optional=True), sums_buffer("ss_out", "hidden", _h, optional=True))
_SUMSQ_QKV = (decode_rows("hidden"), dense("norm_weight", "w_qkv"), sums_buffer("ss_in", "hidden", _h),
              matrix_for("out", "hidden", _m("hidden"), _rows_of("w_qkv")))

# The row-sum forms (rowsq.py): their plain operator's rules, then the layout the
# bare-pointer entry points assume.
CONTRACT.update({
    "linear_sumsq": (*CONTRACT["linear_decode"], dot_kind_if("ss_out"), *_SUMSQ_LINEAR),
    "post_attn_mlp_sumsq": (*CONTRACT["post_attn_mlp"], dot_kind_if("ss_in", "ss_out"), *_SUMSQ_MLP),
    "pre_attn_qkv_sumsq": (*CONTRACT["pre_attn_qkv"], dot_kind_if("ss_in"), *_SUMSQ_QKV),
    "linear_fp8_sumsq": (*CONTRACT["linear_decode_fp8"], *_SUMSQ_LINEAR),
    "post_attn_mlp_fp8_sumsq": (*CONTRACT["post_attn_mlp_fp8"], dense("gate_up_scale", "down_scale"),
                                *_SUMSQ_MLP),
    "pre_attn_qkv_fp8_sumsq": (*CONTRACT["pre_attn_qkv_fp8"], dense("scale"), *_SUMSQ_QKV),
})


def check(op: str, **args) -> dict:
    """Apply ``op``'s rules to its named arguments; returns them with values
    normalised (eps as a float). Raises on the first broken rule."""
    for rule in CONTRACT[op]:
        rule(args)
    return args
