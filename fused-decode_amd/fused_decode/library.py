"""torch.library registration of the operator set, namespace ``fused_decode``.

    torch.ops.fused_decode.rms_norm(x, weight, eps)
    torch.ops.fused_decode.add_rms_norm(x, residual, weight, eps) -> (out, residual_out)
    torch.ops.fused_decode.rope(x, cos, sin)
    torch.ops.fused_decode.swiglu(gate, up)
    torch.ops.fused_decode.linear_decode(x, weight, bias, row_add, kind)
    torch.ops.fused_decode.post_attn_mlp(hidden, norm_weight, w_gate_up, w_down, eps, kind)
    torch.ops.fused_decode.pre_attn_qkv(hidden, norm_weight, w_qkv, cos, sin, eps, rope_cols, bias, kind)
    torch.ops.fused_decode.linear_decode_fp8(x, weight, scale, bias, row_add)
    torch.ops.fused_decode.post_attn_mlp_fp8(hidden, norm_weight, w_gate_up, gate_up_scale, w_down, down_scale, eps)
    torch.ops.fused_decode.pre_attn_qkv_fp8(hidden, norm_weight, w_qkv, scale, cos, sin, eps, rope_cols, bias)

Each is the functional form (no ``out=``) of the operator of the same name in
``fused_decode.ops``, registered as a custom op with a fake (meta) kernel, so
``torch.compile``, ``torch.export`` and AOT tracing keep the HIP launch as one
opaque node: the Python argument checks run once per call at run time, and
graph breaks do not happen around the operators. The reference names this as a
gap (README.md:101); it registers nothing. Importing ``fused_decode`` registers
the ops.

The fake kernels return what the real ones return: new contiguous tensors of
the result shape and the input dtype.
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import fp8, ops

_NS = "fused_decode"


def _lead(t: Tensor) -> tuple:
    return tuple(t.shape[:-1])


@torch.library.custom_op(f"{_NS}::rms_norm", mutates_args=())
def rms_norm(x: Tensor, weight: Tensor, eps: float = 1e-6) -> Tensor:
    return ops.rms_norm(x, weight, eps)


@rms_norm.register_fake
def _rms_norm_fake(x, weight, eps=1e-6):
    return x.new_empty(x.shape)


@torch.library.custom_op(f"{_NS}::add_rms_norm", mutates_args=())
def add_rms_norm(x: Tensor, residual: Tensor, weight: Tensor, eps: float = 1e-6) -> tuple[Tensor, Tensor]:
    return ops.add_rms_norm(x, residual, weight, eps)


@add_rms_norm.register_fake
def _add_rms_norm_fake(x, residual, weight, eps=1e-6):
    return x.new_empty(x.shape), x.new_empty(x.shape)


@torch.library.custom_op(f"{_NS}::rope", mutates_args=())
def rope(x: Tensor, cos: Tensor, sin: Tensor) -> Tensor:
    return ops.rope(x, cos, sin)


@rope.register_fake
def _rope_fake(x, cos, sin):
    return x.new_empty(x.shape)


@torch.library.custom_op(f"{_NS}::swiglu", mutates_args=())
def swiglu(gate: Tensor, up: Tensor) -> Tensor:
    return ops.swiglu(gate, up)


@swiglu.register_fake
def _swiglu_fake(gate, up):
    return gate.new_empty(gate.shape)


@torch.library.custom_op(f"{_NS}::linear_decode", mutates_args=())
def linear_decode(x: Tensor, weight: Tensor, bias: Tensor | None = None,
                  row_add: Tensor | None = None, kind: str | None = None) -> Tensor:
    return ops.linear_decode(x, weight, bias, row_add=row_add, kind=kind)


@linear_decode.register_fake
def _linear_decode_fake(x, weight, bias=None, row_add=None, kind=None):
    return x.new_empty((*_lead(x), weight.shape[0]))


@torch.library.custom_op(f"{_NS}::post_attn_mlp", mutates_args=())
def post_attn_mlp(hidden: Tensor, norm_weight: Tensor, w_gate_up: Tensor, w_down: Tensor,
                  eps: float = 1e-6, kind: str | None = None) -> Tensor:
    return ops.post_attn_mlp(hidden, norm_weight, w_gate_up, w_down, eps, kind=kind)


@post_attn_mlp.register_fake
def _post_attn_mlp_fake(hidden, norm_weight, w_gate_up, w_down, eps=1e-6, kind=None):
    return hidden.new_empty(hidden.shape)


@torch.library.custom_op(f"{_NS}::pre_attn_qkv", mutates_args=())
def pre_attn_qkv(hidden: Tensor, norm_weight: Tensor, w_qkv: Tensor, cos: Tensor, sin: Tensor,
                 eps: float, rope_cols: int, bias: Tensor | None = None,
                 kind: str | None = None) -> Tensor:
    return ops.pre_attn_qkv(hidden, norm_weight, w_qkv, cos, sin, eps, rope_cols=rope_cols,
                            bias=bias, kind=kind)


@pre_attn_qkv.register_fake
def _pre_attn_qkv_fake(hidden, norm_weight, w_qkv, cos, sin, eps, rope_cols, bias=None, kind=None):
    return hidden.new_empty((*_lead(hidden), w_qkv.shape[0]))


@torch.library.custom_op(f"{_NS}::linear_decode_fp8", mutates_args=())
def linear_decode_fp8(x: Tensor, weight: Tensor, scale: Tensor, bias: Tensor | None = None,
                      row_add: Tensor | None = None) -> Tensor:
    return fp8.linear_decode_fp8(x, weight, scale, bias, row_add=row_add)


@linear_decode_fp8.register_fake
def _linear_decode_fp8_fake(x, weight, scale, bias=None, row_add=None):
    return x.new_empty((*_lead(x), weight.shape[0]))


@torch.library.custom_op(f"{_NS}::post_attn_mlp_fp8", mutates_args=())
def post_attn_mlp_fp8(hidden: Tensor, norm_weight: Tensor, w_gate_up: Tensor, gate_up_scale: Tensor,
                      w_down: Tensor, down_scale: Tensor, eps: float = 1e-6) -> Tensor:
    return fp8.post_attn_mlp_fp8(hidden, norm_weight, w_gate_up, gate_up_scale, w_down, down_scale, eps)


@post_attn_mlp_fp8.register_fake
def _post_attn_mlp_fp8_fake(hidden, norm_weight, w_gate_up, gate_up_scale, w_down, down_scale, eps=1e-6):
    return hidden.new_empty(hidden.shape)


@torch.library.custom_op(f"{_NS}::pre_attn_qkv_fp8", mutates_args=())
def pre_attn_qkv_fp8(hidden: Tensor, norm_weight: Tensor, w_qkv: Tensor, scale: Tensor, cos: Tensor,
                     sin: Tensor, eps: float, rope_cols: int, bias: Tensor | None = None) -> Tensor:
    return fp8.pre_attn_qkv_fp8(hidden, norm_weight, w_qkv, scale, cos, sin, eps, rope_cols=rope_cols,
                                bias=bias)


@pre_attn_qkv_fp8.register_fake
def _pre_attn_qkv_fp8_fake(hidden, norm_weight, w_qkv, scale, cos, sin, eps, rope_cols, bias=None):
    return hidden.new_empty((*_lead(hidden), w_qkv.shape[0]))


OPS = ("rms_norm", "add_rms_norm", "rope", "swiglu", "linear_decode", "post_attn_mlp", "pre_attn_qkv",
       "linear_decode_fp8", "post_attn_mlp_fp8", "pre_attn_qkv_fp8")
