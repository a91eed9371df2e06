"""MI355X (gfx950) decode operators: the non-attention half of a Llama decode step.

Drop-in for the reference package ``fused_decode`` (src/fused_decode/__init__.py):
same names and signatures, hand-written HIP kernels behind a C ABI. The same
operators are registered as torch custom ops, ``torch.ops.fused_decode.*``
(``fused_decode.library``), for torch.compile / export callers.
"""

from .ops import (
    DECODE_LINEAR_MAX_M,
    add_rms_norm,
    linear_decode,
    post_attn_mlp,
    pre_attn_qkv,
    rms_norm,
    rope,
    swiglu,
)

from .fp8 import dequantize_fp8, linear_decode_fp8, post_attn_mlp_fp8, pre_attn_qkv_fp8, quantize_fp8
from . import library  # registers torch.ops.fused_decode.* (custom ops with fake kernels)

__version__ = "0.1.0"

__all__ = [
    "DECODE_LINEAR_MAX_M",
    "add_rms_norm",
    "dequantize_fp8",
    "linear_decode_fp8",
    "post_attn_mlp_fp8",
    "pre_attn_qkv_fp8",
    "quantize_fp8",
    "linear_decode",
    "post_attn_mlp",
    "pre_attn_qkv",
    "rms_norm",
    "rope",
    "swiglu",
]
