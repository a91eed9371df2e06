"""MI355X (gfx950) decode operators: the non-attention half of a Llama decode step.

Drop-in for the reference package ``fused_decode`` (src/fused_decode/__init__.py):
same names and signatures, hand-written HIP kernels behind a C ABI.
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

__version__ = "0.1.0"

__all__ = [
    "DECODE_LINEAR_MAX_M",
    "add_rms_norm",
    "linear_decode",
    "post_attn_mlp",
    "pre_attn_qkv",
    "rms_norm",
    "rope",
    "swiglu",
]
