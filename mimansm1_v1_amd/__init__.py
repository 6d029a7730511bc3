"""MI355X (gfx950) causal GQA flash attention for Mimans M1.

The public surface mirrors ``mimans.model.attention_tilelang``; see
``mimansm1_v1_amd.attention``.
"""
from .attention import (  # noqa: F401
    AUTOTUNE, DTYPE, Attention, AttnConfig, FlashAttention, RMSNorm, Rotary, _kernels,
    apply_rope, attention_flops, benchmark, check_gpu, check_math, flash_attention,
    flash_attention_with_lse, flash_delta, get_kernel, reference, rope_reference,
    rotate_half, tune, warmup,
)
