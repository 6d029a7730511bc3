"""MI355X (gfx950) causal GQA flash attention for Mimans M1.

The public surface mirrors ``mimans.model.attention_tilelang``; see
``mimansm1_v1_amd.attention``.  Tile
tuning: ``python -m mimansm1_v1_amd.tune``; the tile records: ``mimansm1_v1_amd.tuned``.
"""
from .attention import (  # noqa: F401
    AUTOTUNE, DTYPE, Attention, AttnConfig, FlashAttention, RMSNorm, Rotary, _kernels,
    apply_rope, attention_flops, benchmark, check_gpu, check_math, flash_attention,
    flash_attention_with_lse, flash_delta, get_kernel, reference, rope_reference,
    rotate_half, warmup,
)
# The harness ``attention.tune`` is not re-exported: ``mimansm1_v1_amd.tune``
# is the tuning CLI module.
