"""Callers of the MLA backend: the DeepSeek-V3 / Kimi-K2 latent attention layer."""

from .mla_attention import (
    MLAAttentionLayer,
    MLALayerConfig,
    MLAWeights,
    apply_rope,
    rms_norm,
    rope_cos_sin_cache,
    softmax_mscale,
    yarn_mscale,
)

__all__ = [
    "MLAAttentionLayer",
    "MLALayerConfig",
    "MLAWeights",
    "apply_rope",
    "rms_norm",
    "rope_cos_sin_cache",
    "softmax_mscale",
    "yarn_mscale",
]
