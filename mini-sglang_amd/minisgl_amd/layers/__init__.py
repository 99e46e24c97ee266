"""Callers of the MLA backend: the DeepSeek-V3 / Kimi-K2 latent attention layer."""

from .mla_attention import (
    HipLayerOps,
    MLAAttentionLayer,
    MLALayerConfig,
    MLAWeights,
    rope_cos_sin_cache,
    softmax_mscale,
    yarn_mscale,
)

__all__ = [
    "HipLayerOps",
    "MLAAttentionLayer",
    "MLALayerConfig",
    "MLAWeights",
    "rope_cos_sin_cache",
    "softmax_mscale",
    "yarn_mscale",
]
