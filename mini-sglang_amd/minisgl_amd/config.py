"""MLA attention shape of a DeepSeek-V3 / Kimi-K2 style layer (per rank)."""

from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class MLAConfig:
    num_heads: int = 64  # query heads on this rank
    num_layers: int = 1
    kv_lora_rank: int = 512  # latent width; also the absorbed value width
    qk_rope_head_dim: int = 64
    qk_nope_head_dim: int = 128
    v_head_dim: int = 128
    softmax_mscale: float = 1.0  # YaRN attention factor; the scale is multiplied by its square

    @property
    def kv_dim(self) -> int:
        """Latent KV row: latent + rope (576)."""
        return self.kv_lora_rank + self.qk_rope_head_dim

    @property
    def qk_head_dim(self) -> int:
        """Decompressed per-head q/k width used by prefill (192)."""
        return self.qk_nope_head_dim + self.qk_rope_head_dim

    @property
    def softmax_scale(self) -> float:
        return self.softmax_mscale**2 * self.qk_head_dim**-0.5
