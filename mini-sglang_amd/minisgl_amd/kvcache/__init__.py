"""KV pools. ``create_kvcache_pool`` mirrors python/minisgl/kvcache/__init__.py:27-44
with the MLA variant that the reference leaves as a TODO."""

from __future__ import annotations

import torch

from ..config import MLAConfig
from .base import BaseKVCachePool
from .mla_pool import MLAKVCache
from .page_table import PagedTokenTable


def create_kvcache_pool(
    model_config: MLAConfig,
    num_pages: int,
    page_size: int,
    dtype: torch.dtype,
    device: torch.device,
) -> BaseKVCachePool:
    return MLAKVCache(
        num_layers=model_config.num_layers,
        num_pages=num_pages,
        page_size=page_size,
        dtype=dtype,
        device=device,
        kv_lora_rank=model_config.kv_lora_rank,
        qk_rope_head_dim=model_config.qk_rope_head_dim,
    )


__all__ = ["BaseKVCachePool", "MLAKVCache", "PagedTokenTable", "create_kvcache_pool"]
