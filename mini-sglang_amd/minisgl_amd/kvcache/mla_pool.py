"""MLA KV pool: one latent row (512 latent + 64 rope, bf16) per token per layer.

Layout ``[num_layers, num_pages, page_size, 576]``: 1152 bytes per token per
layer, a 64-token page is one contiguous 73,728-byte block, which the decode
kernel streams with 16-byte DMA loads. ``k_cache(layer)`` is the full latent
row and ``v_cache(layer)`` the view of its first 512 dims (absorbed MLA reads
the value out of the key row).

Chunked prefill reads the same rows: the attention backend decompresses the
keys of a prefill batch into its own scratch (K = [W_UK c | k_pe],
V = W_UV c per head), so the pool holds 1152 bytes per token and layer
whatever the number of heads.

Replaces the MHA-only pool of the reference (python/minisgl/kvcache/
mha_pool.py:10-68, whose creator has a TODO for MLA at kvcache/__init__.py:34).
"""

from __future__ import annotations

import torch

from ..kernel import store_rows
from .base import BaseKVCachePool


class MLAKVCache(BaseKVCachePool):
    def __init__(
        self,
        num_layers: int,
        num_pages: int,
        page_size: int,
        dtype: torch.dtype,
        device: torch.device,
        kv_lora_rank: int = 512,
        qk_rope_head_dim: int = 64,
    ) -> None:
        self._kv_dim = kv_lora_rank + qk_rope_head_dim
        self._v_dim = kv_lora_rank
        self._latent = torch.empty((num_layers, num_pages, page_size, self._kv_dim), dtype=dtype, device=device)
        self._num_layers = num_layers
        self._num_pages = num_pages
        self._page_size = page_size
        self._device = torch.device(device)

    # ---- BaseKVCachePool
    def k_cache(self, index: int) -> torch.Tensor:
        return self._latent[index]

    def v_cache(self, index: int) -> torch.Tensor:
        return self._latent[index][..., : self._v_dim]

    def store_kv(self, k: torch.Tensor, v: torch.Tensor | None, out_loc: torch.Tensor, layer_id: int) -> None:
        """Store new tokens' latent rows ``k [T, 576]`` at flat token locations ``out_loc`` (``v``
        is ignored: the values are the latent's first 512 dims)."""
        assert k.dim() == 2 and k.shape[-1] == self._kv_dim, f"latent rows must be [T, {self._kv_dim}]"
        store_rows(self._latent[layer_id].view(-1, self._kv_dim), out_loc, k)

    @property
    def device(self) -> torch.device:
        return self._device

    @property
    def dtype(self) -> torch.dtype:
        return self._latent.dtype

    @property
    def num_layers(self) -> int:
        return self._num_layers

    # ---- MLA extras
    @property
    def num_pages(self) -> int:
        return self._num_pages

    @property
    def page_size(self) -> int:
        return self._page_size

    def latent_cache(self, index: int) -> torch.Tensor:
        return self._latent[index]
