"""MLA KV pool: one latent row (512 latent + 64 rope, bf16) per token per layer.

Layout ``[num_layers, num_pages, page_size, 576]``: 1152 bytes per token per
layer, a 64-token page is one contiguous 73,728-byte block, which the decode
kernel streams with 16-byte DMA loads. ``k_cache(layer)`` is the full latent
row and ``v_cache(layer)`` the view of its first 512 dims (absorbed MLA reads
the value out of the key row).

The pool can also hold decompressed per-head K (qk 192) and V (v 128) pages,
``[num_layers, num_pages, page_size, heads, 192 | 128]``, which the chunked
prefill kernel reads; both are indexed by the same page ids.

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
        prefill_heads: int = 0,
        qk_head_dim: int = 192,
        v_head_dim: int = 128,
    ) -> None:
        self._kv_dim = kv_lora_rank + qk_rope_head_dim
        self._v_dim = kv_lora_rank
        self._latent = torch.empty((num_layers, num_pages, page_size, self._kv_dim), dtype=dtype, device=device)
        self._num_layers = num_layers
        self._num_pages = num_pages
        self._page_size = page_size
        self._device = torch.device(device)
        self._prefill_heads = prefill_heads
        self._k_heads = self._v_heads = None
        if prefill_heads > 0:
            self._k_heads = torch.empty(
                (num_layers, num_pages, page_size, prefill_heads, qk_head_dim), dtype=dtype, device=device
            )
            self._v_heads = torch.empty(
                (num_layers, num_pages, page_size, prefill_heads, v_head_dim), dtype=dtype, device=device
            )

    # ---- BaseKVCachePool
    def k_cache(self, index: int) -> torch.Tensor:
        return self._latent[index]

    def v_cache(self, index: int) -> torch.Tensor:
        return self._latent[index][..., : self._v_dim]

    def store_kv(self, k: torch.Tensor, v: torch.Tensor | None, out_loc: torch.Tensor, layer_id: int) -> None:
        """Store new tokens at flat token locations ``out_loc``.

        ``k [T, 576]`` is a latent row (``v`` is then ignored: it is the
        latent's first 512 dims); ``k [T, H, 192]`` / ``v [T, H, 128]`` go to
        the per-head prefill pages.
        """
        if k.dim() == 2:
            assert k.shape[-1] == self._kv_dim, f"latent rows must be {self._kv_dim} wide"
            store_rows(self._latent[layer_id].view(-1, self._kv_dim), out_loc, k)
            return
        assert self._k_heads is not None, "pool was built without per-head prefill pages"
        T = k.shape[0]
        store_rows(self._k_heads[layer_id].view(self._num_pages * self._page_size, -1), out_loc, k.reshape(T, -1))
        store_rows(self._v_heads[layer_id].view(self._num_pages * self._page_size, -1), out_loc, v.reshape(T, -1))

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

    @property
    def has_prefill_pages(self) -> bool:
        return self._k_heads is not None

    def latent_cache(self, index: int) -> torch.Tensor:
        return self._latent[index]

    def prefill_k_cache(self, index: int) -> torch.Tensor:
        assert self._k_heads is not None
        return self._k_heads[index]

    def prefill_v_cache(self, index: int) -> torch.Tensor:
        assert self._v_heads is not None
        return self._v_heads[index]
