"""Request / batch / context state read by the attention backend.

Same field semantics as python/minisgl/core.py:28-136: ``device_len`` counts
the tokens whose KV is (or is being) stored, ``cached_len`` those already
stored before this step, ``extend_len = device_len - cached_len``; the
context's ``page_table`` holds one token location per column (page size 1),
whatever the pool's page size.
"""

from __future__ import annotations

from contextlib import contextmanager
from dataclasses import dataclass, field
from typing import TYPE_CHECKING, Any, List, Literal

import torch

if TYPE_CHECKING:
    from .attention import BaseAttnBackend, BaseAttnMetadata
    from .kvcache import BaseKVCachePool


@dataclass(eq=False)
class Req:
    """A request as the backend sees it (python/minisgl/core.py:28-68)."""

    table_idx: int
    cached_len: int
    device_len: int
    uid: int = -1
    input_ids: torch.Tensor | None = None
    output_len: int = 0
    sampling_params: Any = None
    cache_handle: Any = None

    def __post_init__(self) -> None:
        assert 0 <= self.cached_len <= self.device_len, "need 0 <= cached_len <= device_len"

    @property
    def extend_len(self) -> int:
        return self.device_len - self.cached_len

    def complete_one(self) -> None:
        self.cached_len = self.device_len
        self.device_len += 1


@dataclass
class Batch:
    """python/minisgl/core.py:71-97; scheduler fills the init=False fields."""

    reqs: List[Req]
    phase: Literal["prefill", "decode"]
    input_ids: torch.Tensor = field(init=False)
    positions: torch.Tensor = field(init=False)
    out_loc: torch.Tensor = field(init=False)
    padded_reqs: List[Req] = field(init=False)
    attn_metadata: "BaseAttnMetadata" = field(init=False)

    @property
    def is_prefill(self) -> bool:
        return self.phase == "prefill"

    @property
    def is_decode(self) -> bool:
        return self.phase == "decode"

    @property
    def size(self) -> int:
        return len(self.reqs)

    @property
    def padded_size(self) -> int:
        return len(self.padded_reqs)


@dataclass
class Context:
    """python/minisgl/core.py:100-122."""

    page_size: int
    page_table: torch.Tensor = field(init=False)  # int32 [max_running_req + 1, align32(max_seq_len)]
    attn_backend: "BaseAttnBackend" = field(init=False)
    kv_cache: "BaseKVCachePool" = field(init=False)
    _batch: Batch | None = field(default=None, init=False)

    @property
    def batch(self) -> Batch:
        assert self._batch is not None, "No active batch in context"
        return self._batch

    @contextmanager
    def forward_batch(self, batch: Batch):
        assert self._batch is None, "Nested forward_batch is not allowed"
        try:
            self._batch = batch
            yield
        finally:
            self._batch = None


_GLOBAL_CTX: Context | None = None


def set_global_ctx(ctx: Context) -> None:
    global _GLOBAL_CTX
    assert _GLOBAL_CTX is None, "Global context is already set"
    _GLOBAL_CTX = ctx


def get_global_ctx() -> Context:
    assert _GLOBAL_CTX is not None, "Global context is not set"
    return _GLOBAL_CTX


def reset_global_ctx() -> None:
    """Drop the global context (tests and benchmarks build several)."""
    global _GLOBAL_CTX
    _GLOBAL_CTX = None
