"""Attention-backend interface: the drop-in boundary.

Same abstract methods and HybridBackend dispatch as
python/minisgl/attention/base.py:12-63.
"""

from __future__ import annotations

from abc import ABC, abstractmethod
from dataclasses import dataclass
from typing import TYPE_CHECKING, List

if TYPE_CHECKING:
    import torch

    from ..core import Batch


@dataclass
class BaseAttnMetadata(ABC):
    @abstractmethod
    def get_last_indices(self, bs: int) -> "torch.Tensor": ...


class BaseAttnBackend(ABC):
    @abstractmethod
    def forward(
        self, q: "torch.Tensor", k: "torch.Tensor", v: "torch.Tensor", layer_id: int, batch: "Batch"
    ) -> "torch.Tensor": ...

    @abstractmethod
    def prepare_metadata(self, batch: "Batch") -> None: ...

    @abstractmethod
    def init_capture_graph(self, max_seq_len: int, bs_list: List[int]) -> None: ...

    @abstractmethod
    def prepare_for_capture(self, batch: "Batch") -> None: ...

    @abstractmethod
    def prepare_for_replay(self, batch: "Batch") -> None: ...


class HybridBackend(BaseAttnBackend):
    """Prefill batches to one backend, decode batches (and graph hooks) to another."""

    def __init__(self, prefill_backend: BaseAttnBackend, decode_backend: BaseAttnBackend) -> None:
        self.prefill_backend = prefill_backend
        self.decode_backend = decode_backend

    def forward(self, q, k, v, layer_id: int, batch: "Batch"):
        backend = self.prefill_backend if batch.is_prefill else self.decode_backend
        return backend.forward(q, k, v, layer_id, batch)

    def prepare_metadata(self, batch: "Batch") -> None:
        backend = self.prefill_backend if batch.is_prefill else self.decode_backend
        return backend.prepare_metadata(batch)

    def init_capture_graph(self, max_seq_len: int, bs_list: List[int]) -> None:
        self.decode_backend.init_capture_graph(max_seq_len, bs_list)

    def prepare_for_capture(self, batch: "Batch") -> None:
        self.decode_backend.prepare_for_capture(batch)

    def prepare_for_replay(self, batch: "Batch") -> None:
        self.decode_backend.prepare_for_replay(batch)
