"""Attention backends and their registry (python/minisgl/attention/__init__.py:15-68)."""

from __future__ import annotations

from typing import Protocol

from ..config import MLAConfig
from ..utils import Registry
from .base import BaseAttnBackend, BaseAttnMetadata, HybridBackend


class BackendCreator(Protocol):
    def __call__(self, config: MLAConfig) -> BaseAttnBackend: ...


SUPPORTED_ATTENTION_BACKENDS = Registry[BackendCreator]("Attention Backend")


@SUPPORTED_ATTENTION_BACKENDS.register("mla")
def create_mla_backend(config: MLAConfig):
    from .mla import MLAAttnBackend

    return MLAAttnBackend(config)


def validate_attn_backend(backend: str, allow_auto: bool = True) -> str:
    if backend != "auto":
        required = backend.split(",") if "," in backend else [backend]
        SUPPORTED_ATTENTION_BACKENDS.assert_supported(required)
    else:
        assert allow_auto, "auto is not allowed here"
    return backend


def create_attention_backend(backend: str, config: MLAConfig) -> BaseAttnBackend:
    validate_attn_backend(backend, allow_auto=False)
    if "," in backend:
        assert backend.count(",") == 1, "Only one comma is allowed in hybrid backend"
        p_name, d_name = backend.split(",", 1)
        if p_name != d_name:
            return HybridBackend(create_attention_backend(p_name, config), create_attention_backend(d_name, config))
        backend = p_name
    return SUPPORTED_ATTENTION_BACKENDS[backend](config)


__all__ = [
    "BaseAttnBackend",
    "BaseAttnMetadata",
    "HybridBackend",
    "SUPPORTED_ATTENTION_BACKENDS",
    "create_attention_backend",
    "validate_attn_backend",
]
