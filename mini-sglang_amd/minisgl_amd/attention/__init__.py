"""Attention backends by name, and the ``"prefill,decode"`` hybrid selection.

Backend names map to creators taking the model's attention config, as in the
reference (python/minisgl/attention/__init__.py:15-68): a plain name picks one
backend, ``"p,d"`` builds a ``HybridBackend`` of two. Only ``"mla"`` exists
here; a deployment of the reference registers ``create_mla_backend`` in the
reference's own table instead.
"""

from __future__ import annotations

from argparse import ArgumentTypeError
from typing import Dict, List, Protocol

from ..config import MLAConfig
from .base import BaseAttnBackend, BaseAttnMetadata, HybridBackend


class BackendCreator(Protocol):
    def __call__(self, config: MLAConfig) -> BaseAttnBackend: ...


def create_mla_backend(config: MLAConfig) -> BaseAttnBackend:
    from .mla import MLAAttnBackend

    return MLAAttnBackend(config)


SUPPORTED_ATTENTION_BACKENDS: Dict[str, BackendCreator] = {"mla": create_mla_backend}


def supported_backends() -> List[str]:
    return sorted(SUPPORTED_ATTENTION_BACKENDS)


def validate_attn_backend(backend: str, allow_auto: bool = True) -> str:
    """Check a backend spec (``"auto"``, ``"name"`` or ``"prefill,decode"``); unknown names raise
    ``ArgumentTypeError`` as the reference's argument parser expects."""
    if backend == "auto":
        assert allow_auto, "auto is not allowed here"
        return backend
    unknown = [n for n in backend.split(",") if n not in SUPPORTED_ATTENTION_BACKENDS]
    if unknown:
        raise ArgumentTypeError(f"unknown attention backend(s) {unknown}; known: {supported_backends()}")
    return backend


def create_attention_backend(backend: str, config: MLAConfig) -> BaseAttnBackend:
    validate_attn_backend(backend, allow_auto=False)
    names = backend.split(",")
    assert len(names) <= 2, "a hybrid backend names one prefill and one decode backend"
    if len(names) == 2 and names[0] != names[1]:
        return HybridBackend(create_attention_backend(names[0], config), create_attention_backend(names[1], config))
    return SUPPORTED_ATTENTION_BACKENDS[names[0]](config)


__all__ = [
    "BaseAttnBackend",
    "BaseAttnMetadata",
    "HybridBackend",
    "SUPPORTED_ATTENTION_BACKENDS",
    "create_attention_backend",
    "create_mla_backend",
    "supported_backends",
    "validate_attn_backend",
]
