"""Backend registry, mirroring ``sparse_attentions/attention/__init__.py:8-21``.

``get_backend("hip_block_sparse")`` returns the gfx950 backend.  To make the
reference's own registry (and every caller that selects a backend by name)
see it, call :func:`register_into` with the reference's registry dict.
"""
from __future__ import annotations

from .base import AttentionBackend
from .hip_block_sparse import HipBlockSparseBackend

BACKEND_NAME = "hip_block_sparse"

_REGISTRY: dict[str, type[AttentionBackend]] = {
    BACKEND_NAME: HipBlockSparseBackend,
}


def get_backend(name: str, **kwargs) -> AttentionBackend:
    """Instantiates a registered backend; ``ValueError`` names the available ones."""
    if name not in _REGISTRY:
        available = ", ".join(sorted(_REGISTRY))
        raise ValueError(f"Unknown backend {name!r}. Available: {available}")
    return _REGISTRY[name](**kwargs)


def register_backend(name: str, cls: type[AttentionBackend]) -> None:
    """Adds a backend class under ``name`` (callers then select it with :func:`get_backend`)."""
    _REGISTRY[name] = cls


def register_into(registry: dict) -> None:
    """Adds this backend to another registry dict (e.g. the reference's ``_REGISTRY``)."""
    registry[BACKEND_NAME] = HipBlockSparseBackend


__all__ = ["AttentionBackend", "HipBlockSparseBackend", "get_backend", "register_backend", "register_into",
           "BACKEND_NAME"]
