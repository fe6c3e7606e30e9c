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


def register_into(registry: dict, fallback=None) -> type[AttentionBackend]:
    """Adds this backend to another registry dict (e.g. the reference's ``_REGISTRY``).

    ``fallback`` (a backend class or instance, e.g. the reference's ``MaskedSdpaBackend``)
    restores the reference backends' contract (``triton_universal_backend.py:47-66``): inputs
    the kernels cannot take run there and ``actual_backend`` reads ``"masked_sdpa_fallback"``.
    Without it such inputs raise.  Returns the registered class.
    """
    cls = HipBlockSparseBackend
    if fallback is not None:
        cls = type("HipBlockSparseBackendWithFallback", (HipBlockSparseBackend,), {"default_fallback": fallback})
    registry[BACKEND_NAME] = cls
    return cls


__all__ = ["AttentionBackend", "HipBlockSparseBackend", "get_backend", "register_backend", "register_into",
           "BACKEND_NAME"]
