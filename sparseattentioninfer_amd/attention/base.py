"""Backend interface, mirroring ``sparse_attentions/attention/base.py:9-40``."""
from __future__ import annotations

from abc import ABC, abstractmethod

import torch

from ..patterns.base import PatternMetadata


class AttentionBackend(ABC):
    """Computes attention given pre-projected q/k/v and a pattern."""

    @abstractmethod
    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                pattern: PatternMetadata) -> torch.Tensor:
        """``q [B,H,T_q,D]``, ``k, v [B,H_kv,T_k,D]`` -> ``[B,H,T_q,D]``."""

    @property
    def actual_backend(self) -> str:
        """Name of the path that ran on the last :meth:`forward` call."""
        return type(self).__name__
