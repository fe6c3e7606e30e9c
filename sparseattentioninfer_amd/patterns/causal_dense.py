"""``DenseCausalPattern``: full causal attention (``sparse_attentions/patterns/causal_dense.py:7-11``).

The hip_block_sparse backend runs ``kind="dense"`` on its kernels over a full
causal block schedule.
"""
from __future__ import annotations

import torch

from .base import PatternMetadata, SparsePattern


class DenseCausalPattern(SparsePattern):
    """Every causally visible key is kept."""

    def build(self, q: torch.Tensor, k: torch.Tensor, causal: bool = True) -> PatternMetadata:
        return PatternMetadata(kind="dense", keep_ratio=1.0)
