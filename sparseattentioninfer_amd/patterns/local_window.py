"""Sliding local window, drop-in for ``sparse_attentions/patterns/local_window.py``.

Each query attends to the ``window_size`` most recent positions, itself
included (``local_window.py:58-71``).  With ``block_size`` set, the CSR block
schedule is built as well; it is computed directly from the window geometry
(the blocks a query block's combined window overlaps), which equals the
reference's coarsening of the token mask (``local_window.py:42-47``) without
materialising that mask.  The token mask itself is built on first access.
"""
from __future__ import annotations

import torch

from sparseattentioninfer_amd.patterns.base import PatternMetadata, SparsePattern, block_mask_to_csr
from sparseattentioninfer_amd.patterns.bigbird import LazyMaskMetadata


def local_window_token_mask(T_q: int, T_k: int, H: int, window: int, device=None) -> torch.Tensor:
    """``[H, T_q, T_k]`` bool; query t sits at position ``max(0, T_k - T_q) + t`` (``local_window.py:58-71``)."""
    rows = (max(0, T_k - T_q) + torch.arange(T_q, device=device)).unsqueeze(1)
    cols = torch.arange(T_k, device=device).unsqueeze(0)
    keep = (cols >= rows - window + 1) & (cols <= rows)
    return keep.unsqueeze(0).expand(H, -1, -1)


def local_window_block_mask(T_q: int, T_k: int, window: int, block_size: int, device=None) -> torch.Tensor:
    """``[NQB, NKB]`` bool: key block kb is active for query block qb iff some query row of qb
    keeps some key of kb.  The rows of qb see the contiguous key range
    ``[first_row - window + 1, last_row]``, so this is an interval overlap test."""
    bs = int(block_size)
    nqb, nkb = -(-T_q // bs), -(-T_k // bs)
    qo = max(0, T_k - T_q)
    qb = torch.arange(nqb, device=device)
    first = qo + qb * bs
    last = qo + torch.minimum((qb + 1) * bs, torch.full_like(qb, T_q)) - 1
    lo = (first - window + 1).clamp(min=0)
    kb = torch.arange(nkb, device=device)
    k_first = kb * bs
    k_last = torch.minimum((kb + 1) * bs, torch.full_like(kb, T_k)) - 1
    return (k_first[None, :] <= last[:, None]) & (k_last[None, :] >= lo[:, None]) & (window > 0)


class LocalWindowPattern(SparsePattern):
    """``local_window.py:11-80``."""

    def __init__(self, window_size: int, block_size: int | None = None):
        self.window_size = window_size
        self.block_size = block_size
        self._cache: dict = {}

    def build(self, q: torch.Tensor, k: torch.Tensor, causal: bool = True) -> PatternMetadata:
        T_q, T_k, H, device = q.size(2), k.size(2), q.size(1), q.device
        key = (T_q, T_k, H, f"{device.type}:{device.index}", self.window_size, self.block_size)
        if key not in self._cache:
            pairs = offsets = None
            if self.block_size is not None:
                bm = local_window_block_mask(T_q, T_k, self.window_size, self.block_size, device)
                pairs, offsets = block_mask_to_csr(bm.unsqueeze(0).expand(H, -1, -1))
            self._cache[key] = {"pairs": pairs, "offsets": offsets, "mask": None}
        e = self._cache[key]

        def mask_fn():
            if e["mask"] is None:
                e["mask"] = local_window_token_mask(T_q, T_k, H, self.window_size, device)
            return e["mask"]

        return LazyMaskMetadata(mask_fn=mask_fn, kind="local", keep_ratio=self._estimate_keep_ratio(T_q, T_k),
                                block_size=self.block_size, block_pairs=e["pairs"], block_pair_offsets=e["offsets"])

    def _estimate_keep_ratio(self, T_q: int, T_k: int) -> float:
        """``local_window.py:73-80``."""
        W = self.window_size
        if T_q == 0 or T_k == 0:
            return 0.0
        qo = max(0, T_k - T_q)
        kept = sum(min(W, qo + i + 1) for i in range(T_q))
        return min(1.0, kept / (T_q * T_k))
