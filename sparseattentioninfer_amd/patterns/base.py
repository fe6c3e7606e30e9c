"""Pattern metadata and CSR block-schedule construction (device-side, vectorised).

Interface mirror of ``sparse_attentions/patterns/base.py``: the same
``PatternMetadata`` fields and ``SparsePattern.build(q, k, causal)`` contract,
and CSR builders whose outputs are bit-identical to
``build_block_pairs_from_mask`` (``base.py:36-89``) and
``kv_block_list_to_pairs`` (``base.py:92-133``): int32 ``pairs [H, max(1,
max_nnz)]`` zero-padded, int32 ``offsets [H, NQB+1]``, ascending rows.

Unlike the reference, which loops over heads and rows on the host with a
device sync per row, these build the schedule with a few tensor ops on the
tensors' own device and one host sync (the padded width).
"""
from __future__ import annotations

from abc import ABC, abstractmethod
from dataclasses import dataclass

import torch
import torch.nn.functional as F


@dataclass
class PatternMetadata:
    """Output of :meth:`SparsePattern.build` (fields of ``base.py:11-33``).

    ``block_pairs`` / ``block_pair_offsets`` may carry one row per query head
    (the reference's layout) or one row per KV group, shared by the
    ``H / H_kv`` query heads of the group; the backends tell the two apart by
    the row count.
    """
    kind: str                                   # "dense" | "mask" | "topk" | "local"
    mask: torch.Tensor | None = None            # [H, T_q, T_k] bool, True = keep
    topk: int | None = None
    keep_ratio: float = 1.0
    build_time_ms: float = 0.0
    block_size: int | None = None
    kv_block_list: torch.Tensor | None = None   # [H, NQB, MAX_KV] int32, -1 = padding
    block_pairs: torch.Tensor | None = None     # [R, max_pairs] int32
    block_pair_offsets: torch.Tensor | None = None  # [R, NQB + 1] int32


class SparsePattern(ABC):
    """Which positions may attend (``base.py:136-154``)."""

    @abstractmethod
    def build(self, q: torch.Tensor, k: torch.Tensor, causal: bool = True) -> PatternMetadata:
        ...


def coarsen_token_mask(mask: torch.Tensor, block_size: int) -> torch.Tensor:
    """``[H, T_q, T_k]`` bool -> ``[H, NQB, NKB]``: a tile is active iff any token is."""
    H, T_q, T_k = mask.shape
    bs = int(block_size)
    nqb, nkb = -(-T_q // bs), -(-T_k // bs)
    m = F.pad(mask.to(torch.uint8), (0, nkb * bs - T_k, 0, nqb * bs - T_q))
    return m.reshape(H, nqb, bs, nkb, bs).amax(dim=(2, 4)).bool()


def _pack_flat(rows: torch.Tensor, vals: torch.Tensor, counts: torch.Tensor, nqb_counts: torch.Tensor):
    """Scatter per-row values (row-major order) into zero-padded ``[R, width]``."""
    R = counts.shape[0]
    device = counts.device
    width = max(1, int(counts.max().item())) if R else 1
    pairs = torch.zeros(R, width, dtype=torch.int32, device=device)
    if vals.numel():
        starts = torch.cumsum(counts, 0) - counts
        pos = torch.arange(vals.numel(), device=device) - starts[rows]
        pairs[rows, pos] = vals.to(torch.int32)
    offsets = torch.zeros(R, nqb_counts.shape[1] + 1, dtype=torch.int32, device=device)
    offsets[:, 1:] = torch.cumsum(nqb_counts, dim=1).to(torch.int32)
    return pairs, offsets


def block_mask_to_csr(block_active: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """``[R, NQB, NKB]`` bool -> ``(pairs, offsets)`` in the reference's CSR format.

    GPU masks go through the HIP builder (``ops.block_mask_to_csr_gpu``); CPU
    masks are packed with torch.  Both give the same bits.
    """
    if block_active.is_cuda:
        from ..ops import block_mask_to_csr_gpu
        return block_mask_to_csr_gpu(block_active)
    R, nqb, nkb = block_active.shape
    per_row = block_active.sum(dim=2)                       # [R, NQB]
    counts = per_row.sum(dim=1)                             # [R]
    nz = block_active.reshape(R, nqb * nkb).nonzero()       # row-major: (r, qb, kb) ascending
    return _pack_flat(nz[:, 0], nz[:, 1] % nkb, counts, per_row)


def build_block_pairs_from_mask(mask: torch.Tensor, block_size: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Token mask -> CSR; bit-identical to ``base.py:36-89``."""
    return block_mask_to_csr(coarsen_token_mask(mask, block_size))


def kv_block_list_to_pairs(kv_block_list: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Padded ``[H, NQB, MAX_KV]`` (-1 = pad) -> CSR; bit-identical to ``base.py:92-133``."""
    H, nqb, mk = kv_block_list.shape
    valid = kv_block_list >= 0
    per_row = valid.sum(dim=2)
    counts = per_row.sum(dim=1)
    nz = valid.reshape(H, nqb * mk).nonzero()
    vals = kv_block_list.reshape(H, nqb * mk)[nz[:, 0], nz[:, 1]]
    return _pack_flat(nz[:, 0], vals, counts, per_row)


def csr_to_block_mask(pairs: torch.Tensor, offsets: torch.Tensor, nkb: int) -> torch.Tensor:
    """Inverse of :func:`block_mask_to_csr` (rows must hold valid, unique ids)."""
    R, nqb1 = offsets.shape
    nqb = nqb1 - 1
    counts = (offsets[:, 1:] - offsets[:, :-1]).long()        # [R, NQB]
    total = counts.sum(dim=1)
    out = torch.zeros(R, nqb, nkb, dtype=torch.bool, device=pairs.device)
    if int(total.sum().item()) == 0:
        return out
    r_idx = torch.repeat_interleave(torch.arange(R, device=pairs.device), total)
    qb_idx = torch.repeat_interleave(torch.arange(nqb, device=pairs.device).repeat(R), counts.reshape(-1))
    starts = torch.repeat_interleave(torch.cumsum(total, 0) - total, total)
    pos = torch.arange(int(total.sum().item()), device=pairs.device) - starts
    out[r_idx, qb_idx, pairs[r_idx, pos].long()] = True
    return out


def causal_block_keep_ratio(offsets: torch.Tensor, T_q: int, T_k: int, block_size: int) -> float:
    """Kept pairs over the causal block triangle; ``bigbird_pattern.py:108-125``."""
    H = offsets.shape[0]
    nqb = offsets.shape[1] - 1
    nkb = -(-T_k // block_size)
    qbo = max(0, T_k - T_q) // block_size
    denom = sum(min(qbo + i + 1, nkb) for i in range(nqb))
    if denom <= 0:
        return 0.0
    kept = int(offsets[:, -1].long().sum().item())
    return min(1.0, kept / (H * denom))
