"""CSR block schedule construction, restated on the CPU with numpy.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Format (``sparse_attentions/patterns/base.py:26-33``): for head ``h`` and query
block ``qb``, the retained key blocks are
``pairs[h, offsets[h, qb]:offsets[h, qb + 1]]``, ascending.  ``pairs`` is
int32 ``[H, max(1, max_nnz)]`` zero-padded on the right, ``offsets`` int32
``[H, NQB + 1]``.
"""
from __future__ import annotations

import numpy as np


def coarsen_token_mask(mask: np.ndarray, block_size: int) -> np.ndarray:
    """``[H, T_q, T_k]`` bool -> ``[H, NQB, NKB]``: a tile is active iff any token is.

    Follows ``sparse_attentions/patterns/base.py:53-64`` (zero-pad to whole
    blocks, then ``any`` over each ``BS x BS`` tile).
    """
    mask = np.asarray(mask, dtype=bool)
    H, T_q, T_k = mask.shape
    bs = int(block_size)
    nqb = -(-T_q // bs)
    nkb = -(-T_k // bs)
    padded = np.zeros((H, nqb * bs, nkb * bs), dtype=bool)
    padded[:, :T_q, :T_k] = mask
    return padded.reshape(H, nqb, bs, nkb, bs).any(axis=(2, 4))


def _pack_rows(rows_per_head: list[list[int]], offsets_per_head: list[list[int]], nqb: int):
    """Zero-padded packing of ``base.py:81-89``."""
    H = len(rows_per_head)
    max_pairs = max((len(r) for r in rows_per_head), default=0)
    pairs = np.zeros((H, max(1, max_pairs)), dtype=np.int32)
    offsets = np.zeros((H, nqb + 1), dtype=np.int32)
    for h in range(H):
        n = len(rows_per_head[h])
        if n:
            pairs[h, :n] = np.asarray(rows_per_head[h], dtype=np.int32)
        offsets[h] = np.asarray(offsets_per_head[h], dtype=np.int32)
    return pairs, offsets


def csr_from_block_mask(block_active: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """``[H, NQB, NKB]`` bool -> ``(pairs, offsets)``; rows in ascending key-block order.

    Follows the per-head, per-row loop of ``base.py:66-79``.
    """
    block_active = np.asarray(block_active, dtype=bool)
    H, nqb, _ = block_active.shape
    rows, offs = [], []
    for h in range(H):
        row_h: list[int] = []
        off_h = [0]
        for qb in range(nqb):
            row_h.extend(int(x) for x in np.flatnonzero(block_active[h, qb]))
            off_h.append(len(row_h))
        rows.append(row_h)
        offs.append(off_h)
    return _pack_rows(rows, offs, nqb)


def build_block_pairs_from_mask(mask: np.ndarray, block_size: int) -> tuple[np.ndarray, np.ndarray]:
    """Token mask -> CSR, restating ``base.py:36-89``."""
    return csr_from_block_mask(coarsen_token_mask(mask, block_size))


def kv_block_list_to_pairs(kv_block_list: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Padded ``[H, NQB, MAX_KV]`` list (-1 = pad) -> CSR, restating ``base.py:92-133``.

    Entries are kept in their stored order with the -1 slots dropped, wherever
    they sit in the row.
    """
    kv = np.asarray(kv_block_list)
    H, nqb, _ = kv.shape
    rows, offs = [], []
    for h in range(H):
        row_h: list[int] = []
        off_h = [0]
        for qb in range(nqb):
            vals = kv[h, qb]
            row_h.extend(int(x) for x in vals[vals >= 0])
            off_h.append(len(row_h))
        rows.append(row_h)
        offs.append(off_h)
    return _pack_rows(rows, offs, nqb)


def brute_force_block_pairs(mask, block_size: int):
    """Pure-Python token loop: the definition of "a tile is active iff any token is".

    Used only to pin :func:`build_block_pairs_from_mask` on small masks.
    Returns plain lists ``(rows, offsets)`` per head, without padding.
    """
    H = len(mask)
    T_q = len(mask[0]) if H else 0
    T_k = len(mask[0][0]) if T_q else 0
    bs = block_size
    nqb = -(-T_q // bs)
    nkb = -(-T_k // bs)
    all_rows, all_offs = [], []
    for h in range(H):
        row_h, off_h = [], [0]
        for qb in range(nqb):
            for kb in range(nkb):
                hit = False
                for i in range(qb * bs, min(T_q, (qb + 1) * bs)):
                    for j in range(kb * bs, min(T_k, (kb + 1) * bs)):
                        if mask[h][i][j]:
                            hit = True
                            break
                    if hit:
                        break
                if hit:
                    row_h.append(kb)
            off_h.append(len(row_h))
        all_rows.append(row_h)
        all_offs.append(off_h)
    return all_rows, all_offs


def csr_to_block_mask(pairs: np.ndarray, offsets: np.ndarray, nkb: int) -> np.ndarray:
    """Inverse of :func:`csr_from_block_mask` for sorted, unique rows."""
    pairs = np.asarray(pairs)
    offsets = np.asarray(offsets)
    H, nqb1 = offsets.shape
    out = np.zeros((H, nqb1 - 1, nkb), dtype=bool)
    for h in range(H):
        for qb in range(nqb1 - 1):
            s, e = int(offsets[h, qb]), int(offsets[h, qb + 1])
            out[h, qb, pairs[h, s:e]] = True
    return out
