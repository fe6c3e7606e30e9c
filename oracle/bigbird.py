"""BigBird / local-window pattern semantics, restated on the CPU.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Every function follows one function of the reference's
``sparse_attentions/patterns/bigbird_pattern.py`` (cited per function) or
``local_window.py``.  The "random" blocks of the reference are not random: a
rotation of the candidate list by ``(131*head + 17*qb + 7*num_blocks) mod n``
(``bigbird_pattern.py:39``).  That formula is the reference's own table and is
kept literally, since bit-exact CSR parity depends on it.
"""
from __future__ import annotations

import math

import numpy as np

from oracle.csr import build_block_pairs_from_mask


# ----------------------------------------------------------------------------- layout helpers

def bigbird_layout_from_topk(seq_len: int, top_k: int) -> tuple[int, int, int, int]:
    """``(block_size, global, sliding, random)`` from a token budget; ``bigbird_pattern.py:12-20``."""
    if seq_len <= 1:
        return 1, 1, 1, 0
    bs = max(1, min(seq_len, int(math.sqrt(max(1, top_k)))))
    budget = max(1, -(-top_k // bs))
    sliding = min(2, budget)
    return bs, 1, sliding, max(0, budget - 1 - sliding)


def select_bigbird_random_block_ids(query_block: int, head_idx: int, num_blocks: int,
                                    global_blocks: int, sliding_blocks: int,
                                    random_blocks: int) -> list[int]:
    """Deterministic "random" block pick; ``bigbird_pattern.py:23-41``.

    Candidates are the blocks strictly between the global prefix and the
    sliding window; the list is rotated by the hash and its head is taken.
    """
    if random_blocks <= 0 or query_block <= 0:
        return []
    window_start = max(global_blocks, query_block - sliding_blocks + 1)
    cand = list(range(global_blocks, min(query_block, window_start)))
    if not cand:
        return []
    if len(cand) <= random_blocks:
        return cand
    rot = (head_idx * 131 + query_block * 17 + num_blocks * 7) % len(cand)
    return (cand[rot:] + cand[:rot])[:random_blocks]


def causal_token_pairs(seq_len: int) -> int:
    """``T (T + 1) / 2``; ``topk_pattern.py:105-106``."""
    return seq_len * (seq_len + 1) // 2


def estimate_bigbird_attention_keep_ratio(seq_len: int, top_k: int) -> float:
    """Token-level prefill keep ratio of head 0; ``bigbird_pattern.py:44-72``."""
    if seq_len <= 0:
        return 0.0
    if seq_len == 1:
        return 1.0
    bs, g, s, r = bigbird_layout_from_topk(seq_len, top_k)
    nb = -(-seq_len // bs)
    total = 0
    for pos in range(seq_len):
        qb = pos // bs
        vis = set(range(g)) | set(range(max(0, qb - s + 1), qb + 1))
        vis.update(select_bigbird_random_block_ids(qb, 0, nb, g, s, r))
        cnt = 0
        for b in vis:
            lo = b * bs
            hi = min(seq_len, (b + 1) * bs)
            cnt += max(0, min(hi, pos + 1) - lo)
        total += min(cnt, pos + 1)
    return min(1.0, total / max(1, causal_token_pairs(seq_len)))


def estimate_bigbird_decode_keep_ratio(seq_len: int, top_k: int) -> float:
    """Token-level keep ratio of the last query row; ``bigbird_pattern.py:75-94``."""
    if seq_len <= 0:
        return 0.0
    if seq_len == 1:
        return 1.0
    bs, g, s, r = bigbird_layout_from_topk(seq_len, top_k)
    nb = -(-seq_len // bs)
    qb = (seq_len - 1) // bs
    vis = set(range(g)) | set(range(max(0, qb - s + 1), qb + 1))
    vis.update(select_bigbird_random_block_ids(qb, 0, nb, g, s, r))
    tokens = sum(max(0, min(seq_len, (b + 1) * bs) - b * bs) for b in vis)
    return min(1.0, tokens / seq_len)


def next_pow2_min16(x: int) -> int:
    """Smallest power of two that is >= max(16, x); ``bigbird_pattern.py:99-105``."""
    p = max(16, x)
    return 1 << (p - 1).bit_length()


def causal_block_keep_ratio_from_offsets(offsets: np.ndarray, T_q: int, T_k: int,
                                         block_size: int) -> float:
    """Kept pairs over the causal block triangle; ``bigbird_pattern.py:108-125``."""
    offsets = np.asarray(offsets)
    H = offsets.shape[0]
    nqb = offsets.shape[1] - 1
    nkb = -(-T_k // block_size)
    qbo = max(0, T_k - T_q) // block_size
    denom = sum(min(qbo + i + 1, nkb) for i in range(nqb))
    if denom <= 0:
        return 0.0
    kept = int(offsets[:, -1].astype(np.int64).sum())
    return min(1.0, kept / (H * denom))


def bigbird_layout_from_keep_ratio(seq_len: int, keep_ratio: float, *, decode: bool,
                                   block_size: int | None = None) -> tuple[int, int, int, int]:
    """Layout from a target keep ratio; ``bigbird_pattern.py:338-363``."""
    if seq_len <= 1:
        return 1, 1, 1, 0
    kr = min(max(keep_ratio, 1.0 / seq_len), 1.0)
    if decode:
        target = max(1, math.ceil(kr * seq_len))
    else:
        target = max(1, math.ceil(kr * ((seq_len + 1) / 2)))
    if block_size is None:
        bs = max(1, min(seq_len, int(math.sqrt(max(1, target)))))
    else:
        bs = max(1, min(seq_len, int(block_size)))
    nb = -(-seq_len // bs)
    budget = max(1, min(nb, math.ceil(target / bs)))
    sliding = min(2, budget)
    return bs, 1, sliding, max(0, budget - 1 - sliding)


def keep_ratio_group_layouts(T_q: int, T_k: int, group_keep_ratios: tuple[float, ...]):
    """Per-group layouts of ``BigBirdKeepRatioPattern._layout``; ``bigbird_pattern.py:421-449``."""
    decode = T_q != T_k
    if len(group_keep_ratios) == 1:
        return (bigbird_layout_from_keep_ratio(T_k, group_keep_ratios[0], decode=decode),)
    desired = [bigbird_layout_from_keep_ratio(T_k, kr, decode=decode)[0] for kr in group_keep_ratios]
    shared = next_pow2_min16(min(desired))
    return tuple(bigbird_layout_from_keep_ratio(T_k, kr, decode=decode, block_size=shared)
                 for kr in group_keep_ratios)


# ----------------------------------------------------------------------------- per-row block sets

def _row_blocks(qb_abs: int, head: int, nkb: int, g: int, s: int, r: int) -> list[int]:
    """Sorted retained key blocks of one CSR row (``bigbird_pattern.py:246-255``)."""
    allowed = set(range(g))
    allowed.update(range(max(0, qb_abs - s + 1), min(qb_abs + 1, nkb)))
    allowed.update(select_bigbird_random_block_ids(qb_abs, head, nkb, g, s, r))
    return sorted(allowed)


def _pack(rows: list[list[list[int]]]):
    """Per-head list of per-row block lists -> zero-padded CSR (``bigbird_pattern.py:261-267``)."""
    H = len(rows)
    nqb = len(rows[0]) if H else 0
    flat = [[b for row in rows[h] for b in row] for h in range(H)]
    mp = max((len(f) for f in flat), default=0)
    pairs = np.zeros((H, max(1, mp)), dtype=np.int32)
    offsets = np.zeros((H, nqb + 1), dtype=np.int32)
    for h in range(H):
        if flat[h]:
            pairs[h, :len(flat[h])] = flat[h]
        offsets[h, 1:] = np.cumsum([len(row) for row in rows[h]], dtype=np.int64)
    return pairs, offsets


def _kv_list(rows: list[list[list[int]]], max_kv: int) -> np.ndarray:
    H = len(rows)
    nqb = len(rows[0]) if H else 0
    out = np.full((H, nqb, max_kv), -1, dtype=np.int32)
    for h in range(H):
        for qb in range(nqb):
            vals = rows[h][qb][:max_kv]
            out[h, qb, :len(vals)] = vals
    return out


def _token_mask_from_block_rows(block_mask: np.ndarray, q_rows_block: np.ndarray, bs: int,
                                T_q: int, T_k: int) -> np.ndarray:
    """``block_mask[:, q2b][:, :, k2b] & causal`` with the diagonal forced (``:196-207``)."""
    qbo_tok = max(0, T_k - T_q)
    q_pos = qbo_tok + np.arange(T_q)
    k2b = np.arange(T_k) // bs
    tm = block_mask[:, q_rows_block][:, :, k2b]
    tm = tm & (np.arange(T_k)[None, :] <= q_pos[:, None])[None]
    tm[:, np.arange(T_q), q_pos] = True
    return tm


# ----------------------------------------------------------------------------- BigBirdPattern

def bigbird_topk_schedule(T_q: int, T_k: int, top_k: int, n_heads: int):
    """``BigBirdPattern`` CSR, padded list and block size; ``bigbird_pattern.py:212-335``."""
    obs, g, s, r = bigbird_layout_from_topk(T_k, top_k)
    tbs = next_pow2_min16(obs)
    nqb = -(-T_q // tbs)
    nkb = -(-T_k // tbs)
    qbo = max(0, T_k - T_q) // tbs
    rows = [[_row_blocks(qbo + i, h, nkb, g, s, r) for i in range(nqb)] for h in range(n_heads)]
    pairs, offsets = _pack(rows)
    kv = _kv_list(rows, max(1, g + s + r))
    return pairs, offsets, kv, tbs


def bigbird_topk_token_mask(T_q: int, T_k: int, top_k: int, n_heads: int) -> np.ndarray:
    """``BigBirdPattern._get_mask``; ``bigbird_pattern.py:173-210``."""
    bs, g, s, r = bigbird_layout_from_topk(T_k, top_k)
    nb = -(-T_k // bs)
    bm = np.zeros((n_heads, nb, nb), dtype=bool)
    for h in range(n_heads):
        for qb in range(nb):
            bm[h, qb, :g] = True
            bm[h, qb, max(0, qb - s + 1):qb + 1] = True
            ids = select_bigbird_random_block_ids(qb, h, nb, g, s, r)
            if ids:
                bm[h, qb, ids] = True
    q_pos = max(0, T_k - T_q) + np.arange(T_q)
    return _token_mask_from_block_rows(bm, q_pos // bs, bs, T_q, T_k)


def bigbird_topk_keep_ratio(T_q: int, T_k: int, top_k: int, n_heads: int) -> float:
    _, offsets, _, tbs = bigbird_topk_schedule(T_q, T_k, top_k, n_heads)
    return causal_block_keep_ratio_from_offsets(offsets, T_q, T_k, tbs)


# ----------------------------------------------------------------------------- BigBirdKeepRatioPattern

def keep_ratio_group_keep_ratios(keep_ratio=None, group_sparsities=None) -> tuple[float, ...]:
    """``bigbird_pattern.py:377-399``."""
    if (keep_ratio is None) == (group_sparsities is None):
        raise ValueError("exactly one of keep_ratio / group_sparsities")
    if group_sparsities is not None:
        return tuple(1.0 - float(x) for x in group_sparsities)
    return (float(keep_ratio),)


def bigbird_keep_ratio_schedule(T_q: int, T_k: int, n_heads: int, group_keep_ratios):
    """CSR + padded list of ``BigBirdKeepRatioPattern``; ``bigbird_pattern.py:533-634``."""
    layouts = keep_ratio_group_layouts(T_q, T_k, tuple(group_keep_ratios))
    gsize = n_heads // len(layouts)
    tbs = next_pow2_min16(layouts[0][0])
    nqb = -(-T_q // tbs)
    nkb = -(-T_k // tbs)
    qbo = max(0, T_k - T_q) // tbs
    rows = []
    for h in range(n_heads):
        _, g, s, r = layouts[h // gsize]
        rows.append([_row_blocks(qbo + i, h, nkb, g, s, r) for i in range(nqb)])
    pairs, offsets = _pack(rows)
    max_kv = max(1, max(g + s + r for _, g, s, r in layouts))
    return pairs, offsets, _kv_list(rows, max_kv), tbs, layouts


def bigbird_keep_ratio_token_mask(T_q: int, T_k: int, n_heads: int, group_keep_ratios) -> np.ndarray:
    """``BigBirdKeepRatioPattern._get_mask``; ``bigbird_pattern.py:487-531``."""
    layouts = keep_ratio_group_layouts(T_q, T_k, tuple(group_keep_ratios))
    gsize = n_heads // len(layouts)
    qoff = max(0, T_k - T_q)
    q_pos = qoff + np.arange(T_q)
    causal = np.arange(T_k)[None, :] <= q_pos[:, None]
    tm = np.zeros((n_heads, T_q, T_k), dtype=bool)
    for h in range(n_heads):
        bs, g, s, r = layouts[h // gsize]
        nb = -(-T_k // bs)
        nqb = -(-T_q // bs)
        qbo = qoff // bs
        bm = np.zeros((nqb, nb), dtype=bool)
        for i in range(nqb):
            qa = qbo + i
            bm[i, :g] = True
            bm[i, max(0, qa - s + 1):min(qa + 1, nb)] = True
            ids = select_bigbird_random_block_ids(qa, h, nb, g, s, r)
            if ids:
                bm[i, ids] = True
        tm[h] = bm[np.arange(T_q) // bs][:, np.arange(T_k) // bs] & causal
    tm[:, np.arange(T_q), q_pos] = True
    return tm


# ----------------------------------------------------------------------------- BigBird2Pattern

def bigbird2_schedule(T_q: int, T_k: int, top_k: int, n_heads: int):
    """``BigBird2Pattern`` CSR + padded list; ``bigbird_pattern.py:697-806``."""
    obs, g, s, r = bigbird_layout_from_topk(T_k, top_k)
    tbs = next_pow2_min16(obs)
    nqb = -(-T_q // tbs)
    nkb = -(-T_k // tbs)
    qbo = max(0, T_k - T_q) // tbs
    rows = []
    for h in range(n_heads):
        rows.append([list(range(nkb)) if i == nqb - 1 else _row_blocks(qbo + i, h, nkb, g, s, r)
                     for i in range(nqb)])
    pairs, offsets = _pack(rows)
    kv = _kv_list(rows, max(nkb, g + s + r))
    return pairs, offsets, kv, tbs


def bigbird2_token_mask(T_q: int, T_k: int, top_k: int, n_heads: int) -> np.ndarray:
    """``BigBird2Pattern._get_mask``; ``bigbird_pattern.py:648-695``."""
    bs, g, s, r = bigbird_layout_from_topk(T_k, top_k)
    nb = -(-T_k // bs)
    qoff = max(0, T_k - T_q)
    nqb = -(-T_q // bs)
    bm = np.zeros((n_heads, nqb, nb), dtype=bool)
    for h in range(n_heads):
        for i in range(nqb):
            qa = qoff // bs + i
            if i == nqb - 1:
                bm[h, i, :] = True
            else:
                bm[h, i, :g] = True
                bm[h, i, max(0, qa - s + 1):qa + 1] = True
                ids = select_bigbird_random_block_ids(qa, h, nb, g, s, r)
                if ids:
                    bm[h, i, ids] = True
    return _token_mask_from_block_rows(bm, np.arange(T_q) // bs, bs, T_q, T_k)


# ----------------------------------------------------------------------------- LocalWindowPattern

def local_window_token_mask(T_q: int, T_k: int, H: int, window: int, causal: bool = True) -> np.ndarray:
    """``LocalWindowPattern._build_mask``; ``local_window.py:58-71``."""
    rows = (max(0, T_k - T_q) + np.arange(T_q))[:, None]
    cols = np.arange(T_k)[None, :]
    keep = (cols >= rows - window + 1) & (cols <= rows)
    return np.broadcast_to(keep, (H, T_q, T_k)).copy()


def local_window_keep_ratio(T_q: int, T_k: int, window: int) -> float:
    """``local_window.py:73-80``."""
    if T_q == 0 or T_k == 0:
        return 0.0
    qoff = max(0, T_k - T_q)
    return min(1.0, sum(min(window, qoff + i + 1) for i in range(T_q)) / (T_q * T_k))


def local_window_schedule(T_q: int, T_k: int, H: int, window: int, block_size: int):
    """CSR of ``LocalWindowPattern`` with a block size; ``local_window.py:42-47``."""
    return build_block_pairs_from_mask(local_window_token_mask(T_q, T_k, H, window), block_size)
