"""The seeded block-mask generators of the GPU pattern builder, restated in numpy.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The reference's BigBird "random" blocks are a hash (``sparse_attentions/patterns/
bigbird_pattern.py:23-41``), and its benchmark generators are not part of it; the
seeded BigBird and Bernoulli workloads of this build are drawn on the GPU from the
counter-based generator Philox4x64-10 (Salmon, Moraes, Dror and Shaw, "Parallel
random numbers: as easy as 1, 2, 3", SC'11).  This module restates:

* :func:`philox4x64` -- the generator (10 rounds, multipliers ``0xD2E7470EE14C6C93``,
  ``0xCA5A826395121157``, Weyl key increments ``0x9E3779B97F4A7C15``,
  ``0xBB67AE8584CAA73B``).  It is pinned against numpy's own ``numpy.random.Philox``
  (an independent C implementation of the same generator) in the tests;
* :func:`block_draws` -- the draw of block ``kb`` of query block ``qa`` in row ``row``:
  the first output word for counter ``(kb, qa, row, 0)`` and key ``(seed, stream)``;
* :func:`bernoulli_block_mask` and :func:`seeded_bigbird_block_mask` -- the masks the
  GPU kernels build from those draws (rules in ``include/sparse_attn.h``).
"""
from __future__ import annotations

import numpy as np

_M0 = np.uint64(0xD2E7470EE14C6C93)
_M1 = np.uint64(0xCA5A826395121157)
_W0 = np.uint64(0x9E3779B97F4A7C15)
_W1 = np.uint64(0xBB67AE8584CAA73B)
_LO32 = np.uint64(0xFFFFFFFF)
_S32 = np.uint64(32)

STREAM_BIGBIRD = 1
STREAM_BERNOULLI = 2


def _mulhilo(a: np.ndarray, b: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """High and low 64-bit words of the 128-bit product, from 32-bit limbs."""
    a0, a1 = a & _LO32, a >> _S32
    b0, b1 = b & _LO32, b >> _S32
    p00, p01, p10, p11 = a0 * b0, a0 * b1, a1 * b0, a1 * b1
    mid = (p00 >> _S32) + (p01 & _LO32) + (p10 & _LO32)
    hi = p11 + (p01 >> _S32) + (p10 >> _S32) + (mid >> _S32)
    return hi, a * b


def philox4x64(counter, key) -> list[np.ndarray]:
    """Philox4x64-10 of ``counter`` (4 uint64 arrays, broadcast) under ``key`` (2 uint64)."""
    c = [np.asarray(x, dtype=np.uint64) for x in np.broadcast_arrays(*counter)]
    k0 = np.uint64(key[0])
    k1 = np.uint64(key[1])
    with np.errstate(over="ignore"):
        for i in range(10):
            if i:
                k0 = k0 + _W0
                k1 = k1 + _W1
            hi0, lo0 = _mulhilo(_M0, c[0])
            hi1, lo1 = _mulhilo(_M1, c[2])
            c = [hi1 ^ c[1] ^ k0, lo1, hi0 ^ c[3] ^ k1, lo0]
    return c


def block_draws(seed: int, stream: int, rows: int, qa: np.ndarray, nkb: int) -> np.ndarray:
    """``[rows, len(qa), nkb]`` uint64: the draw of every (row, query block, key block)."""
    r = np.arange(rows, dtype=np.uint64)[:, None, None]
    q = np.asarray(qa, dtype=np.uint64)[None, :, None]
    kb = np.arange(nkb, dtype=np.uint64)[None, None, :]
    return philox4x64((kb, q, r, np.uint64(0)), (int(seed) & (2 ** 64 - 1), stream))[0]


def _causal_limit(nqb: int, nkb: int, q_block_offset: int) -> np.ndarray:
    return np.minimum(q_block_offset + np.arange(nqb), nkb - 1)


def bernoulli_block_mask(rows: int, nqb: int, nkb: int, *, density: float, seed: int,
                         q_block_offset: int = 0) -> np.ndarray:
    """Keep kb < qa where the draw's top 53 bits fall below floor(density * 2^53); keep qa."""
    qa = _causal_limit(nqb, nkb, q_block_offset)
    draws = block_draws(seed, STREAM_BERNOULLI, rows, qa, nkb)
    threshold = np.uint64(2 ** 53) if density >= 1.0 else np.uint64(np.floor(float(density) * 2.0 ** 53))
    kb = np.arange(nkb)[None, None, :]
    q = qa[None, :, None]
    return ((draws >> np.uint64(11)) < threshold) & (kb < q) | (kb == q)


def seeded_bigbird_block_mask(rows: int, nqb: int, nkb: int, *, window: int, global_blocks: int,
                              random_blocks, seed: int, window_align: str = "trailing",
                              q_block_offset: int = 0) -> np.ndarray:
    """Global prefix, window and diagonal (causal), plus the ``random_blocks[row]`` eligible
    blocks with the smallest (draw, kb)."""
    qa = _causal_limit(nqb, nkb, q_block_offset)
    kb = np.arange(nkb)[None, :]
    q = qa[:, None]
    if window_align == "trailing":
        lo, hi = q - window + 1, q
    else:
        lo, hi = q - window // 2, q + window // 2
    base = (((kb >= lo) & (kb <= hi)) | (kb < global_blocks) | (kb == q)) & (kb <= q)      # [NQB, NKB]
    counts = np.broadcast_to(np.asarray(random_blocks, dtype=np.int64).reshape(-1), (rows,))
    draws = block_draws(seed, STREAM_BIGBIRD, rows, qa, nkb)
    out = np.broadcast_to(base, (rows, nqb, nkb)).copy()
    eligible = (kb < q) & ~base
    for r in range(rows):
        for i in range(nqb):
            cand = np.nonzero(eligible[i])[0]
            if cand.size == 0 or counts[r] == 0:
                continue
            order = np.lexsort((cand, draws[r, i, cand]))          # by draw, then block id
            out[r, i, cand[order[:counts[r]]]] = True
    return out
