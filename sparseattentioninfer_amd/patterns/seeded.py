"""Seeded block-mask generators for the benchmark workloads.

The reference's BigBird "random" blocks are a deterministic hash
(``sparse_attentions/patterns/bigbird_pattern.py:23-41``); the workloads this
build is measured on instead draw random blocks from a seeded generator, and
use per-KV-group masks shared by the query heads of a group.  Masks are
generated at block level ``[R, NQB, NKB]``, then turned into the reference's
CSR format by :func:`block_mask_to_csr`: by default on the CPU with a
``torch.Generator`` (reproducible across machines; the committed benchmark
workloads use it), or with ``rng="philox"`` on the query's GPU by the HIP
generators (``ops.seeded_bigbird_block_mask_gpu`` / ``bernoulli_block_mask_gpu``,
Philox4x64-10), with the CSR built there too -- no host round trip but the
one read of the CSR width.

Rows here are CSR rows: one per KV group when the pattern is group-shared.
"""
from __future__ import annotations

from collections import OrderedDict

import torch

from .base import PatternMetadata, SparsePattern, block_mask_to_csr


def _causal_limit(nqb: int, nkb: int, q_block_offset: int) -> torch.Tensor:
    """Absolute query block index per row, clipped to the last key block."""
    return (q_block_offset + torch.arange(nqb)).clamp(max=nkb - 1)


def _pick_random(eligible: torch.Tensor, counts: torch.Tensor, gen: torch.Generator) -> torch.Tensor:
    """Uniformly choose ``counts[r]`` eligible blocks per (r, qb) row, without replacement.

    Rows with fewer eligible blocks take all of them.  ``eligible [R,NQB,NKB]``.
    """
    R, nqb, nkb = eligible.shape
    keys = torch.rand(R, nqb, nkb, generator=gen)
    keys = torch.where(eligible, keys, torch.full_like(keys, -1.0))
    kmax = int(counts.max().item()) if counts.numel() else 0
    out = torch.zeros_like(eligible)
    if kmax == 0:
        return out
    top = torch.topk(keys, k=min(kmax, nkb), dim=2)
    take = (torch.arange(top.indices.shape[2])[None, None, :] < counts[:, None, None]) & (top.values >= 0)
    out.scatter_(2, top.indices, take)
    return out


def seeded_bigbird_block_mask(rows: int, nqb: int, nkb: int, *, window: int, global_blocks: int,
                              random_blocks, seed: int, window_align: str = "trailing",
                              q_block_offset: int = 0) -> torch.Tensor:
    """BigBird rows: global prefix, sliding window, seeded random; causal-truncated.

    * ``window_align="trailing"``: the window is ``{qb-window+1 .. qb}`` (the
      reference's ``local_start = qb - sliding + 1``, ``bigbird_pattern.py:248``);
      ``"centred"``: ``{qb - window//2 .. qb + window//2}`` before truncation.
    * ``random_blocks``: an int, or one count per row (per KV group), drawn
      from the causal blocks outside the global prefix and the window.
    * every row keeps its diagonal block; nothing above the diagonal is kept.
    """
    if window_align not in ("trailing", "centred"):
        raise ValueError(f"window_align must be 'trailing' or 'centred', got {window_align!r}")
    gen = torch.Generator().manual_seed(int(seed))
    qa = _causal_limit(nqb, nkb, q_block_offset)[:, None]             # [NQB, 1]
    kb = torch.arange(nkb)[None, :]                                    # [1, NKB]
    causal = kb <= qa
    if window_align == "trailing":
        lo, hi = qa - window + 1, qa
    else:
        lo, hi = qa - window // 2, qa + window // 2
    win = (kb >= lo) & (kb <= hi)
    glob = kb < global_blocks
    base = (win | glob | (kb == qa)) & causal                         # [NQB, NKB]
    base = base[None].expand(rows, nqb, nkb)
    counts = torch.as_tensor(random_blocks, dtype=torch.long).reshape(-1)
    if counts.numel() == 1:
        counts = counts.expand(rows)
    if counts.numel() != rows:
        raise ValueError(f"random_blocks has {counts.numel()} entries for {rows} rows")
    eligible = causal[None] & ~base
    return base | _pick_random(eligible, counts, gen)


def bernoulli_block_mask(rows: int, nqb: int, nkb: int, *, density: float, seed: int,
                         q_block_offset: int = 0) -> torch.Tensor:
    """Independent Bernoulli(density) over strictly-lower causal blocks, diagonal kept."""
    gen = torch.Generator().manual_seed(int(seed))
    qa = _causal_limit(nqb, nkb, q_block_offset)[:, None]
    kb = torch.arange(nkb)[None, :]
    draw = torch.rand(rows, nqb, nkb, generator=gen) < density
    return (draw & (kb < qa)[None]) | (kb == qa)[None]


class _BlockMaskPattern(SparsePattern):
    """Shared plumbing: block mask -> PatternMetadata.

    The CSR depends on the shape only through the block counts (nqb, nkb) and
    the query block offset, so decode steps inside one KV block reuse it; the
    device copies live in a small LRU keyed that way.  The keep ratio is
    computed from host-side counts, so ``build`` never waits for the GPU.
    """

    CACHE_SIZE = 32

    def __init__(self, block_size: int, rows: int, rng: str = "torch"):
        if rng not in ("torch", "philox"):
            raise ValueError(f"rng must be 'torch' (CPU generator) or 'philox' (GPU generator), got {rng!r}")
        self.block_size = int(block_size)
        self.rows = int(rows)
        self.rng = rng
        self._cache: OrderedDict = OrderedDict()

    def _block_mask(self, nqb: int, nkb: int, q_block_offset: int, device) -> torch.Tensor:
        raise NotImplementedError

    def _device_for(self, device: torch.device):
        """Where the block mask is generated: the CPU generator's masks on the CPU, the Philox
        generator's on the query's GPU (it has no CPU implementation in the product)."""
        if self.rng == "torch":
            return torch.device("cpu")
        if device.type != "cuda":
            raise RuntimeError("rng='philox' generates block masks on the GPU; the query is on "
                               f"{device.type}")
        return device

    def build(self, q: torch.Tensor, k: torch.Tensor, causal: bool = True) -> PatternMetadata:
        T_q, T_k = q.size(2), k.size(2)
        bs = self.block_size
        nqb, nkb, qbo = -(-T_q // bs), -(-T_k // bs), max(0, T_k - T_q) // bs
        key = (nqb, nkb, qbo, str(q.device))
        entry = self._cache.get(key)
        if entry is None:
            pairs, offsets = block_mask_to_csr(self._block_mask(nqb, nkb, qbo, self._device_for(q.device)))
            kept = int(offsets[:, -1].long().sum())
            entry = (pairs.to(q.device), offsets.to(q.device), kept)
            self._cache[key] = entry
            if len(self._cache) > self.CACHE_SIZE:
                self._cache.popitem(last=False)
        else:
            self._cache.move_to_end(key)
        pairs, offsets, kept = entry
        denom = sum(min(qbo + i + 1, nkb) for i in range(nqb)) * self.rows
        kr = min(1.0, kept / denom) if denom > 0 else 0.0
        return PatternMetadata(kind="mask", keep_ratio=kr, block_size=bs,
                               block_pairs=pairs, block_pair_offsets=offsets)


class SeededBigBirdPattern(_BlockMaskPattern):
    """BigBird with seeded random blocks; ``rows`` CSR rows (Hq, or Hkv for group sharing)."""

    def __init__(self, *, rows: int, block_size: int = 64, window: int = 3, global_blocks: int = 2,
                 random_blocks=3, seed: int = 0, window_align: str = "trailing", rng: str = "torch"):
        super().__init__(block_size, rows, rng)
        self.window, self.global_blocks = window, global_blocks
        self.random_blocks, self.seed, self.window_align = random_blocks, seed, window_align

    def _block_mask(self, nqb, nkb, qbo, device):
        if self.rng == "philox":
            from .. import ops
            return ops.seeded_bigbird_block_mask_gpu(self.rows, nqb, nkb, window=self.window,
                                                     global_blocks=self.global_blocks,
                                                     random_blocks=self.random_blocks, seed=self.seed,
                                                     window_align=self.window_align, q_block_offset=qbo,
                                                     device=device)
        return seeded_bigbird_block_mask(self.rows, nqb, nkb, window=self.window,
                                         global_blocks=self.global_blocks,
                                         random_blocks=self.random_blocks, seed=self.seed,
                                         window_align=self.window_align, q_block_offset=qbo)


class BernoulliBlockPattern(_BlockMaskPattern):
    """Arbitrary-pattern workload: Bernoulli(density) blocks per CSR row, diagonal kept."""

    def __init__(self, *, rows: int, density: float, block_size: int = 64, seed: int = 0, rng: str = "torch"):
        super().__init__(block_size, rows, rng)
        self.density, self.seed = density, seed

    def _block_mask(self, nqb, nkb, qbo, device):
        if self.rng == "philox":
            from .. import ops
            return ops.bernoulli_block_mask_gpu(self.rows, nqb, nkb, density=self.density, seed=self.seed,
                                                q_block_offset=qbo, device=device)
        return bernoulli_block_mask(self.rows, nqb, nkb, density=self.density, seed=self.seed,
                                    q_block_offset=qbo)


def decode_selection(batch: int, rows: int, num_blocks, *, local: int, global_blocks: int,
                     random_blocks: int, seed: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-(sequence, row) retained logical blocks for one decode step.

    Keeps the last ``local`` blocks, the first ``global_blocks`` and
    ``random_blocks`` seeded-random blocks from the rest.  ``num_blocks`` is an
    int or one count per sequence.  Returns ``sel [B, rows, max_sel]`` int32
    (ascending ids, zero-padded) and ``sel_off [B, rows, 2]`` int32
    (``[start, end)`` into the row).
    """
    gen = torch.Generator().manual_seed(int(seed))
    nb = torch.as_tensor(num_blocks, dtype=torch.long).reshape(-1)
    if nb.numel() == 1:
        nb = nb.expand(batch)
    nmax = int(nb.max().item())
    kb = torch.arange(nmax)[None, None, :]
    n = nb[:, None, None]
    base = ((kb >= n - local) | (kb < global_blocks)) & (kb < n)
    base = base.expand(batch, rows, nmax)
    eligible = (kb < n) & ~base
    bm = base | _pick_random(eligible.reshape(batch * rows, 1, nmax),
                             torch.full((batch * rows,), random_blocks), gen).reshape(batch, rows, nmax)
    counts = bm.sum(dim=2)
    width = max(1, int(counts.max().item()))
    sel = torch.zeros(batch, rows, width, dtype=torch.int32)
    order = torch.sort(torch.where(bm, kb.expand_as(bm), nmax + kb.expand_as(bm)), dim=2).values
    sel[:, :, :] = torch.where(order[:, :, :width] < nmax, order[:, :, :width], torch.zeros_like(order[:, :, :width])).to(torch.int32)
    sel_off = torch.zeros(batch, rows, 2, dtype=torch.int32)
    sel_off[:, :, 1] = counts.to(torch.int32)
    return sel, sel_off
