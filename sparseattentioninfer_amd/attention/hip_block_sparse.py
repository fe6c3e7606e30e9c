"""``hip_block_sparse``: the gfx950 block-sparse backend.

Drop-in for ``TritonUniversalBackend`` / ``TritonBigBirdBackend``
(``sparse_attentions/attention/triton_universal_backend.py:24-103``,
``triton_bigbird_backend.py:21-102``): same ``forward(q, k, v, pattern)``
signature and ``actual_backend`` property, and it consumes the same
``PatternMetadata`` fields (CSR ``block_pairs``/``block_pair_offsets``, or the
padded ``kv_block_list``, plus ``block_size``).

Differences from the reference, all deliberate:

* Fallback only when the caller supplies one.  The reference's Triton backends
  run ``MaskedSdpaBackend`` for inputs their kernel cannot take (CPU tensors,
  dtypes other than fp16/bf16, no block schedule or block size) and report
  ``actual_backend == "masked_sdpa_fallback"``
  (``triton_universal_backend.py:47-66``).  This backend does the same for
  exactly those inputs (and top-k patterns) when it is constructed with
  ``fallback=`` -- inside the reference, its own ``MaskedSdpaBackend`` class,
  injected by :func:`~sparseattentioninfer_amd.attention.register_into`.
  Without one it raises.  A missing or broken HIP library is never a reason to
  fall back: GPU fp16/bf16 inputs with a schedule always run the kernels or
  raise.
* ``k``/``v`` may carry ``H_kv < H`` heads (grouped-query attention); the
  caller need not ``repeat_kv``.  A CSR with ``H_kv`` rows is shared by the
  query heads of each KV group, letting one K/V tile feed all of them.
* ``kind == "dense"`` runs the kernels over a full causal schedule
  (bottom-right aligned: the query is the last ``T_q`` positions).

Schedules derived from a pattern's tensors (the CSR of a padded list, the
64 x 64 tile schedule of a block-16/32 CSR) are computed once and reused while
the same tensors, unmodified, come back -- the reference's patterns hand every
layer the same metadata.
"""
from __future__ import annotations

import torch

from .. import ops
from ..patterns.base import PatternMetadata, block_mask_to_csr, kv_block_list_to_pairs
from .base import AttentionBackend

_DENSE_BLOCK = 64
_DERIVED_CACHE_SIZE = 8


class _DerivedCache:
    """Small LRU of schedules derived from tensors.

    An entry holds its source tensors, so their memory cannot be reused by
    another tensor while it is cached; it is valid while the same objects come
    back with unchanged version counters (no in-place writes since).
    """

    def __init__(self, size: int = _DERIVED_CACHE_SIZE):
        self._size = size
        self._entries: list = []   # (sources, versions, extra key, value), most recent last

    def get(self, sources: tuple, extra, make):
        versions = tuple(t._version for t in sources)
        for i, (src, ver, ex, val) in enumerate(self._entries):
            if ex == extra and ver == versions and len(src) == len(sources) \
                    and all(a is b for a, b in zip(src, sources)):
                self._entries.append(self._entries.pop(i))
                return val
        val = make()
        self._entries.append((sources, versions, extra, val))
        if len(self._entries) > self._size:
            self._entries.pop(0)
        return val


class HipBlockSparseBackend(AttentionBackend):
    """Block-sparse attention on hand-written HIP kernels for gfx950."""

    supports_gqa = True   # k/v may carry H_kv < H heads; callers need not repeat them
    FALLBACK_NAME = "masked_sdpa_fallback"
    # Backend class or instance used for inputs the kernels cannot take; subclasses made by
    # register_into(..., fallback=cls) set it, so the registry's no-argument construction has it.
    default_fallback = None

    def __init__(self, fallback=None):
        fb = fallback if fallback is not None else self.default_fallback
        self._fallback = fb() if isinstance(fb, type) else fb
        self._last_actual_backend = "unknown"
        self.last_kernel = None          # "prefill" or "decode" after a forward
        self._dense_cache: dict = {}
        self._list_cache = _DerivedCache()
        self._tile_cache = _DerivedCache()

    @property
    def actual_backend(self) -> str:
        return self._last_actual_backend

    def _dense_schedule(self, T_q: int, T_k: int, rows: int, device) -> tuple:
        """Full causal schedule: query block qb keeps key blocks 0 .. the block of its last
        row's absolute position (``T_k - T_q`` need not be a multiple of the block).  It
        depends on the shape only through those limits, so decode steps inside one KV block
        share it."""
        bs = _DENSE_BLOCK
        nqb, nkb = -(-T_q // bs), -(-T_k // bs)
        off = T_k - T_q
        last = tuple(min((off + min((qb + 1) * bs, T_q) - 1) // bs, nkb - 1) for qb in range(nqb))
        key = (nkb, last, rows, str(device))
        hit = self._dense_cache.get(key)
        if hit is None:
            qa = torch.tensor(last, dtype=torch.long)
            bm = (torch.arange(nkb)[None, :] <= qa[:, None])[None].expand(rows, nqb, nkb)
            pairs, offsets = block_mask_to_csr(bm.contiguous())
            hit = (pairs.to(device), offsets.to(device), bs)
            self._dense_cache[key] = hit
            if len(self._dense_cache) > _DERIVED_CACHE_SIZE:
                self._dense_cache.pop(next(iter(self._dense_cache)))
        return hit

    def _list_schedule(self, kv_block_list: torch.Tensor) -> tuple:
        return self._list_cache.get((kv_block_list,), None, lambda: kv_block_list_to_pairs(kv_block_list))

    def _tiles(self, pairs: torch.Tensor, offsets: torch.Tensor, bs: int):
        if bs >= 64 or not pairs.is_cuda or pairs.dtype != torch.int32 or offsets.dtype != torch.int32:
            return None   # ops validates and reports what is wrong
        # validated once per schedule (one synchronisation), then reused
        return self._tile_cache.get((pairs, offsets), bs, lambda: ops.csr_to_tiles(pairs, offsets, bs).check())

    def _schedule(self, T_q: int, T_k: int, kv_heads: int, device, pattern: PatternMetadata) -> tuple:
        if pattern.kind == "dense":
            return self._dense_schedule(T_q, T_k, kv_heads, device)
        if pattern.kind in ("mask", "local"):
            bs = pattern.block_size
            if bs is None:
                raise ValueError("hip_block_sparse needs a block-sparse schedule; pattern.block_size is None")
            if pattern.block_pairs is not None and pattern.block_pair_offsets is not None:
                pairs, offsets = pattern.block_pairs, pattern.block_pair_offsets
            elif pattern.kv_block_list is not None:
                pairs, offsets = self._list_schedule(pattern.kv_block_list)
            else:
                raise ValueError("hip_block_sparse needs block_pairs/block_pair_offsets or kv_block_list")
            return pairs, offsets, bs
        raise NotImplementedError(
            f"hip_block_sparse does not run pattern kind {pattern.kind!r} (data-dependent top-k "
            "selection is not a block schedule)")

    @staticmethod
    def unsupported_reason(q: torch.Tensor, pattern: PatternMetadata):
        """Why the kernels cannot take these inputs (the reference backends' fallback conditions,
        ``triton_universal_backend.py:54-61``, plus head dims other than 64 and 128 and top-k
        patterns), or None when they can."""
        if not q.is_cuda:
            return "a CPU tensor"
        if q.dtype not in (torch.float16, torch.bfloat16):
            return f"dtype {q.dtype} (the kernels take float16 and bfloat16)"
        if q.size(-1) not in (64, 128):
            return f"head dim {q.size(-1)} (the kernels take 64 and 128)"
        if pattern.kind in ("mask", "local"):
            if pattern.block_size is None:
                return "pattern.block_size is None"
            if (pattern.block_pairs is None or pattern.block_pair_offsets is None) and pattern.kv_block_list is None:
                return "no block schedule (block_pairs/block_pair_offsets or kv_block_list)"
        elif pattern.kind != "dense":
            return f"pattern kind {pattern.kind!r} (data-dependent top-k selection is not a block schedule)"
        return None

    def _run_fallback(self, q, k, v, pattern, reason: str) -> torch.Tensor:
        if self._fallback is None:
            if not q.is_cuda:
                raise RuntimeError("hip_block_sparse runs on ROCm GPU tensors only; got a CPU tensor "
                                   "(no fallback backend was given)")
            if pattern.kind not in ("mask", "local", "dense"):
                raise NotImplementedError(f"hip_block_sparse does not run {reason}; no fallback backend was given")
            raise ValueError(f"hip_block_sparse cannot run {reason}; no fallback backend was given")
        # The reference's backends take K/V with the query's head count (its callers repeat them).
        n_rep = q.size(1) // k.size(1)
        if n_rep > 1:
            k = k[:, :, None].expand(-1, -1, n_rep, -1, -1).reshape(q.size(0), q.size(1), k.size(2), k.size(3))
            v = v[:, :, None].expand(-1, -1, n_rep, -1, -1).reshape(q.size(0), q.size(1), v.size(2), v.size(3))
        self._last_actual_backend = self.FALLBACK_NAME
        self.last_kernel = None
        return self._fallback.forward(q, k, v, pattern)

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                pattern: PatternMetadata) -> torch.Tensor:
        reason = self.unsupported_reason(q, pattern)
        if reason is not None:
            return self._run_fallback(q, k, v, pattern, reason)
        pairs, offsets, bs = self._schedule(q.size(2), k.size(2), k.size(1), q.device, pattern)
        tiles = self._tiles(pairs, offsets, bs) if q.size(2) > 1 else None
        out = ops.universal_sparse_attn(q, k, v, pairs, offsets, bs, tiles=tiles)
        self.last_kernel = "decode" if q.size(2) == 1 else "prefill"
        self._last_actual_backend = "hip_block_sparse"
        return out

    def forward_paged(self, q: torch.Tensor, store, pattern: PatternMetadata) -> torch.Tensor:
        """One decode token per sequence (``q [B, H, 1, D]``) against a paged store.

        ``store`` is a :class:`~sparseattentioninfer_amd.models.kv_cache.PagedKVStore` already
        holding the new token; the pattern's single CSR query block (the row of the last
        position) is shared by the batch, and its block size must equal the page size.
        """
        if not q.is_cuda:
            raise RuntimeError("hip_block_sparse runs on ROCm GPU tensors only")
        if q.size(2) != 1:
            raise ValueError(f"forward_paged decodes one token per sequence; got T_q={q.size(2)}")
        pairs, offsets, bs = self._schedule(1, store.seq_len(), store.heads, q.device, pattern)
        if bs != store.page:
            raise ValueError(f"schedule block {bs} differs from the cache page {store.page}")
        if offsets.size(1) != 2:
            raise ValueError(f"decode expects one CSR query block, got {offsets.size(1) - 1}")
        B, R = q.size(0), pairs.size(0)
        sel = pairs.contiguous()[None].expand(B, R, pairs.size(1))
        sel_off = offsets.contiguous()[None].expand(B, R, 2)
        out = ops.paged_sparse_decode(q, store.k_pages, store.v_pages, store.block_table, store.kv_lens,
                                      sel, sel_off, num_splits=0)
        self.last_kernel = "decode"
        self._last_actual_backend = "hip_block_sparse"
        return out
