"""KV caches for decoding: the reference's per-layer ``KVCache`` API over preallocated storage, and
a paged cache (page pool + block table) that the paged decode kernel reads directly.

``KVCache`` keeps the method names and meaning of
``sparse_attentions/models/kv_cache.py:7-59`` (``init``, ``clone``, ``append``,
``seq_len``, ``clear``) but stores each layer in a ``[B, H, capacity, D]`` buffer:
``append`` writes the new tokens in place and returns ``[B, H, T, D]`` views
(head dim contiguous, token stride D), where the reference concatenates and
copies the whole cache on every step.  The capacity grows by doubling (one
copy) only when exceeded.

``PagedKVStore`` holds one layer's pages ``[P, H, page, D]``, a block table
``[B, max_blocks]`` (logical block -> page) and the sequence lengths; pages
are taken from a free list as sequences grow.  It is the layout
``sa_decode`` reads in paged mode.
"""
from __future__ import annotations

import torch


def _round_up(x: int, m: int) -> int:
    return -(-x // m) * m


class KVCache:
    """Per-layer KV cache for autoregressive decoding (reference API, in-place storage).

    ``max_len`` (optional) sizes every layer's buffer up front; otherwise the
    first ``init``/``append`` sizes it and later appends double it as needed.
    """

    GRANULE = 64   # capacity rounding, one KV block

    def __init__(self, num_layers: int, max_len: int | None = None):
        self.num_layers = num_layers
        self.max_len = max_len
        self._kbuf: list[torch.Tensor | None] = [None] * num_layers
        self._vbuf: list[torch.Tensor | None] = [None] * num_layers
        self._len = [0] * num_layers

    # -- storage -------------------------------------------------------------------------
    def _reserve(self, layer_idx: int, like: torch.Tensor, need: int) -> None:
        kb = self._kbuf[layer_idx]
        if kb is not None and kb.size(2) >= need and kb.shape[:2] == like.shape[:2] and kb.size(3) == like.size(3):
            return
        cap = max(need, self.max_len or 0, 2 * kb.size(2) if kb is not None else 0)
        cap = _round_up(cap, self.GRANULE)
        B, H, _, D = like.shape
        nk = torch.empty(B, H, cap, D, dtype=like.dtype, device=like.device)
        nv = torch.empty_like(nk)
        n = self._len[layer_idx]
        if kb is not None and n:
            nk[:, :, :n].copy_(kb[:, :, :n])
            nv[:, :, :n].copy_(self._vbuf[layer_idx][:, :, :n])
        self._kbuf[layer_idx], self._vbuf[layer_idx] = nk, nv

    def _view(self, layer_idx: int) -> tuple[torch.Tensor, torch.Tensor]:
        n = self._len[layer_idx]
        return self._kbuf[layer_idx][:, :, :n], self._vbuf[layer_idx][:, :, :n]

    # -- reference API -------------------------------------------------------------------
    def init(self, k_list: list[torch.Tensor], v_list: list[torch.Tensor]) -> None:
        """Fills every layer from a prefill's K/V (``[B, H, T, D]`` each)."""
        assert len(k_list) == self.num_layers
        assert len(v_list) == self.num_layers
        self.clear()
        for i, (k, v) in enumerate(zip(k_list, v_list)):
            self.append(i, k, v)

    def clone(self) -> "KVCache":
        """Deep copy, so decode benchmarks can reuse a fixed prefix."""
        out = KVCache(self.num_layers, self.max_len)
        for i in range(self.num_layers):
            if self._kbuf[i] is not None:
                out._kbuf[i] = self._kbuf[i].clone()
                out._vbuf[i] = self._vbuf[i].clone()
            out._len[i] = self._len[i]
        return out

    def append(self, layer_idx: int, k_new: torch.Tensor, v_new: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """Appends ``[B, H, t, D]`` new K/V and returns the full ``[B, H, T + t, D]`` views."""
        if k_new.shape != v_new.shape:
            raise ValueError(f"k_new {tuple(k_new.shape)} and v_new {tuple(v_new.shape)} differ")
        n, t = self._len[layer_idx], k_new.size(2)
        self._reserve(layer_idx, k_new, n + t)
        self._kbuf[layer_idx][:, :, n:n + t].copy_(k_new)
        self._vbuf[layer_idx][:, :, n:n + t].copy_(v_new)
        self._len[layer_idx] = n + t
        return self._view(layer_idx)

    def seq_len(self, layer_idx: int = 0) -> int:
        return self._len[layer_idx]

    def clear(self) -> None:
        """Forgets the cached tokens; the buffers are kept for reuse."""
        self._len = [0] * self.num_layers

    def truncate(self, length: int) -> None:
        """Drops every layer's tokens past ``length`` (no copy): a benchmark's decode step can
        restart from the same prefix."""
        self._len = [min(n, length) for n in self._len]

    def get(self, layer_idx: int) -> tuple[torch.Tensor, torch.Tensor]:
        """The cached ``[B, H, T, D]`` views of one layer."""
        if self._kbuf[layer_idx] is None:
            raise KeyError(f"layer {layer_idx} holds no tokens")
        return self._view(layer_idx)


class PagedKVStore:
    """One layer's paged K/V: ``k_pages, v_pages [P, H, page, D]``, ``block_table [B, max_blocks]``.

    Pages are handed out from a free list (in a seeded shuffled order when
    ``shuffle_seed`` is given, to exercise non-contiguous tables) as
    sequences grow; ``lens`` counts the valid tokens per sequence on the host
    and ``kv_lens`` mirrors it on the device.
    """

    def __init__(self, batch: int, heads: int, head_dim: int, max_len: int, *, page: int = 64,
                 dtype=torch.bfloat16, device="cuda", num_pages: int | None = None,
                 shuffle_seed: int | None = None):
        if page % 16 or not 16 <= page <= 128:
            raise ValueError(f"page {page} must be a multiple of 16 in [16, 128]")
        self.batch, self.heads, self.head_dim, self.page = batch, heads, head_dim, page
        self.max_blocks = -(-max_len // page)
        self.num_pages = num_pages if num_pages is not None else batch * self.max_blocks
        self.k_pages = torch.empty(self.num_pages, heads, page, head_dim, dtype=dtype, device=device)
        self.v_pages = torch.empty_like(self.k_pages)
        self.block_table = torch.zeros(batch, self.max_blocks, dtype=torch.int32, device=device)
        self.kv_lens = torch.zeros(batch, dtype=torch.int32, device=device)
        self.lens = [0] * batch
        self._table_host = [[] for _ in range(batch)]
        self._page_cols: dict = {}
        order = torch.arange(self.num_pages)
        if shuffle_seed is not None:
            order = order[torch.randperm(self.num_pages, generator=torch.Generator().manual_seed(shuffle_seed))]
        self._free = order.tolist()[::-1]   # pop() hands out order[0] first

    def _grow_all(self, new_len: int) -> None:
        """Gives every sequence the pages that ``new_len`` tokens need (one table update)."""
        need = -(-new_len // self.page)
        if need > self.max_blocks:
            raise ValueError(f"sequences need {need} blocks > max_blocks {self.max_blocks}")
        have = len(self._table_host[0])
        if need <= have:
            return
        if len(self._free) < self.batch * (need - have):
            raise RuntimeError("paged KV cache: out of pages")
        added = []
        for row in self._table_host:
            for _ in range(need - have):
                row.append(self._free.pop())
            added.append(row[have:need])
        self.block_table[:, have:need] = torch.tensor(added, dtype=torch.int32).to(self.block_table.device)
        self._page_cols.clear()

    def _page_col(self, lb: int) -> torch.Tensor:
        """Pages of logical block ``lb`` for every sequence, as a device index tensor (cached)."""
        col = self._page_cols.get(lb)
        if col is None:
            col = self.block_table[:, lb].long()
            self._page_cols[lb] = col
        return col

    def write(self, k_new: torch.Tensor, v_new: torch.Tensor) -> None:
        """Appends ``[B, H, t, D]`` K/V at every sequence's end (all sequences advance by t)."""
        B, H, t, D = k_new.shape
        if (B, H, D) != (self.batch, self.heads, self.head_dim) or v_new.shape != k_new.shape:
            raise ValueError(f"write of {tuple(k_new.shape)} into a [{self.batch}, {self.heads}, *, "
                             f"{self.head_dim}] store")
        start = self.lens[0]
        self._grow_all(start + t)
        if t == 1:   # decode: one slot of one page per sequence
            idx = self._page_col(start // self.page)
            slot = start % self.page
            self.k_pages[idx, :, slot] = k_new[:, :, 0].to(self.k_pages.dtype)
            self.v_pages[idx, :, slot] = v_new[:, :, 0].to(self.v_pages.dtype)
        else:
            pos = torch.arange(start, start + t, device=k_new.device)
            pages = self.block_table[:, pos // self.page].long()          # [B, t]
            slots = (pos % self.page).expand(B, t)                         # [B, t]
            # advanced indices on dims 0 and 2 put [B, t] first: [B, t, H, D]
            self.k_pages[pages, :, slots] = k_new.transpose(1, 2).to(self.k_pages.dtype)
            self.v_pages[pages, :, slots] = v_new.transpose(1, 2).to(self.v_pages.dtype)
        self.lens = [start + t] * B
        self.kv_lens.fill_(start + t)

    def gather(self) -> tuple[torch.Tensor, torch.Tensor]:
        """Contiguous ``[B, H, T, D]`` copies of the cached K/V (slow path for generic callers)."""
        T = self.lens[0]
        nb = -(-T // self.page)
        pages = self.block_table[:, :nb].long()                         # [B, nb]
        k = self.k_pages[pages].permute(0, 2, 1, 3, 4).reshape(self.batch, self.heads, nb * self.page, -1)
        v = self.v_pages[pages].permute(0, 2, 1, 3, 4).reshape(self.batch, self.heads, nb * self.page, -1)
        return k[:, :, :T].contiguous(), v[:, :, :T].contiguous()

    def seq_len(self) -> int:
        return self.lens[0]

    def reset(self) -> None:
        """Returns every page to the free list (contents are left as they are)."""
        for row in self._table_host:
            self._free.extend(reversed(row))
            row.clear()
        self._page_cols.clear()
        self.lens = [0] * self.batch
        self.kv_lens.zero_()
