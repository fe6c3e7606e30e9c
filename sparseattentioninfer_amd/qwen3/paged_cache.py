"""Hugging Face ``Cache`` over paged K/V: the bridge between HF generation and the paged decode kernel.

``PagedKVCache`` is a ``transformers.cache_utils.Cache`` whose layers keep
their K/V in a :class:`~sparseattentioninfer_amd.models.kv_cache.PagedKVStore`
(page pool + block table).  HF code that calls ``update()`` gets contiguous
``[B, H_kv, T, D]`` copies gathered from the pages (correct, but a copy per
call); :class:`~sparseattentioninfer_amd.qwen3.modeling_sparse_qwen3.Qwen3SparseKernelAttention`
instead writes the new tokens with :meth:`PagedKVLayer.write` and decodes straight
from the pages, with no ``repeat_kv`` and no ``torch.cat`` growth of the cache.
"""
from __future__ import annotations

import torch
from transformers.cache_utils import Cache, CacheLayerMixin

from ..models.kv_cache import PagedKVStore


class PagedKVLayer(CacheLayerMixin):
    """One decoder layer's paged K/V, allocated on the first write."""

    is_sliding = False
    is_compileable = False

    def __init__(self, max_len: int, *, page: int = 64, shuffle_seed: int | None = None):
        super().__init__()
        self.max_len, self.page, self.shuffle_seed = max_len, page, shuffle_seed
        self.store: PagedKVStore | None = None

    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        B, H, _, D = key_states.shape
        self.dtype, self.device = key_states.dtype, key_states.device
        self.store = PagedKVStore(B, H, D, self.max_len, page=self.page, dtype=key_states.dtype,
                                  device=key_states.device, shuffle_seed=self.shuffle_seed)
        self.is_initialized = True

    def write(self, key_states: torch.Tensor, value_states: torch.Tensor) -> PagedKVStore:
        """Appends ``[B, H_kv, t, D]`` K/V to the pages; returns the store."""
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        self.store.write(key_states, value_states)
        return self.store

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args, **kwargs):
        """HF interface: appends, then returns contiguous copies of the whole cache."""
        self.write(key_states, value_states)
        return self.store.gather()

    def get_mask_sizes(self, query_length: int) -> tuple[int, int]:
        return self.get_seq_length() + query_length, 0

    def get_seq_length(self) -> int:
        return self.store.seq_len() if self.store is not None else 0

    def get_max_length(self) -> int:
        return self.max_len

    def reset(self) -> None:
        if self.store is not None:
            self.store.reset()

    def offload(self):
        raise NotImplementedError("PagedKVCache does not offload to the host")

    def prefetch(self):
        raise NotImplementedError("PagedKVCache does not offload to the host")

    def reorder_cache(self, beam_idx: torch.LongTensor) -> None:
        raise NotImplementedError("PagedKVCache does not reorder sequences (no beam search)")

    def crop(self, tokens_to_remove: int) -> None:
        raise NotImplementedError("PagedKVCache does not crop")


class PagedKVCache(Cache):
    """``num_layers`` paged layers of up to ``max_len`` tokens per sequence."""

    def __init__(self, num_layers: int, max_len: int, *, page: int = 64, shuffle_seed: int | None = None):
        super().__init__(layers=[PagedKVLayer(max_len, page=page, shuffle_seed=shuffle_seed)
                                 for _ in range(num_layers)])
        self.page = page

    @property
    def max_cache_len(self) -> int:
        return self.layers[0].max_len
