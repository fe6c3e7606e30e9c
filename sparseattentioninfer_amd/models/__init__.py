"""Callers of the attention backends: the reference's ``AttentionLayer`` and ``KVCache`` API
(``sparse_attentions/models``), plus a paged K/V store for the paged decode kernel."""
from .attention_layer import AttentionLayer, repeat_kv
from .kv_cache import KVCache, PagedKVStore

__all__ = ["AttentionLayer", "KVCache", "PagedKVStore", "repeat_kv"]
