"""``AttentionLayer``: QKV projection, sparse pattern, attention backend, output projection.

Same constructor arguments and ``forward(x, kv_cache=None, layer_idx=0)`` as
``sparse_attentions/models/attention_layer.py:20-74``: q/k/v are produced as
``[B, H, T, D]``, appended to the cache when one is given, the pattern is
built from ``(q, k)`` and the backend runs the attention.  One extension:
``num_kv_heads`` (default ``num_heads``) gives grouped-query attention.  K/V
then carry ``num_kv_heads`` heads and are handed over un-repeated to a
backend that declares ``supports_gqa``; other backends get them repeated to
``num_heads`` (Hugging Face ``repeat_kv`` order: query head h reads KV head
``h // (num_heads / num_kv_heads)``).
"""
from __future__ import annotations

import torch
import torch.nn as nn

from ..attention.base import AttentionBackend
from ..patterns.base import SparsePattern
from .kv_cache import KVCache


def repeat_kv(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    """``[B, Hkv, T, D] -> [B, Hkv * n_rep, T, D]``, each KV head repeated n_rep times in place."""
    if n_rep == 1:
        return x
    B, H, T, D = x.shape
    return x[:, :, None].expand(B, H, n_rep, T, D).reshape(B, H * n_rep, T, D)


class AttentionLayer(nn.Module):
    """Causal multi-head (or grouped-query) attention with a pluggable pattern and backend."""

    def __init__(self, d_model: int, num_heads: int, pattern: SparsePattern, backend: AttentionBackend,
                 causal: bool = True, bias: bool = False, *, num_kv_heads: int | None = None):
        super().__init__()
        assert d_model % num_heads == 0
        if not causal:
            raise ValueError("AttentionLayer currently supports causal decoder attention only.")
        num_kv_heads = num_kv_heads or num_heads
        if num_heads % num_kv_heads:
            raise ValueError(f"num_heads {num_heads} is not a multiple of num_kv_heads {num_kv_heads}")
        self.d_model = d_model
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = d_model // num_heads
        self.causal = causal
        kv_dim = num_kv_heads * self.head_dim
        self.q_proj = nn.Linear(d_model, d_model, bias=bias)
        self.k_proj = nn.Linear(d_model, kv_dim, bias=bias)
        self.v_proj = nn.Linear(d_model, kv_dim, bias=bias)
        self.o_proj = nn.Linear(d_model, d_model, bias=bias)
        self.pattern = pattern
        self.backend = backend

    def forward(self, x: torch.Tensor, kv_cache: KVCache | None = None, layer_idx: int = 0) -> torch.Tensor:
        B, T, C = x.shape
        q = self.q_proj(x).view(B, T, self.num_heads, self.head_dim).transpose(1, 2).contiguous()
        k = self.k_proj(x).view(B, T, self.num_kv_heads, self.head_dim).transpose(1, 2).contiguous()
        v = self.v_proj(x).view(B, T, self.num_kv_heads, self.head_dim).transpose(1, 2).contiguous()
        if kv_cache is not None:
            k, v = kv_cache.append(layer_idx, k, v)
        if not getattr(self.backend, "supports_gqa", False):
            n_rep = self.num_heads // self.num_kv_heads
            k, v = repeat_kv(k, n_rep).contiguous(), repeat_kv(v, n_rep).contiguous()
        pattern_meta = self.pattern.build(q, k, causal=self.causal)
        out = self.backend.forward(q, k, v, pattern_meta)   # [B, H, T, D]
        out = out.transpose(1, 2).contiguous().view(B, T, C)
        return self.o_proj(out)
