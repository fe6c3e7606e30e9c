"""Toy decoder for the layer and decoder benchmarks.

Drop-in for the constructors of ``sparse_attentions/models/decoder_block.py:49-125``:
``DecoderBlock(d_model, num_heads, pattern, backend, mlp_ratio=4, causal=True)`` and
``ToyDecoder(vocab_size, d_model, num_heads, num_layers, pattern, backend, max_seq_len=4096,
mlp_ratio=4, causal=True)`` with ``forward(x, kv_cache=None, layer_idx=0)`` and
``forward(input_ids, kv_cache=None, pos_offset=0)``.  The computation is the same pre-norm
decoder (RMSNorm with eps 1e-6, GELU feed-forward of width ``mlp_ratio * d_model``, learned
absolute positions, output head tied to the token embedding); the module structure is this
build's own:

* a block is two :class:`PreNormResidual` sublayers, ``x + body(rms_norm(x))``, one around the
  attention layer and one around the feed-forward ``nn.Sequential``;
* norms call ``torch.nn.functional.rms_norm`` with a learned scale;
* the output head is ``F.linear(h, embedding.weight)``, so the tie needs no second module;
* ``pattern`` and ``backend`` may also be sequences with one entry per layer (e.g. sparse
  attention in the first layers only), and ``num_kv_heads`` gives grouped-query attention.

State dicts round-trip between two ``ToyDecoder`` instances of equal shape, which is how the
benchmarks give a sparse and a dense model the same weights.
"""
from __future__ import annotations

from typing import Sequence, Union

import torch
import torch.nn as nn
import torch.nn.functional as F

from ..attention.base import AttentionBackend
from ..patterns.base import SparsePattern
from .attention_layer import AttentionLayer
from .kv_cache import KVCache

NORM_EPS = 1e-6


class PreNormResidual(nn.Module):
    """``x + body(rms_norm(x) * scale)``; keyword arguments of the call go to ``body``."""

    def __init__(self, dim: int, body: nn.Module, eps: float = NORM_EPS):
        super().__init__()
        self.scale = nn.Parameter(torch.ones(dim))
        self.eps = eps
        self.body = body

    def forward(self, x: torch.Tensor, **body_kwargs) -> torch.Tensor:
        h = F.rms_norm(x, (x.size(-1),), self.scale, self.eps)
        return x + self.body(h, **body_kwargs)


def feed_forward(d_model: int, mlp_ratio: int) -> nn.Sequential:
    """``d_model -> mlp_ratio * d_model -> d_model`` with an exact GELU, no biases."""
    width = d_model * mlp_ratio
    return nn.Sequential(nn.Linear(d_model, width, bias=False), nn.GELU(), nn.Linear(width, d_model, bias=False))


class DecoderBlock(nn.Module):
    """Pre-norm attention sublayer followed by a pre-norm feed-forward sublayer."""

    def __init__(self, d_model: int, num_heads: int, pattern: SparsePattern, backend: AttentionBackend,
                 mlp_ratio: int = 4, causal: bool = True, *, num_kv_heads: int | None = None):
        super().__init__()
        attn = AttentionLayer(d_model=d_model, num_heads=num_heads, pattern=pattern, backend=backend,
                              causal=causal, num_kv_heads=num_kv_heads)
        self.attention = PreNormResidual(d_model, attn)
        self.ffn = PreNormResidual(d_model, feed_forward(d_model, mlp_ratio))

    @property
    def attn(self) -> AttentionLayer:
        return self.attention.body

    def forward(self, x: torch.Tensor, kv_cache: KVCache | None = None, layer_idx: int = 0) -> torch.Tensor:
        return self.ffn(self.attention(x, kv_cache=kv_cache, layer_idx=layer_idx))


def _per_layer(value, n: int, what: str) -> list:
    """``value`` repeated for ``n`` layers, or a sequence of exactly ``n`` entries."""
    if isinstance(value, (list, tuple)):
        if len(value) != n:
            raise ValueError(f"{what}: {len(value)} entries for {n} layers")
        return list(value)
    return [value] * n


class ToyDecoder(nn.Module):
    """Token and position embeddings, ``num_layers`` decoder blocks, final norm, tied head."""

    def __init__(self, vocab_size: int, d_model: int, num_heads: int, num_layers: int,
                 pattern: Union[SparsePattern, Sequence[SparsePattern]],
                 backend: Union[AttentionBackend, Sequence[AttentionBackend]],
                 max_seq_len: int = 4096, mlp_ratio: int = 4, causal: bool = True, *,
                 num_kv_heads: int | None = None):
        super().__init__()
        self.max_seq_len = max_seq_len
        self.embedding = nn.Embedding(vocab_size, d_model)
        self.positions = nn.Parameter(torch.randn(max_seq_len, d_model))
        patterns = _per_layer(pattern, num_layers, "pattern")
        backends = _per_layer(backend, num_layers, "backend")
        self.layers = nn.ModuleList(
            DecoderBlock(d_model, num_heads, p, be, mlp_ratio=mlp_ratio, causal=causal, num_kv_heads=num_kv_heads)
            for p, be in zip(patterns, backends))
        self.final_scale = nn.Parameter(torch.ones(d_model))

    def forward(self, input_ids: torch.Tensor, kv_cache: KVCache | None = None, pos_offset: int = 0) -> torch.Tensor:
        T = input_ids.size(1)
        if pos_offset + T > self.max_seq_len:
            raise ValueError(f"positions {pos_offset}..{pos_offset + T - 1} exceed max_seq_len {self.max_seq_len}")
        h = self.embedding(input_ids) + self.positions[pos_offset:pos_offset + T]
        for idx, layer in enumerate(self.layers):
            h = layer(h, kv_cache=kv_cache, layer_idx=idx)
        h = F.rms_norm(h, (h.size(-1),), self.final_scale, NORM_EPS)
        return F.linear(h, self.embedding.weight)
