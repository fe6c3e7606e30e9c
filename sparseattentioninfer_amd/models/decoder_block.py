"""Toy decoder for the layer and decoder benchmarks.

Drop-in for ``sparse_attentions/models/decoder_block.py:18-125``: the classes ``RMSNorm``, ``MLP``,
``DecoderBlock`` and ``ToyDecoder`` with the reference's constructors,
``DecoderBlock.forward(x, kv_cache=None, layer_idx=0)`` and
``ToyDecoder.forward(input_ids, kv_cache=None, pos_offset=0)``.

The submodule names are part of the interface, not a choice made here: the reference's decoder
runner reads ``model.blocks[0].attn.backend.actual_backend``
(``sparse_attention_bench/runners/decoder_sweep_runner.py:116``) and copies weights between a
dense and a sparse decoder with ``load_state_dict``, so a checkpoint's keys (``token_emb``,
``pos_emb``, ``blocks.<i>.norm1 / attn / norm2 / mlp.fc1 / mlp.fc2``, ``norm_f``, ``lm_head``)
must mean the same thing here.  The computation is the same pre-norm decoder (RMSNorm with eps
1e-6, exact-GELU feed-forward of width ``mlp_ratio * d_model``, learned absolute positions,
output head tied to the token embedding).  Beyond the reference:

* ``pattern`` and ``backend`` may be sequences with one entry per layer (sparse attention in the
  first layers only, say), and ``num_kv_heads`` gives grouped-query attention;
* norms run ``torch.nn.functional.rms_norm`` (one fused kernel) instead of a chain of
  elementwise operations;
* positions past ``max_seq_len`` raise ``ValueError`` with the offending range.
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


class RMSNorm(nn.Module):
    """``x / sqrt(mean(x^2) + eps) * weight`` over the last dimension; parameter ``weight``."""

    def __init__(self, dim: int, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return F.rms_norm(x, self.weight.shape, self.weight, self.eps)


class MLP(nn.Module):
    """``fc2(gelu(fc1(x)))`` with hidden width ``mlp_ratio * d_model``."""

    def __init__(self, d_model: int, mlp_ratio: int = 4, bias: bool = False):
        super().__init__()
        self.fc1 = nn.Linear(d_model, mlp_ratio * d_model, bias=bias)
        self.act = nn.GELU()
        self.fc2 = nn.Linear(mlp_ratio * d_model, d_model, bias=bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.fc2(self.act(self.fc1(x)))


class DecoderBlock(nn.Module):
    """``x + attn(norm1(x))``, then ``x + mlp(norm2(x))``."""

    def __init__(self, d_model: int, num_heads: int, pattern: SparsePattern, backend: AttentionBackend,
                 mlp_ratio: int = 4, causal: bool = True, *, num_kv_heads: int | None = None):
        super().__init__()
        self.norm1 = RMSNorm(d_model)
        self.attn = AttentionLayer(d_model=d_model, num_heads=num_heads, pattern=pattern, backend=backend,
                                   causal=causal, num_kv_heads=num_kv_heads)
        self.norm2 = RMSNorm(d_model)
        self.mlp = MLP(d_model, mlp_ratio)

    def forward(self, x: torch.Tensor, kv_cache: KVCache | None = None, layer_idx: int = 0) -> torch.Tensor:
        h = x + self.attn(self.norm1(x), kv_cache=kv_cache, layer_idx=layer_idx)
        return h + self.mlp(self.norm2(h))


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
        self.token_emb = nn.Embedding(vocab_size, d_model)
        self.pos_emb = nn.Embedding(max_seq_len, d_model)
        per_layer = zip(_per_layer(pattern, num_layers, "pattern"), _per_layer(backend, num_layers, "backend"))
        self.blocks = nn.ModuleList(
            DecoderBlock(d_model, num_heads, p, be, mlp_ratio=mlp_ratio, causal=causal, num_kv_heads=num_kv_heads)
            for p, be in per_layer)
        self.norm_f = RMSNorm(d_model)
        self.lm_head = nn.Linear(d_model, vocab_size, bias=False)
        self.lm_head.weight = self.token_emb.weight  # tied: one parameter under both keys

    def forward(self, input_ids: torch.Tensor, kv_cache: KVCache | None = None, pos_offset: int = 0) -> torch.Tensor:
        T = input_ids.size(1)
        if pos_offset < 0 or pos_offset + T > self.max_seq_len:
            raise ValueError(f"positions {pos_offset}..{pos_offset + T - 1} outside max_seq_len {self.max_seq_len}")
        h = self.token_emb(input_ids) + self.pos_emb.weight[pos_offset:pos_offset + T]
        for idx, blk in enumerate(self.blocks):
            h = blk(h, kv_cache=kv_cache, layer_idx=idx)
        return self.lm_head(self.norm_f(h))
