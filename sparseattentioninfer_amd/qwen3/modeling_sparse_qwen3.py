"""Qwen3 with its attention core on a sparse backend (default: the gfx950 ``hip_block_sparse``).

Drop-in for ``sparse_llm/qwen3/integrations/modeling_sparse_qwen3.py``: the same
classes and functions (``Qwen3SparseKernelAttention``,
``build_sparse_attention_from_dense``, ``replace_qwen3_attention_with_sparse``,
``Qwen3SparseKernelModel``, ``Qwen3SparseKernelForCausalLM``) with the same
arguments and ``config.sparse_attention_*`` attributes.  The attention math is
the reference's (``:192-315``): q/k RMSNorm per head, rotary embedding, cache
update, pattern build, backend call, output projection.  Differences:

* Grouped-query attention: K/V are not repeated for a backend that declares
  ``supports_gqa``; the pattern may hold one CSR row per KV group.
* The cache arrives as ``past_key_values`` (what transformers 5 passes; the
  reference reads ``past_key_value`` and so never sees it there).  With a
  :class:`~sparseattentioninfer_amd.qwen3.paged_cache.PagedKVCache` the layer
  writes pages directly and decodes from them with the paged decode kernel.
* Fallback by injection: when no candidate backend passes
  ``validate_sparse_kernel_runtime`` the layer warns once and still calls the
  first candidate, as the reference does (``:259-299``); the kernel backend then
  runs the masked fallback it was given (``fallback=`` here, or
  ``attention.register_into(..., fallback=)``) and reports
  ``actual_backend == "masked_sdpa_fallback"``.  Without one it raises.
* More patterns: ``"seeded_bigbird"`` (window / global / seeded random blocks
  shared per KV group) and ``"dense"`` (full causal, on the same kernels);
  ``config.sparse_attention_layers`` lists the sparse layers, the others run
  ``"dense"``.
"""
from __future__ import annotations

import warnings
from typing import Optional

import torch
from torch import nn
from transformers.models.qwen3.configuration_qwen3 import Qwen3Config
from transformers.models.qwen3.modeling_qwen3 import (Qwen3Attention, Qwen3ForCausalLM, Qwen3Model,
                                                       apply_rotary_pos_emb)

from ..attention import get_backend
from ..models.attention_layer import repeat_kv
from ..patterns import (BigBirdKeepRatioPattern, BigBirdPattern, DenseCausalPattern, LocalWindowPattern,
                        SeededBigBirdPattern)
from .paged_cache import PagedKVCache
from .sparse_config import (KERNEL_BACKEND, GroupSparsitySpec, backend_candidates, config_value,
                            ensure_attn_implementation, is_plain_causal_mask, pattern_stats,
                            validate_sparse_kernel_runtime)


def _layer_pattern_name(config, layer_idx: int) -> str:
    name = config_value(config, "sparse_attention_pattern", "local")
    layers = config_value(config, "sparse_attention_layers", None)
    if layers is not None and layer_idx not in set(int(i) for i in layers):
        return "dense"
    return name


class Qwen3SparseKernelAttention(Qwen3Attention):
    """HF Qwen3 attention with the attention core replaced by a sparse backend."""

    def __init__(self, config: Qwen3Config, layer_idx: int, *, backend_name: Optional[str] = None,
                 window_size: Optional[int] = None, block_size: Optional[int] = None, group_sparsities=None,
                 fallback=None):
        super().__init__(config, layer_idx)
        self.num_heads = config.num_attention_heads
        self.num_key_value_heads = config.num_key_value_heads
        pattern_name = _layer_pattern_name(config, layer_idx)
        raw_backend = backend_name or config_value(config, "sparse_attention_backend", "auto")
        window_size = window_size or config_value(config, "sparse_attention_window_size", 512)
        block_size = block_size or config_value(config, "sparse_attention_block_size", 64)
        top_k = config_value(config, "sparse_attention_top_k", 128)
        keep_ratio = config_value(config, "sparse_attention_keep_ratio", None)
        groups = GroupSparsitySpec.build(group_sparsities, where=f"layer_{layer_idx}_group_sparsities").default
        if groups is None:
            groups = GroupSparsitySpec.resolve_layer(config, layer_idx)
        self.backend_candidates = backend_candidates(raw_backend)
        self.pattern_name = pattern_name
        self.backend_name = self.backend_candidates[0]
        self.window_size, self.block_size, self.top_k = window_size, block_size, top_k
        self.keep_ratio = None if groups is not None else keep_ratio
        self.group_sparsities = groups
        # fallback: a backend class or instance for inputs the kernels cannot take (the reference's
        # MaskedSdpaBackend inside the reference); only the kernel backend takes one
        self.sparse_backends = {name: get_backend(name, fallback=fallback) if name == KERNEL_BACKEND and fallback
                                is not None else get_backend(name) for name in self.backend_candidates}
        self.sparse_backend = self.sparse_backends[self.backend_name]
        self.sparse_pattern = self._make_pattern(config, layer_idx)
        self.last_pattern_stats: Optional[dict[str, float]] = None
        self.validate_causal_mask = True
        self.collect_pattern_stats = True
        self.lock_runtime_backend = False
        self._locked_backend_name: Optional[str] = None
        self._fallback_warning_emitted = False
        self._runtime_ok = True          # whether the last selected backend passed validation

    def _make_pattern(self, config, layer_idx: int):
        H, Hkv = config.num_attention_heads, config.num_key_value_heads
        if self.pattern_name == "bigbird":
            if self.group_sparsities is not None:
                return BigBirdKeepRatioPattern(group_sparsities=self.group_sparsities, n_heads=H, n_kv_heads=Hkv)
            if self.keep_ratio is not None:
                return BigBirdKeepRatioPattern(keep_ratio=self.keep_ratio, n_heads=H, n_kv_heads=Hkv)
            return BigBirdPattern(top_k=self.top_k, n_heads=H)
        if self.pattern_name == "seeded_bigbird":
            return SeededBigBirdPattern(
                rows=Hkv, block_size=self.block_size,
                window=config_value(config, "sparse_attention_bigbird_window", 3),
                global_blocks=config_value(config, "sparse_attention_bigbird_global", 2),
                random_blocks=config_value(config, "sparse_attention_bigbird_random", 3),
                seed=config_value(config, "sparse_attention_seed", 0) + layer_idx)
        if self.pattern_name == "dense":
            return DenseCausalPattern()
        if self.pattern_name == "local":
            return LocalWindowPattern(window_size=self.window_size, block_size=self.block_size)
        raise ValueError(f"unknown sparse_attention_pattern {self.pattern_name!r}")

    def _select_backend(self, q: torch.Tensor, pattern):
        """The first candidate that can run these inputs.  With none, the first candidate all the
        same, after a one-time warning: its forward then takes its fallback path (or raises)."""
        if self.lock_runtime_backend and self._locked_backend_name is not None:
            return self._locked_backend_name
        self._runtime_ok = True
        chosen, reason = None, None
        for name in self.backend_candidates:
            ok, why = validate_sparse_kernel_runtime(backend_name=name, device=q.device, dtype=q.dtype,
                                                     block_size=pattern.block_size,
                                                     has_block_list=pattern.kv_block_list is not None,
                                                     head_dim=q.size(-1), kind=pattern.kind)
            if ok:
                chosen = name
                break
            reason = reason or why
        if chosen is None:
            chosen = self.backend_candidates[0]
            self._runtime_ok = False
            if chosen == KERNEL_BACKEND and not self._fallback_warning_emitted:
                warnings.warn(f"Sparse attention will fall back instead of using the HIP kernel. Reason: {reason}",
                              stacklevel=3)
                self._fallback_warning_emitted = True
        if self.lock_runtime_backend:
            self._locked_backend_name = chosen
        return chosen

    def forward(self, hidden_states: torch.Tensor, position_embeddings: tuple[torch.Tensor, torch.Tensor],
                attention_mask: Optional[torch.Tensor] = None, past_key_values=None,
                cache_position: Optional[torch.LongTensor] = None, **kwargs):
        if kwargs.get("output_attentions", False):
            raise NotImplementedError("Sparse kernel path does not return attention weights.")
        cache = past_key_values if past_key_values is not None else kwargs.get("past_key_value")
        input_shape = hidden_states.shape[:-1]
        bsz, q_len = input_shape
        hidden_shape = (*input_shape, -1, self.head_dim)
        q = self.q_norm(self.q_proj(hidden_states).view(hidden_shape)).transpose(1, 2)
        k = self.k_norm(self.k_proj(hidden_states).view(hidden_shape)).transpose(1, 2)
        v = self.v_proj(hidden_states).view(hidden_shape).transpose(1, 2)
        cos, sin = position_embeddings
        q, k = apply_rotary_pos_emb(q, k, cos, sin)
        q = q.contiguous()

        store = None
        if isinstance(cache, PagedKVCache):
            layer = cache.layers[self.layer_idx]
            prefix = layer.get_seq_length()
            store = layer.write(k, v)
            if prefix == 0:
                store = None                      # fresh prompt: attend on the new K/V directly
            elif q_len > 1:
                k, v = store.gather()             # chunked prefill over cached pages: contiguous copy
                store = None
        elif cache is not None:
            k, v = cache.update(k, v, self.layer_idx, {"sin": sin, "cos": cos, "cache_position": cache_position})
        k_len = store.seq_len() if store is not None else k.size(2)

        if self.validate_causal_mask and not is_plain_causal_mask(attention_mask, q_len=q_len, k_len=k_len):
            raise NotImplementedError("Sparse kernel path supports plain causal masks only; padding-aware or "
                                      "custom attention masks are not wired up.")
        # shape stand-in for the pattern when K/V live in pages (no data)
        k_like = k if store is None else q.new_empty((bsz, self.num_key_value_heads, k_len, 0))
        pattern = self.sparse_pattern.build(q, k_like, causal=True)
        self.last_pattern_stats = pattern_stats(pattern) if self.collect_pattern_stats else None
        self.backend_name = self._select_backend(q, pattern)
        backend = self.sparse_backend = self.sparse_backends[self.backend_name]

        if store is not None and self._runtime_ok and hasattr(backend, "forward_paged") and \
                (pattern.kind == "dense" or pattern.block_size == store.page):
            out = backend.forward_paged(q, store, pattern)
        else:
            if store is not None:
                k, v = store.gather()
            if not getattr(backend, "supports_gqa", False):
                k = repeat_kv(k, self.num_key_value_groups)
                v = repeat_kv(v, self.num_key_value_groups)
            out = backend.forward(q, k.contiguous(), v.contiguous(), pattern)
        expected = (bsz, self.num_heads, q_len, self.head_dim)
        if out.size() != expected:
            raise ValueError(f"`attn_output` should be of size {expected}, but is {tuple(out.size())}.")
        out = out.transpose(1, 2).reshape(*input_shape, -1).contiguous()
        return self.o_proj(out), None


def build_sparse_attention_from_dense(attention: nn.Module, *, backend_name: str = "hip_block_sparse",
                                      window_size: int = 512, block_size: int = 64,
                                      target_dtype: Optional[torch.dtype] = None,
                                      group_sparsities=None, fallback=None) -> Qwen3SparseKernelAttention:
    """Sparse twin of a Qwen3 attention module with its weights (``:318-342``)."""
    if not hasattr(attention, "config") or not hasattr(attention, "layer_idx"):
        raise TypeError("Expected a Qwen3 attention module with `config` and `layer_idx` attributes.")
    w = attention.q_proj.weight
    with torch.device(w.device):
        sparse = Qwen3SparseKernelAttention(attention.config, layer_idx=attention.layer_idx,
                                            backend_name=backend_name, window_size=window_size,
                                            block_size=block_size, group_sparsities=group_sparsities,
                                            fallback=fallback)
    sparse.to(dtype=w.dtype)
    sparse.load_state_dict(attention.state_dict(), strict=False)
    if target_dtype is not None:
        sparse.to(dtype=target_dtype)
    return sparse


def replace_qwen3_attention_with_sparse(model: nn.Module, *, backend_name: str = "hip_block_sparse",
                                        window_size: int = 512, block_size: int = 64,
                                        target_dtype: Optional[torch.dtype] = None, group_sparsities=None,
                                        layer_group_sparsities=None, fallback=None) -> nn.Module:
    """Replaces every ``layer.self_attn`` of a Qwen3 decoder model (``:345-399``)."""
    if not hasattr(model, "layers"):
        raise TypeError("Expected a Qwen3 decoder model with a `.layers` attribute.")
    spec = GroupSparsitySpec.with_config_defaults(model.config, group_sparsities, layer_group_sparsities)
    if spec.per_layer is not None and len(spec.per_layer) > len(model.layers):
        raise ValueError("layer_group_sparsities has more entries than there are decoder layers.")
    for layer in model.layers:
        layer.self_attn = build_sparse_attention_from_dense(
            layer.self_attn, backend_name=backend_name, window_size=window_size, block_size=block_size,
            target_dtype=target_dtype, group_sparsities=spec.for_layer(layer.self_attn.layer_idx),
            fallback=fallback)
    return model


def _apply_sparse_config_to_hf_config(config: Qwen3Config, *, group_sparsities=None,
                                      layer_group_sparsities=None) -> None:
    ensure_attn_implementation(config)
    GroupSparsitySpec.build(group_sparsities, layer_group_sparsities).write_to(config)


def _replace_sparse_attention_from_config(model: nn.Module, config: Qwen3Config, fallback=None) -> None:
    replace_qwen3_attention_with_sparse(
        model,
        backend_name=config_value(config, "sparse_attention_backend", "hip_block_sparse"),
        window_size=config_value(config, "sparse_attention_window_size", 512),
        block_size=config_value(config, "sparse_attention_block_size", 64),
        target_dtype=config_value(config, "sparse_attention_target_dtype", None),
        group_sparsities=config_value(config, "sparse_attention_group_sparsities", None),
        layer_group_sparsities=config_value(config, "sparse_attention_layer_group_sparsities", None),
        fallback=fallback)


class Qwen3SparseKernelModel(Qwen3Model):
    def __init__(self, config: Qwen3Config, *, group_sparsities=None, layer_group_sparsities=None, fallback=None):
        _apply_sparse_config_to_hf_config(config, group_sparsities=group_sparsities,
                                          layer_group_sparsities=layer_group_sparsities)
        super().__init__(config)
        _replace_sparse_attention_from_config(self, config, fallback)


class Qwen3SparseKernelForCausalLM(Qwen3ForCausalLM):
    def __init__(self, config: Qwen3Config, *, group_sparsities=None, layer_group_sparsities=None, fallback=None):
        _apply_sparse_config_to_hf_config(config, group_sparsities=group_sparsities,
                                          layer_group_sparsities=layer_group_sparsities)
        super().__init__(config)
        _replace_sparse_attention_from_config(self.model, config, fallback)
