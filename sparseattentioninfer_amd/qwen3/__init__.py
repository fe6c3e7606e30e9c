"""Qwen3 integration: HF Qwen3 with its attention core on the gfx950 sparse backend.

Mirrors ``sparse_llm/qwen3/integrations`` (modeling, config helpers) and adds
a paged HF cache and a random-init runtime for the end-to-end workload.
"""
from .modeling_sparse_qwen3 import (Qwen3SparseKernelAttention, Qwen3SparseKernelForCausalLM,
                                    Qwen3SparseKernelModel, build_sparse_attention_from_dense,
                                    replace_qwen3_attention_with_sparse)
from .paged_cache import PagedKVCache, PagedKVLayer

__all__ = ["Qwen3SparseKernelAttention", "Qwen3SparseKernelForCausalLM", "Qwen3SparseKernelModel",
           "build_sparse_attention_from_dense", "replace_qwen3_attention_with_sparse", "PagedKVCache",
           "PagedKVLayer"]
