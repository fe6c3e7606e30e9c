"""Random-init Qwen3 models and timed greedy generation (TTFT, decode tokens/s).

The end-to-end workload is a Qwen3-4B-architecture decoder with random
weights (no checkpoint is loaded): 36 layers, hidden 2560, 32 query / 8 KV
heads of dim 128, SwiGLU 9728, vocab 151936, RoPE theta 1e6, tied
embeddings, weights N(0, 0.02) from a seeded generator.  Timing follows the
reference's generation benchmark (``sparse_llm/common/benchmark/generation.py:21-138``):
TTFT is the synchronised wall time of the prompt forward; decode tokens/s is
``B * steps`` over the summed synchronised step times.
"""
from __future__ import annotations

import time
from contextlib import contextmanager

import torch
from transformers.models.qwen3.configuration_qwen3 import Qwen3Config

from .modeling_sparse_qwen3 import Qwen3SparseKernelForCausalLM
from .paged_cache import PagedKVCache

QWEN3_4B = dict(vocab_size=151936, hidden_size=2560, intermediate_size=9728, num_hidden_layers=36,
                num_attention_heads=32, num_key_value_heads=8, head_dim=128, rope_theta=1e6,
                rms_norm_eps=1e-6, max_position_embeddings=40960, tie_word_embeddings=True,
                initializer_range=0.02)


def qwen3_config(*, sparse_layers=None, pattern: str = "seeded_bigbird", block_size: int = 64,
                 window: int = 3, global_blocks: int = 2, random_blocks=3, seed: int = 0,
                 backend: str = "hip_block_sparse", **overrides) -> Qwen3Config:
    """Qwen3-4B hyper-parameters (``overrides`` replace any of them) plus the sparse settings.

    ``sparse_layers``: indices of the layers that run ``pattern``; the others
    run dense causal attention on the same backend (None = every layer sparse).
    """
    params = {**QWEN3_4B, **overrides}
    rope = params.pop("rope_theta")
    cfg = Qwen3Config(**params, rope_parameters={"rope_type": "default", "rope_theta": rope})
    cfg._attn_implementation = "sdpa"     # lets HF skip building a dense causal mask
    cfg.sparse_attention_pattern = pattern
    cfg.sparse_attention_backend = backend
    cfg.sparse_attention_block_size = block_size
    cfg.sparse_attention_bigbird_window = window
    cfg.sparse_attention_bigbird_global = global_blocks
    cfg.sparse_attention_bigbird_random = random_blocks
    cfg.sparse_attention_seed = seed
    cfg.sparse_attention_layers = None if sparse_layers is None else list(sparse_layers)
    return cfg


@contextmanager
def _default_dtype(dtype):
    prev = torch.get_default_dtype()
    torch.set_default_dtype(dtype)
    try:
        yield
    finally:
        torch.set_default_dtype(prev)


def build_model(config: Qwen3Config, *, device="cuda", dtype=torch.bfloat16, seed: int = 0):
    """Qwen3SparseKernelForCausalLM with seeded N(0, initializer_range) weights, built on ``device``."""
    torch.manual_seed(seed)
    with torch.device(device), _default_dtype(dtype):
        model = Qwen3SparseKernelForCausalLM(config)
    return model.to(device=device, dtype=dtype).eval()


def _sync(device):
    if torch.device(device).type == "cuda":
        torch.cuda.synchronize(device)


@torch.inference_mode()
def greedy_generate(model, input_ids: torch.Tensor, steps: int, *, cache: str = "paged",
                    max_len: int | None = None, shuffle_seed: int | None = None, graph: bool = False) -> dict:
    """Prompt forward (timed: TTFT) then ``steps`` greedy decode forwards (each timed).

    ``cache``: ``"paged"`` (:class:`PagedKVCache`, decode reads pages) or
    ``"dynamic"`` (HF ``DynamicCache``).  ``graph`` (paged cache only): decode
    with :class:`~sparseattentioninfer_amd.qwen3.graph_decode.GraphDecoder`, one
    HIP graph replay per token, instead of the eager Hugging Face forward.
    Returns the timings, the generated ids ``[B, steps + 1]`` and the
    last-position logits of the prompt forward.
    """
    B, T = input_ids.shape
    dev = input_ids.device
    cfg = model.config
    if cache == "paged":
        pkv = PagedKVCache(cfg.num_hidden_layers, max_len or (T + steps + 1),
                           page=getattr(cfg, "sparse_attention_block_size", 64), shuffle_seed=shuffle_seed)
    elif cache == "dynamic":
        from transformers.cache_utils import DynamicCache
        pkv = DynamicCache(config=cfg)
    else:
        raise ValueError(f"unknown cache kind {cache!r}")
    _sync(dev)
    t0 = time.perf_counter()
    out = model(input_ids=input_ids, past_key_values=pkv, use_cache=True, logits_to_keep=1)
    nxt = out.logits[:, -1].argmax(-1)
    _sync(dev)
    ttft = time.perf_counter() - t0
    first_logits = out.logits[:, -1].float()
    tokens = [nxt]
    step_times = []
    if graph:
        if cache != "paged":
            raise ValueError("graph decode needs the paged cache")
        from .graph_decode import GraphDecoder
        t0 = time.perf_counter()
        dec = GraphDecoder(model, pkv, nxt, T + steps)
        _sync(dev)
        graph_setup = time.perf_counter() - t0
        for _ in range(steps):
            _sync(dev)
            t0 = time.perf_counter()
            ids = dec.step()
            _sync(dev)
            step_times.append(time.perf_counter() - t0)
            tokens.append(ids.clone())
        dec.finish()
        steps = len(step_times)
    for _ in range(0 if graph else steps):
        _sync(dev)
        t0 = time.perf_counter()
        out = model(input_ids=nxt[:, None], past_key_values=pkv, use_cache=True, logits_to_keep=1)
        nxt = out.logits[:, -1].argmax(-1)
        _sync(dev)
        step_times.append(time.perf_counter() - t0)
        tokens.append(nxt)
    decode_s = sum(step_times)
    extra = {"graph_setup_s": graph_setup} if graph else {}
    return {**extra, "ttft_s": ttft, "decode_step_times_s": step_times, "decode_total_s": decode_s,
            "decode_tokens_per_s": (B * steps / decode_s) if decode_s > 0 else None,
            "tokens": torch.stack(tokens, dim=1), "first_logits": first_logits, "cache": pkv}
