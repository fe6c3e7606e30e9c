"""Pattern factory and the layer benchmark (``sparse_attention_bench/runners/benchmark_runner.py:16-145``).

``BenchmarkRunner.run(cfg)`` times the pattern build, the attention call and both together,
measures peak memory, and compares the output with dense causal attention run by the same backend
(``DenseCausalPattern``), returning the reference's result keys.
"""
from __future__ import annotations

import torch

from ..attention import get_backend
from ..models.attention_layer import repeat_kv
from ..patterns import (BernoulliBlockPattern, BigBird2Pattern, BigBirdKeepRatioPattern, BigBirdPattern,
                        DenseCausalPattern, LocalWindowPattern, PatternMetadata, SeededBigBirdPattern)
from .config import ExperimentConfig
from .metrics import cosine_sim, marker, mean_kl_divergence, measure_latency, measure_peak_memory_mb, relative_error


def get_pattern(cfg: ExperimentConfig):
    """The SparsePattern a config names (``benchmark_runner.py:16-43``, plus the seeded workloads)."""
    t = cfg.pattern_type
    if t == "dense":
        return DenseCausalPattern()
    if t == "topk":
        raise NotImplementedError("pattern_type 'topk' selects keys by score at run time; it is not a block "
                                  "schedule, so the block-sparse backend does not run it")
    if t == "bigbird":
        if cfg.keep_ratio is not None:
            return BigBirdKeepRatioPattern(keep_ratio=cfg.keep_ratio, n_heads=cfg.num_heads,
                                           n_kv_heads=cfg.num_kv_heads)
        assert cfg.topk is not None, "topk must be set for pattern_type='bigbird'"
        return BigBirdPattern(top_k=cfg.topk, n_heads=cfg.num_heads)
    if t == "bigbird2":
        assert cfg.topk is not None, "topk must be set for pattern_type='bigbird2'"
        return BigBird2Pattern(top_k=cfg.topk, n_heads=cfg.num_heads)
    if t == "local_window":
        assert cfg.window_size is not None, "window_size must be set for pattern_type='local_window'"
        return LocalWindowPattern(window_size=cfg.window_size, block_size=cfg.block_size)
    if t == "seeded_bigbird":
        return SeededBigBirdPattern(rows=cfg.kv_heads, block_size=cfg.block_size or 64, seed=cfg.seed)
    if t == "bernoulli":
        assert cfg.density is not None, "density must be set for pattern_type='bernoulli'"
        return BernoulliBlockPattern(rows=cfg.kv_heads, density=cfg.density, block_size=cfg.block_size or 64,
                                     seed=cfg.seed)
    raise ValueError(f"Unknown pattern_type: {t!r}")


def _kv_for(backend, q, k, v):
    if getattr(backend, "supports_gqa", False) or k.size(1) == q.size(1):
        return k, v
    n_rep = q.size(1) // k.size(1)
    return repeat_kv(k, n_rep).contiguous(), repeat_kv(v, n_rep).contiguous()


class BenchmarkRunner:
    """Runs one ExperimentConfig on one attention call (``q, k, v`` from ``cfg.make_qkv``)."""

    def __init__(self, markers: bool = True):
        self.markers = markers

    def run(self, cfg: ExperimentConfig) -> dict:
        cfg.validate_supported()
        q, k, v = cfg.make_qkv()
        pattern_obj = get_pattern(cfg)
        backend = get_backend(cfg.backend)
        k, v = _kv_for(backend, q, k, v)
        with torch.no_grad():
            dense_out = get_backend(cfg.backend).forward(q, k, v, PatternMetadata(kind="dense"))

        def lat(fn):
            return measure_latency(fn, num_iters=cfg.num_iters, num_warmup=cfg.num_warmup, device=cfg.device)

        with marker("pattern_build", self.markers):
            pattern_latency = lat(lambda: pattern_obj.build(q, k, causal=cfg.causal))
        pattern = pattern_obj.build(q, k, causal=cfg.causal)
        with marker("attention", self.markers):
            attn_latency = lat(lambda: backend.forward(q, k, v, pattern))

        def _full():
            return backend.forward(q, k, v, pattern_obj.build(q, k, causal=cfg.causal))

        with marker("build_and_attention", self.markers):
            total_latency = lat(_full)
        peak_mem_mb = measure_peak_memory_mb(_full, device=cfg.device)
        with torch.no_grad():
            sparse_out = backend.forward(q, k, v, pattern)
        d32, s32 = dense_out.float(), sparse_out.float()
        keep_ratio = float(pattern.keep_ratio)
        return {
            "config": cfg.as_dict(),
            "timing_source": "hip_kernel" if cfg.backend == "hip_block_sparse" else "backend",
            "actual_backend": backend.actual_backend,
            "pattern_build_time_ms_mean": pattern_latency["mean_ms"],
            "pattern_build_time_ms_p50": pattern_latency["p50_ms"],
            "pattern_build_time_ms_p95": pattern_latency["p95_ms"],
            "attention_time_ms_mean": attn_latency["mean_ms"],
            "attention_time_ms_p50": attn_latency["p50_ms"],
            "attention_time_ms_p95": attn_latency["p95_ms"],
            "total_time_ms_mean": total_latency["mean_ms"],
            "total_time_ms_p50": total_latency["p50_ms"],
            "total_time_ms_p95": total_latency["p95_ms"],
            "peak_memory_mb": peak_mem_mb,
            "rel_err": relative_error(s32, d32),
            "cosine_sim": cosine_sim(s32, d32),
            "kl_divergence": mean_kl_divergence(d32, s32),
            "keep_ratio": keep_ratio,
            "sparsity_ratio": 1.0 - keep_ratio,
        }
