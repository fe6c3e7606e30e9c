"""Latency, memory and accuracy metrics (``sparse_attention_bench/metrics``), plus profiler ranges.

GPU latency is timed with HIP events on the current stream, one event pair per call after the
warm-up, as the reference does with CUDA events.  ``marker(name)`` brackets a phase with a roctx
range (``torch.cuda.nvtx`` on ROCm), which ``rocprofv3 --marker-trace`` records.
"""
from __future__ import annotations

import time
from contextlib import contextmanager
from typing import Callable

import torch
import torch.nn.functional as F


def _on_gpu(device: str) -> bool:
    return "cuda" in str(device) and torch.cuda.is_available()


def measure_latency(fn: Callable, num_iters: int = 100, num_warmup: int = 20, device: str = "cpu") -> dict:
    """mean / std / p50 / p95 / min / max of ``fn()`` in milliseconds."""
    for _ in range(num_warmup):
        fn()
    times = []
    if _on_gpu(device):
        torch.cuda.synchronize()
        for _ in range(num_iters):
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            fn()
            end.record()
            torch.cuda.synchronize()
            times.append(start.elapsed_time(end))
    else:
        for _ in range(num_iters):
            t0 = time.perf_counter()
            fn()
            times.append((time.perf_counter() - t0) * 1e3)
    t = torch.tensor(times, dtype=torch.float64)
    return {"mean_ms": t.mean().item(), "std_ms": t.std(unbiased=False).item(),
            "p50_ms": t.quantile(0.5).item(), "p95_ms": t.quantile(0.95).item(),
            "min_ms": t.min().item(), "max_ms": t.max().item()}


def measure_peak_memory_mb(fn: Callable, device: str = "cpu") -> float:
    """Peak GPU memory allocated while ``fn()`` runs, in MB (0 on the CPU)."""
    if not _on_gpu(device):
        fn()
        return 0.0
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    fn()
    torch.cuda.synchronize()
    return torch.cuda.max_memory_allocated() / (1024 ** 2)


def relative_error(x: torch.Tensor, y: torch.Tensor, eps: float = 1e-8) -> float:
    return (torch.norm(x - y) / (torch.norm(y) + eps)).item()


def cosine_sim(x: torch.Tensor, y: torch.Tensor, eps: float = 1e-8) -> float:
    return F.cosine_similarity(x.reshape(-1), y.reshape(-1), dim=0, eps=eps).item()


def top1_match_rate(logits_a: torch.Tensor, logits_b: torch.Tensor) -> float:
    """Fraction of positions whose argmax agrees (logits ``[B, T, V]``)."""
    return (logits_a.argmax(dim=-1) == logits_b.argmax(dim=-1)).float().mean().item()


def mean_kl_divergence(reference_logits: torch.Tensor, approx_logits: torch.Tensor) -> float:
    """Average position-wise KL(reference || approx) over the last dim, in float64."""
    ref = F.log_softmax(reference_logits.double(), dim=-1)
    app = F.log_softmax(approx_logits.double(), dim=-1)
    return max((ref.exp() * (ref - app)).sum(dim=-1).mean().item(), 0.0)


def summarize_scalar(values) -> dict:
    t = torch.tensor(values, dtype=torch.float64)
    return {"mean": t.mean().item(), "std": t.std(unbiased=False).item()}


@contextmanager
def marker(name: str, enabled: bool = True):
    """A roctx range around a benchmark phase (no-op on the CPU or when disabled)."""
    if enabled and torch.cuda.is_available():
        torch.cuda.nvtx.range_push(name)
        try:
            yield
        finally:
            torch.cuda.nvtx.range_pop()
    else:
        yield
