"""``ExperimentConfig``: one benchmark run (fields of ``sparse_attention_bench/config.py:9-79``).

Defaults select this build's backend (``hip_block_sparse``) and bf16 on the GPU; ``num_kv_heads``
(default ``num_heads``) adds grouped-query attention and ``seed`` makes the random inputs
reproducible.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class ExperimentConfig:
    batch_size: int = 1
    num_heads: int = 8
    head_dim: int = 64
    seq_len: int = 512
    dtype: str = "bf16"          # "fp32" | "fp16" | "bf16"
    device: str = "cuda"
    mode: str = "prefill"        # "prefill" | "decode"
    pattern_type: str = "dense"  # "dense" | "bigbird" | "bigbird2" | "local_window" | "seeded_bigbird" | "bernoulli"
    backend: str = "hip_block_sparse"
    causal: bool = True
    # pattern parameters (only those of pattern_type are used)
    topk: int | None = None
    keep_ratio: float | None = None
    window_size: int | None = None
    block_size: int | None = None
    density: float | None = None
    # measurement
    num_warmup: int = 20
    num_iters: int = 100
    # extensions
    num_kv_heads: int | None = None
    seed: int = 0

    def __post_init__(self) -> None:
        self.validate_supported()

    def validate_supported(self) -> None:
        if not self.causal:
            raise ValueError("This codebase currently supports causal decoder attention only; set causal=True.")
        if self.mode not in ("prefill", "decode"):
            raise ValueError(f"mode must be 'prefill' or 'decode', got {self.mode!r}")
        if self.num_kv_heads is not None and self.num_heads % self.num_kv_heads:
            raise ValueError(f"num_heads {self.num_heads} is not a multiple of num_kv_heads {self.num_kv_heads}")

    @property
    def kv_heads(self) -> int:
        return self.num_kv_heads or self.num_heads

    def torch_dtype(self) -> torch.dtype:
        return {"fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}[self.dtype]

    def make_qkv(self) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """Seeded N(0, 1) q ``[B, H, T_q, D]`` and k, v ``[B, H_kv, T, D]`` (T_q = 1 in decode mode)."""
        g = torch.Generator().manual_seed(self.seed)
        t_q = self.seq_len if self.mode == "prefill" else 1
        q = torch.randn(self.batch_size, self.num_heads, t_q, self.head_dim, generator=g)
        k = torch.randn(self.batch_size, self.kv_heads, self.seq_len, self.head_dim, generator=g)
        v = torch.randn(self.batch_size, self.kv_heads, self.seq_len, self.head_dim, generator=g)
        dev, dt = torch.device(self.device), self.torch_dtype()
        return q.to(dev, dt), k.to(dev, dt), v.to(dev, dt)

    def as_dict(self) -> dict:
        return {k: getattr(self, k) for k in (
            "batch_size", "num_heads", "head_dim", "seq_len", "dtype", "device", "mode", "pattern_type",
            "backend", "causal", "topk", "keep_ratio", "window_size", "block_size", "density", "num_kv_heads",
            "seed")}
