"""Layer and Toy-Decoder benchmarks over the attention backends (counterparts of the reference's
``sparse_attention_bench``: ``ExperimentConfig``, the pattern factory, the layer runner, the decoder
benchmark and YAML sweeps)."""
from .config import ExperimentConfig
from .runner import BenchmarkRunner, get_pattern

__all__ = ["ExperimentConfig", "BenchmarkRunner", "get_pattern"]
