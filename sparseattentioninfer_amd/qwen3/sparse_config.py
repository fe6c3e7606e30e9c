"""Configuration helpers of the Qwen3 sparse-attention integration.

Same names and meaning as ``sparse_llm/qwen3/integrations/sparse_config.py``
(``:13-219``), with the gfx950 backend in place of the Triton ones:
``"auto"`` resolves to ``hip_block_sparse`` for every pattern, and
:func:`validate_sparse_kernel_runtime` states that backend's conditions.
A ROCm GPU tensor reports ``device.type == "cuda"``.
"""
from __future__ import annotations

import json
from pathlib import Path
from typing import Optional

import torch

KERNEL_BACKEND = "hip_block_sparse"
SUPPORTED_BLOCK_SIZES = (16, 32, 64, 128)
SUPPORTED_HEAD_DIMS = (64, 128)


def _get_config_attr(config, name: str, default):
    return getattr(config, name, default)


def _normalize_group_sparsities(values, *, name: str) -> Optional[tuple[float, ...]]:
    """Tuple of floats in [0, 1), or None (``sparse_config.py:17-27``)."""
    if values is None:
        return None
    normalized = tuple(float(v) for v in values)
    if any(not 0.0 <= v < 1.0 for v in normalized):
        raise ValueError(f"{name} values must satisfy 0 <= sparsity < 1.")
    return normalized


def _normalize_layer_group_sparsities(values, *, name: str):
    """Per-layer group sparsities, entries may be None (``sparse_config.py:30-47``)."""
    if values is None:
        return None
    return tuple(None if layer is None else _normalize_group_sparsities(layer, name=f"{name}[{i}]")
                 for i, layer in enumerate(values))


def _materialize_layer_group_sparsities(values):
    """JSON-friendly lists (``sparse_config.py:50-58``)."""
    if values is None:
        return None
    return [None if layer is None else list(layer) for layer in values]


def _parse_group_sparsities_arg(raw_value: Optional[str]) -> Optional[tuple[float, ...]]:
    """``"0.5, 0.7"`` -> (0.5, 0.7); empty -> None (``sparse_config.py:61-70``)."""
    if raw_value is None or not raw_value.strip():
        return None
    return _normalize_group_sparsities([c.strip() for c in raw_value.split(",") if c.strip()],
                                       name="--group-sparsities")


def _parse_layer_group_sparsities_arg(raw_value: Optional[str]):
    """JSON list, given inline or as a file path (``sparse_config.py:73-89``)."""
    if raw_value is None:
        return None
    path = Path(raw_value)
    payload = path.read_text(encoding="utf-8") if path.is_file() else raw_value
    parsed = json.loads(payload)
    if not isinstance(parsed, list):
        raise ValueError("--layer-group-sparsities must decode to a JSON list.")
    return _normalize_layer_group_sparsities(parsed, name="--layer-group-sparsities")


def _ensure_attn_implementation(config) -> None:
    if getattr(config, "_attn_implementation", None) is None:
        config._attn_implementation = "sdpa"


def _resolve_backend_candidates(pattern_name: str, backend_name: str, keep_ratio: Optional[float] = None,
                                group_sparsities=None) -> list[str]:
    """Ordered backend names to try (``sparse_config.py:97-109``); "auto" -> the HIP kernel backend."""
    if backend_name != "auto":
        return [backend_name]
    return [KERNEL_BACKEND]


def _resolve_backend_name(pattern_name: str, backend_name: str, keep_ratio: Optional[float] = None,
                          group_sparsities=None) -> str:
    return _resolve_backend_candidates(pattern_name, backend_name, keep_ratio, group_sparsities)[0]


def _describe_pattern(attn) -> str:
    """One-line description of a layer's pattern (``sparse_config.py:126-141``)."""
    if attn.pattern_name == "bigbird":
        if attn.group_sparsities is not None:
            layouts = getattr(attn.sparse_pattern, "last_group_layouts", None)
            resolved = f", layouts={layouts}" if layouts is not None else ""
            return f"BigBirdGroupSparsity(group_sparsities={list(attn.group_sparsities)}{resolved})"
        if attn.keep_ratio is not None:
            layout = getattr(attn.sparse_pattern, "last_layout", None)
            resolved = f", layout={layout}" if layout is not None else ""
            return f"BigBirdKeepRatio(keep_ratio={attn.keep_ratio:.4f}{resolved})"
        return f"BigBird(top_k={attn.top_k})"
    if attn.pattern_name == "seeded_bigbird":
        p = attn.sparse_pattern
        return (f"SeededBigBird(window={p.window}, global={p.global_blocks}, random={p.random_blocks}, "
                f"block_size={p.block_size}, seed={p.seed})")
    if attn.pattern_name == "dense":
        return "DenseCausal()"
    return f"LocalWindow(window_size={attn.window_size}, block_size={attn.block_size})"


def _is_plain_causal_mask(attention_mask: Optional[torch.Tensor], q_len: int, k_len: int) -> bool:
    """True when the additive mask hides nothing a bottom-right causal mask keeps (``:144-164``)."""
    if attention_mask is None:
        return True
    if attention_mask.dim() != 4:
        return False
    if attention_mask.shape[-2] != q_len or attention_mask.shape[-1] < k_len:
        return False
    mask = attention_mask[..., :k_len]
    q_pos = max(0, k_len - q_len) + torch.arange(q_len, device=mask.device)
    k_pos = torch.arange(k_len, device=mask.device)
    causal_keep = k_pos[None, :] <= q_pos[:, None]
    if mask.dtype == torch.bool:     # boolean masks: True = attend
        violations = (~mask) & causal_keep
    else:
        violations = (mask < 0) & causal_keep
    return not bool(violations.any().item())


def validate_sparse_kernel_runtime(*, backend_name: str, device: torch.device, dtype: torch.dtype,
                                   block_size: Optional[int], has_block_list: bool = False,
                                   head_dim: Optional[int] = None, kind: Optional[str] = None
                                   ) -> tuple[bool, Optional[str]]:
    """Whether the kernel backend can run these inputs, else the reason (``sparse_config.py:167-200``)."""
    if backend_name != KERNEL_BACKEND:
        return True, None
    if device.type != "cuda":
        return False, f"{backend_name} requires a ROCm GPU tensor; current device is {device.type}."
    if dtype not in (torch.float16, torch.bfloat16):
        return False, f"{backend_name} requires float16 or bfloat16 inputs; current dtype is {dtype}."
    if head_dim is not None and head_dim not in SUPPORTED_HEAD_DIMS:
        return False, f"{backend_name} supports head dims {SUPPORTED_HEAD_DIMS}; got {head_dim}."
    if kind == "dense":
        return True, None
    if block_size is None:
        return False, f"{backend_name} requires a block-sparse schedule; block_size is None."
    if block_size not in SUPPORTED_BLOCK_SIZES:
        return False, f"{backend_name} supports block sizes {SUPPORTED_BLOCK_SIZES}; got {block_size}."
    return True, None


def _compute_pattern_stats(pattern, q_len: int, k_len: int) -> dict[str, float]:
    """Keep ratio / sparsity of a built pattern (``sparse_config.py:203-219``).

    Block-scheduled patterns report their scheduled ratio without touching a
    token mask (which may be lazy and large).
    """
    stats = {"keep_ratio": float(pattern.keep_ratio), "sparsity": 1.0 - float(pattern.keep_ratio)}
    if pattern.block_pairs is not None or pattern.kv_block_list is not None:
        return stats
    mask = pattern.mask
    if mask is None:
        return stats
    exact = float(mask.float().mean().item())
    return {"keep_ratio": exact, "sparsity": 1.0 - exact}
