"""Configuration of the Qwen3 sparse-attention integration.

The integration reads the reference's ``config.sparse_attention_*`` attributes
(``sparse_llm/qwen3/integrations/sparse_config.py``).  This module organises them its own way:

* :class:`GroupSparsitySpec` holds the per-KV-group sparsities of a model -- one default tuple
  and optional per-layer overrides -- validates them once, resolves the precedence the
  reference applies (explicit argument, then per-layer config, then model-wide config) in
  :meth:`GroupSparsitySpec.for_layer`, writes them back to a config as JSON-friendly lists and
  parses the command-line forms (``"0.5,0.7"``; a JSON list inline or in a file);
* :func:`validate_sparse_kernel_runtime` (the reference's public check, ``:167-200``) states
  the conditions of the gfx950 backend; ``"auto"`` resolves to that backend for every pattern;
* :func:`is_plain_causal_mask`, :func:`describe_pattern` and :func:`pattern_stats` serve the
  attention module.

A ROCm GPU tensor reports ``device.type == "cuda"``.
"""
from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path
from typing import Optional

import torch

KERNEL_BACKEND = "hip_block_sparse"
SUPPORTED_BLOCK_SIZES = (16, 32, 64, 128)
SUPPORTED_HEAD_DIMS = (64, 128)

Sparsities = tuple[float, ...]


def config_value(config, name: str, default):
    """``config.<name>``, or ``default`` where the config does not carry it."""
    return getattr(config, name, default)


def _as_sparsities(values, where: str) -> Optional[Sparsities]:
    if values is None:
        return None
    out = tuple(float(x) for x in values)
    outside = [x for x in out if not 0.0 <= x < 1.0]
    if outside:
        raise ValueError(f"{where} values must satisfy 0 <= sparsity < 1 (got {outside}).")
    return out


@dataclass(frozen=True)
class GroupSparsitySpec:
    """Per-KV-group sparsities: ``default`` for every layer, ``per_layer[i]`` (or None) for layer i."""

    default: Optional[Sparsities] = None
    per_layer: Optional[tuple[Optional[Sparsities], ...]] = None

    @classmethod
    def build(cls, default=None, per_layer=None, *, where: str = "group_sparsities") -> "GroupSparsitySpec":
        layers = None
        if per_layer is not None:
            layers = tuple(None if entry is None else _as_sparsities(entry, f"layer_{where}[{i}]")
                           for i, entry in enumerate(per_layer))
        return cls(_as_sparsities(default, where), layers)

    @classmethod
    def from_config(cls, config) -> "GroupSparsitySpec":
        return cls.build(config_value(config, "sparse_attention_group_sparsities", None),
                         config_value(config, "sparse_attention_layer_group_sparsities", None),
                         where="config.sparse_attention_group_sparsities")

    def overridden_by(self, other: "GroupSparsitySpec") -> "GroupSparsitySpec":
        """``other``'s entries where it has them, else this spec's."""
        return GroupSparsitySpec(other.default if other.default is not None else self.default,
                                 other.per_layer if other.per_layer is not None else self.per_layer)

    @classmethod
    def with_config_defaults(cls, config, default=None, per_layer=None) -> "GroupSparsitySpec":
        """The arguments, each validated, with the config's value standing in for an argument that
        is None; a config value is validated only when it is used, as the reference's
        ``replace_qwen3_attention_with_sparse`` does (``modeling_sparse_qwen3.py:358-376``)."""
        spec = cls.build(default, per_layer)
        if spec.default is None:
            spec = cls(_as_sparsities(config_value(config, "sparse_attention_group_sparsities", None),
                                      "config.sparse_attention_group_sparsities"), spec.per_layer)
        if spec.per_layer is None:
            spec = cls(spec.default, cls.build(None, config_value(config, "sparse_attention_layer_group_sparsities",
                                                                   None),
                                               where="config.sparse_attention_group_sparsities").per_layer)
        return spec

    @staticmethod
    def resolve_layer(config, layer_idx: int) -> Optional[Sparsities]:
        """A layer's sparsities from the config alone: its per-layer entry (the whole per-layer list is
        validated), else the model-wide default, validated only when it is the one used
        (``modeling_sparse_qwen3.py:123-141``)."""
        layers = GroupSparsitySpec.build(None, config_value(config, "sparse_attention_layer_group_sparsities", None),
                                         where="config.sparse_attention_group_sparsities").per_layer
        if layers is not None and layer_idx < len(layers) and layers[layer_idx] is not None:
            return layers[layer_idx]
        return _as_sparsities(config_value(config, "sparse_attention_group_sparsities", None),
                              "config.sparse_attention_group_sparsities")

    def for_layer(self, layer_idx: int) -> Optional[Sparsities]:
        if self.per_layer is not None and layer_idx < len(self.per_layer) \
                and self.per_layer[layer_idx] is not None:
            return self.per_layer[layer_idx]
        return self.default

    def write_to(self, config) -> None:
        """Stores the spec on a config as plain lists (JSON-serialisable)."""
        if self.default is not None:
            config.sparse_attention_group_sparsities = list(self.default)
        if self.per_layer is not None:
            config.sparse_attention_layer_group_sparsities = [None if e is None else list(e) for e in self.per_layer]

    @staticmethod
    def parse_groups(text: Optional[str]) -> Optional[Sparsities]:
        """Command-line form ``"0.5, 0.7"``; None or blank -> None."""
        if text is None or not text.strip():
            return None
        return _as_sparsities([t for t in (p.strip() for p in text.split(",")) if t], "--group-sparsities")

    @staticmethod
    def parse_layers(text_or_path: Optional[str]) -> Optional[tuple[Optional[Sparsities], ...]]:
        """A JSON list of per-layer lists (or nulls), inline or in a file."""
        if text_or_path is None:
            return None
        src = Path(text_or_path)
        doc = json.loads(src.read_text(encoding="utf-8") if src.is_file() else text_or_path)
        if not isinstance(doc, list):
            raise ValueError("--layer-group-sparsities must decode to a JSON list.")
        return GroupSparsitySpec.build(None, doc, where="--layer-group-sparsities").per_layer


def ensure_attn_implementation(config) -> None:
    """Hugging Face needs an attention implementation name; the sparse layers replace it anyway."""
    if getattr(config, "_attn_implementation", None) is None:
        config._attn_implementation = "sdpa"


def backend_candidates(backend_name: str) -> list[str]:
    """Backends a layer may use, in order: the named one, or the kernel backend for ``"auto"``."""
    return [KERNEL_BACKEND] if backend_name == "auto" else [backend_name]


_DESCRIBED = ("top_k", "keep_ratio", "group_sparsities", "window_size", "window", "global_blocks",
              "random_blocks", "block_size", "seed", "last_layout", "last_group_layouts")


def describe_pattern(attn) -> str:
    """``PatternClass(field=value, ...)`` for the parameters a layer's pattern carries."""
    p = attn.sparse_pattern
    fields = ", ".join(f"{f}={getattr(p, f)}" for f in _DESCRIBED if getattr(p, f, None) is not None)
    return f"{type(p).__name__}({fields})"


def is_plain_causal_mask(attention_mask: Optional[torch.Tensor], q_len: int, k_len: int) -> bool:
    """Whether an attention mask hides nothing that the bottom-right aligned causal mask shows.

    Accepts None, a 4-d additive float mask (negative = hidden) or a 4-d bool mask
    (True = attend) of ``q_len`` rows and at least ``k_len`` columns.
    """
    if attention_mask is None:
        return True
    m = attention_mask
    if m.dim() != 4 or m.size(-2) != q_len or m.size(-1) < k_len:
        return False
    m = m[..., :k_len]
    shown = torch.ones(q_len, k_len, dtype=torch.bool, device=m.device).tril(max(0, k_len - q_len))
    hidden = ~m if m.dtype == torch.bool else m < 0
    return not bool((hidden & shown).any())


def validate_sparse_kernel_runtime(*, backend_name: str, device: torch.device, dtype: torch.dtype,
                                   block_size: Optional[int], has_block_list: bool = False,
                                   head_dim: Optional[int] = None, kind: Optional[str] = None
                                   ) -> tuple[bool, Optional[str]]:
    """Whether the kernel backend can run these inputs, else the reason (``sparse_config.py:167-200``)."""
    if backend_name != KERNEL_BACKEND:
        return True, None
    checks = [
        (device.type == "cuda", f"requires a ROCm GPU tensor; current device is {device.type}."),
        (dtype in (torch.float16, torch.bfloat16), f"requires float16 or bfloat16 inputs; current dtype is {dtype}."),
        (head_dim is None or head_dim in SUPPORTED_HEAD_DIMS, f"supports head dims {SUPPORTED_HEAD_DIMS}; got {head_dim}."),
        (kind == "dense" or block_size is not None, "requires a block-sparse schedule; block_size is None."),
        (kind == "dense" or block_size is None or block_size in SUPPORTED_BLOCK_SIZES,
         f"supports block sizes {SUPPORTED_BLOCK_SIZES}; got {block_size}."),
    ]
    for ok, why in checks:
        if not ok:
            return False, f"{backend_name} {why}"
    return True, None


def pattern_stats(pattern) -> dict[str, float]:
    """Keep ratio and sparsity of a built pattern.

    Block-scheduled patterns report their scheduled ratio; only a pattern with nothing but a
    token mask has its ratio measured from the mask (a lazy mask would otherwise be built).
    """
    keep = float(pattern.keep_ratio)
    scheduled = pattern.block_pairs is not None or pattern.kv_block_list is not None
    if not scheduled and pattern.mask is not None:
        keep = float(pattern.mask.float().mean().item())
    return {"keep_ratio": keep, "sparsity": 1.0 - keep}

