"""Pattern layer: metadata, CSR builders, the reference's pattern classes and the benchmark generators."""
from .base import (PatternMetadata, SparsePattern, block_mask_to_csr, build_block_pairs_from_mask,
                   causal_block_keep_ratio, coarsen_token_mask, csr_to_block_mask,
                   kv_block_list_to_pairs)
from .bigbird import (BigBird2Pattern, BigBirdKeepRatioPattern, BigBirdPattern, LazyMaskMetadata,
                      bigbird_block_rows, bigbird_layout_from_keep_ratio, bigbird_layout_from_topk,
                      next_pow2_min16)
from .causal_dense import DenseCausalPattern
from .local_window import LocalWindowPattern, local_window_block_mask, local_window_token_mask
from .seeded import (BernoulliBlockPattern, SeededBigBirdPattern, bernoulli_block_mask,
                     decode_selection, seeded_bigbird_block_mask)

__all__ = [
    "PatternMetadata", "SparsePattern", "block_mask_to_csr", "build_block_pairs_from_mask",
    "causal_block_keep_ratio", "coarsen_token_mask", "csr_to_block_mask", "kv_block_list_to_pairs",
    "BigBirdPattern", "BigBird2Pattern", "BigBirdKeepRatioPattern", "LazyMaskMetadata",
    "bigbird_block_rows", "bigbird_layout_from_keep_ratio", "bigbird_layout_from_topk", "next_pow2_min16",
    "DenseCausalPattern", "LocalWindowPattern", "local_window_block_mask", "local_window_token_mask",
    "BernoulliBlockPattern", "SeededBigBirdPattern", "bernoulli_block_mask", "decode_selection",
    "seeded_bigbird_block_mask",
]
