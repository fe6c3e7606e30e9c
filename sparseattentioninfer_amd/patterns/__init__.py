"""Pattern layer: metadata, CSR builders and the benchmark generators."""
from .base import (PatternMetadata, SparsePattern, block_mask_to_csr, build_block_pairs_from_mask,
                   causal_block_keep_ratio, coarsen_token_mask, csr_to_block_mask,
                   kv_block_list_to_pairs)
from .seeded import (BernoulliBlockPattern, SeededBigBirdPattern, bernoulli_block_mask,
                     decode_selection, seeded_bigbird_block_mask)

__all__ = [
    "PatternMetadata", "SparsePattern", "block_mask_to_csr", "build_block_pairs_from_mask",
    "causal_block_keep_ratio", "coarsen_token_mask", "csr_to_block_mask", "kv_block_list_to_pairs",
    "BernoulliBlockPattern", "SeededBigBirdPattern", "bernoulli_block_mask", "decode_selection",
    "seeded_bigbird_block_mask",
]
