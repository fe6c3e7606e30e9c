"""MI355X-native (gfx950) block-sparse attention backend.

Hot path: ``ops.universal_sparse_attn`` (block-sparse prefill over a CSR
schedule, bf16/fp16 MFMA) and ``ops.paged_sparse_decode`` (memory-bound
sparse decode), behind ``attention.get_backend("hip_block_sparse")``.
The HIP library is loaded lazily on the first kernel call.
"""
from . import ops
from .attention import HipBlockSparseBackend, get_backend
from .patterns import PatternMetadata

__all__ = ["ops", "HipBlockSparseBackend", "get_backend", "PatternMetadata"]
