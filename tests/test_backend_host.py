"""Backend registry and loud failure paths, on the CPU."""
import pytest
import torch

from sparseattentioninfer_amd import ops
from sparseattentioninfer_amd.attention import BACKEND_NAME, get_backend, register_into
from sparseattentioninfer_amd.patterns import PatternMetadata


def test_registry_and_unknown_name():
    be = get_backend(BACKEND_NAME)
    assert be.actual_backend == "unknown"
    with pytest.raises(ValueError, match="Available: hip_block_sparse"):
        get_backend("triton_universal")
    reg = {}
    register_into(reg)
    assert reg[BACKEND_NAME] is type(be)


def test_cpu_tensors_raise_instead_of_falling_back():
    q = torch.zeros(1, 2, 64, 64, dtype=torch.bfloat16)
    meta = PatternMetadata(kind="mask", block_size=64, block_pairs=torch.zeros(2, 1, dtype=torch.int32),
                           block_pair_offsets=torch.tensor([[0, 1]] * 2, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        get_backend(BACKEND_NAME).forward(q, q, q, meta)
    with pytest.raises(AssertionError, match="requires CUDA tensors"):
        ops.universal_sparse_attn(q, q, q, meta.block_pairs, meta.block_pair_offsets, 64)


def test_topk_kind_is_rejected():
    meta = PatternMetadata(kind="topk", topk=8)
    with pytest.raises((NotImplementedError, RuntimeError)):
        get_backend(BACKEND_NAME).forward(torch.zeros(1, 1, 4, 64), torch.zeros(1, 1, 4, 64),
                                          torch.zeros(1, 1, 4, 64), meta)
