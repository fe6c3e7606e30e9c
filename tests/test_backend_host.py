"""Backend registry, the injected fallback and loud failure paths, on the CPU."""
from types import SimpleNamespace

import pytest
import torch

from sparseattentioninfer_amd import ops
from sparseattentioninfer_amd.attention import BACKEND_NAME, HipBlockSparseBackend, get_backend, register_into
from sparseattentioninfer_amd.patterns import PatternMetadata


def get_backend_from(registry, name, **kwargs):
    """The reference's get_backend over another registry dict (attention/__init__.py:17-21)."""
    return registry[name](**kwargs)


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
    with pytest.raises(RuntimeError, match="no fallback backend was given"):
        get_backend(BACKEND_NAME).forward(q, q, q, meta)
    with pytest.raises(AssertionError, match="requires CUDA tensors"):
        ops.universal_sparse_attn(q, q, q, meta.block_pairs, meta.block_pair_offsets, 64)


def test_topk_kind_is_rejected():
    meta = PatternMetadata(kind="topk", topk=8)
    with pytest.raises((NotImplementedError, RuntimeError)):
        get_backend(BACKEND_NAME).forward(torch.zeros(1, 1, 4, 64), torch.zeros(1, 1, 4, 64),
                                          torch.zeros(1, 1, 4, 64), meta)


class _StandInMasked:
    """Stands in for the reference's ``MaskedSdpaBackend``: records what it was handed."""

    def __init__(self):
        self.calls = []

    def forward(self, q, k, v, pattern):
        self.calls.append((q.shape, k.shape, v.shape, q.dtype, pattern.kind))
        return torch.full_like(q, 7.0)


def _csr_meta(H=2):
    return PatternMetadata(kind="mask", block_size=64, block_pairs=torch.zeros(H, 1, dtype=torch.int32),
                           block_pair_offsets=torch.tensor([[0, 1]] * H, dtype=torch.int32))


@pytest.mark.parametrize("what", ["cpu_bf16", "cpu_fp32", "topk", "no_block_size", "no_schedule"])
def test_injected_fallback_takes_what_the_kernels_cannot(what):
    """The reference backends' contract (triton_universal_backend.py:47-66): inputs the kernel
    cannot take run the masked backend and actual_backend reads "masked_sdpa_fallback"."""
    q = torch.zeros(1, 4, 64, 64, dtype=torch.float32 if what == "cpu_fp32" else torch.bfloat16)
    kv = torch.zeros(1, 2, 64, 64, dtype=q.dtype)           # GQA: repeated before the fallback
    meta = {"topk": PatternMetadata(kind="topk", topk=8),
            "no_block_size": PatternMetadata(kind="mask", block_size=None,
                                             block_pairs=torch.zeros(4, 1, dtype=torch.int32),
                                             block_pair_offsets=torch.tensor([[0, 1]] * 4, dtype=torch.int32)),
            "no_schedule": PatternMetadata(kind="mask", block_size=64)}.get(what, _csr_meta(4))
    reg = {}
    cls = register_into(reg, fallback=_StandInMasked)
    be = get_backend_from(reg, BACKEND_NAME)
    assert isinstance(be, cls)
    out = be.forward(q, kv, kv, meta)
    assert be.actual_backend == "masked_sdpa_fallback"
    assert torch.equal(out, torch.full_like(q, 7.0))
    (qs, ks, vs, dt, kind), = be._fallback.calls
    assert qs == ks == vs == (1, 4, 64, 64) and dt == q.dtype and kind == meta.kind


def _gpu_like(dtype=torch.bfloat16, head_dim=64):
    """What unsupported_reason reads of a GPU tensor (no GPU here)."""
    return SimpleNamespace(is_cuda=True, dtype=dtype, size=lambda d: head_dim if d == -1 else 1)


def test_fallback_instance_and_no_fallback_still_raises():
    fb = _StandInMasked()
    q = torch.zeros(1, 2, 64, 64)
    out = HipBlockSparseBackend(fallback=fb).forward(q, q, q, _csr_meta())
    assert len(fb.calls) == 1 and out[0, 0, 0, 0] == 7.0
    be = HipBlockSparseBackend()
    with pytest.raises(ValueError, match="no fallback backend"):
        be._run_fallback(_gpu_like(), q, q, PatternMetadata(kind="mask", block_size=None), "pattern.block_size is None")


def test_reasons_name_each_unsupported_input():
    bf = torch.zeros(1, 1, 4, 64, dtype=torch.bfloat16)
    reason = HipBlockSparseBackend.unsupported_reason
    assert "CPU" in reason(bf, _csr_meta(1))
    assert "top-k" in reason(_gpu_like(), PatternMetadata(kind="topk", topk=2))
    assert "float32" in reason(_gpu_like(torch.float32), _csr_meta(1))
    assert "block_size" in reason(_gpu_like(), PatternMetadata(kind="mask", block_size=None))
    assert "schedule" in reason(_gpu_like(), PatternMetadata(kind="mask", block_size=64))
    assert reason(_gpu_like(), PatternMetadata(kind="dense")) is None
    assert "head dim 96" in reason(_gpu_like(head_dim=96), PatternMetadata(kind="dense"))
    assert reason(_gpu_like(torch.float16), _csr_meta(1)) is None
