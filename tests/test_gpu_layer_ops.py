"""Fused decode-layer kernels (sa_rmsnorm, sa_qk_rope_kv, sa_swiglu) against the Hugging Face Qwen3 modules
they replace, at the Qwen3-4B sizes (hidden 2560, 32Q/8KV heads of 128, SwiGLU 9728), batch 8.  The
kernels keep Hugging Face's roundings, so every element must be within one or two bf16 ulps (reductions
may sum in another order); page writes must land in the right (page, head, slot)."""
import sys

import pytest
import torch
import torch.nn.functional as F
from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm, Qwen3RotaryEmbedding, apply_rotary_pos_emb

from sparseattentioninfer_amd import ops
from sparseattentioninfer_amd.models.kv_cache import PagedKVStore
from sparseattentioninfer_amd.qwen3.runtime import qwen3_config
from tests.helpers import assert_within_ulps

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _rand(*shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16).to(DEV)


@pytest.mark.parametrize("with_residual", [False, True])
@pytest.mark.parametrize("dtype,n", [(torch.bfloat16, 2560), (torch.float16, 2560), (torch.bfloat16, 8192),
                                     (torch.bfloat16, 200)])
def test_rmsnorm_matches_qwen3_rmsnorm(with_residual, dtype, n):
    """HF's Qwen3RMSNorm (and residual add) at the Qwen3-4B width, in fp16, at the largest width (four
    16-byte chunks per thread) and at a width that leaves most threads without a chunk."""
    _say(f"[layer-ops] rmsnorm residual={with_residual} {dtype} n={n}")
    B, eps = 8, 1e-6
    norm = Qwen3RMSNorm(n, eps=eps).to(DEV, dtype)
    with torch.no_grad():
        norm.weight.copy_(_rand(n, seed=1, scale=0.5) + 1)
    x, res = _rand(B, n, seed=2, scale=3.0).to(dtype), _rand(B, n, seed=3).to(dtype)
    r = res.clone()
    out = ops.rmsnorm(x, norm.weight, eps, residual=r if with_residual else None)
    src = (res + x) if with_residual else x
    with torch.no_grad():
        want = norm(src)
    if with_residual:
        assert torch.equal(r, res + x)
    # The mean of squares is summed in another order than torch's reduction; fp16's finer rounding can
    # turn the last-bit difference of 1/rms into one more ulp of the output than bf16's.
    assert_within_ulps(out, want, 1 if dtype == torch.bfloat16 else 2, "rmsnorm")


def test_qk_rope_kv_matches_hf_attention_prologue():
    _say("[layer-ops] qk_rope_kv")
    cfg = qwen3_config()
    B, Hq, Hkv, D, page, eps = 8, 32, 8, 128, 64, 1e-6
    qn, kn = (Qwen3RMSNorm(D, eps=eps).to(DEV, torch.bfloat16) for _ in range(2))
    with torch.no_grad():
        qn.weight.copy_(_rand(D, seed=4, scale=0.3) + 1)
        kn.weight.copy_(_rand(D, seed=5, scale=0.3) + 1)
    rope = Qwen3RotaryEmbedding(cfg).to(DEV)
    qkv = _rand(B, (Hq + 2 * Hkv) * D, seed=6, scale=2.0)
    store = PagedKVStore(B, Hkv, D, 9000, page=page, dtype=torch.bfloat16, device=DEV, shuffle_seed=9)
    store.k_pages.zero_()
    store.v_pages.zero_()
    for p in (0, 63, 64, 8191, 8990):
        store._grow_all(p + 1)
        pos = torch.tensor([p], dtype=torch.int64, device=DEV)
        q_out = torch.empty(B, Hq, D, dtype=torch.bfloat16, device=DEV)
        ops.qk_rope_kv(qkv, qn.weight, kn.weight, rope.inv_freq.float(), pos, store, q_out, num_heads=Hq, eps=eps)
        with torch.no_grad():
            q = qn(qkv[:, :Hq * D].view(B, 1, Hq, D)).transpose(1, 2)
            k = kn(qkv[:, Hq * D:(Hq + Hkv) * D].view(B, 1, Hkv, D)).transpose(1, 2)
            v = qkv[:, (Hq + Hkv) * D:].view(B, 1, Hkv, D).transpose(1, 2)
            cos, sin = rope(qkv.view(B, 1, -1), pos.view(1, 1))
            q, k = apply_rotary_pos_emb(q, k, cos, sin)
        assert_within_ulps(q_out, q[:, :, 0], 2, f"q at position {p}")
        pg = store.block_table[:, p // page].long()
        assert_within_ulps(store.k_pages[pg, :, p % page], k[:, :, 0], 2, f"k page at position {p}")
        assert torch.equal(store.v_pages[pg, :, p % page], v[:, :, 0]), f"v page at position {p}"
    # only the written slots changed
    written = (store.k_pages != 0).any(dim=-1).sum().item()
    assert written == 5 * B * Hkv


def test_swiglu_matches_silu_times_up():
    _say("[layer-ops] swiglu")
    B, I = 8, 9728
    gu = _rand(B, 2 * I, seed=7, scale=3.0)
    out = ops.swiglu(gu)
    want = F.silu(gu[:, :I]) * gu[:, I:]
    assert_within_ulps(out, want, 1, "swiglu")


# The decode shapes of Qwen3-4B (q|k|v, gate|up and the LM head on the LDS-staged matrix-core
# kernel, o and down on the dot-product kernel), the matrix-core kernel with M < 8, ragged N and
# one 128-wide K stage, then M < 8 with ragged N, the largest K (10240) and K not a multiple of 64
# on the dot-product kernel.
@pytest.mark.parametrize("M,N,K", [(8, 6144, 2560), (8, 2560, 4096), (8, 19456, 2560), (8, 2560, 9728),
                                   (8, 151936, 2560), (5, 6200, 1280), (1, 6150, 128), (5, 1000, 1024),
                                   (2, 300, 10240), (8, 2560, 4160), (3, 100, 2056), (1, 37, 8)])
def test_skinny_gemm_matches_fp32_product(M, N, K):
    _say(f"[layer-ops] gemm_skinny M={M} N={N} K={K}")
    x = _rand(M, K, seed=10 + M)
    w = _rand(N, K, seed=20 + N % 97, scale=0.05)
    out = ops.gemm_skinny(x, w).float()
    want = x.float() @ w.float().t()
    # one rounding of the output (half an ulp of bf16) plus fp32 summation in another order, which is
    # bounded by a small multiple of sum_k |x w| (it matters only where the sum nearly cancels)
    ulp = torch.exp2(torch.floor(torch.log2(want.abs().clamp_min(1e-30))) - 7)
    bound = 0.5 * ulp + 1e-5 * (x.float().abs() @ w.float().abs().t())
    bad = (out - want).abs() > bound
    assert not bad.any(), f"{int(bad.sum())} of {out.numel()} outputs beyond the bound"


@pytest.mark.parametrize("M,N,K", [(8, 2560, 4096), (4, 77, 264), (8, 6144, 2560)])
def test_skinny_gemm_fp16(M, N, K):
    """fp16 on both kernels (N = 2560 and 6144) and at a small ragged shape."""
    _say(f"[layer-ops] gemm_skinny fp16 M={M} N={N} K={K}")
    x = _rand(M, K, seed=30 + M).to(torch.float16)
    w = (_rand(N, K, seed=40 + N % 97, scale=0.05)).to(torch.float16)
    out = ops.gemm_skinny(x, w).float()
    want = x.float() @ w.float().t()
    ulp = torch.exp2(torch.floor(torch.log2(want.abs().clamp_min(1e-30))) - 10)
    bound = 0.5 * ulp + 1e-5 * (x.float().abs() @ w.float().abs().t())
    bad = (out - want).abs() > bound
    assert not bad.any(), f"{int(bad.sum())} of {out.numel()} outputs beyond the bound"


@pytest.mark.parametrize("M,I,K,dtype", [(8, 9728, 2560, torch.bfloat16), (5, 3100, 1280, torch.bfloat16),
                                         (1, 3072, 128, torch.bfloat16), (8, 9728, 2560, torch.float16)])
def test_gemm_skinny_swiglu(M, I, K, dtype):
    """Gate|up product with the SwiGLU in its epilogue, on interleaved weights, gives the bits of the
    product on the concatenated weights followed by sa_swiglu (both products on the matrix-core
    kernel, which holds for 2I >= 24 columns per CU); with a ragged last column tile and a single
    128-wide K stage."""
    _say(f"[layer-ops] gemm_skinny_swiglu M={M} I={I} K={K} {dtype}")
    x = _rand(M, K, seed=130 + M).to(dtype)
    gate = _rand(I, K, seed=140 + I % 97, scale=0.05).to(dtype)
    up = _rand(I, K, seed=150 + I % 97, scale=0.05).to(dtype)
    fused = ops.gemm_skinny_swiglu(x, ops.interleave_gate_up(gate, up))
    two = ops.swiglu(ops.gemm_skinny(x, torch.cat([gate, up], 0).contiguous()))
    # The fused product always runs on the matrix-core kernel; the plain product does when K is a
    # multiple of 128 and N = 2I >= 24 columns per CU (layer_ops.hip's dispatch), which depends on the
    # part's CU count.  Same kernel: the same bits; otherwise the dot-product kernel sums K in another
    # order, and the results agree to a bf16/fp16 ulp of the SwiGLU output.
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if K % 128 == 0 and 2 * I >= 24 * cus:
        assert torch.equal(fused, two)
    else:
        assert_within_ulps(fused, two, 1, "fused vs two-step SwiGLU (different product kernels)")
