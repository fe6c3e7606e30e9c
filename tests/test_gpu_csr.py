"""The GPU block-mask -> CSR builder (sa_block_mask_to_csr) against the torch packing and the
reference's own schedules: bit-exact pairs, offsets and width."""
import sys

import pytest
import torch

from sparseattentioninfer_amd import ops
from sparseattentioninfer_amd.patterns import (BigBirdKeepRatioPattern, BigBirdPattern, bernoulli_block_mask,
                                               block_mask_to_csr, build_block_pairs_from_mask)
from tests.helpers import golden_case

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _same(gpu, cpu):
    (gp, go), (cp, co) = gpu, cpu
    assert gp.device.type == "cuda" and gp.dtype == torch.int32 and go.dtype == torch.int32
    assert gp.shape == cp.shape and go.shape == co.shape
    assert torch.equal(gp.cpu(), cp) and torch.equal(go.cpu(), co)


@pytest.mark.parametrize("R,nqb,nkb,density", [(3, 37, 41, 0.3), (8, 600, 600, 0.02), (2, 5, 1, 0.5),
                                                (4, 300, 16, 0.0), (1, 257, 64, 1.0)])
def test_gpu_builder_matches_torch_packing(R, nqb, nkb, density):
    _say(f"[csr] R={R} nqb={nqb} nkb={nkb} density={density}")
    g = torch.Generator().manual_seed(R * 1000 + nqb)
    bm = torch.rand(R, nqb, nkb, generator=g) < density
    if R > 1:
        bm[1] = False                  # an empty row
    cpu = block_mask_to_csr(bm)
    _same(ops.block_mask_to_csr_gpu(bm.to(DEV)), cpu)
    _same(block_mask_to_csr(bm.to(DEV)), cpu)       # the pattern layer dispatches GPU masks here
    # strided (non-contiguous) view of a larger mask
    big = torch.zeros(R, nqb, nkb + 7, dtype=torch.bool)
    big[:, :, 3:3 + nkb] = bm
    _same(ops.block_mask_to_csr_gpu(big.to(DEV)[:, :, 3:3 + nkb]), cpu)


def test_causal_bernoulli_at_configs1_shape():
    _say("[csr] configs[1] schedule")
    bm = bernoulli_block_mask(8, 128, 128, density=0.1, seed=3)
    _same(block_mask_to_csr(bm.to(DEV)), block_mask_to_csr(bm))


def test_token_mask_builder_on_gpu():
    _say("[csr] token mask")
    case, d = golden_case("bb_t1000_k256")
    mask = torch.from_numpy(d["mask"])
    cpu = build_block_pairs_from_mask(mask, case["block_size"])
    _same(build_block_pairs_from_mask(mask.to(DEV), case["block_size"]), cpu)
    assert torch.equal(cpu[0], torch.from_numpy(d["block_pairs"]))


@pytest.mark.parametrize("name", ["bb_t512_k128", "bb_t4096_k2048", "bb_t1500_k1024", "bb_dec_t777_k256"])
def test_reference_bigbird_schedule_built_on_gpu(name):
    """BigBirdPattern run on GPU tensors reproduces the reference-written CSR bit for bit."""
    case, d = golden_case(name)
    _say(f"[csr] {name} on the GPU")
    H, T_q, T_k = case["n_heads"], case["T_q"], case["T_k"]
    q = torch.zeros(1, H, T_q, 8, device=DEV)
    k = torch.zeros(1, H, T_k, 8, device=DEV)
    meta = BigBirdPattern(top_k=case["params"]["top_k"], n_heads=H).build(q, k)
    assert meta.block_pairs.is_cuda and meta.block_size == case["block_size"]
    assert torch.equal(meta.block_pairs.cpu(), torch.from_numpy(d["block_pairs"]))
    assert torch.equal(meta.block_pair_offsets.cpu(), torch.from_numpy(d["block_pair_offsets"]))


def test_reference_keep_ratio_groups_built_on_gpu():
    case, d = golden_case("kr_groups_t1024")
    _say("[csr] kr_groups_t1024 on the GPU")
    H = case["n_heads"]
    p = case["params"]
    pat = BigBirdKeepRatioPattern(group_sparsities=p["group_sparsities"], n_heads=H, n_kv_heads=p["n_kv_heads"])
    q = torch.zeros(1, H, case["T_q"], 8, device=DEV)
    meta = pat.build(q, torch.zeros(1, H, case["T_k"], 8, device=DEV))
    assert torch.equal(meta.block_pairs.cpu(), torch.from_numpy(d["block_pairs"]))
    assert torch.equal(meta.block_pair_offsets.cpu(), torch.from_numpy(d["block_pair_offsets"]))
