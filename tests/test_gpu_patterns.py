"""GPU block-mask generators against their oracles, bit for bit, and straight into the GPU CSR builder.

* sa_bernoulli_block_mask / sa_seeded_bigbird_block_mask against the numpy restatement of the
  Philox4x64-10 generator (oracle.seeded, itself pinned to numpy's own Philox);
* sa_bigbird_block_mask (the reference's rotation hash) against the vectorised torch rows and, through
  the pattern classes, against schedules the reference's own classes wrote (tests/golden);
* the mask -> CSR step with no host round trip, against the torch packing of the same mask.
"""
import sys

import numpy as np
import pytest
import torch

from oracle import seeded as osd
from sparseattentioninfer_amd import ops
from sparseattentioninfer_amd.patterns import (BernoulliBlockPattern, BigBird2Pattern, SeededBigBirdPattern,
                                               block_mask_to_csr)
from sparseattentioninfer_amd.patterns.bigbird import bigbird_block_rows
from tests.helpers import golden_case

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("rows,nqb,nkb,qbo,p,seed", [(3, 37, 41, 0, 0.3, 1), (8, 128, 128, 0, 0.1, 17),
                                                     (2, 20, 301, 281, 0.25, 2 ** 63 + 5), (1, 5, 3, 0, 1.0, 0),
                                                     (4, 64, 64, 0, 0.0, 9)])
def test_bernoulli_generator_matches_oracle(rows, nqb, nkb, qbo, p, seed):
    _say(f"[patterns] bernoulli rows={rows} nqb={nqb} nkb={nkb} qbo={qbo} p={p}")
    got = ops.bernoulli_block_mask_gpu(rows, nqb, nkb, density=p, seed=seed, q_block_offset=qbo)
    torch.cuda.synchronize()
    want = osd.bernoulli_block_mask(rows, nqb, nkb, density=p, seed=seed, q_block_offset=qbo)
    assert got.dtype == torch.uint8 and got.shape == (rows, nqb, nkb)
    assert np.array_equal(got.cpu().numpy().astype(bool), want)
    assert set(np.unique(got.cpu().numpy()).tolist()) <= {0, 1}


@pytest.mark.parametrize("align", ["trailing", "centred"])
@pytest.mark.parametrize("rows,nqb,nkb,qbo,counts", [(8, 96, 96, 0, [0, 1, 2, 3, 3, 4, 6, 8]),
                                                     (2, 10, 300, 290, [5, 64]), (3, 70, 70, 0, [100, 0, 2])])
def test_seeded_bigbird_generator_matches_oracle(align, rows, nqb, nkb, qbo, counts):
    _say(f"[patterns] seeded bigbird {align} rows={rows} nqb={nqb} nkb={nkb}")
    got = ops.seeded_bigbird_block_mask_gpu(rows, nqb, nkb, window=3, global_blocks=2, random_blocks=counts,
                                            seed=7, window_align=align, q_block_offset=qbo)
    torch.cuda.synchronize()
    want = osd.seeded_bigbird_block_mask(rows, nqb, nkb, window=3, global_blocks=2, random_blocks=counts, seed=7,
                                         window_align=align, q_block_offset=qbo)
    assert np.array_equal(got.cpu().numpy().astype(bool), want)


@pytest.mark.parametrize("nqb,nkb,qbo,layout", [
    (64, 64, 0, [(1, 2, 5)] * 4),
    (33, 300, 267, [(1, 2, 3), (1, 2, 0), (2, 3, 7), (1, 1, 40)]),       # decode-like offsets, mixed layouts
    (128, 128, 0, [(1, 2, 13)] * 8),
])
def test_reference_bigbird_generator_matches_torch_rows(nqb, nkb, qbo, layout):
    _say(f"[patterns] reference bigbird nqb={nqb} nkb={nkb}")
    lay = torch.tensor(layout, dtype=torch.int32)
    got = ops.bigbird_block_mask_gpu(nqb, nkb, qbo, lay, device=DEV)
    want = bigbird_block_rows(qbo + torch.arange(nqb), torch.arange(len(layout)), nkb, lay[:, 0], lay[:, 1], lay[:, 2])
    assert torch.equal(got.cpu().bool(), want)


@pytest.mark.parametrize("name", ["bb2_t512_k128", "bb2_dec_t700_k64"])
def test_bigbird2_classes_on_gpu_match_reference_schedules(name):
    case, d = golden_case(name)
    _say(f"[patterns] {name} on the GPU")
    H, T_q, T_k = case["n_heads"], case["T_q"], case["T_k"]
    meta = BigBird2Pattern(top_k=case["params"]["top_k"], n_heads=H).build(
        torch.zeros(1, H, T_q, 8, device=DEV), torch.zeros(1, H, T_k, 8, device=DEV))
    assert torch.equal(meta.block_pairs.cpu(), torch.from_numpy(d["block_pairs"]))
    assert torch.equal(meta.block_pair_offsets.cpu(), torch.from_numpy(d["block_pair_offsets"]))
    assert torch.equal(meta.kv_block_list.cpu(), torch.from_numpy(d["kv_block_list"]))


def test_philox_patterns_build_csr_on_the_gpu():
    """The pattern classes with rng='philox': mask and CSR both built on the GPU, equal to the torch
    packing of the oracle's mask."""
    _say("[patterns] philox pattern classes")
    q = torch.zeros(1, 32, 8192, 0, device=DEV)
    k = torch.zeros(1, 8, 8192, 0, device=DEV)
    bb = SeededBigBirdPattern(rows=8, window=3, global_blocks=2, random_blocks=[0, 1, 2, 3, 3, 4, 6, 8], seed=7,
                              rng="philox").build(q, k)
    want = osd.seeded_bigbird_block_mask(8, 128, 128, window=3, global_blocks=2,
                                         random_blocks=[0, 1, 2, 3, 3, 4, 6, 8], seed=7)
    wp, wo = block_mask_to_csr(torch.from_numpy(want))
    assert bb.block_pairs.is_cuda and torch.equal(bb.block_pairs.cpu(), wp) and torch.equal(bb.block_pair_offsets.cpu(), wo)
    be = BernoulliBlockPattern(rows=8, density=0.1, seed=17, rng="philox").build(q, k)
    wp, wo = block_mask_to_csr(torch.from_numpy(osd.bernoulli_block_mask(8, 128, 128, density=0.1, seed=17)))
    assert torch.equal(be.block_pairs.cpu(), wp) and torch.equal(be.block_pair_offsets.cpu(), wo)


@pytest.mark.parametrize("rows,nqb,nkb", [(8, 512, 512), (3, 100, 37), (2, 0, 5), (2, 9, 1000)])
def test_gpu_csr_of_generated_masks(rows, nqb, nkb):
    """Word-wide (NKB % 4 == 0) and byte-wide reads of the CSR builder on generator output and on
    a strided view, including rows with no query blocks."""
    _say(f"[patterns] csr rows={rows} nqb={nqb} nkb={nkb}")
    m = ops.bernoulli_block_mask_gpu(rows, nqb, nkb, density=0.2, seed=nkb) if nqb else \
        torch.zeros(rows, 0, nkb, dtype=torch.uint8, device=DEV)
    got = block_mask_to_csr(m)
    want = block_mask_to_csr(m.cpu().bool())
    assert torch.equal(got[0].cpu(), want[0]) and torch.equal(got[1].cpu(), want[1])
    if nqb:
        wide = torch.zeros(rows, nqb, nkb + 5, dtype=torch.uint8, device=DEV)
        wide[:, :, 1:1 + nkb] = m
        got = block_mask_to_csr(wide[:, :, 1:1 + nkb])
        assert torch.equal(got[0].cpu(), want[0]) and torch.equal(got[1].cpu(), want[1])
