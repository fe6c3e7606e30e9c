"""Block-16/32 schedules on the GPU: the CSR -> 64 x 64 tile regrouping (sa_csr_to_tiles) and
prefill over it, against the oracle and against the reference's own BigBird schedules."""
import sys

import numpy as np
import pytest
import torch

from oracle import attention as oa
from sparseattentioninfer_amd import ops
from sparseattentioninfer_amd.attention import get_backend
from sparseattentioninfer_amd.patterns import (PatternMetadata, bernoulli_block_mask, block_mask_to_csr,
                                               seeded_bigbird_block_mask)
from tests.helpers import assert_close_bf16, golden_case, seeded

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _dense_tiles(pairs, offsets, bs):
    """Tile schedule of a CSR computed through its dense block mask (not the kernel's list merge):
    per row, (tile ids, masks, offsets) with mask bit (qb % s) * s + (kb % s)."""
    pairs, offsets = np.asarray(pairs), np.asarray(offsets)
    R, nqb = offsets.shape[0], offsets.shape[1] - 1
    s = 64 // bs
    nkb = max(int(pairs.max()) + 1 if pairs.size else 1, 1)
    bm = np.zeros((R, nqb, nkb), bool)
    for r in range(R):
        for qb in range(nqb):
            ids = pairs[r, offsets[r, qb]:offsets[r, qb + 1]]
            bm[r, qb, ids[ids >= 0]] = True
    nqt, nkt = -(-nqb // s), -(-nkb // s)
    pad = np.zeros((R, nqt * s, nkt * s), bool)
    pad[:, :nqb, :nkb] = bm
    sub = pad.reshape(R, nqt, s, nkt, s).transpose(0, 1, 3, 2, 4).reshape(R, nqt, nkt, s * s)
    masks = (sub.astype(np.int64) << np.arange(s * s)).sum(-1)
    rows = []
    for r in range(R):
        tp, tm, to = [], [], [0]
        for qt in range(nqt):
            kts = np.nonzero(masks[r, qt])[0]
            tp += kts.tolist()
            tm += masks[r, qt, kts].tolist()
            to.append(len(tp))
        rows.append((tp, tm, to))
    return rows


def _check_tiles(pairs, offsets, bs):
    ts = ops.csr_to_tiles(pairs.to(DEV), offsets.to(DEV), bs)
    torch.cuda.synchronize()
    assert ts.status.item() == 0
    tp, tm, to = ts.pairs.cpu().numpy(), ts.masks.cpu().numpy(), ts.offsets.cpu().numpy()
    for r, (wp, wm, wo) in enumerate(_dense_tiles(pairs.numpy(), offsets.numpy(), bs)):
        assert to[r].tolist() == wo, f"row {r} offsets"
        n = wo[-1]
        assert tp[r, :n].tolist() == wp and tm[r, :n].tolist() == wm, f"row {r} tiles"
        assert not tp[r, n:].any() and not tm[r, n:].any(), f"row {r} padding"


@pytest.mark.parametrize("bs", [16, 32])
@pytest.mark.parametrize("nqb,density", [(37, 0.3), (64, 0.05), (1200, 0.01)])
def test_csr_to_tiles_matches_dense_regrouping(bs, nqb, density):
    """Ragged last tile (37 blocks), and more than 256 query tiles per row (1200 blocks of 16)."""
    _say(f"[tiles] bs={bs} nqb={nqb}")
    bm = bernoulli_block_mask(3, nqb, nqb, density=density, seed=nqb)
    bm[1] = False  # an empty row
    bm[1, nqb // 2, :3] = True
    _check_tiles(*block_mask_to_csr(bm), bs)


def test_csr_to_tiles_drops_negative_ids_and_handles_empty_rows():
    _say("[tiles] negative ids")
    pairs = torch.tensor([[0, -1, 1, -5, 2, 0, 3, 7],
                          [0, 0, 0, 0, 0, 0, 0, 0]], dtype=torch.int32)
    offsets = torch.tensor([[0, 1, 3, 5, 8],
                            [0, 0, 0, 0, 0]], dtype=torch.int32)
    _check_tiles(pairs, offsets, 16)
    ts = ops.csr_to_tiles(pairs.to(DEV), offsets.to(DEV), 16).check()
    # query blocks 0..3 = query tile 0: blocks {0}, {1}, {2}, {0, 3, 7} -> tiles 0 and 1
    assert ts.offsets.cpu()[0].tolist() == [0, 2]
    assert ts.pairs.cpu()[0, :2].tolist() == [0, 1]
    assert ts.masks.cpu()[0, :2].tolist() == [(1 << 0) | (1 << 5) | (1 << 10) | (1 << 15) | (1 << 12),
                                              1 << (12 + 3)]


@pytest.mark.parametrize("bs", [16, 32])
def test_csr_to_tiles_negative_ids_after_tile_zero_entries(bs):
    """Negative ids inside a query block's list, right after entries of key tile 0: an id in (-s, 0)
    divided by s truncates to 0, the tile being collected, and must still be dropped rather than set
    a sub-block bit (regression: it set bit i*s - 1, a pair of another query sub-block)."""
    _say(f"[tiles] negative ids after tile 0, bs={bs}")
    s = 64 // bs
    # query blocks 0..3, ascending ids once the negatives are dropped: {0, 1}, {s-1, s}, {0}, {1, s, 2s+1}
    pairs = torch.tensor([[0, -1, 1, s - 1, -(s - 1), s, -1, 0, -1, -1, 1, -2, s, -1, 2 * s + 1, -3]],
                         dtype=torch.int32)
    offsets = torch.tensor([[0, 3, 6, 9, 16]], dtype=torch.int32)
    _check_tiles(pairs, offsets, bs)


def _mask(kind, rows, T_q, T_k, bs, seed):
    nqb, nkb = -(-T_q // bs), -(-T_k // bs)
    qbo = (T_k - T_q) // bs
    if kind.startswith("bernoulli"):
        return bernoulli_block_mask(rows, nqb, nkb, density=float(kind[9:]), seed=seed, q_block_offset=qbo)
    return seeded_bigbird_block_mask(rows, nqb, nkb, window=3, global_blocks=2, random_blocks=2, seed=seed,
                                     q_block_offset=qbo)


CASES = [
    # name, B, Hq, Hkv, T_q, T_k, D, bs, mask kind, CSR rows, dtype  (heads per CSR row -> 1, 2, 4 head tiles)
    ("b16_mha", 1, 8, 8, 1024, 1024, 128, 16, "bernoulli0.2", "q", torch.bfloat16),
    ("b32_gqa_group", 2, 8, 2, 1000, 1000, 128, 32, "bernoulli0.3", "kv", torch.bfloat16),
    ("b16_gqa2_d64", 1, 4, 2, 300, 300, 64, 16, "bigbird", "kv", torch.bfloat16),
    ("b16_group4_d64", 1, 8, 2, 700, 700, 64, 16, "bigbird", "kv", torch.bfloat16),
    ("b32_mha_ragged", 1, 4, 4, 333, 333, 128, 32, "bigbird", "q", torch.bfloat16),
    ("b16_chunk_tail", 1, 4, 2, 200, 1010, 128, 16, "bernoulli0.3", "kv", torch.bfloat16),
    ("b32_fp16_group", 1, 8, 2, 640, 640, 128, 32, "bernoulli0.2", "kv", torch.float16),
    ("b16_cfg2_slice", 1, 32, 8, 2048, 2048, 128, 16, "bernoulli0.05", "kv", torch.bfloat16),
    # four-head kernel over rows of about 94 tiles (the schedule is read 64 positions at a time) and
    # of 625 tiles (past the 512-entry LDS cache of the sub-block kernels: read from global memory)
    ("b16_long_rows", 1, 8, 2, 256, 6000, 128, 16, "bernoulli0.5", "kv", torch.bfloat16),
    ("b32_uncached_rows", 1, 4, 1, 64, 40000, 128, 32, "bernoulli0.6", "kv", torch.bfloat16),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_block16_32_prefill_matches_oracle(case):
    name, B, Hq, Hkv, T_q, T_k, D, bs, kind, rows, dtype = case
    _say(f"[prefill-b{bs}] {name}")
    R = Hq if rows == "q" else Hkv
    pairs, offsets = block_mask_to_csr(_mask(kind, R, T_q, T_k, bs, seed=13))
    q = seeded((B, Hq, T_q, D), 31, dtype).to(DEV)
    k = seeded((B, Hkv, T_k, D), 32, dtype).to(DEV)
    v = seeded((B, Hkv, T_k, D), 33, dtype).to(DEV)
    out = ops.universal_sparse_attn(q, k, v, pairs.to(DEV), offsets.to(DEV), bs)
    torch.cuda.synchronize()
    assert out.shape == (B, Hq, T_q, D) and out.dtype == dtype
    want = oa.block_sparse_attention(q, k, v, pairs, offsets, bs)
    assert torch.isfinite(out.float()).all()
    assert_close_bf16(out, want, name)


def test_prepared_block16_launch_matches_direct_call():
    _say("[prefill-b16] prepared launch")
    B, Hq, Hkv, T, D, bs = 1, 8, 2, 512, 128, 16
    pairs, offsets = (x.to(DEV) for x in block_mask_to_csr(_mask("bigbird", Hkv, T, T, bs, seed=2)))
    q = seeded((B, Hq, T, D), 41, torch.bfloat16).to(DEV)
    k = seeded((B, Hkv, T, D), 42, torch.bfloat16).to(DEV)
    v = seeded((B, Hkv, T, D), 43, torch.bfloat16).to(DEV)
    direct = ops.universal_sparse_attn(q, k, v, pairs, offsets, bs)
    launch = ops.prepare_prefill(q, k, v, pairs, offsets, bs)
    for _ in range(3):
        assert torch.equal(launch(), direct)


@pytest.mark.parametrize("name", ["bb_t1000_k256", "bb_t1500_k1024", "kr_groups_t1024", "bb2_t512_k128",
                                  "bb_t512_k128"])
def test_reference_block16_32_schedules_through_backend(name):
    """CSRs written by the reference's BigBird / keep-ratio patterns at block 16 or 32."""
    case, d = golden_case(name)
    _say(f"[prefill-b{case['block_size']}] reference {name}")
    H, T, bs = case["n_heads"], case["T_q"], case["block_size"]
    pairs, offsets = torch.from_numpy(d["block_pairs"]), torch.from_numpy(d["block_pair_offsets"])
    meta = PatternMetadata(kind="mask", block_size=bs, block_pairs=pairs.to(DEV), block_pair_offsets=offsets.to(DEV))
    q = seeded((1, H, T, 128), 51, torch.bfloat16).to(DEV)
    k = seeded((1, H, T, 128), 52, torch.bfloat16).to(DEV)
    v = seeded((1, H, T, 128), 53, torch.bfloat16).to(DEV)
    be = get_backend("hip_block_sparse")
    out = be.forward(q, k, v, meta)
    again = be.forward(q, k, v, meta)     # cached tile schedule
    assert be.actual_backend == "hip_block_sparse" and be.last_kernel == "prefill"
    assert torch.equal(out, again)
    want = oa.block_sparse_attention(q, k, v, pairs, offsets, bs)
    assert_close_bf16(out, want, name)
    if name == "bb_t1000_k256":
        # here the reference's token mask equals the CSR's coverage: dense masked semantics too
        dense = oa.masked_sdpa(q.float().cpu(), k.float().cpu(), v.float().cpu(), "mask", torch.from_numpy(d["mask"]))
        assert_close_bf16(out, dense, name + " dense")


def test_csr_to_tiles_reports_unsorted_lists():
    _say("[tiles] unsorted ids")
    pairs = torch.tensor([[0, 1, 2, 3, 7, 0]], dtype=torch.int32)     # query block 3: 3, 7, 0
    offsets = torch.tensor([[0, 1, 2, 3, 6]], dtype=torch.int32)
    ts = ops.csr_to_tiles(pairs.to(DEV), offsets.to(DEV), 16)
    with pytest.raises(AssertionError, match="not ascending"):
        ts.check()
