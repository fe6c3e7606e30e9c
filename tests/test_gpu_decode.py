"""GPU parity of the HIP decode kernel (paged and contiguous) against the oracle."""
import math
import sys

import numpy as np
import pytest
import torch

from oracle import attention as oa
from sparseattentioninfer_amd import ops
from sparseattentioninfer_amd.attention import get_backend
from sparseattentioninfer_amd.patterns import PatternMetadata, decode_selection
from tests.helpers import assert_close_bf16, golden_case, seeded

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _paged_case(B, Hq, Hkv, D, page, lens, rows, seed, dtype=torch.bfloat16, extra_pages=3):
    nblk = [-(-L // page) for L in lens]
    max_blocks = max(nblk)
    P = sum(nblk) + extra_pages
    kp = seeded((P, Hkv, page, D), seed, dtype)
    vp = seeded((P, Hkv, page, D), seed + 1, dtype)
    q = seeded((B, Hq, D), seed + 2, dtype)
    perm = torch.randperm(P, generator=torch.Generator().manual_seed(seed))
    table = torch.zeros(B, max_blocks, dtype=torch.int32)
    used = 0
    for b, n in enumerate(nblk):
        table[b, :n] = perm[used:used + n].to(torch.int32)
        used += n
    R = Hq if rows == "q" else Hkv
    sel, sel_off = decode_selection(B, R, nblk, local=4, global_blocks=2, random_blocks=8, seed=seed)
    return q, kp, vp, table, torch.tensor(lens, dtype=torch.int32), sel, sel_off


DCASES = [
    # name, B, Hq, Hkv, D, page, lens, rows, splits, dtype
    ("group_ragged", 5, 8, 2, 128, 64, [1, 64, 65, 1000, 4097], "kv", 1, torch.bfloat16),
    ("per_head", 3, 8, 2, 128, 64, [700, 64, 2000], "q", 1, torch.bfloat16),
    ("splits3", 4, 32, 8, 128, 64, [5000, 16384, 33, 900], "kv", 3, torch.bfloat16),
    ("page16_d64", 3, 4, 4, 64, 16, [17, 300, 1000], "kv", 1, torch.bfloat16),
    ("page128", 2, 8, 2, 128, 128, [1000, 129], "kv", 2, torch.bfloat16),
    ("fp16", 2, 8, 2, 128, 64, [999, 3000], "kv", 1, torch.float16),
    # the combine reads 16 splits per memory round trip: exactly one chunk, then a second chunk with
    # more splits than retained blocks (empty splits carry m = -inf, l = 0)
    ("splits16", 2, 8, 2, 128, 64, [9000, 2100], "kv", 16, torch.bfloat16),
    ("splits21_empty", 3, 8, 2, 128, 64, [5000, 700, 64], "kv", 21, torch.bfloat16),
    # at least two units (sequence, row, split) per CU run two per workgroup: an odd count leaves
    # the last workgroup's second half without a unit (513 and 3 * 171 units on 256 CUs)
    ("paired_odd", 513, 4, 1, 128, 64, [(64, 200, 1000, 65, 1)[i % 5] for i in range(513)], "kv", 1,
     torch.bfloat16),
    ("paired_odd_splits", 171, 4, 1, 128, 64, [(3000, 64, 700)[i % 3] for i in range(171)], "kv", 3,
     torch.bfloat16),
]


@pytest.mark.parametrize("case", DCASES, ids=[c[0] for c in DCASES])
def test_paged_decode_matches_oracle(case):
    name, B, Hq, Hkv, D, page, lens, rows, splits, dtype = case
    _say(f"[decode] {name}")
    q, kp, vp, table, kv_lens, sel, sel_off = _paged_case(B, Hq, Hkv, D, page, lens, rows, seed=3, dtype=dtype)
    out = ops.paged_sparse_decode(q.to(DEV), kp.to(DEV), vp.to(DEV), table.to(DEV), kv_lens.to(DEV),
                                  sel.to(DEV), sel_off.to(DEV), num_splits=splits)
    torch.cuda.synchronize()
    want = oa.paged_decode_attention(q, kp, vp, table.numpy(), kv_lens.numpy(), sel.numpy(), sel_off.numpy())
    assert torch.isfinite(out.float()).all()
    assert_close_bf16(out, want, name)


def test_reference_bigbird_decode_through_backend():
    """Reference-written decode CSR (keep-ratio groups, block 32, one row per head) on a
    contiguous cache, against the reference's dense masked semantics on its own token mask.
    (Block 32 is a layout where the reference's token mask and CSR describe the same pattern.)"""
    case, d = golden_case("kr_groups_dec_t3000")
    _say("[decode] reference kr_groups_dec_t3000")
    H, T_k = case["n_heads"], case["T_k"]
    q = seeded((2, H, 1, 128), 31, torch.bfloat16)
    k = seeded((2, H, T_k, 128), 32, torch.bfloat16)
    v = seeded((2, H, T_k, 128), 33, torch.bfloat16)
    meta = PatternMetadata(kind="mask", block_size=case["block_size"],
                           block_pairs=torch.from_numpy(d["block_pairs"]).to(DEV),
                           block_pair_offsets=torch.from_numpy(d["block_pair_offsets"]).to(DEV))
    be = get_backend("hip_block_sparse")
    out = be.forward(q.to(DEV), k.to(DEV), v.to(DEV), meta)
    assert be.last_kernel == "decode"
    want = oa.masked_sdpa(q.float(), k.float(), v.float(), "mask", torch.from_numpy(d["mask"]))
    assert_close_bf16(out, want, "kr_groups_dec_t3000")


@pytest.mark.parametrize("random_blocks", [8, 16], ids=["14_blocks", "22_blocks"])
def test_configs_3_full_size_every_sequence(random_blocks):
    """B=64, 32Q/8KV, D=128, 16384 tokens in 64-token pages, shuffled page table; every
    sequence and head checked. 2 global + 4 local + 8 random = 14 retained blocks per (sequence, KV
    group) is the configuration's block count (5.5 % of 256); 16 random blocks give 22 (8.6 %), the
    retention its description quotes."""
    _say(f"[decode] configs[3] full size, {random_blocks} random blocks")
    B, Hq, Hkv, D, page, L = 64, 32, 8, 128, 64, 16384
    nblk = L // page
    P = B * nblk
    gen = torch.Generator(device=DEV).manual_seed(77)
    kp = torch.randn(P, Hkv, page, D, generator=gen, device=DEV).to(torch.bfloat16)
    vp = torch.randn(P, Hkv, page, D, generator=gen, device=DEV).to(torch.bfloat16)
    q = seeded((B, Hq, D), 78, torch.bfloat16)
    table = torch.randperm(P, generator=torch.Generator().manual_seed(79)).to(torch.int32).reshape(B, nblk)
    kv_lens = torch.full((B,), L, dtype=torch.int32)
    sel, sel_off = decode_selection(B, Hkv, nblk, local=4, global_blocks=2, random_blocks=random_blocks, seed=80)
    assert (sel_off[:, :, 1] == 6 + random_blocks).all()
    for splits in (1, 2):
        out = ops.paged_sparse_decode(q.to(DEV), kp, vp, table.to(DEV), kv_lens.to(DEV), sel.to(DEV),
                                      sel_off.to(DEV), num_splits=splits)
        torch.cuda.synchronize()
        want = oa.paged_decode_attention(q, kp, vp, table.numpy(), kv_lens.numpy(), sel.numpy(), sel_off.numpy(),
                                         device=DEV)
        max_abs, mean_abs = assert_close_bf16(out, want, f"configs[3] {6 + random_blocks} blocks splits={splits}")
        _say(f"[decode] configs[3] {6 + random_blocks} blocks splits={splits}: all 64 sequences, "
             f"max-abs {max_abs:.3e}, mean-abs {mean_abs:.3e}")


def _with_skipped_entries(valid: list[int], junk: list[int], seed: int) -> list[int]:
    """``valid`` with each entry of ``junk`` inserted at a seeded position."""
    g = torch.Generator().manual_seed(seed)
    out = list(valid)
    for x in junk:
        out.insert(int(torch.randint(0, len(out) + 1, (1,), generator=g)), x)
    return out


@pytest.mark.parametrize("splits", [1, 2, 3])
def test_paged_lists_longer_than_the_lds_stage(splits):
    """Rows of 1,000+ retained blocks (page 16, 16384 keys): longer than the 512 entries a
    workgroup stages in LDS, so num_splits 1 and 2 read the list and the block table where they
    are used and 3 stages them.  Mixed in are entries the kernel skips: -1 and -7, ids past kv_len,
    past the table's columns, 2^30, and block 7, whose page lies outside the pool.  The third
    sequence is empty (kv_len 0, output 0).  Expected: the oracle over the valid entries only."""
    _say(f"[decode] long lists, splits={splits}")
    B, Hq, Hkv, D, page = 3, 8, 2, 128, 16
    lens = [16384, 9000, 0]
    nblk = [-(-L // page) for L in lens]
    max_blocks = max(nblk)
    P = sum(nblk) + 2
    kp = seeded((P, Hkv, page, D), 41, torch.bfloat16)
    vp = seeded((P, Hkv, page, D), 42, torch.bfloat16)
    q = seeded((B, Hq, D), 43, torch.bfloat16)
    perm = torch.randperm(P, generator=torch.Generator().manual_seed(44)).to(torch.int32)
    table = torch.zeros(B, max_blocks, dtype=torch.int32)
    used = 0
    for b, n in enumerate(nblk):
        table[b, :n] = perm[used:used + n]
        used += n
    table[0, 7] = P + 100
    table[1, 7] = -5
    lists, clean = [], []
    for b in range(B):
        for r in range(Hkv):
            valid = list(range(nblk[b]))
            junk = [-1, nblk[b], nblk[b] + 3, max_blocks + 9, 1 << 30, -7]
            lists.append(_with_skipped_entries(valid, junk, seed=100 * b + r))
            clean.append([x for x in valid if x != 7])
    assert max(len(x) for x in lists) // splits > 512 or splits == 3

    def pack(rows):
        width = max(1, max(len(x) for x in rows))
        sel = torch.zeros(B, Hkv, width, dtype=torch.int32)
        off = torch.zeros(B, Hkv, 2, dtype=torch.int32)
        for i, x in enumerate(rows):
            sel[i // Hkv, i % Hkv, :len(x)] = torch.tensor(x, dtype=torch.int32)
            off[i // Hkv, i % Hkv, 1] = len(x)
        return sel, off

    sel, sel_off = pack(lists)
    csel, csel_off = pack(clean)
    kv_lens = torch.tensor(lens, dtype=torch.int32)
    out = ops.paged_sparse_decode(q.to(DEV), kp.to(DEV), vp.to(DEV), table.to(DEV), kv_lens.to(DEV),
                                  sel.to(DEV), sel_off.to(DEV), num_splits=splits)
    torch.cuda.synchronize()
    want = oa.paged_decode_attention(q, kp.to(DEV), vp.to(DEV), table.numpy(), kv_lens.numpy(),
                                     csel.numpy(), csel_off.numpy(), device=DEV)
    assert torch.isfinite(out.float()).all()
    assert (out[2].float() == 0).all()
    max_abs, _ = assert_close_bf16(out, want, f"long lists splits={splits}")
    _say(f"[decode] long lists, splits={splits}: max-abs {max_abs:.3e}")


def test_contiguous_lists_longer_than_the_lds_stage():
    """A contiguous cache (the backend's T_q == 1 path) with every one of 1,024 blocks of 16 keys
    retained, in a list longer than the LDS stage, plus entries it skips: -1, -2, the block at T_k,
    2^30 and 2^31 - 1 (whose key offset does not fit 32 bits).  Expected: attention over all keys,
    which is what a full decode row is (fp32 torch reference)."""
    _say("[decode] contiguous long list")
    B, Hq, Hkv, D, bs, T = 2, 8, 2, 128, 16, 16384
    q = seeded((B, Hq, 1, D), 51, torch.bfloat16).to(DEV)
    k = seeded((B, Hkv, T, D), 52, torch.bfloat16).to(DEV)
    v = seeded((B, Hkv, T, D), 53, torch.bfloat16).to(DEV)
    lst = _with_skipped_entries(list(range(T // bs)), [-1, T // bs, 1 << 30, (1 << 31) - 1, -2], seed=54)
    pairs = torch.tensor([lst] * Hkv, dtype=torch.int32, device=DEV)
    offsets = torch.tensor([[0, len(lst)]] * Hkv, dtype=torch.int32, device=DEV)
    out = ops.universal_sparse_attn(q, k, v, pairs, offsets, bs)
    torch.cuda.synchronize()
    kf = k.float().repeat_interleave(Hq // Hkv, dim=1)
    vf = v.float().repeat_interleave(Hq // Hkv, dim=1)
    s = (q.float() @ kf.transpose(-1, -2).contiguous()) / math.sqrt(D)
    want = torch.softmax(s, dim=-1) @ vf
    assert torch.isfinite(out.float()).all()
    max_abs, _ = assert_close_bf16(out, want, "contiguous long list")
    _say(f"[decode] contiguous long list: max-abs {max_abs:.3e}")
