"""Pins the attention oracle: float64 textbook loops, special cases, block-gather vs dense."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as oa
from oracle import bigbird as ob
from oracle import csr as ocsr


def _rand(shape, seed, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=torch.float32).to(dtype)


@pytest.mark.parametrize("T,p", [(9, 0.3), (12, 0.6), (5, 0.0)])
def test_masked_sdpa_matches_textbook(T, p):
    H, D = 2, 6
    q, k, v = (_rand((1, H, T, D), s) for s in (1, 2, 3))
    rng = np.random.default_rng(T)
    mask = rng.random((H, T, T)) < p
    out = oa.masked_sdpa(q, k, v, "mask", torch.from_numpy(mask))
    causal = np.tril(np.ones((T, T), bool))
    for h in range(H):
        want = oa.textbook_attention(q[0, h].numpy(), k[0, h].numpy(), v[0, h].numpy(), mask[h] & causal)
        np.testing.assert_allclose(out[0, h].numpy(), want, atol=1e-12)


def test_all_ones_mask_is_causal_sdpa():
    q, k, v = (_rand((2, 3, 17, 8), s) for s in (4, 5, 6))
    out = oa.masked_sdpa(q, k, v, "mask", torch.ones(3, 17, 17, dtype=torch.bool))
    ref = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    torch.testing.assert_close(out, ref, atol=1e-12, rtol=0)


def test_single_kept_key_returns_that_value_row():
    T = 6
    q, k, v = (_rand((1, 1, T, 4), s) for s in (7, 8, 9))
    mask = torch.zeros(1, T, T, dtype=torch.bool)
    mask[0, :, 0] = True
    out = oa.masked_sdpa(q, k, v, "mask", mask)
    torch.testing.assert_close(out[0, 0], v[0, 0, 0].expand(T, 4), atol=1e-12, rtol=0)


def test_decode_row_sees_every_key():
    q = _rand((1, 2, 1, 8), 10)
    k, v = _rand((1, 2, 13, 8), 11), _rand((1, 2, 13, 8), 12)
    out = oa.masked_sdpa(q, k, v, "mask", torch.ones(2, 1, 13, dtype=torch.bool))
    w = torch.softmax((q @ k.transpose(-1, -2)) / math.sqrt(8), dim=-1)
    torch.testing.assert_close(out, w @ v, atol=1e-12, rtol=0)


def test_planted_scale_mistake_is_caught():
    q, k, v = (_rand((1, 1, 8, 4), s) for s in (13, 14, 15))
    keep = np.tril(np.ones((8, 8), bool))
    good = oa.textbook_attention(q[0, 0].numpy(), k[0, 0].numpy(), v[0, 0].numpy(), keep)
    wrong = oa.textbook_attention(q[0, 0].numpy() * 2.0, k[0, 0].numpy(), v[0, 0].numpy(), keep)
    assert np.abs(good - wrong).max() > 1e-3


@pytest.mark.parametrize("B,Hq,Hkv,T_q,T_k,bs,group_rows", [
    (1, 4, 4, 96, 96, 16, False),
    (2, 4, 2, 80, 80, 16, True),      # GQA, group-shared CSR, ragged tail
    (1, 4, 2, 70, 70, 32, False),     # GQA, per-head CSR
    (2, 4, 1, 1, 77, 16, False),      # decode row
])
def test_block_sparse_matches_masked_sdpa(B, Hq, Hkv, T_q, T_k, bs, group_rows):
    D = 8
    q = _rand((B, Hq, T_q, D), 21)
    k = _rand((B, Hkv, T_k, D), 22)
    v = _rand((B, Hkv, T_k, D), 23)
    R = Hkv if group_rows else Hq
    rng = np.random.default_rng(T_k)
    nqb, nkb = -(-T_q // bs), -(-T_k // bs)
    qbo = (T_k - T_q) // bs
    bm = rng.random((R, nqb, nkb)) < 0.4
    for i in range(nqb):            # keep the diagonal, as the benchmark generators do
        bm[:, i, min(nkb - 1, qbo + i)] = True
    pairs, offsets = ocsr.csr_from_block_mask(bm)
    keep = oa.csr_keep_mask(pairs, offsets, bs, T_q, T_k, T_k - T_q)      # [R, T_q, T_k]
    rowmap = np.arange(Hq) // (Hq // R) if R != Hq else np.arange(Hq)
    keep_q = torch.from_numpy(keep[rowmap])
    n_rep = Hq // Hkv
    dense = oa.masked_sdpa(q, oa.repeat_kv(k, n_rep), oa.repeat_kv(v, n_rep), "mask", keep_q)
    sparse = oa.block_sparse_attention(q, k, v, pairs, offsets, bs, compute_dtype=torch.float64)
    torch.testing.assert_close(sparse.double(), dense, atol=1e-6, rtol=0)


def test_block_sparse_on_reference_bigbird_matches_masked_sdpa():
    """At a power-of-two block >= 16 the BigBird token mask equals the coarsened CSR mask."""
    T, H, top_k = 256, 4, 256      # layout block 16 == kernel block 16
    mask = ob.bigbird_topk_token_mask(T, T, top_k, H)
    pairs, offsets, _, bs = ob.bigbird_topk_schedule(T, T, top_k, H)
    assert bs == 16
    keep = oa.csr_keep_mask(pairs, offsets, bs, T, T, 0)
    np.testing.assert_array_equal(keep, mask)
    q, k, v = (_rand((1, H, T, 8), s) for s in (31, 32, 33))
    dense = oa.masked_sdpa(q, k, v, "mask", torch.from_numpy(mask))
    sparse = oa.block_sparse_attention(q, k, v, pairs, offsets, bs, compute_dtype=torch.float64)
    torch.testing.assert_close(sparse.double(), dense, atol=1e-6, rtol=0)


def test_paged_decode_matches_block_sparse():
    B, Hq, Hkv, D, page = 2, 4, 2, 8, 16
    L = [50, 33]
    nblk = 4
    q = _rand((B, Hq, D), 41, torch.float32)
    P = B * nblk + 3
    kp = _rand((P, Hkv, page, D), 42, torch.float32)
    vp = _rand((P, Hkv, page, D), 43, torch.float32)
    rng = np.random.default_rng(0)
    table = rng.permutation(P)[:B * nblk].reshape(B, nblk).astype(np.int32)
    sel = np.zeros((B, Hkv, nblk), np.int32)
    soff = np.zeros((B, Hkv, 2), np.int32)
    for b in range(B):
        used = -(-L[b] // page)
        for r in range(Hkv):
            chosen = sorted(rng.choice(used, size=min(used, 2), replace=False).tolist())
            sel[b, r, :len(chosen)] = chosen
            soff[b, r] = (0, len(chosen))
    got = oa.paged_decode_attention(q, kp, vp, table, np.array(L), sel, soff)
    for b in range(B):
        k = torch.stack([torch.cat([kp[table[b, j], h] for j in range(nblk)])[:L[b]] for h in range(Hkv)])[None]
        v = torch.stack([torch.cat([vp[table[b, j], h] for j in range(nblk)])[:L[b]] for h in range(Hkv)])[None]
        pairs = np.zeros((Hkv, nblk), np.int32)
        offs = np.zeros((Hkv, 2), np.int32)
        for r in range(Hkv):
            n = soff[b, r, 1]
            pairs[r, :n] = sel[b, r, :n]
            offs[r, 1] = n
        want = oa.block_sparse_attention(q[b:b + 1, :, None], k, v, pairs, offs, page)
        torch.testing.assert_close(got[b], want[0, :, 0], atol=1e-5, rtol=0)


def test_masked_sdpa_rows_equals_full_masked_sdpa():
    """The row-chunk form used for the CPU baseline equals masked_sdpa on those rows."""
    T, H = 24, 2
    q, k, v = (_rand((1, H, T, 8), s) for s in (51, 52, 53))
    mask = torch.from_numpy(np.random.default_rng(3).random((H, T, T)) < 0.4)
    full = oa.masked_sdpa(q, k, v, "mask", mask)
    causal = torch.tril(torch.ones(T, T, dtype=torch.bool))
    for h in range(H):
        rows = oa.masked_sdpa_rows(q[0, h, 5:17], k[0, h], v[0, h], (mask[h] & causal)[5:17])
        torch.testing.assert_close(rows, full[0, h, 5:17], atol=1e-12, rtol=0)


@pytest.mark.parametrize("B,Hq,Hkv,T_q,T_k,bs,group_rows,chunk", [
    (2, 4, 2, 80, 80, 16, True, 24),     # GQA, group rows, ragged tail, chunks not block-aligned
    (1, 4, 4, 96, 96, 32, False, 1000),  # one chunk
    (1, 2, 1, 40, 100, 16, True, 16),    # chunked prefill: T_q < T_k, q_offset = 60
])
def test_masked_sdpa_blockwise_equals_masked_sdpa(B, Hq, Hkv, T_q, T_k, bs, group_rows, chunk):
    """The row-chunked block-mask form used for exhaustive checks at 32K tokens equals
    masked_sdpa on the expanded token mask (and so, transitively, the float64 textbook loop)."""
    D = 8
    q, k, v = _rand((B, Hq, T_q, D), 61), _rand((B, Hkv, T_k, D), 62), _rand((B, Hkv, T_k, D), 63)
    R = Hkv if group_rows else Hq
    nqb, nkb = -(-T_q // bs), -(-T_k // bs)
    bm = torch.from_numpy(np.random.default_rng(T_q).random((R, nqb, nkb)) < 0.45)
    got = oa.masked_sdpa_blockwise(q, k, v, bm, bs, row_chunk=chunk)
    rowmap = np.arange(Hq) // (Hq // R)
    tok = bm.repeat_interleave(bs, 1).repeat_interleave(bs, 2)[:, :T_q, :T_k][rowmap]
    off = T_k - T_q
    causal = torch.arange(T_k)[None, :] <= (off + torch.arange(T_q))[:, None]
    n_rep = Hq // Hkv
    if T_q == T_k:
        want = oa.masked_sdpa(q, oa.repeat_kv(k, n_rep), oa.repeat_kv(v, n_rep), "mask", tok)
    else:   # masked_sdpa cannot broadcast its causal mask for 1 < T_q < T_k: textbook loop per head
        want = torch.stack([torch.from_numpy(oa.textbook_attention(
            q[b, h], k[b, h // n_rep], v[b, h // n_rep], (tok[h] & causal).numpy())).float()
            for b in range(B) for h in range(Hq)]).reshape(B, Hq, T_q, D)
    torch.testing.assert_close(got, want.float(), atol=2e-6, rtol=0)
    # and it matches the block-gather oracle over the same schedule
    pairs, offsets = ocsr.csr_from_block_mask(bm.numpy())
    gather = oa.block_sparse_attention(q, k, v, pairs, offsets, bs)
    torch.testing.assert_close(got, gather, atol=2e-6, rtol=0)
