"""Pins the oracle's CSR construction against brute force and its invariants (CPU)."""
import numpy as np
import pytest
from hypothesis import given, settings, strategies as st

from oracle import csr as ocsr


def _rows_from_csr(pairs, offsets):
    return [[list(map(int, pairs[h, offsets[h, i]:offsets[h, i + 1]]))
             for i in range(offsets.shape[1] - 1)] for h in range(offsets.shape[0])]


def _rows_from_brute(rows, offs):
    return [[rows[h][offs[h][i]:offs[h][i + 1]] for i in range(len(offs[h]) - 1)]
            for h in range(len(rows))]


@pytest.mark.parametrize("H,T_q,T_k,bs,p", [
    (2, 32, 32, 16, 0.05), (3, 40, 40, 16, 0.02), (1, 1, 50, 16, 0.2),
    (2, 17, 33, 8, 0.1), (4, 64, 64, 32, 0.001), (2, 7, 7, 16, 0.0), (1, 96, 96, 32, 1.0),
])
def test_build_block_pairs_matches_brute_force(H, T_q, T_k, bs, p):
    rng = np.random.default_rng(H * 1000 + T_q + T_k + bs)
    mask = rng.random((H, T_q, T_k)) < p
    pairs, offsets = ocsr.build_block_pairs_from_mask(mask, bs)
    b_rows, b_offs = ocsr.brute_force_block_pairs(mask.tolist(), bs)
    assert _rows_from_csr(pairs, offsets) == _rows_from_brute(b_rows, b_offs)
    # packing invariants of base.py:81-89
    nnz = offsets[:, -1]
    assert pairs.dtype == np.int32 and offsets.dtype == np.int32
    assert pairs.shape == (H, max(1, int(nnz.max(initial=0))))
    assert offsets.shape == (H, -(-T_q // bs) + 1)
    assert (offsets[:, 0] == 0).all() and (np.diff(offsets, axis=1) >= 0).all()
    for h in range(H):
        assert (pairs[h, nnz[h]:] == 0).all()
        for row in _rows_from_csr(pairs, offsets)[h]:
            assert row == sorted(set(row))


@settings(max_examples=60, deadline=None)
@given(st.integers(1, 3), st.integers(1, 40), st.integers(1, 40), st.sampled_from([4, 8, 16]),
       st.integers(0, 2**31 - 1))
def test_build_block_pairs_property(H, T_q, T_k, bs, seed):
    rng = np.random.default_rng(seed)
    mask = rng.random((H, T_q, T_k)) < rng.random()
    pairs, offsets = ocsr.build_block_pairs_from_mask(mask, bs)
    b_rows, b_offs = ocsr.brute_force_block_pairs(mask.tolist(), bs)
    assert _rows_from_csr(pairs, offsets) == _rows_from_brute(b_rows, b_offs)
    back = ocsr.csr_to_block_mask(pairs, offsets, -(-T_k // bs))
    assert (back == ocsr.coarsen_token_mask(mask, bs)).all()


def test_kv_block_list_to_pairs_drops_padding_in_place():
    kv = np.array([[[0, 2, -1, -1], [1, -1, 3, -1], [-1, -1, -1, -1]],
                   [[5, 4, -1, -1], [0, 1, 2, 3], [7, -1, -1, -1]]], dtype=np.int32)
    pairs, offsets = ocsr.kv_block_list_to_pairs(kv)
    assert offsets.tolist() == [[0, 2, 4, 4], [0, 2, 6, 7]]
    assert pairs.tolist() == [[0, 2, 1, 3, 0, 0, 0], [5, 4, 0, 1, 2, 3, 7]]


def test_empty_mask_gives_single_zero_column():
    pairs, offsets = ocsr.build_block_pairs_from_mask(np.zeros((2, 20, 20), bool), 16)
    assert pairs.shape == (2, 1) and (pairs == 0).all()
    assert (offsets == 0).all() and offsets.shape == (2, 3)


def test_planted_mistake_is_caught():
    """A coarsening that forgets the tail of a ragged block must disagree with brute force."""
    rng = np.random.default_rng(7)
    mask = np.zeros((1, 20, 20), bool)
    mask[0, 18, 19] = True  # only in the ragged tail tile
    truncated = ocsr.build_block_pairs_from_mask(mask[:, :16, :16], 16)
    b_rows, b_offs = ocsr.brute_force_block_pairs(mask.tolist(), 16)
    assert _rows_from_brute(b_rows, b_offs) == [[[], [1]]]
    assert _rows_from_csr(*truncated) != _rows_from_brute(b_rows, b_offs)
    del rng
