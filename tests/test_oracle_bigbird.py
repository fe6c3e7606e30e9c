"""Pins the oracle's BigBird semantics: published keep ratios, reference-written vectors, closed forms."""
import json
from pathlib import Path

import numpy as np
import pytest

from oracle import bigbird as ob
from oracle import csr as ocsr

GOLDEN = Path(__file__).resolve().parent / "golden"

# keep_ratio column of the reference's published benchmark CSVs, keyed by (seq_len, top_k):
# sparse_attention_bench/outputs/csv/bigbird_triton_vs_masked.csv and sweep.csv (prefill rows),
# sparse_attention_bench/outputs/csv/qwen_bigbird_keep_ratio.csv (prefill and decode rows).
PUBLISHED_PREFILL = {
    (64, 64): 1.0, (64, 128): 1.0, (128, 64): 0.7209302325581395, (128, 128): 1.0,
    (256, 64): 0.4163424124513619, (256, 128): 0.7451969844357976,
    (512, 64): 0.2222222222222222, (512, 128): 0.43420291179337234,
    (1024, 64): 0.11463414634146342, (1024, 128): 0.232578125,
    (2048, 64): 0.058199121522694, (2048, 128): 0.12015245622864812,
}
PUBLISHED_DECODE = {
    (64, 64): 1.0, (64, 128): 1.0, (128, 64): 0.5, (128, 128): 1.0,
    (256, 64): 0.25, (256, 128): 0.484375, (512, 64): 0.125, (512, 128): 0.248046875,
    (1024, 64): 0.0625, (1024, 128): 0.119140625, (2048, 64): 0.03125, (2048, 128): 0.06005859375,
}


@pytest.mark.parametrize("key", sorted(PUBLISHED_PREFILL))
def test_published_prefill_keep_ratio(key):
    assert ob.estimate_bigbird_attention_keep_ratio(*key) == pytest.approx(PUBLISHED_PREFILL[key], abs=1e-12)


@pytest.mark.parametrize("key", sorted(PUBLISHED_DECODE))
def test_published_decode_keep_ratio(key):
    assert ob.estimate_bigbird_decode_keep_ratio(*key) == pytest.approx(PUBLISHED_DECODE[key], abs=1e-12)


def test_planted_hash_mistake_breaks_published_ratio(monkeypatch):
    """Changing the query-block coefficient of the hash must move a published ratio."""
    orig = ob.select_bigbird_random_block_ids

    def wrong(qb, h, nb, g, s, r):
        return orig(qb + 1, h, nb, g, s, r) if qb > 1 else orig(qb, h, nb, g, s, r)

    monkeypatch.setattr(ob, "select_bigbird_random_block_ids", wrong)
    assert ob.estimate_bigbird_attention_keep_ratio(2048, 64) != pytest.approx(
        PUBLISHED_PREFILL[(2048, 64)], abs=1e-12)


def _golden():
    """The BigBird-family golden cases (the local-window ones are pinned with the pattern classes)."""
    idx = [c for c in json.loads((GOLDEN / "reference_patterns.json").read_text()) if c["kind"] != "local"]
    data = np.load(GOLDEN / "reference_patterns.npz")
    return idx, data


GOLDEN_INDEX, GOLDEN_DATA = _golden()


def _oracle_schedule(case):
    kind, T_q, T_k, H, p = case["kind"], case["T_q"], case["T_k"], case["n_heads"], case["params"]
    if kind == "bigbird":
        pairs, offsets, kv, bs = ob.bigbird_topk_schedule(T_q, T_k, p["top_k"], H)
        return pairs, offsets, kv, bs, None
    if kind == "bigbird2":
        pairs, offsets, kv, bs = ob.bigbird2_schedule(T_q, T_k, p["top_k"], H)
        return pairs, offsets, kv, bs, None
    krs = ob.keep_ratio_group_keep_ratios(p.get("keep_ratio"), p.get("group_sparsities"))
    pairs, offsets, kv, bs, layouts = ob.bigbird_keep_ratio_schedule(T_q, T_k, H, krs)
    return pairs, offsets, kv, bs, layouts


def _oracle_mask(case):
    kind, T_q, T_k, H, p = case["kind"], case["T_q"], case["T_k"], case["n_heads"], case["params"]
    if kind == "bigbird":
        return ob.bigbird_topk_token_mask(T_q, T_k, p["top_k"], H)
    if kind == "bigbird2":
        return ob.bigbird2_token_mask(T_q, T_k, p["top_k"], H)
    krs = ob.keep_ratio_group_keep_ratios(p.get("keep_ratio"), p.get("group_sparsities"))
    return ob.bigbird_keep_ratio_token_mask(T_q, T_k, H, krs)


@pytest.mark.parametrize("case", GOLDEN_INDEX, ids=[c["name"] for c in GOLDEN_INDEX])
def test_reference_golden_schedule(case):
    name = case["name"]
    pairs, offsets, kv, bs, layouts = _oracle_schedule(case)
    assert bs == case["block_size"]
    np.testing.assert_array_equal(pairs, GOLDEN_DATA[f"{name}/block_pairs"])
    np.testing.assert_array_equal(offsets, GOLDEN_DATA[f"{name}/block_pair_offsets"])
    np.testing.assert_array_equal(kv, GOLDEN_DATA[f"{name}/kv_block_list"])
    kr = ob.causal_block_keep_ratio_from_offsets(offsets, case["T_q"], case["T_k"], bs)
    assert kr == case["keep_ratio"]
    if layouts is not None:
        assert [list(x) for x in layouts] == case["group_layouts"]
    # the padded list and the CSR describe the same schedule
    p2, o2 = ocsr.kv_block_list_to_pairs(kv)
    np.testing.assert_array_equal(o2, offsets)


@pytest.mark.parametrize("case", [c for c in GOLDEN_INDEX if c["has_mask"]],
                         ids=[c["name"] for c in GOLDEN_INDEX if c["has_mask"]])
def test_reference_golden_token_mask(case):
    want = np.unpackbits(GOLDEN_DATA[f"{case['name']}/mask_bits"], axis=-1,
                         count=case["T_k"]).astype(bool)
    got = _oracle_mask(case)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("T,top_k,H", [(256, 64, 3), (1000, 256, 2), (4096, 4096, 1)])
def test_bigbird_row_length_closed_form(T, top_k, H):
    """Row length = |{0..g-1} U window U rand|, with rand = min(r, #candidates) disjoint from both."""
    pairs, offsets, _, tbs = ob.bigbird_topk_schedule(T, T, top_k, H)
    _, g, s, r = ob.bigbird_layout_from_topk(T, top_k)
    nkb = -(-T // tbs)
    for h in range(H):
        for qb in range(offsets.shape[1] - 1):
            window = set(range(max(0, qb - s + 1), min(qb + 1, nkb)))
            n_cand = max(0, min(qb, max(g, qb - s + 1)) - g) if qb > 0 else 0
            expect = len(set(range(g)) | window) + (min(r, n_cand) if r > 0 else 0)
            assert offsets[h, qb + 1] - offsets[h, qb] == expect


def test_next_pow2_min16():
    assert [ob.next_pow2_min16(x) for x in (1, 8, 16, 17, 45, 64, 65)] == [16, 16, 16, 32, 64, 64, 128]


def test_local_window_schedule_matches_brute_force():
    T, H, W, bs = 100, 2, 20, 16
    mask = ob.local_window_token_mask(T, T, H, W)
    for i in range(T):
        for j in range(T):
            assert mask[0, i, j] == (i - W + 1 <= j <= i)
    pairs, offsets = ob.local_window_schedule(T, T, H, W, bs)
    rows, offs = ocsr.brute_force_block_pairs(mask.tolist(), bs)
    assert offsets[0].tolist() == offs[0]
    assert ob.local_window_keep_ratio(T, T, W) == pytest.approx(mask[0].sum() / (T * T))
