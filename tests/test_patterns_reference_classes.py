"""Drop-in pattern classes against the reference's own outputs and the oracle.

The golden cases were written by the reference's pattern classes themselves
(``tests/golden/make_reference_vectors.py``); every tensor must match bit for
bit.  Shapes the fixtures do not cover are checked against the oracle's
restatement, and the local window against its token-mask definition.
"""
import json

import numpy as np
import pytest
import torch

from oracle import bigbird as ob
from oracle import csr as oc
from sparseattentioninfer_amd.patterns import (BigBird2Pattern, BigBirdKeepRatioPattern, BigBirdPattern,
                                               LocalWindowPattern, build_block_pairs_from_mask,
                                               local_window_block_mask)
from tests.helpers import GOLDEN, golden_case

CASES = [c["name"] for c in json.loads((GOLDEN / "reference_patterns.json").read_text())]


def _qk(T_q, T_k, H):
    return torch.zeros(1, H, T_q, 8), torch.zeros(1, H, T_k, 8)


def _pattern(case):
    p = case["params"]
    if case["kind"] == "bigbird":
        return BigBirdPattern(top_k=p["top_k"], n_heads=case["n_heads"])
    if case["kind"] == "bigbird2":
        return BigBird2Pattern(top_k=p["top_k"], n_heads=case["n_heads"])
    if case["kind"] == "local":
        return LocalWindowPattern(window_size=p["window_size"], block_size=p["block_size"])
    if "group_sparsities" in p:
        return BigBirdKeepRatioPattern(group_sparsities=p["group_sparsities"], n_heads=case["n_heads"],
                                       n_kv_heads=p.get("n_kv_heads"))
    return BigBirdKeepRatioPattern(keep_ratio=p["keep_ratio"], n_heads=case["n_heads"])


@pytest.mark.parametrize("name", CASES)
def test_pattern_classes_match_reference_outputs(name):
    case, d = golden_case(name)
    pat = _pattern(case)
    meta = pat.build(*_qk(case["T_q"], case["T_k"], case["n_heads"]))
    assert meta.kind == ("local" if case["kind"] == "local" else "mask")
    assert meta.block_size == case["block_size"]
    assert np.array_equal(meta.block_pairs.numpy(), d["block_pairs"])
    assert np.array_equal(meta.block_pair_offsets.numpy(), d["block_pair_offsets"])
    assert meta.block_pairs.dtype == torch.int32
    if "kv_block_list" in d:
        assert np.array_equal(meta.kv_block_list.numpy(), d["kv_block_list"])
        assert meta.kv_block_list.dtype == torch.int32
    else:
        assert meta.kv_block_list is None
    assert meta.keep_ratio == pytest.approx(case["keep_ratio"], abs=0, rel=1e-15)
    if "mask" in d:
        assert np.array_equal(meta.mask.numpy(), d["mask"])
    if "group_layouts" in case:
        assert [list(x) for x in pat.last_group_layouts] == case["group_layouts"]


@pytest.mark.parametrize("T_q,T_k,top_k,H", [(96, 96, 40, 3), (1, 1500, 300, 4), (700, 700, 900, 2),
                                             (17, 333, 50, 2), (1024, 1024, 16, 5)])
def test_bigbird_classes_match_oracle_on_other_shapes(T_q, T_k, top_k, H):
    for cls, sched, tmask in ((BigBirdPattern, ob.bigbird_topk_schedule, ob.bigbird_topk_token_mask),
                              (BigBird2Pattern, ob.bigbird2_schedule, ob.bigbird2_token_mask)):
        meta = cls(top_k=top_k, n_heads=H).build(*_qk(T_q, T_k, H))
        pairs, offsets, kv, tbs = sched(T_q, T_k, top_k, H)
        assert meta.block_size == tbs
        assert np.array_equal(meta.block_pairs.numpy(), pairs)
        assert np.array_equal(meta.block_pair_offsets.numpy(), offsets)
        assert np.array_equal(meta.kv_block_list.numpy(), kv)
        assert np.array_equal(meta.mask.numpy(), tmask(T_q, T_k, top_k, H))


@pytest.mark.parametrize("T_q,T_k,H,ratios", [(640, 640, 8, (0.25,)), (1, 4000, 4, (0.1,)),
                                              (900, 900, 6, (0.6, 0.2, 0.05)), (1, 2500, 8, (0.5, 0.3))])
def test_keep_ratio_class_matches_oracle(T_q, T_k, H, ratios):
    kw = {"keep_ratio": ratios[0]} if len(ratios) == 1 else {"group_sparsities": [1 - x for x in ratios]}
    meta = BigBirdKeepRatioPattern(n_heads=H, **kw).build(*_qk(T_q, T_k, H))
    grk = ob.keep_ratio_group_keep_ratios(**({"keep_ratio": ratios[0]} if len(ratios) == 1
                                             else {"group_sparsities": [1 - x for x in ratios]}))
    pairs, offsets, kv, tbs, _ = ob.bigbird_keep_ratio_schedule(T_q, T_k, H, grk)
    assert meta.block_size == tbs
    assert np.array_equal(meta.block_pairs.numpy(), pairs)
    assert np.array_equal(meta.block_pair_offsets.numpy(), offsets)
    assert np.array_equal(meta.kv_block_list.numpy(), kv)
    assert np.array_equal(meta.mask.numpy(), ob.bigbird_keep_ratio_token_mask(T_q, T_k, H, grk))


def test_keep_ratio_argument_errors():
    with pytest.raises(ValueError):
        BigBirdKeepRatioPattern(n_heads=4)
    with pytest.raises(ValueError):
        BigBirdKeepRatioPattern(keep_ratio=0.2, group_sparsities=[0.5], n_heads=4)
    with pytest.raises(ValueError):
        BigBirdKeepRatioPattern(group_sparsities=[0.5, 0.5, 0.5], n_heads=4)
    with pytest.raises(ValueError):
        BigBirdKeepRatioPattern(group_sparsities=[0.5, 1.0], n_heads=4)
    with pytest.raises(ValueError):
        BigBirdKeepRatioPattern(group_sparsities=[0.5, 0.2], n_heads=4, n_kv_heads=4)


@pytest.mark.parametrize("T_q,T_k,W,bs", [(256, 256, 40, 16), (300, 300, 64, 64), (1, 999, 100, 32),
                                          (77, 500, 1, 16), (512, 512, 700, 128), (33, 33, 5, 16)])
def test_local_window_schedule_equals_coarsened_token_mask(T_q, T_k, W, bs):
    H = 3
    meta = LocalWindowPattern(W, block_size=bs).build(*_qk(T_q, T_k, H))
    tm = ob.local_window_token_mask(T_q, T_k, H, W)
    assert np.array_equal(meta.mask.numpy(), tm)
    pairs, offsets = oc.build_block_pairs_from_mask(tm, bs)
    assert np.array_equal(meta.block_pairs.numpy(), pairs)
    assert np.array_equal(meta.block_pair_offsets.numpy(), offsets)
    assert meta.keep_ratio == pytest.approx(ob.local_window_keep_ratio(T_q, T_k, W), rel=1e-15)


def test_local_window_block_mask_is_interval_overlap():
    # every (qb, kb) with any kept token pair is active, and no other (brute force on tokens)
    T_q, T_k, W, bs = 70, 150, 23, 16
    tm = ob.local_window_token_mask(T_q, T_k, 1, W)[0]
    want = oc.coarsen_token_mask(tm[None], bs)[0]
    assert np.array_equal(local_window_block_mask(T_q, T_k, W, bs).numpy(), want)


def test_mask_is_lazy_and_cached():
    pat = BigBirdPattern(top_k=256, n_heads=2)
    m1 = pat.build(*_qk(512, 512, 2))
    assert m1._mask_value is None            # schedule built, mask not yet
    first = m1.mask
    m2 = pat.build(*_qk(512, 512, 2))
    assert m2.mask is first                   # built once per shape


@pytest.mark.parametrize("name", [c for c in CASES if c.startswith("lw_")])
def test_oracle_local_window_matches_reference_outputs(name):
    """The oracle's restatement against the reference's own LocalWindowPattern, including
    queries after a cached prefix (T_q < T_k: rows at max(0, T_k - T_q) + t)."""
    case, d = golden_case(name)
    T_q, T_k, H, p = case["T_q"], case["T_k"], case["n_heads"], case["params"]
    mask = ob.local_window_token_mask(T_q, T_k, H, p["window_size"])
    assert np.array_equal(mask, d["mask"])
    pairs, offsets = ob.local_window_schedule(T_q, T_k, H, p["window_size"], p["block_size"])
    assert np.array_equal(pairs, d["block_pairs"]) and np.array_equal(offsets, d["block_pair_offsets"])
    assert ob.local_window_keep_ratio(T_q, T_k, p["window_size"]) == pytest.approx(case["keep_ratio"], rel=1e-15)
