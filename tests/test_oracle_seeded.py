"""Pins the oracle of the GPU seeded generators: Philox4x64-10 against numpy's own implementation,
and the mask rules by brute force and by their statistics."""
import numpy as np
import pytest

from oracle import seeded as osd


@pytest.mark.parametrize("key", [(1, 2), (0, 0), (2 ** 64 - 1, 12345), (0xDEADBEEF, 1)])
@pytest.mark.parametrize("counter", [(1, 0, 0, 0), (7, 3, 9, 0), (2 ** 40, 2 ** 33, 17, 5), (123456, 0, 8, 2 ** 63)])
def test_philox_matches_numpy_philox(key, counter):
    """numpy's Philox bit generator increments its counter, then emits the four words of the
    block: started at counter - 1 its first four raw outputs are philox(counter)."""
    bg = np.random.Philox(key=np.array(key, dtype=np.uint64),
                          counter=np.array([counter[0] - 1, *counter[1:]], dtype=np.uint64))
    want = bg.random_raw(4)
    got = [int(x) for x in osd.philox4x64([np.uint64(c) for c in counter], key)]
    assert got == [int(x) for x in want]


def test_planted_round_mistake_is_caught():
    good = osd.philox4x64([np.uint64(5), np.uint64(0), np.uint64(0), np.uint64(0)], (3, 4))[0]
    bg = np.random.Philox(key=np.array([3, 4], dtype=np.uint64), counter=np.array([4, 0, 0, 0], dtype=np.uint64))
    assert int(good) == int(bg.random_raw(1)[0])
    wrong = osd.philox4x64([np.uint64(5), np.uint64(0), np.uint64(0), np.uint64(0)], (4, 3))[0]
    assert int(wrong) != int(good)


def test_bernoulli_rules_and_density():
    rows, nqb, nkb, p = 3, 200, 200, 0.1
    m = osd.bernoulli_block_mask(rows, nqb, nkb, density=p, seed=17)
    kb, qb = np.arange(nkb)[None, :], np.arange(nqb)[:, None]
    assert m[:, kb == qb].all() and not m[:, (kb > qb)].any()                 # diagonal kept, nothing above
    strict = m[:, kb < qb]
    n = strict.size
    assert abs(strict.mean() - p) < 5 * np.sqrt(p * (1 - p) / n)              # binomial 5-sigma band
    assert np.array_equal(m, osd.bernoulli_block_mask(rows, nqb, nkb, density=p, seed=17))
    assert not np.array_equal(m, osd.bernoulli_block_mask(rows, nqb, nkb, density=p, seed=18))
    assert not osd.bernoulli_block_mask(1, 50, 50, density=0.0, seed=1)[:, kb[:, :50] < qb[:50]].any()
    assert osd.bernoulli_block_mask(1, 50, 50, density=1.0, seed=1)[:, kb[:, :50] <= qb[:50]].all()
    # a draw depends on (row, qa, kb) only: a chunk after a cached prefix sees the same blocks
    chunk = osd.bernoulli_block_mask(rows, 40, nkb, density=p, seed=17, q_block_offset=160)
    assert np.array_equal(chunk, m[:, 160:200])


@pytest.mark.parametrize("align", ["trailing", "centred"])
def test_seeded_bigbird_picks_are_the_smallest_eligible_draws(align):
    rows, nqb, nkb, w, g = 4, 60, 60, 3, 2
    counts = [0, 1, 3, 8]
    m = osd.seeded_bigbird_block_mask(rows, nqb, nkb, window=w, global_blocks=g, random_blocks=counts, seed=9,
                                      window_align=align)
    draws = osd.block_draws(9, osd.STREAM_BIGBIRD, rows, np.arange(nqb), nkb)
    for r in range(rows):
        for qa in range(nqb):
            lo, hi = (qa - w + 1, qa) if align == "trailing" else (qa - w // 2, qa + w // 2)
            base = {kb for kb in range(qa + 1) if kb < g or lo <= kb <= hi or kb == qa}
            eligible = [kb for kb in range(qa) if kb not in base]
            picks = {kb for _, kb in sorted((int(draws[r, qa, kb]), kb) for kb in eligible)[:counts[r]]}
            assert set(np.nonzero(m[r, qa])[0].tolist()) == base | picks, (r, qa)


def test_seeded_bigbird_picks_are_uniform():
    """Each of n eligible blocks is picked with probability r / n: a chi-square test over many rows."""
    rows, nqb, nkb, r = 64, 40, 40, 3
    qa = 30                               # eligible blocks: 2 .. 27 (global 0-1, window 28-30): n = 26
    m = osd.seeded_bigbird_block_mask(rows, nqb, nkb, window=3, global_blocks=2, random_blocks=r, seed=5)
    hits = m[:, qa, 2:28].sum(axis=0).astype(float)
    assert hits.sum() == rows * r
    expect = rows * r / 26
    chi2 = ((hits - expect) ** 2 / expect).sum()
    assert chi2 < 60                      # 25 degrees of freedom: p(chi2 > 60) < 1e-4
