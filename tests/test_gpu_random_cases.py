"""Seeded random cases of both kernels against the oracle: shapes, head ratios, CSR row layouts,
block sizes, chunked query offsets, ragged cache lengths, page sizes, split counts and dtypes drawn
per case.  Each prefill case also runs on a copy of its CSR with entries the kernel skips (negative
ids anywhere, ids past T_k at the end of a query block's list) and must give the same bits; each
decode case mixes such entries into its lists and is checked against the oracle over the valid
entries only.  The backend cases build the reference-compatible pattern classes at random shapes
and run them through ``HipBlockSparseBackend.forward``."""
import sys

import numpy as np
import pytest
import torch

from oracle import attention as oa
from sparseattentioninfer_amd import ops
from tests.helpers import assert_close_bf16, seeded

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def prefill_case(seed: int) -> dict:
    """Shapes and a causal block schedule (clean and with skipped entries) for one prefill case."""
    rng = np.random.default_rng(1000 + seed)
    bs = int(rng.choice([16, 32, 64, 128]))
    D = int(rng.choice([64, 128]))
    Hkv = int(rng.integers(1, 4))
    Hq = Hkv * int(rng.choice([1, 2, 4, 8]))
    B = int(rng.integers(1, 3))
    T_k = int(rng.integers(2, 2049))
    T_q = T_k if rng.random() < 0.5 else int(rng.integers(2, T_k + 1))
    R = Hq if rng.random() < 0.3 else Hkv
    dtype = torch.bfloat16 if rng.random() < 0.7 else torch.float16
    nqb, nkb = -(-T_q // bs), -(-T_k // bs)
    q_off = T_k - T_q
    density = float(rng.choice([0.05, 0.2, 0.5, 1.0]))
    clean, junk = [], []
    for _ in range(R):
        rc, rj = [], []
        for qb in range(nqb):
            last = min(nkb - 1, (q_off + min(T_q, (qb + 1) * bs) - 1) // bs)   # last block with a visible key
            ids = [kb for kb in range(last + 1) if kb == last or rng.random() < density]
            if rng.random() < 0.05:
                ids = []                                   # an empty query block
            bad = list(ids)
            for _ in range(int(rng.integers(0, 3))):
                bad.insert(int(rng.integers(0, len(bad) + 1)), int(rng.choice([-1, -5])))
            tail = sorted(set(int(x) for x in rng.integers(nkb, nkb + 50, size=int(rng.integers(0, 2)))))
            if bs >= 64 and rng.random() < 0.3:
                tail.append(1 << 30)
            rc.append(ids)
            rj.append(bad + tail)
        clean.append(rc)
        junk.append(rj)
    return dict(bs=bs, D=D, Hkv=Hkv, Hq=Hq, B=B, T_q=T_q, T_k=T_k, dtype=dtype, clean=clean, junk=junk)


def _csr(rows):
    width = max(1, max(sum(len(e) for e in r) for r in rows))
    pairs = torch.full((len(rows), width), -3, dtype=torch.int32)
    offsets = torch.zeros(len(rows), len(rows[0]) + 1, dtype=torch.int32)
    for r, blocks in enumerate(rows):
        flat = [b for e in blocks for b in e]
        if flat:
            pairs[r, :len(flat)] = torch.tensor(flat, dtype=torch.int32)
        offsets[r, 1:] = torch.tensor(np.cumsum([len(e) for e in blocks]), dtype=torch.int32)
    return pairs, offsets


def run_prefill_case(seed: int):
    c = prefill_case(seed)
    tag = (f"seed {seed}: B={c['B']} Hq={c['Hq']} Hkv={c['Hkv']} rows={len(c['clean'])} D={c['D']} bs={c['bs']} "
           f"T_q={c['T_q']} T_k={c['T_k']} {str(c['dtype'])[6:]}")
    _say(f"[random prefill] {tag}")
    q = seeded((c["B"], c["Hq"], c["T_q"], c["D"]), seed, c["dtype"]).to(DEV)
    k = seeded((c["B"], c["Hkv"], c["T_k"], c["D"]), seed + 1, c["dtype"]).to(DEV)
    v = seeded((c["B"], c["Hkv"], c["T_k"], c["D"]), seed + 2, c["dtype"]).to(DEV)
    pairs, offsets = _csr(c["clean"])
    pairs_j, offsets_j = _csr(c["junk"])
    out = ops.universal_sparse_attn(q, k, v, pairs.to(DEV), offsets.to(DEV), c["bs"])
    out_j = ops.universal_sparse_attn(q, k, v, pairs_j.to(DEV), offsets_j.to(DEV), c["bs"])
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all(), tag
    assert torch.equal(out, out_j), f"{tag}: skipped entries changed the result"
    want = oa.block_sparse_attention(q, k, v, pairs, offsets, c["bs"])
    return assert_close_bf16(out, want, tag)


def decode_case(seed: int, many: bool = False) -> dict:
    """A paged cache, its block table and per-row lists (clean and with skipped entries).  ``many``:
    129-257 sequences with shorter caches, so that a launch has at least two units (sequence, row,
    split) per CU of an MI355X and runs two per workgroup."""
    rng = np.random.default_rng((7000 if many else 5000) + seed)
    page = int(rng.choice([16, 32, 64, 128]))
    D = int(rng.choice([64, 128]))
    Hkv = int(rng.integers(2, 5)) if many else int(rng.integers(1, 5))
    Hq = Hkv * int(rng.choice([1, 2, 4, 8]))
    B = int(rng.choice([129, 200, 257])) if many else int(rng.integers(1, 7))
    top = 1500 if many else 6000
    lens = [int(rng.choice([0, 1, int(rng.integers(2, top))], p=[0.05, 0.05, 0.9])) for _ in range(B)]
    nblk = [-(-L // page) for L in lens]
    max_blocks = max(1, max(nblk)) + int(rng.integers(0, 3))
    P = sum(nblk) + 3
    R = Hq if rng.random() < 0.3 else Hkv
    splits = int(rng.choice([1, 1, 2, 3, 5]))
    dtype = torch.bfloat16 if rng.random() < 0.7 else torch.float16
    perm = rng.permutation(P).astype(np.int32)
    table = np.zeros((B, max_blocks), dtype=np.int32)
    used = 0
    for b, n in enumerate(nblk):
        table[b, :n] = perm[used:used + n]
        used += n
    density = float(rng.choice([0.05, 0.3, 1.0]))
    clean, junk = [], []
    for b in range(B):
        for _ in range(R):
            ids = [kb for kb in range(nblk[b]) if rng.random() < density]
            bad = list(ids)
            for x in (-1, nblk[b], max_blocks + 4, 1 << 30)[:int(rng.integers(0, 5))]:
                bad.insert(int(rng.integers(0, len(bad) + 1)), int(x))
            clean.append(ids)
            junk.append(bad)
    return dict(page=page, D=D, Hkv=Hkv, Hq=Hq, B=B, lens=lens, P=P, R=R, splits=splits, dtype=dtype,
                table=table, clean=clean, junk=junk)


def _pack(rows, B, R):
    width = max(1, max(len(x) for x in rows))
    sel = np.zeros((B, R, width), dtype=np.int32)
    off = np.zeros((B, R, 2), dtype=np.int32)
    for i, x in enumerate(rows):
        sel[i // R, i % R, :len(x)] = x
        off[i // R, i % R, 1] = len(x)
    return sel, off


def run_decode_case(seed: int, many: bool = False):
    c = decode_case(seed, many)
    tag = (f"seed {seed}: B={c['B']} Hq={c['Hq']} Hkv={c['Hkv']} rows={c['R']} D={c['D']} page={c['page']} "
           f"splits={c['splits']} lens={c['lens']} {str(c['dtype'])[6:]}")
    _say(f"[random decode] {tag}")
    kp = seeded((c["P"], c["Hkv"], c["page"], c["D"]), seed, c["dtype"])
    vp = seeded((c["P"], c["Hkv"], c["page"], c["D"]), seed + 1, c["dtype"])
    q = seeded((c["B"], c["Hq"], c["D"]), seed + 2, c["dtype"])
    sel, off = _pack(c["junk"], c["B"], c["R"])
    csel, coff = _pack(c["clean"], c["B"], c["R"])
    t = lambda a: torch.from_numpy(a).to(DEV)
    out = ops.paged_sparse_decode(q.to(DEV), kp.to(DEV), vp.to(DEV), t(c["table"]),
                                  torch.tensor(c["lens"], dtype=torch.int32, device=DEV), t(sel), t(off),
                                  num_splits=c["splits"])
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all(), tag
    want = oa.paged_decode_attention(q, kp.to(DEV), vp.to(DEV), c["table"], np.array(c["lens"]), csel, coff,
                                     device=DEV)
    return assert_close_bf16(out, want, tag)


@pytest.mark.parametrize("seed", range(24))
def test_random_prefill_case(seed):
    run_prefill_case(seed)


@pytest.mark.parametrize("seed", range(24))
def test_random_decode_case(seed):
    run_decode_case(seed)


@pytest.mark.parametrize("seed", range(6))
def test_random_decode_case_two_units_per_workgroup(seed):
    c = decode_case(seed, many=True)
    hpr = c["Hq"] // c["R"]
    nh = 4 if hpr % 4 == 0 else 2 if hpr % 2 == 0 else 1
    units = c["B"] * c["R"] * (hpr // nh) * c["splits"]
    assert units >= 2 * 256, units   # two per CU of the 256 an MI355X has
    run_decode_case(seed, many=True)


def backend_case(seed: int):
    """A reference-compatible pattern class at a random shape, prefill, decode or chunked."""
    from sparseattentioninfer_amd import patterns as P
    rng = np.random.default_rng(9000 + seed)
    Hkv = int(rng.integers(1, 5))
    Hq = Hkv * int(rng.choice([1, 2, 4]))
    B = int(rng.integers(1, 3))
    D = int(rng.choice([64, 128]))
    T_k = int(rng.integers(16, 3000))
    mode = str(rng.choice(["prefill", "decode", "chunk"]))
    T_q = T_k if mode == "prefill" else (1 if mode == "decode" else int(rng.integers(2, T_k + 1)))
    kind = str(rng.choice(["bigbird", "bigbird2", "keep", "keep_groups", "local", "dense", "seeded", "bernoulli"]))
    dtype = torch.bfloat16 if rng.random() < 0.7 else torch.float16
    bs = int(rng.choice([16, 32, 64, 128]))
    if kind == "bigbird":
        pat = P.BigBirdPattern(top_k=int(rng.choice([16, 32, 64, 128, 256])), n_heads=Hq)
    elif kind == "bigbird2":
        pat = P.BigBird2Pattern(top_k=int(rng.choice([16, 32, 64, 128])), n_heads=Hq)
    elif kind == "keep":
        pat = P.BigBirdKeepRatioPattern(keep_ratio=float(rng.choice([0.1, 0.25, 0.5])), n_heads=Hq)
    elif kind == "keep_groups":
        pat = P.BigBirdKeepRatioPattern(group_sparsities=[float(x) for x in rng.choice([0.5, 0.7, 0.9], size=Hkv)],
                                        n_heads=Hq, n_kv_heads=Hkv)
    elif kind == "local":
        pat = P.LocalWindowPattern(window_size=int(rng.integers(8, 700)), block_size=bs)
    elif kind == "dense":
        pat = P.DenseCausalPattern()
    elif kind == "seeded":
        pat = P.SeededBigBirdPattern(rows=Hkv, block_size=bs, seed=seed)
    else:
        pat = P.BernoulliBlockPattern(rows=Hkv, density=float(rng.choice([0.05, 0.3])), block_size=bs, seed=seed)
    return dict(pat=pat, kind=kind, mode=mode, B=B, Hq=Hq, Hkv=Hkv, D=D, T_q=T_q, T_k=T_k, dtype=dtype)


def run_backend_case(seed: int):
    from sparseattentioninfer_amd.attention import get_backend
    c = backend_case(seed)
    tag = (f"seed {seed}: {c['kind']} {c['mode']} B={c['B']} Hq={c['Hq']} Hkv={c['Hkv']} D={c['D']} "
           f"T_q={c['T_q']} T_k={c['T_k']} {str(c['dtype'])[6:]}")
    _say(f"[random backend] {tag}")
    Hq, Hkv, D, T_q, T_k = c["Hq"], c["Hkv"], c["D"], c["T_q"], c["T_k"]
    q = seeded((c["B"], Hq, T_q, D), seed, c["dtype"]).to(DEV)
    k = seeded((c["B"], Hkv, T_k, D), seed + 1, c["dtype"]).to(DEV)
    v = seeded((c["B"], Hkv, T_k, D), seed + 2, c["dtype"]).to(DEV)
    meta = c["pat"].build(q, k, causal=True)
    be = get_backend("hip_block_sparse")
    out = be.forward(q, k, v, meta)
    torch.cuda.synchronize()
    assert be.actual_backend == "hip_block_sparse" and torch.isfinite(out.float()).all(), tag
    if meta.kind == "dense":   # bottom-right causal over all keys, fp32
        kf, vf = oa.repeat_kv(k.float(), Hq // Hkv), oa.repeat_kv(v.float(), Hq // Hkv)
        s = (q.float() @ kf.transpose(-1, -2).contiguous()) / D ** 0.5
        keep = torch.arange(T_k, device=DEV)[None, :] <= (T_k - T_q) + torch.arange(T_q, device=DEV)[:, None]
        want = torch.softmax(s.masked_fill(~keep, float("-inf")), dim=-1) @ vf
    else:                      # the kernels' semantics on the pattern's own CSR
        want = oa.block_sparse_attention(q, k, v, meta.block_pairs.cpu(), meta.block_pair_offsets.cpu(),
                                         meta.block_size)
    return assert_close_bf16(out, want, tag)


@pytest.mark.parametrize("seed", range(16))
def test_random_backend_case(seed):
    run_backend_case(seed)
