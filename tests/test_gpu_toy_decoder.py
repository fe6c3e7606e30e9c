"""ToyDecoder on the HIP backend against the same weights on the oracle, prefill and cached decode.

The reference compares a sparse ToyDecoder with a dense one of shared weights
(``sparse_attention_bench/runners/decoder_sweep_runner.py:69-202``); here the check is parity
of the sparse path itself: every attention layer runs the twin backend (HIP kernel and the
reference's dense-masked arithmetic on the same inputs, the oracle's result passed on), so each
layer's kernel output is held to the kernel tolerance on the oracle path's inputs, and the
all-kernel model's logits are compared with that oracle path.
"""
import sys

import pytest
import torch

from sparseattentioninfer_amd.attention import get_backend
from sparseattentioninfer_amd.models import KVCache
from sparseattentioninfer_amd.models.decoder_block import ToyDecoder
from sparseattentioninfer_amd.patterns import DenseCausalPattern, SeededBigBirdPattern
from tests.helpers import MAX_ABS, MEAN_ABS
from tests.twin_backend import TwinBackend

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@torch.no_grad()
def test_toy_decoder_hip_tracks_oracle_prefill_and_decode():
    L, vocab, H, Hkv, D = 4, 2000, 8, 2, 128
    B, T, steps = 2, 2048, 3
    pats = [SeededBigBirdPattern(rows=Hkv, block_size=64, window=3, global_blocks=2, random_blocks=2, seed=i)
            for i in range(L - 1)] + [DenseCausalPattern()]          # last layer dense causal
    twins = [TwinBackend("oracle") for _ in range(L)]
    torch.manual_seed(0)
    ref = ToyDecoder(vocab, H * D, H, L, pats, twins, max_seq_len=T + 8, num_kv_heads=Hkv)
    ref = ref.to(device="cuda", dtype=torch.bfloat16).eval()
    hip = ToyDecoder(vocab, H * D, H, L, pats, [get_backend("hip_block_sparse") for _ in range(L)],
                     max_seq_len=T + 8, num_kv_heads=Hkv).to(device="cuda", dtype=torch.bfloat16).eval()
    hip.load_state_dict(ref.state_dict())
    ids = torch.randint(0, vocab, (B, T + steps), generator=torch.Generator().manual_seed(1)).cuda()
    c_ref, c_hip = KVCache(num_layers=L, max_len=T + steps), KVCache(num_layers=L, max_len=T + steps)
    for s in range(steps + 1):
        inp = ids[:, :T] if s == 0 else ids[:, T + s - 1:T + s]
        pos = 0 if s == 0 else T + s - 1
        lr = ref(inp, kv_cache=c_ref, pos_offset=pos)[:, -1].float()
        lh = hip(inp, kv_cache=c_hip, pos_offset=pos)[:, -1].float()
        recs = [t.records[-1] for t in twins]
        for i, r in enumerate(recs):
            assert r["max_abs"] <= MAX_ABS and r["mean_abs"] <= MEAN_ABS, (s, i, r)
            assert r["T_q"] == (T if s == 0 else 1)
        diff, scale = (lh - lr).abs().max().item(), lr.abs().max().item()
        _say(f"[toy] {'prefill' if s == 0 else f'decode {s}'}: worst layer max-abs "
             f"{max(r['max_abs'] for r in recs):.3e}; logits max-abs diff {diff:.3e} (scale {scale:.3e})")
        assert diff <= 0.05 * max(1.0, scale)
    assert all(be.last_kernel == "decode" for be in (blk.attn.backend for blk in hip.blocks))
    assert c_hip.seq_len(0) == T + steps
