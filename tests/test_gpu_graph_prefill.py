"""The persistent prefill kernel under HIP graph capture (``torch.cuda.CUDAGraph``): one captured launch,
replayed several times with eager launches, writes and synchronisations between the replays, gives the
eager launch's bits at every replay. The kernel resets its own work-item counters at the end of each
launch, so nothing in the graph clears the workspace (no memset node), and its status word stays clear.
Launches on two streams at once use one workspace per stream and give their single-stream bits."""
import sys

import pytest
import torch

from sparseattentioninfer_amd import ops
from sparseattentioninfer_amd.patterns import bernoulli_block_mask, block_mask_to_csr, seeded_bigbird_block_mask
from tests.helpers import seeded

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("kind", ["bernoulli_group_rows", "bigbird_head_rows"])
def test_prefill_graph_replays_give_the_eager_bits(kind):
    B, Hq, Hkv, T, D, bs = 2, 8, 2, 1500, 128, 64
    nqb = -(-T // bs)
    if kind == "bernoulli_group_rows":   # one CSR row per KV group: four-head persistent kernel
        bm = bernoulli_block_mask(Hkv, nqb, nqb, density=0.3, seed=9)
    else:                                # one CSR row per query head: one-head kernel
        bm = seeded_bigbird_block_mask(Hq, nqb, nqb, window=3, global_blocks=2, random_blocks=3, seed=11)
    pairs, offsets = (x.to(DEV) for x in block_mask_to_csr(bm))
    q = seeded((B, Hq, T, D), 21, torch.bfloat16).to(DEV)
    k = seeded((B, Hkv, T, D), 22, torch.bfloat16).to(DEV)
    v = seeded((B, Hkv, T, D), 23, torch.bfloat16).to(DEV)
    q2 = seeded((B, Hq, T, D), 24, torch.bfloat16).to(DEV)
    _say(f"[graph prefill] {kind}: eager warm-up on the capture stream")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        want = ops.universal_sparse_attn(q, k, v, pairs, offsets, bs)   # also creates the stream's workspace
    torch.cuda.synchronize()
    _say(f"[graph prefill] {kind}: capture")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out = ops.universal_sparse_attn(q, k, v, pairs, offsets, bs)
    torch.cuda.synchronize()
    for rep in range(4):
        out.zero_()
        other = ops.universal_sparse_attn(q2, k, v, pairs, offsets, bs)   # eager, on the current stream
        torch.cuda.synchronize()
        _say(f"[graph prefill] {kind}: replay {rep}")
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {rep}: max-abs {(out.float() - want.float()).abs().max()}"
        assert not torch.equal(other, want)
    with torch.cuda.stream(s):
        assert ops.prefill_workspace_status() == 0
    assert ops.prefill_workspace_status() == 0


def test_prefill_on_two_streams_at_once_uses_a_workspace_each():
    """Persistent launches on two streams overlap in time; each stream has its own counter pair, so each
    launch processes all its items (status words clear) and gives its single-stream bits."""
    B, Hq, Hkv, T, D, bs = 2, 8, 2, 2000, 128, 64
    nqb = -(-T // bs)
    pairs, offsets = (x.to(DEV) for x in block_mask_to_csr(bernoulli_block_mask(Hkv, nqb, nqb, density=0.3, seed=3)))
    ins = [tuple(seeded(shape, 40 + 3 * i + j, torch.bfloat16).to(DEV)
                 for j, shape in enumerate(((B, Hq, T, D), (B, Hkv, T, D), (B, Hkv, T, D)))) for i in range(2)]
    want = [ops.universal_sparse_attn(q, k, v, pairs, offsets, bs) for (q, k, v) in ins]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for st in streams:
        st.wait_stream(torch.cuda.current_stream())
    _say("[two streams] 8 rounds of overlapping launches")
    for rnd in range(8):
        got = [None, None]
        for i, st in enumerate(streams):
            with torch.cuda.stream(st):
                got[i] = ops.universal_sparse_attn(*ins[i], pairs, offsets, bs)
        torch.cuda.synchronize()
        for i in range(2):
            assert torch.equal(got[i], want[i]), f"round {rnd}, stream {i}"
    for st in streams:
        with torch.cuda.stream(st):
            assert ops.prefill_workspace_status() == 0
