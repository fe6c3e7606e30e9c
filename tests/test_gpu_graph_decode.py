"""Graph-captured decode (GraphDecoder) against the eager Hugging Face decode on the paged cache.

Qwen3-4B layer shapes (hidden 2560, 32Q/8KV, head dim 128, vocab 151936) with four layers, BigBird in
layers 0-1 and dense causal in 2-3, batch 2, a 300-token prompt and 40 greedy steps, so decoding crosses
the query-block boundary at position 320 (a new decode selection row).  Every step of the graph run is a
replay of the one captured graph (after two eager warm-up steps), with synchronisations and eager work
between the replays.  The steps are teacher-forced with the eager run's tokens: each step's logits must
match the eager step's within bf16 tolerance and its chosen tokens must agree wherever that tolerance cannot
reorder the eager top two logits.
"""
import sys

import pytest
import torch

from sparseattentioninfer_amd.qwen3 import PagedKVCache
from sparseattentioninfer_amd.qwen3.graph_decode import GraphDecoder, _argmax_rows
from sparseattentioninfer_amd.qwen3.runtime import build_model, qwen3_config
from tests.helpers import assert_within_ulps

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def model_cfg():
    _say("[graph] building 4-layer Qwen3-4B-shaped model")
    cfg = qwen3_config(num_hidden_layers=4, sparse_layers=[0, 1], pattern="seeded_bigbird", block_size=64,
                       window=3, global_blocks=2, random_blocks=3, seed=5)
    return cfg, build_model(cfg, device="cuda", dtype=torch.bfloat16, seed=1)


@torch.inference_mode()
def test_graph_decode_within_one_query_block_is_bit_identical(model_cfg):
    """Module-by-module graph step (fused=False).  Positions 300-309 stay in query block 4: the graph holds
    the same selection width as every eager step, so both choose the same decode split count and the
    logits agree bit for bit."""
    cfg, model = model_cfg
    B, T, steps = 2, 300, 10
    ids = torch.randint(0, cfg.vocab_size, (B, T), generator=torch.Generator().manual_seed(8)).cuda()
    ce = PagedKVCache(cfg.num_hidden_layers, T + steps + 1, page=64, shuffle_seed=4)
    cg = PagedKVCache(cfg.num_hidden_layers, T + steps + 1, page=64, shuffle_seed=4)
    first = [model(input_ids=ids, past_key_values=c, use_cache=True, logits_to_keep=1).logits[:, -1].argmax(-1)
             for c in (ce, cg)]
    assert torch.equal(first[0], first[1])
    dec = GraphDecoder(model, cg, first[1], T + steps, keep_logits=True, fused=False)
    nxt = first[0]
    for s in range(steps):
        want = model(input_ids=nxt[:, None], past_key_values=ce, use_cache=True, logits_to_keep=1).logits[:, -1]
        got = dec.step().clone()
        torch.cuda.synchronize()
        assert torch.equal(dec.logits, want), f"step {s}: max-abs diff {(dec.logits.float() - want.float()).abs().max()}"
        nxt = want.argmax(-1)
        assert torch.equal(got, nxt), f"step {s}"
    assert dec.graph is not None
    _say(f"[graph] {steps} steps (2 eager, {steps - 2} replays) bit-identical to the eager decode")


@pytest.mark.parametrize("fused", [True, False], ids=["fused", "modules"])
@torch.inference_mode()
def test_graph_decode_matches_eager_paged_decode(model_cfg, fused):
    cfg, model = model_cfg
    B, T, steps = 2, 300, 40
    ids = torch.randint(0, cfg.vocab_size, (B, T), generator=torch.Generator().manual_seed(7)).cuda()

    def prompt(cache):
        out = model(input_ids=ids, past_key_values=cache, use_cache=True, logits_to_keep=1)
        return out.logits[:, -1].argmax(-1)

    _say("[graph] eager decode")
    ce = PagedKVCache(cfg.num_hidden_layers, T + steps + 1, page=64, shuffle_seed=2)
    nxt = prompt(ce)
    inputs, eager_logits = [], []
    for _ in range(steps):
        inputs.append(nxt.clone())
        out = model(input_ids=nxt[:, None], past_key_values=ce, use_cache=True, logits_to_keep=1)
        lg = out.logits[:, -1]
        nxt = lg.argmax(-1)
        eager_logits.append(lg.float().clone())

    # Teacher-forced: every step decodes the eager run's input token, so logits compare step by step.
    # The graph picks its decode split count from the widest selection it holds (the eager path picks
    # it per step), so bf16 roundings differ slightly.  With every logit within `diff` of the eager
    # one, the chosen token can differ only where the eager top two logits are within 2 * diff.
    _say("[graph] graph decode")
    cg = PagedKVCache(cfg.num_hidden_layers, T + steps + 1, page=64, shuffle_seed=2)
    dec = GraphDecoder(model, cg, prompt(cg), T + steps, keep_logits=True, fused=fused)
    checked = 0
    for s in range(steps):
        dec.ids.copy_(inputs[s])
        got = dec.step().clone()
        torch.cuda.synchronize()
        lg, ref = dec.logits.float(), eager_logits[s]
        diff, scale = (lg - ref).abs().max().item(), ref.abs().max().item()
        assert diff <= 2e-2 * max(1.0, scale), f"step {s}: logits max-abs diff {diff:.3e} (scale {scale:.3e})"
        top2 = ref.topk(2, dim=-1).values
        clear = (top2[:, 0] - top2[:, 1]) > 2 * diff + 1e-6
        assert torch.equal(got[clear], ref.argmax(-1)[clear]), f"step {s}: tokens differ"
        checked += int(clear.sum())
        if s in (0, 2, 19, 20, steps - 1):
            _say(f"[graph] step {s} ({'eager warm-up' if s < 2 else 'replay'}): logits max-abs diff {diff:.2e}"
                 f" (scale {scale:.2e})")
    _say(f"[graph] tokens compared at {checked} of {B * steps} (sequence, step) pairs")
    assert checked >= B * steps // 4
    dec.finish()
    assert dec.graph is not None
    assert cg.layers[0].store.seq_len() == T + steps
    # Layer 0's K/V depend only on the (teacher-forced) input tokens: the graph's paged writes went to
    # the same pages and slots as the eager writes, with the same bits (module path) or within the
    # rounding of the fused path (its q|k|v product sums K in another order; K then goes through the
    # head RMSNorm and the rotation k1 cos - k2 sin, whose outputs near zero keep the last-bit
    # differences of O(1) inputs, hence the ulp at magnitude 1 for K).
    ke, ve = ce.layers[0].store.gather()
    kg, vg = cg.layers[0].store.gather()
    if fused:
        assert_within_ulps(kg, ke, 2, "layer-0 K pages", scale=1.0)
        assert_within_ulps(vg, ve, 2, "layer-0 V pages")
    else:
        assert torch.equal(ke, kg) and torch.equal(ve, vg)


def test_two_stage_argmax_equals_argmax():
    """First maximum of each row, ties included (bf16 rows hold repeated values)."""
    g = torch.Generator().manual_seed(3)
    for x in (torch.randn(8, 151936, generator=g), torch.randn(8, 151936, generator=g).bfloat16(),
              torch.randint(0, 4, (8, 151936), generator=g).float()):
        x = x.cuda()
        assert torch.equal(_argmax_rows(x, 128), x.argmax(-1))


@torch.inference_mode()
def test_graph_decode_local_window_moving_inside_a_page():
    """A local window of 100 keys on 64-token pages moves its first block inside a page (positions
    675, 739, ...): the graph must attend to exactly the blocks the eager step does at every position,
    so teacher-forced logits track the eager ones across those positions and the page boundaries."""
    _say("[graph] local window 100, 2 layers")
    cfg = qwen3_config(num_hidden_layers=2, sparse_layers=[0], pattern="local", block_size=64,
                       sparse_attention_window_size=100)
    model = build_model(cfg, device="cuda", dtype=torch.bfloat16, seed=3)
    assert model.model.layers[0].self_attn.sparse_pattern.window_size == 100
    B, T, steps = 2, 630, 120                   # positions 630 .. 749
    ids = torch.randint(0, cfg.vocab_size, (B, T), generator=torch.Generator().manual_seed(9)).cuda()
    ce = PagedKVCache(cfg.num_hidden_layers, T + steps + 1, page=64, shuffle_seed=6)
    nxt = model(input_ids=ids, past_key_values=ce, use_cache=True, logits_to_keep=1).logits[:, -1].argmax(-1)
    inputs, eager = [], []
    for _ in range(steps):
        inputs.append(nxt.clone())
        lg = model(input_ids=nxt[:, None], past_key_values=ce, use_cache=True, logits_to_keep=1).logits[:, -1]
        nxt = lg.argmax(-1)
        eager.append(lg.float().clone())
    cg = PagedKVCache(cfg.num_hidden_layers, T + steps + 1, page=64, shuffle_seed=6)
    first = model(input_ids=ids, past_key_values=cg, use_cache=True, logits_to_keep=1).logits[:, -1].argmax(-1)
    dec = GraphDecoder(model, cg, first, T + steps, keep_logits=True, fused=True)
    worst = 0.0
    for s in range(steps):
        dec.ids.copy_(inputs[s])
        dec.step()
        torch.cuda.synchronize()
        diff = (dec.logits.float() - eager[s]).abs().max().item()
        scale = eager[s].abs().max().item()
        worst = max(worst, diff / max(1.0, scale))
        assert diff <= 2e-2 * max(1.0, scale), f"step {s} (position {T + s}): logits max-abs diff {diff:.3e}"
    _say(f"[graph] local window: {steps} teacher-forced steps, worst relative logit diff {worst:.2e}")
