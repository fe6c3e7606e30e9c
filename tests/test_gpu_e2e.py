"""End to end at configs[4]: the Qwen3-4B architecture (36 layers, hidden 2560, 32Q/8KV, head dim
128, SwiGLU 9728, vocab 151936, random init), BigBird (window 3, global 2, random 3, block 64) in
layers 0-17 and dense causal in 18-35, batch 8, an 8192-token prompt, paged KV cache.

* Per-layer teacher forcing: every attention layer runs a twin backend that computes the HIP kernel
  and the reference's dense-masked arithmetic (fp32, row-chunked) on the same q/k/v and passes the
  oracle's result on, so each layer's kernel sees exactly the oracle path's inputs.  Every layer's
  attention core, in the prompt forward and in paged decode steps, must meet the kernel tolerance
  against the fp32 oracle: max-abs 2e-2 and mean-abs 2e-3.  The error relative to one bf16 ulp of
  the oracle value is printed beside it (the deeper layers of the random-init model produce
  attention outputs above 4, where one bf16 ulp is 3.1e-2).
* The logit max-abs difference of the all-kernel model against that oracle path (the reference's
  sparse path, which cannot run on this machine) is reported at the stated size
  (``sparse_llm/common/benchmark/generation.py:232-271`` defines the metrics).
"""
import sys

import pytest
import torch

from sparseattentioninfer_amd.qwen3 import PagedKVCache
from sparseattentioninfer_amd.qwen3.runtime import build_model, qwen3_config
from tests.helpers import MAX_ABS, MEAN_ABS
from tests.twin_backend import TwinBackend

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _use(model, backend_for_layer):
    for layer in model.model.layers:
        a = layer.self_attn
        be = backend_for_layer(a.layer_idx)
        a.sparse_backends = {"twin": be}
        a.backend_candidates = ["twin"]
        a.backend_name = "twin"
        a.sparse_backend = be


@torch.no_grad()
def test_configs_4_stated_size_teacher_forced_layers_and_logits():
    B, T, steps = 8, 8192, 2
    _say(f"[e2e] Qwen3-4B architecture, B={B}, prompt {T}")
    cfg = qwen3_config(sparse_layers=range(18), pattern="seeded_bigbird", block_size=64, window=3,
                       global_blocks=2, random_blocks=3, seed=11)
    model = build_model(cfg, device="cuda", dtype=torch.bfloat16, seed=0)
    assert {layer.self_attn.pattern_name for layer in model.model.layers} == {"seeded_bigbird", "dense"}
    hip_backends = [layer.self_attn.sparse_backend for layer in model.model.layers]
    ids = torch.randint(0, cfg.vocab_size, (B, T), generator=torch.Generator().manual_seed(12)).cuda()

    # oracle path, every layer's kernel checked on the oracle path's inputs
    twins = [TwinBackend("oracle") for _ in model.model.layers]
    _use(model, lambda i: twins[i])
    cache = PagedKVCache(cfg.num_hidden_layers, T + steps + 1, page=64, shuffle_seed=3)
    ref_logits, inputs = [], []
    nxt = None
    for s in range(steps + 1):
        inp = ids if s == 0 else nxt[:, None]
        lg = model(input_ids=inp, past_key_values=cache, use_cache=True, logits_to_keep=1).logits[:, -1].float()
        ref_logits.append(lg)
        nxt = lg.argmax(-1)
        inputs.append(nxt)
        recs = [t.records[-1] for t in twins]
        worst_max = max(r["max_abs"] for r in recs)
        worst_mean = max(r["mean_abs"] for r in recs)
        worst_ulp = max(r["ulp_ratio"] for r in recs)
        scale = max(r["out_scale"] for r in recs)
        _say(f"[e2e] {'prompt' if s == 0 else f'decode step {s}'}: worst layer attention max-abs {worst_max:.3e}, "
             f"mean-abs {worst_mean:.3e}, error / max(2e-2, 2^-7 |oracle|) {worst_ulp:.3f} over {len(recs)} layers "
             f"(largest attention output {scale:.2f})")
        for i, r in enumerate(recs):
            assert r["max_abs"] <= MAX_ABS and r["mean_abs"] <= MEAN_ABS, (s, i, r)
    assert all(t.last_kernel == "decode" for t in twins)
    del cache
    torch.cuda.empty_cache()

    # the all-kernel model against the oracle path, teacher-forced with the oracle path's tokens
    _use(model, lambda i: hip_backends[i])
    cache = PagedKVCache(cfg.num_hidden_layers, T + steps + 1, page=64, shuffle_seed=3)
    for s in range(steps + 1):
        inp = ids if s == 0 else inputs[s - 1][:, None]
        lg = model(input_ids=inp, past_key_values=cache, use_cache=True, logits_to_keep=1).logits[:, -1].float()
        ref = ref_logits[s]
        diff, scale = (lg - ref).abs().max().item(), ref.abs().max().item()
        agree = (lg.argmax(-1) == ref.argmax(-1)).float().mean().item()
        _say(f"[e2e] {'prompt' if s == 0 else f'decode step {s}'}: logit max-abs diff {diff:.4e} "
             f"(logit scale {scale:.3e}), top-1 agreement {agree:.3f}")
        assert torch.isfinite(lg).all()
        # bf16 activations over 36 layers compound (measured 4.3-4.8 % of the logit scale); each
        # layer is held to the kernel tolerance above
        assert diff <= 0.1 * max(1.0, scale), (s, diff, scale)
