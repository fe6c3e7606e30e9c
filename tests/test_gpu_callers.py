"""Callers on the GPU: AttentionLayer and the Qwen3 integration running the HIP kernels (prefill, and
decode from the paged cache), against the same modules on the fp32 dense-masked oracle backend."""
import copy
import sys

import pytest
import torch

from sparseattentioninfer_amd.attention import get_backend
from sparseattentioninfer_amd.models import AttentionLayer, KVCache
from sparseattentioninfer_amd.patterns import SeededBigBirdPattern
from sparseattentioninfer_amd.qwen3 import PagedKVCache, replace_qwen3_attention_with_sparse
from sparseattentioninfer_amd.qwen3.runtime import build_model, greedy_generate, qwen3_config
from transformers.cache_utils import DynamicCache
from tests import oracle_backend
from tests.helpers import assert_close_bf16

pytestmark = pytest.mark.gpu

DEV = "cuda"
ORACLE = oracle_backend.register()


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@torch.no_grad()
def test_attention_layer_prefill_and_cached_decode_match_oracle():
    _say("[callers] AttentionLayer")
    torch.manual_seed(0)
    pat = SeededBigBirdPattern(rows=2, block_size=64, window=3, global_blocks=2, random_blocks=2, seed=1)
    hip = AttentionLayer(512, 4, pat, get_backend("hip_block_sparse"), num_kv_heads=2).to(DEV, torch.bfloat16).eval()
    ref = copy.deepcopy(hip)
    ref.backend = get_backend(ORACLE)
    x = torch.randn(2, 700, 512, generator=torch.Generator().manual_seed(2)).to(DEV, torch.bfloat16)
    # the attention core is what differs: compare the pre-projection attention outputs
    core = {}
    hip.o_proj.register_forward_hook(lambda m, i, o: core.__setitem__("hip", i[0]))
    ref.o_proj.register_forward_hook(lambda m, i, o: core.__setitem__("ref", i[0]))
    hip(x)
    ref(x)
    assert hip.backend.last_kernel == "prefill"
    assert_close_bf16(core["hip"], core["ref"], "layer prefill")
    c_hip, c_ref = KVCache(1), KVCache(1)
    hip(x[:, :699], kv_cache=c_hip)
    ref(x[:, :699], kv_cache=c_ref)
    hip(x[:, 699:], kv_cache=c_hip)
    ref(x[:, 699:], kv_cache=c_ref)
    assert hip.backend.last_kernel == "decode" and c_hip.seq_len(0) == 700
    assert_close_bf16(core["hip"], core["ref"], "layer decode")


def _small_qwen3(backend):
    return qwen3_config(pattern="seeded_bigbird", backend=backend, sparse_layers=[0, 1], block_size=64,
                        window=3, global_blocks=2, random_blocks=2, seed=5, vocab_size=1000, hidden_size=512,
                        intermediate_size=1024, num_hidden_layers=4, num_attention_heads=4,
                        num_key_value_heads=2, head_dim=128, max_position_embeddings=4096)


@torch.no_grad()
def test_qwen3_hip_prefill_and_paged_decode_track_the_oracle():
    _say("[callers] qwen3 small")
    hip = build_model(_small_qwen3("hip_block_sparse"), device=DEV, dtype=torch.bfloat16, seed=3)
    ref = copy.deepcopy(hip)
    replace_qwen3_attention_with_sparse(ref.model, backend_name=ORACLE, block_size=64)
    kinds = [(layer.self_attn.pattern_name, layer.self_attn.backend_name) for layer in hip.model.layers]
    assert kinds == [("seeded_bigbird", "hip_block_sparse")] * 2 + [("dense", "hip_block_sparse")] * 2
    ids = torch.randint(0, 1000, (2, 640), generator=torch.Generator().manual_seed(4)).to(DEV)
    c_hip = PagedKVCache(4, 700, page=64, shuffle_seed=7)
    c_ref = DynamicCache(config=ref.config)
    # teacher-forced: both models see the same tokens, so their logits stay comparable every step
    worst = 0.0
    for step in range(9):
        inp = ids if step == 0 else nxt[:, None]
        la = hip(input_ids=inp, past_key_values=c_hip, use_cache=True, logits_to_keep=1).logits[:, -1].float()
        lb = ref(input_ids=inp, past_key_values=c_ref, use_cache=True, logits_to_keep=1).logits[:, -1].float()
        scale = lb.abs().max().item()
        diff = (la - lb).abs().max().item()
        _say(f"[callers] qwen3 step {step}: logits max-abs diff {diff:.3e} (scale {scale:.3e})")
        worst = max(worst, diff / scale)
        nxt = lb.argmax(-1)
    assert c_hip.get_seq_length() == 648
    assert all(layer.self_attn.sparse_backend.last_kernel == "decode" for layer in hip.model.layers)
    assert worst <= 0.05


@torch.no_grad()
def test_greedy_generate_reports_timings():
    _say("[callers] greedy_generate")
    model = build_model(_small_qwen3("hip_block_sparse"), device=DEV, dtype=torch.bfloat16, seed=3)
    ids = torch.randint(0, 1000, (2, 256), generator=torch.Generator().manual_seed(4)).to(DEV)
    g = greedy_generate(model, ids, 4, cache="paged")
    assert g["tokens"].shape == (2, 5) and len(g["decode_step_times_s"]) == 4
    assert g["ttft_s"] > 0 and g["decode_tokens_per_s"] > 0
    assert g["cache"].get_seq_length() == 260
