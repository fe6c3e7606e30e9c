"""Layer / Toy-Decoder benchmark harness on the CPU, through the oracle backend: configuration,
YAML expansion, the pattern factory, result keys, and the toy decoder's cache path."""
from pathlib import Path

import pytest
import torch

from sparseattentioninfer_amd.attention import get_backend
from sparseattentioninfer_amd.bench import BenchmarkRunner, ExperimentConfig, get_pattern
from sparseattentioninfer_amd.bench.bench_decoder import run_decoder_bench
from sparseattentioninfer_amd.bench.sweep import build_configs_from_yaml, load_yaml, run_sweep
from sparseattentioninfer_amd.models import KVCache
from sparseattentioninfer_amd.models.decoder_block import ToyDecoder
from sparseattentioninfer_amd.patterns import (BigBirdKeepRatioPattern, BigBirdPattern, DenseCausalPattern,
                                               LocalWindowPattern, SeededBigBirdPattern)
from tests import oracle_backend

ORACLE = oracle_backend.register()
CONFIGS = Path(__file__).resolve().parent.parent / "sparseattentioninfer_amd" / "bench" / "configs"


def _cfg(**kw):
    base = dict(device="cpu", dtype="fp32", backend=ORACLE, num_heads=4, head_dim=16, seq_len=64,
                num_warmup=1, num_iters=2)
    base.update(kw)
    return ExperimentConfig(**base)


def test_config_validation_and_inputs():
    with pytest.raises(ValueError):
        _cfg(causal=False)
    with pytest.raises(ValueError):
        _cfg(num_kv_heads=3)
    q, k, v = _cfg(num_kv_heads=2, mode="decode").make_qkv()
    assert q.shape == (1, 4, 1, 16) and k.shape == v.shape == (1, 2, 64, 16)
    a, b = _cfg(seed=3).make_qkv()[0], _cfg(seed=3).make_qkv()[0]
    assert torch.equal(a, b)


def test_pattern_factory():
    assert isinstance(get_pattern(_cfg()), DenseCausalPattern)
    assert isinstance(get_pattern(_cfg(pattern_type="bigbird", topk=16)), BigBirdPattern)
    assert isinstance(get_pattern(_cfg(pattern_type="bigbird", keep_ratio=0.5)), BigBirdKeepRatioPattern)
    assert isinstance(get_pattern(_cfg(pattern_type="local_window", window_size=16, block_size=16)),
                      LocalWindowPattern)
    assert isinstance(get_pattern(_cfg(pattern_type="seeded_bigbird", block_size=16)), SeededBigBirdPattern)
    with pytest.raises(NotImplementedError):
        get_pattern(_cfg(pattern_type="topk", topk=8))
    with pytest.raises(ValueError):
        get_pattern(_cfg(pattern_type="nope"))


def test_yaml_expansion(tmp_path):
    y = tmp_path / "s.yaml"
    y.write_text("experiment:\n  seq_len: [64, 128]\n  mode: [prefill, decode]\n  device: cpu\n"
                 "  patterns:\n    - type: dense\n    - type: bigbird\n      topk: [8, 16]\n")
    cfgs = build_configs_from_yaml(load_yaml(y))
    assert len(cfgs) == 2 * 2 * 3
    assert {(c.pattern_type, c.topk) for c in cfgs} == {("dense", None), ("bigbird", 8), ("bigbird", 16)}
    assert all(c.backend == "hip_block_sparse" for c in cfgs)
    for f in CONFIGS.glob("*.yaml"):
        assert build_configs_from_yaml(load_yaml(f))


def test_layer_runner_keys_and_dense_identity():
    res = BenchmarkRunner(markers=False).run(_cfg())
    for key in ("pattern_build_time_ms_mean", "attention_time_ms_p95", "total_time_ms_mean", "peak_memory_mb",
                "rel_err", "cosine_sim", "kl_divergence", "keep_ratio", "sparsity_ratio"):
        assert key in res
    assert res["rel_err"] < 1e-6 and res["keep_ratio"] == 1.0
    sparse = BenchmarkRunner(markers=False).run(_cfg(pattern_type="seeded_bigbird", block_size=16, seq_len=256,
                                                     num_kv_heads=2))
    assert 0 < sparse["keep_ratio"] < 1 and sparse["rel_err"] > 0


def test_decoder_bench_prefill_and_decode():
    pre = run_decoder_bench(_cfg(pattern_type="bigbird", topk=16), num_layers=2, vocab_size=50, markers=False)
    assert pre["d_model"] == 64 and pre["prefill"]["rel_err"] >= 0 and 0 <= pre["prefill"]["top1_match"] <= 1
    dec = run_decoder_bench(_cfg(mode="decode"), num_layers=2, vocab_size=50, kv_lens=[16, 48, 100],
                            markers=False)
    assert [d["kv_len"] for d in dec["decode"]] == [16, 48]       # kv_len > seq_len skipped
    assert all(d["rel_err"] < 1e-5 for d in dec["decode"])        # dense vs dense


def test_sweep_records_errors(tmp_path):
    cfgs = [_cfg(), _cfg(pattern_type="topk", topk=4)]
    res = run_sweep(cfgs, kind="layer", verbose=False)
    assert [r["_status"] for r in res] == ["ok", "error"] and "topk" in res[1]["_error"]


@torch.no_grad()
def test_toy_decoder_cached_decode_matches_full_forward():
    torch.manual_seed(0)
    model = ToyDecoder(vocab_size=40, d_model=64, num_heads=4, num_layers=2, pattern=DenseCausalPattern(),
                       backend=get_backend(ORACLE), max_seq_len=64, num_kv_heads=2).eval()
    ids = torch.randint(0, 40, (2, 20), generator=torch.Generator().manual_seed(1))
    full = model(ids)
    cache = KVCache(num_layers=2)
    model(ids[:, :19], kv_cache=cache)
    last = model(ids[:, 19:], kv_cache=cache, pos_offset=19)
    assert torch.allclose(last, full[:, 19:], atol=1e-5)
    cache.truncate(19)
    assert cache.seq_len(0) == 19 and torch.allclose(model(ids[:, 19:], kv_cache=cache, pos_offset=19), last)


@torch.no_grad()
def test_toy_decoder_reference_attribute_path_and_state_dict_keys():
    """The reference's decoder runner reads ``model.blocks[0].attn.backend.actual_backend`` after a
    forward and copies weights with ``load_state_dict`` (decoder_sweep_runner.py:101-116); the
    checkpoint keys are those of sparse_attentions/models/decoder_block.py."""
    torch.manual_seed(0)
    kw = dict(vocab_size=50, d_model=32, num_heads=4, num_layers=2, max_seq_len=24)
    a = ToyDecoder(pattern=DenseCausalPattern(), backend=get_backend(ORACLE), **kw).eval()
    b = ToyDecoder(pattern=DenseCausalPattern(), backend=get_backend(ORACLE), **kw).eval()
    keys = set(a.state_dict())
    per_block = {"norm1.weight", "norm2.weight", "mlp.fc1.weight", "mlp.fc2.weight",
                 "attn.q_proj.weight", "attn.k_proj.weight", "attn.v_proj.weight", "attn.o_proj.weight"}
    want = {"token_emb.weight", "pos_emb.weight", "norm_f.weight", "lm_head.weight"}
    want |= {f"blocks.{i}.{k}" for i in range(2) for k in per_block}
    assert keys == want, keys ^ want
    assert a.lm_head.weight is a.token_emb.weight                        # tied head
    ids = torch.randint(0, 50, (2, 10), generator=torch.Generator().manual_seed(3))
    b.load_state_dict(a.state_dict())
    assert torch.equal(a(ids), b(ids))
    assert a.blocks[0].attn.backend.actual_backend == get_backend(ORACLE).actual_backend
    # RMSNorm is x / sqrt(mean(x^2) + eps) * weight, MLP is fc2(gelu(fc1(x)))
    x = torch.randn(3, 32)
    n = a.blocks[1].norm2
    n.weight.copy_(torch.rand(32) + 0.5)
    assert torch.allclose(n(x), x / x.pow(2).mean(-1, keepdim=True).add(1e-6).sqrt() * n.weight, atol=1e-6)
    m = a.blocks[0].mlp
    assert torch.allclose(m(x), torch.nn.functional.gelu(x @ m.fc1.weight.T) @ m.fc2.weight.T, atol=1e-6)
