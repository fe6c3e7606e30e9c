"""The layer / Toy-Decoder benchmark harness on the HIP backend (prefill and decode), and the sweep
and decoder-bench command lines end to end."""
import json
import sys

import pytest

from sparseattentioninfer_amd.bench import BenchmarkRunner, ExperimentConfig
from sparseattentioninfer_amd.bench import bench_decoder, sweep

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _cfg(**kw):
    base = dict(num_heads=8, num_kv_heads=2, head_dim=128, seq_len=1024, num_warmup=2, num_iters=3)
    base.update(kw)
    return ExperimentConfig(**base)


@pytest.mark.parametrize("mode", ["prefill", "decode"])
def test_layer_runner_on_hip(mode):
    _say(f"[bench] layer {mode}")
    dense = BenchmarkRunner().run(_cfg(mode=mode))
    assert dense["actual_backend"] == "hip_block_sparse" and dense["rel_err"] == 0.0
    bb = BenchmarkRunner().run(_cfg(mode=mode, pattern_type="bigbird", topk=256))
    # the approximation error itself depends on the pattern; the harness must report a sane one
    assert 0 < bb["keep_ratio"] < 1 and bb["attention_time_ms_mean"] > 0
    assert bb["rel_err"] > 0 and -1.0 <= bb["cosine_sim"] <= 1.0 and bb["kl_divergence"] >= 0
    sb = BenchmarkRunner().run(_cfg(mode=mode, pattern_type="seeded_bigbird", block_size=64, seq_len=4096))
    assert 0 < sb["keep_ratio"] < 1


def test_decoder_bench_on_hip():
    _say("[bench] decoder")
    pre = bench_decoder.run_decoder_bench(_cfg(pattern_type="bigbird", topk=256), num_layers=2, vocab_size=500)
    assert pre["prefill"]["total_time_ms_mean"] > 0 and -1.0 <= pre["prefill"]["cosine_sim"] <= 1.0
    dec = bench_decoder.run_decoder_bench(_cfg(mode="decode"), num_layers=2, vocab_size=500, kv_lens=[256, 1000])
    assert [d["kv_len"] for d in dec["decode"]] == [256, 1000]
    assert all(d["rel_err"] == 0.0 for d in dec["decode"])     # dense pattern vs its dense twin


def test_command_lines(tmp_path):
    _say("[bench] command lines")
    y = tmp_path / "s.yaml"
    y.write_text("experiment:\n  num_heads: 8\n  num_kv_heads: 2\n  head_dim: 128\n  seq_len: [512]\n"
                 "  mode: [prefill, decode]\n  num_warmup: 1\n  num_iters: 2\n"
                 "  patterns:\n    - type: dense\n    - type: bigbird\n      topk: [128]\n")
    res = sweep.main(["--config", str(y), "--kind", "decoder", "--kv-lens", "256", "--output-dir", str(tmp_path)])
    assert len(res) == 4 and all(r["_status"] == "ok" for r in res)
    assert json.loads((tmp_path / "sweep_decoder_s.json").read_text())[0]["_status"] == "ok"
    out = bench_decoder.main(["--pattern", "seeded_bigbird", "--block-size", "64", "--seq-len", "2048",
                              "--num-kv-heads", "2", "--num-iters", "2", "--num-warmup", "1", "--no-print"])
    assert out["prefill"]["seq_len"] == 2048
