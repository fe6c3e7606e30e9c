"""Toy-Decoder benchmark (``sparse_attention_bench/benchmarks/bench_decoder.py:29-236``).

Prefill: one forward of ``[B, seq_len]`` token ids; decode: one token against a KV cache filled to
each ``kv_len``.  The sparse decoder's logits are compared with a dense-causal twin (same weights,
same backend, ``DenseCausalPattern``).  Decode steps restart from the same cached prefix by
truncating the cache (no copy inside the timed call).

    python -m sparseattentioninfer_amd.bench.bench_decoder --pattern seeded_bigbird --seq-len 4096 \\
        --num-heads 8 --head-dim 128 --mode decode --kv-lens 1024 4096
"""
from __future__ import annotations

import argparse
import json
import sys
from pathlib import Path

import torch

from ..attention import get_backend
from ..models.decoder_block import ToyDecoder
from ..models.kv_cache import KVCache
from ..patterns import DenseCausalPattern
from .config import ExperimentConfig
from .metrics import cosine_sim, marker, measure_latency, measure_peak_memory_mb, relative_error, top1_match_rate
from .runner import get_pattern


def build_decoder(cfg: ExperimentConfig, num_layers: int, pattern, backend_name: str, vocab_size: int,
                  d_model: int) -> ToyDecoder:
    torch.manual_seed(cfg.seed)
    model = ToyDecoder(vocab_size=vocab_size, d_model=d_model, num_heads=cfg.num_heads, num_layers=num_layers,
                       pattern=pattern, backend=get_backend(backend_name),
                       max_seq_len=max(cfg.seq_len + 1, 4096), causal=cfg.causal, num_kv_heads=cfg.num_kv_heads)
    return model.to(device=cfg.device, dtype=cfg.torch_dtype()).eval()


@torch.no_grad()
def run_decoder_bench(cfg: ExperimentConfig, num_layers: int = 2, vocab_size: int = 5000,
                      d_model: int | None = None, kv_lens: list[int] | None = None, markers: bool = True) -> dict:
    d_model = d_model or cfg.num_heads * cfg.head_dim
    sparse_dec = build_decoder(cfg, num_layers, get_pattern(cfg), cfg.backend, vocab_size, d_model)
    dense_dec = build_decoder(cfg, num_layers, DenseCausalPattern(), cfg.backend, vocab_size, d_model)
    dense_dec.load_state_dict(sparse_dec.state_dict())
    dev = torch.device(cfg.device)
    g = torch.Generator().manual_seed(cfg.seed + 1)
    results = {"config": cfg.as_dict(), "num_layers": num_layers, "d_model": d_model, "vocab_size": vocab_size}

    def lat(fn):
        return measure_latency(fn, num_iters=cfg.num_iters, num_warmup=cfg.num_warmup, device=cfg.device)

    if cfg.mode == "prefill":
        ids = torch.randint(0, vocab_size, (cfg.batch_size, cfg.seq_len), generator=g).to(dev)
        dense_out = dense_dec(ids)
        with marker("decoder_prefill", markers):
            latency = lat(lambda: sparse_dec(ids))
        peak = measure_peak_memory_mb(lambda: sparse_dec(ids), device=cfg.device)
        sparse_out = sparse_dec(ids)
        results["prefill"] = {
            "seq_len": cfg.seq_len,
            "total_time_ms_mean": latency["mean_ms"], "total_time_ms_p50": latency["p50_ms"],
            "total_time_ms_p95": latency["p95_ms"], "peak_memory_mb": peak,
            "rel_err": relative_error(sparse_out.float(), dense_out.float()),
            "cosine_sim": cosine_sim(sparse_out.float(), dense_out.float()),
            "top1_match": top1_match_rate(sparse_out.float(), dense_out.float()),
        }
        return results

    results["decode"] = []
    for kv_len in kv_lens or [128, 512, 2048]:
        if kv_len > cfg.seq_len:
            continue
        prefix = torch.randint(0, vocab_size, (cfg.batch_size, kv_len), generator=g).to(dev)
        token = torch.randint(0, vocab_size, (cfg.batch_size, 1), generator=g).to(dev)
        caches = {}
        for name, model in (("sparse", sparse_dec), ("dense", dense_dec)):
            caches[name] = KVCache(num_layers=num_layers, max_len=kv_len + 1)
            model(prefix, kv_cache=caches[name])

        def step(model=sparse_dec, cache=caches["sparse"]):
            out = model(token, kv_cache=cache, pos_offset=kv_len)
            cache.truncate(kv_len)
            return out

        with marker(f"decoder_decode_{kv_len}", markers):
            latency = lat(step)
        peak = measure_peak_memory_mb(step, device=cfg.device)
        sparse_out = step()
        dense_out = step(dense_dec, caches["dense"])
        results["decode"].append({
            "kv_len": kv_len,
            "total_time_ms_mean": latency["mean_ms"], "total_time_ms_p50": latency["p50_ms"],
            "total_time_ms_p95": latency["p95_ms"], "peak_memory_mb": peak,
            "rel_err": relative_error(sparse_out.float(), dense_out.float()),
            "cosine_sim": cosine_sim(sparse_out.float(), dense_out.float()),
        })
    return results


def parse_args(argv=None):
    p = argparse.ArgumentParser(description="End-to-end Toy-Decoder benchmark.")
    p.add_argument("--batch-size", type=int, default=1)
    p.add_argument("--num-heads", type=int, default=8)
    p.add_argument("--num-kv-heads", type=int, default=None)
    p.add_argument("--head-dim", type=int, default=128)
    p.add_argument("--seq-len", type=int, default=512)
    p.add_argument("--num-layers", type=int, default=2)
    p.add_argument("--d-model", type=int, default=None, help="default num_heads * head_dim")
    p.add_argument("--vocab-size", type=int, default=5000)
    p.add_argument("--dtype", default="bf16", choices=["fp16", "bf16"])
    p.add_argument("--device", default="cuda")
    p.add_argument("--mode", default="prefill", choices=["prefill", "decode"])
    p.add_argument("--pattern", default="dense",
                   choices=["dense", "bigbird", "bigbird2", "local_window", "seeded_bigbird", "bernoulli"])
    p.add_argument("--backend", default="hip_block_sparse")
    p.add_argument("--topk", type=int, default=None)
    p.add_argument("--keep-ratio", type=float, default=None)
    p.add_argument("--window-size", type=int, default=None)
    p.add_argument("--block-size", type=int, default=None)
    p.add_argument("--density", type=float, default=None)
    p.add_argument("--kv-lens", type=int, nargs="+", default=[128, 512, 2048])
    p.add_argument("--num-warmup", type=int, default=20)
    p.add_argument("--num-iters", type=int, default=100)
    p.add_argument("--output-dir", default=None)
    p.add_argument("--no-print", action="store_true")
    return p.parse_args(argv)


def main(argv=None):
    a = parse_args(argv)
    cfg = ExperimentConfig(batch_size=a.batch_size, num_heads=a.num_heads, num_kv_heads=a.num_kv_heads,
                           head_dim=a.head_dim, seq_len=a.seq_len, dtype=a.dtype, device=a.device, mode=a.mode,
                           pattern_type=a.pattern, backend=a.backend, topk=a.topk, keep_ratio=a.keep_ratio,
                           window_size=a.window_size, block_size=a.block_size, density=a.density,
                           num_warmup=a.num_warmup, num_iters=a.num_iters)
    result = run_decoder_bench(cfg, num_layers=a.num_layers, vocab_size=a.vocab_size, d_model=a.d_model,
                               kv_lens=a.kv_lens)
    if not a.no_print:
        print(json.dumps(result, indent=2))
    if a.output_dir:
        out = Path(a.output_dir)
        out.mkdir(parents=True, exist_ok=True)
        tag = f"{cfg.pattern_type}_{cfg.backend}_seq{cfg.seq_len}_{cfg.mode}_{cfg.dtype}"
        path = out / f"bench_decoder_{tag}.json"
        path.write_text(json.dumps(result, indent=2))
        print(f"Saved to: {path}", file=sys.stderr)
    return result


if __name__ == "__main__":
    main()
