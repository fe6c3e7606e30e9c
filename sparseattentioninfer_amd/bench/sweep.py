"""YAML sweeps over ExperimentConfigs (``sparse_attention_bench/runners/sweep_runner.py:34-140`` and
``decoder_sweep_runner.py``): list values are swept, scalars fixed; each entry of ``patterns`` adds
its own sweep of pattern parameters.

    python -m sparseattentioninfer_amd.bench.sweep --config sparseattentioninfer_amd/bench/configs/bigbird.yaml
    python -m sparseattentioninfer_amd.bench.sweep --config ... --kind decoder --num-layers 2 --output-dir out/
"""
from __future__ import annotations

import argparse
import itertools
import json
import sys
from pathlib import Path

import yaml

from .config import ExperimentConfig

_PATTERN_KEYS = ("topk", "keep_ratio", "window_size", "block_size", "density")


def _as_list(x):
    return list(x) if isinstance(x, (list, tuple)) else [x]


def load_yaml(path) -> dict:
    with open(path, encoding="utf-8") as f:
        return yaml.safe_load(f)


def build_configs_from_yaml(data: dict) -> list[ExperimentConfig]:
    sweep = data.get("experiment", data)
    axes = {
        "batch_size": _as_list(sweep.get("batch_size", 1)),
        "num_heads": _as_list(sweep.get("num_heads", 8)),
        "num_kv_heads": _as_list(sweep.get("num_kv_heads", None)),
        "head_dim": _as_list(sweep.get("head_dim", 128)),
        "seq_len": _as_list(sweep.get("seq_len", 512)),
        "dtype": _as_list(sweep.get("dtype", "bf16")),
        "device": _as_list(sweep.get("device", "cuda")),
        "mode": _as_list(sweep.get("mode", "prefill")),
    }
    fixed = {"causal": sweep.get("causal", True), "num_warmup": sweep.get("num_warmup", 20),
             "num_iters": sweep.get("num_iters", 100), "seed": sweep.get("seed", 0)}
    pattern_cfgs = []
    for p in sweep.get("patterns", [{"type": "dense", "backend": "hip_block_sparse"}]):
        values = [_as_list(p[k]) if k in p else [None] for k in _PATTERN_KEYS]
        for combo in itertools.product(*values):
            pattern_cfgs.append({"pattern_type": p["type"], "backend": p.get("backend", "hip_block_sparse"),
                                 **dict(zip(_PATTERN_KEYS, combo))})
    configs = []
    for combo in itertools.product(*axes.values(), pattern_cfgs):
        *vals, pat = combo
        configs.append(ExperimentConfig(**dict(zip(axes.keys(), vals)), **pat, **fixed))
    return configs


def run_sweep(configs: list[ExperimentConfig], kind: str = "layer", verbose: bool = True, **decoder_kw) -> list[dict]:
    """Runs every config (``kind`` "layer": BenchmarkRunner; "decoder": run_decoder_bench); errors are
    recorded per config, as the reference does."""
    from .bench_decoder import run_decoder_bench
    from .runner import BenchmarkRunner
    runner = BenchmarkRunner()
    results = []
    for i, cfg in enumerate(configs):
        if verbose:
            print(f"[{i + 1}/{len(configs)}] {cfg.pattern_type}/{cfg.backend} seq={cfg.seq_len} mode={cfg.mode} "
                  f"dtype={cfg.dtype}", flush=True)
        try:
            res = runner.run(cfg) if kind == "layer" else run_decoder_bench(cfg, **decoder_kw)
            res["_status"] = "ok"
        except Exception as exc:  # one failing config does not stop the sweep
            res = {"config": cfg.as_dict(), "_status": "error", "_error": f"{type(exc).__name__}: {exc}"}
            if verbose:
                print(f"  ERROR: {res['_error']}", flush=True)
        results.append(res)
    return results


def main(argv=None):
    ap = argparse.ArgumentParser(description="YAML benchmark sweep")
    ap.add_argument("--config", required=True)
    ap.add_argument("--kind", choices=("layer", "decoder"), default="layer")
    ap.add_argument("--num-layers", type=int, default=2)
    ap.add_argument("--vocab-size", type=int, default=5000)
    ap.add_argument("--kv-lens", type=int, nargs="+", default=None)
    ap.add_argument("--output-dir", default=None)
    a = ap.parse_args(argv)
    configs = build_configs_from_yaml(load_yaml(a.config))
    kw = {"num_layers": a.num_layers, "vocab_size": a.vocab_size, "kv_lens": a.kv_lens} if a.kind == "decoder" else {}
    results = run_sweep(configs, kind=a.kind, **kw)
    text = json.dumps(results, indent=2)
    if a.output_dir:
        out = Path(a.output_dir)
        out.mkdir(parents=True, exist_ok=True)
        path = out / f"sweep_{a.kind}_{Path(a.config).stem}.json"
        path.write_text(text)
        print(f"Saved to: {path}", file=sys.stderr)
    else:
        print(text)
    return results


if __name__ == "__main__":
    main()
