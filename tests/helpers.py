"""Shared test helpers: seeded inputs, tolerance checks, golden fixtures."""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import torch

GOLDEN = Path(__file__).resolve().parent / "golden"

# BASELINE tolerances for bf16/fp16 outputs against the fp32 oracle.
MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def seeded(shape, seed, dtype, scale=None):
    """N(0,1) drawn on the CPU in fp32 with a seeded generator, optionally scaled, then cast."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g)
    if scale is not None:
        x = x * scale
    return x.to(dtype)


def assert_close_bf16(got: torch.Tensor, want: torch.Tensor, what: str = ""):
    diff = (got.float().cpu() - want.float().cpu()).abs()
    max_abs, mean_abs = diff.max().item(), diff.mean().item()
    assert max_abs <= MAX_ABS and mean_abs <= MEAN_ABS, (
        f"{what}: max-abs {max_abs:.3e} (tol {MAX_ABS}), mean-abs {mean_abs:.3e} (tol {MEAN_ABS})")
    return max_abs, mean_abs


def assert_within_ulps(got: torch.Tensor, want: torch.Tensor, ulps: int, what: str = "", scale: float = 0.0):
    """Every element of ``got`` within ``ulps`` units in the last place of ``want``'s dtype (bf16:
    2^-7 of the magnitude's power of two), for results whose arithmetic rounds the same way but
    may order a reduction differently.  With ``scale``, the ulp is taken at magnitude
    max(|want|, scale): for values computed as differences of terms of that size (a rotation), whose
    inputs' last-bit differences do not shrink with the result."""
    g, w = got.float().cpu(), want.float().cpu()
    mant = {torch.bfloat16: 7, torch.float16: 10}[want.dtype]
    ulp = torch.exp2(torch.floor(torch.log2(w.abs().clamp_min(max(scale, 1e-30)))) - mant)
    bad = (g - w).abs() > ulps * ulp
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {w.numel()} elements beyond {ulps} ulp; worst "
                           f"{((g - w).abs() / ulp).max().item():.1f} ulp")


def golden_case(name: str):
    idx = {c["name"]: c for c in json.loads((GOLDEN / "reference_patterns.json").read_text())}
    data = np.load(GOLDEN / "reference_patterns.npz")
    case = idx[name]
    out = {k.split("/", 1)[1]: data[k] for k in data.files if k.startswith(name + "/")}
    if "mask_bits" in out:
        out["mask"] = np.unpackbits(out.pop("mask_bits"), axis=-1, count=case["T_k"]).astype(bool)
    return case, out
