"""Write golden CSR vectors from the reference's own pattern classes.

Run in the build container only (the reference is not present on GPU boxes)::

    python tests/golden/make_reference_vectors.py /root/reference

It imports ``sparse_attentions.patterns`` from the reference checkout (pure
torch, CPU) and stores, per case, the inputs and the outputs the reference
produced: ``block_pairs``, ``block_pair_offsets``, ``kv_block_list``,
``block_size``, ``keep_ratio`` and, for small shapes, the bit-packed token
mask.  These pin the functions that no published number or closed form pins:
the rotation hash for heads other than 0 (``bigbird_pattern.py:23-41``), the
per-group layout resolution of ``BigBirdKeepRatioPattern``
(``bigbird_pattern.py:421-449``), ``BigBird2Pattern`` rows, the
causal-block keep ratio (``bigbird_pattern.py:108-125``) and the
``LocalWindowPattern`` schedule when queries sit after a cached prefix
(``local_window.py:58-71``).

Output: ``tests/golden/reference_patterns.npz`` (data only) and
``tests/golden/reference_patterns.json`` (the case list).
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent

# (name, pattern kind, T_q, T_k, n_heads, params); all small enough for the CPU.
CASES = [
    ("bb_t128_k64", "bigbird", 128, 128, 4, {"top_k": 64}),
    ("bb_t256_k64", "bigbird", 256, 256, 8, {"top_k": 64}),
    ("bb_t512_k128", "bigbird", 512, 512, 8, {"top_k": 128}),
    ("bb_t1000_k256", "bigbird", 1000, 1000, 4, {"top_k": 256}),
    ("bb_t2048_k4096", "bigbird", 2048, 2048, 4, {"top_k": 4096}),
    ("bb_t4096_k2048", "bigbird", 4096, 4096, 4, {"top_k": 2048}),
    ("bb_t1500_k1024", "bigbird", 1500, 1500, 2, {"top_k": 1024}),
    ("bb_dec_t777_k256", "bigbird", 1, 777, 8, {"top_k": 256}),
    ("bb_dec_t2048_k64", "bigbird", 1, 2048, 4, {"top_k": 64}),
    ("kr_single_t512", "keep_ratio", 512, 512, 8, {"keep_ratio": 0.3}),
    ("kr_single_t1024_dec", "keep_ratio", 1, 1024, 8, {"keep_ratio": 0.2}),
    ("kr_groups_t1024", "keep_ratio", 1024, 1024, 8,
     {"group_sparsities": [0.5, 0.7, 0.8, 0.9], "n_kv_heads": 4}),
    ("kr_groups_t4096", "keep_ratio", 4096, 4096, 8,
     {"group_sparsities": [0.6, 0.95], "n_kv_heads": 2}),
    ("kr_groups_dec_t3000", "keep_ratio", 1, 3000, 8,
     {"group_sparsities": [0.5, 0.7, 0.8, 0.9], "n_kv_heads": 4}),
    ("bb2_t512_k128", "bigbird2", 512, 512, 4, {"top_k": 128}),
    ("bb2_dec_t700_k64", "bigbird2", 1, 700, 4, {"top_k": 64}),
    # sliding window: square, decode (T_q = 1) and a chunk after a cached prefix (1 < T_q < T_k),
    # where the query rows sit at max(0, T_k - T_q) + t (local_window.py:58-71)
    ("lw_t300_w100_b32", "local", 300, 300, 2, {"window_size": 100, "block_size": 32}),
    ("lw_dec_t777_w256_b64", "local", 1, 777, 2, {"window_size": 256, "block_size": 64}),
    ("lw_chunk_q96_k300_w80_b16", "local", 96, 300, 2, {"window_size": 80, "block_size": 16}),
    ("lw_chunk_q130_k1000_w512_b64", "local", 130, 1000, 3, {"window_size": 512, "block_size": 64}),
]

MASK_LIMIT = 1 << 22   # store token masks up to 4M entries


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from sparse_attentions.patterns import (  # noqa: E402  (reference, this container only)
        BigBird2Pattern, BigBirdKeepRatioPattern, BigBirdPattern, LocalWindowPattern)

    arrays: dict[str, np.ndarray] = {}
    index = []
    for name, kind, T_q, T_k, H, params in CASES:
        if kind == "bigbird":
            pat = BigBirdPattern(top_k=params["top_k"], n_heads=H)
        elif kind == "bigbird2":
            pat = BigBird2Pattern(top_k=params["top_k"], n_heads=H)
        elif kind == "local":
            pat = LocalWindowPattern(window_size=params["window_size"], block_size=params["block_size"])
        else:
            kw = {k: v for k, v in params.items()}
            pat = BigBirdKeepRatioPattern(n_heads=H, **kw)
        q = torch.zeros(1, H, T_q, 8)
        k = torch.zeros(1, H, T_k, 8)
        meta = pat.build(q, k, causal=True)
        arrays[f"{name}/block_pairs"] = meta.block_pairs.numpy().astype(np.int32)
        arrays[f"{name}/block_pair_offsets"] = meta.block_pair_offsets.numpy().astype(np.int32)
        if meta.kv_block_list is not None:
            arrays[f"{name}/kv_block_list"] = meta.kv_block_list.numpy().astype(np.int32)
        entry = {"name": name, "kind": kind, "T_q": T_q, "T_k": T_k, "n_heads": H,
                 "params": params, "block_size": int(meta.block_size),
                 "keep_ratio": float(meta.keep_ratio), "has_mask": False}
        if kind == "keep_ratio":
            entry["group_layouts"] = [list(map(int, lay)) for lay in pat.last_group_layouts]
        if meta.mask.numel() <= MASK_LIMIT:
            arrays[f"{name}/mask_bits"] = np.packbits(meta.mask.numpy().astype(bool), axis=-1)
            entry["has_mask"] = True
        index.append(entry)
    np.savez_compressed(HERE / "reference_patterns.npz", **arrays)
    (HERE / "reference_patterns.json").write_text(json.dumps(index, indent=1) + "\n")
    print(f"wrote {len(index)} cases")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
