"""Test-only attention backend over the CPU/fp32 oracle, so callers (AttentionLayer, the Qwen3
integration) can be checked end to end against the reference's dense-masked semantics.

It computes ``oracle.attention.masked_sdpa`` (``masked_sdpa.py:23-68``) on an explicit token keep
mask: every causally visible key for ``kind == "dense"`` (bottom-right aligned, so a decode token
sees the whole cache), the CSR's token mask (``csr_keep_mask``) for block schedules.  Inputs are
promoted to fp32 and the result is cast back.
"""
from __future__ import annotations

import torch

from oracle import attention as oa
from sparseattentioninfer_amd.attention import AttentionBackend, register_backend
from sparseattentioninfer_amd.patterns.base import kv_block_list_to_pairs

NAME = "oracle_masked_sdpa"


class OracleBackend(AttentionBackend):
    supports_gqa = False   # callers repeat K/V, as for the reference's backends

    def __init__(self):
        self.calls = 0

    def keep_mask(self, H: int, T_q: int, T_k: int, pattern) -> torch.Tensor:
        if pattern.kind == "dense":
            return torch.ones(H, T_q, T_k, dtype=torch.bool)
        pairs, offsets = pattern.block_pairs, pattern.block_pair_offsets
        if pairs is None:
            pairs, offsets = kv_block_list_to_pairs(pattern.kv_block_list)
        keep = oa.csr_keep_mask(pairs.cpu().numpy(), offsets.cpu().numpy(), pattern.block_size, T_q, T_k, T_k - T_q)
        return torch.from_numpy(keep[oa._row_head_map(H, keep.shape[0])])

    def forward(self, q, k, v, pattern):
        self.calls += 1
        B, H, T_q, _ = q.shape
        T_k = k.size(2)
        if T_q not in (1, T_k):
            raise NotImplementedError("the oracle backend covers T_q == 1 and T_q == T_k")
        keep = self.keep_mask(H, T_q, T_k, pattern).to(q.device)
        out = oa.masked_sdpa(q.float(), k.float(), v.float(), "mask", keep)
        return out.to(q.dtype)

    @property
    def actual_backend(self) -> str:
        return NAME


def register() -> str:
    register_backend(NAME, OracleBackend)
    return NAME
