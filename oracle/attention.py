"""Attention semantics of the reference, restated on the CPU (torch fp32 / fp64).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

* :func:`masked_sdpa` restates ``MaskedSdpaBackend.forward``
  (``sparse_attentions/attention/masked_sdpa.py:23-68``): full scores, keep
  mask AND causal mask, ``-inf`` fill, softmax, NaN rows -> 0, times V.
* :func:`textbook_attention` is the float64 loop definition used to pin it.
* :func:`block_sparse_attention` restates the per-(head, query block) result of
  ``_universal_sparse_attn_kernel`` (``kernels/triton/universal_sparse_attn.py:77-160``):
  keys of the CSR-retained blocks, masked by ``q_abs >= k`` and bounds, with
  the query at absolute position ``q_offset + t``.  It gathers only retained
  blocks, so it runs at the full benchmark sizes; it is pinned against
  :func:`masked_sdpa` on small shapes.
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F


def causal_mask(seq_len: int, device=None) -> torch.Tensor:
    """``[1, 1, T, T]`` bool, True = forbidden; ``sparse_attentions/utils.py:6-12``."""
    m = torch.triu(torch.ones(seq_len, seq_len, dtype=torch.bool, device=device), diagonal=1)
    return m[None, None]


def repeat_kv(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    """``[B, Hkv, T, D] -> [B, Hkv*n_rep, T, D]``: query head ``h`` reads KV head ``h // n_rep``.

    This is the head mapping of Hugging Face ``repeat_kv`` that the reference's
    Qwen3 integration applies before calling a backend
    (``sparse_llm/qwen3/integrations/modeling_sparse_qwen3.py:233-234``).
    """
    if n_rep == 1:
        return x
    B, Hkv, T, D = x.shape
    return x[:, :, None].expand(B, Hkv, n_rep, T, D).reshape(B, Hkv * n_rep, T, D)


def masked_sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, kind: str,
                mask: torch.Tensor | None = None, topk: int | None = None) -> torch.Tensor:
    """Dense masked attention with the reference's exact rules (``masked_sdpa.py:23-68``).

    ``q [B,H,T_q,D]``, ``k, v [B,H,T_k,D]`` (same head count, as in the
    reference), ``mask [H,T_q,T_k]`` bool True = keep.  ``kind == "dense"``
    is SDPA with ``is_causal=True`` (top-left aligned for ``T_q != T_k``).
    Computes in the dtype of the inputs.
    """
    if kind == "dense":
        return F.scaled_dot_product_attention(q, k, v, is_causal=True)
    D = q.shape[-1]
    T_q, T_k = q.shape[2], k.shape[2]
    scores = torch.matmul(q, k.transpose(-2, -1).contiguous()) * (1.0 / math.sqrt(D))
    cm = causal_mask(T_k, q.device)
    if kind in ("mask", "local"):
        causal_keep = ~cm[:, :, -1:, :] if T_q == 1 else ~cm
        combined = mask[None] & causal_keep
        scores = scores.masked_fill(~combined, float("-inf"))
    elif kind == "topk":
        kk = min(topk, T_k)
        scores = scores.masked_fill(cm[:, :, -1:, :] if T_q == 1 else cm, float("-inf"))
        vals, idx = torch.topk(scores, k=kk, dim=-1)
        sparse = torch.full_like(scores, float("-inf"))
        sparse.scatter_(-1, idx, vals)
        scores = sparse
    else:
        raise ValueError(f"unknown pattern kind {kind!r}")
    attn = torch.nan_to_num(F.softmax(scores, dim=-1), nan=0.0)
    return torch.matmul(attn, v)


def masked_sdpa_rows(q_rows: torch.Tensor, k: torch.Tensor, v: torch.Tensor, keep_rows: torch.Tensor) -> torch.Tensor:
    """:func:`masked_sdpa` for a chunk of query rows of one head: dense scores against
    every key, ``-inf`` where ``keep_rows`` is False, softmax, NaN rows -> 0, times V.

    ``q_rows [m, D]``, ``k, v [T_k, D]``, ``keep_rows [m, T_k]`` bool (the pattern
    mask already ANDed with the causal mask).  Same arithmetic as
    ``masked_sdpa.py:35-68`` restricted to those rows, so the dense-masked CPU
    path can be timed on a bounded sample of a workload too large to materialise.
    """
    scores = torch.matmul(q_rows, k.transpose(0, 1).contiguous()) * (1.0 / math.sqrt(q_rows.shape[-1]))
    scores = scores.masked_fill(~keep_rows, float("-inf"))
    attn = torch.nan_to_num(F.softmax(scores, dim=-1), nan=0.0)
    return torch.matmul(attn, v)


def masked_sdpa_blockwise(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, block_mask: torch.Tensor,
                          block_size: int, q_offset: int | None = None, row_chunk: int = 1024) -> torch.Tensor:
    """:func:`masked_sdpa` over a block-level keep mask, in chunks of query rows, on q's device.

    The reference's dense-masked arithmetic (``masked_sdpa.py:35-68``: full scores against
    every key, ``-inf`` outside the keep mask AND the causal mask, softmax, NaN rows -> 0,
    times V), evaluated ``row_chunk`` query rows at a time so that workloads whose
    ``[H, T_q, T_k]`` score tensor cannot be held at once (32 K tokens) are still checked
    exhaustively.  ``q [B,Hq,T_q,D]``, ``k, v [B,Hkv,T_k,D]``; ``block_mask [R, NQB, NKB]``
    bool with ``R = Hq`` (per query head) or ``R = Hkv`` (per KV group); query row ``t`` sits
    at absolute position ``q_offset + t`` (default ``T_k - T_q``).  Computes in fp32.
    """
    B, Hq, T_q, D = q.shape
    Hkv, T_k = k.shape[1], k.shape[2]
    if q_offset is None:
        q_offset = T_k - T_q
    R = block_mask.shape[0]
    rowmap = _row_head_map(Hq, R)
    bs = block_size
    dev = q.device
    bm = block_mask.to(dev)
    out = torch.empty(B, Hq, T_q, D, dtype=torch.float32, device=dev)
    kpos = torch.arange(T_k, device=dev)
    scale = 1.0 / math.sqrt(D)
    for h in range(Hq):
        g = h // (Hq // Hkv)
        kt = k[:, g].float().transpose(1, 2).contiguous()            # [B, D, T_k]
        vg = v[:, g].float()
        for r0 in range(0, T_q, row_chunk):
            r1 = min(T_q, r0 + row_chunk)
            rows = torch.arange(r0, r1, device=dev)
            keep = bm[int(rowmap[h])][rows // bs].repeat_interleave(bs, dim=1)[:, :T_k]
            keep = keep & (kpos[None, :] <= (q_offset + rows)[:, None])
            scores = torch.matmul(q[:, h, r0:r1].float(), kt) * scale
            scores = scores.masked_fill(~keep[None], float("-inf"))
            attn = torch.nan_to_num(F.softmax(scores, dim=-1), nan=0.0)
            out[:, h, r0:r1] = torch.matmul(attn, vg)
    return out


def textbook_attention(q, k, v, keep) -> np.ndarray:
    """float64 loop definition: ``out[i] = sum_j softmax_j(q_i.k_j / sqrt(D))[keep] v_j``.

    ``q [T_q, D]``, ``k, v [T_k, D]``, ``keep [T_q, T_k]`` bool; a row with no
    kept key is zero.
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    T_q, D = q.shape
    out = np.zeros((T_q, v.shape[1]))
    for i in range(T_q):
        js = [j for j in range(k.shape[0]) if keep[i][j]]
        if not js:
            continue
        s = [sum(q[i, d] * k[j, d] for d in range(D)) / math.sqrt(D) for j in js]
        m = max(s)
        w = [math.exp(x - m) for x in s]
        z = sum(w)
        for wj, j in zip(w, js):
            out[i] += (wj / z) * v[j]
    return out


def csr_keep_mask(pairs, offsets, block_size: int, T_q: int, T_k: int, q_offset: int) -> np.ndarray:
    """Token keep mask the block kernel realises: retained tile AND ``q_offset + t >= k``.

    ``[R, T_q, T_k]`` bool for CSR rows ``R``.
    """
    pairs = np.asarray(pairs)
    offsets = np.asarray(offsets)
    R = offsets.shape[0]
    nqb = offsets.shape[1] - 1
    bs = block_size
    keep = np.zeros((R, T_q, T_k), dtype=bool)
    for r in range(R):
        for qb in range(nqb):
            q0, q1 = qb * bs, min(T_q, (qb + 1) * bs)
            for kb in pairs[r, offsets[r, qb]:offsets[r, qb + 1]]:
                k0, k1 = int(kb) * bs, min(T_k, (int(kb) + 1) * bs)
                keep[r, q0:q1, k0:k1] = True
    q_abs = q_offset + np.arange(T_q)
    keep &= (np.arange(T_k)[None, :] <= q_abs[:, None])[None]
    return keep


def _row_head_map(Hq: int, R: int) -> np.ndarray:
    """CSR row used by query head ``h``: its own row, or its KV group's row."""
    if R == Hq:
        return np.arange(Hq)
    if Hq % R:
        raise ValueError(f"CSR rows {R} must equal Hq={Hq} or divide it")
    return np.arange(Hq) // (Hq // R)


def block_sparse_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, pairs, offsets,
                           block_size: int, q_offset: int | None = None,
                           compute_dtype=torch.float32, p_dtype=None, rows=None) -> torch.Tensor:
    """Block-gather attention over a CSR schedule (fp32 by default), on q's device.

    ``q [B,Hq,T_q,D]``, ``k, v [B,Hkv,T_k,D]`` with ``Hq % Hkv == 0``;
    ``pairs/offsets`` have ``Hq`` rows or ``Hkv`` rows (one per KV group).
    ``q_offset`` defaults to ``T_k - T_q``.  ``p_dtype`` (e.g. bf16) rounds
    the probabilities before the PV product, as the kernels do.  ``rows``
    (optional) lists the ``(head, query block)`` pairs to compute; the others
    stay zero.  Returns fp32.
    """
    B, Hq, T_q, D = q.shape
    Hkv, T_k = k.shape[1], k.shape[2]
    n_rep = Hq // Hkv
    if q_offset is None:
        q_offset = T_k - T_q
    pairs = torch.as_tensor(np.asarray(pairs)).long()
    offsets = torch.as_tensor(np.asarray(offsets)).long()
    R = offsets.shape[0]
    nqb = offsets.shape[1] - 1
    rowmap = _row_head_map(Hq, R)
    bs = block_size
    dev = q.device
    qf = q.to(compute_dtype)
    kf = k.to(compute_dtype)
    vf = v.to(compute_dtype)
    out = torch.zeros(B, Hq, T_q, D, dtype=torch.float32, device=dev)
    scale = 1.0 / math.sqrt(D)
    todo = rows if rows is not None else [(h, qb) for h in range(Hq) for qb in range(nqb)]
    for h, qb in todo:
        r = int(rowmap[h])
        kvh = h // n_rep
        q0, q1 = qb * bs, min(T_q, (qb + 1) * bs)
        if q0 >= q1:
            continue
        kbs = pairs[r, offsets[r, qb]:offsets[r, qb + 1]].tolist()
        if not kbs:
            continue
        kidx = torch.cat([torch.arange(kb * bs, min(T_k, (kb + 1) * bs)) for kb in kbs]).to(dev)
        qs = qf[:, h, q0:q1]                        # [B, m, D]
        ks = kf[:, kvh].index_select(1, kidx)       # [B, n, D]
        vs = vf[:, kvh].index_select(1, kidx)
        s = torch.matmul(qs, ks.transpose(1, 2).contiguous()) * scale
        q_abs = q_offset + torch.arange(q0, q1, device=dev)
        allowed = kidx[None, :] <= q_abs[:, None]
        s = s.masked_fill(~allowed[None], float("-inf"))
        m = s.amax(dim=-1, keepdim=True)
        m = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
        p = torch.exp(s - m)
        l = p.sum(dim=-1, keepdim=True)
        if p_dtype is not None:
            p = p.to(p_dtype).to(compute_dtype)
        o = torch.matmul(p, vs) / torch.where(l > 0, l, torch.ones_like(l))
        out[:, h, q0:q1] = o.float()
    return out


def paged_decode_attention(q: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor,
                           block_table, kv_lens, sel, sel_offsets, device="cpu") -> torch.Tensor:
    """One decode token per sequence over a paged cache, fp32.

    ``q [B, Hq, D]``; pools ``[P, Hkv, page, D]``; ``block_table [B, max_blocks]``
    (logical block -> page); ``kv_lens [B]``; retained logical blocks of
    ``(b, row)`` are ``sel[b, row, sel_offsets[b,row,0]:sel_offsets[b,row,1]]``
    with rows = Hkv (group-shared) or Hq.  The query is the newest token, so
    every cached key of a retained block below ``kv_lens[b]`` is visible
    (``masked_sdpa.py:42-46``, decode row of the causal mask).  Computes on ``device``
    (the page pools are read where they are, only the retained pages are moved).
    """
    B, Hq, D = q.shape
    Hkv, page = k_pages.shape[1], k_pages.shape[2]
    n_rep = Hq // Hkv
    sel = np.asarray(sel)
    sel_offsets = np.asarray(sel_offsets)
    block_table = np.asarray(block_table)
    kv_lens = np.asarray(kv_lens)
    R = sel_offsets.shape[1]
    out = torch.zeros(B, Hq, D, dtype=torch.float32, device=device)
    scale = 1.0 / math.sqrt(D)
    kp, vp = k_pages, v_pages
    qf = q.float().to(device)
    for b in range(B):
        L = int(kv_lens[b])
        for h in range(Hq):
            r = h if R == Hq else h // (Hq // R)
            kvh = h // n_rep
            blocks = sel[b, r, sel_offsets[b, r, 0]:sel_offsets[b, r, 1]]
            ks, vs = [], []
            for lb in blocks:
                n = min(page, L - int(lb) * page)
                if n <= 0:
                    continue
                pg = int(block_table[b, int(lb)])
                ks.append(kp[pg, kvh, :n].to(device).float())
                vs.append(vp[pg, kvh, :n].to(device).float())
            if not ks:
                continue
            K = torch.cat(ks)
            V = torch.cat(vs)
            s = (K @ qf[b, h]) * scale
            w = torch.softmax(s, dim=0)
            out[b, h] = w @ V
    return out
