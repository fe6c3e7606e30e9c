"""Torch-facing operators over the gfx950 HIP library.

``universal_sparse_attn`` and ``bigbird_sparse_attn`` keep the names, argument
meaning and assertion messages of the reference's Triton entry points
(``kernels/triton/universal_sparse_attn.py:165-238``,
``kernels/triton/bigbird_sparse_attn.py:163-233``), so they are drop-ins.  Two
extensions: ``k``/``v`` may carry fewer (KV) heads than ``q`` (grouped-query
attention, query head ``h`` reads KV head ``h // (Hq / Hkv)``), and the CSR
may hold one row per KV group.

``paged_sparse_decode`` is new: one query token per sequence over a paged
cache.  All work is enqueued on the current HIP stream; nothing synchronises.
"""
from __future__ import annotations

import math

import torch

from . import _lib
from .patterns.base import kv_block_list_to_pairs

_DTYPES = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_F16}


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


_PREFILL_WS: dict = {}


def _prefill_workspace(t: torch.Tensor) -> torch.Tensor:
    """Zeroed workspace (counters and a status word) for the persistent prefill kernel, one per
    (device, stream).

    Each launch leaves its counters zeroed again; launches on one stream run in order, so they
    can share it.  Launches on other streams get their own.
    """
    stream = _stream(t)
    key = (t.device.index, stream)
    ws = _PREFILL_WS.get(key)
    if ws is None:
        nbytes = int(_lib.load().sa_prefill_workspace_bytes())
        ws = torch.zeros((nbytes + 3) // 4, dtype=torch.int32, device=t.device)
        _PREFILL_WS[key] = ws
    return ws


PREFILL_WS_STATUS_WORD = 3    # status word of the prefill workspace (include/sparse_attn.h)
PREFILL_WS_SKIPPED = 1        # a launch processed fewer work items than it has


def prefill_workspace_status(device=None, clear: bool = True) -> int:
    """Status word of the prefill workspace of the current stream on ``device`` (0: every launch
    so far processed all its work items; bit 0: one did not, its output is incomplete).
    Reads device memory (a synchronisation of the stream); ``clear`` resets the word."""
    dev = torch.device("cuda", torch.cuda.current_device() if device is None else torch.device(device).index)
    ws = _PREFILL_WS.get((dev.index, torch.cuda.current_stream(dev).cuda_stream))
    if ws is None:
        return 0
    st = int(ws[PREFILL_WS_STATUS_WORD].item())
    if clear and st:
        ws[PREFILL_WS_STATUS_WORD].zero_()
    return st


class TileSchedule:
    """A CSR schedule of block size 16 or 32 regrouped into 64 x 64 tiles (``csr_to_tiles``).

    ``pairs`` / ``masks [R, width]`` and ``offsets [R, ceil(NQB / s) + 1]``
    int32 on the GPU (s = 64 / block_size); ``status`` is a device int that
    stays 0 for a well-formed input CSR (bit 0: width overflow, bit 1: a query
    block's ids not ascending).  :meth:`check` reads it (a synchronisation).
    """

    def __init__(self, pairs, masks, offsets, status, block_size):
        self.pairs, self.masks, self.offsets, self.status = pairs, masks, offsets, status
        self.block_size = block_size

    def check(self) -> "TileSchedule":
        st = int(self.status.item())
        _require(not st & 1, "csr_to_tiles: a row needs more tiles than the CSR width (malformed offsets)")
        _require(not st & 2, "csr_to_tiles: block ids of a query block are not ascending "
                 "(the CSR holds sorted KB indices per query block)")
        return self


def csr_to_tiles(block_pairs: torch.Tensor, block_pair_offsets: torch.Tensor, block_size: int) -> TileSchedule:
    """Regroups a block-16/32 CSR into the tile schedule of the prefill kernel (on the GPU).

    One launch on the current stream, no synchronisation.  A row never needs
    more tiles than it has entries, so the tile arrays take the input's width.
    """
    name = "csr_to_tiles"
    _require(block_size in (16, 32), f"{name}: block_size {block_size} is not 16 or 32")
    _require(block_pairs.is_cuda and block_pairs.dtype == torch.int32
             and block_pair_offsets.dtype == torch.int32 and block_pair_offsets.device == block_pairs.device,
             f"{name}: CSR tensors must be int32 on the GPU")
    pairs = block_pairs.contiguous()
    offsets = block_pair_offsets.contiguous()
    R, nqb = pairs.size(0), offsets.size(1) - 1
    nqt = -(-nqb // (64 // block_size))
    width = max(1, pairs.size(1))
    dev = pairs.device
    tp = torch.empty(R, width, dtype=torch.int32, device=dev)
    tm = torch.empty(R, width, dtype=torch.int32, device=dev)
    to = torch.empty(R, nqt + 1, dtype=torch.int32, device=dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    rc = _lib.load().sa_csr_to_tiles(
        pairs.data_ptr(), pairs.stride(0), offsets.data_ptr(), offsets.stride(0),
        R, nqb, block_size, tp.data_ptr(), tm.data_ptr(), tp.stride(0), width,
        to.data_ptr(), to.stride(0), status.data_ptr(), _stream(pairs))
    _lib.check("sa_csr_to_tiles", rc)
    return TileSchedule(tp, tm, to, status, block_size)


def block_mask_to_csr_gpu(block_active: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """``[R, NQB, NKB]`` bool block mask on the GPU -> the reference's ``(pairs, offsets)``.

    Count pass, one read of the widest row (the reference pads every row to
    ``max(1, max nnz)``), write pass; bit-identical to the torch packing.
    """
    name = "block_mask_to_csr"
    _require(block_active.is_cuda and block_active.dim() == 3, f"{name}: needs a [R, NQB, NKB] GPU tensor")
    m = block_active.to(torch.uint8) if block_active.dtype != torch.uint8 else block_active
    if m.stride(2) != 1:
        m = m.contiguous()
    R, nqb, nkb = m.shape
    dev = m.device
    offsets = torch.empty(R, nqb + 1, dtype=torch.int32, device=dev)
    nnz = torch.empty(R, dtype=torch.int32, device=dev)
    lib = _lib.load()
    args = (m.data_ptr(), m.stride(0), m.stride(1), R, nqb, nkb, offsets.data_ptr(), offsets.stride(0),
            nnz.data_ptr())
    _lib.check(name, lib.sa_block_mask_to_csr(*args, None, 0, 0, None, _stream(m)))
    width = max(1, int(nnz.max().item())) if R else 1
    pairs = torch.empty(R, width, dtype=torch.int32, device=dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    _lib.check(name, lib.sa_block_mask_to_csr(*args, pairs.data_ptr(), pairs.stride(0), width,
                                              status.data_ptr(), _stream(m)))
    return pairs, offsets


def _mask_buffer(rows: int, nqb: int, nkb: int, device) -> torch.Tensor:
    """Byte mask ``[rows, nqb, nkb]`` as the generators write it: a view of a buffer whose
    query-block stride is NKB rounded up to 16 bytes."""
    sq = -(-max(1, nkb) // 16) * 16
    return torch.empty(rows, nqb, sq, dtype=torch.uint8, device=device)[:, :, :nkb]


def _mask_call(name: str, fn, buf: torch.Tensor, rows: int, nqb: int, nkb: int, *args) -> torch.Tensor:
    _lib.check(name, fn(buf.data_ptr(), buf.stride(0), buf.stride(1), rows, nqb, nkb, *args))
    return buf


def bigbird_block_mask_gpu(nqb: int, nkb: int, q_block_offset: int, layout: torch.Tensor, *,
                           head_base: int = 0, hash_blocks: int | None = None, dense_last: bool = False,
                           device=None) -> torch.Tensor:
    """The reference's BigBird rows as a ``[R, NQB, NKB]`` uint8 mask built on the GPU.

    ``layout [R, 3]`` int (global, sliding, random) per row; row ``r`` hashes as head
    ``head_base + r`` with ``hash_blocks`` (default NKB) blocks (``bigbird_pattern.py:23-41``).
    """
    device = torch.device(device) if device is not None else layout.device
    _require(device.type == "cuda", "bigbird_block_mask_gpu: needs a GPU device")
    lay = layout.to(device=device, dtype=torch.int32).contiguous()
    _require(lay.dim() == 2 and lay.size(1) == 3, "bigbird_block_mask_gpu: layout must be [R, 3]")
    R = lay.size(0)
    buf = _mask_buffer(R, nqb, nkb, device)
    hb = nkb if hash_blocks is None else int(hash_blocks)
    return _mask_call("sa_bigbird_block_mask", _lib.load().sa_bigbird_block_mask, buf, R, nqb, nkb,
                      int(q_block_offset), lay.data_ptr(), int(head_base), hb, int(bool(dense_last)),
                      torch.cuda.current_stream(device).cuda_stream)


def seeded_bigbird_block_mask_gpu(rows: int, nqb: int, nkb: int, *, window: int, global_blocks: int,
                                  random_blocks, seed: int, window_align: str = "trailing",
                                  q_block_offset: int = 0, device="cuda") -> torch.Tensor:
    """Seeded BigBird rows on Philox4x64-10 (see ``include/sparse_attn.h``), ``[R, NQB, NKB]`` uint8."""
    _require(window_align in ("trailing", "centred"), f"window_align must be 'trailing' or 'centred', got {window_align!r}")
    device = torch.device(device)
    counts = torch.as_tensor(random_blocks, dtype=torch.int32).reshape(-1)
    if counts.numel() == 1:
        counts = counts.expand(rows)
    _require(counts.numel() == rows, f"random_blocks has {counts.numel()} entries for {rows} rows")
    counts = counts.contiguous().to(device)
    buf = _mask_buffer(rows, nqb, nkb, device)
    return _mask_call("sa_seeded_bigbird_block_mask", _lib.load().sa_seeded_bigbird_block_mask, buf, rows, nqb,
                      nkb, int(q_block_offset), int(window), int(global_blocks), int(window_align == "centred"),
                      counts.data_ptr(), int(seed) & ((1 << 64) - 1), torch.cuda.current_stream(device).cuda_stream)


def bernoulli_block_mask_gpu(rows: int, nqb: int, nkb: int, *, density: float, seed: int, q_block_offset: int = 0,
                             device="cuda") -> torch.Tensor:
    """Bernoulli(density) rows on Philox4x64-10, diagonal kept, ``[R, NQB, NKB]`` uint8."""
    device = torch.device(device)
    buf = _mask_buffer(rows, nqb, nkb, device)
    return _mask_call("sa_bernoulli_block_mask", _lib.load().sa_bernoulli_block_mask, buf, rows, nqb, nkb,
                      int(q_block_offset), float(density), int(seed) & ((1 << 64) - 1),
                      torch.cuda.current_stream(device).cuda_stream)


def _schedule_args(pairs, offsets, block_size, tiles: TileSchedule | None):
    """Schedule arguments of sa_prefill: (pairs, offsets, masks) tensors to keep alive, the six
    pointer/stride arguments, and the number of schedule query blocks."""
    if block_size >= 64:
        return pairs, offsets, None, [pairs.data_ptr(), pairs.stride(0), offsets.data_ptr(), offsets.stride(0),
                                      None, 0], offsets.size(1) - 1
    if tiles is None:
        tiles = csr_to_tiles(pairs, offsets, block_size)
    return tiles.pairs, tiles.offsets, tiles.masks, [
        tiles.pairs.data_ptr(), tiles.pairs.stride(0), tiles.offsets.data_ptr(), tiles.offsets.stride(0),
        tiles.masks.data_ptr(), tiles.masks.stride(0)], tiles.offsets.size(1) - 1


def _require(cond: bool, msg: str) -> None:
    # The reference validates with `assert`; the same conditions raise AssertionError here,
    # but independent of Python's -O flag.
    if not cond:
        raise AssertionError(msg)


def _check_qkv(q, k, v, name):
    _require(q.is_cuda, f"{name} requires CUDA tensors")
    _require(k.is_cuda and v.is_cuda and k.device == q.device and v.device == q.device,
             f"{name}: q, k and v must be on the same GPU")
    _require(q.dtype in (torch.float16, torch.bfloat16), f"Expected fp16 or bf16, got {q.dtype}")
    _require(k.dtype == q.dtype and v.dtype == q.dtype, f"{name}: q, k, v dtypes differ")
    _require(q.dim() == 4 and k.dim() == 4 and v.dim() == 4, f"{name}: q, k, v must be [B, H, T, D]")
    _require(k.shape == v.shape, f"{name}: k and v shapes differ")
    _require(q.shape[0] == k.shape[0] and q.shape[3] == k.shape[3], f"{name}: batch/head-dim mismatch")
    _require(q.shape[1] % k.shape[1] == 0,
             f"{name}: {q.shape[1]} query heads not a multiple of {k.shape[1]} KV heads")
    for t in (q, k, v):
        _require(t.stride(3) == 1, f"{name}: the head dim must be contiguous")


def universal_sparse_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                          block_pairs: torch.Tensor, block_pair_offsets: torch.Tensor,
                          block_size: int, *, q_offset: int | None = None,
                          tiles: TileSchedule | None = None) -> torch.Tensor:
    """Block-sparse causal attention over a CSR schedule; returns ``[B, Hq, T_q, D]``.

    ``q [B, Hq, T_q, D]``, ``k, v [B, Hkv, T_k, D]`` fp16/bf16 on the GPU;
    ``block_pairs [R, max_pairs]`` / ``block_pair_offsets [R, NQB+1]`` int32
    with ``R == Hq`` or ``R == Hkv``.  Query row ``t`` is at absolute position
    ``q_offset + t`` (default ``T_k - T_q``).  ``T_q == 1`` runs the decode
    kernel (the reference runs its prefill kernel on one row).  Block sizes 16
    and 32 run the prefill kernel on 64 x 64 tiles with sub-block masks; pass
    ``tiles = csr_to_tiles(...)`` to reuse one conversion across calls.
    """
    name = "universal_sparse_attn"
    _check_qkv(q, k, v, name)
    B, Hq, T_q, D = q.shape
    Hkv, T_k = k.shape[1], k.shape[2]
    _require(block_size >= 16 and (block_size & (block_size - 1)) == 0,
             "block_size must be a power of 2 and >= 16")
    _require(block_pairs.dtype == torch.int32, "block_pairs must be int32")
    _require(block_pair_offsets.dtype == torch.int32, "block_pair_offsets must be int32")
    R = block_pairs.size(0)
    _require(R in (Hq, Hkv), f"block_pairs head dim {R} != H={Hq} (or KV heads {Hkv})")
    _require(block_pair_offsets.size(0) == R,
             f"block_pair_offsets head dim {block_pair_offsets.size(0)} != H={R}")
    _require(block_pairs.device == q.device and block_pair_offsets.device == q.device,
             f"{name}: CSR tensors must be on the GPU of q")
    pairs = block_pairs.contiguous()
    offsets = block_pair_offsets.contiguous()
    nqb = offsets.size(1) - 1
    sm_scale = 1.0 / math.sqrt(D)
    if q_offset is None:
        q_offset = T_k - T_q
    out = torch.empty(B, Hq, T_q, D, dtype=q.dtype, device=q.device)
    lib = _lib.load()
    if T_q == 1 and q_offset == T_k - 1:
        _require(nqb == 1, f"{name}: decode expects one CSR query block, got {nqb}")
        status = lib.sa_decode(
            _DTYPES[q.dtype],
            q.data_ptr(), q.stride(0), q.stride(1),
            k.data_ptr(), v.data_ptr(),
            *_kv_strides(k, v, name),
            None, 0, 0, 0, None, T_k,
            pairs.data_ptr(), 0, pairs.stride(0),
            offsets.data_ptr(), 0, offsets.stride(0),
            R,
            out.data_ptr(), out.stride(0), out.stride(1),
            B, Hq, Hkv, D, block_size, sm_scale,
            1, None, 0, _stream(q))
        _lib.check("sa_decode", status)
        return out
    _require(block_size <= 128, f"{name}: block_size {block_size} not supported by the "
             "gfx950 prefill kernel (16, 32, 64, 128)")
    _require(nqb == -(-T_q // block_size),
             f"{name}: {nqb} CSR query blocks but T_q={T_q} needs {-(-T_q // block_size)}")
    # `held` keeps the schedule tensors alive until the launch is enqueued: freed earlier,
    # their memory could be handed to an allocation (the workspace below) ahead of the kernel.
    *held, sched, nqb_k = _schedule_args(pairs, offsets, block_size, tiles)
    status = lib.sa_prefill(
        _DTYPES[q.dtype],
        q.data_ptr(), q.stride(0), q.stride(1), q.stride(2),
        k.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
        v.data_ptr(), v.stride(0), v.stride(1), v.stride(2),
        out.data_ptr(), out.stride(0), out.stride(1), out.stride(2),
        *sched,
        R, nqb_k, B, Hq, Hkv, T_q, T_k, D, block_size, int(q_offset), sm_scale,
        *_ws_args(_prefill_workspace(q)), _stream(q))
    del held   # enqueued: a later reuse of this memory is ordered after the kernel on the stream
    _lib.check("sa_prefill", status)
    return out


def _ws_args(ws: torch.Tensor):
    return ws.data_ptr(), ws.numel() * ws.element_size()


def _kv_strides(k, v, name):
    _require(k.stride() == v.stride(), f"{name}: k and v must share strides")
    return k.stride(0), k.stride(1), k.stride(2)


def bigbird_sparse_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                        kv_block_list: torch.Tensor, block_size: int) -> torch.Tensor:
    """Padded-list entry point (``bigbird_sparse_attn.py:163-233``): converts to CSR once."""
    _check_qkv(q, k, v, "bigbird_sparse_attn")
    pairs, offsets = kv_block_list_to_pairs(kv_block_list.to(q.device))
    return universal_sparse_attn(q, k, v, pairs, offsets, block_size)


def decode_workspace_bytes(B: int, Hq: int, D: int, num_splits: int) -> int:
    return int(_lib.load().sa_decode_workspace_bytes(B, Hq, D, num_splits))


def auto_decode_splits(B: int, rows: int, max_sel: int, target_workgroups: int = 512) -> int:
    """Splits of each (sequence, row) block list so that a decode launch has about
    ``target_workgroups`` workgroups (two per CU), keeping at least two blocks per split."""
    base = max(1, B * rows)
    want = -(-target_workgroups // base)
    return max(1, min(want, max_sel // 2, 16))


def paged_sparse_decode(q: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor,
                        block_table: torch.Tensor, kv_lens: torch.Tensor,
                        sel: torch.Tensor, sel_off: torch.Tensor, *,
                        num_splits: int = 1, workspace: torch.Tensor | None = None,
                        out: torch.Tensor | None = None) -> torch.Tensor:
    """One decode token per sequence over a paged cache, reading retained blocks only.

    ``q [B, Hq, D]`` (or ``[B, Hq, 1, D]``); pools ``k_pages, v_pages
    [P, Hkv, page, D]``; ``block_table [B, max_blocks]`` int32 (logical block
    -> page); ``kv_lens [B]`` int32; ``sel [B, R, max_sel]`` / ``sel_off
    [B, R, 2]`` int32 retained logical blocks per (sequence, row), R = Hq or
    Hkv.  ``num_splits > 1`` splits each row over workgroups and needs a
    byte workspace of :func:`decode_workspace_bytes` (allocated if omitted);
    ``num_splits=0`` picks the count with :func:`auto_decode_splits`.
    """
    name = "paged_sparse_decode"
    q3 = q.reshape(q.shape[0], q.shape[1], q.shape[-1]) if q.dim() == 4 else q
    _require(q3.is_cuda and k_pages.is_cuda and v_pages.is_cuda, f"{name} requires GPU tensors")
    _require(q3.dtype in _DTYPES and k_pages.dtype == q3.dtype and v_pages.dtype == q3.dtype,
             f"{name}: q/k/v must share an fp16 or bf16 dtype")
    _require(k_pages.shape == v_pages.shape and k_pages.dim() == 4, f"{name}: pools must be [P, Hkv, page, D]")
    B, Hq, D = q3.shape
    _, Hkv, page, Dk = k_pages.shape
    _require(D == Dk and Hq % Hkv == 0, f"{name}: head mismatch")
    for t in (block_table, kv_lens, sel, sel_off):
        _require(t.dtype == torch.int32 and t.device == q3.device, f"{name}: index tensors must be int32 on the GPU")
    _require(sel.dim() == 3 and sel_off.dim() == 3 and sel_off.shape[2] == 2, f"{name}: bad sel shapes")
    _require(block_table.dim() == 2 and block_table.size(0) == B,
             f"{name}: block_table must be [B={B}, max_blocks], got {tuple(block_table.shape)}")
    _require(kv_lens.shape == (B,), f"{name}: kv_lens must be [B={B}], got {tuple(kv_lens.shape)}")
    R = sel.shape[1]
    _require(R in (Hq, Hkv) and sel_off.shape[:2] == (B, R) and sel.shape[0] == B, f"{name}: bad sel rows")
    _require(sel.stride(2) == 1 and block_table.stride(1) == 1 and kv_lens.is_contiguous()
             and sel_off.stride(2) == 1, f"{name}: index tensors must be contiguous in the last dim")
    if num_splits == 0:
        num_splits = auto_decode_splits(B, R, sel.shape[2])
    if out is None:
        out = torch.empty(B, Hq, D, dtype=q3.dtype, device=q3.device)
    lib = _lib.load()
    if num_splits > 1:
        need = decode_workspace_bytes(B, Hq, D, num_splits)
        if workspace is None:
            workspace = torch.empty(need, dtype=torch.uint8, device=q3.device)
        _require(workspace.numel() * workspace.element_size() >= need, f"{name}: workspace too small")
    status = lib.sa_decode(
        _DTYPES[q3.dtype],
        q3.data_ptr(), q3.stride(0), q3.stride(1),
        k_pages.data_ptr(), v_pages.data_ptr(),
        *_kv_strides(k_pages, v_pages, name),
        block_table.data_ptr(), block_table.stride(0), block_table.size(1), k_pages.size(0),
        kv_lens.data_ptr(), 0,
        sel.data_ptr(), sel.stride(0), sel.stride(1),
        sel_off.data_ptr(), sel_off.stride(0), sel_off.stride(1),
        R,
        out.data_ptr(), out.stride(0), out.stride(1),
        B, Hq, Hkv, D, page, 1.0 / math.sqrt(D),
        num_splits, workspace.data_ptr() if workspace is not None else None,
        workspace.numel() * workspace.element_size() if workspace is not None else 0,
        _stream(q3))
    _lib.check("sa_decode", status)
    return out.reshape(q.shape) if q.dim() == 4 else out


class PreparedLaunch:
    """A validated kernel launch with bound pointers; ``__call__`` re-enqueues it.

    The bound tensors are kept alive by this object.  Re-launching writes the
    same output tensor; it enqueues on the stream that was current when the
    launch was prepared.
    """

    def __init__(self, fn_name: str, args: list, keep: tuple, out: torch.Tensor):
        self._fn = getattr(_lib.load(), fn_name)
        self._name = fn_name
        self._args = args
        self._keep = keep
        self.out = out

    def __call__(self) -> torch.Tensor:
        _lib.check(self._name, self._fn(*self._args))
        return self.out


def prepare_prefill(q, k, v, block_pairs, block_pair_offsets, block_size, *, out=None) -> PreparedLaunch:
    """Validates like :func:`universal_sparse_attn` (T_q > 1) and binds the launch.

    For block sizes 16 and 32 the tile schedule is converted once, here.
    """
    name = "prepare_prefill"
    _check_qkv(q, k, v, name)
    B, Hq, T_q, D = q.shape
    Hkv, T_k = k.shape[1], k.shape[2]
    _require(T_q > 1 and block_size in (16, 32, 64, 128), f"{name}: needs T_q > 1 and block 16/32/64/128")
    pairs = block_pairs.contiguous()
    offsets = block_pair_offsets.contiguous()
    _require(pairs.dtype == torch.int32 and offsets.dtype == torch.int32, f"{name}: CSR must be int32")
    R = pairs.size(0)
    _require(R in (Hq, Hkv) and offsets.size(0) == R, f"{name}: CSR rows {R} not Hq or Hkv")
    _require(offsets.size(1) - 1 == -(-T_q // block_size), f"{name}: CSR query blocks do not cover T_q")
    sp, so, sm, sched, nqb_k = _schedule_args(pairs, offsets, block_size, None)
    if out is None:
        out = torch.empty(B, Hq, T_q, D, dtype=q.dtype, device=q.device)
    args = [
        _DTYPES[q.dtype],
        q.data_ptr(), q.stride(0), q.stride(1), q.stride(2),
        k.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
        v.data_ptr(), v.stride(0), v.stride(1), v.stride(2),
        out.data_ptr(), out.stride(0), out.stride(1), out.stride(2),
        *sched,
        R, nqb_k, B, Hq, Hkv, T_q, T_k, D, block_size, T_k - T_q,
        1.0 / math.sqrt(D), *_ws_args(_prefill_workspace(q)), _stream(q)]
    return PreparedLaunch("sa_prefill", args, (q, k, v, pairs, offsets, sp, so, sm), out)


TIMELINE_RECORD_WORDS = 36    # words per workgroup written by sa_prefill_timeline
TIMELINE_PHASES = ("loop_top_reads", "setup_and_q_issue", "first_pops", "first_kv_issue", "lookahead_issue",
                   "load_wait", "barrier", "first_qk", "loop", "last_tile", "epilogue", "after_item")


def prepare_prefill_timeline(q, k, v, block_pairs, block_pair_offsets, block_size, *, out=None) -> PreparedLaunch:
    """:func:`prepare_prefill` through the instrumented copy of the persistent four-head kernel
    (``sa_prefill_timeline``; block 64 or 128, four query heads per CSR row, head dim 128).  Each
    launch writes the same output and a per-workgroup timeline into ``launch.timeline`` (int64,
    :data:`TIMELINE_RECORD_WORDS` words per workgroup; :func:`summarize_prefill_timeline` reads it).
    The stamps cost about 100 shader clocks each, so its timing is not the product kernel's."""
    name = "prepare_prefill_timeline"
    _check_qkv(q, k, v, name)
    B, Hq, T_q, D = q.shape
    Hkv, T_k = k.shape[1], k.shape[2]
    _require(T_q > 1 and block_size in (64, 128), f"{name}: needs T_q > 1 and block 64/128")
    pairs = block_pairs.contiguous()
    offsets = block_pair_offsets.contiguous()
    _require(pairs.dtype == torch.int32 and offsets.dtype == torch.int32, f"{name}: CSR must be int32")
    R = pairs.size(0)
    _require(R in (Hq, Hkv) and offsets.size(1) - 1 == -(-T_q // block_size),
             f"{name}: CSR rows {R} not Hq or Hkv, or its query blocks do not cover T_q")
    lib = _lib.load()
    words = int(lib.sa_prefill_timeline_words(_DTYPES[q.dtype]))
    _lib.check("sa_prefill_timeline_words", 0 if words > 0 else words)
    timeline = torch.zeros(words, dtype=torch.int64, device=q.device)
    if out is None:
        out = torch.empty(B, Hq, T_q, D, dtype=q.dtype, device=q.device)
    args = [
        _DTYPES[q.dtype],
        q.data_ptr(), q.stride(0), q.stride(1), q.stride(2),
        k.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
        v.data_ptr(), v.stride(0), v.stride(1), v.stride(2),
        out.data_ptr(), out.stride(0), out.stride(1), out.stride(2),
        pairs.data_ptr(), pairs.stride(0), offsets.data_ptr(), offsets.stride(0),
        R, offsets.size(1) - 1, B, Hq, Hkv, T_q, T_k, D, block_size, T_k - T_q,
        1.0 / math.sqrt(D), *_ws_args(_prefill_workspace(q)), timeline.data_ptr(), words, _stream(q)]
    launch = PreparedLaunch("sa_prefill_timeline", args, (q, k, v, pairs, offsets, timeline), out)
    launch.timeline = timeline
    return launch


def summarize_prefill_timeline(timeline: torch.Tensor) -> dict:
    """Summary of one ``sa_prefill_timeline`` launch's records (workgroups that wrote none are
    skipped): the shader clock (s_memtime against the 100 MHz s_memrealtime), per-item shader
    clocks of each phase for the first wave of the lower and of the upper 32-row half, loop
    clocks per step, and the spread of workgroup start and end times."""
    import numpy as np
    rec = timeline.detach().cpu().numpy().astype(np.int64).reshape(-1, TIMELINE_RECORD_WORDS)
    rec = rec[rec[:, 3] > rec[:, 1]]
    if rec.shape[0] == 0:
        raise ValueError("summarize_prefill_timeline: no workgroup wrote a record")
    mt0, rt0, mt1, rt1 = (rec[:, i].astype(np.float64) for i in range(4))
    halves = rec[:, 4:].reshape(-1, 2, 16) & 0xFFFFFFFF
    items = halves[:, 0, 12].sum()
    steps = halves[:, 0, 13].sum()
    clock = float(np.median((mt1 - mt0) / (rt1 - rt0))) * 0.1       # GHz: s_memrealtime runs at 100 MHz
    per_item = {}
    for h, half in enumerate(("lower", "upper")):
        tot = halves[:, h, :12].sum(axis=0)
        per_item[half] = {p: round(float(tot[i]) / max(items, 1)) for i, p in enumerate(TIMELINE_PHASES)}
        per_item[half]["total"] = round(float(tot.sum()) / max(items, 1))
    end_us = (rt1 - rt0.min()) / 100.0
    start_us = (rt0 - rt0.min()) / 100.0
    return {
        "workgroups": int(rec.shape[0]),
        "items": int(items),
        "loop_steps": int(steps),
        "clock_ghz": round(clock, 3),
        "steps_per_item": round(float(steps) / max(items, 1), 2),
        "loop_clocks_per_step": {half: round(float(halves[:, h, 8].sum()) / max(int(halves[:, h, 13].sum()), 1))
                                 for h, half in enumerate(("lower", "upper"))},
        "refits": int(halves[:, :, 14].sum()),
        "clocks_per_item": per_item,
        "workgroup_start_spread_us": round(float(start_us.max()), 2),
        "workgroup_end_us": {"min": round(float(end_us.min()), 2), "median": round(float(np.median(end_us)), 2),
                             "max": round(float(end_us.max()), 2)},
        "mean_idle_at_end_us": round(float((end_us.max() - end_us).mean()), 2),
    }


def prepare_paged_decode(q, k_pages, v_pages, block_table, kv_lens, sel, sel_off, *,
                         num_splits: int = 1, out=None) -> PreparedLaunch:
    """Validates like :func:`paged_sparse_decode` and binds the launch (workspace included)."""
    q3 = q.reshape(q.shape[0], q.shape[1], q.shape[-1]) if q.dim() == 4 else q
    B, Hq, D = q3.shape
    if out is None:
        out = torch.empty(B, Hq, D, dtype=q3.dtype, device=q3.device)
    ws = None
    if num_splits > 1:
        ws = torch.empty(decode_workspace_bytes(B, Hq, D, num_splits), dtype=torch.uint8, device=q3.device)
    paged_sparse_decode(q3, k_pages, v_pages, block_table, kv_lens, sel, sel_off,
                        num_splits=num_splits, workspace=ws, out=out)   # validates once
    Hkv, page = k_pages.shape[1], k_pages.shape[2]
    args = [
        _DTYPES[q3.dtype],
        q3.data_ptr(), q3.stride(0), q3.stride(1),
        k_pages.data_ptr(), v_pages.data_ptr(), k_pages.stride(0), k_pages.stride(1), k_pages.stride(2),
        block_table.data_ptr(), block_table.stride(0), block_table.size(1), k_pages.size(0), kv_lens.data_ptr(), 0,
        sel.data_ptr(), sel.stride(0), sel.stride(1), sel_off.data_ptr(), sel_off.stride(0), sel_off.stride(1),
        sel.shape[1], out.data_ptr(), out.stride(0), out.stride(1),
        B, Hq, Hkv, D, page, 1.0 / math.sqrt(D),
        num_splits, ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0,
        _stream(q3)]
    return PreparedLaunch("sa_decode", args, (q3, k_pages, v_pages, block_table, kv_lens, sel, sel_off, ws), out)


# ---- fused stages of a Qwen3 decode step (graph-captured end-to-end decode) ----------------

def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float, *, residual: torch.Tensor | None = None,
            out: torch.Tensor | None = None) -> torch.Tensor:
    """Qwen3RMSNorm of the rows of ``x [rows, n]`` (fp32 inside, Hugging Face's roundings).

    With ``residual [rows, n]``: ``residual += x`` (rounded, in place) first, and the sum is
    normalised -- the residual add and the following norm of a decoder layer in one launch.
    """
    name = "rmsnorm"
    _require(x.is_cuda and x.dim() == 2 and x.stride(1) == 1 and x.dtype in _DTYPES, f"{name}: bad x")
    rows, n = x.shape
    _require(n % 8 == 0 and n <= 8192, f"{name}: n={n} (a multiple of 8, at most 8192)")
    _require(weight.shape == (n,) and weight.dtype == x.dtype and weight.is_contiguous(), f"{name}: bad weight")
    if residual is not None:
        _require(residual.shape == x.shape and residual.dtype == x.dtype and residual.stride(1) == 1,
                 f"{name}: bad residual")
    if out is None:
        out = torch.empty_like(x)
    _require(out.shape == x.shape and out.dtype == x.dtype and out.stride(1) == 1, f"{name}: bad out")
    status = _lib.load().sa_rmsnorm(
        _DTYPES[x.dtype], x.data_ptr(), x.stride(0),
        residual.data_ptr() if residual is not None else None, residual.stride(0) if residual is not None else 0,
        weight.data_ptr(), out.data_ptr(), out.stride(0), rows, n, float(eps), _stream(x))
    _lib.check("sa_rmsnorm", status)
    return out


def qk_rope_kv(qkv: torch.Tensor, q_norm_weight: torch.Tensor, k_norm_weight: torch.Tensor,
               inv_freq: torch.Tensor, position: torch.Tensor, store, q_out: torch.Tensor, *,
               num_heads: int, eps: float) -> torch.Tensor:
    """q/k RMSNorm + rotary embedding of the fused ``qkv [B, (Hq + 2 Hkv) * D]`` row of one new token per
    sequence; the query heads go to ``q_out [B, Hq, D]``, the key and value heads into the pages of the
    :class:`~sparseattentioninfer_amd.models.kv_cache.PagedKVStore` at ``position`` (a device int64
    ``[1]``); the store's page table must already cover that position."""
    name = "qk_rope_kv"
    B = qkv.size(0)
    Hkv, D = store.heads, store.head_dim
    _require(qkv.is_cuda and qkv.dim() == 2 and qkv.stride(1) == 1 and qkv.dtype in _DTYPES, f"{name}: bad qkv")
    _require(qkv.size(1) == (num_heads + 2 * Hkv) * D and B == store.batch, f"{name}: qkv width")
    _require(store.k_pages.dtype == qkv.dtype and store.k_pages.stride(3) == 1, f"{name}: pages")
    _require(inv_freq.dtype == torch.float32 and inv_freq.numel() == D // 2 and inv_freq.is_contiguous(),
             f"{name}: inv_freq must be fp32 [D/2]")
    _require(position.dtype == torch.int64 and position.is_cuda, f"{name}: position must be a device int64")
    _require(q_out.shape == (B, num_heads, D) and q_out.stride(2) == 1 and q_out.dtype == qkv.dtype,
             f"{name}: bad q_out")
    for w in (q_norm_weight, k_norm_weight):
        _require(w.shape == (D,) and w.dtype == qkv.dtype and w.is_contiguous(), f"{name}: bad norm weight")
    kp = store.k_pages
    status = _lib.load().sa_qk_rope_kv(
        _DTYPES[qkv.dtype], qkv.data_ptr(), qkv.stride(0), q_norm_weight.data_ptr(), k_norm_weight.data_ptr(),
        inv_freq.data_ptr(), position.data_ptr(), q_out.data_ptr(), q_out.stride(0), q_out.stride(1),
        kp.data_ptr(), store.v_pages.data_ptr(), kp.stride(0), kp.stride(1), kp.stride(2),
        store.block_table.data_ptr(), store.block_table.stride(0), store.block_table.size(1), kp.size(0),
        B, num_heads, Hkv, D, store.page, float(eps), _stream(qkv))
    _lib.check("sa_qk_rope_kv", status)
    return q_out


def swiglu(gate_up: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """``silu(gate) * up`` of Qwen3MLP from the fused ``gate_up [B, 2I]`` (gate first)."""
    name = "swiglu"
    _require(gate_up.is_cuda and gate_up.dim() == 2 and gate_up.stride(1) == 1 and gate_up.dtype in _DTYPES
             and gate_up.size(1) % 2 == 0, f"{name}: bad gate_up")
    B, I = gate_up.size(0), gate_up.size(1) // 2
    if out is None:
        out = torch.empty(B, I, dtype=gate_up.dtype, device=gate_up.device)
    _require(out.shape == (B, I) and out.stride(1) == 1 and out.dtype == gate_up.dtype, f"{name}: bad out")
    status = _lib.load().sa_swiglu(_DTYPES[gate_up.dtype], gate_up.data_ptr(), gate_up.stride(0), out.data_ptr(),
                                   out.stride(0), B, I, _stream(gate_up))
    _lib.check("sa_swiglu", status)
    return out


def gemm_skinny(x: torch.Tensor, w: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """``x [M, K] @ w[N, K]^T`` for M <= 8 (a decode step's projections): streams the weights once,
    fp32 accumulation, one rounding of each output."""
    name = "gemm_skinny"
    _require(x.is_cuda and w.is_cuda and x.dim() == 2 and w.dim() == 2 and x.dtype in _DTYPES
             and w.dtype == x.dtype and x.stride(1) == 1 and w.stride(1) == 1, f"{name}: bad operands")
    M, K = x.shape
    N = w.size(0)
    _require(w.size(1) == K and M <= 8 and K % 8 == 0 and K <= 10240, f"{name}: M={M} (<= 8), K={K}")
    if out is None:
        out = torch.empty(M, N, dtype=x.dtype, device=x.device)
    _require(out.shape == (M, N) and out.stride(1) == 1 and out.dtype == x.dtype, f"{name}: bad out")
    status = _lib.load().sa_gemm_skinny(_DTYPES[x.dtype], x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0),
                                        out.data_ptr(), out.stride(0), M, N, K, _stream(x))
    _lib.check("sa_gemm_skinny", status)
    return out


def interleave_gate_up(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """``[I, K]`` gate and up weights as one ``[2I, K]`` tensor with row 2i = gate row i and row
    2i + 1 = up row i (the layout ``gemm_skinny_swiglu`` reads)."""
    _require(gate.shape == up.shape and gate.dim() == 2 and gate.dtype == up.dtype, "interleave_gate_up: shapes")
    return torch.stack([gate, up], dim=1).reshape(2 * gate.size(0), gate.size(1)).contiguous()


def gemm_skinny_swiglu(x: torch.Tensor, w_gate_up: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """SwiGLU of the gate and up projections of ``x [M, K]`` (M <= 8) in one launch, from the
    interleaved weights of :func:`interleave_gate_up`: the bits of ``gemm_skinny`` on the
    concatenated ``[gate; up]`` rows followed by ``swiglu``."""
    name = "gemm_skinny_swiglu"
    _require(x.is_cuda and w_gate_up.is_cuda and x.dim() == 2 and w_gate_up.dim() == 2 and x.dtype in _DTYPES
             and w_gate_up.dtype == x.dtype and x.stride(1) == 1 and w_gate_up.stride(1) == 1, f"{name}: bad operands")
    M, K = x.shape
    N2 = w_gate_up.size(0)
    _require(w_gate_up.size(1) == K and M <= 8 and N2 % 2 == 0 and K % 128 == 0,
             f"{name}: M={M} (<= 8), K={K} (a multiple of 128), {N2} weight rows (even)")
    I = N2 // 2
    if out is None:
        out = torch.empty(M, I, dtype=x.dtype, device=x.device)
    _require(out.shape == (M, I) and out.stride(1) == 1 and out.dtype == x.dtype, f"{name}: bad out")
    status = _lib.load().sa_gemm_skinny_swiglu(_DTYPES[x.dtype], x.data_ptr(), x.stride(0), w_gate_up.data_ptr(),
                                               w_gate_up.stride(0), out.data_ptr(), out.stride(0), M, I, K, _stream(x))
    _lib.check("sa_gemm_skinny_swiglu", status)
    return out
