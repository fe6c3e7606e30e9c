"""Greedy decode of a Qwen3SparseKernelForCausalLM, one HIP graph replay per generated token.

The eager decode step (Hugging Face's ``Qwen3ForCausalLM.forward`` with
:class:`~sparseattentioninfer_amd.qwen3.modeling_sparse_qwen3.Qwen3SparseKernelAttention`)
spends most of its time launching about twenty small kernels per layer from
Python.  :class:`GraphDecoder` runs the same per-layer computation -- input
RMSNorm, q/k/v projections, q/k RMSNorm, rotary embedding, paged K/V write,
the paged sparse decode kernel, output projection, residuals, post-attention
RMSNorm, SwiGLU MLP, final norm, LM head, greedy argmax -- on the model's own
modules, captures it once with ``torch.cuda.CUDAGraph`` (a hipGraph on ROCm)
and replays it for every token.

Everything that changes from token to token lives on the device, so one
capture serves every step: the position, the token ids, ``kv_lens``, the page
and slot of the paged write, and each layer's decode block selection.  The
selection of a step is whatever the layer's own pattern and the backend's
schedule give for that step's key length (``pattern.build`` at ``T_k = pos + 1``,
exactly as the eager path does per step).  BigBird selections change only at
page boundaries (the reference's decode row ``qb = (T_k - 1) // bs``,
``sparse_attentions/patterns/bigbird_pattern.py:236,246``), but a local window
whose length is not a multiple of the page moves inside a page, and keep-ratio
layouts take their budget from ``T_k``.  So the decoder builds the selection of
every position the run can reach, keeps the distinct combinations of all
layers' selections in one table, and a step gathers its row through a
per-position index on the device.

With ``fused=True`` (the default) a layer is eight launches: one GEMM for the
concatenated q|k|v projection (``sa_gemm_skinny``, which streams the weights
once for the batch's few rows), ``sa_qk_rope_kv`` (q/k RMSNorm, rotary
embedding, paged K/V write), the paged decode kernel, the output GEMM,
``sa_rmsnorm`` (residual add + post-attention norm), one GEMM for the gate and
up projections with the SwiGLU in its epilogue (``sa_gemm_skinny_swiglu``, on
the weights interleaved once), the down GEMM and ``sa_rmsnorm`` (residual add +
the next layer's input norm).  ``fused=False`` calls the model's
own modules instead (Hugging Face's arithmetic op by op, about 66 launches per
layer).

The graph holds no ``hipMemsetAsync`` node: the argmax over the vocabulary is
taken in two small stages, so no multi-block reduction needs a zeroed
semaphore.
"""
from __future__ import annotations

import torch
from transformers.models.qwen3.modeling_qwen3 import apply_rotary_pos_emb

from .. import ops
from .paged_cache import PagedKVCache


def _argmax_rows(x: torch.Tensor, chunk: int) -> torch.Tensor:
    """Row-wise argmax of ``x [B, V]`` as two single-block reductions (V % chunk == 0)."""
    B, V = x.shape
    v1, i1 = x.view(B, V // chunk, chunk).max(dim=2)        # [B, V / chunk]
    _, i2 = v1.max(dim=1)                                    # [B]
    return i2 * chunk + i1.gather(1, i2[:, None])[:, 0]


def _argmax_chunk(V: int) -> int:
    for c in (128, 256, 64, 512, 32, 1024, 16):
        if V % c == 0:
            return c
    return 0


class _LayerSchedule:
    """Decode block selections of one layer for every position ``pos0 .. pos1 - 1``.

    ``table [n_rows, R, width]`` / ``counts [n_rows, R]`` hold the distinct selections in
    order of first use and ``row_of[p - pos0]`` the row of position ``p``.  A schedule the
    pattern returns again as the same tensors (its cache) is not read again; a new one is
    compared with the previous row, so runs of equal selections share one row.
    """

    def __init__(self, attn, store, pos0: int, pos1: int, batch: int, device):
        page, H, D = store.page, attn.num_heads, attn.head_dim
        backend = attn.sparse_backend
        rows, counts, row_of = [], [], []
        last_src = None        # (pairs, offsets) of the previous position, kept alive for the identity test
        q_like = torch.empty(batch, H, 1, 0, device=device)
        for pos in range(pos0, pos1):
            T_k = pos + 1
            k_like = torch.empty(batch, attn.num_key_value_heads, T_k, 0, device=device)
            pattern = attn.sparse_pattern.build(q_like, k_like, causal=True)
            pairs, offsets, bs = backend._schedule(1, T_k, attn.num_key_value_heads, device, pattern)
            if last_src is not None and pairs is last_src[0] and offsets is last_src[1]:
                row_of.append(len(rows) - 1)
                continue
            last_src = (pairs, offsets)
            if bs != page:
                raise ValueError(f"layer {attn.layer_idx}: schedule block {bs} differs from the page {page}")
            if offsets.size(1) != 2:
                raise ValueError(f"layer {attn.layer_idx}: decode expects one CSR query block")
            start = offsets[:, 0].long()
            cnt = (offsets[:, 1] - offsets[:, 0]).long()
            # each row's entries from its own start, zero-padded to the row width
            width = max(1, int(cnt.max().item()))
            idx = start[:, None] + torch.arange(width, device=pairs.device)[None, :]
            ok = torch.arange(width, device=pairs.device)[None, :] < cnt[:, None]
            row = torch.where(ok, pairs.gather(1, idx.clamp(max=pairs.size(1) - 1)), torch.zeros_like(idx))
            row, cnt = row.to(torch.int32), cnt.to(torch.int32)
            if rows and rows[-1].shape == row.shape and torch.equal(rows[-1], row) and torch.equal(counts[-1], cnt):
                row_of.append(len(rows) - 1)
                continue
            rows.append(row)
            counts.append(cnt)
            row_of.append(len(rows) - 1)
        R = rows[0].size(0)
        self.width = max(r.size(1) for r in rows)
        self.table = torch.zeros(len(rows), R, self.width, dtype=torch.int32, device=device)
        for i, r in enumerate(rows):
            self.table[i, :, :r.size(1)] = r
        self.counts = torch.stack(counts).to(device)              # [n_rows, R]
        self.row_of = row_of
        self.sel = self.sel_off = None  # views of the decoder's gathered selections (set by the decoder)
        self.rows = R
        self.num_splits = ops.auto_decode_splits(batch, R, self.width)
        need = ops.decode_workspace_bytes(batch, H, D, self.num_splits)
        self.workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=device)


class GraphDecoder:
    """Greedy decode steps of ``model`` as replays of one captured HIP graph.

    ``cache`` is the :class:`PagedKVCache` the prompt forward filled, ``ids``
    the ``[B]`` tokens chosen from the prompt (the next inputs) and ``max_len``
    the longest sequence the run reaches (the stores' pages are taken up to it
    once, before capture).  Each :meth:`step` decodes one token per sequence and
    returns the ``[B]`` device tensor of the chosen next tokens (overwritten by
    the following step).  The first ``warmup`` steps run eagerly (they warm the
    libraries the capture records); the next one captures the graph and replays
    it, and every later one replays it.
    """

    def __init__(self, model, cache: PagedKVCache, ids: torch.Tensor, max_len: int, *, warmup: int = 2,
                 keep_logits: bool = False, fused: bool = True):
        self.model = model
        inner = model.model
        cfg = model.config
        self.layers = list(inner.layers)
        self.stores = [cache.layers[i].store for i in range(len(self.layers))]
        if any(s is None for s in self.stores):
            raise ValueError("GraphDecoder needs a PagedKVCache filled by a prompt forward")
        st0 = self.stores[0]
        self.B, self.page, self.dev = st0.batch, st0.page, ids.device
        self.start = st0.seq_len()
        if max_len > st0.max_blocks * self.page:
            raise ValueError(f"max_len {max_len} exceeds the cache capacity {st0.max_blocks * self.page}")
        self.max_len = max_len
        for s in self.stores:
            s._grow_all(max_len)
        self.head_dim = cfg.head_dim
        V = cfg.vocab_size
        self.chunk = _argmax_chunk(V)
        if not self.chunk:
            raise ValueError(f"vocab {V} has no power-of-two chunk for the two-stage argmax")
        for layer in self.layers:
            if not hasattr(layer.self_attn.sparse_backend, "forward_paged"):
                raise ValueError("GraphDecoder needs a backend with paged decode (hip_block_sparse)")
        # one selection table per distinct pattern (dense causal layers all share one)
        sched: dict = {}
        self.sched = []
        for layer, store in zip(self.layers, self.stores):
            attn = layer.self_attn
            key = "dense" if attn.pattern_name == "dense" else id(attn.sparse_pattern)
            if key not in sched:
                sched[key] = _LayerSchedule(attn, store, self.start, max_len, self.B, self.dev)
            self.sched.append(sched[key])
        self.uniq_sched = list(sched.values())
        self._merge_selections()
        # device state
        self.ids = ids.reshape(self.B).to(torch.long).clone()
        self.pos = torch.full((1,), self.start, dtype=torch.long, device=self.dev)
        self.graph = None
        self.warmup = warmup
        self.steps_done = 0
        # last step's LM-head output [B, V] (tests); None unless keep_logits
        self.logits = torch.empty(self.B, V, dtype=model.lm_head.weight.dtype, device=self.dev) \
            if keep_logits else None
        self.fused = fused
        if fused:
            self._init_fused(cfg)

    @property
    def position(self) -> int:
        """Position of the next token to decode (host view)."""
        return self.start + self.steps_done

    @torch.inference_mode()
    def _init_fused(self, cfg) -> None:
        m = self.model.model
        if getattr(m.rotary_emb, "attention_scaling", 1.0) != 1.0:
            raise ValueError("fused decode supports the default rotary embedding (attention_scaling 1)")
        if self.head_dim != 128:
            raise ValueError("fused decode supports head dim 128")
        B, dev = self.B, self.dev
        dt = self.model.lm_head.weight.dtype
        attn0 = self.layers[0].self_attn
        self.num_heads = attn0.num_heads
        self.eps = float(cfg.rms_norm_eps)
        self.inv_freq = m.rotary_emb.inv_freq.to(device=dev, dtype=torch.float32).contiguous()
        self.w_qkv, self.w_gu = [], []
        for layer in self.layers:
            a, mlp = layer.self_attn, layer.mlp
            self.w_qkv.append(torch.cat([a.q_proj.weight, a.k_proj.weight, a.v_proj.weight], 0).contiguous())
            self.w_gu.append(ops.interleave_gate_up(mlp.gate_proj.weight, mlp.up_proj.weight))
        hidden = cfg.hidden_size
        H, D = self.num_heads, self.head_dim
        new = lambda *shape: torch.empty(*shape, dtype=dt, device=dev)  # noqa: E731
        self.h = new(B, hidden)                      # residual stream
        self.x = new(B, hidden)                      # normed activations
        self.a = new(B, hidden)                      # attention / MLP output before the residual add
        self.qkv = new(B, self.w_qkv[0].size(0))
        self.q = new(B, H, D)
        self.att = new(B, H, D)
        self.mid = new(B, self.w_gu[0].size(0) // 2)
        inter = self.mid.size(1)
        self.down_skinny = inter % 8 == 0 and inter <= 10240  # sa_gemm_skinny's K limit
        self.lg = new(B, cfg.vocab_size)
        self.kv_lens = torch.zeros(B, dtype=torch.int32, device=dev)   # shared by every layer's decode

    @torch.inference_mode()
    def _step_fused(self) -> None:
        m = self.model.model
        L = len(self.layers)
        self.h.copy_(m.embed_tokens(self.ids))
        ops.rmsnorm(self.h, self.layers[0].input_layernorm.weight, self.eps, out=self.x)
        self.kv_lens.copy_((self.pos + 1).to(torch.int32).expand(self.B))
        self._select()
        B = self.B
        # Every projection on the skinny GEMM (the down projection on hipBLASLt when its K, the
        # intermediate size, is past the skinny kernel's limit).
        for i, (layer, store, sched) in enumerate(zip(self.layers, self.stores, self.sched)):
            attn = layer.self_attn
            ops.gemm_skinny(self.x, self.w_qkv[i], out=self.qkv)
            ops.qk_rope_kv(self.qkv, attn.q_norm.weight, attn.k_norm.weight, self.inv_freq, self.pos, store, self.q,
                           num_heads=self.num_heads, eps=self.eps)
            ops.paged_sparse_decode(
                self.q, store.k_pages, store.v_pages, store.block_table, self.kv_lens,
                sched.sel.expand(B, sched.rows, sched.width), sched.sel_off.expand(B, sched.rows, 2),
                num_splits=sched.num_splits, workspace=sched.workspace if sched.num_splits > 1 else None,
                out=self.att)
            ops.gemm_skinny(self.att.view(B, -1), attn.o_proj.weight, out=self.a)
            ops.rmsnorm(self.a, layer.post_attention_layernorm.weight, self.eps, residual=self.h, out=self.x)
            ops.gemm_skinny_swiglu(self.x, self.w_gu[i], out=self.mid)
            if self.down_skinny:
                ops.gemm_skinny(self.mid, layer.mlp.down_proj.weight, out=self.a)
            else:
                torch.mm(self.mid, layer.mlp.down_proj.weight.t(), out=self.a)
            nxt = self.layers[i + 1].input_layernorm.weight if i + 1 < L else m.norm.weight
            ops.rmsnorm(self.a, nxt, self.eps, residual=self.h, out=self.x)
        ops.gemm_skinny(self.x, self.model.lm_head.weight, out=self.lg)
        if self.logits is not None:
            self.logits.copy_(self.lg)
        self.ids.copy_(_argmax_rows(self.lg, self.chunk))
        self.pos.add_(1)

    def _merge_selections(self) -> None:
        """Stacks the distinct combinations of every schedule's selection (one per position the run
        reaches, deduplicated) into one table, so that a step gathers the selections of all layers
        with three launches (position -> combination, then the two tables); each schedule's
        ``sel`` / ``sel_off`` become views of the gathered buffers (the decode kernel takes their
        row strides)."""
        S = len(self.uniq_sched)
        R = max(s.rows for s in self.uniq_sched)
        W = max(s.width for s in self.uniq_sched)
        combos: dict = {}
        combo_of = []
        for p in range(self.max_len - self.start):
            key = tuple(s.row_of[p] for s in self.uniq_sched)
            combo_of.append(combos.setdefault(key, len(combos)))
        self.combo_of = torch.tensor(combo_of, dtype=torch.long, device=self.dev)   # [positions]
        self.sel_table = torch.zeros(len(combos), S, R, W, dtype=torch.int32, device=self.dev)
        self.off_table = torch.zeros(len(combos), S, R, 2, dtype=torch.int32, device=self.dev)
        for key, c in combos.items():
            for i, (s, row) in enumerate(zip(self.uniq_sched, key)):
                self.sel_table[c, i, :s.rows, :s.width] = s.table[row]
                self.off_table[c, i, :s.rows, 1] = s.counts[row]
        self.sel_all = torch.zeros(1, S, R, W, dtype=torch.int32, device=self.dev)
        self.off_all = torch.zeros(1, S, R, 2, dtype=torch.int32, device=self.dev)
        for i, s in enumerate(self.uniq_sched):
            s.sel = self.sel_all[:, i, :s.rows, :s.width]
            s.sel_off = self.off_all[:, i, :s.rows, :]

    def _select(self) -> None:
        """Gathers every layer's selection for the current device position."""
        combo = torch.index_select(self.combo_of, 0, self.pos - self.start)
        torch.index_select(self.sel_table, 0, combo, out=self.sel_all)
        torch.index_select(self.off_table, 0, combo, out=self.off_all)

    def _step(self) -> None:
        if self.fused:
            self._step_fused()
        else:
            self._step_modules()

    @torch.inference_mode()
    def _step_modules(self) -> None:
        m = self.model.model
        B, D, page = self.B, self.head_dim, self.page
        h = m.embed_tokens(self.ids[:, None])                                   # [B, 1, hidden]
        cos, sin = m.rotary_emb(h, self.pos.view(1, 1))
        blk = torch.div(self.pos, page, rounding_mode="floor")                  # [1]
        slot = (self.pos % page).expand(B)                                      # [B]
        kv_len = (self.pos + 1).to(torch.int32).expand(B)
        self._select()
        for layer, store, sched in zip(self.layers, self.stores, self.sched):
            attn = layer.self_attn
            res = h
            x = layer.input_layernorm(h)
            shape = (B, 1, -1, D)
            q = attn.q_norm(attn.q_proj(x).view(shape)).transpose(1, 2)
            k = attn.k_norm(attn.k_proj(x).view(shape)).transpose(1, 2)
            v = attn.v_proj(x).view(shape).transpose(1, 2)
            q, k = apply_rotary_pos_emb(q, k, cos, sin)
            pg = store.block_table.index_select(1, blk).view(B).long()
            store.k_pages[pg, :, slot] = k[:, :, 0].to(store.k_pages.dtype)
            store.v_pages[pg, :, slot] = v[:, :, 0].to(store.v_pages.dtype)
            store.kv_lens.copy_(kv_len)
            out = ops.paged_sparse_decode(
                q.reshape(B, attn.num_heads, D).contiguous(), store.k_pages, store.v_pages, store.block_table,
                store.kv_lens, sched.sel.expand(B, sched.rows, sched.width), sched.sel_off.expand(B, sched.rows, 2),
                num_splits=sched.num_splits, workspace=sched.workspace if sched.num_splits > 1 else None)
            h = res + attn.o_proj(out.reshape(B, 1, -1))
            res = h
            h = res + layer.mlp(layer.post_attention_layernorm(h))
        h = m.norm(h)
        logits = self.model.lm_head(h[:, -1])                                   # [B, V]
        if self.logits is not None:
            self.logits.copy_(logits)
        self.ids.copy_(_argmax_rows(logits, self.chunk))
        self.pos.add_(1)

    def step(self) -> torch.Tensor:
        """Decodes one token per sequence; returns the chosen next tokens."""
        if self.position >= self.max_len:
            raise RuntimeError(f"GraphDecoder reached max_len {self.max_len}")
        if self.steps_done < self.warmup:
            self._step()
        else:
            if self.graph is None:
                torch.cuda.synchronize(self.dev)
                self.graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(self.graph):
                    self._step()       # recorded, not run
            self.graph.replay()
        self.steps_done += 1
        return self.ids

    def finish(self) -> None:
        """Brings the stores' lengths up to date (graph replays advance only the device state)."""
        n = self.position
        for s in self.stores:
            s.lens = [n] * s.batch
            s.kv_lens.fill_(n)
