/*
 * sparse_attn.h -- C ABI of the gfx950 block-sparse attention library
 * (libsparse_attn_hip.so).
 *
 * Plain pointers, sizes and element strides only: no torch or C++ types cross
 * this boundary.  Every entry point returns 0 on success, a negative SA_E*
 * code for a rejected argument, or a positive hipError_t from the runtime;
 * sa_last_error() then describes the failure (thread-local, valid until the
 * next call on the same thread).  Nothing here allocates device memory or
 * synchronises: kernels are enqueued on the given stream (a hipStream_t,
 * NULL = the default stream), and any scratch space is passed in by the
 * caller.
 *
 * Tensor conventions (all strides in elements, innermost head dim contiguous):
 *   q  [B, Hq,  T_q, D]      o [B, Hq, T_q, D]
 *   k  [B, Hkv, T_k, D]      v [B, Hkv, T_k, D]      Hq % Hkv == 0
 * Query head h reads KV head h / (Hq / Hkv), the head mapping of Hugging Face
 * repeat_kv that the reference's Qwen3 integration applies before its kernel
 * (sparse_llm/qwen3/integrations/modeling_sparse_qwen3.py:233-234).
 *
 * CSR schedule (sparse_attentions/patterns/base.py:26-33): for CSR row r and
 * query block qb the retained key blocks are
 *   pairs[r * pairs_stride + offsets[r * offsets_stride + qb] ...
 *         pairs[r * pairs_stride + offsets[r * offsets_stride + qb + 1] - 1]
 * There is one row per query head (csr_rows == Hq, the reference's layout) or
 * one row per KV group shared by its Hq/Hkv query heads (csr_rows == Hkv).
 */
#ifndef SPARSE_ATTN_H
#define SPARSE_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SA_ABI_VERSION 6

/* element types */
#define SA_DTYPE_BF16 0
#define SA_DTYPE_F16 1

/* argument error codes (negative) */
#define SA_E_DTYPE (-1)      /* unsupported element type */
#define SA_E_SHAPE (-2)      /* inconsistent or unsupported sizes */
#define SA_E_HEADDIM (-3)    /* head dim not supported by the kernels */
#define SA_E_BLOCK (-4)      /* unsupported block size */
#define SA_E_CSR (-5)        /* csr_rows not Hq or Hkv */
#define SA_E_NULL (-6)       /* required pointer is NULL */
#define SA_E_WORKSPACE (-7)  /* workspace missing or too small */
#define SA_E_ALIGN (-8)      /* pointer or stride breaks 16-byte vector access */

/* Version of this ABI; a loader refuses a library whose value differs. */
int sa_abi_version(void);

/* Description of the last failure on the calling thread ("" if none). */
const char* sa_last_error(void);

/*
 * Block-sparse causal attention over a CSR block schedule (prefill, and any
 * T_q >= 1).  Replaces kernels/triton/universal_sparse_attn.py:165-238
 * (universal_sparse_attn) and its kernel :45-160.
 *
 * Query row t sits at absolute position q_offset + t and sees key j iff the
 * key block of j is retained for its query block, j <= q_offset + t and
 * j < T_k.  q_offset = T_k - T_q reproduces the reference for T_q == T_k and
 * T_q == 1 (universal_sparse_attn.py:203-205).  A row that sees no key is 0.
 * Per row: out = sum_j softmax(q.k_j * sm_scale) v_j with fp32 accumulation;
 * probabilities are rounded to the element type before the PV product, as in
 * the reference kernel (:147).
 *
 * block_size: 64 or 128 (the CSR granularity; the kernel tiles by 64), or 16
 * or 32 with a tile schedule: pairs/offsets then list the 64-key tiles of
 * each 64-row query tile (as sa_csr_to_tiles writes them) and tile_masks,
 * laid out like pairs with row stride tile_masks_stride, holds each entry's
 * retained block_size x block_size sub-blocks: bit sr * (64 / block_size) + sc
 * for query sub-block sr and key sub-block sc of the tile.  tile_masks must be
 * NULL for block sizes 64 and 128.
 * head_dim D: 64 or 128.  nqb = number of CSR query blocks (offsets has
 * nqb + 1 entries per row), nqb == ceil(T_q / max(block_size, 64)).
 *
 * workspace (optional, sa_prefill_workspace_bytes() bytes, 4-byte aligned):
 * with it the kernel runs one persistent workgroup per resident slot that
 * claims work items from counters in the workspace.  It must be zeroed before
 * its first use; every completed launch leaves its counters zeroed again.
 * Launches that may run concurrently (other streams, graph replays on other
 * streams) must not share one workspace: keep one per stream.  Word 3 of the
 * workspace is a status word that launches only set and the caller clears:
 * bit 0 means a launch processed fewer work items than it has (its counters
 * were not zero at launch, or an overlapping launch shared them) and left the
 * skipped items' outputs unwritten.  NULL launches one workgroup per work
 * item instead.
 */
int sa_prefill(int dtype,
               const void* q, int64_t q_sb, int64_t q_sh, int64_t q_st,
               const void* k, int64_t k_sb, int64_t k_sh, int64_t k_st,
               const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st,
               void* o, int64_t o_sb, int64_t o_sh, int64_t o_st,
               const int32_t* pairs, int64_t pairs_stride,
               const int32_t* offsets, int64_t offsets_stride,
               const int32_t* tile_masks, int64_t tile_masks_stride,
               int csr_rows, int nqb,
               int B, int Hq, int Hkv, int T_q, int T_k, int D,
               int block_size, int q_offset, float sm_scale,
               void* workspace, int64_t workspace_bytes,
               void* stream);

/* Bytes of the optional sa_prefill workspace (counters and the status word). */
int64_t sa_prefill_workspace_bytes(void);

/*
 * Regroups a CSR schedule of block size 16 or 32 -- the granularity of the
 * reference's BigBird layouts, whose CSR block is the next power of two of at
 * least 16 (sparse_attentions/patterns/bigbird_pattern.py:99-101, :233) --
 * into the tile schedule that
 * sa_prefill takes for those block sizes.  One output row per input row.
 * Query tile qt holds query blocks s*qt .. s*qt + s - 1 (s = 64 / block_size);
 * its entries, ascending, are the key tiles kt = kb / s holding a retained
 * block kb of any of those query blocks, each with its sub-block mask.
 * Outputs: tile_pairs and tile_masks [rows, width] (row stride tile_stride,
 * zero padded), tile_offsets [rows, ceil(nqb / s) + 1] (row stride
 * tile_offsets_stride).  The ids of each query block must ascend, as the
 * reference's CSR promises (sparse_attentions/patterns/base.py:48); negative
 * ids are dropped.  *status, a device int the caller zeroes, receives bit 0
 * if a row needed more than width tiles (never for a well-formed CSR: a row
 * has no more tiles than entries, so the input's pairs width suffices) and
 * bit 1 if some query block's ids did not ascend; either makes the schedule
 * unusable.  Nothing is synchronised: read *status after the stream.
 */
/*
 * Block mask -> CSR on the GPU: the reference's build_block_pairs_from_mask
 * (sparse_attentions/patterns/base.py:36-89) applied to a block mask, without
 * the host round trips of its per-row loop.  mask [rows, nqb, nkb], one byte
 * per block (nonzero = retained), byte strides mask_row_stride and
 * mask_qb_stride, key blocks contiguous.  Writes offsets [rows, nqb + 1]
 * (row stride offsets_stride) and nnz [rows] (retained blocks per row).  With
 * pairs == NULL this is the count pass; with pairs [rows, width] (row stride
 * pairs_stride) it is the write pass: it reads the offsets the count pass
 * wrote, writes the ascending key blocks of every query block and zero-pads
 * each row to width.  The reference's width is max(1, max nnz), known after
 * the count pass.  *status (a device int the caller zeroes) receives 1 if a
 * row holds more than width blocks.  Each mask row is read by one wave with
 * consecutive lanes on consecutive bytes.
 */
int sa_block_mask_to_csr(const uint8_t* mask, int64_t mask_row_stride, int64_t mask_qb_stride,
                         int rows, int nqb, int nkb,
                         int32_t* offsets, int64_t offsets_stride, int32_t* nnz,
                         int32_t* pairs, int64_t pairs_stride, int64_t width,
                         int* status, void* stream);

/*
 * Block-mask generators (byte masks as sa_block_mask_to_csr reads them, 1 =
 * retained).  mask [rows, nqb, mask_qb_stride] with mask_qb_stride and
 * mask_row_stride multiples of 16 and at least nkb (resp. nqb *
 * mask_qb_stride); bytes past nkb are written 0.  Query block i sits at
 * absolute block q_block_offset + i.  No host round trip, nothing
 * synchronised.
 *
 * sa_bigbird_block_mask: the reference's BigBird rows (bigbird_pattern.py:23-41
 * random pick, :246-255 row sets) with layout[3*row .. 3*row+2] = (global,
 * sliding, random) per row (device int32), hash head head_base + row,
 * num_blocks hash_blocks in the hash; dense_last_block != 0 keeps every block
 * of the last query block (BigBird2Pattern).  Replaces the per-row Python loops
 * of BigBirdPattern._get_block_pairs / BigBirdKeepRatioPattern
 * (bigbird_pattern.py:212-335, :533-634).
 *
 * sa_seeded_bigbird_block_mask / sa_bernoulli_block_mask: this build's seeded
 * benchmark generators (no counterpart in the reference, whose "random" blocks
 * are a hash) on Philox4x64-10: the draw of block kb of query block qa (causal
 * limit min(q_block_offset + i, nkb - 1)) in row `row` is the first word of
 * philox(counter = (kb, qa, row, 0), key = (seed, 1 for BigBird, 2 for
 * Bernoulli)).  Bernoulli keeps kb < qa iff (draw >> 11) < floor(density *
 * 2^53), and the diagonal.  Seeded BigBird keeps the global prefix, the window
 * (trailing {qa-window+1..qa}, or centred {qa-window/2..qa+window/2} when
 * centred != 0) and the diagonal, causal-truncated, plus the
 * random_counts[row] (device int32) eligible blocks with the smallest
 * (draw, kb).
 */
int sa_bigbird_block_mask(uint8_t* mask, int64_t mask_row_stride, int64_t mask_qb_stride, int rows, int nqb,
                          int nkb, int q_block_offset, const int32_t* layout, int head_base, int hash_blocks,
                          int dense_last_block, void* stream);
int sa_seeded_bigbird_block_mask(uint8_t* mask, int64_t mask_row_stride, int64_t mask_qb_stride, int rows,
                                 int nqb, int nkb, int q_block_offset, int window, int global_blocks, int centred,
                                 const int32_t* random_counts, uint64_t seed, void* stream);
int sa_bernoulli_block_mask(uint8_t* mask, int64_t mask_row_stride, int64_t mask_qb_stride, int rows, int nqb,
                            int nkb, int q_block_offset, double density, uint64_t seed, void* stream);

int sa_csr_to_tiles(const int32_t* pairs, int64_t pairs_stride,
                    const int32_t* offsets, int64_t offsets_stride,
                    int rows, int nqb, int block_size,
                    int32_t* tile_pairs, int32_t* tile_masks, int64_t tile_stride, int64_t width,
                    int32_t* tile_offsets, int64_t tile_offsets_stride,
                    int* status, void* stream);

/*
 * Sparse decode: one new query token per sequence against a KV cache, reading
 * only the retained KV blocks.  Replaces the T_q == 1 use of the reference
 * kernel (universal_sparse_attn.py:203-205 via triton_universal_backend.py:47-66)
 * with a memory-bound kernel; adds a paged cache (the reference has none).
 *
 * q [B, Hq, D] (strides q_sb, q_sh); o likewise.
 * KV addressing of (sequence b, KV head g, token t of logical block lb):
 *   paged      (block_table != NULL): base + block_table[b*bt_stride + lb]*kv_sb
 *                                      + g*kv_sh + (t % page)*kv_st
 *   contiguous (block_table == NULL): base + b*kv_sb + g*kv_sh + t*kv_st
 * where t = lb*page + i.  K and V share strides.  kv_lens[b] (or kv_len for
 * every sequence when kv_lens == NULL) is the number of valid tokens.  A paged
 * block_table has max_blocks columns (row stride bt_stride >= max_blocks) over
 * pools of num_pages pages: a retained block at or past max_blocks, or whose
 * page lies outside [0, num_pages), is skipped (it contributes no keys), so a
 * kv_len beyond the table or a corrupt page id is never read out of bounds.
 *
 * Retained blocks of (b, row): sel[b*sel_sb + row*sel_sr + i] for
 * i in [sel_off[b*off_sb + row*off_sr], sel_off[b*off_sb + row*off_sr + 1]);
 * sel_sb / off_sb may be 0 to share one schedule across the batch (the
 * reference's CSR has no batch axis).  sel_rows is Hq or Hkv.
 *
 * page is the block size of both the cache pages and the schedule (16..128,
 * a multiple of 16).  num_splits >= 1 splits each (b, row) list across
 * workgroups; num_splits > 1 needs a workspace of
 * sa_decode_workspace_bytes(B, Hq, D, num_splits) bytes (fp32 partials).
 */
int sa_decode(int dtype,
              const void* q, int64_t q_sb, int64_t q_sh,
              const void* k, const void* v,
              int64_t kv_sb, int64_t kv_sh, int64_t kv_st,
              const int32_t* block_table, int64_t bt_stride, int max_blocks, int num_pages,
              const int32_t* kv_lens, int kv_len,
              const int32_t* sel, int64_t sel_sb, int64_t sel_sr,
              const int32_t* sel_off, int64_t off_sb, int64_t off_sr,
              int sel_rows,
              void* o, int64_t o_sb, int64_t o_sh,
              int B, int Hq, int Hkv, int D, int page, float sm_scale,
              int num_splits, void* workspace, int64_t workspace_bytes,
              void* stream);

/* Bytes of fp32 workspace sa_decode needs for num_splits > 1 (0 otherwise). */
int64_t sa_decode_workspace_bytes(int B, int Hq, int D, int num_splits);

/*
 * sa_decode without a workspace argument: no counterpart in the reference.  For
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  The split partials
 * (num_splits > 1) live in a file-scope device array of
 * sa_decode_noalloc_scratch_bytes() = 16 MiB that each GPU holds until the
 * process ends; sizes needing more are refused with SA_E_WORKSPACE.  It calls
 * no hipMalloc, hipFree or allocating routine (the array's device address is
 * looked up once per device on the first call).  Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (other streams, other
 * threads) race, so serialise them.  Same results, bit for bit, as sa_decode.
 */
int sa_decode_noalloc(int dtype,
                      const void* q, int64_t q_sb, int64_t q_sh,
                      const void* k, const void* v,
                      int64_t kv_sb, int64_t kv_sh, int64_t kv_st,
                      const int32_t* block_table, int64_t bt_stride, int max_blocks, int num_pages,
                      const int32_t* kv_lens, int kv_len,
                      const int32_t* sel, int64_t sel_sb, int64_t sel_sr,
                      const int32_t* sel_off, int64_t off_sb, int64_t off_sr,
                      int sel_rows,
                      void* o, int64_t o_sb, int64_t o_sh,
                      int B, int Hq, int Hkv, int D, int page, float sm_scale,
                      int num_splits, void* stream);

/* Bytes of the scratch array sa_decode_noalloc holds per GPU. */
int64_t sa_decode_noalloc_scratch_bytes(void);

/*
 * Measurement aid, no counterpart in the reference: reads `bytes` (a multiple
 * of 16) at src once with 16-byte non-temporal loads from
 * sa_stream_read_workgroups() workgroups (8 per CU), each reading one
 * contiguous chunk, and writes one xor-folded word per workgroup to sink (that
 * many uint32).  Its rate is the HBM streaming-read ceiling that the
 * memory-bound decode kernel is compared with.
 */
int sa_stream_read(const void* src, int64_t bytes, uint32_t* sink, void* stream);
int sa_stream_read_workgroups(void);

/*
 * Measurement aids, no counterpart in the reference: the ceilings the prefill
 * kernel is read against.  sa_mfma_rate launches per_cu (1..8) 4-wave
 * workgroups per CU (so per_cu waves per SIMD); every wave runs `iters` rounds
 * of 4 independent v_mfma_f32_32x32x16_bf16 (32768 FLOP each) on register
 * operands: 4 * iters * 32768 * 4 * per_cu * sa_measure_cus() FLOP per
 * launch (four waves per workgroup); each thread writes one float to sink,
 * so sink_len >= 256 * per_cu * sa_measure_cus().
 * sa_lds_read_rate launches one 8-wave workgroup per CU; every wave reads a
 * 16 KiB LDS tile `iters` times with the prefill kernel's K-fragment read
 * (tr16 = 0: ds_read_b128) or V-fragment read (tr16 = 1: two
 * ds_read_b64_tr_b16): 8 * 16384 * iters bytes per CU and launch; sink_len >=
 * 512 * sa_measure_cus() words.  A shorter sink is refused (SA_E_SHAPE).
 */
int sa_mfma_rate(int per_cu, int iters, float* sink, int64_t sink_len, void* stream);
int sa_lds_read_rate(int tr16, int iters, uint32_t* sink, int64_t sink_len, void* stream);
int sa_measure_cus(void);

/*
 * Measurement aid, no counterpart in the reference: the per-CU rate of the
 * load path that stages the prefill kernel's K/V tiles.  One 8-wave workgroup
 * per CU moves a 16 KiB tile of src (L2-resident: 4 tiles in turn, so
 * src_bytes >= 65536, 16-byte aligned) into LDS with direct loads
 * (global_load_lds_dwordx4), waits and meets at a barrier, `iters` times:
 * 16384 * iters bytes per CU and launch.  sink_len >= 512 * sa_measure_cus()
 * words.
 */
int sa_stage_rate(const void* src, int64_t src_bytes, int iters, uint32_t* sink, int64_t sink_len, void* stream);

/*
 * Measurement aid, no counterpart in the reference: the steady-state step of
 * the prefill loop (one 64-key tile: 2,048 matrix cycles per SIMD of
 * v_mfma 32x32x16-equivalents, its exponentials, the K and V fragment reads
 * from LDS, 32 KiB of direct K/V loads per workgroup from src and one barrier)
 * in one of three wave layouts, one workgroup per CU, `steps` times:
 * layout 0 = 8 waves x 32 query rows (the shipped kernel's layout), 1 = 16
 * waves x 16 rows (v_mfma_f32_16x16x32, four waves per SIMD), 2 = 4 waves x 64
 * rows (one wave per SIMD, O^T in AGPRs).  src: >= 65536 bytes, 16-byte
 * aligned, L2-resident.  sink_len >= sa_step_rate_threads(layout) *
 * sa_measure_cus() floats; the sink values are not meaningful.
 * sa_step_rate_threads returns the workgroup size of a layout, -1 for others.
 */
int sa_step_rate(int layout, const void* src, int64_t src_bytes, int steps, float* sink, int64_t sink_len,
                 void* stream);
int sa_step_rate_threads(int layout);

/*
 * Measurement aid, no counterpart in the reference: sa_prefill (block size 64
 * or 128, so no tile masks) through an instrumented copy of the persistent
 * four-head kernel, which also writes a per-workgroup timeline.  Needs what
 * that kernel needs: a workspace, Hq / csr_rows a multiple of four (four query
 * heads per workgroup) and D = 128; other shapes are refused (SA_E_SHAPE).  The output
 * o is the same as sa_prefill's.  timeline receives, for each workgroup w of the
 * launch, 36 words at timeline[36 * w]: start and end in shader clocks
 * (s_memtime) and in the 100 MHz constant clock (s_memrealtime); then for the
 * first wave of the lower and of the upper 32-row half, 16 words each: the
 * shader clocks spent in the phases of its items (11 from the end of the
 * previous item to the top of the item loop, 0 from there to the item's setup,
 * 1 setup and Q load issue, 2 first tile-queue pops, 3 first K/V load issue,
 * 4 lookahead issue, 5 load wait, 6 barrier, 7 first S^T, 8 tile loop, 9 last
 * tile, 10 epilogue) and counts (12 items, 13 loop steps, 14 row
 * reference refits; 15 the last stamp).  Each stamp costs about 100 shader
 * clocks of its own.  timeline_words >= sa_prefill_timeline_words(dtype), the
 * size for the largest grid on the current device.
 */
int sa_prefill_timeline(int dtype,
                        const void* q, int64_t q_sb, int64_t q_sh, int64_t q_st,
                        const void* k, int64_t k_sb, int64_t k_sh, int64_t k_st,
                        const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st,
                        void* o, int64_t o_sb, int64_t o_sh, int64_t o_st,
                        const int32_t* pairs, int64_t pairs_stride,
                        const int32_t* offsets, int64_t offsets_stride,
                        int csr_rows, int nqb,
                        int B, int Hq, int Hkv, int T_q, int T_k, int D,
                        int block_size, int q_offset, float sm_scale,
                        void* workspace, int64_t workspace_bytes,
                        uint64_t* timeline, int64_t timeline_words,
                        void* stream);
int64_t sa_prefill_timeline_words(int dtype);

/*
 * Fused elementwise stages of one decode step of a Qwen3 decoder layer, for the
 * graph-captured end-to-end decode (callers of the attention path, not the
 * attention itself).  They keep Hugging Face's arithmetic: fp32 inside,
 * rounding to the element type where Hugging Face rounds.
 *
 * sa_rmsnorm replaces Qwen3RMSNorm.forward and the residual add before it
 * (transformers/models/qwen3/modeling_qwen3.py, Qwen3DecoderLayer.forward):
 * for each of `rows` rows of n elements, r = residual + x rounded and stored
 * back into residual when residual is not NULL (else r = x), then
 * out = weight * round(r * rsqrt(mean(r^2) + eps)), rounded.  n a multiple of 8
 * and at most 8192; rows 16-byte aligned.
 */
int sa_rmsnorm(int dtype, const void* x, int64_t x_stride, void* residual, int64_t residual_stride,
               const void* weight, void* out, int64_t out_stride, int rows, int n, float eps, void* stream);

/*
 * q/k RMSNorm, rotary embedding and paged K/V write of one new token per
 * sequence, from the fused projection row qkv[b] = q heads | k heads | v heads
 * (Hq + 2 Hkv heads of D = 128).  Replaces the q_norm / k_norm /
 * apply_rotary_pos_emb / cache update of the reference's attention forward
 * (sparse_llm/qwen3/integrations/modeling_sparse_qwen3.py:207-234).
 * *position (device int64) is the token's position p: cos/sin of
 * inv_freq[i] * p (D/2 fp32 frequencies), rotate_half convention.  Query heads
 * go to q_out[b, h, :]; key and value heads to the pages of logical block
 * p / page (block_table, `max_blocks` columns) at slot p % page of pools
 * holding num_pages pages (strides in elements: page, head, token); a
 * position past the table or a page outside the pool is not written.
 */
int sa_qk_rope_kv(int dtype, const void* qkv, int64_t qkv_stride, const void* q_norm_weight,
                  const void* k_norm_weight, const float* inv_freq, const int64_t* position,
                  void* q_out, int64_t q_out_sb, int64_t q_out_sh,
                  void* k_pages, void* v_pages, int64_t pages_sp, int64_t pages_sh, int64_t pages_st,
                  const int32_t* block_table, int64_t block_table_stride, int max_blocks, int num_pages,
                  int B, int Hq, int Hkv, int D, int page, float eps, void* stream);

/*
 * SwiGLU of Qwen3MLP: out[b, i] = round(round(silu(g)) * u) with g = gate_up[b, i]
 * and u = gate_up[b, I + i] (the gate and up projections fused into one row).
 */
int sa_swiglu(int dtype, const void* gate_up, int64_t gate_up_stride, void* out, int64_t out_stride,
              int B, int I, void* stream);

/*
 * out[m, n] = sum_k x[m, k] * w[n, k] for M <= 8 rows of x (the projections of a
 * decode step: F.linear of Hugging Face's Qwen3 modules with M = batch), fp32
 * accumulation, one rounding of each output.  Streams w once; x rows and w rows
 * 16-byte aligned, K a multiple of 8 and at most 10240.
 */
int sa_gemm_skinny(int dtype, const void* x, int64_t x_stride, const void* w, int64_t w_stride, void* out,
                   int64_t out_stride, int M, int N, int K, void* stream);

/*
 * Qwen3MLP's gate and up projections and its SwiGLU for M <= 8 rows in one launch:
 * w_gate_up holds the 2I gate and up rows interleaved (row 2i = gate row i, row 2i + 1 =
 * up row i), and out[m, i] = round(round(silu(g)) * u) with g and u the bf16-rounded
 * products of the pair -- the bits of sa_gemm_skinny on the concatenated [gate; up] rows
 * followed by sa_swiglu.  K a multiple of 128.
 */
int sa_gemm_skinny_swiglu(int dtype, const void* x, int64_t x_stride, const void* w_gate_up, int64_t w_stride,
                          void* out, int64_t out_stride, int M, int I, int K, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SPARSE_ATTN_H */
