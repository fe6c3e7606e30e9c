// Block-sparse causal attention over a CSR block schedule, gfx950 (CDNA4).
//
// Semantics follow the reference kernel kernels/triton/universal_sparse_attn.py:77-160:
// per query row, an online softmax over the keys of the retained blocks, masked by
// q_abs >= k and k < T_k, fp32 accumulation, probabilities rounded to the element
// type before the PV product, output acc / (l > 0 ? l : 1).
//
// Mapping onto the hardware:
//  * one work item = (batch b, CSR row r, 64-row query tile qt, head split hs); its
//    workgroup has two waves (two 32-row halves) per query head that shares row r, so the
//    Hq/Hkv heads of a KV group share every K/V tile staged in LDS (GQA: K/V are read
//    once per group, not once per head);
//  * per wave and 64-key tile: S^T = K Q^T and O^T = V^T P^T on v_mfma_f32_32x32x16.
//    Computing the transposed products puts one query row in each lane column, so the
//    softmax statistics, the rescale of O and the P operand of the second product all
//    stay in the lane that owns the row;
//  * K/V tiles go from global memory straight into LDS (global_load_lds, no registers)
//    in a swizzled layout whose fragment reads are bank-conflict free; the V^T operand is
//    read with the transposing ds_read_b64_tr_b16, so V is staged row-major as loaded;
//  * four-head workgroups (8 waves, one per SIMD pair) run a software pipeline: the next
//    tile's S^T = K Q^T is issued under the current tile's exponentials, and its row max
//    under the current tile's O^T += V^T P^T; Q is staged in LDS there to leave the
//    registers to the accumulators.  Smaller workgroups run one tile at a time;
//  * the softmax works in base 2 with scale*log2(e) folded into one FMA before the
//    hardware v_exp_f32 (2^x).  Four-head workgroups take each row's reference from its
//    first tile's (masked) max and refit it (raise it to the tile max, rescale O and l)
//    only when a lane's probabilities of one tile sum past 2^16 or overflow; smaller
//    workgroups raise it when a row max exceeds it by more than 2^8.  Either way the
//    common case never touches O with VALU;
//  * the last tile of a four-head item skips the PV half (and the probabilities) of keys
//    32..63 in a wave whose rows all end before them: the lower half on a diagonal tile;
//  * O is written back through LDS so that every global store is a 16-byte piece of a
//    contiguous row;
//  * with a workspace, one persistent workgroup per CU slot claims work items from an
//    atomic counter, heaviest query tiles first.
//
// MFMA 32x32x16 lane layouts used (l = lane, g = l / 32):
//   A (32 x 16): lane l holds row l % 32, k = 8g .. 8g+7
//   B (16 x 32): lane l holds column l % 32, k = 8g .. 8g+7
//   D (32 x 32): lane l, register r holds row 8(r/4) + 4g + r%4, column l % 32
// With K rows permuted by krow, register r = 8h + e of the 32-key half j of S^T holds
// key 32j + 16h + 8g + e.
#include <algorithm>
#include <type_traits>

#include "sa_common.h"

namespace sa {

constexpr int QT = 32;           // query rows per wave
constexpr int QTILE = 64;        // query rows per work item (two waves per query head)
constexpr int KT = 64;           // keys per K/V tile
constexpr int ROW_CACHE = 1024;  // CSR entries of one row cached in LDS
constexpr int N_XCD = 8;         // XCDs of an MI355X; workgroups are dealt to them in turn
constexpr int XCD_CHUNK = 4;     // query tiles per chunk dealt to one XCD
// Largest token stride (elements) of K and V: per-lane offsets within a tile are 32-bit.
constexpr int64_t MAX_KV_STRIDE = (int64_t)1 << 24;

struct PrefillArgs {
  const elem_t* q;
  const elem_t* k;
  const elem_t* v;
  elem_t* o;
  int64_t q_sb, q_sh, q_st;
  int64_t k_sb, k_sh, k_st;
  int64_t v_sb, v_sh, v_st;
  int64_t o_sb, o_sh, o_st;
  const int32_t* pairs;
  int64_t pairs_stride;
  const int32_t* offsets;
  int64_t offsets_stride;
  // Tile schedules of finer blocks (16 or 32): pairs hold 64-key tiles of 64-row query tiles,
  // tile_masks[r * masks_stride + e] the retained sub-blocks of entry e (bit sr * (64 / b) + sc
  // for query sub-block sr, key sub-block sc); sub_log2 = log2(b), 0 without masks.
  const int32_t* tile_masks;
  int64_t masks_stride;
  int sub_log2;
  int R;             // CSR rows
  int heads_per_row; // query heads that read one CSR row
  int head_splits;   // heads_per_row / heads per workgroup
  int B, Hq, Hkv, Tq, Tk;
  int ntq;           // 64-row query tiles
  int qpb_log2;      // log2(block_size / 64): query tiles per CSR block
  int tpb_log2;      // log2(block_size / 64): key tiles per CSR block
  int q_offset;
  float scale_log2;  // sm_scale * log2(e)
  // Persistent mode: the workspace words (WS_* below), zero at launch; every completed launch
  // leaves the counters zero and the status word as it found it, or with WS_SKIPPED set.
  unsigned int* counter;
  // Work-item decoding without integer division: per_tile = R * B * head_splits, and
  // floor((2^32 - 1) / d) for d = per_tile, R, head_splits (see fast_div).
  int per_tile;
  uint32_t mul_tile, mul_R, mul_hs;
  // Persistent launches (row_order) take the query tiles from q_split up latest first with all
  // rows of a tile together, then the tiles below q_split row by row, the CSR rows in
  // descending order of retained blocks (s_row_rank), latest first within a row: the lightest
  // items come last, so workgroups run out of work at nearly the same time, while most of the
  // launch keeps every row's tiles in flight.  head_items = (ntq - q_split) * per_tile;
  // per_group = q_split * bhs items per row below q_split; bhs = B * head_splits.
  int row_order;
  int nqb;
  int q_split, head_items, per_group, bhs;
  uint32_t mul_group, mul_bhs;
  // Timeline launches only (sa_prefill_timeline): TL_WORDS words per workgroup.
  unsigned long long* timeline;
};

// Words of the persistent-launch workspace: the next unclaimed item, the workgroups done, the
// items processed, and a status word that only the host clears.  A launch whose workgroups
// processed fewer items than it has (the counters were not zero at launch, or two launches
// that overlapped in time shared them) sets WS_SKIPPED: the skipped items' outputs are not
// written, so the caller must not use the output.
enum : int { WS_NEXT = 0, WS_DONE_WG = 1, WS_DONE_ITEMS = 2, WS_STATUS = 3, WS_WORDS = 8 };
constexpr unsigned WS_SKIPPED = 1u;

// CSR rows of a persistent launch in descending order of retained blocks (row_order).
constexpr int MAX_ORDERED_ROWS = 256;
__shared__ int s_row_rank[MAX_ORDERED_ROWS];

// Timeline instantiation (TL) of the persistent four-head loop: shader-clock cycles (s_memtime)
// spent in each phase of an item, summed over the workgroup's items, for the first wave of each
// 32-row half; plus counts of items, loop steps and refits.  Each stamp costs about 100 cycles of
// its own, so the instrumented launch runs a little slower than the product's.  Per workgroup
// the record holds TL_WORDS words: start and end in shader clocks and in the 100 MHz constant
// clock (s_memrealtime), then the 16 words of the lower half and the 16 of the upper half.
enum : int {
  TL_GAP = 0,        // top of the item loop to this item's setup (metadata reads)
  TL_SETUP_Q = 1,    // item setup and the Q load issue
  TL_POPS = 2,       // tile queue start and the first two pops
  TL_KV = 3,         // direct loads of the first K/V tiles issued
  TL_LOOK = 4,       // lookahead reads and the next claim issued
  TL_WAIT = 5,       // wait for every load, lookahead committed to LDS
  TL_BARRIER = 6,    // the barrier that publishes the first tiles
  TL_FIRST_QK = 7,   // Q fragments, the first tile's S^T and row max, the second barrier
  TL_LOOP = 8,       // the tile loop (every step but the last tile's)
  TL_LAST = 9,       // the last tile's probabilities and PV
  TL_EPILOGUE = 10,  // normalisation, O staged and stored
  TL_LOOP_TOP = 11,  // end of the previous item (or workgroup start) to the top of the item loop
  TL_ITEMS = 12,     // counts: items,
  TL_STEPS = 13,     // loop steps,
  TL_REFITS = 14,    // refits of the row reference
  TL_NOW = 15,       // (last stamp)
  TL_HALF_WORDS = 16,
  TL_WORDS = 4 + 2 * TL_HALF_WORDS
};
__shared__ unsigned s_tl[2][TL_HALF_WORDS];

// Sum / max of a value over lanes l and l ^ 32, in every lane: one v_permlane32_swap of the
// value with itself puts the lower half's values in one result and the upper half's in the other.
__device__ __forceinline__ float halves_sum(float x) {
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}
__device__ __forceinline__ float halves_max(float x) {
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}

__device__ __forceinline__ __attribute__((address_space(3))) void* lds_ptr(const void* p) {
  return (__attribute__((address_space(3))) void*)(p);
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)lds_ptr(p);
}

// Direct global -> LDS loads of 16 bytes per lane (global_load_lds_dwordx4: lane l's bytes
// land at the LDS address in M0 plus 16 l).  They are issued from assembly so that the
// compiler does not make every later LDS read wait for them (it cannot tell the staging
// buffers apart); callers wait with wait_dma() before the barrier that publishes the data.
// M0 is written one instruction ahead of its use by the load, as the hardware requires.
//
// Uniform base address `sbase` plus a per-lane 32-bit byte offset.
__device__ __forceinline__ void load_lds16(const void* sbase, uint32_t voff, uint32_t lds) {
  asm volatile(
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, %1"
      :
      : "v"(voff), "s"(sbase), "s"(lds)
      : "memory", "m0");
}

// Uniform base plus per-lane offset plus the immediate IMM (a signed 13-bit field of the
// instruction), so consecutive loads from one base need no address arithmetic.  The
// instruction adds IMM to the LDS address as well (M0 + IMM + 16 l), so M0 is lds - IMM.
template <int IMM>
__device__ __forceinline__ void load_lds16_at(const void* sbase, uint32_t voff, uint32_t lds) {
  static_assert(IMM >= -4096 && IMM < 4096, "global instruction offsets are 13-bit signed");
  asm volatile(
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, %1 offset:%3"
      :
      : "v"(voff), "s"(sbase), "s"(lds - (uint32_t)IMM), "i"(IMM)
      : "memory", "m0");
}

// Per-lane 64-bit address.
__device__ __forceinline__ void load_lds16(const void* vaddr, uint32_t lds) {
  asm volatile(
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, off"
      :
      : "v"(vaddr), "s"(lds)
      : "memory", "m0");
}

// Waits for the calling wave's direct loads (and any other vector memory access).
__device__ __forceinline__ void wait_dma() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)

// Wave-uniform 32-bit global read that has completed when it returns (it waits for every
// vector memory access of the wave).  For the rare reads of a CSR row past its LDS cache:
// written as one opaque block, it leaves the compiler no pending load into a register that
// the LDS path reuses, which would otherwise make every LDS read of the row wait for the
// direct loads.
__device__ __forceinline__ int32_t load_uniform_now(const int32_t* p) {
  int32_t x;
  asm volatile(
      "global_load_dword %0, %1, off\n\t"
      "s_waitcnt vmcnt(0)"
      : "=v"(x)
      : "v"(p)
      : "memory");
  return __builtin_amdgcn_readfirstlane(x);
}

// Per-lane 32-bit global read that has completed when it returns (same reason as above).
__device__ __forceinline__ int32_t load_lane_now(const int32_t* p) {
  int32_t x;
  asm volatile(
      "global_load_dword %0, %1, off\n\t"
      "s_waitcnt vmcnt(0)"
      : "=v"(x)
      : "v"(p)
      : "memory");
  return x;
}

// SUB: tile schedules with sub-block masks (block sizes 16 and 32); without it the mask
// bookkeeping compiles away.  TL: the timeline instantiation (stamps compile away without it).
template <bool BF16, int D, int HW, bool SUB, bool TL = false>
struct Prefill {
  using E = Elem<BF16>;
  static constexpr int NW = 2 * HW;              // waves: HW query heads x two 32-row halves
  static constexpr int NT = 64 * NW;             // threads
  static constexpr int NCG = D / 32;             // column groups of a staged tile
  static constexpr int TILE_BYTES = KT * D * 2;  // one staged K or V tile
  static constexpr int NI = TILE_BYTES / 1024;   // 1 KiB wave-wide direct loads per tile
  static constexpr int NIW = NI / NW;            // ... issued by each wave
  static constexpr int WAVE_BYTES = QT * D * 2;  // 32 rows of Q or O (one wave's share)
  // Four-head workgroups run the software-pipelined loop with K double- and V triple-
  // buffered and Q staged in LDS.  Other shapes run one tile at a time over double-buffered
  // K/V (single-buffered for one-head workgroups, so that more of them share a CU).
  static constexpr bool PIPE = HW == 4;
  static constexpr int NBK = PIPE ? 2 : (HW == 1 ? 1 : 2);
  static constexpr int NBV = PIPE ? 3 : NBK;
  static constexpr int LDS_KV = (NBK + NBV) * TILE_BYTES;
  static constexpr int LDS_Q = PIPE ? NW * WAVE_BYTES : 16;
  static constexpr float RESCALE_LOG2 = 8.f;
  // Pipelined loop: the row reference is refit when one lane's probabilities of a tile (32 of a
  // row's keys) sum past this; below it no probability exceeds 2^16, far from fp32 / bf16 overflow.
  static constexpr float REFIT_SUM = 65536.f;
  static_assert(NI % NW == 0, "direct loads must split evenly over the waves");
  static_assert(NW * WAVE_BYTES <= LDS_KV, "the epilogue stages O in the K/V buffers");
  static_assert(!TL || PIPE, "the timeline instruments the persistent four-head loop");

  // TL only: charge the cycles since the last stamp to phase k (lane 0 of the first wave of each half).
  static __device__ __forceinline__ void tl_stamp(int k) {
    if constexpr (TL) {
      const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
      if (wave % HW == 0 && (threadIdx.x & 63) == 0) {
        const unsigned t = (unsigned)__builtin_amdgcn_s_memtime();
        unsigned* p = s_tl[wave / HW];
        p[k] += t - p[TL_NOW];
        p[TL_NOW] = t;
      }
    }
  }
  // TL only: count one event of kind k.
  static __device__ __forceinline__ void tl_count(int k) {
    if constexpr (TL) {
      const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
      if (wave % HW == 0 && (threadIdx.x & 63) == 0) s_tl[wave / HW][k] += 1;
    }
  }

  // LDS row of key k within a staged K tile: bits 2 and 3 swapped.  With this order the S^T
  // accumulator gives each lane half 8 consecutive keys per 16-key chunk, the k-order of the
  // V^T operand.
  static __device__ __forceinline__ int krow(int k) {
    return (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1);
  }

  // ---- staging ------------------------------------------------------------------------
  // Staged tile layout (K and V alike, 64 rows x D, no padding): D/32 column groups of
  // 4 KiB; row r of a group is 64 bytes at r*64 holding 16-byte chunks c = 0..3 (columns
  // 8c..8c+7 of the group) at position c ^ ((r >> 2) & 3).  One wave-wide direct load
  // (global_load_lds, 16 bytes per lane, lane l at base + 16 l) fills 16 rows of one group;
  // the K fragment reads (16 lanes: 16 consecutive rows, one chunk) and the transposing
  // V^T reads (32 lanes: 4 rows x 64 bytes) are both bank-conflict free.
  //
  // Wave w issues the direct loads k = w*NIW .. w*NIW + NIW - 1 of a tile; load k fills
  // column group k % NCG, rows 16 (k / NCG) .. + 15, and its lane l carries row
  // 16 (k / NCG) + l/4, columns 32 (k % NCG) + col(l), col(l) = 8 ((l & 3) ^ ((l >> 4) & 3))
  // ((row >> 2) & 3 == (l >> 4) & 3).  Either a wave's loads share one row block
  // (NIW <= NCG) or they cover whole row blocks (NIW > NCG), so every per-load address
  // difference is a compile-time constant or one uniform multiple of the row stride.
  static_assert(NCG % NIW == 0 || NIW % NCG == 0, "direct loads must tile row blocks evenly");
  static __device__ __forceinline__ int dma_col(int lane) { return 8 * ((lane & 3) ^ ((lane >> 4) & 3)); }

  // Byte offset of this lane's 16 bytes within a direct load of K (rows permuted by krow)
  // and of V, relative to the load's first row and column group; krow(16 rb + x) ==
  // 16 rb + krow(x), so the rest of each load's address is uniform.
  struct DmaLane {
    uint32_t k, v;
    __device__ __forceinline__ DmaLane(const PrefillArgs& a, int lane) {
      k = (uint32_t)((krow(lane >> 2) * a.k_st + dma_col(lane)) * 2);
      v = (uint32_t)(((lane >> 2) * a.v_st + dma_col(lane)) * 2);
    }
  };

  // Fills one staged tile of key tile kt from `base` (token stride st; lane offset off).
  // Rows past T_k read row T_k - 1: their scores are masked and their probabilities are 0.
  template <bool PERMUTE>
  static __device__ __forceinline__ void dma(const elem_t* base, int64_t st, uint32_t off, char* tile, int kt,
                                             int Tk, int wave, int lane) {
    const char* tb = reinterpret_cast<const char*>(base + (int64_t)kt * KT * st);
    const int k0 = wave * NIW;
    const int cg0 = k0 % NCG, rb0 = k0 / NCG;
    if (kt * KT + KT <= Tk) {
      const char* wb = tb + ((int64_t)16 * rb0 * st + 32 * cg0) * 2;  // uniform
      char* wl = tile + cg0 * 4096 + rb0 * 1024;
#pragma unroll
      for (int u = 0; u < NIW; ++u) {
        const int du = NIW <= NCG ? 0 : u / NCG;  // row blocks past rb0
        const int cu = NIW <= NCG ? u : u % NCG;  // column groups past cg0
        load_lds16(wb + (int64_t)32 * du * st + 64 * cu, off, lds_addr(wl + cu * 4096 + du * 1024));
      }
    } else {
      const int last = Tk - 1 - kt * KT;
#pragma unroll
      for (int u = 0; u < NIW; ++u) {
        const int k = k0 + u;
        const int cg = k % NCG, rb = k / NCG;
        const int row = 16 * rb + (lane >> 2);
        const int r = min(PERMUTE ? krow(row) : row, last);
        load_lds16(tb + ((int64_t)r * st + 32 * cg + dma_col(lane)) * 2, lds_addr(tile + cg * 4096 + rb * 1024));
      }
    }
  }

  // ---- fragments ----------------------------------------------------------------------
  // Per-lane byte offsets of the fragment reads (tile-invariant).  The K offset of odd
  // chunk pairs is k0 ^ 32 and the V^T offset of the upper key quad is (v0 + 256) ^ 16.
  struct Frag {
    int k0, v0;
    __device__ __forceinline__ Frag(int lane) {
      const int l32 = lane & 31, g = lane >> 5;
      k0 = l32 * 64 + 16 * (g ^ ((l32 >> 2) & 3));
      const int i = lane & 15, G = lane >> 4;
      const int c4 = 2 * (G & 1) + ((i >> 1) & 1);
      v0 = (8 * g + (i >> 2)) * 64 + 16 * (c4 ^ (2 * g)) + 8 * (i & 1);
    }
  };

  // A operand of S^T = K Q^T: row 32j + l32 of the staged K tile (key krow of it),
  // columns 16cc + 8g .. +7.
  static __device__ __forceinline__ u32x4 kfrag(const char* cK, const Frag& f, int j, int cc) {
    const int off = (cc & 1) ? (f.k0 ^ 32) : f.k0;
    return *reinterpret_cast<const u32x4*>(cK + 4096 * (cc >> 1) + 2048 * j + off);
  }

  static __device__ __forceinline__ u32x2 ds_tr16(const char* p) {
    typedef short v4i16 __attribute__((ext_vector_type(4)));
    const v4i16 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16*)(p));
    return __builtin_bit_cast(u32x2, r);
  }

  // A operand of O^T = V^T P^T: lane l holds d = 32dt + l32 of keys 32j + 16h + 8g + 0..7.
  // ds_read_b64_tr_b16 gives lane i of each 16-lane group element e = the (i & 3)-th value
  // at the address of lane 4e + (i >> 2); each lane addresses key (i >> 2) of a 4-key quad
  // at columns 4(i & 3) of its 16-column group, so lane i receives column i of 4 keys.
  static __device__ __forceinline__ u32x4 vfrag(const char* cV, const Frag& f, int j, int h, int dt) {
    const char* p = cV + 4096 * dt + 2048 * j + 1024 * h;
    const u32x2 lo = ds_tr16(p + f.v0);
    const u32x2 hi = ds_tr16(p + ((f.v0 + 256) ^ 16));
    return u32x4{lo[0], lo[1], hi[0], hi[1]};
  }

  // B operand of S^T = K Q^T from a wave's staged Q, laid out like a staged K/V tile of 32
  // rows: column group cg (32 columns) at cg*2048, row r at r*64, its 16-byte chunk c at
  // position c ^ ((r >> 2) & 3).  Lane l needs row l32, columns 16cc + 8g .. +7 (chunk
  // 2(cc & 1) + g of group cc/2), which is the K fragment offset of the same lane.
  static __device__ __forceinline__ u32x4 qfrag(const char* sQw, const Frag& f, int cc) {
    const int off = (cc & 1) ? (f.k0 ^ 32) : f.k0;
    return *reinterpret_cast<const u32x4*>(sQw + 2048 * (cc >> 1) + off);
  }

  // Direct loads of this wave's 32 rows of Q into that layout: load k fills rows 16(k / NCG) ..
  // +15 of column group k % NCG, lane i row 16(k / NCG) + i/4, columns 32(k % NCG) + dma_col(i)
  // (16 rows x 64 bytes per instruction, as for K and V).  Rows past T_q read row T_q - 1.
  static __device__ __forceinline__ void load_q(const PrefillArgs& a, const elem_t* qh, int row0, char* sQw,
                                                int lane) {
#pragma unroll
    for (int k = 0; k < 2 * NCG; ++k) {
      const int cg = k % NCG, rb = k / NCG;
      const int grow = min(row0 + 16 * rb + (lane >> 2), a.Tq - 1);
      load_lds16(qh + (int64_t)grow * a.q_st + 32 * cg + dma_col(lane), lds_addr(sQw + cg * 2048 + rb * 1024));
    }
  }

  // ---- work items ---------------------------------------------------------------------
  struct Item {
    int g, l32, hf, hq;
    const elem_t* qb;
    const elem_t* kb;
    const elem_t* vb;
    const int32_t* prow;
    const int32_t* mrow;  // tile masks of the row (sub-block schedules)
    int e0, n_tiles, tpb_mask;
    bool cached;
    int q_row0, q_abs_tile_max, q_abs_min;
  };

  // CSR entries of one row cached in LDS.  The persistent four-head loop keeps two rows
  // (this item's and the next one's), so tile schedules, which also cache their masks, hold
  // fewer entries per row there.
  static constexpr int RC = (PIPE && SUB) ? ROW_CACHE / 2 : ROW_CACHE;

  // Work item (qt, r, hs, b) whose CSR row holds entries [e0, e0 + n_ent): pointers and
  // positions only, no memory reads.
  static __device__ __forceinline__ Item setup_base(const PrefillArgs& a, int qt, int r, int hs, int b, int e0,
                                                    int n_ent) {
    Item it;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    it.g = lane >> 5;
    it.l32 = lane & 31;
    const int hw = wave % HW;  // head within the workgroup
    it.hf = wave / HW;         // 32-row half of the query tile
    it.hq = r * a.heads_per_row + hs * HW + hw;
    const int kvh = (r * a.heads_per_row + hs * HW) / (a.Hq / a.Hkv);  // shared by the waves
    it.qb = a.q + b * a.q_sb + it.hq * a.q_sh;
    it.kb = a.k + b * a.k_sb + kvh * a.k_sh;
    it.vb = a.v + b * a.v_sb + kvh * a.v_sh;
    it.prow = a.pairs + r * a.pairs_stride;
    it.mrow = SUB ? a.tile_masks + r * a.masks_stride : nullptr;
    it.e0 = e0;
    it.cached = n_ent <= RC;
    it.n_tiles = n_ent << a.tpb_log2;
    it.tpb_mask = (1 << a.tpb_log2) - 1;
    const int q_tile0 = qt * QTILE;
    it.q_row0 = q_tile0 + QT * it.hf;  // this wave's first row
    it.q_abs_tile_max = a.q_offset + min(a.Tq, q_tile0 + QTILE) - 1;
    it.q_abs_min = a.q_offset + it.q_row0;  // this wave's first absolute position
    return it;
  }

  // Sets up work item (qt, r, hs, b): query tile qt (64 rows) of CSR row r, batch b, head
  // split hs.  Each wave owns 32 rows (half hf) of one query head; every K/V tile staged in
  // LDS feeds all NW waves.  Caches the CSR row of the query tile in s_row (callers barrier
  // before, so no wave still reads it).
  static __device__ __forceinline__ Item setup(const PrefillArgs& a, int qt, int r, int hs, int b, int32_t* s_row,
                                               int32_t* s_mask) {
    // CSR row of this query tile; each block holds 2^tpb_log2 key tiles.
    const int32_t* offs = a.offsets + r * a.offsets_stride + (qt >> a.qpb_log2);
    const int e0 = offs[0];
    const Item it = setup_base(a, qt, r, hs, b, e0, offs[1] - e0);
    if (it.cached) {
      const int n_ent = it.n_tiles >> a.tpb_log2;
      for (int x = threadIdx.x; x < n_ent; x += NT) s_row[x] = it.prow[e0 + x];
      if (SUB)
        for (int x = threadIdx.x; x < n_ent; x += NT) s_mask[x] = it.mrow[e0 + x];
    }
    return it;
  }

  // Rows of Q past T_q read a clamped (valid) row; their outputs are never stored.
  static __device__ __forceinline__ const elem_t* q_src(const PrefillArgs& a, const Item& it) {
    const int row = min(it.q_row0 + it.l32, a.Tq - 1);
    return it.qb + (int64_t)row * a.q_st + 8 * it.g;
  }

  // Last key tile an item can use: it starts before T_k and at or before the causal limit of the
  // whole query tile (-1: none).
  static __device__ __forceinline__ int kt_limit(const PrefillArgs& a, const Item& it) {
    return it.q_abs_tile_max < 0 ? -1 : min((a.Tk + KT - 1) / KT - 1, it.q_abs_tile_max / KT);
  }

  // Key tile of schedule position t, or -1 for a negative block id or one past kt_hi's block
  // (rejected before the shift, which cannot overflow then).
  static __device__ __forceinline__ int tile_of(const PrefillArgs& a, const Item& it, const int32_t* s_row, int t,
                                                int kt_hi) {
    const int e = t >> a.tpb_log2;
    // Two distinct loads (LDS cache, or a global read past the cached entries), so the two are
    // not merged into one flat load of a selected pointer.
    const int blk = it.cached ? s_row[e] : load_uniform_now(it.prow + it.e0 + e);
    if (blk < 0 || blk > (kt_hi >> a.tpb_log2)) return -1;
    return (blk << a.tpb_log2) + (t & it.tpb_mask);
  }

  static __device__ __forceinline__ int sub_log2(const PrefillArgs& a) { return SUB ? a.sub_log2 : 0; }

  // Sub-block mask of schedule position t (tile schedules only; t indexes entries there).
  static __device__ __forceinline__ uint32_t mask_of(const Item& it, const int32_t* s_mask, int t) {
    return (uint32_t)(it.cached ? s_mask[t] : load_uniform_now(it.mrow + it.e0 + t));
  }

  // Whether a sub-block mask drops any sub-block of its tile.
  static __device__ __forceinline__ bool partial_mask(const PrefillArgs& a, uint32_t m) {
    if (!sub_log2(a)) return false;
    const int s = 64 >> sub_log2(a);
    return m != (s == 4 ? 0xffffu : 0xfu);
  }

  // Key sub-blocks of the tile visible to this lane's query row (local row hf*32 + l32 of
  // the 64-row query tile) under sub-block mask m: bit sc for key sub-block sc; all ones
  // without sub-blocks.
  static __device__ __forceinline__ uint32_t row_bits(const PrefillArgs& a, uint32_t m, int hf, int l32) {
    return sub_log2(a) ? m >> (((hf * QT + l32) >> sub_log2(a)) * (64 >> sub_log2(a))) : 0xffffffffu;
  }

  // This lane's key limit in 32-key half j, 16-key chunk h of a tile: lim (the last visible
  // key offset minus 8g), or -1 (nothing visible) where the row's bits drop the sub-block
  // of that chunk.  A 16-key chunk never straddles sub-blocks (b >= 16).
  static __device__ __forceinline__ int chunk_lim(const PrefillArgs& a, uint32_t bits, int lim, int j, int h) {
    const int sh = sub_log2(a) ? (32 * j + 16 * h) >> sub_log2(a) : 0;
    return ((bits >> sh) & 1u) ? lim : -1;
  }

  // First tile at or after t that can contribute (0 <= kt <= kt_hi = kt_limit()): tiles entirely
  // past T_k or above the causal limit of the whole 64-row query tile are skipped, and so are
  // negative ids (malformed schedules) rather than read.
  static __device__ __forceinline__ int next_usable(const PrefillArgs& a, const Item& it, const int32_t* s_row,
                                                    int t, int kt_hi) {
    for (; t < it.n_tiles; ++t) {
      const int kt = tile_of(a, it, s_row, t, kt_hi);
      if (kt >= 0 && kt <= kt_hi) break;
    }
    return t;
  }

  // The usable tiles of an item in schedule order, read 64 schedule positions at a time:
  // lane i of `kt` holds the key tile of position `next - 64 + i` (and lane i of `m` its
  // sub-block mask), bit i of `live` marks it usable and not yet taken.  A tile is usable
  // under the rule of next_usable: 0 <= kt <= kt_hi, the last key tile that starts before T_k
  // and at or before the causal limit of the query tile.
  struct TileQueue {
    int kt;
    uint32_t m;
    uint64_t live;
    int next;
    int kt_hi;
  };

  static __device__ __forceinline__ TileQueue queue_begin(const PrefillArgs& a, const Item& it) {
    TileQueue q;
    q.kt = 0;
    q.m = 0;
    q.live = 0;
    q.next = 0;
    q.kt_hi = min((a.Tk + KT - 1) / KT - 1, it.q_abs_tile_max / KT);  // kt_limit() for q_abs_tile_max >= 0
    return q;
  }

  static __device__ __forceinline__ void queue_fill(const PrefillArgs& a, const Item& it, const int32_t* s_row,
                                                    const int32_t* s_mask, TileQueue& q) {
    const int t = q.next + (threadIdx.x & 63);
    int blk = -1;
    uint32_t m = 0;
    if (t < it.n_tiles) {
      const int e = t >> a.tpb_log2;
      blk = it.cached ? s_row[e] : load_lane_now(it.prow + it.e0 + e);
      if (SUB) m = (uint32_t)(it.cached ? s_mask[e] : load_lane_now(it.mrow + it.e0 + e));
    }
    // Block ids past kt_hi's block are rejected before the product, which cannot overflow then.
    const bool ok = blk >= 0 && blk <= (q.kt_hi >> a.tpb_log2);
    q.kt = ok ? blk * (1 << a.tpb_log2) + (t & it.tpb_mask) : -1;
    q.m = m;
    q.live = __builtin_amdgcn_ballot_w64(ok && q.kt <= q.kt_hi);
    q.next += 64;
  }

  // Takes the next usable tile (key tile kt, sub-block mask m); false when none is left.
  static __device__ __forceinline__ bool queue_pop(const PrefillArgs& a, const Item& it, const int32_t* s_row,
                                                   const int32_t* s_mask, TileQueue& q, int& kt, uint32_t& m) {
    while (q.live == 0) {
      if (q.next >= it.n_tiles) return false;
      queue_fill(a, it, s_row, s_mask, q);
    }
    const int l = __builtin_ctzll(q.live);
    q.live &= q.live - 1;
    kt = __builtin_amdgcn_readlane(q.kt, l);
    if (SUB) m = (uint32_t)__builtin_amdgcn_readlane((int)q.m, l);
    return true;
  }

  // Source of this wave's direct loads for key tile 0 of K or V (uniform) and the bytes per
  // key tile; the wave's NIW loads of a tile share one row block (NIW <= NCG).
  struct Src {
    const char* p;
    uint32_t tile_bytes;
  };
  static __device__ __forceinline__ Src src_of(const elem_t* base, int64_t st, int wave) {
    const int k0 = wave * NIW;
    return {reinterpret_cast<const char*>(base) + ((int64_t)16 * (k0 / NCG) * st + 32 * (k0 % NCG)) * 2,
            (uint32_t)(KT * st * 2)};
  }

  // LDS address of this wave's share of a staged tile.
  static __device__ __forceinline__ uint32_t dma_lds(const char* tile, int wave) {
    const int k0 = wave * NIW;
    return lds_addr(tile + (k0 % NCG) * 4096 + (k0 / NCG) * 1024);
  }

  // dma() for a key tile wholly before T_k: one 64-bit product for the tile's address, the
  // column groups 64 bytes apart in the load instructions' offsets.
  static __device__ __forceinline__ void dma_full(const Src& s, uint32_t off, uint32_t lds, int kt) {
    static_assert(NIW <= NCG && NIW <= 2, "one row block, at most two loads per wave");
    const char* wb = s.p + (uint64_t)(uint32_t)kt * s.tile_bytes;
    load_lds16_at<0>(wb, off, lds);
    if constexpr (NIW > 1) load_lds16_at<64>(wb, off, lds + 4096);
  }

  // O / l written through this wave's 32 x D staging area in LDS (rows at 2D bytes, 16-byte
  // chunk c of row r at position c ^ (r % (D/8))), then stored as 16-byte row pieces: each
  // global store instruction writes whole contiguous rows.  The caller guarantees that no
  // other wave uses `stage` (a barrier after the last read of the K/V buffers).
  static __device__ __forceinline__ void epilogue(const PrefillArgs& a, const Item& it, int b,
                                                  const f32x16 (&O)[D / 32], float l_run, char* stage, int lane) {
    constexpr int NCH = D / 8;         // 16-byte chunks per row
    constexpr int RPI = 1024 / (2 * D);  // rows per 1 KiB wave-wide read
    const float lt = halves_sum(l_run);
    const float inv = lt > 0.f ? 1.f / lt : 1.f;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {  // d = 32dt + 8rq + 4g + 0..3: chunk 4dt + rq, half g
        const int c = 4 * dt + rq;
        const u32x2 w = {E::pack2f(O[dt][4 * rq] * inv, O[dt][4 * rq + 1] * inv),
                         E::pack2f(O[dt][4 * rq + 2] * inv, O[dt][4 * rq + 3] * inv)};
        *reinterpret_cast<u32x2*>(stage + it.l32 * 2 * D + 16 * (c ^ (it.l32 & (NCH - 1))) + 8 * it.g) = w;
      }
    // The wave reads back what its own lanes wrote: LDS executes one wave's accesses in
    // order, so only the compiler must keep the order.
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    asm volatile("" ::: "memory");
    elem_t* ob = a.o + b * a.o_sb + it.hq * a.o_sh;
    constexpr int NR = QT / RPI;  // wave-wide reads (and stores) of the 32 rows
    // The lane's chunk, opaque to the compiler: the per-row offsets below are then computed here
    // instead of being hoisted out of the item loop, where they would stay live across the tile
    // loop (and spill).
    int lane_e = lane;
    asm volatile("" : "+v"(lane_e));
    const int p = lane_e % NCH;
    auto dst = [&](int row) {
      return reinterpret_cast<u32x4*>(ob + (int64_t)(it.q_row0 + row) * a.o_st + 8 * (p ^ (row & (NCH - 1))));
    };
    // Non-temporal stores: O is not read again here, so it need not displace K/V lines in L2.
    if (it.q_row0 + QT <= a.Tq) {
      // Every row exists: all reads are issued before the first store, so the LDS round trips
      // overlap (a store guarded per lane would keep its read inside the guard, one wait each).
      u32x4 w[NR];
#pragma unroll
      for (int k = 0; k < NR; ++k) w[k] = *reinterpret_cast<const u32x4*>(stage + (RPI * k + lane_e / NCH) * 2 * D + 16 * p);
#pragma unroll
      for (int k = 0; k < NR; ++k) __builtin_nontemporal_store(w[k], dst(RPI * k + lane_e / NCH));
    } else {
#pragma unroll
      for (int k = 0; k < NR; ++k) {
        const int row = RPI * k + lane_e / NCH;
        const u32x4 w = *reinterpret_cast<const u32x4*>(stage + row * 2 * D + 16 * p);
        if (it.q_row0 + row < a.Tq) __builtin_nontemporal_store(w, dst(row));
      }
    }
  }

  // ---- one tile at a time (one- and two-head workgroups) -------------------------------
  // Online softmax over the 32-key half j of the current tile for this wave's 32 rows.
  // Scores are raw; p = 2^(s*c - m_ref).  Returns the P^T operands of the two 16-key chunks.
  template <bool MASK>
  static __device__ __forceinline__ void softmax_half(const PrefillArgs& a, f32x16& S, u32x4 (&P)[2],
                                                      f32x16 (&O)[D / 32], float& m_ref, float& l_run, float c,
                                                      uint32_t bits, int lim, int j) {
    if (MASK) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int lh = chunk_lim(a, bits, lim, j, h);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int key = 32 * j + 16 * h + e;  // minus 8g, folded into the limit
          if (key > lh) S[8 * h + e] = -__builtin_inff();
        }
      }
    }
    float mx = S[0];
#pragma unroll
    for (int rr = 1; rr < 16; ++rr) mx = fmaxf(mx, S[rr]);
    mx = halves_max(mx);
    const float m_tile = mx * c;  // -inf stays -inf (c > 0)
    float m = m_ref == -__builtin_inff() ? m_tile : m_ref;
    if (__any(m_tile > m + RESCALE_LOG2)) {
      const float m_new = fmaxf(m, m_tile);
      const float alpha = m_new == -__builtin_inff() ? 1.f : fast_exp2(m - m_new);
      m = m_new;
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt) O[dt] *= alpha;
    }
    m_ref = m;
    const float neg_m = m == -__builtin_inff() ? 0.f : -m;
    float ls = 0.f;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float pf[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pf[e] = fast_exp2(fmaf(S[8 * h + e], c, neg_m));
        ls += pf[e];
      }
      P[h] = u32x4{E::pack2f(pf[0], pf[1]), E::pack2f(pf[2], pf[3]), E::pack2f(pf[4], pf[5]), E::pack2f(pf[6], pf[7])};
    }
    l_run += ls;
  }

  // One 64-key tile: S^T = K Q^T per 32-key half, softmax, O^T += V^T P^T.  The softmax of
  // one half can run under the matrix instructions of the other half.
  template <bool MASK>
  static __device__ __forceinline__ void tile(const PrefillArgs& a, const char* cK, const char* cV, const Frag& f,
                                              const u32x4 (&qf)[D / 16], f32x16 (&O)[D / 32], float& m_ref,
                                              float& l_run, float c, uint32_t bits, int lim) {
    // The two key halves are independent accumulation chains; alternating them keeps the
    // matrix pipe busy while each MFMA waits for its predecessor's result.
    f32x16 S[2] = {f32x16{}, f32x16{}};
#pragma unroll
    for (int cc = 0; cc < D / 16; ++cc)
#pragma unroll
      for (int j = 0; j < 2; ++j) S[j] = E::mfma32(kfrag(cK, f, j, cc), qf[cc], S[j]);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      u32x4 P[2];
      softmax_half<MASK>(a, S[j], P, O, m_ref, l_run, c, bits, lim, j);
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) O[dt] = E::mfma32(vfrag(cV, f, j, h, dt), P[h], O[dt]);
    }
  }

  // One work item, one tile at a time: the next tile's direct loads run under the current
  // tile's compute (double buffer), or after it (single buffer).
  static __device__ __forceinline__ void item(const PrefillArgs& a, int qt, int r, int hs, int b, char* sKV,
                                              int32_t* s_row, int32_t* s_mask) {
    char* sK = sKV;
    char* sV = sKV + NBK * TILE_BYTES;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const Item it = setup(a, qt, r, hs, b, s_row, s_mask);
    // Q^T as the B operand of S^T = K Q^T: lane holds row l32, d = 16c + 8g .. +7.
    u32x4 qf[D / 16];
    {
      const elem_t* qs = q_src(a, it);
#pragma unroll
      for (int c = 0; c < D / 16; ++c) qf[c] = *reinterpret_cast<const u32x4*>(qs + 16 * c);
    }
    const Frag f(lane);
    const DmaLane dl(a, lane);
    __syncthreads();  // s_row visible

    f32x16 O[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) O[dt] = f32x16{};
    float m_ref = -__builtin_inff();
    float l_run = 0.f;  // this lane's half of the row sum
    const float c = a.scale_log2;

    const int kt_hi = kt_limit(a, it);
    int t = next_usable(a, it, s_row, 0, kt_hi);
    int buf = 0;
    if (t < it.n_tiles) {
      const int kt = tile_of(a, it, s_row, t, kt_hi);
      dma<true>(it.kb, a.k_st, dl.k, sK, kt, a.Tk, wave, lane);
      dma<false>(it.vb, a.v_st, dl.v, sV, kt, a.Tk, wave, lane);
    }
    wait_dma();
    __syncthreads();

    while (t < it.n_tiles) {
      const int kt = tile_of(a, it, s_row, t, kt_hi);
      const int tn = next_usable(a, it, s_row, t + 1, kt_hi);
      if (NBK == 2 && tn < it.n_tiles) {
        const int ktn = tile_of(a, it, s_row, tn, kt_hi);
        dma<true>(it.kb, a.k_st, dl.k, sK + (buf ^ 1) * TILE_BYTES, ktn, a.Tk, wave, lane);
        dma<false>(it.vb, a.v_st, dl.v, sV + (buf ^ 1) * TILE_BYTES, ktn, a.Tk, wave, lane);
      }
      const char* cK = sK + buf * TILE_BYTES;
      const char* cV = sV + buf * TILE_BYTES;

      // A wave whose 32 rows all precede the tile skips it (the other half may not).
      if (kt * KT <= it.q_abs_min + QT - 1) {
        const uint32_t m = sub_log2(a) ? mask_of(it, s_mask, t) : 0u;
        const bool need_mask = (kt * KT + KT - 1 > it.q_abs_min) || (kt * KT + KT > a.Tk) || partial_mask(a, m);
        const int lim = min(it.q_abs_min + it.l32, a.Tk - 1) - kt * KT - 8 * it.g;
        const uint32_t bits = row_bits(a, m, it.hf, it.l32);
        if (need_mask)
          tile<true>(a, cK, cV, f, qf, O, m_ref, l_run, c, bits, lim);
        else
          tile<false>(a, cK, cV, f, qf, O, m_ref, l_run, c, bits, lim);
      }

      if (NBK == 1 && tn < it.n_tiles) {
        __syncthreads();  // single buffer: every wave is done reading it
        const int ktn = tile_of(a, it, s_row, tn, kt_hi);
        dma<true>(it.kb, a.k_st, dl.k, sK, ktn, a.Tk, wave, lane);
        dma<false>(it.vb, a.v_st, dl.v, sV, ktn, a.Tk, wave, lane);
      }
      wait_dma();
      __syncthreads();
      if (NBK == 2) buf ^= 1;
      t = tn;
    }
    // Every wave has passed the last barrier: the K/V buffers are free for the staging.
    epilogue(a, it, b, O, l_run, sKV + wave * WAVE_BYTES, lane);
  }

  // ---- software-pipelined loop (four-head workgroups) ----------------------------------
  // Masks one tile's S^T (causal / past T_k / sub-blocks, branch-free): keys past the
  // chunk limits of (bits, lim) become -inf.
  static __device__ __forceinline__ void mask_tile(const PrefillArgs& a, f32x16 (&S)[2], uint32_t bits, int lim) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int lh = chunk_lim(a, bits, lim, j, h);
#pragma unroll
        for (int e = 0; e < 8; ++e)
          S[j][8 * h + e] = (32 * j + 16 * h + e > lh) ? -__builtin_inff() : S[j][8 * h + e];
      }
  }

  // Masks one tile's S^T (mask_tile) and returns its scaled row max.
  static __device__ __forceinline__ float mask_rowmax(const PrefillArgs& a, f32x16 (&S)[2], uint32_t bits,
                                                      int lim, float c) {
    mask_tile(a, S, bits, lim);
    float mx = S[0][0];
#pragma unroll
    for (int rr = 1; rr < 16; ++rr) mx = fmaxf(mx, S[0][rr]);
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) mx = fmaxf(mx, S[1][rr]);
    mx = halves_max(mx);
    return mx * c;  // -inf stays -inf (c > 0)
  }

  // ---- lookahead metadata (persistent four-head loop) -----------------------------------
  // While an item's first tiles load, the persistent loop fetches the CSR row of the next
  // item, the CSR offsets and decoded (qt, r, hs, b) of the item after it and a new claim
  // from the counter.  All of it lands in LDS before the barrier that publishes the item's
  // first tiles, so the next item starts without a dependent global read and no register
  // stays live across the tile loop.
  struct Look {
    int e0, n_ent;        // this item's CSR entries
    int v1, e0_1, n_1;    // next item (>= n_items: none) and its CSR entries
    int r_1;              // CSR row of the next item
    int v2;               // the item after it
    int n_items;
    int32_t* row_dst;     // row cache of the next item (and its sub-block masks)
    int32_t* mask_dst;
    int* meta2;           // metadata slot of item v2: CSR offsets (first, end) and (qt, r, hs, b)
    int* vid3;            // id slot of the newly claimed item
  };
  static constexpr int RPT = (RC + NT - 1) / NT;  // cached row entries per thread
  struct LookLoads {
    int32_t rv[RPT];
    int32_t mv[SUB ? RPT : 1];
    int o0, o1, qt2, r2, hs2, b2;
    unsigned nv;
  };

  static __device__ __forceinline__ void look_issue(const PrefillArgs& a, const Look& lk, LookLoads& ld) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int u = 0; u < RPT; ++u) ld.rv[u] = ld.mv[SUB ? u : 0] = 0;
    ld.o0 = ld.o1 = ld.qt2 = ld.r2 = ld.hs2 = ld.b2 = 0;
    ld.nv = 0;
    if (lk.v1 < lk.n_items && lk.n_1 <= RC) {
      const int r = lk.r_1;
      const int32_t* src = a.pairs + r * a.pairs_stride + lk.e0_1;
#pragma unroll
      for (int u = 0; u < RPT; ++u)
        if (tid + u * NT < lk.n_1) ld.rv[u] = src[tid + u * NT];
      if (SUB) {
        const int32_t* msrc = a.tile_masks + r * a.masks_stride + lk.e0_1;
#pragma unroll
        for (int u = 0; u < RPT; ++u)
          if (tid + u * NT < lk.n_1) ld.mv[u] = msrc[tid + u * NT];
      }
    }
    if (tid == 0) {
      if (lk.v2 < lk.n_items) {
        decode_item(a, lk.v2, ld.qt2, ld.r2, ld.hs2, ld.b2);
        const int32_t* o = a.offsets + ld.r2 * a.offsets_stride + (ld.qt2 >> a.qpb_log2);
        ld.o0 = o[0];
        ld.o1 = o[1];
      }
      ld.nv = atomicAdd(&a.counter[WS_NEXT], 1u);
    }
  }

  static __device__ __forceinline__ void look_commit(const Look& lk, const LookLoads& ld) {
    const int tid = threadIdx.x;
    if (lk.v1 < lk.n_items && lk.n_1 <= RC) {
#pragma unroll
      for (int u = 0; u < RPT; ++u)
        if (tid + u * NT < lk.n_1) {
          lk.row_dst[tid + u * NT] = ld.rv[u];
          if (SUB) lk.mask_dst[tid + u * NT] = ld.mv[u];
        }
    }
    if (tid == 0) {
      lk.meta2[1] = ld.o0;
      lk.meta2[2] = ld.o1;
      lk.meta2[3] = ld.qt2;
      lk.meta2[4] = ld.r2;
      lk.meta2[5] = ld.hs2;
      lk.meta2[6] = ld.b2;
      lk.vid3[0] = (int)ld.nv;
    }
  }

  // Same work item as item(), with the tile loop software-pipelined: each step computes the
  // probabilities of tile i while the matrix cores already run S^T = K Q^T of tile i+1,
  // then O^T += V^T P^T of tile i while the VALU reduces the row max of tile i+1.
  // Meanwhile the direct loads fetch K of tile i+2 (two K buffers) and V of tile i+1 (three
  // V buffers, for the upper half's lag).  Q goes through the wave's own LDS slot into
  // registers once; the slot then stages O for the epilogue.  Tiles that lie wholly after
  // this wave's rows cost matrix work but add p == 0.  LOOK: the item's CSR row is already
  // in s_row (lk->e0, lk->n_ent) and the lookahead reads of *lk run under the first tiles'
  // loads.
  // vb_first: V buffer for the item's first tile, the one that the previous item's last step
  // does not read (K buffers are never read in an item's last step); set to the next item's on
  // return.  So an item starts loading without waiting for the other waves to finish the
  // previous one.
  template <bool LOOK>
  static __device__ __forceinline__ void item_pipelined(const PrefillArgs& a, int qt, int r, int hs, int b,
                                                        char* sKV, char* sQ, int32_t* s_row, int32_t* s_mask,
                                                        const Look* lk, int& vb_first) {
    char* sK = sKV;
    char* sV = sKV + NBK * TILE_BYTES;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    tl_stamp(TL_GAP);
    const Item it = LOOK ? setup_base(a, qt, r, hs, b, lk->e0, lk->n_ent) : setup(a, qt, r, hs, b, s_row, s_mask);
    char* sQw = sQ + wave * WAVE_BYTES;
    load_q(a, it.qb, it.q_row0, sQw, lane);  // Q^T operand of this wave into LDS
    tl_stamp(TL_SETUP_Q);
    const Frag f(lane);
    const DmaLane dl(a, lane);
    // lim of tile kt: min(q_abs, T_k - 1) - kt*KT - 8g (past the tile when no key is masked)
    const int lim0 = min(it.q_abs_min + it.l32, a.Tk - 1) - 8 * it.g;
    if (!LOOK) __syncthreads();  // s_row visible (LOOK: it was before the item began)

    f32x16 O[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) O[dt] = f32x16{};
    float m_ref = -__builtin_inff();
    float l_run = 0.f;
    const float c = a.scale_log2;

    // Direct loads of key tile kt into K buffer kb / V buffer vb (full tiles from one uniform
    // address per load, the tile at T_k row by row).
    const Src src_k = src_of(it.kb, a.k_st, wave);
    const Src src_v = src_of(it.vb, a.v_st, wave);
    const uint32_t lds_k = dma_lds(sK, wave);
    const uint32_t lds_v = dma_lds(sV, wave);
    const int kt_full = a.Tk / KT;  // key tiles wholly before T_k
    auto load_k = [&](int kt, int kb) {
      if (kt < kt_full)
        dma_full(src_k, dl.k, lds_k + kb * TILE_BYTES, kt);
      else
        dma<true>(it.kb, a.k_st, dl.k, sK + kb * TILE_BYTES, kt, a.Tk, wave, lane);
    };
    auto load_v = [&](int kt, int vb) {
      if (kt < kt_full)
        dma_full(src_v, dl.v, lds_v + vb * TILE_BYTES, kt);
      else
        dma<false>(it.vb, a.v_st, dl.v, sV + vb * TILE_BYTES, kt, a.Tk, wave, lane);
    };

    // Prime: K of the first two usable tiles in K buffers 0, 1 and V of the first in V
    // buffer vb_first; S^T and row max of the first.  No wave reads those buffers until every
    // wave has passed the barrier below: the K buffers were last read before the previous
    // item's last barrier, and its last step reads only the other two V buffers.
    TileQueue q = queue_begin(a, it);
    int kt_cur = 0, kt_nxt = 0;
    uint32_t m_cur = 0u, m_nxt = 0u;
    bool has_cur = queue_pop(a, it, s_row, s_mask, q, kt_cur, m_cur);
    bool has_nxt = has_cur && queue_pop(a, it, s_row, s_mask, q, kt_nxt, m_nxt);
    tl_stamp(TL_POPS);
    if (has_cur) {
      load_k(kt_cur, 0);
      load_v(kt_cur, vb_first);
    }
    if (has_nxt) load_k(kt_nxt, 1);
    tl_stamp(TL_KV);
    LookLoads ld;
    if constexpr (LOOK) look_issue(a, *lk, ld);
    tl_stamp(TL_LOOK);
    wait_dma();
    if constexpr (LOOK) look_commit(*lk, ld);
    tl_stamp(TL_WAIT);
    __syncthreads();
    tl_stamp(TL_BARRIER);
    u32x4 Qr[D / 16];
#pragma unroll
    for (int cc = 0; cc < D / 16; ++cc) Qr[cc] = qfrag(sQw, f, cc);
    f32x16 S[2] = {f32x16{}, f32x16{}};  // scores of the current tile
    if (has_cur) {
#pragma unroll
      for (int cc = 0; cc < D / 16; ++cc) {
        const u32x4 qv = Qr[cc];
#pragma unroll
        for (int j = 0; j < 2; ++j) S[j] = E::mfma32(kfrag(sK, f, j, cc), qv, S[j]);
      }
      // The row reference is the first tile's (masked) row max; later tiles keep it unless their
      // probabilities grow past REFIT_SUM (refit below).
      m_ref = mask_rowmax(a, S, row_bits(a, m_cur, it.hf, it.l32), lim0 - kt_cur * KT, c);
    }
    float neg_m = m_ref == -__builtin_inff() ? 0.f : -m_ref;
    bool ref_ok = !__any(m_ref == -__builtin_inff());  // every row of the wave has a reference
    // The first step loads K of tile t2 into the buffer of t0, which the prime just read.
    __syncthreads();
    tl_stamp(TL_FIRST_QK);

    // Each step holds two half-steps per wave: A = S^T of the next tile on the matrix cores
    // under the exponentials of this tile, B = O^T += V^T P^T of a tile under the row max of
    // the following one.  The lower 32-row half runs A(i), B(i) in step i; the upper half
    // runs B(i-1), A(i), so the two waves on each SIMD (one of each half) run the VALU-heavy
    // A and the matrix-only B at the same time.  K is double-buffered (K of tile i+1 is read
    // in step i by both halves, K of tile i+2 loads); V is triple-buffered (V of tiles i-1
    // and i are read, V of tile i+1 loads), so one barrier per step still suffices.
    const bool lag = it.hf == 1;  // upper half: one half-step behind
    int vb_cur = vb_first;  // V buffer of the current tile (buffers in turn)
    bool pending = false;  // upper half: B of the previous tile still to run
    u32x4 P[2][2];         // probabilities of the tile whose B is next
    constexpr int NQ = D / 8;    // QK MFMAs per tile: i -> (key half j = i % 2, cc = i / 2)
    constexpr int PE = 32 / NQ;  // probabilities per QK MFMA
    constexpr int NP = D / 8;    // PV MFMAs: i -> (dt = i % (D/32), h, j)
    constexpr int ND = D / 32;

    // Block B: PV of the tile in V buffer cV with probabilities P (D/8 MFMAs; V fragments
    // read two MFMAs ahead).  No VALU work: the row reference stays fixed between refits.
    auto block_b = [&](const char* cV) {
      auto vfr = [&](int i) { return vfrag(cV, f, i / (2 * ND), (i / ND) & 1, i % ND); };
      u32x4 vf[2] = {vfr(0), vfr(1)};
      __builtin_amdgcn_s_setprio(0);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < NP; ++i) {
        O[i % ND] = E::mfma32(vf[i & 1], P[i / (2 * ND)][(i / ND) & 1], O[i % ND]);
        if (i + 2 < NP) vf[i & 1] = vfr(i + 2);
        __builtin_amdgcn_sched_barrier(0);
      }
    };

    // Probabilities of the tile whose masked scores are Sc, against the current reference:
    // P and this lane's share of the row sum.
    auto probs = [&](const f32x16 (&Sc)[2], float& ls, auto halves_tag) {
      constexpr int NJ = decltype(halves_tag)::value;  // key halves with visible keys (2, or 1: the second is all 0)
      uint32_t pw[2][2][4] = {};
      ls = 0.f;
#pragma unroll
      for (int x = 0; x < 16 * NJ; x += 2) {
        const int j = x >> 4, rr = x & 15;
        const float p0 = fast_exp2(fmaf(Sc[j][rr], c, neg_m));
        const float p1 = fast_exp2(fmaf(Sc[j][rr + 1], c, neg_m));
        ls += p0 + p1;
        pw[j][rr >> 3][(rr & 7) >> 1] = E::pack2f(p0, p1);
      }
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int h = 0; h < 2; ++h) P[j][h] = u32x4{pw[j][h][0], pw[j][h][1], pw[j][h][2], pw[j][h][3]};
    };

    // Refit (rare): a row had no reference yet, or a lane's probabilities of this tile sum past
    // REFIT_SUM (or to inf / NaN).  Raises each row's reference to its max over this tile, rescales
    // O and l to it and recomputes the tile's probabilities.  Any reference gives the same result
    // up to rounding; the refit only keeps 2^(s c - m_ref) finite.
    auto refit = [&](const f32x16 (&Sc)[2], float& ls) {
      tl_count(TL_REFITS);
      float mx = Sc[0][0];
#pragma unroll
      for (int rr = 1; rr < 16; ++rr) mx = fmaxf(mx, Sc[0][rr]);
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) mx = fmaxf(mx, Sc[1][rr]);
      const float m_tile = halves_max(mx) * c;  // -inf stays -inf (c > 0)
      const float m_new = m_ref == -__builtin_inff() ? m_tile : fmaxf(m_ref, m_tile);
      const float alpha = (m_ref == -__builtin_inff() || m_new == -__builtin_inff()) ? 1.f : fast_exp2(m_ref - m_new);
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt) O[dt] *= alpha;
      m_ref = m_new;
      neg_m = m_ref == -__builtin_inff() ? 0.f : -m_ref;
      ref_ok = !__any(m_ref == -__builtin_inff());
      probs(Sc, ls, std::integral_constant<int, 2>{});
    };

    // One step on the tile whose scores are in Sc and whose K is in buffer KB, filling Sx
    // with the next tile's.  The loop runs two steps per iteration with the two score sets
    // and K buffers trading roles, so scores are never copied and K buffers are constants.
    auto step = [&](auto kb_tag, f32x16 (&Sc)[2], f32x16 (&Sx)[2]) {
      constexpr int kb_cur = decltype(kb_tag)::value;
      constexpr int kb_nxt = kb_cur ^ 1;
      const int vb_prev = vb_cur == 0 ? 2 : vb_cur - 1;
      const int vb_nxt = vb_cur == 2 ? 0 : vb_cur + 1;
      int kt_nn = 0;
      uint32_t m_nn = 0u;
      const bool has_nn = has_nxt && queue_pop(a, it, s_row, s_mask, q, kt_nn, m_nn);
      if (has_nn) load_k(kt_nn, kb_cur);
      if (has_nxt) load_v(kt_nxt, vb_nxt);

      // Upper half: B of the previous tile.
      if (lag && pending) block_b(sV + vb_prev * TILE_BYTES);

      const char* cK = sK + kb_nxt * TILE_BYTES;
      // Branch-free on purpose: after the last tile the QK half runs on a stale K buffer
      // (no direct load is in flight then) and its result is dropped.  A separate last-tile
      // path would let the compiler merge the two copies of the exponentials ahead of the
      // branch, which undoes the interleaving.
      //
      // Block A: QK of the next tile (D/8 MFMAs; K fragments read three MFMAs ahead, Q
      // fragments two chunk pairs ahead) with this tile's probabilities spread over it.
      // The sched_barrier fences keep the order as written: one MFMA, its LDS reads, its
      // share of the VALU work.
      auto kfr = [&](int i) { return kfrag(cK, f, i & 1, i >> 1); };
      u32x4 kf[3] = {kfr(0), kfr(1), kfr(2)};
      Sx[0] = f32x16{};
      Sx[1] = f32x16{};
      float ls = 0.f;
      uint32_t pw[2][2][4];
      // Raising the priority of the wave in the VALU-heavy block A lets its exponentials go
      // first while the other wave's matrix instructions fill the MFMA pipe.
      __builtin_amdgcn_s_setprio(1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < NQ; ++i) {
        Sx[i & 1] = E::mfma32(kf[i % 3], Qr[i >> 1], Sx[i & 1]);
        if (i + 3 < NQ) kf[i % 3] = kfr(i + 3);
#pragma unroll
        for (int u = 0; u < PE; u += 2) {
          const int x = PE * i + u;
          const int j = x >> 4, rr = x & 15;
          const float p0 = fast_exp2(fmaf(Sc[j][rr], c, neg_m));
          const float p1 = fast_exp2(fmaf(Sc[j][rr + 1], c, neg_m));
          ls += p0 + p1;
          uint32_t w = E::pack2f(p0, p1);
          // Pins the computation here: without it the compiler sinks the exponentials past
          // the mask branch to their use in block B.
          asm volatile("" : "+v"(w), "+v"(ls));
          pw[j][rr >> 3][(rr & 7) >> 1] = w;
        }
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int h = 0; h < 2; ++h) P[j][h] = u32x4{pw[j][h][0], pw[j][h][1], pw[j][h][2], pw[j][h][3]};
      if (!ref_ok || __any(!(ls <= REFIT_SUM))) refit(Sc, ls);
      l_run += ls;

      // Causal / T_k mask of the next tile, only where it cuts into the tile (uniform per
      // wave; about one tile in a row's window).
      const int kbase_n = kt_nxt * KT;
      if (kbase_n + KT - 1 > it.q_abs_min || kbase_n + KT > a.Tk || partial_mask(a, m_nxt)) {
        mask_tile(a, Sx, row_bits(a, m_nxt, it.hf, it.l32), lim0 - kbase_n);
      }

      // Lower half: B of this tile.
      if (!lag) block_b(sV + vb_cur * TILE_BYTES);
      pending = true;

      wait_dma();
      __syncthreads();
      tl_count(TL_STEPS);
      has_cur = has_nxt;
      kt_cur = kt_nxt;
      has_nxt = has_nn;
      kt_nxt = kt_nn;
      m_nxt = m_nn;
      vb_cur = vb_nxt;
    };
    // O^T += V^T P^T of the tile in V buffer cV, nothing else (the last tile).
    auto block_pv = [&](const char* cV, auto halves_tag) {
      constexpr int NPJ = NP / 2 * decltype(halves_tag)::value;  // MFMAs over the key halves that count
      auto vfr = [&](int i) { return vfrag(cV, f, i / (2 * ND), (i / ND) & 1, i % ND); };
      u32x4 vf[2] = {vfr(0), vfr(1)};
      __builtin_amdgcn_s_setprio(0);
#pragma unroll
      for (int i = 0; i < NPJ; ++i) {
        O[i % ND] = E::mfma32(vf[i & 1], P[i / (2 * ND)][(i / ND) & 1], O[i % ND]);
        if (i + 2 < NPJ) vf[i & 1] = vfr(i + 2);
      }
    };

    // The last tile: its probabilities and PV only.  There is no next tile, so no S^T half, no
    // loads and no barrier (the one before the epilogue follows); the upper half's PV of this
    // tile runs after it.
    auto last_step = [&](f32x16 (&Sc)[2]) {
      const int vb_prev = vb_cur == 0 ? 2 : vb_cur - 1;
      if (lag && pending) block_b(sV + vb_prev * TILE_BYTES);
      // Keys 32..63 of the last tile lie past every row of this wave (the lower half on a diagonal
      // tile): their probabilities are 0, so neither they nor their half of the PV product is computed.
      const int wave_lim = __builtin_amdgcn_readfirstlane(min(it.q_abs_min + QT - 1, a.Tk - 1));
      const bool lo_only = kt_cur * KT + KT / 2 > wave_lim;
      float ls;
      if (lo_only)
        probs(Sc, ls, std::integral_constant<int, 1>{});
      else
        probs(Sc, ls, std::integral_constant<int, 2>{});
      if (!ref_ok || __any(!(ls <= REFIT_SUM))) refit(Sc, ls);
      l_run += ls;
      if (!lag) {
        if (lo_only)
          block_pv(sV + vb_cur * TILE_BYTES, std::integral_constant<int, 1>{});
        else
          block_pv(sV + vb_cur * TILE_BYTES, std::integral_constant<int, 2>{});
      }
    };

    f32x16 Sn[2];
    if (has_cur) {
      bool odd = false;  // the last tile's scores are in Sn
      while (has_nxt) {
        step(std::integral_constant<int, 0>{}, S, Sn);
        if (!has_nxt) {
          odd = true;
          break;
        }
        step(std::integral_constant<int, 1>{}, Sn, S);
      }
      if (odd) {
        S[0] = Sn[0];
        S[1] = Sn[1];
      }
      tl_stamp(TL_LOOP);
      last_step(S);
      // Upper half: PV of the last tile.
      if (lag) block_pv(sV + vb_cur * TILE_BYTES, std::integral_constant<int, 2>{});
      vb_first = vb_cur == 2 ? 0 : vb_cur + 1;  // read by neither half in the last step
    }
    tl_stamp(TL_LAST);
    // O is staged in the wave's own Q slot (Q is in registers): no other wave touches it.
    epilogue(a, it, b, O, l_run, sQw, lane);
    tl_stamp(TL_EPILOGUE);
    tl_count(TL_ITEMS);
  }

  // Item index -> (qt, r, hs, b).  Per lane: v may differ between lanes (the startup reads two
  // items' offsets in two lanes).  Without row_order: query tiles latest first, all rows of a
  // tile together; with it: row by row (s_row_rank), latest query tiles first within a row.
  static __device__ __forceinline__ void decode_item(const PrefillArgs& a, int v, int& qt, int& r, int& hs, int& b) {
    uint32_t rem;
    if (a.row_order && v >= a.head_items) {
      const uint32_t w = (uint32_t)(v - a.head_items);
      const uint32_t k = fast_div(w, (uint32_t)a.per_group, a.mul_group);
      r = s_row_rank[k];
      const uint32_t rq = w - k * (uint32_t)a.per_group;
      const uint32_t t = fast_div(rq, (uint32_t)a.bhs, a.mul_bhs);
      qt = a.q_split - 1 - (int)t;
      rem = rq - t * (uint32_t)a.bhs;  // (hs, b) with hs fastest
    } else {
      const uint32_t t = fast_div((uint32_t)v, (uint32_t)a.per_tile, a.mul_tile);
      qt = a.ntq - 1 - (int)t;
      const uint32_t rt = (uint32_t)v - t * (uint32_t)a.per_tile;  // (r, hs, b) with r fastest
      const uint32_t t2 = fast_div(rt, (uint32_t)a.R, a.mul_R);
      r = (int)(rt - t2 * (uint32_t)a.R);
      rem = t2;
    }
    const uint32_t t3 = fast_div(rem, (uint32_t)a.head_splits, a.mul_hs);
    hs = (int)(rem - t3 * (uint32_t)a.head_splits);
    b = (int)t3;
  }

  // Ranks the CSR rows by retained blocks (descending, ties by row) into s_row_rank; callers
  // barrier before the first decode_item.
  static __device__ __forceinline__ void rank_rows(const PrefillArgs& a, int* s_len) {
    for (int r = threadIdx.x; r < a.R; r += NT) {
      const int32_t* o = a.offsets + r * a.offsets_stride;
      s_len[r] = o[a.nqb] - o[0];
    }
    __syncthreads();
    for (int r = threadIdx.x; r < a.R; r += NT) {
      const int len = s_len[r];
      int rank = 0;
      for (int u = 0; u < a.R; ++u) {
        const int lu = s_len[u];
        rank += (lu > len || (lu == len && u < r)) ? 1 : 0;
      }
      s_row_rank[rank] = r;
    }
  }

  // decode_item for an item index that is the same in every lane of the wave: the results are
  // moved to scalar registers, and so is every address derived from them.
  static __device__ __forceinline__ void decode_item_uniform(const PrefillArgs& a, int v, int& qt, int& r, int& hs,
                                                             int& b) {
    decode_item(a, __builtin_amdgcn_readfirstlane(v), qt, r, hs, b);
    qt = __builtin_amdgcn_readfirstlane(qt);
    r = __builtin_amdgcn_readfirstlane(r);
    hs = __builtin_amdgcn_readfirstlane(hs);
    b = __builtin_amdgcn_readfirstlane(b);
  }

  static __device__ __forceinline__ void process(const PrefillArgs& a, int v, char* sKV, char* sQ,
                                                 int32_t* s_row, int32_t* s_mask) {
    int qt, r, hs, b;
    decode_item_uniform(a, v, qt, r, hs, b);
    if constexpr (PIPE)
    {
      int vb_first = 0;
      item_pipelined<false>(a, qt, r, hs, b, sKV, sQ, s_row, s_mask, nullptr, vb_first);
    }
    else
      item(a, qt, r, hs, b, sKV, s_row, s_mask);
  }

  // Persistent four-head loop with lookahead.  Item i of this workgroup finds in LDS its id,
  // CSR offsets and (qt, r, hs, b) (slot i % 4 of s_meta) and its row (row cache i % 2), and
  // the id, offsets and row of item i + 1 and the id of item i + 2; its prologue fetches the
  // row of item i + 1, the offsets and (qt, r, hs, b) of item i + 2 and claims item i + 3
  // (Look).  Claims only grow, so the first id past the end ends the loop in every wave at
  // once.
  static __device__ __forceinline__ int run_lookahead(const PrefillArgs& a, int n_items, char* sKV, char* sQ,
                                                      int32_t* s_row, int32_t* s_mask) {
    int done = 0;      // items this workgroup processed
    int vb_first = 0;  // V buffer free for the next item's first tile
    // Per slot k = item index mod 4: id, CSR offsets (first, end) and (qt, r, hs, b); the loop
    // top reads an item's whole slot (and the ids and offsets of the next two) in one batch.
    __shared__ __attribute__((aligned(16))) int s_meta[4][8];
    const int tid = threadIdx.x;
    if (tid == 0) {
      const unsigned v0 = atomicAdd(&a.counter[WS_NEXT], 1u);
      const unsigned v1 = atomicAdd(&a.counter[WS_NEXT], 1u);
      const unsigned v2 = atomicAdd(&a.counter[WS_NEXT], 1u);
      s_meta[0][0] = (int)v0;
      s_meta[1][0] = (int)v1;
      s_meta[2][0] = (int)v2;
    }
    __syncthreads();
    if (tid < 2) {
      const int v = s_meta[tid][0];
      if (v < n_items) {
        int qt, r, hs, b;
        decode_item(a, v, qt, r, hs, b);
        const int32_t* o = a.offsets + r * a.offsets_stride + (qt >> a.qpb_log2);
        s_meta[tid][1] = o[0];
        s_meta[tid][2] = o[1];
        s_meta[tid][3] = qt;
        s_meta[tid][4] = r;
        s_meta[tid][5] = hs;
        s_meta[tid][6] = b;
      }
    }
    __syncthreads();
    {
      const int v = s_meta[0][0];
      const int e0 = s_meta[0][1], n = s_meta[0][2] - e0;
      if (v < n_items && n <= RC) {
        const int r = __builtin_amdgcn_readfirstlane(s_meta[0][4]);
        for (int x = tid; x < n; x += NT) {
          s_row[x] = a.pairs[r * a.pairs_stride + e0 + x];
          if (SUB) s_mask[x] = a.tile_masks[r * a.masks_stride + e0 + x];
        }
      }
    }
    __syncthreads();  // publishes the row cache of item 0
    for (int i = 0;; ++i) {
      tl_stamp(TL_LOOP_TOP);
      // The metadata of item i was published by item i - 1's barriers; the K/V buffers are
      // freed by the barrier in the item's prologue.  Values read from LDS are the same in
      // every lane; readfirstlane keeps them (and the addresses derived from them) in scalar
      // registers.
      const int k0 = i & 3, k1 = (i + 1) & 3, k2 = (i + 2) & 3;
      const int4 m0 = *reinterpret_cast<const int4*>(&s_meta[k0][0]);  // id, first, end, qt
      const int4 m0b = *reinterpret_cast<const int4*>(&s_meta[k0][4]);  // r, hs, b
      const int4 m1 = *reinterpret_cast<const int4*>(&s_meta[k1][0]);
      const int r1 = s_meta[k1][4];
      const int v2 = s_meta[k2][0];
      const int v = __builtin_amdgcn_readfirstlane(m0.x);
      if (v >= n_items) break;
      Look lk;
      lk.e0 = __builtin_amdgcn_readfirstlane(m0.y);
      lk.n_ent = __builtin_amdgcn_readfirstlane(m0.z) - lk.e0;
      lk.v1 = __builtin_amdgcn_readfirstlane(m1.x);
      lk.e0_1 = __builtin_amdgcn_readfirstlane(m1.y);
      lk.n_1 = __builtin_amdgcn_readfirstlane(m1.z) - lk.e0_1;
      lk.r_1 = __builtin_amdgcn_readfirstlane(r1);
      lk.v2 = __builtin_amdgcn_readfirstlane(v2);
      lk.n_items = n_items;
      lk.row_dst = s_row + ((i + 1) & 1) * RC;
      lk.mask_dst = SUB ? s_mask + ((i + 1) & 1) * RC : s_mask;
      lk.meta2 = &s_meta[k2][0];
      lk.vid3 = &s_meta[(i + 3) & 3][0];
      const int qt = __builtin_amdgcn_readfirstlane(m0.w);
      const int r = __builtin_amdgcn_readfirstlane(m0b.x);
      const int hs = __builtin_amdgcn_readfirstlane(m0b.y);
      const int b = __builtin_amdgcn_readfirstlane(m0b.z);
      item_pipelined<true>(a, qt, r, hs, b, sKV, sQ, s_row + (i & 1) * RC, SUB ? s_mask + (i & 1) * RC : s_mask,
                           &lk, vb_first);
      ++done;
    }
    return done;
  }

  static __device__ void run(const PrefillArgs& a) {
    __shared__ __attribute__((aligned(16))) char sKV[LDS_KV];
    __shared__ __attribute__((aligned(16))) char sQ[LDS_Q];
    // Row caches: two for the persistent four-head loop (this item and the next one).
    constexpr int NROW = PIPE ? 2 : 1;
    __shared__ int32_t s_row[NROW * RC];
    __shared__ int32_t s_mask[SUB ? NROW * RC : 1];  // sub-block masks of the cached rows
    __shared__ int s_item;
    const int n_items = a.ntq * a.R * a.B * a.head_splits;

    if (!a.counter) {
      // One workgroup per item.  Consecutive workgroups go to the 8 XCDs in turn; chunks of
      // XCD_CHUNK consecutive query tiles (all rows) are dealt to the XCDs round-robin so every
      // XCD gets an even share of each row's work, while neighbouring tiles (which share
      // window and global key blocks) stay in one XCD's L2.
      const int per_tile = a.R * a.B * a.head_splits;
      const int chunk = XCD_CHUNK * per_tile;
      const int xcd = blockIdx.x % N_XCD, seq = blockIdx.x / N_XCD;
      const int v = ((seq / chunk) * N_XCD + xcd) * chunk + seq % chunk;
      if (v >= n_items) return;  // padding workgroup of the last round
      process(a, v, sKV, sQ, s_row, s_mask);
      return;
    }

    // Persistent: claim items from a counter until none is left.  The last workgroup to
    // finish resets the counter pair to zero for the next launch on the stream.
    unsigned long long* rec = nullptr;  // TL: this workgroup's record
    if constexpr (TL) {
      rec = a.timeline + (int64_t)blockIdx.x * TL_WORDS;
      if (threadIdx.x == 0) {
        rec[0] = __builtin_amdgcn_s_memtime();
        rec[1] = __builtin_amdgcn_s_memrealtime();
      }
      if (threadIdx.x < 2 * TL_HALF_WORDS) s_tl[threadIdx.x / TL_HALF_WORDS][threadIdx.x % TL_HALF_WORDS] = 0;
      __syncthreads();
      const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
      if (wave % HW == 0 && (threadIdx.x & 63) == 0) s_tl[wave / HW][TL_NOW] = (unsigned)__builtin_amdgcn_s_memtime();
    }
    if (a.row_order) rank_rows(a, reinterpret_cast<int*>(sKV));  // K/V buffers are free here
    int done = 0;
    if constexpr (PIPE) {
      done = run_lookahead(a, n_items, sKV, sQ, s_row, s_mask);
      if constexpr (TL) {
        __syncthreads();  // every stamp is in LDS
        if (threadIdx.x == 0) {
          rec[2] = __builtin_amdgcn_s_memtime();
          rec[3] = __builtin_amdgcn_s_memrealtime();
        }
        if (threadIdx.x < 2 * TL_HALF_WORDS) rec[4 + threadIdx.x] = s_tl[threadIdx.x / TL_HALF_WORDS][threadIdx.x % TL_HALF_WORDS];
      }
    } else {
      for (;;) {
        if (threadIdx.x == 0) s_item = (int)atomicAdd(&a.counter[WS_NEXT], 1u);
        __syncthreads();
        const int v = s_item;
        __syncthreads();
        if (v >= n_items) break;
        process(a, v, sKV, sQ, s_row, s_mask);
        ++done;
      }
    }
    // Items processed, then this workgroup done; the last one checks the total and zeroes the
    // counters for the next launch on the stream.
    if (threadIdx.x == 0) {
      atomicAdd(&a.counter[WS_DONE_ITEMS], (unsigned)done);
      __threadfence();
      if (atomicAdd(&a.counter[WS_DONE_WG], 1u) == gridDim.x - 1) {
        __threadfence();
        if (atomicAdd(&a.counter[WS_DONE_ITEMS], 0u) != (unsigned)n_items) atomicOr(&a.counter[WS_STATUS], WS_SKIPPED);
        atomicExch(&a.counter[WS_NEXT], 0u);
        atomicExch(&a.counter[WS_DONE_ITEMS], 0u);
        atomicExch(&a.counter[WS_DONE_WG], 0u);
      }
    }
  }
};

// At most 256 registers per wave: two waves per SIMD (one 8-wave workgroup per CU).
template <bool BF16, int D, int HW, bool SUB>
__global__ __launch_bounds__(128 * HW) __attribute__((amdgpu_waves_per_eu(2)))
void prefill_kernel(PrefillArgs a) {
  Prefill<BF16, D, HW, SUB>::run(a);
}

// The timeline instantiation of the persistent four-head kernel (head dim 128, blocks of 64 or 128).
template <bool BF16>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2)))
void prefill_timeline_kernel(PrefillArgs a) {
  Prefill<BF16, 128, 4, false, true>::run(a);
}

// Resident workgroups of one kernel instance per CU, and CUs, cached per device.
template <bool BF16, int D, int HW, bool SUB>
static int resident_per_cu() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 1;
  if (!cached[dev]) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, prefill_kernel<BF16, D, HW, SUB>, 128 * HW, 0) != hipSuccess || n < 1)
      n = 1;
    cached[dev] = n;
  }
  return cached[dev];
}

static int num_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

template <bool BF16, int D, int HW, bool SUB>
static hipError_t launch_sub(const PrefillArgs& a, int64_t n_items, int64_t item_grid, hipStream_t s) {
  int64_t grid = item_grid;
  if (a.counter) grid = std::min<int64_t>(n_items, (int64_t)num_cus() * resident_per_cu<BF16, D, HW, SUB>());
  hipLaunchKernelGGL((prefill_kernel<BF16, D, HW, SUB>), dim3(grid), dim3(128 * HW), 0, s, a);
  return hipGetLastError();
}

template <bool BF16, int D, int HW>
static hipError_t launch_hw(const PrefillArgs& a, int64_t n_items, int64_t item_grid, hipStream_t s) {
  return a.sub_log2 ? launch_sub<BF16, D, HW, true>(a, n_items, item_grid, s)
                    : launch_sub<BF16, D, HW, false>(a, n_items, item_grid, s);
}

template <bool BF16, int D>
static hipError_t launch_d(const PrefillArgs& a, int hw, int64_t n_items, int64_t item_grid, hipStream_t s) {
  switch (hw) {
    case 4: return launch_hw<BF16, D, 4>(a, n_items, item_grid, s);
    case 2: return launch_hw<BF16, D, 2>(a, n_items, item_grid, s);
    default: return launch_hw<BF16, D, 1>(a, n_items, item_grid, s);
  }
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Workgroups of a timeline launch on the current device: one per resident slot.
static int64_t timeline_grid(bool bf16) {
  int n = 0;
  const hipError_t e = bf16 ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, prefill_timeline_kernel<true>, 512, 0)
                            : hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, prefill_timeline_kernel<false>, 512, 0);
  if (e != hipSuccess || n < 1) n = 1;
  return (int64_t)num_cus() * n;
}

static int prefill_impl(const char* fn, int dtype,
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
                        void* stream,
                        unsigned long long* timeline, int64_t timeline_words) {
  clear_error();
  if (dtype != SA_DTYPE_BF16 && dtype != SA_DTYPE_F16)
    return set_error(SA_E_DTYPE, "%s: dtype %d is not bf16 (0) or f16 (1)", fn, dtype);
  if (B < 0 || Hq < 1 || Hkv < 1 || T_q < 0 || T_k < 0)
    return set_error(SA_E_SHAPE, "%s: bad sizes B=%d Hq=%d Hkv=%d T_q=%d T_k=%d", fn, B, Hq, Hkv, T_q, T_k);
  if (Hq % Hkv)
    return set_error(SA_E_SHAPE, "%s: Hq=%d is not a multiple of Hkv=%d", fn, Hq, Hkv);
  if (D != 64 && D != 128)
    return set_error(SA_E_HEADDIM, "%s: head dim %d not supported (64, 128)", fn, D);
  if (block_size != 16 && block_size != 32 && block_size != 64 && block_size != 128)
    return set_error(SA_E_BLOCK, "%s: block size %d not supported (16, 32, 64, 128)", fn, block_size);
  const bool tiled = block_size < 64;  // schedule of 64 x 64 tiles with sub-block masks
  if (tiled != (tile_masks != nullptr))
    return set_error(SA_E_BLOCK, "%s: block size %d %s tile masks", fn, block_size,
                     tiled ? "needs" : "takes no");
  if (csr_rows != Hq && csr_rows != Hkv)
    return set_error(SA_E_CSR, "%s: csr_rows=%d must be Hq=%d or Hkv=%d", fn, csr_rows, Hq, Hkv);
  const int row_block = tiled ? 64 : block_size;  // query rows per CSR query block
  if (nqb != (int)ceil_div(T_q, row_block))
    return set_error(SA_E_SHAPE, "%s: nqb=%d but ceil(T_q/%d)=%lld", fn, nqb, row_block,
                     (long long)ceil_div(T_q, row_block));
  if (B == 0 || T_q == 0) return 0;
  if (!q || !k || !v || !o || !pairs || !offsets)
    return set_error(SA_E_NULL, "%s: NULL tensor pointer", fn);
  const int64_t strides[] = {q_sb, q_sh, q_st, k_sb, k_sh, k_st, v_sb, v_sh, v_st, o_sb, o_sh, o_st};
  for (int64_t s : strides)
    if (s % 8) return set_error(SA_E_ALIGN, "%s: stride %lld is not a multiple of 8 elements", fn, (long long)s);
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
    return set_error(SA_E_ALIGN, "%s: tensor base pointers must be 16-byte aligned", fn);
  if (k_st < 0 || v_st < 0 || k_st > MAX_KV_STRIDE || v_st > MAX_KV_STRIDE)
    return set_error(SA_E_SHAPE, "%s: K/V token strides %lld, %lld outside [0, %lld]", fn, (long long)k_st,
                     (long long)v_st, (long long)MAX_KV_STRIDE);

  PrefillArgs a;
  a.q = static_cast<const elem_t*>(q);
  a.k = static_cast<const elem_t*>(k);
  a.v = static_cast<const elem_t*>(v);
  a.o = static_cast<elem_t*>(o);
  a.q_sb = q_sb; a.q_sh = q_sh; a.q_st = q_st;
  a.k_sb = k_sb; a.k_sh = k_sh; a.k_st = k_st;
  a.v_sb = v_sb; a.v_sh = v_sh; a.v_st = v_st;
  a.o_sb = o_sb; a.o_sh = o_sh; a.o_st = o_st;
  a.pairs = pairs; a.pairs_stride = pairs_stride;
  a.offsets = offsets; a.offsets_stride = offsets_stride;
  a.tile_masks = tile_masks;
  a.masks_stride = tile_masks_stride;
  a.sub_log2 = block_size == 16 ? 4 : block_size == 32 ? 5 : 0;
  a.R = csr_rows;
  a.heads_per_row = Hq / csr_rows;
  const int hw = (a.heads_per_row % 4 == 0) ? 4 : (a.heads_per_row % 2 == 0) ? 2 : 1;
  a.head_splits = a.heads_per_row / hw;
  a.B = B; a.Hq = Hq; a.Hkv = Hkv; a.Tq = T_q; a.Tk = T_k;
  a.ntq = (int)ceil_div(T_q, QTILE);
  a.qpb_log2 = block_size == 128 ? 1 : 0;
  a.tpb_log2 = block_size == 128 ? 1 : 0;
  a.q_offset = q_offset;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  a.per_tile = a.R * B * a.head_splits;
  a.nqb = nqb;
  a.row_order = (workspace != nullptr && csr_rows <= MAX_ORDERED_ROWS) ? 1 : 0;
  a.bhs = B * a.head_splits;
  a.q_split = 0;
  if (a.row_order) {  // tail of about four items per persistent workgroup
    const int64_t tail = 4 * (int64_t)num_cus();
    a.q_split = (int)std::min<int64_t>(a.ntq, ceil_div(tail, a.per_tile));
  }
  a.head_items = (a.ntq - a.q_split) * a.per_tile;
  a.per_group = std::max(1, a.q_split * a.bhs);
  a.mul_group = div_mul((uint32_t)a.per_group);
  a.mul_bhs = div_mul((uint32_t)a.bhs);
  a.mul_tile = div_mul((uint32_t)a.per_tile);
  a.mul_R = div_mul((uint32_t)a.R);
  a.mul_hs = div_mul((uint32_t)a.head_splits);
  if (workspace && workspace_bytes < sa_prefill_workspace_bytes())
    return set_error(SA_E_WORKSPACE, "%s: workspace of %lld bytes, need %lld", fn, (long long)workspace_bytes,
                     (long long)sa_prefill_workspace_bytes());
  if (workspace && (reinterpret_cast<uintptr_t>(workspace) & 3))
    return set_error(SA_E_ALIGN, "%s: workspace must be 4-byte aligned", fn);
  a.counter = static_cast<unsigned int*>(workspace);

  const int64_t per_tile = (int64_t)a.R * B * a.head_splits;
  const int64_t n_items = (int64_t)a.ntq * per_tile;
  const int64_t chunk = XCD_CHUNK * per_tile;
  const int64_t item_grid = ceil_div(ceil_div(n_items, chunk), N_XCD) * N_XCD * chunk;
  if (item_grid > 0x7fffffff) return set_error(SA_E_SHAPE, "%s: %lld work items is too many", fn, (long long)n_items);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool bf16 = dtype == SA_DTYPE_BF16;
  hipError_t err;
  a.timeline = timeline;
  if (timeline) {
    if (!workspace || hw != 4 || D != 128 || tiled)
      return set_error(SA_E_SHAPE, "%s: the timeline instruments the persistent four-head kernel (a workspace, "
                       "four query heads per CSR row, head dim 128, block 64 or 128)", fn);
    const int64_t grid = std::min<int64_t>(n_items, timeline_grid(bf16));
    if (timeline_words < grid * TL_WORDS)
      return set_error(SA_E_WORKSPACE, "%s: timeline of %lld words, need %lld", fn, (long long)timeline_words,
                       (long long)(grid * TL_WORDS));
    if (bf16)
      hipLaunchKernelGGL((prefill_timeline_kernel<true>), dim3(grid), dim3(512), 0, s, a);
    else
      hipLaunchKernelGGL((prefill_timeline_kernel<false>), dim3(grid), dim3(512), 0, s, a);
    err = hipGetLastError();
  } else if (D == 128)
    err = bf16 ? launch_d<true, 128>(a, hw, n_items, item_grid, s) : launch_d<false, 128>(a, hw, n_items, item_grid, s);
  else
    err = bf16 ? launch_d<true, 64>(a, hw, n_items, item_grid, s) : launch_d<false, 64>(a, hw, n_items, item_grid, s);
  if (err != hipSuccess) return set_error((int)err, "%s: launch failed: %s", fn, hipGetErrorString(err));
  return 0;
}

}  // namespace sa

extern "C" int sa_prefill(int dtype,
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
                          void* stream) {
  return sa::prefill_impl("sa_prefill", dtype, q, q_sb, q_sh, q_st, k, k_sb, k_sh, k_st, v, v_sb, v_sh, v_st,
                          o, o_sb, o_sh, o_st, pairs, pairs_stride, offsets, offsets_stride, tile_masks,
                          tile_masks_stride, csr_rows, nqb, B, Hq, Hkv, T_q, T_k, D, block_size, q_offset,
                          sm_scale, workspace, workspace_bytes, stream, nullptr, 0);
}

extern "C" int sa_prefill_timeline(int dtype,
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
                                   void* stream) {
  sa::clear_error();
  if (!timeline) return sa::set_error(SA_E_NULL, "sa_prefill_timeline: NULL timeline");
  return sa::prefill_impl("sa_prefill_timeline", dtype, q, q_sb, q_sh, q_st, k, k_sb, k_sh, k_st, v, v_sb, v_sh,
                          v_st, o, o_sb, o_sh, o_st, pairs, pairs_stride, offsets, offsets_stride, nullptr, 0,
                          csr_rows, nqb, B, Hq, Hkv, T_q, T_k, D, block_size, q_offset, sm_scale, workspace,
                          workspace_bytes, stream, reinterpret_cast<unsigned long long*>(timeline),
                          timeline_words);
}

extern "C" int64_t sa_prefill_timeline_words(int dtype) {
  sa::clear_error();
  if (dtype != SA_DTYPE_BF16 && dtype != SA_DTYPE_F16)
    return sa::set_error(SA_E_DTYPE, "sa_prefill_timeline_words: dtype %d is not bf16 (0) or f16 (1)", dtype);
  return sa::timeline_grid(dtype == SA_DTYPE_BF16) * sa::TL_WORDS;
}

extern "C" int64_t sa_prefill_workspace_bytes(void) { return sa::WS_WORDS * (int64_t)sizeof(unsigned int); }
