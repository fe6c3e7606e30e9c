// Block-sparse causal attention over a CSR block schedule, gfx950 (CDNA4).
//
// Semantics follow the reference kernel kernels/triton/universal_sparse_attn.py:77-160:
// per query row, an online softmax over the keys of the retained blocks, masked by
// q_abs >= k and k < T_k, fp32 accumulation, probabilities rounded to the element
// type before the PV product, output acc / (l > 0 ? l : 1).
//
// Mapping onto the hardware:
//  * one workgroup = (batch b, CSR row r, 32-row query tile qt); one wave per query head
//    that shares row r (GQA: the Hq/Hkv heads of a KV group share every K/V tile staged
//    in LDS, so K/V are read once per group instead of once per head);
//  * at most 256 registers per wave and ~75 KiB of LDS per workgroup, so two workgroups
//    share a CU: one's load latency (Q, the first K/V tile, the CSR row) and epilogue
//    overlap the other's compute, and two waves per SIMD let one wave's softmax (VALU)
//    run under the other's matrix instructions;
//  * per wave and 64-key tile: S^T = K Q^T and O^T = V^T P^T on v_mfma_f32_32x32x16.
//    Computing the transposed products puts one query row in each lane column, so the
//    softmax statistics, the rescale of O and the P operand of the second product all
//    stay in the lane that owns the row;
//  * K rows are staged in LDS in a permuted order (krow) that makes each lane half of the
//    S^T accumulator hold 8 consecutive keys per 16-key chunk; V is staged transposed
//    ([d][key]), so the A operand of O^T = V^T P^T is one 16-byte LDS read per lane; the
//    staging writes and the fragment reads of both layouts are bank-conflict free;
//  * K/V tiles are double-buffered in LDS: the next tile is fetched into registers while
//    the current one is computed, with one barrier per tile;
//  * the softmax works in base 2 with scale*log2(e) folded into one FMA before the
//    hardware v_exp_f32 (2^x); the row reference max is only raised (and O rescaled) when
//    a row max exceeds it by more than 2^8, so the common case never touches O with VALU.
//
// MFMA 32x32x16 lane layouts used (l = lane, g = l / 32):
//   A (32 x 16): lane l holds row l % 32, k = 8g .. 8g+7
//   B (16 x 32): lane l holds column l % 32, k = 8g .. 8g+7
//   D (32 x 32): lane l, register r holds row 8(r/4) + 4g + r%4, column l % 32
// With K rows permuted by krow, register r = 8h + e of the 32-key half j of S^T holds
// key 32j + 16h + 8g + e.
#include <algorithm>

#include "sa_common.h"

namespace sa {

constexpr int QT = 32;           // query rows per wave
constexpr int QTILE = 64;        // query rows per work item (two waves per query head)
constexpr int KT = 64;           // keys per K/V tile
constexpr int ROW_CACHE = 1024;  // CSR entries of one row cached in LDS
constexpr int N_XCD = 8;         // XCDs of an MI355X; workgroups are dealt to them in turn
constexpr int XCD_CHUNK = 4;     // query tiles per chunk dealt to one XCD

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
  int R;             // CSR rows
  int heads_per_row; // query heads that read one CSR row
  int head_splits;   // heads_per_row / waves per workgroup
  int B, Hq, Hkv, Tq, Tk;
  int ntq;           // 64-row query tiles
  int qpb_log2;      // log2(block_size / 64): query tiles per CSR block
  int tpb_log2;      // log2(block_size / 64): key tiles per CSR block
  int q_offset;
  float scale_log2;  // sm_scale * log2(e)
  unsigned int* counter;  // persistent mode: 2 zeroed counters (next item, finished workgroups)
};

template <bool BF16, int D, int HW>
struct Prefill {
  using E = Elem<BF16>;
  static constexpr int NW = 2 * HW;         // waves: HW query heads x two 32-row halves
  static constexpr int NT = 64 * NW;        // threads
  static constexpr int KS = D + 8;          // sK row stride (elements), 16 B pad
  static constexpr int VS = KT + 8;         // sVt row stride (elements), 16 B pad
  static constexpr int DC = D / 8;          // 16-byte chunks per row
  static constexpr int K_TOTAL = KT * DC;        // 16-byte K chunks per tile
  static constexpr int V_TOTAL = DC * (KT / 4);  // V units (4 keys x 8 d) per tile
  static constexpr int KCH = (K_TOTAL + NT - 1) / NT;
  static constexpr int VUN = (V_TOTAL + NT - 1) / NT;
  // Double-buffer and prefetch the next tile into registers during compute when that costs
  // at most 32 VGPRs; one-wave workgroups single-buffer and stage after compute.
  static constexpr bool PREFETCH = (KCH + 4 * VUN) <= 8;
  static constexpr int NBUF = PREFETCH ? 2 : 1;
  static constexpr float RESCALE_LOG2 = 8.f;

  // LDS row of key k within a tile: bits 2 and 3 swapped.  With this order the S^T
  // accumulator gives each lane half 8 consecutive keys per 16-key chunk, so the matching
  // V^T operand is one contiguous 16-byte LDS read.
  static __device__ __forceinline__ int krow(int k) {
    return (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1);
  }

  struct Stage {
    u32x4 kr[KCH];
    u32x4 vr[VUN][4];
  };

  // Rows past T_k read row T_k - 1: their scores are masked and their probabilities are 0.
  static __device__ __forceinline__ void load(Stage& st, const elem_t* kb, const elem_t* vb,
                                              const PrefillArgs& a, int kt, int tid) {
#pragma unroll
    for (int u = 0; u < KCH; ++u) {
      const int c = tid + u * NT;
      if (K_TOTAL % NT && c >= K_TOTAL) break;
      const int key = c / DC, dc = c % DC;
      const int tok = min(kt * KT + key, a.Tk - 1);
      st.kr[u] = *reinterpret_cast<const u32x4*>(kb + tok * a.k_st + dc * 8);
    }
#pragma unroll
    for (int u = 0; u < VUN; ++u) {
      const int c = tid + u * NT;
      if (V_TOTAL % NT && c >= V_TOTAL) break;
      const int kg = c % (KT / 4), dc = c / (KT / 4);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int tok = min(kt * KT + 4 * kg + kk, a.Tk - 1);
        st.vr[u][kk] = *reinterpret_cast<const u32x4*>(vb + tok * a.v_st + dc * 8);
      }
    }
  }

  static __device__ __forceinline__ void store(const Stage& st, elem_t* sK, elem_t* sVt, int tid) {
#pragma unroll
    for (int u = 0; u < KCH; ++u) {
      const int c = tid + u * NT;
      if (K_TOTAL % NT && c >= K_TOTAL) break;
      const int key = c / DC, dc = c % DC;
      *reinterpret_cast<u32x4*>(sK + krow(key) * KS + dc * 8) = st.kr[u];
    }
#pragma unroll
    for (int u = 0; u < VUN; ++u) {
      const int c = tid + u * NT;
      if (V_TOTAL % NT && c >= V_TOTAL) break;
      const int kg = c % (KT / 4), dc = c / (KT / 4);
#pragma unroll
      for (int w = 0; w < 4; ++w) {  // d = dc*8 + 2w (low halves) and 2w+1 (high halves)
        const uint32_t x0 = st.vr[u][0][w], x1 = st.vr[u][1][w];
        const uint32_t x2 = st.vr[u][2][w], x3 = st.vr[u][3][w];
        const u32x2 even = {(x0 & 0xffffu) | (x1 << 16), (x2 & 0xffffu) | (x3 << 16)};
        const u32x2 odd = {(x0 >> 16) | (x1 & 0xffff0000u), (x2 >> 16) | (x3 & 0xffff0000u)};
        *reinterpret_cast<u32x2*>(sVt + (dc * 8 + 2 * w) * VS + 4 * kg) = even;
        *reinterpret_cast<u32x2*>(sVt + (dc * 8 + 2 * w + 1) * VS + 4 * kg) = odd;
      }
    }
  }

  // Online softmax over the 32-key half j of the current tile for this wave's 32 rows.
  // Scores are raw; p = 2^(s*c - m_ref).  Returns the P^T operands of the two 16-key chunks.
  template <bool MASK>
  static __device__ __forceinline__ void softmax_half(f32x16& S, u32x4 (&P)[2], f32x16 (&O)[D / 32],
                                                      float& m_ref, float& l_run, float c, int lim, int j) {
    if (MASK) {
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) {
        const int key = 32 * j + 16 * (rr >> 3) + (rr & 7);  // minus 8g, folded into lim
        if (key > lim) S[rr] = -__builtin_inff();
      }
    }
    float mx = S[0];
#pragma unroll
    for (int rr = 1; rr < 16; ++rr) mx = fmaxf(mx, S[rr]);
    mx = fmaxf(mx, swap_halves(mx));
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
      elem_t pe[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float p = fast_exp2(fmaf(S[8 * h + e], c, neg_m));
        ls += p;
        pe[e] = E::from_f32(p);
      }
      P[h] = u32x4{pack2(pe[0], pe[1]), pack2(pe[2], pe[3]), pack2(pe[4], pe[5]), pack2(pe[6], pe[7])};
    }
    l_run += ls;
  }

  // One 64-key tile: S^T = K Q^T per 32-key half, softmax, O^T += V^T P^T.  The softmax of
  // one half can run under the matrix instructions of the other half.
  template <bool MASK>
  static __device__ __forceinline__ void tile(const elem_t* cK, const elem_t* cV, const u32x4 (&qf)[D / 16],
                                              f32x16 (&O)[D / 32], float& m_ref, float& l_run, float c,
                                              int lim, int l32, int g) {
    // The two key halves are independent accumulation chains; alternating them keeps the
    // matrix pipe busy while each MFMA waits for its predecessor's result.
    f32x16 S[2] = {f32x16{}, f32x16{}};
#pragma unroll
    for (int cc = 0; cc < D / 16; ++cc) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const u32x4 kf = *reinterpret_cast<const u32x4*>(cK + (32 * j + l32) * KS + 16 * cc + 8 * g);
        S[j] = E::mfma32(kf, qf[cc], S[j]);
      }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      u32x4 P[2];
      softmax_half<MASK>(S[j], P, O, m_ref, l_run, c, lim, j);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int kbase = 32 * j + 16 * h + 8 * g;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
          const u32x4 vf = *reinterpret_cast<const u32x4*>(cV + (32 * dt + l32) * VS + kbase);
          O[dt] = E::mfma32(vf, P[h], O[dt]);
        }
      }
    }
  }

  // Processes one work item: query tile qt (64 rows) of CSR row r, batch b, head split hs.
  // Each wave owns 32 rows (half hf) of one query head; every K/V tile staged in LDS feeds
  // all NW waves.  s_row must not be in use by other waves (callers barrier before).
  static __device__ __forceinline__ void item(const PrefillArgs& a, int qt, int r, int hs, int b,
                                              elem_t (*sK)[KT * KS], elem_t (*sVt)[D * VS],
                                              int32_t* s_row) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int g = lane >> 5;
    const int l32 = lane & 31;
    const int hw = wave % HW;        // head within the workgroup
    const int hf = wave / HW;        // 32-row half of the query tile
    const int hq = r * a.heads_per_row + hs * HW + hw;
    const int kvh = (r * a.heads_per_row + hs * HW) / (a.Hq / a.Hkv);  // shared by the waves

    const elem_t* qb = a.q + b * a.q_sb + hq * a.q_sh;
    const elem_t* kb = a.k + b * a.k_sb + kvh * a.k_sh;
    const elem_t* vb = a.v + b * a.v_sb + kvh * a.v_sh;

    // CSR row of this query tile, cached in LDS; each block holds 2^tpb_log2 key tiles.
    const int qblk = qt >> a.qpb_log2;
    const int32_t* offs = a.offsets + r * a.offsets_stride;
    const int32_t* prow = a.pairs + r * a.pairs_stride;
    const int e0 = offs[qblk];
    const int n_ent = offs[qblk + 1] - e0;
    const bool cached = n_ent <= ROW_CACHE;
    if (cached)
      for (int x = tid; x < n_ent; x += NT) s_row[x] = prow[e0 + x];
    const int n_tiles = n_ent << a.tpb_log2;
    const int tpb_mask = (1 << a.tpb_log2) - 1;
    const int q_tile0 = qt * QTILE;
    const int q_row0 = q_tile0 + QT * hf;            // this wave's first row
    const int q_abs_tile_max = a.q_offset + min(a.Tq, q_tile0 + QTILE) - 1;
    const int q_abs_min = a.q_offset + q_row0;       // this wave's first absolute position

    // Q^T as the B operand of S^T = K Q^T: lane holds row l32, d = 16c + 8g .. +7.
    // Rows past T_q read a clamped (valid) row; their outputs are never stored.
    u32x4 qf[D / 16];
    {
      const int row = min(q_row0 + l32, a.Tq - 1);
#pragma unroll
      for (int c = 0; c < D / 16; ++c)
        qf[c] = *reinterpret_cast<const u32x4*>(qb + row * a.q_st + 16 * c + 8 * g);
    }
    __syncthreads();  // s_row visible

    auto tile_of = [&](int t) {
      const int e = t >> a.tpb_log2;
      const int blk = cached ? s_row[e] : prow[e0 + e];
      return (blk << a.tpb_log2) + (t & tpb_mask);
    };
    // Tiles entirely past T_k or above the causal limit of the whole 64-row tile contribute
    // nothing; negative ids (malformed schedules) are skipped rather than read.
    auto next_usable = [&](int t) {
      for (; t < n_tiles; ++t) {
        const int kt = tile_of(t);
        if (kt >= 0 && kt * KT < a.Tk && kt * KT <= q_abs_tile_max) break;
      }
      return t;
    };

    f32x16 O[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) O[dt] = f32x16{};
    float m_ref = -__builtin_inff();
    float l_run = 0.f;  // this lane's half of the row sum
    const float c = a.scale_log2;

    Stage st;
    int t = next_usable(0);
    int buf = 0;
    if (t < n_tiles) {
      load(st, kb, vb, a, tile_of(t), tid);
      store(st, sK[0], sVt[0], tid);
    }
    __syncthreads();

    while (t < n_tiles) {
      const int kt = tile_of(t);
      const int tn = next_usable(t + 1);
      if (PREFETCH && tn < n_tiles) load(st, kb, vb, a, tile_of(tn), tid);
      const elem_t* cK = sK[buf];
      const elem_t* cV = sVt[buf];

      // A wave whose 32 rows all precede the tile skips it (the other half may not).
      if (kt * KT <= q_abs_min + QT - 1) {
        const bool need_mask = (kt * KT + KT - 1 > q_abs_min) || (kt * KT + KT > a.Tk);
        const int lim = min(q_abs_min + l32, a.Tk - 1) - kt * KT - 8 * g;
        if (need_mask)
          tile<true>(cK, cV, qf, O, m_ref, l_run, c, lim, l32, g);
        else
          tile<false>(cK, cV, qf, O, m_ref, l_run, c, lim, l32, g);
      }

      if (tn < n_tiles) {
        if (PREFETCH) {
          store(st, sK[buf ^ 1], sVt[buf ^ 1], tid);
        } else {
          __syncthreads();  // single buffer: every wave is done reading it
          Stage st2;
          load(st2, kb, vb, a, tile_of(tn), tid);
          store(st2, sK[0], sVt[0], tid);
        }
      }
      __syncthreads();
      if (PREFETCH) buf ^= 1;
      t = tn;
    }

    // ---- epilogue: O / l, one row per lane column ---------------------------------------
    const float lt = l_run + swap_halves(l_run);
    const float inv = lt > 0.f ? 1.f / lt : 1.f;
    const int row = q_row0 + l32;
    if (row < a.Tq) {
      elem_t* orow = a.o + b * a.o_sb + hq * a.o_sh + row * a.o_st;
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const int d0 = 32 * dt + 8 * rq + 4 * g;
          const u32x2 w = {pack2(E::from_f32(O[dt][4 * rq] * inv), E::from_f32(O[dt][4 * rq + 1] * inv)),
                           pack2(E::from_f32(O[dt][4 * rq + 2] * inv), E::from_f32(O[dt][4 * rq + 3] * inv))};
          *reinterpret_cast<u32x2*>(orow + d0) = w;
        }
    }
  }

  // Item index -> (qt, r, hs, b), the heaviest (latest) query tiles first.
  static __device__ __forceinline__ void decode_item(const PrefillArgs& a, int v, int& qt, int& r, int& hs, int& b) {
    const int per_tile = a.R * a.B * a.head_splits;
    qt = a.ntq - 1 - v / per_tile;
    int rem = v % per_tile;
    r = rem % a.R;
    rem /= a.R;
    hs = rem % a.head_splits;
    b = rem / a.head_splits;
  }

  static __device__ void run(const PrefillArgs& a) {
    __shared__ __attribute__((aligned(16))) elem_t sK[NBUF][KT * KS];
    __shared__ __attribute__((aligned(16))) elem_t sVt[NBUF][D * VS];
    __shared__ int32_t s_row[ROW_CACHE];
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
      int qt, r, hs, b;
      decode_item(a, v, qt, r, hs, b);
      item(a, qt, r, hs, b, sK, sVt, s_row);
      return;
    }

    // Persistent: claim items from a counter until none is left.  The last workgroup to
    // finish resets the counter pair to zero for the next launch on the stream.
    for (;;) {
      if (threadIdx.x == 0) s_item = (int)atomicAdd(&a.counter[0], 1u);
      __syncthreads();
      const int v = s_item;
      __syncthreads();
      if (v >= n_items) break;
      int qt, r, hs, b;
      decode_item(a, v, qt, r, hs, b);
      item(a, qt, r, hs, b, sK, sVt, s_row);
    }
    if (threadIdx.x == 0 && atomicAdd(&a.counter[1], 1u) == gridDim.x - 1) {
      atomicExch(&a.counter[0], 0u);
      atomicExch(&a.counter[1], 0u);
    }
  }
};

// At most 256 registers per wave: two waves per SIMD (one 8-wave workgroup per CU).
template <bool BF16, int D, int HW>
__global__ __launch_bounds__(128 * HW) __attribute__((amdgpu_waves_per_eu(2)))
void prefill_kernel(PrefillArgs a) {
  Prefill<BF16, D, HW>::run(a);
}

// Resident workgroups of one kernel instance per CU, and CUs, cached per device.
template <bool BF16, int D, int HW>
static int resident_per_cu() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 1;
  if (!cached[dev]) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, prefill_kernel<BF16, D, HW>, 128 * HW, 0) != hipSuccess || n < 1)
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

template <bool BF16, int D, int HW>
static hipError_t launch_hw(const PrefillArgs& a, int64_t n_items, int64_t item_grid, hipStream_t s) {
  int64_t grid = item_grid;
  if (a.counter) grid = std::min<int64_t>(n_items, (int64_t)num_cus() * resident_per_cu<BF16, D, HW>());
  hipLaunchKernelGGL((prefill_kernel<BF16, D, HW>), dim3(grid), dim3(128 * HW), 0, s, a);
  return hipGetLastError();
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

}  // namespace sa

extern "C" int sa_prefill(int dtype,
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
                          void* stream) {
  using namespace sa;
  clear_error();
  if (dtype != SA_DTYPE_BF16 && dtype != SA_DTYPE_F16)
    return set_error(SA_E_DTYPE, "sa_prefill: dtype %d is not bf16 (0) or f16 (1)", dtype);
  if (B < 0 || Hq < 1 || Hkv < 1 || T_q < 0 || T_k < 0)
    return set_error(SA_E_SHAPE, "sa_prefill: bad sizes B=%d Hq=%d Hkv=%d T_q=%d T_k=%d", B, Hq, Hkv, T_q, T_k);
  if (Hq % Hkv)
    return set_error(SA_E_SHAPE, "sa_prefill: Hq=%d is not a multiple of Hkv=%d", Hq, Hkv);
  if (D != 64 && D != 128)
    return set_error(SA_E_HEADDIM, "sa_prefill: head dim %d not supported (64, 128)", D);
  if (block_size != 64 && block_size != 128)
    return set_error(SA_E_BLOCK, "sa_prefill: block size %d not supported (64, 128)", block_size);
  if (csr_rows != Hq && csr_rows != Hkv)
    return set_error(SA_E_CSR, "sa_prefill: csr_rows=%d must be Hq=%d or Hkv=%d", csr_rows, Hq, Hkv);
  if (nqb != (int)ceil_div(T_q, block_size))
    return set_error(SA_E_SHAPE, "sa_prefill: nqb=%d but ceil(T_q/block)=%lld", nqb,
                     (long long)ceil_div(T_q, block_size));
  if (B == 0 || T_q == 0) return 0;
  if (!q || !k || !v || !o || !pairs || !offsets)
    return set_error(SA_E_NULL, "sa_prefill: NULL tensor pointer");
  const int64_t strides[] = {q_sb, q_sh, q_st, k_sb, k_sh, k_st, v_sb, v_sh, v_st, o_sb, o_sh, o_st};
  for (int64_t s : strides)
    if (s % 8) return set_error(SA_E_ALIGN, "sa_prefill: stride %lld is not a multiple of 8 elements", (long long)s);
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
    return set_error(SA_E_ALIGN, "sa_prefill: tensor base pointers must be 16-byte aligned");

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
  if (workspace && workspace_bytes < sa_prefill_workspace_bytes())
    return set_error(SA_E_WORKSPACE, "sa_prefill: workspace of %lld bytes, need %lld", (long long)workspace_bytes,
                     (long long)sa_prefill_workspace_bytes());
  if (workspace && (reinterpret_cast<uintptr_t>(workspace) & 3))
    return set_error(SA_E_ALIGN, "sa_prefill: workspace must be 4-byte aligned");
  a.counter = static_cast<unsigned int*>(workspace);

  const int64_t per_tile = (int64_t)a.R * B * a.head_splits;
  const int64_t n_items = (int64_t)a.ntq * per_tile;
  const int64_t chunk = XCD_CHUNK * per_tile;
  const int64_t item_grid = ceil_div(ceil_div(n_items, chunk), N_XCD) * N_XCD * chunk;
  if (item_grid > 0x7fffffff) return set_error(SA_E_SHAPE, "sa_prefill: %lld work items is too many", (long long)n_items);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool bf16 = dtype == SA_DTYPE_BF16;
  hipError_t err;
  if (D == 128)
    err = bf16 ? launch_d<true, 128>(a, hw, n_items, item_grid, s) : launch_d<false, 128>(a, hw, n_items, item_grid, s);
  else
    err = bf16 ? launch_d<true, 64>(a, hw, n_items, item_grid, s) : launch_d<false, 64>(a, hw, n_items, item_grid, s);
  if (err != hipSuccess) return set_error((int)err, "sa_prefill: launch failed: %s", hipGetErrorString(err));
  return 0;
}

extern "C" int64_t sa_prefill_workspace_bytes(void) { return 2 * (int64_t)sizeof(unsigned int); }
