// Sparse decode: one query token per sequence over the retained KV blocks of a
// (paged or contiguous) cache, gfx950.  Memory-bound: no MFMA.
//
// Semantics: the query is the newest token, so every cached key below kv_len of a
// retained block is visible (the decode row of the causal mask,
// sparse_attentions/attention/masked_sdpa.py:42-46; universal_sparse_attn.py:203-205);
// softmax with fp32 statistics; a sequence/head with no visible key yields 0.
//
// Mapping:
//  * one unit (4 waves) = (sequence b, schedule row r, split s): the NH query
//    heads that read row r share every K/V load (GQA: one read per KV group); a
//    workgroup runs one unit, or two (8 waves) once there are two units per CU;
//  * a wave streams whole rounds of a retained block: each lane loads 16-byte
//    chunks (8 head-dim elements) of K and V, D/8 consecutive lanes cover one key
//    row, so a load instruction reads 64/(D/8) full rows back to back;
//  * q.k partial dots are reduced across the D/8 lanes of a row with xor-shuffles;
//    the online softmax keeps (m, l, acc) per head; waves merge through LDS, and
//    splits (num_splits > 1) merge in decode_combine_kernel.
#include <mutex>

#include "sa_common.h"

namespace sa {

struct DecodeArgs {
  const elem_t* q;
  int64_t q_sb, q_sh;
  const elem_t* k;
  const elem_t* v;
  int64_t kv_sb, kv_sh, kv_st;
  const int32_t* block_table;
  int64_t bt_stride;
  int max_blocks;  // columns of block_table
  int num_pages;   // pages in each pool
  const int32_t* kv_lens;
  int kv_len;
  const int32_t* sel;
  int64_t sel_sb, sel_sr;
  const int32_t* sel_off;
  int64_t off_sb, off_sr;
  int rows, heads_per_row, head_splits;
  elem_t* o;
  int64_t o_sb, o_sh;
  float* part;  // [splits][B][Hq][D + 2] when num_splits > 1
  int B, Hq, Hkv, page, num_splits;
  float scale_log2;
  // Divisions by launch constants done by multiply-high (fast_div), multipliers from the host:
  // the workgroup index by num_splits, rows and head_splits, a head by the group size
  // kv_group = Hq / Hkv, key counts by page, and round indices by the rounds per retained
  // block rpb = ceil(page / keys per round).
  int kv_group, rpb;
  uint32_t mul_splits, mul_rows, mul_hs, mul_group, mul_page, mul_rpb;
};

constexpr int DEC_WAVES = 4;
constexpr int DEC_NI = 4;        // 16-byte loads of K (and of V) per lane per round
constexpr int DEC_CACHE = 512;   // retained blocks of a workgroup staged in LDS (longer lists read HBM)

// Keys one round of a wave covers at head dim D: DEC_NI loads of 64 / (D / 8) key rows.
constexpr int dec_keys_per_round(int D) { return DEC_NI * (64 / (D / 8)); }

// x as held by the lane that DPP control CTRL selects (quad permutes, row mirrors: within 16 lanes).
template <int CTRL>
__device__ __forceinline__ float dpp_get(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

// Sum over the LPR (8 or 16) consecutive lanes of one key row; every lane of the row receives it.
template <int LPR>
__device__ __forceinline__ float row_sum(float x) {
  static_assert(LPR == 8 || LPR == 16, "key rows span 8 or 16 lanes");
  x += dpp_get<0xB1>(x);   // quad_perm [1,0,3,2]: lane pairs
  x += dpp_get<0x4E>(x);   // quad_perm [2,3,0,1]: quads
  x += dpp_get<0x141>(x);  // row_half_mirror (lane i <-> 7 - i): the two quads of 8 lanes
  if constexpr (LPR == 16) x += dpp_get<0x140>(x);  // row_mirror (lane i <-> 15 - i): the two halves
  return x;
}

// Max (MAX) or sum of x over the lanes that differ from this one only in lane bits log2(LPR)..5,
// i.e. over the key rows of a round, in every lane and without an LDS round trip: xor 8 by a DPP
// row rotation (LPR 8), then xor 16 and xor 32 by v_permlane16_swap / v_permlane32_swap of the
// value with itself, whose two results hold the values of the two lanes.  The steps and the pairs
// they combine are those of __shfl_xor by 8, 16, 32, so the results are the same bits.
template <int LPR, bool MAX>
__device__ __forceinline__ float over_rows(float x) {
  static_assert(LPR == 8 || LPR == 16, "key rows span 8 or 16 lanes");
  auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
  if constexpr (LPR == 8) x = op(x, dpp_get<0x128>(x));  // row_ror:8: lane i <-> i ^ 8 within its row
  const auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = op(__uint_as_float(s16[0]), __uint_as_float(s16[1]));
  const auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return op(__uint_as_float(s32[0]), __uint_as_float(s32[1]));
}

// 32-bit global read that has completed when it returns: written as one opaque block, so the
// compiler's count of outstanding loads (and its waits for the K/V rounds) never includes it.
__device__ __forceinline__ int32_t load_now(const int32_t* p) {
  int32_t x;
  asm volatile(
      "global_load_dword %0, %1, off\n\t"
      "s_waitcnt vmcnt(0)"
      : "=v"(x)
      : "v"(p)
      : "memory");
  return x;
}

// Block-table entry of logical block lb of sequence b, or NULL where the block has no keys below
// L or lies past the table's max_blocks columns.
__device__ __forceinline__ const int32_t* table_slot(const DecodeArgs& a, int b, int lb, int L) {
  if (lb < 0 || lb >= a.max_blocks || (int64_t)lb * a.page >= L) return nullptr;
  return a.block_table + b * a.bt_stride + lb;
}

// Page of logical block lb of sequence b in a paged cache, or -1 where the block has no keys
// below L, lies past the table's max_blocks columns, or maps outside the pool: such blocks load
// nothing.  NOW: read the table with load_now (inside the round loop).
template <bool NOW = false>
__device__ __forceinline__ int page_of(const DecodeArgs& a, int b, int lb, int L) {
  const int32_t* t = table_slot(a, b, lb, L);
  if (!t) return -1;
  const int pg = NOW ? load_now(t) : *t;
  return (pg >= 0 && pg < a.num_pages) ? pg : -1;
}

template <bool BF16, int D, int NH>
struct Decode {
  using E = Elem<BF16>;
  static constexpr int LPR = D / 8;        // lanes per key row
  static constexpr int KPI = 64 / LPR;     // key rows per load instruction
  static constexpr int CH = dec_keys_per_round(D);  // keys per round
  static_assert(CH == DEC_NI * KPI, "keys per round");

  // One round of a wave: DEC_NI key rows of K and of V per lane, and the valid key count.
  struct Round {
    u32x4 k[DEC_NI], v[DEC_NI];
    int nk;
  };

  struct Ctx {
    const int32_t* s_blk;  // staged logical blocks (when cached)
    const int32_t* s_pg;   // staged pages (paged caches)
    const int32_t* selp;   // the global list (when not cached)
    const elem_t* safe;    // 16 readable, finite bytes per lane (the query): loads of keys past nk
    int lo, b, kvh, L, rpb, kg, dc;
    uint32_t mul_rpb;
    uint32_t nb;           // blocks holding keys below L: ids at or past it (or negative) have none
    int n_it;              // rounds of the workgroup; rounds past it are dead (nk = 0)
    bool cached;
  };

  // Logical block lb and page pg of round `it` (entry it / rpb of the list; lb = -1 for rounds
  // past the list).  Lists longer than the LDS stage: the entry and its page are read from
  // global memory with load_now (each waits for every load issued before it).
  static __device__ __forceinline__ void entry(const DecodeArgs& a, const Ctx& c, int it, int& lb, int& pg) {
    const int x = (int)fast_div((uint32_t)it, (uint32_t)c.rpb, c.mul_rpb);  // it >= 0
    pg = 0;
    if (it >= c.n_it) {
      lb = -1;
    } else if (c.cached) {
      lb = c.s_blk[x];
      pg = c.s_pg[x];
    } else {
      lb = load_now(c.selp + c.lo + x);
      if (a.block_table) {
        pg = page_of<true>(a, c.b, lb, c.L);
        if (pg < 0) lb = -1;
      }
    }
  }

  static __device__ __forceinline__ void issue(const DecodeArgs& a, const Ctx& c, int it, Round& R) {
    int lb, pg;
    entry(a, c, it, lb, pg);
    issue_at(a, c, it, lb, pg, R);
  }

  // Loads round `it` of the workgroup's list: keys k0 .. k0 + CH - 1 of logical block lb (page pg).
  // Blocks past kv_len or with negative ids, and rounds past the list, have no keys (nk = 0).
  static __device__ __forceinline__ void issue_at(const DecodeArgs& a, const Ctx& c, int it, int lb, int pg,
                                                  Round& R) {
    const int x = (int)fast_div((uint32_t)it, (uint32_t)c.rpb, c.mul_rpb);  // it >= 0
    const int k0 = (it - x * c.rpb) * CH;
    lb = __builtin_amdgcn_readfirstlane(lb);
    pg = __builtin_amdgcn_readfirstlane(pg);
    // one unsigned test for negative ids and ids at or past the last block (no lb * page overflow)
    const int nk = (uint32_t)lb >= c.nb ? 0 : max(0, min(min(CH, a.page - k0), c.L - lb * a.page - k0));
    R.nk = nk;
    const elem_t* kb;
    const elem_t* vb;
    if (a.block_table) {
      const int64_t base = (int64_t)pg * a.kv_sb + c.kvh * a.kv_sh + (int64_t)k0 * a.kv_st;
      kb = a.k + base;
      vb = a.v + base;
    } else {
      const int64_t base = c.b * a.kv_sb + c.kvh * a.kv_sh + ((int64_t)lb * a.page + k0) * a.kv_st;
      kb = a.k + base;
      vb = a.v + base;
    }
    // Every lane issues all its loads (lanes past nk read c.safe, and compute() masks their
    // scores), so the compiler's wait before the round is computed covers exactly the loads
    // issued before it and leaves the next round's loads in flight.  The loads are
    // non-temporal: K/V are read once per step, and reads that do not allocate in the Infinity
    // Cache leave more of HBM's bandwidth to the stream (a cache-cold step: 42.4 against 47.7 us
    // at 236 MB per launch).  All K loads go before the V loads, so the scores of a round wait
    // only for its K (configs[3]: 41.01-41.16 against 41.12-41.36 us with K and V interleaved).
#pragma unroll
    for (int i = 0; i < DEC_NI; ++i) {
      const int key = c.kg + KPI * i;
      const elem_t* pk = key < nk ? kb + key * a.kv_st + c.dc * 8 : c.safe;
      R.k[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(pk));
    }
#pragma unroll
    for (int i = 0; i < DEC_NI; ++i) {
      const int key = c.kg + KPI * i;
      const elem_t* pv = key < nk ? vb + key * a.kv_st + c.dc * 8 : c.safe;
      R.v[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(pv));
    }
  }

  // Online softmax over one round for the NH heads: scores by packed dot products, summed over
  // the LPR lanes of each key row; P rounded to the element type, PV by packed dot products over
  // key pairs.
  static __device__ __forceinline__ void compute(const Round& R, const uint32_t (&qp)[NH][4], float scale,
                                                 int kg, float (&m_run)[NH], float (&l_run)[NH],
                                                 float (&acc)[NH][8]) {
    float sc[DEC_NI][NH];
#pragma unroll
    for (int i = 0; i < DEC_NI; ++i)
#pragma unroll
      for (int h = 0; h < NH; ++h) {
        float p = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) p = E::dot2(qp[h][w], R.k[i][w], p);
        sc[i][h] = row_sum<LPR>(p);
      }
    uint32_t pp[NH][DEC_NI / 2];
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      float mx = -__builtin_inff();
#pragma unroll
      for (int i = 0; i < DEC_NI; ++i) {
        const float x = (kg + KPI * i < R.nk) ? sc[i][h] * scale : -__builtin_inff();
        sc[i][h] = x;
        mx = fmaxf(mx, x);
      }
      mx = over_rows<LPR, true>(mx);
      const float m_new = fmaxf(m_run[h], mx);
      const float m_use = m_new == -__builtin_inff() ? 0.f : m_new;
      const float alpha = fast_exp2(m_run[h] - m_use);
      m_run[h] = m_new;
      l_run[h] *= alpha;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[h][e] *= alpha;
#pragma unroll
      for (int j = 0; j < DEC_NI / 2; ++j) {
        const float p0 = fast_exp2(sc[2 * j][h] - m_use);
        const float p1 = fast_exp2(sc[2 * j + 1][h] - m_use);
        l_run[h] += p0 + p1;
        pp[h][j] = E::pack2f(p0, p1);
      }
    }
#pragma unroll
    for (int j = 0; j < DEC_NI / 2; ++j)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        // (v of key 2j, v of key 2j+1) for dims 2w and 2w+1
        const uint32_t lo = __builtin_amdgcn_perm(R.v[2 * j + 1][w], R.v[2 * j][w], 0x05040100u);
        const uint32_t hi = __builtin_amdgcn_perm(R.v[2 * j + 1][w], R.v[2 * j][w], 0x07060302u);
#pragma unroll
        for (int h = 0; h < NH; ++h) {
          acc[h][2 * w] = E::dot2(pp[h][j], lo, acc[h][2 * w]);
          acc[h][2 * w + 1] = E::dot2(pp[h][j], hi, acc[h][2 * w + 1]);
        }
      }
  }

  // UNITS (1 or 2) independent units per workgroup, DEC_WAVES waves each: unit UNITS * blockIdx.x
  // + h is run by threads 256 h .. 256 h + 255 with LDS of its own; the units share only the
  // workgroup's barriers.  A unit index at or past n_units (the second half of the last
  // workgroup) runs no rounds and writes nothing.
  template <int UNITS>
  static __device__ void run(const DecodeArgs& a, int n_units) {
    __shared__ float s_m_[UNITS][DEC_WAVES][NH];
    __shared__ float s_l_[UNITS][DEC_WAVES][NH];
    __shared__ float s_acc_[UNITS][DEC_WAVES][NH][D];
    __shared__ int32_t s_blk_[UNITS][DEC_CACHE];
    __shared__ int32_t s_pg_[UNITS][DEC_CACHE];
    const int half = UNITS == 1 ? 0 : __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 8);
    auto& s_m = s_m_[half];
    auto& s_l = s_l_[half];
    auto& s_acc = s_acc_[half];
    int32_t* s_blk = s_blk_[half];
    int32_t* s_pg = s_pg_[half];

    const int tid = threadIdx.x & (64 * DEC_WAVES - 1);
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int unit_raw = UNITS * (int)blockIdx.x + half;
    const bool idle = unit_raw >= n_units;
    const int unit = idle ? n_units - 1 : unit_raw;

    // unit = s + num_splits * (r + rows * (hs + head_splits * b))
    const uint32_t w0 = (uint32_t)unit;
    const uint32_t w1 = fast_div(w0, (uint32_t)a.num_splits, a.mul_splits);
    const int s = (int)(w0 - w1 * (uint32_t)a.num_splits);
    const uint32_t w2 = fast_div(w1, (uint32_t)a.rows, a.mul_rows);
    const int r = (int)(w1 - w2 * (uint32_t)a.rows);
    const uint32_t w3 = fast_div(w2, (uint32_t)a.head_splits, a.mul_hs);
    const int hs = (int)(w2 - w3 * (uint32_t)a.head_splits);
    const int b = (int)w3;
    const int h0 = r * a.heads_per_row + hs * NH;  // first query head of this workgroup

    Ctx c;
    c.dc = lane % LPR;  // head-dim chunk
    c.kg = lane / LPR;  // key row within a load instruction
    c.b = b;
    c.safe = a.q + b * a.q_sb + h0 * a.q_sh + c.dc * 8;
    c.kvh = (int)fast_div((uint32_t)h0, (uint32_t)a.kv_group, a.mul_group);
    const int32_t* offp = a.sel_off + b * a.off_sb + r * a.off_sr;
    const int lo_all = offp[0];
    const int cnt = offp[1] - lo_all;
    int hi = lo_all + cnt;
    c.lo = lo_all;
    if (a.num_splits > 1) {  // split s takes entries [cnt * s / S, cnt * (s + 1) / S)
      c.lo = lo_all + (int)((int64_t)cnt * s / a.num_splits);
      hi = lo_all + (int)((int64_t)cnt * (s + 1) / a.num_splits);
    }
    c.selp = a.sel + b * a.sel_sb + r * a.sel_sr;
    c.L = a.kv_lens ? a.kv_lens[b] : a.kv_len;
    c.rpb = a.rpb;  // rounds per block
    c.mul_rpb = a.mul_rpb;
    // blocks holding keys below L: ceil(L / page), L < 2^31 and page <= 128
    c.nb = fast_div((uint32_t)max(c.L, 0) + (uint32_t)a.page - 1u, (uint32_t)a.page, a.mul_page);
    const int nsel = idle ? 0 : hi - c.lo;
    c.cached = nsel <= DEC_CACHE;
    c.s_blk = s_blk;
    c.s_pg = s_pg;
    const int n_items = nsel * c.rpb;
    c.n_it = n_items;

    // Stage the list (and its pages) once: the round loop then reads LDS, not dependent HBM loads.
    // The first pass (one entry per thread) interleaves with the lookup of this wave's first round,
    // which reads its entry and page directly: each of the two load_now reads also waits for the
    // staging load issued before it, so the staging costs no round trip of its own and the first
    // round's K/V loads go out without waiting for the staged list.
    Round A, B;
    int it = wave;
    const bool st1 = c.cached && tid < nsel;
    int st_lb = -1, st_pg = 0;
    if (st1) st_lb = c.selp[c.lo + tid];
    int lb0, pg0;
    const int x0 = (int)fast_div((uint32_t)it, (uint32_t)c.rpb, c.mul_rpb);
    lb0 = it < c.n_it ? load_now(c.selp + c.lo + x0) : -1;
    // The staged entry's table read is issued here and checked after the next load_now, so it
    // adds no wait of its own.
    const int32_t* st_t = (st1 && a.block_table) ? table_slot(a, b, st_lb, c.L) : nullptr;
    if (st_t) st_pg = *st_t;
    pg0 = 0;
    if (it < c.n_it && a.block_table) {
      pg0 = page_of<true>(a, b, lb0, c.L);
      if (pg0 < 0) lb0 = -1;
    }
    if (st1) {
      if (a.block_table) {
        st_pg = (st_t && st_pg >= 0 && st_pg < a.num_pages) ? st_pg : -1;
        if (st_pg < 0) st_lb = -1;
      }
      s_blk[tid] = st_lb;
      s_pg[tid] = st_pg;
    }
    issue_at(a, c, it, lb0, pg0, A);
    if (c.cached)  // entries past the first pass (lists of more than 64 * DEC_WAVES blocks)
      for (int x = tid + 64 * DEC_WAVES; x < nsel; x += 64 * DEC_WAVES) {
        int lb = c.selp[c.lo + x];
        int pg = 0;
        if (a.block_table) {
          pg = page_of(a, b, lb, c.L);
          if (pg < 0) lb = -1;
        }
        s_blk[x] = lb;
        s_pg[x] = pg;
      }

    uint32_t qp[NH][4];  // this lane's 8 head dims of each query head, packed pairs
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      const u32x4 w = *reinterpret_cast<const u32x4*>(a.q + b * a.q_sb + (h0 + h) * a.q_sh + c.dc * 8);
#pragma unroll
      for (int e = 0; e < 4; ++e) qp[h][e] = w[e];
    }
    float m_run[NH], l_run[NH], acc[NH][8];
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      m_run[h] = -__builtin_inff();
      l_run[h] = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;
    }
    __syncthreads();  // staged list visible

    // Rounds it = wave, wave + DEC_WAVES, ...: the next round's loads are issued before the
    // current round is computed (two register sets, alternating).  Every issue is unconditional
    // (a round past the end is a dead one), so the loads form one straight sequence and the wait
    // before a round's compute leaves the next round in flight.  The fences keep each round's
    // loads where they are written, ahead of the previous round's compute (the compiler would
    // otherwise sink them below it).
    // A wave's last round issues nothing after it: loads still in flight when the loop ends would
    // be waited for before the merge.
    for (;;) {
      if (it >= n_items) break;
      if (it + DEC_WAVES >= n_items) {
        compute(A, qp, a.scale_log2, c.kg, m_run, l_run, acc);
        break;
      }
      issue(a, c, it + DEC_WAVES, B);
      asm volatile("" ::: "memory");
      compute(A, qp, a.scale_log2, c.kg, m_run, l_run, acc);
      it += DEC_WAVES;
      if (it + DEC_WAVES >= n_items) {
        compute(B, qp, a.scale_log2, c.kg, m_run, l_run, acc);
        break;
      }
      issue(a, c, it + DEC_WAVES, A);
      asm volatile("" ::: "memory");
      compute(B, qp, a.scale_log2, c.kg, m_run, l_run, acc);
      it += DEC_WAVES;
    }

    // merge the key rows of the wave (lanes with equal dc), then the waves through LDS
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      l_run[h] = over_rows<LPR, false>(l_run[h]);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[h][e] = over_rows<LPR, false>(acc[h][e]);
    }
    // every lane of a row group holds the same sums; lanes 0..LPR-1 publish them
    if (c.kg == 0) {
#pragma unroll
      for (int h = 0; h < NH; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) s_acc[wave][h][c.dc * 8 + e] = acc[h][e];
    }
    if (lane == 0) {
#pragma unroll
      for (int h = 0; h < NH; ++h) {
        s_m[wave][h] = m_run[h];
        s_l[wave][h] = l_run[h];  // lanes of one row group hold equal sums: each key counted once
      }
    }
    __syncthreads();

    for (int x = tid; x < NH * D; x += 64 * DEC_WAVES) {
      const int h = x / D, d = x % D;
      float M = -__builtin_inff();
#pragma unroll
      for (int w = 0; w < DEC_WAVES; ++w) M = fmaxf(M, s_m[w][h]);
      const float Mu = M == -__builtin_inff() ? 0.f : M;
      float Ls = 0.f, As = 0.f;
#pragma unroll
      for (int w = 0; w < DEC_WAVES; ++w) {
        const float f = fast_exp2(s_m[w][h] - Mu);
        Ls += s_l[w][h] * f;
        As += s_acc[w][h][d] * f;
      }
      const int hq = h0 + h;
      if (idle) {
      } else if (a.num_splits == 1) {
        const float out = Ls > 0.f ? As / Ls : 0.f;
        a.o[b * a.o_sb + hq * a.o_sh + d] = E::from_f32(out);
      } else {
        float* pp = a.part + (((int64_t)s * a.B + b) * a.Hq + hq) * (D + 2);
        pp[d] = As;
        if (d == 0) {
          pp[D] = M;
          pp[D + 1] = Ls;
        }
      }
    }
  }
};

// At most 256 registers per lane: at least two waves per SIMD.
template <bool BF16, int D, int NH, int UNITS>
__global__ __launch_bounds__(64 * DEC_WAVES * UNITS) __attribute__((amdgpu_waves_per_eu(2)))
void decode_kernel(DecodeArgs a, int n_units) {
  Decode<BF16, D, NH>::template run<UNITS>(a, n_units);
}

// Merges split partials: out = sum_s acc_s 2^(m_s - M) / sum_s l_s 2^(m_s - M).
// The partials are read COMB_CHUNK splits at a time, every load of a chunk issued before the first
// is used (one memory round trip per chunk, not one per split); chunks merge online. With at most
// COMB_CHUNK splits, M and the summation order are those of a plain loop over s.
constexpr int COMB_CHUNK = 16;
template <bool BF16>
__global__ void decode_combine_kernel(const float* part, elem_t* o, int64_t o_sb, int64_t o_sh,
                                      int B, int Hq, int D, int S) {
  using E = Elem<BF16>;
  const int bh = blockIdx.x;
  const int b = bh / Hq, h = bh % Hq;
  const int64_t stride_s = (int64_t)B * Hq * (D + 2);
  const float* p0 = part + (int64_t)bh * (D + 2);
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    float M = -__builtin_inff(), Ls = 0.f, As = 0.f;
    for (int s0 = 0; s0 < S; s0 += COMB_CHUNK) {
      float m[COMB_CHUNK], l[COMB_CHUNK], v[COMB_CHUNK];
#pragma unroll
      for (int i = 0; i < COMB_CHUNK; ++i) {
        const float* ps = p0 + min(s0 + i, S - 1) * stride_s;  // past S: a repeat, skipped below
        m[i] = ps[D];
        l[i] = ps[D + 1];
        v[i] = ps[d];
      }
      float Mc = M;
#pragma unroll
      for (int i = 0; i < COMB_CHUNK; ++i)
        if (s0 + i < S) Mc = fmaxf(Mc, m[i]);
      const float Mu = Mc == -__builtin_inff() ? 0.f : Mc;
      const float r = fast_exp2(M - Mu);  // 0 while nothing has been merged (M = -inf)
      Ls *= r;
      As *= r;
#pragma unroll
      for (int i = 0; i < COMB_CHUNK; ++i)
        if (s0 + i < S) {
          const float f = fast_exp2(m[i] - Mu);
          Ls += l[i] * f;
          As += v[i] * f;
        }
      M = Mc;
    }
    o[b * o_sb + h * o_sh + d] = E::from_f32(Ls > 0.f ? As / Ls : 0.f);
  }
}

static int decode_cus() {
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

template <bool BF16, int D, int UNITS>
static void launch_decode_units(const DecodeArgs& a, int nh, int64_t units, hipStream_t st) {
  const dim3 grid((unsigned)((units + UNITS - 1) / UNITS)), block(64 * DEC_WAVES * UNITS);
  switch (nh) {
    case 4: hipLaunchKernelGGL((decode_kernel<BF16, D, 4, UNITS>), grid, block, 0, st, a, (int)units); break;
    case 2: hipLaunchKernelGGL((decode_kernel<BF16, D, 2, UNITS>), grid, block, 0, st, a, (int)units); break;
    default: hipLaunchKernelGGL((decode_kernel<BF16, D, 1, UNITS>), grid, block, 0, st, a, (int)units); break;
  }
}

// Two units per workgroup once there are at least two per CU: one 8-wave workgroup per CU starts
// sooner than two 4-wave ones (configs[3]: 41.39-41.48 against 41.65-41.74 us).  Fewer units keep
// one per workgroup, so every CU gets one.
template <bool BF16, int D>
static hipError_t launch_decode_d(const DecodeArgs& a, int nh, int64_t units, hipStream_t st) {
  if (units >= 2 * (int64_t)decode_cus())
    launch_decode_units<BF16, D, 2>(a, nh, units, st);
  else
    launch_decode_units<BF16, D, 1>(a, nh, units, st);
  return hipGetLastError();
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace sa

extern "C" int64_t sa_decode_workspace_bytes(int B, int Hq, int D, int num_splits) {
  if (num_splits <= 1 || B <= 0 || Hq <= 0 || D <= 0) return 0;
  return (int64_t)num_splits * B * Hq * (D + 2) * (int64_t)sizeof(float);
}

extern "C" int sa_decode(int dtype,
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
                         void* stream) {
  using namespace sa;
  clear_error();
  if (dtype != SA_DTYPE_BF16 && dtype != SA_DTYPE_F16)
    return set_error(SA_E_DTYPE, "sa_decode: dtype %d is not bf16 (0) or f16 (1)", dtype);
  if (B < 0 || Hq < 1 || Hkv < 1 || Hq % Hkv)
    return set_error(SA_E_SHAPE, "sa_decode: bad heads Hq=%d Hkv=%d (B=%d)", Hq, Hkv, B);
  if (D != 64 && D != 128)
    return set_error(SA_E_HEADDIM, "sa_decode: head dim %d not supported (64, 128)", D);
  if (page < 16 || page > 128 || page % 16)
    return set_error(SA_E_BLOCK, "sa_decode: page/block size %d not supported (16..128, multiple of 16)", page);
  if (sel_rows != Hq && sel_rows != Hkv)
    return set_error(SA_E_CSR, "sa_decode: sel_rows=%d must be Hq=%d or Hkv=%d", sel_rows, Hq, Hkv);
  if (num_splits < 1) return set_error(SA_E_SHAPE, "sa_decode: num_splits=%d < 1", num_splits);
  if (B == 0) return 0;
  if (!q || !k || !v || !o || !sel || !sel_off)
    return set_error(SA_E_NULL, "sa_decode: NULL pointer argument");
  if (!kv_lens && kv_len < 0) return set_error(SA_E_SHAPE, "sa_decode: kv_len=%d < 0", kv_len);
  if (block_table && (max_blocks < 0 || num_pages < 0 || bt_stride < max_blocks))
    return set_error(SA_E_SHAPE, "sa_decode: block table of %d columns (row stride %lld) over %d pages", max_blocks,
                     (long long)bt_stride, num_pages);
  const int64_t strides[] = {q_sb, q_sh, kv_sb, kv_sh, kv_st};
  for (int64_t s : strides)
    if (s % 8) return set_error(SA_E_ALIGN, "sa_decode: stride %lld is not a multiple of 8 elements", (long long)s);
  if (!aligned16(q) || !aligned16(k) || !aligned16(v))
    return set_error(SA_E_ALIGN, "sa_decode: q/k/v base pointers must be 16-byte aligned");
  if (num_splits > 1 && (!workspace || workspace_bytes < sa_decode_workspace_bytes(B, Hq, D, num_splits)))
    return set_error(SA_E_WORKSPACE, "sa_decode: num_splits=%d needs %lld workspace bytes", num_splits,
                     (long long)sa_decode_workspace_bytes(B, Hq, D, num_splits));

  DecodeArgs a;
  a.q = static_cast<const elem_t*>(q);
  a.q_sb = q_sb; a.q_sh = q_sh;
  a.k = static_cast<const elem_t*>(k);
  a.v = static_cast<const elem_t*>(v);
  a.kv_sb = kv_sb; a.kv_sh = kv_sh; a.kv_st = kv_st;
  a.block_table = block_table; a.bt_stride = bt_stride;
  a.max_blocks = max_blocks; a.num_pages = num_pages;
  a.kv_lens = kv_lens; a.kv_len = kv_len;
  a.sel = sel; a.sel_sb = sel_sb; a.sel_sr = sel_sr;
  a.sel_off = sel_off; a.off_sb = off_sb; a.off_sr = off_sr;
  a.rows = sel_rows;
  a.heads_per_row = Hq / sel_rows;
  const int nh = (a.heads_per_row % 4 == 0) ? 4 : (a.heads_per_row % 2 == 0) ? 2 : 1;
  a.head_splits = a.heads_per_row / nh;
  a.o = static_cast<elem_t*>(o);
  a.o_sb = o_sb; a.o_sh = o_sh;
  a.part = static_cast<float*>(workspace);
  a.B = B; a.Hq = Hq; a.Hkv = Hkv; a.page = page; a.num_splits = num_splits;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  a.kv_group = Hq / Hkv;
  a.rpb = (int)ceil_div(page, dec_keys_per_round(D));
  a.mul_splits = div_mul((uint32_t)num_splits);
  a.mul_rows = div_mul((uint32_t)sel_rows);
  a.mul_hs = div_mul((uint32_t)a.head_splits);
  a.mul_group = div_mul((uint32_t)a.kv_group);
  a.mul_page = div_mul((uint32_t)page);
  a.mul_rpb = div_mul((uint32_t)a.rpb);

  const int64_t grid = (int64_t)num_splits * sel_rows * a.head_splits * B;
  if (grid > 0x7fffffff) return set_error(SA_E_SHAPE, "sa_decode: grid too large");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool bf16 = dtype == SA_DTYPE_BF16;
  hipError_t err;
  if (D == 128)
    err = bf16 ? launch_decode_d<true, 128>(a, nh, grid, st) : launch_decode_d<false, 128>(a, nh, grid, st);
  else
    err = bf16 ? launch_decode_d<true, 64>(a, nh, grid, st) : launch_decode_d<false, 64>(a, nh, grid, st);
  if (err == hipSuccess && num_splits > 1) {
    if (bf16)
      hipLaunchKernelGGL(decode_combine_kernel<true>, dim3(B * Hq), dim3(D), 0, st, a.part, a.o, o_sb, o_sh, B, Hq, D, num_splits);
    else
      hipLaunchKernelGGL(decode_combine_kernel<false>, dim3(B * Hq), dim3(D), 0, st, a.part, a.o, o_sb, o_sh, B, Hq, D, num_splits);
    err = hipGetLastError();
  }
  if (err != hipSuccess) return set_error((int)err, "sa_decode: launch failed: %s", hipGetErrorString(err));
  return 0;
}

// ---- no-allocation entry point ------------------------------------------------------------
// sa_decode with its split partials in a file-scope device array instead of a caller workspace,
// for callers that cannot allocate device memory.  Each GPU holds its own copy of the array; its
// device address comes from hipGetSymbolAddress once per device (the array's name in host code
// is not a device address) and is kept in noalloc_ptr.
namespace sa {

constexpr int64_t NOALLOC_SCRATCH_BYTES = (int64_t)16 << 20;
constexpr int NOALLOC_MAX_DEVICES = 64;

static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

static std::mutex noalloc_mu;
static void* noalloc_ptr[NOALLOC_MAX_DEVICES] = {nullptr};

// Device address of the current device's scratch array (set up on the first call per device).
static int noalloc_scratch(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error((int)e, "sa_decode_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= NOALLOC_MAX_DEVICES)
    return set_error(SA_E_SHAPE, "sa_decode_noalloc: device %d past the %d supported", dev, NOALLOC_MAX_DEVICES);
  std::lock_guard<std::mutex> lock(noalloc_mu);
  if (!noalloc_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(e != hipSuccess ? (int)e : SA_E_NULL, "sa_decode_noalloc: hipGetSymbolAddress(scratch) failed: %s",
                       hipGetErrorString(e));
    noalloc_ptr[dev] = p;
  }
  *out = noalloc_ptr[dev];
  return 0;
}

}  // namespace sa

extern "C" int64_t sa_decode_noalloc_scratch_bytes(void) { return sa::NOALLOC_SCRATCH_BYTES; }

extern "C" int sa_decode_noalloc(int dtype,
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
                                 int num_splits, void* stream) {
  using namespace sa;
  clear_error();
  const int64_t need = sa_decode_workspace_bytes(B, Hq, D, num_splits);
  if (need > NOALLOC_SCRATCH_BYTES)
    return set_error(SA_E_WORKSPACE,
                     "sa_decode_noalloc: B=%d Hq=%d D=%d num_splits=%d needs %lld scratch bytes, more than the %lld "
                     "held (use sa_decode with a workspace, or fewer splits)",
                     B, Hq, D, num_splits, (long long)need, (long long)NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if (need > 0) {
    const int rc = noalloc_scratch(&ws);
    if (rc) return rc;
  }
  return sa_decode(dtype, q, q_sb, q_sh, k, v, kv_sb, kv_sh, kv_st, block_table, bt_stride, max_blocks, num_pages,
                   kv_lens, kv_len, sel, sel_sb, sel_sr, sel_off, off_sb, off_sr, sel_rows, o, o_sb, o_sh, B, Hq,
                   Hkv, D, page, sm_scale, num_splits, ws, need, stream);
}
