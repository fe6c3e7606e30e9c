// Block-sparse causal attention over a CSR block schedule, gfx950 (CDNA4).
//
// Semantics follow the reference kernel kernels/triton/universal_sparse_attn.py:77-160:
// per query row, an online softmax over the keys of the retained blocks, masked by
// q_abs >= k and k < T_k, fp32 accumulation, probabilities rounded to the element
// type before the PV product, output acc / (l > 0 ? l : 1).
//
// Mapping onto the hardware:
//  * one workgroup = (batch b, CSR row r, 64-row query tile qt); one wave per query
//    head that shares row r (GQA: the Hq/Hkv heads of a KV group share one K/V tile
//    staged in LDS, so K/V are read once per group instead of once per head);
//  * per wave and 64-key tile: S^T = K Q^T and O^T = V^T P^T on the
//    v_mfma_f32_32x32x16 matrix cores.  Computing the transposed products puts one
//    query row in each lane column, so the softmax statistics, the rescale of O and
//    the P operand of the second product all stay in the lane that owns the row;
//  * V is staged transposed in LDS ([d][key]) so the A operand of O^T = V^T P^T is
//    two 8-byte LDS reads per lane;
//  * the softmax works in base 2 with scale*log2(e) folded into the scores and the
//    hardware v_exp_f32 (2^x).
//
// MFMA 32x32x16 lane layouts used (l = lane, g = l / 32):
//   A (32 x 16): lane l holds row l % 32, k = 8g .. 8g+7
//   B (16 x 32): lane l holds column l % 32, k = 8g .. 8g+7
//   D (32 x 32): lane l, register r holds row 8(r/4) + 4g + r%4, column l % 32
#include "sa_common.h"

namespace sa {

constexpr int TILE = 64;  // query rows and keys per tile

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
  int tpb_log2;      // log2(block_size / 64)
  int q_offset;
  float scale_log2;  // sm_scale * log2(e)
};

template <bool BF16, int D, int NW>
struct Prefill {
  using E = Elem<BF16>;
  static constexpr int NT = 64 * NW;        // threads
  static constexpr int KS = D + 8;          // sK row stride (elements), 16 B pad
  static constexpr int VS = TILE + 8;       // sVt row stride (elements)
  static constexpr int DC = D / 8;          // 16-byte chunks per row
  static constexpr int K_TOTAL = TILE * DC;       // 16-byte K chunks per tile
  static constexpr int V_TOTAL = DC * (TILE / 4);  // V units (4 keys x 8 d) per tile
  static constexpr int KCH = (K_TOTAL + NT - 1) / NT;
  static constexpr int VUN = (V_TOTAL + NT - 1) / NT;
  static constexpr bool PREFETCH = (KCH + 4 * VUN) <= 8;

  struct Stage {
    u32x4 kr[KCH];
    u32x4 vr[VUN][4];
  };

  static __device__ __forceinline__ void load(Stage& st, const elem_t* kb, const elem_t* vb,
                                              const PrefillArgs& a, int kt, int tid) {
#pragma unroll
    for (int u = 0; u < KCH; ++u) {
      const int c = tid + u * NT;
      if (K_TOTAL % NT && c >= K_TOTAL) break;
      const int key = c / DC, dc = c % DC;
      const int tok = kt * TILE + key;
      st.kr[u] = tok < a.Tk ? *reinterpret_cast<const u32x4*>(kb + tok * a.k_st + dc * 8)
                            : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < VUN; ++u) {
      const int c = tid + u * NT;
      if (V_TOTAL % NT && c >= V_TOTAL) break;
      const int dc = c % DC, kg = c / DC;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int tok = kt * TILE + 4 * kg + kk;
        st.vr[u][kk] = tok < a.Tk ? *reinterpret_cast<const u32x4*>(vb + tok * a.v_st + dc * 8)
                                  : u32x4{0, 0, 0, 0};
      }
    }
  }

  static __device__ __forceinline__ void store(const Stage& st, elem_t* sK, elem_t* sVt, int tid) {
#pragma unroll
    for (int u = 0; u < KCH; ++u) {
      const int c = tid + u * NT;
      if (K_TOTAL % NT && c >= K_TOTAL) break;
      const int key = c / DC, dc = c % DC;
      *reinterpret_cast<u32x4*>(sK + key * KS + dc * 8) = st.kr[u];
    }
#pragma unroll
    for (int u = 0; u < VUN; ++u) {
      const int c = tid + u * NT;
      if (V_TOTAL % NT && c >= V_TOTAL) break;
      const int dc = c % DC, kg = c / DC;
#pragma unroll
      for (int w = 0; w < 4; ++w) {       // d = dc*8 + 2w (low halves) and 2w+1 (high halves)
        const uint32_t x0 = st.vr[u][0][w], x1 = st.vr[u][1][w];
        const uint32_t x2 = st.vr[u][2][w], x3 = st.vr[u][3][w];
        const u32x2 even = {(x0 & 0xffffu) | (x1 << 16), (x2 & 0xffffu) | (x3 << 16)};
        const u32x2 odd = {(x0 >> 16) | (x1 & 0xffff0000u), (x2 >> 16) | (x3 & 0xffff0000u)};
        *reinterpret_cast<u32x2*>(sVt + (dc * 8 + 2 * w) * VS + 4 * kg) = even;
        *reinterpret_cast<u32x2*>(sVt + (dc * 8 + 2 * w + 1) * VS + 4 * kg) = odd;
      }
    }
  }

  static __device__ void run(const PrefillArgs& a) {
    __shared__ __attribute__((aligned(16))) elem_t sK[TILE * KS];
    __shared__ __attribute__((aligned(16))) elem_t sVt[D * VS];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int g = lane >> 5;
    const int l32 = lane & 31;

    // Work item; the heaviest (latest) query tiles are dispatched first.
    const int per_tile = a.R * a.B * a.head_splits;
    const int wid = blockIdx.x;
    const int qt = a.ntq - 1 - wid / per_tile;
    int rem = wid % per_tile;
    const int r = rem % a.R;
    rem /= a.R;
    const int hs = rem % a.head_splits;
    const int b = rem / a.head_splits;
    const int hq = r * a.heads_per_row + hs * NW + wave;
    const int kvh = (r * a.heads_per_row + hs * NW) / (a.Hq / a.Hkv);  // shared by the waves

    const elem_t* qb = a.q + b * a.q_sb + hq * a.q_sh;
    const elem_t* kb = a.k + b * a.k_sb + kvh * a.k_sh;
    const elem_t* vb = a.v + b * a.v_sb + kvh * a.v_sh;

    // CSR row of this query tile; each block holds 2^tpb_log2 key tiles.
    const int qblk = qt >> a.tpb_log2;
    const int32_t* offs = a.offsets + r * a.offsets_stride;
    const int32_t* prow = a.pairs + r * a.pairs_stride;
    const int e0 = offs[qblk];
    const int n_tiles = (offs[qblk + 1] - e0) << a.tpb_log2;
    const int tpb_mask = (1 << a.tpb_log2) - 1;
    const int q_row0 = qt * TILE;
    const int q_abs_min = a.q_offset + q_row0;
    const int q_abs_max = a.q_offset + min(a.Tq, q_row0 + TILE) - 1;
    auto tile_of = [&](int t) { return (prow[e0 + (t >> a.tpb_log2)] << a.tpb_log2) + (t & tpb_mask); };
    // Tiles entirely past T_k or entirely above the causal limit contribute nothing; negative
    // ids (malformed schedules) are skipped rather than read.
    auto next_usable = [&](int t) {
      for (; t < n_tiles; ++t) {
        const int kt = tile_of(t);
        if (kt >= 0 && kt * TILE < a.Tk && kt * TILE <= q_abs_max) break;
      }
      return t;
    };

    // Q^T as the B operand of S^T = K Q^T: lane holds row 32i + l32, d = 16c + 8g .. +7.
    u32x4 qf[2][D / 16];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int row = q_row0 + 32 * i + l32;
#pragma unroll
      for (int c = 0; c < D / 16; ++c)
        qf[i][c] = row < a.Tq ? *reinterpret_cast<const u32x4*>(qb + row * a.q_st + 16 * c + 8 * g)
                              : u32x4{0, 0, 0, 0};
    }

    f32x16 O[2][D / 32];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt) O[i][dt] = f32x16{};
    float m_run[2] = {-__builtin_inff(), -__builtin_inff()};
    float l_run[2] = {0.f, 0.f};  // this lane's half of the row sum

    Stage st;
    int t = next_usable(0);
    if (t < n_tiles) {
      load(st, kb, vb, a, tile_of(t), tid);
      store(st, sK, sVt, tid);
    }
    __syncthreads();

    while (t < n_tiles) {
      const int kt = tile_of(t);
      const int tn = next_usable(t + 1);
      if (PREFETCH && tn < n_tiles) load(st, kb, vb, a, tile_of(tn), tid);

      // ---- S^T = K Q^T (64 keys x 64 rows) -------------------------------------
      f32x16 S[2][2];
#pragma unroll
      for (int j = 0; j < 2; ++j) S[j][0] = S[j][1] = f32x16{};
#pragma unroll
      for (int c = 0; c < D / 16; ++c) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const u32x4 kf = *reinterpret_cast<const u32x4*>(sK + (32 * j + l32) * KS + 16 * c + 8 * g);
          S[j][0] = E::mfma32(kf, qf[0][c], S[j][0]);
          S[j][1] = E::mfma32(kf, qf[1][c], S[j][1]);
        }
      }

      // ---- online softmax, one query row per lane column --------------------------
      const bool need_mask = (kt * TILE + TILE - 1 > q_abs_min) || (kt * TILE + TILE > a.Tk);
      u32x4 P[2][2][2];  // [key tile j][q tile i][half h]: B operand of O^T = V^T P^T
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int q_abs = q_abs_min + 32 * i + l32;
        float mx = -__builtin_inff();
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int rr = 0; rr < 16; ++rr) {
            float s = S[j][i][rr] * a.scale_log2;
            if (need_mask) {
              const int key = kt * TILE + 32 * j + 8 * (rr >> 2) + 4 * g + (rr & 3);
              if (key > q_abs || key >= a.Tk) s = -__builtin_inff();
            }
            S[j][i][rr] = s;
            mx = fmaxf(mx, s);
          }
        mx = fmaxf(mx, swap_halves(mx));
        const float m_new = fmaxf(m_run[i], mx);
        const float m_use = m_new == -__builtin_inff() ? 0.f : m_new;
        const float alpha = fast_exp2(m_run[i] - m_use);
        m_run[i] = m_new;
        float ls = 0.f;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            elem_t pe[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const float p = fast_exp2(S[j][i][8 * h + e] - m_use);
              ls += p;
              pe[e] = E::from_f32(p);
            }
            P[j][i][h] = u32x4{pack2(pe[0], pe[1]), pack2(pe[2], pe[3]), pack2(pe[4], pe[5]),
                               pack2(pe[6], pe[7])};
          }
        l_run[i] = l_run[i] * alpha + ls;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) O[i][dt] *= alpha;
      }

      // ---- O^T += V^T P^T ---------------------------------------------------------
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int kbase = 32 * j + 16 * h + 4 * g;
#pragma unroll
          for (int dt = 0; dt < D / 32; ++dt) {
            const elem_t* vp = sVt + (32 * dt + l32) * VS + kbase;
            const u32x2 lo = *reinterpret_cast<const u32x2*>(vp);
            const u32x2 hi = *reinterpret_cast<const u32x2*>(vp + 8);
            const u32x4 vf = {lo[0], lo[1], hi[0], hi[1]};
            O[0][dt] = E::mfma32(vf, P[j][0][h], O[0][dt]);
            O[1][dt] = E::mfma32(vf, P[j][1][h], O[1][dt]);
          }
        }

      __syncthreads();
      if (tn < n_tiles) {
        if (!PREFETCH) load(st, kb, vb, a, tile_of(tn), tid);
        store(st, sK, sVt, tid);
      }
      __syncthreads();
      t = tn;
    }

    // ---- epilogue: O / l, rows owned by lane columns ----------------------------------
    elem_t* ob = a.o + b * a.o_sb + hq * a.o_sh;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const float lt = l_run[i] + swap_halves(l_run[i]);
      const float inv = lt > 0.f ? 1.f / lt : 1.f;
      const int row = q_row0 + 32 * i + l32;
      if (row < a.Tq) {
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
          for (int rq = 0; rq < 4; ++rq) {
            const int d0 = 32 * dt + 8 * rq + 4 * g;
            const u32x2 w = {pack2(E::from_f32(O[i][dt][4 * rq] * inv), E::from_f32(O[i][dt][4 * rq + 1] * inv)),
                             pack2(E::from_f32(O[i][dt][4 * rq + 2] * inv), E::from_f32(O[i][dt][4 * rq + 3] * inv))};
            *reinterpret_cast<u32x2*>(ob + row * a.o_st + d0) = w;
          }
      }
    }
  }
};

template <bool BF16, int D, int NW>
__global__ __launch_bounds__(64 * NW) void prefill_kernel(PrefillArgs a) {
  Prefill<BF16, D, NW>::run(a);
}

template <bool BF16, int D>
static hipError_t launch_d(const PrefillArgs& a, int nw, int64_t grid, hipStream_t s) {
  switch (nw) {
    case 4: hipLaunchKernelGGL((prefill_kernel<BF16, D, 4>), dim3(grid), dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL((prefill_kernel<BF16, D, 2>), dim3(grid), dim3(128), 0, s, a); break;
    default: hipLaunchKernelGGL((prefill_kernel<BF16, D, 1>), dim3(grid), dim3(64), 0, s, a); break;
  }
  return hipGetLastError();
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
  const int nw = (a.heads_per_row % 4 == 0) ? 4 : (a.heads_per_row % 2 == 0) ? 2 : 1;
  a.head_splits = a.heads_per_row / nw;
  a.B = B; a.Hq = Hq; a.Hkv = Hkv; a.Tq = T_q; a.Tk = T_k;
  a.ntq = (int)ceil_div(T_q, TILE);
  a.tpb_log2 = block_size == 128 ? 1 : 0;
  a.q_offset = q_offset;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  if (csr_rows == Hkv && Hq != Hkv && a.heads_per_row != Hq / Hkv)
    return set_error(SA_E_CSR, "sa_prefill: inconsistent group mapping");

  const int64_t grid = (int64_t)a.ntq * a.R * B * a.head_splits;
  if (grid > 0x7fffffff) return set_error(SA_E_SHAPE, "sa_prefill: grid of %lld workgroups too large", (long long)grid);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool bf16 = dtype == SA_DTYPE_BF16;
  hipError_t err;
  if (D == 128)
    err = bf16 ? launch_d<true, 128>(a, nw, grid, s) : launch_d<false, 128>(a, nw, grid, s);
  else
    err = bf16 ? launch_d<true, 64>(a, nw, grid, s) : launch_d<false, 64>(a, nw, grid, s);
  if (err != hipSuccess) return set_error((int)err, "sa_prefill: launch failed: %s", hipGetErrorString(err));
  return 0;
}
