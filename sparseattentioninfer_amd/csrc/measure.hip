// Measurement aids: the HBM streaming-read rate of this GPU, the practical ceiling against which
// the memory-bound decode kernel is read, the dense bf16 matrix-core rate and LDS fragment-read
// rates that bound the prefill kernel, and the steady-state step of its loop in three wave layouts
// (bench.py reports them beside the kernels, in the same run).  Not part of the attention path.
//
// Streaming read:
// A grid of 8 workgroups per CU; each workgroup reads one contiguous chunk of `src` (1/grid of
// it) front to back, its 256 threads covering 4 KiB per load instruction, eight non-temporal
// loads in flight, and folds the words with xor into one word per workgroup (written to
// sink[blockIdx.x], so the loads cannot be dropped).  Of the patterns measured on MI355X this is
// the fastest: per-workgroup chunks 7.0-7.2 TB/s against 6.2 TB/s for a grid-stride loop over the
// same 4 GiB, and non-temporal loads (no Infinity Cache allocation) 7.0 against 6.1 TB/s for
// ordinary ones.  Pieces past the chunk's last whole group of eight are read by the tail loop.
#include "sa_common.h"

namespace sa {

constexpr int SR_THREADS = 256;

__global__ __launch_bounds__(SR_THREADS) void stream_read_kernel(const u32x4* src, int64_t n, uint32_t* sink) {
  __shared__ uint32_t s_acc[SR_THREADS / 64];
  constexpr int NL = 8;
  const int64_t per = (n + gridDim.x - 1) / gridDim.x;
  const int64_t lo = min(n, (int64_t)blockIdx.x * per);
  const int64_t hi = min(n, lo + per);
  int64_t i = lo + threadIdx.x;
  u32x4 acc = {0, 0, 0, 0};
  for (; i + (NL - 1) * SR_THREADS < hi; i += NL * SR_THREADS) {
    u32x4 x[NL];
#pragma unroll
    for (int u = 0; u < NL; ++u) x[u] = __builtin_nontemporal_load(src + i + u * SR_THREADS);
#pragma unroll
    for (int u = 0; u < NL; ++u) acc ^= x[u];
  }
  for (; i < hi; i += SR_THREADS) acc ^= __builtin_nontemporal_load(src + i);
  uint32_t x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) x ^= __shfl_xor(x, d, 64);
  if ((threadIdx.x & 63) == 0) s_acc[threadIdx.x >> 6] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t y = 0;
    for (int w = 0; w < SR_THREADS / 64; ++w) y ^= s_acc[w];
    sink[blockIdx.x] = y;
  }
}

// Dense matrix-core rate: every wave runs `iters` rounds of MR_CHAINS independent
// v_mfma_f32_32x32x16_bf16 accumulations (32768 FLOP each) on register operands, and folds its
// accumulators into sink[global thread] so nothing is dropped.  Launched with `per_cu` 4-wave
// workgroups per CU, the SIMDs run `per_cu` waves each.
constexpr int MR_THREADS = 256;
constexpr int MR_CHAINS = 4;

__global__ __launch_bounds__(MR_THREADS) void mfma_rate_kernel(int iters, float* sink) {
  using E = Elem<true>;
  const uint32_t t = threadIdx.x;
  const uint32_t seed = t + MR_THREADS * blockIdx.x;
  // bf16 values in [0.5, 1) with hashed mantissas and signs, different per lane and element: the
  // multipliers toggle as they do on attention data (operand bits set how much power, and so how
  // much clock, the matrix cores draw)
  auto h = [&](uint32_t k) {
    uint32_t x = (seed + 1u) * 0x9e3779b9u ^ (k * 0x85ebca6bu);
    x ^= x >> 15;
    x *= 0x2c1b3c6du;
    x ^= x >> 12;
    return (x & 0x807f807fu) | 0x3f003f00u;
  };
  const u32x4 a = {h(0), h(1), h(2), h(3)};
  const u32x4 b = {h(4), h(5), h(6), h(7)};
  f32x16 acc[MR_CHAINS];
#pragma unroll
  for (int c = 0; c < MR_CHAINS; ++c) acc[c] = f32x16{};
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int c = 0; c < MR_CHAINS; ++c) acc[c] = E::mfma32(a, b, acc[c]);
  }
  float x = 0.f;
#pragma unroll
  for (int c = 0; c < MR_CHAINS; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) x += acc[c][e];
  sink[(int64_t)blockIdx.x * MR_THREADS + t] = x;
}

// LDS fragment-read rate: one 8-wave workgroup per CU (two waves per SIMD, as the prefill kernel
// runs) reads a 16 KiB staged tile `iters` times per wave with the prefill kernel's two fragment
// reads: 16-byte ds_read_b128 (lane l: row l % 32, 16-byte chunk l / 32 of a 64-byte row, chunks
// swizzled by (row / 4) % 4 as in the staged K tiles) or two 8-byte ds_read_b64_tr_b16 (the
// transposing V^T read of four 16-bit keys); 16 reads per round, xor-folded into sink.
constexpr int LR_THREADS = 512;
constexpr int LR_TILE = 16384;

__device__ __forceinline__ u32x2 lr_tr16(const char* p) {
  typedef short v4i16 __attribute__((ext_vector_type(4)));
  const v4i16 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16*)(p));
  return __builtin_bit_cast(u32x2, r);
}

template <bool TR16>
__global__ __launch_bounds__(LR_THREADS) void lds_rate_kernel(int iters, uint32_t* sink) {
  __shared__ __attribute__((aligned(16))) char tile[LR_TILE];
  const int t = threadIdx.x, lane = t & 63;
  for (int x = t; x < LR_TILE / 4; x += LR_THREADS) reinterpret_cast<uint32_t*>(tile)[x] = 0x9e3779b9u * x;
  __syncthreads();
  const int l32 = lane & 31, g = lane >> 5;
  const int k0 = l32 * 64 + 16 * (g ^ ((l32 >> 2) & 3));
  const int i16 = lane & 15, G = lane >> 4;
  const int c4 = 2 * (G & 1) + ((i16 >> 1) & 1);
  const int v0 = (8 * g + (i16 >> 2)) * 64 + 16 * (c4 ^ (2 * g)) + 8 * (i16 & 1);
  u32x4 acc = {0, 0, 0, 0};
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      // 16 KiB per round: 4 column groups x 2 row halves x 2 chunk parities (b128), or
      // 4 x 2 x 2 1 KiB blocks of two transposing reads each (tr16)
      const char* p = tile + 4096 * (r & 3) + 2048 * ((r >> 2) & 1);
      if constexpr (TR16) {
        const char* q = p + 1024 * (r >> 3);
        const u32x2 lo = lr_tr16(q + v0);
        const u32x2 hi = lr_tr16(q + ((v0 + 256) ^ 16));
        acc ^= u32x4{lo[0], lo[1], hi[0], hi[1]};
      } else {
        acc ^= *reinterpret_cast<const u32x4*>(p + ((r >> 3) ? (k0 ^ 32) : k0));
      }
    }
    // keeps each round's reads from being merged across rounds
    asm volatile("" : "+v"(acc));
  }
  sink[(int64_t)blockIdx.x * LR_THREADS + t] = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
}

// Staging rate: one 8-wave workgroup per CU moves 16 KiB tiles of an L2-resident source into LDS
// with the prefill kernel's direct loads (global_load_lds_dwordx4, two 1 KiB loads per wave and
// tile), waits for them and meets at a barrier, `iters` times: the per-CU rate of the load path
// that stages K/V tiles (and Q) in the prefill kernel.  src: at least 64 KiB, 16-byte aligned;
// tiles rotate over it.
constexpr int ST_THREADS = 512;

__global__ __launch_bounds__(ST_THREADS) void stage_rate_kernel(const char* src, int iters, uint32_t* sink) {
  __shared__ __attribute__((aligned(16))) char tile[2 * LR_TILE];
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const uint32_t voff = 16u * lane;
  for (int i = 0; i < iters; ++i) {
    const char* s = src + (int64_t)(i & 3) * LR_TILE;  // 4 tiles of the 64 KiB source in turn
    char* d = tile + (i & 1) * LR_TILE;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int k = 2 * wave + u;  // 1 KiB piece k of the 16 KiB tile
      const uint32_t lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)(d + 1024 * k);
      asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                   :
                   : "v"(voff), "s"(s + 1024 * k), "s"(lds)
                   : "memory", "m0");
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
  }
  sink[(int64_t)blockIdx.x * ST_THREADS + t] = reinterpret_cast<const uint32_t*>(tile)[t];
}

// Step rate: the steady-state step of the prefill loop (one 64-key tile) in three wave layouts, each
// on one workgroup per CU with the same matrix work per SIMD (64 v_mfma 32x32x16-equivalents, 2,048
// matrix cycles per step), the same exponentials per SIMD, K and V fragment reads from a staged 16 KiB
// tile per product as the kernel does them, 32 KiB of direct K/V loads per workgroup and step from an
// L2-resident source, and one barrier per step.  Only the time counts; sink values are not meaningful.
//   layout 0: 8 waves x 32 query rows (the shipped kernel's layout, two waves per SIMD, the second
//             half of the waves one block behind), v_mfma_f32_32x32x16;
//   layout 1: 16 waves x 16 rows (four waves per SIMD), v_mfma_f32_16x16x32: twice the fragment
//             bytes per FLOP;
//   layout 2: 4 waves x 64 rows (one wave per SIMD, O^T in AGPRs): each fragment read feeds two
//             products, and one wave interleaves its own exponentials with its products.
constexpr int SP_TILE = 16384;

struct StepFrag {
  int k0, v0;
  __device__ explicit StepFrag(int lane) {
    const int l32 = lane & 31, g = lane >> 5;
    k0 = l32 * 64 + 16 * (g ^ ((l32 >> 2) & 3));
    const int i = lane & 15, G = lane >> 4;
    const int c4 = 2 * (G & 1) + ((i >> 1) & 1);
    v0 = (8 * g + (i >> 2)) * 64 + 16 * (c4 ^ (2 * g)) + 8 * (i & 1);
  }
  __device__ u32x4 k(const char* cK, int j, int cc) const {
    return *reinterpret_cast<const u32x4*>(cK + 4096 * (cc >> 1) + 2048 * j + ((cc & 1) ? (k0 ^ 32) : k0));
  }
  __device__ u32x4 v(const char* cV, int j, int h, int dt) const {
    const char* p = cV + 4096 * dt + 2048 * j + 1024 * h;
    const u32x2 lo = lr_tr16(p + v0);
    const u32x2 hi = lr_tr16(p + ((v0 + 256) ^ 16));
    return u32x4{lo[0], lo[1], hi[0], hi[1]};
  }
};

__device__ __forceinline__ void sp_mfma_agpr(f32x16& acc, u32x4 a, u32x4 b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
__device__ __forceinline__ void sp_mfma_vgpr(f32x16& acc, u32x4 a, u32x4 b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "v"(b));
}

template <int LAYOUT>
struct StepLayout {
  static constexpr int WAVES = LAYOUT == 0 ? 8 : LAYOUT == 1 ? 16 : 4;
  static constexpr int THREADS = 64 * WAVES;
};

template <int LAYOUT>
__global__ __launch_bounds__(StepLayout<LAYOUT>::THREADS) __attribute__((amdgpu_waves_per_eu(StepLayout<LAYOUT>::WAVES / 4)))
void step_rate_kernel(const char* src, int steps, float* sink) {
  using E = Elem<true>;
  constexpr int NW = StepLayout<LAYOUT>::WAVES;
  constexpr int LPW = 32 / NW;  // 1 KiB direct loads per wave and step (32 KiB per workgroup)
  __shared__ __attribute__((aligned(16))) char sKV[5 * SP_TILE];  // two K and three V tiles
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const StepFrag f(lane);
  for (int x = tid; x < 5 * SP_TILE / 4; x += 64 * NW) reinterpret_cast<uint32_t*>(sKV)[x] = 0x3f803f80u ^ (x & 7);
  __syncthreads();
  const float c = 0.0625f;
  const uint32_t voff = 16u * lane;
  float l = 0.f, acc = 0.f;
  auto issue_loads = [&](int s, int kb, int vb) {
#pragma unroll
    for (int u = 0; u < LPW; ++u) {
      const int k = wave * LPW + u;  // 16 K pieces, then 16 V pieces
      char* dst = sKV + (k < 16 ? ((kb ^ 1) * SP_TILE) : ((2 + (vb + 1) % 3) * SP_TILE)) + (k & 15) * 1024;
      const uint32_t lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)(dst);
      asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                   :
                   : "v"(voff), "s"(src + (s & 1) * 32768 + k * 1024), "s"(lds)
                   : "memory", "m0");
    }
  };
  auto expo = [&](float s0, float s1, uint32_t& w) {
    const float p0 = fast_exp2(fmaf(s0, c, -1.f));
    const float p1 = fast_exp2(fmaf(s1, c, -1.f));
    l += p0 + p1;
    w = E::pack2f(p0, p1);
    asm volatile("" : "+v"(w), "+v"(l));
  };
  if constexpr (LAYOUT == 0) {
    const bool lag = wave >= NW / 2;  // the second half of the waves runs the PV block first
    f32x16 O[4], S[2], Sn[2];
    u32x4 Qr[8], P[2][2];
#pragma unroll
    for (int i = 0; i < 4; ++i) O[i] = f32x16{};
#pragma unroll
    for (int i = 0; i < 2; ++i) S[i] = Sn[i] = f32x16{} + (float)lane;
#pragma unroll
    for (int i = 0; i < 8; ++i) Qr[i] = u32x4{0x3f80u + i, 0x3f81u, 0x3f82u, 0x3f83u};
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int h = 0; h < 2; ++h) P[j][h] = u32x4{0x3f803f80u, 0, 0, 0};
    for (int s = 0; s < steps; ++s) {
      const int kb = s & 1, vb = s % 3;
      const char* cK = sKV + kb * SP_TILE;
      const char* cV = sKV + (2 + vb) * SP_TILE;
      issue_loads(s, kb, vb);
      auto block_b = [&]() {
        __builtin_amdgcn_s_setprio(0);
        __builtin_amdgcn_sched_barrier(0);
        u32x4 vf[2] = {f.v(cV, 0, 0, 0), f.v(cV, 0, 0, 1)};
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          O[i % 4] = E::mfma32(vf[i & 1], P[i / 8][(i / 4) & 1], O[i % 4]);
          if (i + 2 < 16) vf[i & 1] = f.v(cV, (i + 2) / 8, ((i + 2) / 4) & 1, (i + 2) % 4);
          __builtin_amdgcn_sched_barrier(0);
        }
      };
      if (lag) block_b();
      __builtin_amdgcn_s_setprio(1);
      __builtin_amdgcn_sched_barrier(0);
      uint32_t pw[16];
      u32x4 kf[3] = {f.k(cK, 0, 0), f.k(cK, 1, 0), f.k(cK, 0, 1)};
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        Sn[i & 1] = E::mfma32(kf[i % 3], Qr[i >> 1], Sn[i & 1]);
        if (i + 3 < 16) kf[i % 3] = f.k(cK, (i + 3) & 1, (i + 3) >> 1);
        const int x = 2 * i, j = x >> 4, rr = x & 15;
        expo(S[j][rr], S[j][rr + 1], pw[i]);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          P[j][h] = u32x4{pw[8 * j + 4 * h], pw[8 * j + 4 * h + 1], pw[8 * j + 4 * h + 2], pw[8 * j + 4 * h + 3]};
      if (!lag) block_b();
      S[0] = Sn[0] * 0.5f;  // keeps the scores bounded
      S[1] = Sn[1] * 0.5f;
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
      __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc += O[i][e];
  } else if constexpr (LAYOUT == 1) {
    const bool lag = wave >= NW / 2;
    f32x4 O[8], S[4], Sn[4];
    u32x4 Qr[4], P[2];
#pragma unroll
    for (int i = 0; i < 8; ++i) O[i] = f32x4{};
#pragma unroll
    for (int i = 0; i < 4; ++i) S[i] = Sn[i] = f32x4{} + (float)lane;
#pragma unroll
    for (int i = 0; i < 4; ++i) Qr[i] = u32x4{0x3f80u + i, 0x3f81u, 0x3f82u, 0x3f83u};
#pragma unroll
    for (int j = 0; j < 2; ++j) P[j] = u32x4{0x3f803f80u, 0, 0, 0};
    for (int s = 0; s < steps; ++s) {
      const int kb = s & 1, vb = s % 3;
      const char* cK = sKV + kb * SP_TILE;
      const char* cV = sKV + (2 + vb) * SP_TILE;
      issue_loads(s, kb, vb);
      auto block_b = [&]() {
        __builtin_amdgcn_s_setprio(0);
        __builtin_amdgcn_sched_barrier(0);
        u32x4 vf[2] = {f.v(cV, 0, 0, 0), f.v(cV, 0, 0, 1)};
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          // O^T (128 d x 16 rows) += V^T (d tile i % 8) P^T (key half i / 8)
          O[i % 8] = E::mfma16(vf[i & 1], P[i / 8], O[i % 8]);
          if (i + 2 < 16) vf[i & 1] = f.v(cV, (i + 2) / 8, ((i + 2) / 4) & 1, (i + 2) % 4);
          __builtin_amdgcn_sched_barrier(0);
        }
      };
      if (lag) block_b();
      __builtin_amdgcn_s_setprio(1);
      __builtin_amdgcn_sched_barrier(0);
      // K fragments one product ahead (two ahead does not fit the 128 registers of four waves per SIMD)
      u32x4 kf = f.k(cK, 0, 0);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        // S^T (64 keys x 16 rows): key tile i % 4, d step i / 4
        Sn[i & 3] = E::mfma16(kf, Qr[i >> 2], Sn[i & 3]);
        if (i + 1 < 16) kf = f.k(cK, (i + 1) & 1, (i + 1) >> 1);
        if (i & 1) {  // 16 scores per lane: one pair of exponentials per two products, written into
                      // P directly (a lagging wave has already used this step's P)
          const int x = i - 1, j = x >> 2, rr = x & 3;
          uint32_t w;
          expo(S[j][rr], S[j][rr + 1], w);
          P[(i >> 1) >> 2][(i >> 1) & 3] = w;
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if (!lag) block_b();
#pragma unroll
      for (int i = 0; i < 4; ++i) S[i] = Sn[i] * 0.5f;
      __builtin_amdgcn_s_waitcnt(0x0F70);
      __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc += O[i][e];
  } else {
    // The products are inline asm so that S^T stays in VGPRs (the exponentials read it) and O^T in
    // AGPRs; the compiler otherwise gives both to AGPRs and copies 64 scores back per step.
    f32x16 O[2][4], S[2][2], Sn[2][2];
    u32x4 Qr[2][8], P[2][2][2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
#pragma unroll
      for (int i = 0; i < 4; ++i) O[r][i] = f32x16{};
#pragma unroll
      for (int i = 0; i < 2; ++i) S[r][i] = Sn[r][i] = f32x16{} + (float)lane;
#pragma unroll
      for (int i = 0; i < 8; ++i) Qr[r][i] = u32x4{0x3f80u + i + r, 0x3f81u, 0x3f82u, 0x3f83u};
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int h = 0; h < 2; ++h) P[r][j][h] = u32x4{0x3f803f80u, 0, 0, 0};
    }
    for (int s = 0; s < steps; ++s) {
      const int kb = s & 1, vb = s % 3;
      const char* cK = sKV + kb * SP_TILE;
      const char* cV = sKV + (2 + vb) * SP_TILE;
      issue_loads(s, kb, vb);
      __builtin_amdgcn_sched_barrier(0);
      // QK of the next tile: each K fragment feeds both 32-row blocks; this tile's 64 exponentials
      // per lane in between
      uint32_t pw[2][16];
      u32x4 kf[3] = {f.k(cK, 0, 0), f.k(cK, 1, 0), f.k(cK, 0, 1)};
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int x = 2 * i, j = x >> 4, rr = x & 15;
        sp_mfma_vgpr(Sn[0][i & 1], kf[i % 3], Qr[0][i >> 1]);
        expo(S[0][j][rr], S[0][j][rr + 1], pw[0][i]);
        sp_mfma_vgpr(Sn[1][i & 1], kf[i % 3], Qr[1][i >> 1]);
        expo(S[1][j][rr], S[1][j][rr + 1], pw[1][i]);
        if (i + 3 < 16) kf[i % 3] = f.k(cK, (i + 3) & 1, (i + 3) >> 1);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int h = 0; h < 2; ++h)
            P[r][j][h] = u32x4{pw[r][8 * j + 4 * h], pw[r][8 * j + 4 * h + 1], pw[r][8 * j + 4 * h + 2],
                               pw[r][8 * j + 4 * h + 3]};
      // PV of this tile: each V fragment feeds both row blocks
      u32x4 vf[2] = {f.v(cV, 0, 0, 0), f.v(cV, 0, 0, 1)};
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        sp_mfma_agpr(O[0][i % 4], vf[i & 1], P[0][i / 8][(i / 4) & 1]);
        sp_mfma_agpr(O[1][i % 4], vf[i & 1], P[1][i / 8][(i / 4) & 1]);
        if (i + 2 < 16) vf[i & 1] = f.v(cV, (i + 2) / 8, ((i + 2) / 4) & 1, (i + 2) % 4);
        __builtin_amdgcn_sched_barrier(0);
      }
      // the VALU reads of S^T below wait for the last products writing it (the compiler does not
      // track inline-asm products)
      asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        S[r][0] = Sn[r][0] * 0.5f;
        S[r][1] = Sn[r][1] * 0.5f;
      }
      __builtin_amdgcn_s_waitcnt(0x0F70);
      __syncthreads();
    }
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc += O[r][i][e];
  }
  sink[(int64_t)blockIdx.x * (64 * NW) + tid] = acc + l;
}

}  // namespace sa

extern "C" int sa_measure_cus(void) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
    cus = 256;
  return cus;
}

extern "C" int sa_mfma_rate(int per_cu, int iters, float* sink, int64_t sink_len, void* stream) {
  using namespace sa;
  clear_error();
  if (per_cu < 1 || per_cu > 8 || iters < 1) return set_error(SA_E_SHAPE, "sa_mfma_rate: per_cu %d (1..8), iters %d", per_cu, iters);
  if (!sink) return set_error(SA_E_NULL, "sa_mfma_rate: NULL sink");
  const int cus = sa_measure_cus();
  if (sink_len < (int64_t)MR_THREADS * per_cu * cus)
    return set_error(SA_E_SHAPE, "sa_mfma_rate: sink of %lld floats, needs %lld", (long long)sink_len,
                     (long long)MR_THREADS * per_cu * cus);
  hipLaunchKernelGGL(mfma_rate_kernel, dim3(cus * per_cu), dim3(MR_THREADS), 0, static_cast<hipStream_t>(stream),
                     iters, sink);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return set_error((int)err, "sa_mfma_rate: launch failed: %s", hipGetErrorString(err));
  return 0;
}

extern "C" int sa_lds_read_rate(int tr16, int iters, uint32_t* sink, int64_t sink_len, void* stream) {
  using namespace sa;
  clear_error();
  if (iters < 1) return set_error(SA_E_SHAPE, "sa_lds_read_rate: iters %d", iters);
  if (!sink) return set_error(SA_E_NULL, "sa_lds_read_rate: NULL sink");
  const int cus = sa_measure_cus();
  if (sink_len < (int64_t)LR_THREADS * cus)
    return set_error(SA_E_SHAPE, "sa_lds_read_rate: sink of %lld words, needs %lld", (long long)sink_len,
                     (long long)LR_THREADS * cus);
  if (tr16)
    hipLaunchKernelGGL(lds_rate_kernel<true>, dim3(cus), dim3(LR_THREADS), 0, static_cast<hipStream_t>(stream), iters, sink);
  else
    hipLaunchKernelGGL(lds_rate_kernel<false>, dim3(cus), dim3(LR_THREADS), 0, static_cast<hipStream_t>(stream), iters, sink);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return set_error((int)err, "sa_lds_read_rate: launch failed: %s", hipGetErrorString(err));
  return 0;
}

extern "C" int sa_stage_rate(const void* src, int64_t src_bytes, int iters, uint32_t* sink, int64_t sink_len,
                             void* stream) {
  using namespace sa;
  clear_error();
  if (iters < 1) return set_error(SA_E_SHAPE, "sa_stage_rate: iters %d", iters);
  if (!src || !sink) return set_error(SA_E_NULL, "sa_stage_rate: NULL pointer");
  if (src_bytes < 4 * LR_TILE) return set_error(SA_E_SHAPE, "sa_stage_rate: src of %lld bytes, needs %d", (long long)src_bytes, 4 * LR_TILE);
  if (reinterpret_cast<uintptr_t>(src) & 15) return set_error(SA_E_ALIGN, "sa_stage_rate: src must be 16-byte aligned");
  const int cus = sa_measure_cus();
  if (sink_len < (int64_t)ST_THREADS * cus)
    return set_error(SA_E_SHAPE, "sa_stage_rate: sink of %lld words, needs %lld", (long long)sink_len,
                     (long long)ST_THREADS * cus);
  hipLaunchKernelGGL(stage_rate_kernel, dim3(cus), dim3(ST_THREADS), 0, static_cast<hipStream_t>(stream),
                     static_cast<const char*>(src), iters, sink);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return set_error((int)err, "sa_stage_rate: launch failed: %s", hipGetErrorString(err));
  return 0;
}

extern "C" int sa_stream_read_workgroups(void) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
    cus = 256;
  return 8 * cus;
}

extern "C" int sa_stream_read(const void* src, int64_t bytes, uint32_t* sink, void* stream) {
  using namespace sa;
  clear_error();
  if (bytes < 0 || bytes % 16) return set_error(SA_E_SHAPE, "sa_stream_read: %lld bytes is not a multiple of 16", (long long)bytes);
  if (bytes == 0) return 0;
  if (!src || !sink) return set_error(SA_E_NULL, "sa_stream_read: NULL pointer");
  if (reinterpret_cast<uintptr_t>(src) & 15) return set_error(SA_E_ALIGN, "sa_stream_read: src must be 16-byte aligned");
  hipLaunchKernelGGL(stream_read_kernel, dim3(sa_stream_read_workgroups()), dim3(SR_THREADS), 0,
                     static_cast<hipStream_t>(stream), static_cast<const u32x4*>(src), bytes / 16, sink);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return set_error((int)err, "sa_stream_read: launch failed: %s", hipGetErrorString(err));
  return 0;
}

extern "C" int sa_step_rate_threads(int layout) {
  return layout == 0 ? sa::StepLayout<0>::THREADS : layout == 1 ? sa::StepLayout<1>::THREADS
                                                 : layout == 2 ? sa::StepLayout<2>::THREADS : -1;
}

extern "C" int sa_step_rate(int layout, const void* src, int64_t src_bytes, int steps, float* sink, int64_t sink_len,
                            void* stream) {
  using namespace sa;
  clear_error();
  const int threads = sa_step_rate_threads(layout);
  if (threads < 0) return set_error(SA_E_SHAPE, "sa_step_rate: layout %d (0, 1 or 2)", layout);
  if (steps < 1) return set_error(SA_E_SHAPE, "sa_step_rate: steps %d", steps);
  if (!src || !sink) return set_error(SA_E_NULL, "sa_step_rate: NULL pointer");
  if (src_bytes < 65536) return set_error(SA_E_SHAPE, "sa_step_rate: src of %lld bytes, needs 65536", (long long)src_bytes);
  if (reinterpret_cast<uintptr_t>(src) & 15) return set_error(SA_E_ALIGN, "sa_step_rate: src must be 16-byte aligned");
  const int cus = sa_measure_cus();
  if (sink_len < (int64_t)threads * cus)
    return set_error(SA_E_SHAPE, "sa_step_rate: sink of %lld floats, needs %lld", (long long)sink_len,
                     (long long)threads * cus);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const char* s = static_cast<const char*>(src);
  if (layout == 0)
    hipLaunchKernelGGL(step_rate_kernel<0>, dim3(cus), dim3(threads), 0, st, s, steps, sink);
  else if (layout == 1)
    hipLaunchKernelGGL(step_rate_kernel<1>, dim3(cus), dim3(threads), 0, st, s, steps, sink);
  else
    hipLaunchKernelGGL(step_rate_kernel<2>, dim3(cus), dim3(threads), 0, st, s, steps, sink);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return set_error((int)err, "sa_step_rate: launch failed: %s", hipGetErrorString(err));
  return 0;
}
