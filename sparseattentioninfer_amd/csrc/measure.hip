// Measurement aids: the HBM streaming-read rate of this GPU, the practical ceiling against which
// the memory-bound decode kernel is read, and the dense bf16 matrix-core rate and LDS fragment-read
// rates that bound the prefill kernel (bench.py reports them beside the kernels, in the same run).
// Not part of the attention path.
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
