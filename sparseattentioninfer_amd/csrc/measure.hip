// Measurement aid: the HBM streaming-read rate of this GPU, the practical ceiling against which
// the memory-bound decode kernel is read (bench.py reports both in the same run).  Not part of the
// attention path.
//
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

}  // namespace sa

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
