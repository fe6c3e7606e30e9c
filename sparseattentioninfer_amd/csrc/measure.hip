// Measurement aid: the HBM streaming-read rate of this GPU, the practical ceiling against which
// the memory-bound decode kernel is read (bench.py reports both in the same run).  Not part of the
// attention path.
//
// Every thread of a grid of 8 workgroups per CU reads 16-byte pieces of `src` in a grid-stride
// loop, eight non-temporal loads in flight, and folds them with xor into one word per workgroup (written to
// sink[blockIdx.x], so the loads cannot be dropped).  Pieces past the last whole group of eight
// strides are read by the tail loop.
#include "sa_common.h"

namespace sa {

constexpr int SR_THREADS = 256;

__global__ __launch_bounds__(SR_THREADS) void stream_read_kernel(const u32x4* src, int64_t n, uint32_t* sink) {
  __shared__ uint32_t s_acc[SR_THREADS / 64];
  const int64_t stride = (int64_t)gridDim.x * SR_THREADS;
  int64_t i = (int64_t)blockIdx.x * SR_THREADS + threadIdx.x;
  u32x4 acc = {0, 0, 0, 0};
  for (; i + 7 * stride < n; i += 8 * stride) {
    u32x4 x[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) x[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
    for (int u = 0; u < 8; ++u) acc ^= x[u];
  }
  for (; i < n; i += stride) acc ^= src[i];
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
