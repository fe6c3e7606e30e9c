// Block mask -> CSR schedule on the GPU.
//
// Input: a byte block mask [R, NQB, NKB] (nonzero = retained).  Output: the reference's CSR
// (sparse_attentions/patterns/base.py:36-89 applied to a block mask):
//   offsets[r][qb] = number of retained blocks of row r before query block qb (offsets[r][0] = 0),
//   pairs[r][offsets[r][qb] ..] = the retained key blocks of (r, qb) in ascending order,
//   pairs[r][nnz_r ..] = 0 (padding to the common width).
// Two calls: the count pass writes offsets and nnz[r]; the caller sizes pairs to
// max(1, max_r nnz[r]) (the reference's width) and runs the write pass, which reads the
// offsets the count pass wrote.
//
// Every mask row is read by one wave with consecutive lanes on consecutive bytes (4 bytes per
// lane when the mask's strides, base and NKB allow, else 1), so each load instruction covers a
// contiguous 256- or 64-byte run:
//   count  - one wave per (row, query block): offsets[r][qb + 1] = popcount of the row;
//   scan   - one workgroup per row: prefix sum of those counts in place, nnz[r] = the total;
//   write  - one wave per (row, query block): an exclusive scan of the per-lane counts gives
//            every lane its slots; the row's padding past nnz[r] is zeroed.
#include "sa_common.h"

namespace sa {

constexpr int CSR_THREADS = 256;
constexpr int CSR_WAVES = CSR_THREADS / 64;

struct CsrArgs {
  const uint8_t* mask;
  int64_t mask_sr, mask_sq;  // byte strides of rows and query blocks (key blocks contiguous)
  int rows, nqb, nkb;
  int32_t* offsets;
  int64_t off_stride;
  int32_t* nnz;              // [R]
  int32_t* pairs;            // nullptr in the count pass
  int64_t pairs_stride, width;
  int* status;               // |= 1 when a row holds more than `width` blocks (write pass)
};

// Bytes [4j, 4j + 3] of a row as a word (VEC 4) or byte j (VEC 1); 0 past NKB.
template <int VEC>
__device__ __forceinline__ uint32_t load_piece(const uint8_t* m, int j, int nkb) {
  if constexpr (VEC == 4) {
    return 4 * j < nkb ? *reinterpret_cast<const uint32_t*>(m + 4 * j) : 0u;
  } else {
    return j < nkb ? (uint32_t)m[j] : 0u;
  }
}

// One bit per nonzero byte of w, at the byte's low bit.
__device__ __forceinline__ uint32_t nonzero_bytes(uint32_t w) {
  w |= w >> 4;
  w |= w >> 2;
  w |= w >> 1;
  return w & 0x01010101u;
}

template <int VEC>
__device__ __forceinline__ int piece_count(uint32_t w) {
  return VEC == 4 ? __builtin_popcount(nonzero_bytes(w)) : (w != 0);
}

// Exclusive prefix sum over the 64 lanes of a wave.
__device__ __forceinline__ int wave_exclusive_scan(int x, int lane) {
  int incl = x;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(incl, d, 64);
    if (lane >= d) incl += y;
  }
  return incl - x;
}

__device__ __forceinline__ int wave_sum(int x) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) x += __shfl_xor(x, d, 64);
  return x;
}

template <int VEC>
__global__ __launch_bounds__(CSR_THREADS) void csr_count_kernel(CsrArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = (int64_t)blockIdx.x * CSR_WAVES + (threadIdx.x >> 6);
  if (wid >= (int64_t)a.rows * a.nqb) return;
  const int qb = (int)(wid % a.nqb), r = (int)(wid / a.nqb);
  const uint8_t* m = a.mask + r * a.mask_sr + (int64_t)qb * a.mask_sq;
  const int pieces = VEC == 4 ? (a.nkb + 3) / 4 : a.nkb;
  int c = 0;
  for (int j = lane; j < pieces; j += 64) c += piece_count<VEC>(load_piece<VEC>(m, j, a.nkb));
  c = wave_sum(c);
  if (lane == 0) a.offsets[r * a.off_stride + qb + 1] = c;
}

__global__ __launch_bounds__(CSR_THREADS) void csr_scan_kernel(CsrArgs a) {
  __shared__ int s_wave[CSR_WAVES];
  const int r = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int32_t* off = a.offsets + r * a.off_stride;
  int base = 0;
  for (int q0 = 0; q0 < a.nqb; q0 += CSR_THREADS) {
    const int qb = q0 + tid;
    const int c = qb < a.nqb ? off[qb + 1] : 0;
    const int excl = wave_exclusive_scan(c, lane);
    if (lane == 63) s_wave[wave] = excl + c;
    __syncthreads();
    int before = base;
    for (int w = 0; w < wave; ++w) before += s_wave[w];
    if (qb < a.nqb) off[qb + 1] = before + excl + c;
    for (int w = 0; w < CSR_WAVES; ++w) base += s_wave[w];
    __syncthreads();  // s_wave reused by the next chunk
  }
  if (tid == 0) {
    off[0] = 0;
    a.nnz[r] = base;
  }
}

template <int VEC>
__global__ __launch_bounds__(CSR_THREADS) void csr_write_kernel(CsrArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = (int64_t)blockIdx.x * CSR_WAVES + (threadIdx.x >> 6);
  if (a.nqb == 0) {  // rows without query blocks: all padding
    if (wid < a.rows)
      for (int64_t x = lane; x < a.width; x += 64) a.pairs[wid * a.pairs_stride + x] = 0;
    return;
  }
  if (wid >= (int64_t)a.rows * a.nqb) return;
  const int qb = (int)(wid % a.nqb), r = (int)(wid / a.nqb);
  const uint8_t* m = a.mask + r * a.mask_sr + (int64_t)qb * a.mask_sq;
  int32_t* prow = a.pairs + r * a.pairs_stride;
  const int32_t* off = a.offsets + r * a.off_stride;
  const int start = off[qb], end = off[qb + 1];
  if (end > a.width && lane == 0) atomicOr(a.status, 1);
  const int pieces = VEC == 4 ? (a.nkb + 3) / 4 : a.nkb;
  int slot = start;
  for (int j0 = 0; j0 < pieces; j0 += 64) {
    const int j = j0 + lane;
    const uint32_t w = j < pieces ? load_piece<VEC>(m, j, a.nkb) : 0u;
    const int c = piece_count<VEC>(w);
    int x = slot + wave_exclusive_scan(c, lane);
    if constexpr (VEC == 4) {
      const uint32_t bits = nonzero_bytes(w);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if ((bits >> (8 * e)) & 1u) {
          if (x < a.width) prow[x] = 4 * j + e;
          ++x;
        }
    } else {
      if (c) {
        if (x < a.width) prow[x] = j;
      }
    }
    slot += wave_sum(c);
  }
  // The last query block of each row zeroes the row's padding.
  if (qb == a.nqb - 1)
    for (int64_t x = (int64_t)end + lane; x < a.width; x += 64) prow[x] = 0;
}

template <int VEC>
static void launch_passes(const CsrArgs& a, hipStream_t s) {
  const int64_t waves = (int64_t)a.rows * (a.nqb ? a.nqb : 1);
  const unsigned grid = (unsigned)ceil_div(waves, CSR_WAVES);
  if (a.pairs) {
    if (waves) hipLaunchKernelGGL(csr_write_kernel<VEC>, dim3(grid), dim3(CSR_THREADS), 0, s, a);
  } else {
    if (a.nqb) hipLaunchKernelGGL(csr_count_kernel<VEC>, dim3(grid), dim3(CSR_THREADS), 0, s, a);
    hipLaunchKernelGGL(csr_scan_kernel, dim3(a.rows), dim3(CSR_THREADS), 0, s, a);
  }
}

}  // namespace sa

extern "C" int sa_block_mask_to_csr(const uint8_t* mask, int64_t mask_row_stride, int64_t mask_qb_stride,
                                    int rows, int nqb, int nkb,
                                    int32_t* offsets, int64_t offsets_stride, int32_t* nnz,
                                    int32_t* pairs, int64_t pairs_stride, int64_t width,
                                    int* status, void* stream) {
  using namespace sa;
  clear_error();
  if (rows < 0 || nqb < 0 || nkb < 0)
    return set_error(SA_E_SHAPE, "sa_block_mask_to_csr: bad sizes rows=%d nqb=%d nkb=%d", rows, nqb, nkb);
  if (pairs && (width < 1 || !status))
    return set_error(SA_E_SHAPE, "sa_block_mask_to_csr: the write pass needs width >= 1 and a status word");
  if ((int64_t)nqb * nkb > 0x7fffffff)
    return set_error(SA_E_SHAPE, "sa_block_mask_to_csr: %d x %d blocks per row is too many", nqb, nkb);
  // One wave per (row, query block) in one launch, whose grid holds fewer than 2^32 threads.
  constexpr int64_t max_waves = ((int64_t)0xffffffff / CSR_THREADS) * CSR_WAVES;
  if ((int64_t)rows * nqb > max_waves)
    return set_error(SA_E_SHAPE, "sa_block_mask_to_csr: %d rows x %d query blocks is more than the %lld one launch covers",
                     rows, nqb, (long long)max_waves);
  if (rows == 0) return 0;
  if (!offsets || !nnz || (nqb && nkb && !mask)) return set_error(SA_E_NULL, "sa_block_mask_to_csr: NULL pointer");
  CsrArgs a;
  a.mask = mask; a.mask_sr = mask_row_stride; a.mask_sq = mask_qb_stride;
  a.rows = rows; a.nqb = nqb; a.nkb = nkb;
  a.offsets = offsets; a.off_stride = offsets_stride; a.nnz = nnz;
  a.pairs = pairs; a.pairs_stride = pairs_stride; a.width = width;
  a.status = status;
  const bool words = nkb % 4 == 0 && mask_qb_stride % 4 == 0 && mask_row_stride % 4 == 0 &&
                     (reinterpret_cast<uintptr_t>(mask) & 3) == 0;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (words)
    launch_passes<4>(a, s);
  else
    launch_passes<1>(a, s);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    return set_error((int)err, "sa_block_mask_to_csr: launch failed: %s", hipGetErrorString(err));
  return 0;
}
