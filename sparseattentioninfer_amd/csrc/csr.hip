// Block mask -> CSR schedule on the GPU.
//
// Input: a bool block mask [R, NQB, NKB] (one byte per block, nonzero = retained).  Output: the
// reference's CSR (sparse_attentions/patterns/base.py:36-89 applied to a block mask):
//   offsets[r][qb] = number of retained blocks of row r before query block qb (offsets[r][0] = 0),
//   pairs[r][offsets[r][qb] ..] = the retained key blocks of (r, qb) in ascending order,
//   pairs[r][nnz_r ..] = 0 (padding to the common width).
// Two launches: the count pass writes offsets and nnz[r]; the caller sizes pairs to
// max(1, max_r nnz[r]) (the reference's width) and runs the write pass.
//
// One 256-thread workgroup per row: each thread counts (then writes) the query blocks
// qb = tid, tid + 256, ...; a workgroup prefix sum over chunks of 256 query blocks gives the
// offsets.
#include "sa_common.h"

namespace sa {

constexpr int CSR_THREADS = 256;

struct CsrArgs {
  const uint8_t* mask;
  int64_t mask_sr, mask_sq;  // byte strides of rows and query blocks (key blocks contiguous)
  int nqb, nkb;
  int32_t* offsets;
  int64_t off_stride;
  int32_t* nnz;              // [R]
  int32_t* pairs;            // nullptr in the count pass
  int64_t pairs_stride, width;
  int* status;               // |= 1 when a row holds more than `width` blocks (write pass)
};

__device__ __forceinline__ int count_row(const uint8_t* m, int nkb) {
  int c = 0;
  for (int kb = 0; kb < nkb; ++kb) c += m[kb] != 0;
  return c;
}

__global__ __launch_bounds__(CSR_THREADS) void block_mask_to_csr_kernel(CsrArgs a) {
  __shared__ int s_scan[CSR_THREADS];
  const int r = blockIdx.x;
  const int tid = threadIdx.x;
  const uint8_t* mrow = a.mask + r * a.mask_sr;
  int32_t* off = a.offsets + r * a.off_stride;
  int32_t* prow = a.pairs ? a.pairs + r * a.pairs_stride : nullptr;
  int base = 0;
  if (tid == 0) off[0] = 0;
  for (int q0 = 0; q0 < a.nqb; q0 += CSR_THREADS) {
    const int qb = q0 + tid;
    const uint8_t* m = mrow + qb * a.mask_sq;
    const int cnt = qb < a.nqb ? count_row(m, a.nkb) : 0;
    // inclusive prefix sum of the counts over the chunk (Hillis-Steele in LDS)
    s_scan[tid] = cnt;
    __syncthreads();
    for (int d = 1; d < CSR_THREADS; d <<= 1) {
      const int v = tid >= d ? s_scan[tid - d] : 0;
      __syncthreads();
      s_scan[tid] += v;
      __syncthreads();
    }
    const int end = base + s_scan[tid];
    if (qb < a.nqb) {
      off[qb + 1] = end;
      if (prow) {
        int w = end - cnt;
        for (int kb = 0; kb < a.nkb; ++kb)
          if (m[kb]) {
            if (w < a.width) prow[w] = kb;
            ++w;
          }
        if (end > a.width) atomicOr(a.status, 1);
      }
    }
    base += s_scan[CSR_THREADS - 1];
    __syncthreads();  // s_scan reused by the next chunk
  }
  if (tid == 0) a.nnz[r] = base;
  if (prow)
    for (int64_t x = base + tid; x < a.width; x += CSR_THREADS) prow[x] = 0;
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
  if (rows == 0) return 0;
  if (!mask || !offsets || !nnz) return set_error(SA_E_NULL, "sa_block_mask_to_csr: NULL pointer");
  CsrArgs a;
  a.mask = mask; a.mask_sr = mask_row_stride; a.mask_sq = mask_qb_stride;
  a.nqb = nqb; a.nkb = nkb;
  a.offsets = offsets; a.off_stride = offsets_stride; a.nnz = nnz;
  a.pairs = pairs; a.pairs_stride = pairs_stride; a.width = width;
  a.status = status;
  hipLaunchKernelGGL(block_mask_to_csr_kernel, dim3(rows), dim3(CSR_THREADS), 0, static_cast<hipStream_t>(stream), a);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    return set_error((int)err, "sa_block_mask_to_csr: launch failed: %s", hipGetErrorString(err));
  return 0;
}
