// CSR block schedule at block size 16 or 32 -> schedule of 64 x 64 tiles with sub-block masks.
//
// The prefill kernel works on 64-row query tiles and 64-key tiles.  A schedule at a finer
// block size b (the reference's BigBird patterns use b = 16 or 32) is regrouped into tiles:
// query tile qt holds the query blocks qb = s*qt .. s*qt + s - 1 (s = 64 / b), and the tile
// schedule of (row r, qt) lists, in ascending order, every key tile kt holding a retained
// block kb (kt = kb / s) of one of those query blocks, with the mask
//   bit (qb % s) * s + (kb % s)  set  <=>  block kb is retained for query block qb.
// The tile schedule keeps the CSR layout of the input (one row per CSR row): tile_pairs
// [R, >= max tiles per row] (zero-padded), tile_masks likewise, tile_offsets [R, NQT + 1].
//
// One workgroup per CSR row: each thread merges the s ascending block lists of one query
// tile (first counting, then, after a workgroup prefix sum of the counts, writing).  Lists
// that are not ascending break the merge (a tile would be listed twice); they are reported
// in the status word instead of being sorted here.
#include "sa_common.h"

namespace sa {

constexpr int TILE_THREADS = 256;

struct TileArgs {
  const int32_t* pairs;
  int64_t pairs_stride;
  const int32_t* offsets;
  int64_t offsets_stride;
  int nqb, nqt, sub;  // query blocks, query tiles, blocks per tile edge
  int32_t* tile_pairs;
  int32_t* tile_masks;
  int64_t tile_stride;
  int32_t* tile_offsets;
  int64_t tile_offsets_stride;
  int64_t width;       // columns available in tile_pairs / tile_masks
  int* status;         // |= STATUS_OVERFLOW, STATUS_UNSORTED
};

constexpr int STATUS_OVERFLOW = 1;  // a row needs more than `width` tiles
constexpr int STATUS_UNSORTED = 2;  // a query block's ids are not ascending

// Walks the tiles of query tile qt of one row in ascending order; calls emit(kt, mask).
// Returns false if the tiles did not come out ascending (an input list was not).
template <typename Emit>
__device__ __forceinline__ bool merge_tiles(const TileArgs& a, const int32_t* prow, const int32_t* offs, int qt,
                                            Emit emit) {
  int pos[4], end[4];
  const int s = a.sub;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int qb = qt * s + i;
    if (i < s && qb < a.nqb) {
      pos[i] = offs[qb];
      end[i] = offs[qb + 1];
    } else {
      pos[i] = end[i] = 0;
    }
  }
  bool ascending = true;
  int last = -1;
  for (;;) {
    int kt = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      while (pos[i] < end[i] && prow[pos[i]] < 0) ++pos[i];  // malformed ids are dropped
      if (pos[i] < end[i]) kt = min(kt, prow[pos[i]] / s);
    }
    if (kt == 0x7fffffff) break;
    ascending &= kt > last;
    last = kt;
    uint32_t m = 0;
    // Negative ids between a tile's entries are skipped here too: tested only as id / s == kt, an
    // id in (-s, 0) would pass for kt = 0 (division truncates toward zero) and set a wrong bit.
#pragma unroll
    for (int i = 0; i < 4; ++i)
      while (pos[i] < end[i]) {
        const int id = prow[pos[i]];
        if (id >= 0 && id / s != kt) break;
        if (id >= 0) m |= 1u << (i * s + id % s);
        ++pos[i];
      }
    emit(kt, m);
  }
  return ascending;
}

__global__ __launch_bounds__(TILE_THREADS) void csr_to_tiles_kernel(TileArgs a) {
  __shared__ int s_scan[TILE_THREADS];
  const int r = blockIdx.x;
  const int tid = threadIdx.x;
  const int32_t* prow = a.pairs + r * a.pairs_stride;
  const int32_t* offs = a.offsets + r * a.offsets_stride;
  int32_t* toffs = a.tile_offsets + r * a.tile_offsets_stride;
  int32_t* tp = a.tile_pairs + r * a.tile_stride;
  int32_t* tm = a.tile_masks + r * a.tile_stride;

  // Query tiles are processed in chunks of TILE_THREADS, one per thread.
  int base = 0;  // tiles written by earlier chunks
  if (tid == 0) toffs[0] = 0;
  for (int q0 = 0; q0 < a.nqt; q0 += TILE_THREADS) {
    const int qt = q0 + tid;
    int count = 0;
    if (qt < a.nqt) merge_tiles(a, prow, offs, qt, [&](int, uint32_t) { ++count; });
    // inclusive prefix sum of the counts over the chunk (Hillis-Steele in LDS)
    s_scan[tid] = count;
    __syncthreads();
    for (int d = 1; d < TILE_THREADS; d <<= 1) {
      const int v = tid >= d ? s_scan[tid - d] : 0;
      __syncthreads();
      s_scan[tid] += v;
      __syncthreads();
    }
    const int start = base + s_scan[tid] - count;
    if (qt < a.nqt) {
      toffs[qt + 1] = start + count;
      int w = start;
      const bool ascending = merge_tiles(a, prow, offs, qt, [&](int kt, uint32_t m) {
        if (w < a.width) {
          tp[w] = kt;
          tm[w] = (int32_t)m;
        }
        ++w;
      });
      const int st = (w > a.width ? STATUS_OVERFLOW : 0) | (ascending ? 0 : STATUS_UNSORTED);
      if (st) atomicOr(a.status, st);
    }
    base += s_scan[TILE_THREADS - 1];
    __syncthreads();  // s_scan reused by the next chunk
  }
  // zero padding past the row's last tile
  for (int64_t x = base + tid; x < a.width; x += TILE_THREADS) {
    tp[x] = 0;
    tm[x] = 0;
  }
}

}  // namespace sa

extern "C" int sa_csr_to_tiles(const int32_t* pairs, int64_t pairs_stride,
                               const int32_t* offsets, int64_t offsets_stride,
                               int rows, int nqb, int block_size,
                               int32_t* tile_pairs, int32_t* tile_masks, int64_t tile_stride, int64_t width,
                               int32_t* tile_offsets, int64_t tile_offsets_stride,
                               int* status, void* stream) {
  using namespace sa;
  clear_error();
  if (block_size != 16 && block_size != 32)
    return set_error(SA_E_BLOCK, "sa_csr_to_tiles: block size %d is not 16 or 32", block_size);
  if (rows < 0 || nqb < 0 || width < 1)
    return set_error(SA_E_SHAPE, "sa_csr_to_tiles: bad sizes rows=%d nqb=%d width=%lld", rows, nqb,
                     (long long)width);
  if (rows == 0) return 0;
  if (!pairs || !offsets || !tile_pairs || !tile_masks || !tile_offsets || !status)
    return set_error(SA_E_NULL, "sa_csr_to_tiles: NULL pointer");
  TileArgs a;
  a.pairs = pairs; a.pairs_stride = pairs_stride;
  a.offsets = offsets; a.offsets_stride = offsets_stride;
  a.sub = 64 / block_size;
  a.nqb = nqb;
  a.nqt = (int)ceil_div(nqb, a.sub);
  a.tile_pairs = tile_pairs; a.tile_masks = tile_masks; a.tile_stride = tile_stride;
  a.tile_offsets = tile_offsets; a.tile_offsets_stride = tile_offsets_stride;
  a.width = width;
  a.status = status;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(csr_to_tiles_kernel, dim3(rows), dim3(TILE_THREADS), 0, s, a);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return set_error((int)err, "sa_csr_to_tiles: launch failed: %s", hipGetErrorString(err));
  return 0;
}
