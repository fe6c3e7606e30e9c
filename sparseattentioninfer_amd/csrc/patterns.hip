// Block-mask generators on the GPU: the retained key blocks of every (CSR row, query block) as a
// byte mask [rows][NQB][mask_qb_stride] (1 = retained, 0 = not; bytes past NKB are written 0),
// ready for sa_block_mask_to_csr with no host round trip.
//
// * Reference BigBird (sparse_attentions/patterns/bigbird_pattern.py:23-41, :246-255): per row
//   a layout (g, s, r); query block qa = qbo + i keeps the global blocks [0, g), the window
//   [max(0, qa - s + 1), min(qa + 1, NKB)) and r "random" blocks that are a rotation of the
//   candidates [g, min(qa, max(g, qa - s + 1))) by (131 * head + 17 * qa + 7 * hash_blocks) mod n
//   (all of them when n <= r).  The rotation is the reference's own formula, kept so that the
//   schedules are bit-identical.  Optionally the last query block keeps every block
//   (BigBird2Pattern, bigbird_pattern.py:697-806).  Each mask byte is a closed-form test, one
//   thread per 16 bytes.
// * Seeded BigBird and Bernoulli, this build's benchmark generators, on the counter-based
//   Philox4x64-10 generator (Salmon, Moraes, Dror, Shaw, SC'11): the draw of block kb of
//   query block qa in row `row` is the first 64-bit word of philox(counter = (kb, qa, row, 0),
//   key = (seed, stream)), stream 1 for BigBird's random picks and 2 for Bernoulli.
//     - Bernoulli: kb < qa is kept iff (draw >> 11) < floor(density * 2^53); the diagonal
//       qa (clipped to NKB - 1) is kept; nothing above it.
//     - Seeded BigBird: the global prefix, the window (trailing {qa-w+1..qa} or centred
//       {qa-w/2..qa+w/2}) and the diagonal, causal-truncated, plus counts[row] random blocks:
//       the eligible (causal, not already kept) blocks with the smallest (draw, kb).  A first
//       kernel writes everything but the random picks (one thread per 16 bytes); a second
//       kernel, one wave per (row, query block), takes the counts[row] smallest draws.
#include <algorithm>

#include "sa_common.h"

namespace sa {

constexpr int PAT_THREADS = 256;

// ---- Philox4x64-10 ---------------------------------------------------------------------
struct u64x4 {
  uint64_t x[4];
};

__device__ __forceinline__ uint64_t philox_first(uint64_t c0, uint64_t c1, uint64_t c2, uint64_t c3, uint64_t k0,
                                                 uint64_t k1) {
  constexpr uint64_t M0 = 0xD2E7470EE14C6C93ull, M1 = 0xCA5A826395121157ull;
  constexpr uint64_t W0 = 0x9E3779B97F4A7C15ull, W1 = 0xBB67AE8584CAA73Bull;
#pragma unroll
  for (int i = 0; i < 10; ++i) {
    if (i > 0) {
      k0 += W0;
      k1 += W1;
    }
    const uint64_t hi0 = __umul64hi(M0, c0), lo0 = M0 * c0;
    const uint64_t hi1 = __umul64hi(M1, c2), lo1 = M1 * c2;
    const uint64_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0;
    c1 = lo1;
    c2 = n2;
    c3 = lo0;
  }
  return c0;
}

__device__ __forceinline__ uint64_t block_draw(uint64_t seed, uint64_t stream, int row, int qa, int kb) {
  return philox_first((uint64_t)(uint32_t)kb, (uint64_t)(uint32_t)qa, (uint64_t)(uint32_t)row, 0ull, seed, stream);
}

// ---- byte-parallel fill ------------------------------------------------------------------
enum FillKind : int { FILL_BIGBIRD_HASH = 0, FILL_SEEDED_BASE = 1, FILL_BERNOULLI = 2 };

struct FillArgs {
  uint8_t* mask;
  int64_t mask_sr, mask_sq;  // byte strides of rows and query blocks (multiples of 16)
  int rows, nqb, nkb, qbo;
  int kind;
  // reference BigBird
  const int32_t* layout;     // [rows][3]: g, s, r
  int head_base;             // hash head of row `row` = head_base + row
  int hash_blocks;           // num_blocks in the hash
  int dense_last;            // last query block keeps every block
  // seeded BigBird base
  int window, global_blocks, centred;
  // Bernoulli
  uint64_t seed;
  uint64_t threshold;        // keep iff (draw >> 11) < threshold
};

__device__ __forceinline__ bool fill_bit(const FillArgs& a, int row, int i, int kb) {
  if (kb >= a.nkb) return false;
  if (a.kind == FILL_BIGBIRD_HASH) {
    if (a.dense_last && i == a.nqb - 1) return true;
    const int qa = a.qbo + i;
    const int g = a.layout[3 * row], s = a.layout[3 * row + 1], r = a.layout[3 * row + 2];
    if (kb < g) return true;
    if (kb >= max(0, qa - s + 1) && kb <= qa) return true;
    if (r <= 0 || qa <= 0) return false;
    const int cand_end = min(qa, max(g, qa - s + 1));
    const int n = cand_end - g;
    if (n <= 0 || kb < g || kb >= cand_end) return false;
    if (n <= r) return true;
    const int64_t h = (int64_t)(a.head_base + row);
    const int rot = (int)((h * 131 + (int64_t)qa * 17 + (int64_t)a.hash_blocks * 7) % n);
    int pos = kb - g - rot;  // position of kb in the rotated candidate list
    if (pos < 0) pos += n;
    return pos < r;
  }
  const int qa = min(a.qbo + i, a.nkb - 1);  // causal limit of the query block
  if (kb > qa) return false;
  if (kb == qa) return true;
  if (a.kind == FILL_SEEDED_BASE) {
    if (kb < a.global_blocks) return true;
    const int lo = a.centred ? qa - a.window / 2 : qa - a.window + 1;
    const int hi = a.centred ? qa + a.window / 2 : qa;
    return kb >= lo && kb <= hi;
  }
  return (block_draw(a.seed, 2, row, qa, kb) >> 11) < a.threshold;  // FILL_BERNOULLI
}

__global__ __launch_bounds__(PAT_THREADS) void block_mask_fill_kernel(FillArgs a) {
  const int64_t chunks = a.mask_sq / 16;  // 16-byte pieces per query block
  const int64_t total = (int64_t)a.rows * a.nqb * chunks;
  for (int64_t t = (int64_t)blockIdx.x * PAT_THREADS + threadIdx.x; t < total; t += (int64_t)gridDim.x * PAT_THREADS) {
    const int64_t c = t % chunks;
    const int64_t ri = t / chunks;
    const int i = (int)(ri % a.nqb);
    const int row = (int)(ri / a.nqb);
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t v = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) v |= (uint32_t)fill_bit(a, row, i, (int)(16 * c + 4 * q + e)) << (8 * e);
      w[q] = v;
    }
    *reinterpret_cast<u32x4*>(a.mask + row * a.mask_sr + (int64_t)i * a.mask_sq + 16 * c) = u32x4{w[0], w[1], w[2], w[3]};
  }
}

// ---- seeded random picks -----------------------------------------------------------------
struct PickArgs {
  uint8_t* mask;
  int64_t mask_sr, mask_sq;
  int rows, nqb, nkb, qbo;
  int window, global_blocks, centred;
  const int32_t* counts;  // [rows] random blocks per query block
  uint64_t seed;
};

__device__ __forceinline__ bool less_key(uint64_t u, int kb, uint64_t v, int kc) {
  return u < v || (u == v && kb < kc);
}

// One wave per (row, query block); PAT_THREADS / 64 of them per workgroup.  Round j takes the
// eligible block with the smallest (draw, kb) greater than round j - 1's, so the picks are the
// counts[row] smallest keys, found without replacement and independent of lane timing.
__global__ __launch_bounds__(PAT_THREADS) void block_mask_pick_kernel(PickArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = (int64_t)blockIdx.x * (PAT_THREADS / 64) + (threadIdx.x >> 6);
  if (wid >= (int64_t)a.rows * a.nqb) return;
  const int i = (int)(wid % a.nqb);
  const int row = (int)(wid / a.nqb);
  const int qa = min(a.qbo + i, a.nkb - 1);
  const int lo = a.centred ? qa - a.window / 2 : qa - a.window + 1;
  const int hi = a.centred ? qa + a.window / 2 : qa;
  uint8_t* m = a.mask + row * a.mask_sr + (int64_t)i * a.mask_sq;
  const int count = a.counts[row];
  uint64_t prev_u = 0;
  int prev_kb = -1;  // (0, -1) precedes every key
  for (int j = 0; j < count; ++j) {
    uint64_t best_u = ~0ull;
    int best_kb = 0x7fffffff;
    for (int kb = lane; kb < qa; kb += 64) {  // eligible: causal, not global / window / diagonal
      if (kb < a.global_blocks || (kb >= lo && kb <= hi)) continue;
      const uint64_t u = block_draw(a.seed, 1, row, qa, kb);
      if (less_key(prev_u, prev_kb, u, kb) && less_key(u, kb, best_u, best_kb)) {
        best_u = u;
        best_kb = kb;
      }
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
      const uint64_t ou = __shfl_xor(best_u, d, 64);
      const int okb = __shfl_xor(best_kb, d, 64);
      if (less_key(ou, okb, best_u, best_kb)) {
        best_u = ou;
        best_kb = okb;
      }
    }
    if (best_kb == 0x7fffffff) break;  // fewer eligible blocks than count: all taken
    if (lane == 0) m[best_kb] = 1;
    prev_u = best_u;
    prev_kb = best_kb;
  }
}

static int fill_launch(const FillArgs& a, void* stream, const char* name) {
  const int64_t total = (int64_t)a.rows * a.nqb * (a.mask_sq / 16);
  if (total == 0) return 0;
  const int64_t grid = std::min<int64_t>(ceil_div(total, PAT_THREADS), 65536);
  hipLaunchKernelGGL(block_mask_fill_kernel, dim3((unsigned)grid), dim3(PAT_THREADS), 0,
                     static_cast<hipStream_t>(stream), a);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return set_error((int)err, "%s: launch failed: %s", name, hipGetErrorString(err));
  return 0;
}

static int check_mask(const char* name, const uint8_t* mask, int64_t mask_sr, int64_t mask_sq, int rows, int nqb,
                      int nkb) {
  if (rows < 0 || nqb < 0 || nkb < 1)
    return set_error(SA_E_SHAPE, "%s: bad sizes rows=%d nqb=%d nkb=%d", name, rows, nqb, nkb);
  if (mask_sq % 16 || mask_sq < nkb || mask_sr % 16 || (rows > 1 && mask_sr < (int64_t)nqb * mask_sq))
    return set_error(SA_E_ALIGN, "%s: mask strides (%lld, %lld) must be multiples of 16 holding %d x %d bytes", name,
                     (long long)mask_sr, (long long)mask_sq, nqb, nkb);
  if (rows && nqb && !mask) return set_error(SA_E_NULL, "%s: NULL mask", name);
  if (reinterpret_cast<uintptr_t>(mask) & 15) return set_error(SA_E_ALIGN, "%s: mask must be 16-byte aligned", name);
  return 0;
}

}  // namespace sa

extern "C" int sa_bigbird_block_mask(uint8_t* mask, int64_t mask_row_stride, int64_t mask_qb_stride, int rows,
                                     int nqb, int nkb, int q_block_offset, const int32_t* layout, int head_base,
                                     int hash_blocks, int dense_last_block, void* stream) {
  using namespace sa;
  clear_error();
  const char* name = "sa_bigbird_block_mask";
  if (int rc = check_mask(name, mask, mask_row_stride, mask_qb_stride, rows, nqb, nkb)) return rc;
  if (rows && nqb && !layout) return set_error(SA_E_NULL, "%s: NULL layout", name);
  if (q_block_offset < 0 || hash_blocks < 0 || head_base < 0)
    return set_error(SA_E_SHAPE, "%s: negative offset / hash blocks / head base", name);
  FillArgs a{};
  a.mask = mask; a.mask_sr = mask_row_stride; a.mask_sq = mask_qb_stride;
  a.rows = rows; a.nqb = nqb; a.nkb = nkb; a.qbo = q_block_offset;
  a.kind = FILL_BIGBIRD_HASH;
  a.layout = layout; a.head_base = head_base; a.hash_blocks = hash_blocks; a.dense_last = dense_last_block != 0;
  return fill_launch(a, stream, name);
}

extern "C" int sa_seeded_bigbird_block_mask(uint8_t* mask, int64_t mask_row_stride, int64_t mask_qb_stride, int rows,
                                            int nqb, int nkb, int q_block_offset, int window, int global_blocks,
                                            int centred, const int32_t* random_counts, uint64_t seed, void* stream) {
  using namespace sa;
  clear_error();
  const char* name = "sa_seeded_bigbird_block_mask";
  if (int rc = check_mask(name, mask, mask_row_stride, mask_qb_stride, rows, nqb, nkb)) return rc;
  if (rows && nqb && !random_counts) return set_error(SA_E_NULL, "%s: NULL random_counts", name);
  if (q_block_offset < 0 || window < 0 || global_blocks < 0)
    return set_error(SA_E_SHAPE, "%s: negative offset / window / global", name);
  FillArgs a{};
  a.mask = mask; a.mask_sr = mask_row_stride; a.mask_sq = mask_qb_stride;
  a.rows = rows; a.nqb = nqb; a.nkb = nkb; a.qbo = q_block_offset;
  a.kind = FILL_SEEDED_BASE;
  a.window = window; a.global_blocks = global_blocks; a.centred = centred != 0;
  if (int rc = fill_launch(a, stream, name)) return rc;
  const int64_t waves = (int64_t)rows * nqb;
  if (waves == 0) return 0;
  PickArgs p{};
  p.mask = mask; p.mask_sr = mask_row_stride; p.mask_sq = mask_qb_stride;
  p.rows = rows; p.nqb = nqb; p.nkb = nkb; p.qbo = q_block_offset;
  p.window = window; p.global_blocks = global_blocks; p.centred = centred != 0;
  p.counts = random_counts; p.seed = seed;
  const int64_t grid = ceil_div(waves, PAT_THREADS / 64);
  if (grid > 0x7fffffff) return set_error(SA_E_SHAPE, "%s: too many query blocks", name);
  hipLaunchKernelGGL(block_mask_pick_kernel, dim3((unsigned)grid), dim3(PAT_THREADS), 0,
                     static_cast<hipStream_t>(stream), p);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return set_error((int)err, "%s: launch failed: %s", name, hipGetErrorString(err));
  return 0;
}

extern "C" int sa_bernoulli_block_mask(uint8_t* mask, int64_t mask_row_stride, int64_t mask_qb_stride, int rows,
                                       int nqb, int nkb, int q_block_offset, double density, uint64_t seed,
                                       void* stream) {
  using namespace sa;
  clear_error();
  const char* name = "sa_bernoulli_block_mask";
  if (int rc = check_mask(name, mask, mask_row_stride, mask_qb_stride, rows, nqb, nkb)) return rc;
  if (!(density >= 0.0 && density <= 1.0)) return set_error(SA_E_SHAPE, "%s: density %g outside [0, 1]", name, density);
  if (q_block_offset < 0) return set_error(SA_E_SHAPE, "%s: negative query block offset", name);
  FillArgs a{};
  a.mask = mask; a.mask_sr = mask_row_stride; a.mask_sq = mask_qb_stride;
  a.rows = rows; a.nqb = nqb; a.nkb = nkb; a.qbo = q_block_offset;
  a.kind = FILL_BERNOULLI;
  a.seed = seed;
  a.threshold = density >= 1.0 ? (1ull << 53) : (uint64_t)(density * 9007199254740992.0);  // floor(d * 2^53)
  return fill_launch(a, stream, name);
}
