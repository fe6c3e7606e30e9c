// Fused elementwise kernels of one decode step of a Qwen3 decoder layer (gfx950).
//
// The decode step of the end-to-end workload moves one token per sequence through each
// layer; between its matrix products the work is small row-wise arithmetic that Hugging Face
// runs as many separate kernels.  These kernels keep Hugging Face's arithmetic (fp32 inside,
// rounding to the element type where it rounds) with one launch per stage:
//  * sa_rmsnorm:      optional residual add (residual += x, rounded), then Qwen3RMSNorm
//                     (transformers/models/qwen3/modeling_qwen3.py Qwen3RMSNorm.forward);
//  * sa_qk_rope_kv:   per-head q/k RMSNorm, rotary embedding (apply_rotary_pos_emb with
//                     rotate_half, cos/sin of inv_freq * position) and the paged K/V write of
//                     the new token (the reference caller's cache update,
//                     sparse_llm/qwen3/integrations/modeling_sparse_qwen3.py:220-234);
//  * sa_swiglu:       act(gate) * up of Qwen3MLP with SiLU.
// One wave per row (head) or one workgroup per row; positions come from device memory so the
// launches can be captured in a graph and replayed at every step.
#include <algorithm>

#include "sa_common.h"

namespace sa {

template <bool BF16>
__device__ __forceinline__ float ld(const elem_t* p) { return Elem<BF16>::to_f32(*p); }

template <bool BF16>
__device__ __forceinline__ float rnd(float x) { return Elem<BF16>::to_f32(Elem<BF16>::from_f32(x)); }

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o, 64);
  return x;
}

constexpr int NORM_THREADS = 256;
constexpr int NORM_MAX_CHUNKS = 4;  // 16-byte chunks (8 elements) per thread: hidden sizes up to 8192

template <bool BF16>
__device__ __forceinline__ float lo_f(uint32_t v) { return Elem<BF16>::to_f32((elem_t)(v & 0xffffu)); }
template <bool BF16>
__device__ __forceinline__ float hi_f(uint32_t v) { return Elem<BF16>::to_f32((elem_t)(v >> 16)); }

// One workgroup per row: r = residual + x (rounded; stored back) when residual is given,
// else r = x; out = w * rnd(r * rsqrt(mean(r^2) + eps)) rounded.  n a multiple of 8 and rows
// 16-byte aligned: thread t owns the 16-byte chunks t, t + NORM_THREADS, ...  Every load of the
// row is issued before the first store: the stores may alias the inputs as far as the compiler
// knows, so interleaving them would serialise the row into one memory round trip per chunk.
template <bool BF16>
__global__ __launch_bounds__(NORM_THREADS) void rmsnorm_kernel(const elem_t* x, int64_t x_st, elem_t* res,
                                                               int64_t res_st, const elem_t* w, elem_t* out,
                                                               int64_t out_st, int n, float eps) {
  __shared__ float s_part[NORM_THREADS / 64];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int nch = n / 8;
  const elem_t* xr = x + row * x_st;
  elem_t* rr = res ? res + row * res_st : nullptr;
  u32x4 xv[NORM_MAX_CHUNKS], rv[NORM_MAX_CHUNKS], wv[NORM_MAX_CHUNKS];
#pragma unroll
  for (int j = 0; j < NORM_MAX_CHUNKS; ++j) {
    const int c = tid + j * NORM_THREADS;
    xv[j] = rv[j] = wv[j] = u32x4{0u, 0u, 0u, 0u};
    if (c < nch) {
      xv[j] = *reinterpret_cast<const u32x4*>(xr + 8 * c);
      if (rr) rv[j] = *reinterpret_cast<const u32x4*>(rr + 8 * c);
      wv[j] = *reinterpret_cast<const u32x4*>(w + 8 * c);
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NORM_MAX_CHUNKS; ++j) {
    if (tid + j * NORM_THREADS >= nch) continue;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float l = lo_f<BF16>(xv[j][e]), h = hi_f<BF16>(xv[j][e]);
      if (rr) {
        l = rnd<BF16>(lo_f<BF16>(rv[j][e]) + l);
        h = rnd<BF16>(hi_f<BF16>(rv[j][e]) + h);
      }
      ss += l * l;
      ss += h * h;
      xv[j][e] = Elem<BF16>::pack2f(l, h);
    }
  }
  if (rr) {
#pragma unroll
    for (int j = 0; j < NORM_MAX_CHUNKS; ++j) {
      const int c = tid + j * NORM_THREADS;
      if (c < nch) *reinterpret_cast<u32x4*>(rr + 8 * c) = xv[j];
    }
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) s_part[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int k = 0; k < NORM_THREADS / 64; ++k) tot += s_part[k];
  const float inv = rsqrtf(tot / (float)n + eps);
  elem_t* orow = out + row * out_st;
#pragma unroll
  for (int j = 0; j < NORM_MAX_CHUNKS; ++j) {
    const int c = tid + j * NORM_THREADS;
    if (c >= nch) continue;
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = Elem<BF16>::pack2f(lo_f<BF16>(wv[j][e]) * rnd<BF16>(lo_f<BF16>(xv[j][e]) * inv),
                                hi_f<BF16>(wv[j][e]) * rnd<BF16>(hi_f<BF16>(xv[j][e]) * inv));
    *reinterpret_cast<u32x4*>(orow + 8 * c) = o;
  }
}

// One wave per (sequence, head) of the fused q|k|v projection row: heads [0, Hq) are query
// heads (q_norm + rotary -> q_out), [Hq, Hq + Hkv) key heads (k_norm + rotary -> k pages),
// [Hq + Hkv, Hq + 2 Hkv) value heads (-> v pages).  D = 128: lane l owns dims l and l + 64,
// which are exactly the pair that rotate_half mixes.
template <bool BF16>
__global__ __launch_bounds__(256) void qk_rope_kv_kernel(const elem_t* qkv, int64_t qkv_st, const elem_t* qw,
                                                         const elem_t* kw, const float* inv_freq,
                                                         const int64_t* pos, elem_t* q_out, int64_t qo_sb,
                                                         int64_t qo_sh, elem_t* k_pages, elem_t* v_pages,
                                                         int64_t pg_sp, int64_t pg_sh, int64_t pg_st,
                                                         const int32_t* block_table, int64_t bt_stride,
                                                         int max_blocks, int num_pages, int B, int Hq, int Hkv,
                                                         int page, float eps) {
  constexpr int D = 128;
  const int lane = threadIdx.x & 63;
  const int gw = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int nh = Hq + 2 * Hkv;
  if (gw >= B * nh) return;
  const int b = gw / nh, h = gw % nh;
  const elem_t* src = qkv + b * qkv_st + h * D;
  float x0 = ld<BF16>(src + lane), x1 = ld<BF16>(src + lane + 64);
  const int64_t p = pos[0];
  if (h < Hq + Hkv) {
    const elem_t* w = h < Hq ? qw : kw;
    const float inv = rsqrtf(wave_sum(x0 * x0 + x1 * x1) / (float)D + eps);
    x0 = rnd<BF16>(ld<BF16>(w + lane) * rnd<BF16>(x0 * inv));
    x1 = rnd<BF16>(ld<BF16>(w + lane + 64) * rnd<BF16>(x1 * inv));
    // emb = cat(freqs, freqs): dims l and l + 64 share the angle inv_freq[l] * p
    const float ang = inv_freq[lane] * (float)p;
    const float c = rnd<BF16>(cosf(ang)), s = rnd<BF16>(sinf(ang));
    const float y0 = rnd<BF16>(rnd<BF16>(x0 * c) + rnd<BF16>(-x1 * s));
    const float y1 = rnd<BF16>(rnd<BF16>(x1 * c) + rnd<BF16>(x0 * s));
    x0 = y0;
    x1 = y1;
  }
  elem_t* dst;
  if (h < Hq) {
    dst = q_out + b * qo_sb + h * qo_sh;
  } else {
    // Positions past the table or pages outside the pool are not written (the host checks both).
    const int64_t lb = p / page;
    if (p < 0 || lb >= max_blocks) return;
    const int pg = block_table[b * bt_stride + lb];
    if (pg < 0 || pg >= num_pages) return;
    const int kvh = h < Hq + Hkv ? h - Hq : h - Hq - Hkv;
    dst = (h < Hq + Hkv ? k_pages : v_pages) + pg * pg_sp + kvh * pg_sh + (p % page) * pg_st;
  }
  dst[lane] = Elem<BF16>::from_f32(x0);
  dst[lane + 64] = Elem<BF16>::from_f32(x1);
}

// out[b, i] = rnd(rnd(silu(g)) * u), g = gu[b, i], u = gu[b, I + i].
template <bool BF16>
__global__ __launch_bounds__(256) void swiglu_kernel(const elem_t* gu, int64_t gu_st, elem_t* out, int64_t out_st,
                                                     int B, int I) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)B * I) return;
  const int b = (int)(t / I), i = (int)(t % I);
  const float g = ld<BF16>(gu + b * gu_st + i);
  const float u = ld<BF16>(gu + b * gu_st + I + i);
  const float a = rnd<BF16>(g / (1.f + expf(-g)));
  out[b * out_st + i] = Elem<BF16>::from_f32(a * u);
}


}  // namespace sa

using namespace sa;

extern "C" int sa_rmsnorm(int dtype, const void* x, int64_t x_stride, void* residual, int64_t residual_stride,
                          const void* weight, void* out, int64_t out_stride, int rows, int n, float eps,
                          void* stream) {
  clear_error();
  if (dtype != SA_DTYPE_BF16 && dtype != SA_DTYPE_F16)
    return set_error(SA_E_DTYPE, "sa_rmsnorm: dtype %d is not bf16 (0) or f16 (1)", dtype);
  if (rows < 0 || n < 8 || n % 8 || n > NORM_THREADS * NORM_MAX_CHUNKS * 8)
    return set_error(SA_E_SHAPE, "sa_rmsnorm: rows=%d, n=%d (a multiple of 8, 8 <= n <= %d)", rows, n,
                     NORM_THREADS * NORM_MAX_CHUNKS * 8);
  if (rows == 0) return 0;
  if (!x || !weight || !out) return set_error(SA_E_NULL, "sa_rmsnorm: NULL tensor pointer");
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(residual) | reinterpret_cast<uintptr_t>(weight) |
       reinterpret_cast<uintptr_t>(out)) & 15 || x_stride % 8 || out_stride % 8 || (residual && residual_stride % 8))
    return set_error(SA_E_ALIGN, "sa_rmsnorm: rows must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto xe = static_cast<const elem_t*>(x);
  auto re = static_cast<elem_t*>(residual);
  auto we = static_cast<const elem_t*>(weight);
  auto oe = static_cast<elem_t*>(out);
  if (dtype == SA_DTYPE_BF16)
    hipLaunchKernelGGL(rmsnorm_kernel<true>, dim3(rows), dim3(NORM_THREADS), 0, s, xe, x_stride, re,
                       residual_stride, we, oe, out_stride, n, eps);
  else
    hipLaunchKernelGGL(rmsnorm_kernel<false>, dim3(rows), dim3(NORM_THREADS), 0, s, xe, x_stride, re,
                       residual_stride, we, oe, out_stride, n, eps);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : set_error((int)err, "sa_rmsnorm: launch failed: %s", hipGetErrorString(err));
}

extern "C" int sa_qk_rope_kv(int dtype, const void* qkv, int64_t qkv_stride, const void* q_norm_weight,
                             const void* k_norm_weight, const float* inv_freq, const int64_t* position,
                             void* q_out, int64_t q_out_sb, int64_t q_out_sh,
                             void* k_pages, void* v_pages, int64_t pages_sp, int64_t pages_sh, int64_t pages_st,
                             const int32_t* block_table, int64_t block_table_stride, int max_blocks,
                             int num_pages, int B, int Hq, int Hkv, int D, int page, float eps, void* stream) {
  clear_error();
  if (dtype != SA_DTYPE_BF16 && dtype != SA_DTYPE_F16)
    return set_error(SA_E_DTYPE, "sa_qk_rope_kv: dtype %d is not bf16 (0) or f16 (1)", dtype);
  if (D != 128) return set_error(SA_E_HEADDIM, "sa_qk_rope_kv: head dim %d not supported (128)", D);
  if (B < 0 || Hq < 1 || Hkv < 1 || Hq % Hkv || page < 1)
    return set_error(SA_E_SHAPE, "sa_qk_rope_kv: bad sizes B=%d Hq=%d Hkv=%d page=%d", B, Hq, Hkv, page);
  if (B == 0) return 0;
  if (!qkv || !q_norm_weight || !k_norm_weight || !inv_freq || !position || !q_out || !k_pages || !v_pages ||
      !block_table)
    return set_error(SA_E_NULL, "sa_qk_rope_kv: NULL pointer");
  const int waves = B * (Hq + 2 * Hkv);
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto in = static_cast<const elem_t*>(qkv);
  auto qw = static_cast<const elem_t*>(q_norm_weight);
  auto kw = static_cast<const elem_t*>(k_norm_weight);
  auto qo = static_cast<elem_t*>(q_out);
  auto kp = static_cast<elem_t*>(k_pages);
  auto vp = static_cast<elem_t*>(v_pages);
  const dim3 grid((waves + 3) / 4), block(256);
  if (dtype == SA_DTYPE_BF16)
    hipLaunchKernelGGL(qk_rope_kv_kernel<true>, grid, block, 0, s, in, qkv_stride, qw, kw, inv_freq, position, qo,
                       q_out_sb, q_out_sh, kp, vp, pages_sp, pages_sh, pages_st, block_table, block_table_stride,
                       max_blocks, num_pages, B, Hq, Hkv, page, eps);
  else
    hipLaunchKernelGGL(qk_rope_kv_kernel<false>, grid, block, 0, s, in, qkv_stride, qw, kw, inv_freq, position,
                       qo, q_out_sb, q_out_sh, kp, vp, pages_sp, pages_sh, pages_st, block_table,
                       block_table_stride, max_blocks, num_pages, B, Hq, Hkv, page, eps);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : set_error((int)err, "sa_qk_rope_kv: launch failed: %s", hipGetErrorString(err));
}

extern "C" int sa_swiglu(int dtype, const void* gate_up, int64_t gate_up_stride, void* out, int64_t out_stride,
                         int B, int I, void* stream) {
  clear_error();
  if (dtype != SA_DTYPE_BF16 && dtype != SA_DTYPE_F16)
    return set_error(SA_E_DTYPE, "sa_swiglu: dtype %d is not bf16 (0) or f16 (1)", dtype);
  if (B < 0 || I < 1) return set_error(SA_E_SHAPE, "sa_swiglu: bad sizes B=%d I=%d", B, I);
  if (B == 0) return 0;
  if (!gate_up || !out) return set_error(SA_E_NULL, "sa_swiglu: NULL pointer");
  const int64_t n = (int64_t)B * I;
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto in = static_cast<const elem_t*>(gate_up);
  auto oe = static_cast<elem_t*>(out);
  const dim3 grid((unsigned)((n + 255) / 256)), block(256);
  if (dtype == SA_DTYPE_BF16)
    hipLaunchKernelGGL(swiglu_kernel<true>, grid, block, 0, s, in, gate_up_stride, oe, out_stride, B, I);
  else
    hipLaunchKernelGGL(swiglu_kernel<false>, grid, block, 0, s, in, gate_up_stride, oe, out_stride, B, I);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : set_error((int)err, "sa_swiglu: launch failed: %s", hipGetErrorString(err));
}

// ---- skinny GEMM: out[m, n] = sum_k x[m, k] * W[n, k], M <= 8 (decode-step projections) ----
//
// Weight-streaming bound (each W element is used M <= 8 times).  A workgroup of 256 threads owns
// batches of R consecutive rows of W; thread t owns the 16-byte chunks c = t, t + 256, ... of the
// K dimension and keeps x's matching chunks for every m in registers for the whole kernel, so W
// is the only operand streamed.  A thread issues all its loads of a batch's W rows at once, and
// for R <= 4 with K in at most two chunks per thread the next batch's rows load while the
// current batch is multiplied and reduced.  Per batch a thread forms R * 8 partial sums with
// packed dot products; a butterfly (each step hands half of the values to the partner lane and adds the
// other half) leaves the wave's sum of value (lane mod R * 8) in each lane, and the four waves'
// partials of an output are added through LDS.  fp32 accumulation, one rounding of the output.
namespace sa {

constexpr int SK_THREADS = 256;
constexpr int SK_M = 8;      // max rows of x
constexpr int SK_MAXC = 5;   // 16-byte chunks of K per thread: K <= 5 * 256 * 8 = 10240

template <bool BF16, int NC, int R, bool PF>
__global__ __launch_bounds__(SK_THREADS) void skinny_gemm_kernel(const elem_t* x, int64_t x_st, const elem_t* w,
                                                                 int64_t w_st, elem_t* out, int64_t out_st, int M,
                                                                 int N, int K) {
  constexpr int V = R * SK_M;                          // partial sums per thread and batch
  constexpr int LV = V == 64 ? 6 : V == 32 ? 5 : 4;    // log2(V)
  static_assert(V == 16 || V == 32 || V == 64, "R must be 2, 4 or 8");
  __shared__ float s_red[SK_THREADS / 64][V];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kc = K / 8;  // 16-byte chunks
  uint32_t xr[NC][SK_M][4];
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int c = tid + j * SK_THREADS;
#pragma unroll
    for (int m = 0; m < SK_M; ++m) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (c < kc && m < M) v = *reinterpret_cast<const u32x4*>(x + m * x_st + 8 * c);
#pragma unroll
      for (int e = 0; e < 4; ++e) xr[j][m][e] = v[e];
    }
  }
  const int nb = (N + R - 1) / R;
  // This thread's NC chunks of the R rows of W in batch bt (zeros past the end).
  auto load_w = [&](int bt, u32x4 (&wv)[NC][R]) {
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const int c = tid + j * SK_THREADS;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int n = bt * R + r;
        wv[j][r] = (bt < nb && c < kc && n < N) ? *reinterpret_cast<const u32x4*>(w + (int64_t)n * w_st + 8 * c)
                                                : u32x4{0u, 0u, 0u, 0u};
      }
    }
  };
  // Dot products, reduction over the workgroup and store of batch bt.
  auto batch = [&](int bt, const u32x4 (&wv)[NC][R]) {
    const int n0 = bt * R;
    float acc[V];
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = 0.f;
#pragma unroll
    for (int j = 0; j < NC; ++j)
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < SK_M; ++m) {
          float a = acc[r * SK_M + m];
#pragma unroll
          for (int e = 0; e < 4; ++e) a = Elem<BF16>::dot2(wv[j][r][e], xr[j][m][e], a);
          acc[r * SK_M + m] = a;
        }
    // Butterfly over lane bits LV-1 .. 0: at step s the partner is lane ^ half (half = V >> (s+1));
    // the lane whose bit is set keeps the upper half of its values.  Afterwards acc[0] holds the sum,
    // over the lanes that differ only in bits below LV, of value index (lane & (V - 1)).
#pragma unroll
    for (int s = 0; s < LV; ++s) {
      const int half = V >> (s + 1);
      const bool upper = lane & half;
#pragma unroll
      for (int i = 0; i < half; ++i) {
        const float give = upper ? acc[i] : acc[i + half];
        const float keep = upper ? acc[i + half] : acc[i];
        acc[i] = keep + __shfl_xor(give, half, 64);
      }
    }
#pragma unroll
    for (int b = V; b < 64; b <<= 1) acc[0] += __shfl_xor(acc[0], b, 64);
    if (lane < V) s_red[wave][lane] = acc[0];
    __syncthreads();
    if (tid < V) {
      const int r = tid / SK_M, m = tid % SK_M;
      const float v = s_red[0][tid] + s_red[1][tid] + s_red[2][tid] + s_red[3][tid];
      if (m < M && n0 + r < N) out[m * out_st + n0 + r] = Elem<BF16>::from_f32(v);
    }
    __syncthreads();
  };
  if constexpr (PF) {
    // The next batch's rows load while this one is multiplied and reduced; two register sets
    // trade roles, so nothing is copied.
    u32x4 wa[NC][R], wb[NC][R];
    int bt = blockIdx.x;
    load_w(bt, wa);
    while (bt < nb) {
      load_w(bt + gridDim.x, wb);
      batch(bt, wa);
      bt += gridDim.x;
      if (bt >= nb) break;
      load_w(bt + gridDim.x, wa);
      batch(bt, wb);
      bt += gridDim.x;
    }
  } else {
    for (int bt = blockIdx.x; bt < nb; bt += gridDim.x) {
      u32x4 wv[NC][R];
      load_w(bt, wv);
      batch(bt, wv);
    }
  }
}

static int num_cus_layer() {
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

template <bool BF16, int R>
static void launch_skinny_r(const elem_t* x, int64_t x_st, const elem_t* w, int64_t w_st, elem_t* out,
                            int64_t out_st, int M, int N, int K, int per_cu, hipStream_t s) {
  const int nb = (N + R - 1) / R;
  const int grid = std::min(nb, per_cu * num_cus_layer());
  const int nc = (K / 8 + SK_THREADS - 1) / SK_THREADS;
  const dim3 g(grid), b(SK_THREADS);
  constexpr bool PF = R <= 4;  // registers for two sets of W chunks when NC <= 2
  switch (nc) {
    case 1: hipLaunchKernelGGL((skinny_gemm_kernel<BF16, 1, R, PF>), g, b, 0, s, x, x_st, w, w_st, out, out_st, M, N, K); break;
    case 2: hipLaunchKernelGGL((skinny_gemm_kernel<BF16, 2, R, PF>), g, b, 0, s, x, x_st, w, w_st, out, out_st, M, N, K); break;
    case 3: hipLaunchKernelGGL((skinny_gemm_kernel<BF16, 3, R, false>), g, b, 0, s, x, x_st, w, w_st, out, out_st, M, N, K); break;
    case 4: hipLaunchKernelGGL((skinny_gemm_kernel<BF16, 4, R, false>), g, b, 0, s, x, x_st, w, w_st, out, out_st, M, N, K); break;
    default: hipLaunchKernelGGL((skinny_gemm_kernel<BF16, 5, R, false>), g, b, 0, s, x, x_st, w, w_st, out, out_st, M, N, K); break;
  }
}

// ---- skinny GEMM on the matrix cores, W staged through LDS ----------------------------------
// out[m, n] = sum_k x[m, k] * W[n, k] for M <= 8 and K a multiple of 128.  A workgroup of NWV
// waves owns 16 NWV output columns (16 per wave) over all of K, in stages of 128 K: the stage's W
// rows (16 NWV x 256 bytes) and x rows (8 x 256 bytes) go global -> LDS with direct loads in whole
// contiguous rows, each load permuting the 16-byte chunks of its row so that chunk c of row r
// lands at position c ^ (r & 15).  Each wave then reads its 16 W rows (the B operand, one
// k-chunk per 16-lane group: conflict-free thanks to the permutation) and the x rows (the A
// operand; rows 8-15 of the 16-row product are never stored) and runs one v_mfma_f32_16x16x32
// per 32 K.  SL_NS stages are in flight; one barrier per stage.
constexpr int SL_KC = 128;  // K per stage
constexpr int SL_NS = 4;    // stages in flight

__device__ __forceinline__ uint32_t sl_lds(const void* p) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)(p);
}

// 16 bytes per lane from a per-lane address into LDS at M0 + 16 lane.
__device__ __forceinline__ void sl_load16(const void* vaddr, uint32_t lds) {
  asm volatile(
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, off"
      :
      : "v"(vaddr), "s"(lds)
      : "memory", "m0");
}

// NWV waves, 16 output columns each.  A stage holds the workgroup's 16 NWV W rows and the 8 x
// rows (each wave loads its own W rows, 4 KiB, and 8 / NWV of the x rows).
// ACT: W's rows are Qwen3MLP's gate and up rows interleaved (row 2i = gate i, row 2i + 1 = up i)
// and out[m, i] = SwiGLU of the pair, rounded as sa_gemm_skinny then sa_swiglu round it (the
// pair sits in adjacent lanes of one wave).
template <bool BF16, int NWV, bool ACT>
__global__ __launch_bounds__(64 * NWV) void skinny_lds_kernel(const elem_t* x, int64_t x_st, const elem_t* w,
                                                              int64_t w_st, elem_t* out, int64_t out_st, int M,
                                                              int N, int K) {
  constexpr int WB = 16 * NWV * SL_KC * 2;       // W bytes per stage
  constexpr int SB = WB + 8 * SL_KC * 2;         // + x bytes
  constexpr int XR = 8 / NWV;                    // x rows loaded per wave
  constexpr int XI = (XR * 256 + 1023) / 1024;   // their direct loads
  constexpr int LOADS = 4 + XI;                  // direct loads per wave per stage
  __shared__ __attribute__((aligned(16))) char sm[SL_NS * SB];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n0 = blockIdx.x * 16 * NWV;
  const int nst = K / SL_KC;
  const int p = lane & 15;  // position within a 256-byte LDS row
  // This lane's load rows: W rows 16 wave + 4 i + lane / 16 (i < 4); x row XR wave + 4 j + lane / 16.
  const elem_t* wsrc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 16 * wave + 4 * i + (lane >> 4);
    wsrc[i] = w + (int64_t)min(n0 + r, N - 1) * w_st + 8 * (p ^ (r & 15));
  }
  const elem_t* xsrc[XI];
#pragma unroll
  for (int j = 0; j < XI; ++j) {
    const int xr = XR * wave + 4 * j + (lane >> 4);
    xsrc[j] = x + (int64_t)min(xr, M - 1) * x_st + 8 * (p ^ (xr & 15));
  }
  const uint32_t base = sl_lds(sm);
  auto issue = [&](int st) {
    const uint32_t b = base + (st % SL_NS) * SB;
    const int k0 = st * SL_KC;
#pragma unroll
    for (int i = 0; i < 4; ++i) sl_load16(wsrc[i] + k0, b + 1024 * (4 * wave + i));
#pragma unroll
    for (int j = 0; j < XI; ++j)
      if (XR >= 4 || lane < XR * 16) sl_load16(xsrc[j] + k0, b + WB + 256 * XR * wave + 1024 * j);
  };
  // Operand offsets within a stage: B = W row 16 wave + lane % 16, A = x row (lane % 16) & 7;
  // k-chunk 4 ks + lane / 16.
  const int g = lane >> 4;
  const int rb = 16 * wave + p, ra = p & 7;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int st = 0; st < SL_NS - 1; ++st)
    if (st < nst) issue(st);
  for (int st = 0; st < nst; ++st) {
    const int after = min(SL_NS - 2, nst - 1 - st);  // stages issued after this one
    if (after >= 2)
      __builtin_amdgcn_s_waitcnt(0x0F70 | ((2 * LOADS) & 15) | (((2 * LOADS) >> 4) << 14));
    else if (after == 1)
      __builtin_amdgcn_s_waitcnt(0x0F70 | LOADS);
    else
      __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
    if (st + SL_NS - 1 < nst) issue(st + SL_NS - 1);
    const char* sb = sm + (st % SL_NS) * SB;
#pragma unroll
    for (int ks = 0; ks < SL_KC / 32; ++ks) {
      const int c = 4 * ks + g;
      const u32x4 bw = *reinterpret_cast<const u32x4*>(sb + rb * 256 + 16 * (c ^ (rb & 15)));
      const u32x4 ax = *reinterpret_cast<const u32x4*>(sb + WB + ra * 256 + 16 * (c ^ ra));
      acc = Elem<BF16>::mfma16(ax, bw, acc);
    }
  }
  // D of the 16x16 product: lane l holds rows 4 (l / 16) + i of column l % 16.
  const int n = n0 + 16 * wave + p;
  if constexpr (ACT) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float v = rnd<BF16>(acc[i]);     // the gate|up output as stored
      const float u = __shfl_xor(v, 1, 64);  // up of the pair, for the even lane
      const int m = 4 * g + i;
      if (!(p & 1) && m < M && n + 1 < N) {
        const float a = rnd<BF16>(v / (1.f + expf(-v)));
        out[m * out_st + n / 2] = Elem<BF16>::from_f32(a * u);
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = 4 * g + i;
    if (m < M && n < N) out[m * out_st + n] = Elem<BF16>::from_f32(acc[i]);
  }
}

// Two waves (32 columns) per workgroup: measured best against one and four at the Qwen3-4B decode
// shapes with the weights streamed from HBM (q|k|v 8.0 us, gate|up 21 us, LM head 134 us).
constexpr int SL_NWV = 2;

// Dot-product kernel: rows per batch and workgroups per CU, measured at the Qwen3-4B decode shapes
// with the weights streamed from HBM: wide products (N >= 64 per CU: gate|up, LM head) take 4 rows per batch and
// three workgroups per CU; the others 2 rows, with four workgroups per CU while K fits two
// chunks per thread (q|k|v, o) and two past that (down, where each workgroup's x is large).
template <bool BF16>
static void launch_skinny(const elem_t* x, int64_t x_st, const elem_t* w, int64_t w_st, elem_t* out,
                          int64_t out_st, int M, int N, int K, hipStream_t s) {
  // Wide products with K a multiple of 128 run on the matrix cores with W staged through LDS
  // (q|k|v, gate|up and the LM head of Qwen3-4B: 20-30 % faster); narrower ones (o, down: 80
  // column tiles) keep more workgroups busy on the dot-product kernel.
  if (K % SL_KC == 0 && N >= 24 * num_cus_layer()) {
    hipLaunchKernelGGL((skinny_lds_kernel<BF16, SL_NWV, false>), dim3((N + 16 * SL_NWV - 1) / (16 * SL_NWV)),
                       dim3(64 * SL_NWV), 0, s, x, x_st, w, w_st, out, out_st, M, N, K);
    return;
  }
  if (N >= 64 * num_cus_layer())
    launch_skinny_r<BF16, 4>(x, x_st, w, w_st, out, out_st, M, N, K, 3, s);
  else
    launch_skinny_r<BF16, 2>(x, x_st, w, w_st, out, out_st, M, N, K, K > 2 * SK_THREADS * 8 ? 2 : 4, s);
}


}  // namespace sa

extern "C" int sa_gemm_skinny(int dtype, const void* x, int64_t x_stride, const void* w, int64_t w_stride, void* out,
                              int64_t out_stride, int M, int N, int K, void* stream) {
  using namespace sa;
  clear_error();
  if (dtype != SA_DTYPE_BF16 && dtype != SA_DTYPE_F16)
    return set_error(SA_E_DTYPE, "sa_gemm_skinny: dtype %d is not bf16 (0) or f16 (1)", dtype);
  if (M < 0 || M > SK_M || N < 0 || K < 8 || K % 8 || K > SK_MAXC * SK_THREADS * 8)
    return set_error(SA_E_SHAPE, "sa_gemm_skinny: M=%d (<= %d), N=%d, K=%d (multiple of 8, <= %d)", M, SK_M, N, K,
                     SK_MAXC * SK_THREADS * 8);
  if (M == 0 || N == 0) return 0;
  if (!x || !w || !out) return set_error(SA_E_NULL, "sa_gemm_skinny: NULL pointer");
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) & 15 || x_stride % 8 || w_stride % 8)
    return set_error(SA_E_ALIGN, "sa_gemm_skinny: x and W rows must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto xe = static_cast<const elem_t*>(x);
  auto we = static_cast<const elem_t*>(w);
  auto oe = static_cast<elem_t*>(out);
  if (dtype == SA_DTYPE_BF16)
    launch_skinny<true>(xe, x_stride, we, w_stride, oe, out_stride, M, N, K, s);
  else
    launch_skinny<false>(xe, x_stride, we, w_stride, oe, out_stride, M, N, K, s);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : set_error((int)err, "sa_gemm_skinny: launch failed: %s", hipGetErrorString(err));
}

extern "C" int sa_gemm_skinny_swiglu(int dtype, const void* x, int64_t x_stride, const void* w_gate_up,
                                     int64_t w_stride, void* out, int64_t out_stride, int M, int I, int K,
                                     void* stream) {
  using namespace sa;
  clear_error();
  if (dtype != SA_DTYPE_BF16 && dtype != SA_DTYPE_F16)
    return set_error(SA_E_DTYPE, "sa_gemm_skinny_swiglu: dtype %d is not bf16 (0) or f16 (1)", dtype);
  if (M < 0 || M > SK_M || I < 0 || K < SL_KC || K % SL_KC)
    return set_error(SA_E_SHAPE, "sa_gemm_skinny_swiglu: M=%d (<= %d), I=%d, K=%d (a multiple of %d)", M, SK_M, I,
                     K, SL_KC);
  if (M == 0 || I == 0) return 0;
  if (!x || !w_gate_up || !out) return set_error(SA_E_NULL, "sa_gemm_skinny_swiglu: NULL pointer");
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w_gate_up)) & 15 || x_stride % 8 || w_stride % 8)
    return set_error(SA_E_ALIGN, "sa_gemm_skinny_swiglu: x and W rows must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int N = 2 * I;
  const dim3 g((N + 16 * SL_NWV - 1) / (16 * SL_NWV)), b(64 * SL_NWV);
  auto xe = static_cast<const elem_t*>(x);
  auto we = static_cast<const elem_t*>(w_gate_up);
  auto oe = static_cast<elem_t*>(out);
  if (dtype == SA_DTYPE_BF16)
    hipLaunchKernelGGL((skinny_lds_kernel<true, SL_NWV, true>), g, b, 0, s, xe, x_stride, we, w_stride, oe,
                       out_stride, M, N, K);
  else
    hipLaunchKernelGGL((skinny_lds_kernel<false, SL_NWV, true>), g, b, 0, s, xe, x_stride, we, w_stride, oe,
                       out_stride, M, N, K);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0
                           : set_error((int)err, "sa_gemm_skinny_swiglu: launch failed: %s", hipGetErrorString(err));
}
