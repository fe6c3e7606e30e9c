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
constexpr int NORM_MAX_PER_THREAD = 32;  // hidden sizes up to 8192

// One workgroup per row: r = residual + x (rounded; stored back) when residual is given,
// else r = x; out = w * rnd(r * rsqrt(mean(r^2) + eps)) rounded.
template <bool BF16>
__global__ __launch_bounds__(NORM_THREADS) void rmsnorm_kernel(const elem_t* x, int64_t x_st, elem_t* res,
                                                               int64_t res_st, const elem_t* w, elem_t* out,
                                                               int64_t out_st, int n, float eps) {
  __shared__ float s_part[NORM_THREADS / 64];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const elem_t* xr = x + row * x_st;
  elem_t* rr = res ? res + row * res_st : nullptr;
  float v[NORM_MAX_PER_THREAD];
  float ss = 0.f;
#pragma unroll
  for (int u = 0; u < NORM_MAX_PER_THREAD; ++u) {
    const int i = tid + u * NORM_THREADS;
    v[u] = 0.f;
    if (i < n) {
      float r = ld<BF16>(xr + i);
      if (rr) {
        r = rnd<BF16>(ld<BF16>(rr + i) + r);
        rr[i] = Elem<BF16>::from_f32(r);
      }
      v[u] = r;
      ss += r * r;
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
  for (int u = 0; u < NORM_MAX_PER_THREAD; ++u) {
    const int i = tid + u * NORM_THREADS;
    if (i < n) orow[i] = Elem<BF16>::from_f32(ld<BF16>(w + i) * rnd<BF16>(v[u] * inv));
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
  if (rows < 0 || n < 1 || n > NORM_THREADS * NORM_MAX_PER_THREAD)
    return set_error(SA_E_SHAPE, "sa_rmsnorm: rows=%d, n=%d (1 <= n <= %d)", rows, n,
                     NORM_THREADS * NORM_MAX_PER_THREAD);
  if (rows == 0) return 0;
  if (!x || !weight || !out) return set_error(SA_E_NULL, "sa_rmsnorm: NULL tensor pointer");
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
