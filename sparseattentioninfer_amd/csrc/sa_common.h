// Shared device/host helpers for the gfx950 block-sparse attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/sparse_attn.h"

namespace sa {

// 16-bit element storage; the MFMA operand vectors reinterpret the same bits.
typedef uint16_t elem_t;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Records a message for sa_last_error(); returns `code` for tail calls.
int set_error(int code, const char* fmt, ...);
void clear_error();

// Element-type traits: conversion to/from fp32 and the 32x32x16 MFMA.
template <bool BF16>
struct Elem;

template <>
struct Elem<true> {
  static __device__ __forceinline__ float to_f32(elem_t x) {
    return __uint_as_float(static_cast<uint32_t>(x) << 16);
  }
  // Round-to-nearest-even fp32 -> bf16 (NaN kept quiet).
  static __device__ __forceinline__ elem_t from_f32(float f) {
    return __builtin_bit_cast(elem_t, static_cast<__bf16>(f));
  }
  // from_f32(lo) | from_f32(hi) << 16 in one v_cvt_pk_bf16_f32.
  static __device__ __forceinline__ uint32_t pack2f(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
  }
  static __device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // c + a.lo * b.lo + a.hi * b.hi over packed pairs, fp32 accumulate (v_dot2_f32_bf16).
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
  }
};

template <>
struct Elem<false> {
  static __device__ __forceinline__ float to_f32(elem_t x) {
    return static_cast<float>(__builtin_bit_cast(_Float16, x));
  }
  static __device__ __forceinline__ elem_t from_f32(float f) {
    return __builtin_bit_cast(elem_t, static_cast<_Float16>(f));
  }
  // from_f32(lo) | from_f32(hi) << 16.
  static __device__ __forceinline__ uint32_t pack2f(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, f16x2));
  }
  static __device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  // c + a.lo * b.lo + a.hi * b.hi over packed pairs, fp32 accumulate (v_dot2_f32_f16).
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c, false);
  }
};

// 2^x on the hardware transcendental unit (v_exp_f32); exp2(-inf) == 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Value held by lane (lane ^ 32): the other half of a wave64.
__device__ __forceinline__ float swap_halves(float x) { return __shfl_xor(x, 32, 64); }

__device__ __forceinline__ uint32_t pack2(elem_t lo, elem_t hi) {
  return static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// floor(n / d) for n < 2^32 and 1 <= d < 2^32, given m = floor((2^32 - 1) / d): m >= (2^32 - d)/d,
// so the high word of n*m is floor(n/d) or one less, and one compare corrects it.
__device__ __forceinline__ uint32_t fast_div(uint32_t n, uint32_t d, uint32_t m) {
  uint32_t q = __umulhi(n, m);
  q += (n - q * d >= d) ? 1u : 0u;
  return q;
}

// The multiplier m of fast_div for divisor d >= 1.
inline uint32_t div_mul(uint32_t d) { return 0xFFFFFFFFu / d; }

}  // namespace sa
