// MFMA operand traits for gfx950 "NT" products (both operands K-contiguous in memory).
//
// v_mfma_f32_16x16x32_{bf16,f16}: lane l holds A[i = l%16][k = 8*(l/16) .. +7] and
// B[k = 8*(l/16) .. +7][j = l%16]; D[i = 4*(l/16) + r][j = l%16] (r = 0..3).
// v_mfma_f32_16x16x4_f32: the same with one k value per lane (k = l/16).
// With KPL k-values per lane per instruction, the kernels let lane group g = l/16 own
// the contiguous quarter [g*K/4, (g+1)*K/4) of the contraction and walk it in steps of
// KPL, so every operand fetch is one contiguous KPL-element vector of a row.
#pragma once

#include "common.h"

namespace hclsm {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

template <int DT> struct MM;

template <> struct MM<HCLSM_BF16> {
  using T = uint16_t;
  static constexpr int KPL = 8;
  using Op = bf16x8_t;
  static __device__ __forceinline__ Op load(const T* p) {
    return __builtin_bit_cast(Op, *reinterpret_cast<const uint4*>(p));
  }
  static __device__ __forceinline__ f32x4 mfma(Op a, Op b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float tof(T v) { return bf16_bits_to_f32(v); }
  static __device__ __forceinline__ T fromf(float v) { return f32_to_bf16_bits(v); }
};

template <> struct MM<HCLSM_F16> {
  using T = _Float16;
  static constexpr int KPL = 8;
  using Op = f16x8_t;
  static __device__ __forceinline__ Op load(const T* p) {
    return __builtin_bit_cast(Op, *reinterpret_cast<const uint4*>(p));
  }
  static __device__ __forceinline__ f32x4 mfma(Op a, Op b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float tof(T v) { return (float)v; }
  static __device__ __forceinline__ T fromf(float v) { return (_Float16)v; }
};

template <> struct MM<HCLSM_F32> {
  using T = float;
  static constexpr int KPL = 1;
  using Op = float;
  static __device__ __forceinline__ Op load(const T* p) { return *p; }
  static __device__ __forceinline__ f32x4 mfma(Op a, Op b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float tof(T v) { return v; }
  static __device__ __forceinline__ T fromf(float v) { return v; }
};

__device__ __forceinline__ float sigmoid_f(float x) { return 1.f / (1.f + __expf(-x)); }
__device__ __forceinline__ float tanh_f(float x) {
  // 1 - 2/(e^{2x}+1): saturates cleanly to +-1 at both ends
  return 1.f - 2.f / (__expf(2.f * x) + 1.f);
}

}  // namespace hclsm
