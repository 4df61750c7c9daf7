// Shared device helpers for the gfx950 kernels of libhclsm_amd.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/hclsm_amd.h"

#define HCLSM_LOG2E 1.4426950408889634f
#define HCLSM_LN2 0.6931471805599453f

namespace hclsm {

// ---- element types ---------------------------------------------------------
// Tensors of bf16 are handled as raw uint16_t bit patterns; conversions are
// explicit so the generated code is exactly the shift / round we want.
struct bf16 { uint16_t bits; };

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Round-to-nearest-even conversions; gfx950 does these with v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2_t r;
  r.x = (__bf16)lo;
  r.y = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, r);
}

template <int DT> struct Elem;
template <> struct Elem<HCLSM_F32> {
  using T = float;
  static __device__ __forceinline__ float ld(const T* p) { return *p; }
  static __device__ __forceinline__ void st(T* p, float v) { *p = v; }
};
template <> struct Elem<HCLSM_BF16> {
  using T = uint16_t;
  static __device__ __forceinline__ float ld(const T* p) { return bf16_bits_to_f32(*p); }
  static __device__ __forceinline__ void st(T* p, float v) { *p = f32_to_bf16_bits(v); }
};
template <> struct Elem<HCLSM_F16> {
  using T = _Float16;
  static __device__ __forceinline__ float ld(const T* p) { return (float)(*p); }
  static __device__ __forceinline__ void st(T* p, float v) { *p = (_Float16)v; }
};

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// softplus(v) = max(v, 0) + log1p(exp(-|v|)), torch's threshold 20 kept.  log1p(e) for e in (0, 1] as
// log(u) * e / (u - 1) with u = 1 + e (the rounding of u cancels to first order; e / (u - 1) = 1
// when u rounds to 1).
__device__ __forceinline__ float softplus_f(float v) {
  const float e = __expf(-fabsf(v));
  const float u = 1.f + e;
  const float d = u - 1.f;
  const float l = d == 0.f ? e : __logf(u) * (e * __builtin_amdgcn_rcpf(d));
  return v > 20.f ? v : fmaxf(v, 0.f) + l;
}

// Max / sum over the four lanes {l, l^16, l^32, l^48} (one per 16-lane row of the wave), with gfx950's row-swap
// permutes (VALU, no LDS round trip).  permlane16_swap of (x, x) leaves, in every lane, its own row's value and
// its neighbour row's in the two results, in row order; permlane32_swap does the same for the two halves.  The
// combination order is the same in every lane, so all four lanes get bit-identical sums.
__device__ __forceinline__ float rows4_max(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float rows4_sum(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// x * sigmoid(x) (torch.nn.functional.silu).
__device__ __forceinline__ float silu_f(float g) { return g * __builtin_amdgcn_rcpf(1.f + __expf(-g)); }

// Word 3 of a gfx9-family buffer resource for raw (stride 0) byte addressing: loads at or past
// num_records bytes return 0, stores there are dropped.
constexpr int kRawBufferWord3 = 0x00020000;

// One element through a raw buffer resource: byte offset = vo (per lane) + so (uniform).
template <int DT>
__device__ __forceinline__ float buf_ld(__amdgpu_buffer_rsrc_t r, int vo, int so) {
  if constexpr (DT == HCLSM_F32) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, vo, so, 0));
  } else {
    const uint16_t b = __builtin_amdgcn_raw_buffer_load_b16(r, vo, so, 0);
    if constexpr (DT == HCLSM_BF16) return bf16_bits_to_f32(b);
    else return (float)__builtin_bit_cast(_Float16, b);
  }
}
template <int DT>
__device__ __forceinline__ void buf_st(float v, __amdgpu_buffer_rsrc_t r, int vo, int so) {
  if constexpr (DT == HCLSM_F32)
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, vo, so, 0);
  else if constexpr (DT == HCLSM_BF16)
    __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16_bits(v), r, vo, so, 0);
  else
    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, (_Float16)v), r, vo, so, 0);
}

}  // namespace hclsm

// Launch helper: returns a hipError_t as int (0 on success).
#define HCLSM_LAUNCH_CHECK()                         \
  do {                                               \
    hipError_t _e = hipGetLastError();               \
    if (_e != hipSuccess) return (int)_e;            \
  } while (0)

namespace hclsm {
// Zero-fill with a kernel (not hipMemsetAsync, so callers may capture it in a graph).
int zero_fill_f32(float* p, int64_t n, hipStream_t st);
int zero_fill_bytes(void* p, int64_t nbytes, hipStream_t st);
}  // namespace hclsm
