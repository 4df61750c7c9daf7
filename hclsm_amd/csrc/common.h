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
