// Library-wide entry points: version, error strings, fill helpers.
#include "common.h"

namespace hclsm {

__global__ void zero_fill_u32_kernel(uint32_t* __restrict__ p, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) p[i] = 0u;
}

__global__ void zero_fill_u8_kernel(uint8_t* __restrict__ p, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) p[i] = 0u;
}

static unsigned fill_grid(int64_t n) {
  int64_t g = (n + 255) / 256;
  if (g > 4096) g = 4096;
  if (g < 1) g = 1;
  return (unsigned)g;
}

int zero_fill_f32(float* p, int64_t n, hipStream_t st) {
  if (n <= 0) return 0;
  hipLaunchKernelGGL(zero_fill_u32_kernel, dim3(fill_grid(n)), dim3(256), 0, st, (uint32_t*)p, n);
  HCLSM_LAUNCH_CHECK();
  return 0;
}

int zero_fill_bytes(void* p, int64_t nbytes, hipStream_t st) {
  if (nbytes <= 0) return 0;
  if ((((uintptr_t)p) & 3) == 0 && (nbytes & 3) == 0)
    return zero_fill_f32((float*)p, nbytes / 4, st);
  hipLaunchKernelGGL(zero_fill_u8_kernel, dim3(fill_grid(nbytes)), dim3(256), 0, st, (uint8_t*)p, nbytes);
  HCLSM_LAUNCH_CHECK();
  return 0;
}

}  // namespace hclsm

extern "C" int hclsm_abi_version(void) { return HCLSM_ABI_VERSION; }

extern "C" const char* hclsm_strerror(int code) {
  switch (code) {
    case 0: return "success";
    case HCLSM_ERR_NULL: return "hclsm: a required pointer argument is NULL";
    case HCLSM_ERR_SHAPE: return "hclsm: invalid size argument (negative, zero where not allowed, or too large)";
    case HCLSM_ERR_DTYPE: return "hclsm: unknown element-type code";
    case HCLSM_ERR_UNSUPPORTED: return "hclsm: argument combination not supported by this build";
    case HCLSM_ERR_MODE: return "hclsm: unknown mode code";
    case HCLSM_ERR_SCRATCH:
      return "hclsm: the call needs more workspace than the allocation-free entry point's static scratch array";
    default: break;
  }
  if (code > 0) return hipGetErrorString((hipError_t)code);
  return "hclsm: unknown error code";
}
