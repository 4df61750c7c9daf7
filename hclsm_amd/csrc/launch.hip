// Per-device launch set-up shared by the kernels that use large dynamic LDS or persistent grids.
#include "internal.h"

namespace hclsm {

int device_launch_setup(const void* fn, int threads, size_t lds, int max_lds, std::atomic<int>* cache, int* grid) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= HCLSM_MAX_DEVICES) return HCLSM_ERR_UNSUPPORTED;
  int g = cache[dev].load(std::memory_order_relaxed);
  if (g == 0) {
    if (max_lds > 0 && (e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, max_lds)) != hipSuccess)
      return (int)e;
    int cus = 0, per_cu = 0;
    if ((e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return (int)e;
    if ((e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, threads, lds)) != hipSuccess) return (int)e;
    g = cus * (per_cu > 0 ? per_cu : 1);
    cache[dev].store(g, std::memory_order_relaxed);   // same value from any racing first call
  }
  *grid = g;
  return 0;
}

int device_cus(int* cus) {
  static std::atomic<int> cache[HCLSM_MAX_DEVICES];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= HCLSM_MAX_DEVICES) return HCLSM_ERR_UNSUPPORTED;
  int c = cache[dev].load(std::memory_order_relaxed);
  if (c == 0) {
    if ((e = hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return (int)e;
    cache[dev].store(c, std::memory_order_relaxed);
  }
  *cus = c;
  return 0;
}

}  // namespace hclsm
