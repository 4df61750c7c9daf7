// VALU issue-rate probe: measurement support for pricing the scan's instruction stream (no counterpart in
// the reference).  Each wave runs `iters` iterations of a fixed block of independent VALU instructions of
// one class -- v_fma_f32, v_exp_f32, or both mixed 1 : 3 as in the scan's essential per-update work -- on
// eight register chains, so the only limit is how fast a SIMD issues that class.  The host launches
// waves_per_simd x SIMDs one-wave workgroups and times the launch; time / (waves per SIMD x iterations x
// instructions per iteration) is the SIMD's time per instruction of that class at that occupancy.
#include "internal.h"

namespace hclsm {

constexpr int PROBE_FMA = 0;        // 32 v_fma_f32 per iteration
constexpr int PROBE_EXP = 1;        // 32 v_exp_f32 per iteration
constexpr int PROBE_MIX = 2;        // 32 v_exp_f32 + 96 v_fma_f32 per iteration, one exp then three FMAs
constexpr int PROBE_MIX_GROUPED = 3;  // the same 128, in blocks of 8 exps then 24 FMAs (scheduling barriers)

template <int KIND>
__global__ void __launch_bounds__(64) issue_probe_kernel(float* __restrict__ sink, int iters, float c1, float c2) {
  float a[8], b[8];
  const float s0 = 0.25f + 1e-3f * (float)threadIdx.x;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = s0 + 0.05f * (float)i;
    b[i] = s0 - 0.05f * (float)i;
  }
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if constexpr (KIND == PROBE_FMA) {
#pragma unroll
        for (int i = 0; i < 8; ++i) a[i] = fmaf(a[i], c1, c2);
      } else if constexpr (KIND == PROBE_EXP) {
        // exp2(-a) maps (0, 1] into [0.5, 1): the chains stay in range
#pragma unroll
        for (int i = 0; i < 8; ++i) a[i] = fast_exp2(-a[i]);
      } else if constexpr (KIND == PROBE_MIX) {
        // one exp, then three FMAs on other chains, in program order
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          a[i] = fast_exp2(-a[i]);
          b[i] = fmaf(b[i], c1, c2);
          b[(i + 3) & 7] = fmaf(b[(i + 3) & 7], c1, c2);
          b[(i + 6) & 7] = fmaf(b[(i + 6) & 7], c1, c2);
        }
        // keep that order in the schedule: groups of one transcendental, then three other VALU instructions
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x400, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) a[i] = fast_exp2(-a[i]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < 3; ++k)
#pragma unroll
          for (int i = 0; i < 8; ++i) b[i] = fmaf(b[i], c1, c2);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) acc += a[i] + b[i];
  // never true for the values above; keeps the chains live
  if (acc == -1.0f) sink[blockIdx.x * 64 + threadIdx.x] = acc;
}

}  // namespace hclsm

extern "C" int hclsm_issue_probe(int kind, int64_t waves, int iters, float* sink, void* stream) {
  if (kind < hclsm::PROBE_FMA || kind > hclsm::PROBE_MIX_GROUPED) return HCLSM_ERR_MODE;
  if (waves < 0 || waves > 0x7fffffffLL || iters < 0) return HCLSM_ERR_SHAPE;
  if (waves == 0 || iters == 0) return 0;
  if (!sink) return HCLSM_ERR_NULL;
  const dim3 grid((unsigned)waves), block(64);
  hipStream_t st = (hipStream_t)stream;
  switch (kind) {
    case hclsm::PROBE_FMA: hipLaunchKernelGGL(hclsm::issue_probe_kernel<hclsm::PROBE_FMA>, grid, block, 0, st, sink, iters, 0.999f, 1e-3f); break;
    case hclsm::PROBE_EXP: hipLaunchKernelGGL(hclsm::issue_probe_kernel<hclsm::PROBE_EXP>, grid, block, 0, st, sink, iters, 0.999f, 1e-3f); break;
    case hclsm::PROBE_MIX: hipLaunchKernelGGL(hclsm::issue_probe_kernel<hclsm::PROBE_MIX>, grid, block, 0, st, sink, iters, 0.999f, 1e-3f); break;
    default: hipLaunchKernelGGL(hclsm::issue_probe_kernel<hclsm::PROBE_MIX_GROUPED>, grid, block, 0, st, sink, iters, 0.999f, 1e-3f); break;
  }
  HCLSM_LAUNCH_CHECK();
  return 0;
}
