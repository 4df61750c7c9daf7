// Pair-tile MFMA building blocks shared by the kernels that run a small MLP over all (i, j) slot pairs of a
// frame (relation-graph edges, tracker matching scores) without materialising the pair features: each wave
// owns a 16-pair MFMA row tile whose operand it forms on the fly from two node rows, and the workgroup
// streams the weight matrix through LDS in KC-column chunks shared by all its waves.
#pragma once

#include "mfma.h"

namespace hclsm {

// k-fragment of one lane per MFMA group: KE contiguous elements at kb + KE*g of a KB-wide block.
// 16-bit: one v_mfma_f32_16x16x32 per block.  fp32: four v_mfma_f32_16x16x4 (MFMA e contracts k = 4g + e
// across the lane groups: the contraction order is permuted, the sum is the same).
template <int DT> struct GFrag;
template <> struct GFrag<HCLSM_BF16> {
  static constexpr int KE = 8, KB = 32;
};
template <> struct GFrag<HCLSM_F16> {
  static constexpr int KE = 8, KB = 32;
};
template <> struct GFrag<HCLSM_F32> {
  static constexpr int KE = 4, KB = 16;
};

template <int DT>
__device__ __forceinline__ void frag_load(const typename MM<DT>::T* p, typename MM<DT>::T* e) {
  if constexpr (DT == HCLSM_F32) {
    const float4 v = *reinterpret_cast<const float4*>(p);
    e[0] = v.x; e[1] = v.y; e[2] = v.z; e[3] = v.w;
  } else {
    *reinterpret_cast<uint4*>(e) = *reinterpret_cast<const uint4*>(p);
  }
}

template <int DT>
__device__ __forceinline__ f32x4 frag_mma(const typename MM<DT>::T* a, const typename MM<DT>::T* b, f32x4 acc) {
  using A = MM<DT>;
  if constexpr (DT == HCLSM_F32) {
#pragma unroll
    for (int e = 0; e < 4; ++e) acc = A::mfma(a[e], b[e], acc);
    return acc;
  } else {
    return A::mfma(A::load(a), A::load(b), acc);
  }
}

// sW[r * pitch + c] = W[r * ldw + k0 + c] for r < nrows, c < kc (16-byte units; kc a multiple of the unit)
template <typename T, int NTH>
__device__ __forceinline__ void stage_rows(const T* __restrict__ W, int ldw, int nrows, int k0, int kc, T* sW,
                                           int pitch, int tid) {
  constexpr int U = 16 / (int)sizeof(T);
  const int upr = kc / U;
  for (int u = tid; u < nrows * upr; u += NTH) {
    const int r = u / upr, c = (u - r * upr) * U;
    *reinterpret_cast<uint4*>(sW + r * pitch + c) = *reinterpret_cast<const uint4*>(W + (size_t)r * ldw + k0 + c);
  }
}

// acc[t] += (this wave's 16 operand rows) x (W rows t*16 + li) over k < K, for t < NT (<= NTMAX).  W (row
// stride ldw) is staged through sW (pitch KC + 8) in KC-column chunks; a_frag(k, op) gives this lane's KE
// operand elements at column k (k = kb + KE*g of the current block).  Every thread of the workgroup calls
// it (it holds barriers); the first barrier also orders any LDS writes made before the call.
// Output layout: acc[t][r] is operand row 4g + r, W row t*16 + li; with WA (W as the MFMA's A operand) it is
// operand row li, W row t*16 + 4g + r, so a lane holds four consecutive outputs of one operand row.
template <int DT, int KC, int NTH, int NTMAX, bool WA = false, typename AF>
__device__ __forceinline__ void tile_gemm(f32x4 (&acc)[NTMAX], int NT, const typename MM<DT>::T* W, int ldw, int K,
                                          typename MM<DT>::T* sW, int tid, AF&& a_frag) {
  using T = typename MM<DT>::T;
  constexpr int KE = GFrag<DT>::KE, KB = GFrag<DT>::KB, PW = KC + 8;
  static_assert(KC % KB == 0, "chunk of whole fragment blocks");
  const int lane = tid & 63, g = lane >> 4, li = lane & 15;
  for (int k0 = 0; k0 < K; k0 += KC) {
    const int kc = K - k0 < KC ? K - k0 : KC;
    __syncthreads();   // the previous chunk is consumed
    stage_rows<T, NTH>(W, ldw, NT * 16, k0, kc, sW, PW, tid);
    __syncthreads();
    for (int kb = 0; kb < kc; kb += KB) {
      T op[KE];
      a_frag(k0 + kb + KE * g, op);
#pragma unroll
      for (int t = 0; t < NTMAX; ++t) {
        if (t < NT) {
          T wb[KE];
          frag_load<DT>(sW + (t * 16 + li) * PW + kb + KE * g, wb);
          acc[t] = WA ? frag_mma<DT>(wb, op, acc[t]) : frag_mma<DT>(op, wb, acc[t]);
        }
      }
    }
  }
}

}  // namespace hclsm
