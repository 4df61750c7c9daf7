// Hierarchy manager output step for gfx950: HierarchyManager.forward of hclsm/dynamics/hierarchy_manager.py:120-162
// after the Level-1 pass, as one launch over the (B, T, N, D) rows plus a small per-clip prologue.
//
//   combined[b, t] = Level-1 row of event (b, t) if t is an event of clip b, else level0[b, t]     (:143)
//   l2            = l2_to_l1(mean_s level2_context[b, s])                                          (:148-149)
//   gate          = sigmoid(W_gate [combined; l2] + b_gate)                                        (:152-154)
//   combined      = gate * l2 + (1 - gate) * combined                                              (:155)
//   out           = combined * obj_mask[b, n]                                                      (:159-160)
//
// The concatenation is never formed: W_gate [x; l2] = W_gate[:, :D] x + (W_gate[:, D:] l2 + b_gate), and the
// bracket is one vector per clip (the prologue computes it with l2).  So the gate is a D x D GEMM over the rows
// with a per-clip bias, on MFMA pair tiles whose operand rows are read straight from Level-0 or from the Level-1
// rows (the scatter is this row choice; combined is never written), and the sigmoid, blend and mask run in its
// epilogue: each row is read from HBM and written once.  Without a Level-2 context the launch is the scatter
// plus the mask.
#include <type_traits>

#include "internal.h"
#include "pair_tile.h"

namespace hclsm {

struct TopDownArgs {
  const float* base;       // Level-0 rows [B * T * N, D]
  const float* events;     // Level-1 rows: packed [capacity, N, D] (kpad == 0) or padded [B, kpad, N, D]
  const int32_t* offsets;  // [B + 1] first packed event of each clip (kpad == 0)
  const int32_t* slot_of;  // [B * T] rank of t among clip b's events, -1 when t is no event
  const float* l2;         // [B, D] projected Level-2 context, or null (no gating)
  const float* gbias;      // [B, D] b_gate + W_gate[:, D:] l2
  const void* Wc;          // W_gate[:, :D] in the operand dtype, row stride ldw
  int64_t ldw;
  const float* obj;        // [B, N] or null
  float* out;              // [B * T * N, D]
  int64_t rows;            // B * T * N
  int T, N, D, kpad;
};

// Source row of output row r: the event's Level-1 row when frame (b, t) is an event the Level-1 rows hold,
// else the Level-0 row.
__device__ __forceinline__ const float* td_row(const TopDownArgs& a, int64_t r) {
  const int64_t f = r / a.N, n = r - f * a.N, b = f / a.T;
  const int32_t s = a.slot_of[f];
  if (s >= 0) {
    if (a.kpad == 0) return a.events + (((int64_t)a.offsets[b] + s) * a.N + n) * a.D;
    if (s < a.kpad) return a.events + ((b * a.kpad + s) * a.N + n) * a.D;
  }
  return a.base + r * a.D;
}

// NW waves, 16 rows each; with GATE the gate GEMM (W_gate[:, :D] staged through LDS in 64-column chunks) puts
// four consecutive gate columns of one row in each lane: lane (g, li) of wave w owns row 16w + li and columns
// 16t + 4g .. +3, t < D / 16.
template <int DT, int NW, int NTMAX, bool GATE>
__global__ void __launch_bounds__(64 * NW)
top_down_kernel(TopDownArgs a) {
  using T = typename MM<DT>::T;
  constexpr int KC = 64, NTH = 64 * NW;
  extern __shared__ __align__(16) unsigned char smem[];
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63, g = lane >> 4, li = lane & 15;
  const int D = a.D, NT = D / 16;
  const int64_t row = (int64_t)blockIdx.x * (16 * NW) + 16 * wid + li;
  const int64_t rc = row < a.rows ? row : a.rows - 1;
  const float* src = td_row(a, rc);
  f32x4 acc[NTMAX];
#pragma unroll
  for (int t = 0; t < NTMAX; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  if constexpr (GATE) {
    tile_gemm<DT, KC, NTH, NTMAX, true>(acc, NT, reinterpret_cast<const T*>(a.Wc), (int)a.ldw, D,
                                        reinterpret_cast<T*>(smem), tid, [&](int k, T* op) {
      if constexpr (DT == HCLSM_F32) {
        frag_load<DT>(src + k, op);
      } else {
        const float4 lo = *reinterpret_cast<const float4*>(src + k);
        const float4 hi = *reinterpret_cast<const float4*>(src + k + 4);
        op[0] = MM<DT>::fromf(lo.x); op[1] = MM<DT>::fromf(lo.y); op[2] = MM<DT>::fromf(lo.z);
        op[3] = MM<DT>::fromf(lo.w); op[4] = MM<DT>::fromf(hi.x); op[5] = MM<DT>::fromf(hi.y);
        op[6] = MM<DT>::fromf(hi.z); op[7] = MM<DT>::fromf(hi.w);
      }
    });
  }
  if (row >= a.rows) return;   // after every barrier of the GEMM
  const int64_t f = row / a.N, n = row - f * a.N, b = f / a.T;
  const float om = a.obj ? a.obj[b * a.N + n] : 1.f;
  float* dst = a.out + row * D;
#pragma unroll
  for (int t = 0; t < NTMAX; ++t) {
    if (t < NT) {
      const int c = 16 * t + 4 * g;
      const float4 x = *reinterpret_cast<const float4*>(src + c);
      float v[4] = {x.x, x.y, x.z, x.w};
      if constexpr (GATE) {
        const float4 l2 = *reinterpret_cast<const float4*>(a.l2 + b * D + c);
        const float4 gb = *reinterpret_cast<const float4*>(a.gbias + b * D + c);
        const float lv[4] = {l2.x, l2.y, l2.z, l2.w}, bv[4] = {gb.x, gb.y, gb.z, gb.w};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float gt = sigmoid_f(acc[t][r] + bv[r]);
          v[r] = gt * lv[r] + (1.f - gt) * v[r];
        }
      }
      if (a.obj) {
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] *= om;
      }
      *reinterpret_cast<float4*>(dst + c) = make_float4(v[0], v[1], v[2], v[3]);
    }
  }
}

// Resident-weight variant (D = 64 .. 256 for 16-bit operands, 64 .. 192 for fp32): W_gate[:, :D] stays in LDS for
// the workgroup's lifetime and every wave walks 16-row tiles on its own, with no barrier after the staging.  Lane
// (g, li) loads columns 16t + 4g .. +3 (t < D / 16) of row li once; those registers are both the MFMA operand and
// the epilogue's x, so each row is read from HBM once.  With PF the next tile's rows are loaded while the current
// tile is multiplied (twice the row registers; used up to D = 192).
//   fp32: the 16x16x4 MFMA contracts k = 4g + e of a 16-column block in four steps e: block t's fragment is x[t].
//   16-bit: the 16x16x32 MFMA takes k = 8g .. 8g + 7 of a 32-column block from lane group g; the lane supplies
//   columns 32j + 4g .. +3 and 32j + 16 + 4g .. +3 (its tiles 2j and 2j + 1), and W's columns are staged into
//   LDS in that order (8-byte groups moved within each 32-column block), so the contraction pairs equal columns.
template <int DT, int D, int NW, bool PF>
__global__ void __launch_bounds__(64 * NW)
top_down_res_kernel(TopDownArgs a, int64_t ntiles) {
  using A = MM<DT>;
  using T = typename A::T;
  constexpr int NT = D / 16;
  constexpr bool F32 = DT == HCLSM_F32;
  constexpr int P = F32 ? D + 4 : D + 8;   // LDS row pitch (elements)
  extern __shared__ __align__(16) unsigned char smem[];
  T* sW = reinterpret_cast<T*>(smem);
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63, g = lane >> 4, li = lane & 15;
  // rows of a tile (clamped to the last row: the loads stay in bounds, the stores are skipped)
  auto load_tile = [&](int64_t tile, float4 (&x)[NT]) {
    const int64_t row = tile * 16 + li;
    const float* src = td_row(a, row < a.rows ? row : a.rows - 1);
#pragma unroll
    for (int t = 0; t < NT; ++t) x[t] = *reinterpret_cast<const float4*>(src + 16 * t + 4 * g);
  };
  const int64_t first = (int64_t)blockIdx.x * NW + wid;
  float4 x[NT];
  load_tile(first < ntiles ? first : ntiles - 1, x);   // in flight while W is staged
  {
    // W into LDS in rounds of RB groups per thread, each round's loads all issued before its stores (D x D / 4
    // groups: a whole number of rounds of the workgroup's threads for every D here)
    using U = std::conditional_t<F32, float4, uint2>;   // 4 elements
    constexpr int UPR = D / 4, NU = D * UPR, PER = NU / (64 * NW);
    static_assert(NU % (64 * NW) == 0, "whole staging rounds");
    constexpr int RB = PER % 8 == 0 ? 8 : PER % 6 == 0 ? 6 : PER % 4 == 0 ? 4 : PER % 2 == 0 ? 2 : 1;
    const T* W = reinterpret_cast<const T*>(a.Wc);
#pragma unroll
    for (int i0 = 0; i0 < PER; i0 += RB) {
      U buf[RB];
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        const int u = tid + (i0 + i) * 64 * NW;
        const int r = u / UPR, q = u - r * UPR;
        buf[i] = *reinterpret_cast<const U*>(W + (size_t)r * a.ldw + 4 * q);
      }
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        const int u = tid + (i0 + i) * 64 * NW;
        const int r = u / UPR, q = u - r * UPR, qq = q & 7;
        const int pos = F32 ? 4 * q : (q & ~7) * 4 + (qq < 4 ? 8 * qq : 8 * (qq - 4) + 4);
        *reinterpret_cast<U*>(sW + r * P + pos) = buf[i];
      }
    }
  }
  __syncthreads();
  const int64_t stride = (int64_t)gridDim.x * NW;
  for (int64_t tile = first; tile < ntiles; tile += stride) {
    float4 xn[NT];
    if constexpr (PF) load_tile(tile + stride < ntiles ? tile + stride : tile, xn);   // next tile in flight
    f32x4 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    // one k-block's W fragments live at a time: the scheduling barrier keeps the next block's LDS reads from
    // being hoisted (all of them at once would not fit the registers)
    if constexpr (F32) {
#pragma unroll
      for (int kb = 0; kb < NT; ++kb) {
        float4 w[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) w[t] = *reinterpret_cast<const float4*>(sW + (16 * t + li) * P + 16 * kb + 4 * g);
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t] = A::mfma(w[t].x, x[kb].x, acc[t]);
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t] = A::mfma(w[t].y, x[kb].y, acc[t]);
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t] = A::mfma(w[t].z, x[kb].z, acc[t]);
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t] = A::mfma(w[t].w, x[kb].w, acc[t]);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
#pragma unroll
      for (int j = 0; j < NT / 2; ++j) {
        const float4 lo = x[2 * j], hi = x[2 * j + 1];
        T e[8] = {A::fromf(lo.x), A::fromf(lo.y), A::fromf(lo.z), A::fromf(lo.w),
                  A::fromf(hi.x), A::fromf(hi.y), A::fromf(hi.z), A::fromf(hi.w)};
        const typename A::Op op = A::load(e);
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t] = A::mfma(A::load(sW + (16 * t + li) * P + 32 * j + 8 * g), op, acc[t]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    const int64_t row = tile * 16 + li;
    if (row < a.rows) {
      const int64_t f = row / a.N, n = row - f * a.N, b = f / a.T;
      const float om = a.obj ? a.obj[b * a.N + n] : 1.f;
      float* dst = a.out + row * D;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int c = 16 * t + 4 * g;
        const float4 l2 = *reinterpret_cast<const float4*>(a.l2 + b * D + c);
        const float4 gb = *reinterpret_cast<const float4*>(a.gbias + b * D + c);
        const float xv[4] = {x[t].x, x[t].y, x[t].z, x[t].w};
        const float lv[4] = {l2.x, l2.y, l2.z, l2.w}, bv[4] = {gb.x, gb.y, gb.z, gb.w};
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float gt = sigmoid_f(acc[t][r] + bv[r]);
          v[r] = gt * lv[r] + (1.f - gt) * xv[r];
          if (a.obj) v[r] *= om;
        }
        *reinterpret_cast<float4*>(dst + c) = make_float4(v[0], v[1], v[2], v[3]);
      }
    }
    if constexpr (PF) {
#pragma unroll
      for (int t = 0; t < NT; ++t) x[t] = xn[t];
    } else if (tile + stride < ntiles) {
      load_tile(tile + stride, x);
    }
  }
}

// Per-clip prologue, grid (B, ceil(D / 32)), 8 threads per output column, each summing every 8th 4-element group of
// the dot product (vector loads when the rows allow) before a reduction over the 8:
//   td_l2_kernel:    l2[b, c] = W_l2[c, :] . mean_s ctx[b, s, :]   (mean: sum in summary order / S2, as torch's)
//   td_gbias_kernel: gbias[b, c] = b_gate[c] + W_gate[c, D:] . l2[b, :]
__device__ __forceinline__ float td_dot8(const float* __restrict__ w, const float* __restrict__ v, int K, bool vec,
                                         int j) {
  float s = 0.f;
  if (vec) {
    const float4* w4 = reinterpret_cast<const float4*>(w);
    const float4* v4 = reinterpret_cast<const float4*>(v);
#pragma unroll 4
    for (int q = j; q < K / 4; q += 8) {
      const float4 a = w4[q], b = v4[q];
      s = fmaf(a.x, b.x, s); s = fmaf(a.y, b.y, s); s = fmaf(a.z, b.z, s); s = fmaf(a.w, b.w, s);
    }
  } else {
#pragma unroll 4
    for (int k = j; k < K; k += 8) s = fmaf(w[k], v[k], s);
  }
  s += __shfl_xor(s, 1, 64);
  s += __shfl_xor(s, 2, 64);
  s += __shfl_xor(s, 4, 64);
  return s;
}

__global__ void __launch_bounds__(256)
td_l2_kernel(const float* __restrict__ ctx, int S2, int DL2, const float* __restrict__ Wl2, int D,
             float* __restrict__ l2) {
  extern __shared__ __align__(16) float sm[];   // DL2 floats
  const int b = blockIdx.x, tid = threadIdx.x;
  for (int k = tid; k < DL2; k += 256) {
    float s = 0.f;
    for (int i = 0; i < S2; ++i) s += ctx[((int64_t)b * S2 + i) * DL2 + k];
    sm[k] = s / (float)S2;
  }
  __syncthreads();
  const int c = blockIdx.y * 32 + (tid >> 3), j = tid & 7;
  const int cr = c < D ? c : D - 1;
  const bool vec = (DL2 % 4) == 0 && (((uintptr_t)Wl2) & 15) == 0;
  const float s = td_dot8(Wl2 + (int64_t)cr * DL2, sm, DL2, vec, j);
  if (j == 0 && c < D) l2[(int64_t)b * D + c] = s;
}

__global__ void __launch_bounds__(256)
td_gbias_kernel(const float* __restrict__ l2, const float* __restrict__ Wg, const float* __restrict__ bg, int D,
                float* __restrict__ gbias) {
  extern __shared__ __align__(16) float sm[];   // D floats
  const int b = blockIdx.x, tid = threadIdx.x;
  for (int k = tid; k < D; k += 256) sm[k] = l2[(int64_t)b * D + k];
  __syncthreads();
  const int c = blockIdx.y * 32 + (tid >> 3), j = tid & 7;
  const int cr = c < D ? c : D - 1;
  const bool vec = (((uintptr_t)Wg) & 15) == 0;   // rows of 2D floats, D a multiple of 32
  const float s = td_dot8(Wg + (int64_t)cr * 2 * D + D, sm, D, vec, j);
  if (j == 0 && c < D) gbias[(int64_t)b * D + c] = s + (bg ? bg[c] : 0.f);
}

template <int DT, int D>
static int launch_top_down_res(const TopDownArgs& a, hipStream_t st) {
  constexpr int NW = 8;
  constexpr size_t lds = (size_t)D * (DT == HCLSM_F32 ? D + 4 : D + 8) * sizeof(typename MM<DT>::T);
  static std::atomic<int> cache[HCLSM_MAX_DEVICES];
  int slots = 0;
  constexpr bool PF = D <= 192;
  const int rc = device_launch_setup((const void*)top_down_res_kernel<DT, D, NW, PF>, 64 * NW, lds,
                                     lds > 64 * 1024 ? (int)lds : 0, cache, &slots);
  if (rc != 0) return rc;
  const int64_t ntiles = (a.rows + 15) / 16;
  const int64_t want = (ntiles + NW - 1) / NW;
  const int64_t grid = want < slots ? want : slots;
  hipLaunchKernelGGL((top_down_res_kernel<DT, D, NW, PF>), dim3((unsigned)(grid < 1 ? 1 : grid)), dim3(64 * NW), lds, st,
                     a, ntiles);
  HCLSM_LAUNCH_CHECK();
  return 0;
}

// 1 when no resident variant covers (dtype, D)
template <int DT>
static int try_top_down_res(const TopDownArgs& a, hipStream_t st) {
  switch (a.D) {
    case 64: return launch_top_down_res<DT, 64>(a, st);
    case 128: return launch_top_down_res<DT, 128>(a, st);
    case 192: return launch_top_down_res<DT, 192>(a, st);
    case 256: if constexpr (DT != HCLSM_F32) return launch_top_down_res<DT, 256>(a, st); else return 1;
    default: return 1;
  }
}

template <int DT, int NTMAX, bool GATE>
static int launch_top_down(const TopDownArgs& a, hipStream_t st) {
  constexpr int NW = 8;
  const size_t lds = GATE ? (size_t)a.D * (64 + 8) * sizeof(typename MM<DT>::T) : 0;
  if (lds > 64 * 1024) {
    static std::atomic<int> cache[HCLSM_MAX_DEVICES];
    int grid_unused = 0;
    const int rc = device_launch_setup((const void*)top_down_kernel<DT, NW, NTMAX, GATE>, 64 * NW, lds,
                                       (int)lds, cache, &grid_unused);
    if (rc != 0) return rc;
  }
  const int64_t wgs = (a.rows + 16 * NW - 1) / (16 * NW);
  hipLaunchKernelGGL((top_down_kernel<DT, NW, NTMAX, GATE>), dim3((unsigned)wgs), dim3(64 * NW), lds, st, a);
  HCLSM_LAUNCH_CHECK();
  return 0;
}

template <int DT, bool GATE>
static int dispatch_top_down(const TopDownArgs& a, hipStream_t st) {
  if (a.D <= 128) return launch_top_down<DT, 8, GATE>(a, st);
  if (a.D <= 256) return launch_top_down<DT, 16, GATE>(a, st);
  return launch_top_down<DT, 24, GATE>(a, st);
}

}  // namespace hclsm

using namespace hclsm;

extern "C" int64_t hclsm_event_top_down_workspace(int64_t B, int64_t D) {
  if (B < 0 || D < 0) return HCLSM_ERR_SHAPE;
  return 2 * B * D * (int64_t)sizeof(float);
}

extern "C" int hclsm_event_top_down(const float* level0, const float* events, const int32_t* offsets,
                                    const int32_t* slot_of, int64_t kpad, const float* level2_context, int64_t S2,
                                    int64_t DL2, const float* W_l2, const float* W_gate, const float* b_gate,
                                    const void* W_gate_x, int64_t ldw, const float* obj_mask, float* out, int64_t B,
                                    int64_t T, int64_t N, int64_t D, int dtype, void* ws, int64_t ws_bytes,
                                    void* stream) {
  if (B < 0 || T < 0 || N < 0 || D < 0 || kpad < 0) return HCLSM_ERR_SHAPE;
  if (dtype != HCLSM_F32 && dtype != HCLSM_BF16 && dtype != HCLSM_F16) return HCLSM_ERR_DTYPE;
  if (D % 32 != 0 || D > 384 || N > (1 << 30) || T > (1 << 30)) return HCLSM_ERR_UNSUPPORTED;
  const int64_t rows = B * T * N;
  if (rows == 0 || D == 0) return 0;
  // events is required even when no frame is an event: the library cannot see that without a sync
  if (!level0 || !events || !out || !slot_of) return HCLSM_ERR_NULL;
  if (kpad == 0 && !offsets) return HCLSM_ERR_NULL;
  const bool gate = level2_context != nullptr;
  if (gate) {
    if (S2 <= 0 || DL2 <= 0 || S2 > (1 << 30)) return HCLSM_ERR_SHAPE;
    if (DL2 > 16384) return HCLSM_ERR_UNSUPPORTED;   // the prologue keeps the mean context in 64 KB of LDS
    if (!W_l2 || !W_gate || !W_gate_x || !ws) return HCLSM_ERR_NULL;
    if (ldw < D || ws_bytes < hclsm_event_top_down_workspace(B, D)) return HCLSM_ERR_SHAPE;
    if ((((uintptr_t)ws) & 15) != 0) return HCLSM_ERR_UNSUPPORTED;
    if ((((uintptr_t)W_gate_x) & 15) != 0 || (ldw * (dtype == HCLSM_F32 ? 4 : 2)) % 16 != 0)
      return HCLSM_ERR_UNSUPPORTED;
  }
  for (const void* p : {(const void*)level0, (const void*)events, (const void*)out})
    if ((((uintptr_t)p) & 15) != 0) return HCLSM_ERR_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  TopDownArgs a{level0, events, offsets, slot_of, nullptr, nullptr, W_gate_x, ldw, obj_mask, out, rows,
                (int)T, (int)N, (int)D, (int)kpad};
  if (!gate) return dispatch_top_down<HCLSM_F32, false>(a, st);
  float* l2 = reinterpret_cast<float*>(ws);
  float* gb = l2 + B * D;
  const dim3 pgrid((unsigned)B, (unsigned)((D + 31) / 32));
  hipLaunchKernelGGL(td_l2_kernel, pgrid, dim3(256), DL2 * sizeof(float), st, level2_context, (int)S2, (int)DL2,
                     W_l2, (int)D, l2);
  HCLSM_LAUNCH_CHECK();
  hipLaunchKernelGGL(td_gbias_kernel, pgrid, dim3(256), D * sizeof(float), st, l2, W_gate, b_gate, (int)D, gb);
  HCLSM_LAUNCH_CHECK();
  a.l2 = l2;
  a.gbias = gb;
  int rc = 1;
  if (dtype == HCLSM_F32) rc = try_top_down_res<HCLSM_F32>(a, st);
  else if (dtype == HCLSM_BF16) rc = try_top_down_res<HCLSM_BF16>(a, st);
  else rc = try_top_down_res<HCLSM_F16>(a, st);
  if (rc != 1) return rc;
  if (dtype == HCLSM_F32) return dispatch_top_down<HCLSM_F32, true>(a, st);
  if (dtype == HCLSM_BF16) return dispatch_top_down<HCLSM_BF16, true>(a, st);
  return dispatch_top_down<HCLSM_F16, true>(a, st);
}
