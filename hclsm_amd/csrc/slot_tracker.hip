// Slot tracker for gfx950: SlotTracker of hclsm/objects/slot_tracker.py:46-158 and the frame-by-frame
// tracking loop of hclsm/model.py:229-252.
//
// Matching cost of pair (i, j) (slot i of the earlier frame, slot j of the later one), slot_tracker.py:74-107:
//   score = w3 . ReLU(W2 ReLU(W1 [a_i; b_j; |a_i - b_j|] + b1) + b2) + b3   (a, b clamped to [-50, 50])
//   cost  = -(score - 1e4 [alive_a_i < 0.5] - 1e4 [alive_b_j < 0.5])
// W1 [a; b; d] = W1a a + W1b b + W1c d: the first two terms are per-node projections (one GEMM over the
// nodes), so only W1c |a_i - b_j| (K = D instead of 3D) is contracted per pair, on MFMA pair tiles whose
// operand is formed on the fly; the second layer and the score follow in the same workgroup.
//
// Tracking loop.  Step t matches the tracked slots of frame t-1 (frame t-1 permuted by the previous step's
// perm, alive permuted with them) against frame t.  Row i of that cost matrix is row perm_{t-1}[i] of the
// cost between the unpermuted frames t-1 and t, penalties included.  So the pair MLP runs once, in one
// launch, over every (t-1, t) frame pair of every clip; only the Sinkhorn matching is sequential in t: one
// workgroup per clip loops over the frames with the previous perm and alive row in LDS.  The tracked slots
// are gathered afterwards in one parallel pass.  The GRU hidden state (slot_tracker.py:137-158) does not
// feed back into the matching; when it is wanted it is carried in a second loop, one GEMM and one gate
// launch per frame, with the input-side GEMM done once for all frames.
//
// Sinkhorn (slot_tracker.py:15-43): log_alpha = -clamp(cost, -1e4, 1e4) * (1 / temperature), then n_iters
// rounds of log-sum-exp normalisation over rows, then over columns, updated in place; perm = argmax over j
// of exp(log_alpha) (lowest index on ties), confidence = that maximum.  A frame's log_alpha lives in LDS
// and is normalised in place; each half-step gives every lane CPL entries of one row (or column) and
// reduces them in the lane and over the line's 8 lanes with DPP, one barrier between half-steps.
#include "internal.h"
#include "pair_tile.h"

namespace hclsm {

constexpr float TRK_PENALTY = 1e4f;
constexpr float TRK_COST_CLAMP = 1e4f;
constexpr float TRK_SLOT_CLAMP = 50.f;

// ------------------------------------------------------------------------------------------------ cost
struct TrackCostArgs {
  const float* S;      // clamped node rows [rows, D] fp32
  const float* UV;     // [rows, 2D] fp32: W1a s + b1 | W1b s
  const void* W1;      // match_mlp.0.weight [D, 3D] (operand dtype)
  const void* W2;      // match_mlp.2.weight [D/4, D] (operand dtype)
  const float* b2;     // [D/4]
  const float* w3;     // match_mlp.4.weight [D/4]
  const float* b3;     // [1]
  const float* alive_a;   // alive of the a rows, indexed by node row, or null (all alive)
  const float* alive_b;   // alive of the b rows, indexed by node row - boff
  int64_t boff;
  float* cost;         // [F, N, N]
  int64_t pairs;       // F * N * N
  int N, D;
  int nt, tstride, fboff;   // cost frame f pairs node frames fa = (f / nt) * tstride + f % nt and fa + fboff
};

template <int DT, int NW, int KC>
__global__ void __launch_bounds__(64 * NW)
track_cost_kernel(TrackCostArgs a) {
  using A = MM<DT>;
  using T = typename A::T;
  constexpr int KE = GFrag<DT>::KE;
  constexpr int ROWS = 16 * NW, NTH = 64 * NW;
  extern __shared__ __align__(16) unsigned char smem[];
  const int N = a.N, D = a.D, LH = D + 8;
  T* sH = reinterpret_cast<T*>(smem);    // [ROWS][LH] first hidden layer of the workgroup's pairs
  T* sW = sH + (size_t)ROWS * LH;        // [D][KC + 8] weight chunk
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63, g = lane >> 4, li = lane & 15;
  const int64_t p0 = (int64_t)blockIdx.x * ROWS;
  const int64_t NN = (int64_t)N * N;
  // pair p (clamped into range) -> node rows of a_i and b_j
  auto nodes_of = [&](int64_t p, int64_t& ra, int64_t& rb) {
    p = p < a.pairs ? p : a.pairs - 1;
    const int64_t f = p / NN;
    const int rem = (int)(p - f * NN);
    const int i = rem / N, j = rem - i * N;
    const int64_t q = f / a.nt;
    const int64_t fa = q * a.tstride + (f - q * a.nt);
    ra = fa * N + i;
    rb = (fa + a.fboff) * N + j;
  };

  // ---- first layer: ReLU(W1c |a_i - b_j| + U_i + V_j) -> sH
  {
    int64_t ra, rb;
    nodes_of(p0 + wid * 16 + li, ra, rb);
    const float* xa = a.S + ra * D;
    const float* xb = a.S + rb * D;
    const int NT = D / 16;
    f32x4 acc[24];
#pragma unroll
    for (int t = 0; t < 24; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    tile_gemm<DT, KC, NTH>(acc, NT, reinterpret_cast<const T*>(a.W1) + 2 * D, 3 * D, D, sW, tid, [&](int k, T* op) {
#pragma unroll
      for (int e = 0; e < KE; e += 4) {
        const float4 x4 = *reinterpret_cast<const float4*>(xa + k + e);
        const float4 y4 = *reinterpret_cast<const float4*>(xb + k + e);
        op[e] = A::fromf(fabsf(x4.x - y4.x));
        op[e + 1] = A::fromf(fabsf(x4.y - y4.y));
        op[e + 2] = A::fromf(fabsf(x4.z - y4.z));
        op[e + 3] = A::fromf(fabsf(x4.w - y4.w));
      }
    });
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int orow = wid * 16 + 4 * g + rr;
      int64_t rao, rbo;
      nodes_of(p0 + orow, rao, rbo);
      const float* U = a.UV + rao * 2 * D;
      const float* V = a.UV + rbo * 2 * D + D;
#pragma unroll
      for (int t = 0; t < 24; ++t) {
        if (t < NT) {
          const int o = t * 16 + li;
          sH[(size_t)orow * LH + o] = A::fromf(fmaxf(acc[t][rr] + U[o] + V[o], 0.f));
        }
      }
    }
  }

  // ---- second layer and score (tile_gemm's first barrier orders the sH writes before these reads)
  {
    const int NT = D / 64;   // D/4 outputs in 16-wide tiles
    f32x4 acc[6];
#pragma unroll
    for (int t = 0; t < 6; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    const T* hrow = sH + (size_t)(wid * 16 + li) * LH;
    tile_gemm<DT, KC, NTH>(acc, NT, reinterpret_cast<const T*>(a.W2), D, D, sW, tid,
                           [&](int k, T* op) { frag_load<DT>(hrow + k, op); });
    float part[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 6; ++t) {
      if (t < NT) {
        const int o = t * 16 + li;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) part[rr] = fmaf(fmaxf(acc[t][rr] + a.b2[o], 0.f), a.w3[o], part[rr]);
      }
    }
#pragma unroll
    for (int rr = 0; rr < 4; ++rr)
#pragma unroll
      for (int m = 1; m < 16; m <<= 1) part[rr] += __shfl_xor(part[rr], m, 64);
    if (li == 0) {
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int64_t p = p0 + wid * 16 + 4 * g + rr;
        if (p < a.pairs) {
          float s = part[rr] + a.b3[0];
          if (a.alive_a) {
            int64_t ra, rb;
            nodes_of(p, ra, rb);
            s = s - (a.alive_a[ra] < 0.5f ? TRK_PENALTY : 0.f);
            s = s - (a.alive_b[rb - a.boff] < 0.5f ? TRK_PENALTY : 0.f);
          }
          a.cost[p] = -s;
        }
      }
    }
  }
}

// Weight-resident variant for 16-bit operands and D <= 192 (the pair tiles of the tiny and small presets):
// a persistent workgroup stages W1c and W2 in LDS once, then walks blocks of 32 NW pairs.  The MFMAs take
// the weights as the A operand and the pairs as the B operand, so lane (g, li) of a 16-output tile holds
// outputs 4g .. 4g+3 of pair li: the U / V epilogue reads float4s, and the first layer's accumulators are,
// without leaving registers, the second layer's B operand, with W2's columns stored in the matching order
// (positions 8g .. 8g+7 of a 32-wide block hold k = 4g .. 4g+3 and 16 + 4g .. 16 + 4g+3).  Two 16-pair
// tiles per wave share each weight fragment read from LDS.
template <int DT, int D, int NW>
__global__ void __launch_bounds__(64 * NW)
track_cost_res_kernel(TrackCostArgs a) {
  using A = MM<DT>;
  using T = typename A::T;
  static_assert(DT != HCLSM_F32 && D % 64 == 0 && D <= 192, "16-bit operands, D a multiple of 64 up to 192");
  constexpr int NTH = 64 * NW, PT = 2, BLK = 16 * PT * NW;
  constexpr int D4 = D / 4, PW = D + 8, NT = D / 16, NT2 = D4 / 16, NKB = D / 32;
  extern __shared__ __align__(16) unsigned char smem[];
  T* sW1 = reinterpret_cast<T*>(smem);                 // [D][PW] W1c, natural k order
  T* sW2 = sW1 + D * PW;                               // [D4][PW] W2, k permuted within 32-wide blocks
  float* sb2 = reinterpret_cast<float*>(sW2 + D4 * PW);
  float* sw3 = sb2 + D4;
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63, g = lane >> 4, li = lane & 15;
  {
    const T* W1 = reinterpret_cast<const T*>(a.W1);
    for (int u = tid; u < D * (D / 8); u += NTH) {
      const int r = u / (D / 8), c = (u - r * (D / 8)) * 8;
      *reinterpret_cast<uint4*>(sW1 + r * PW + c) = *reinterpret_cast<const uint4*>(W1 + (size_t)r * 3 * D + 2 * D + c);
    }
    const T* W2 = reinterpret_cast<const T*>(a.W2);
    for (int u = tid; u < D4 * (D / 8); u += NTH) {
      const int r = u / (D / 8), q = (u - r * (D / 8)) * 8;
      const int kb = q & ~31, gg = (q & 31) >> 3;
      const uint2 lo = *reinterpret_cast<const uint2*>(W2 + (size_t)r * D + kb + 4 * gg);
      const uint2 hi = *reinterpret_cast<const uint2*>(W2 + (size_t)r * D + kb + 16 + 4 * gg);
      *reinterpret_cast<uint4*>(sW2 + r * PW + q) = make_uint4(lo.x, lo.y, hi.x, hi.y);
    }
    for (int u = tid; u < D4; u += NTH) {
      sb2[u] = a.b2[u];
      sw3[u] = a.w3[u];
    }
  }
  __syncthreads();
  const int N = a.N;
  const int64_t NN = (int64_t)N * N;
  auto nodes_of = [&](int64_t p, int64_t& ra, int64_t& rb) {
    p = p < a.pairs ? p : a.pairs - 1;
    const int64_t f = p / NN;
    const int rem = (int)(p - f * NN);
    const int i = rem / N, j = rem - i * N;
    const int64_t q = f / a.nt;
    const int64_t fa = q * a.tstride + (f - q * a.nt);
    ra = fa * N + i;
    rb = (fa + a.fboff) * N + j;
  };
  const int64_t nblk = (a.pairs + BLK - 1) / BLK;
  for (int64_t blk = blockIdx.x; blk < nblk; blk += gridDim.x) {
    const int64_t pw = blk * BLK + (int64_t)wid * 16 * PT;
    int64_t ra[PT], rb[PT];
#pragma unroll
    for (int pt = 0; pt < PT; ++pt) nodes_of(pw + 16 * pt + li, ra[pt], rb[pt]);
    // ---- first layer: acc[pt][t] = W1c rows 16t.. x |a - b| of the tile's pairs
    f32x4 acc[PT][NT];
#pragma unroll
    for (int pt = 0; pt < PT; ++pt)
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[pt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    // raw rows of the next k-block are loaded while the current one is multiplied
    float4 xr[PT][4];
    auto load_k = [&](int kb) {
#pragma unroll
      for (int pt = 0; pt < PT; ++pt) {
        const float* xa = a.S + ra[pt] * D + kb + 8 * g;
        const float* xb = a.S + rb[pt] * D + kb + 8 * g;
        xr[pt][0] = *reinterpret_cast<const float4*>(xa);
        xr[pt][1] = *reinterpret_cast<const float4*>(xa + 4);
        xr[pt][2] = *reinterpret_cast<const float4*>(xb);
        xr[pt][3] = *reinterpret_cast<const float4*>(xb + 4);
      }
    };
    load_k(0);
#pragma unroll 1
    for (int kb = 0; kb < D; kb += 32) {
      T op[PT][8];
#pragma unroll
      for (int pt = 0; pt < PT; ++pt) {
        const float4 x0 = xr[pt][0], x1 = xr[pt][1], y0 = xr[pt][2], y1 = xr[pt][3];
        op[pt][0] = A::fromf(fabsf(x0.x - y0.x)); op[pt][1] = A::fromf(fabsf(x0.y - y0.y));
        op[pt][2] = A::fromf(fabsf(x0.z - y0.z)); op[pt][3] = A::fromf(fabsf(x0.w - y0.w));
        op[pt][4] = A::fromf(fabsf(x1.x - y1.x)); op[pt][5] = A::fromf(fabsf(x1.y - y1.y));
        op[pt][6] = A::fromf(fabsf(x1.z - y1.z)); op[pt][7] = A::fromf(fabsf(x1.w - y1.w));
      }
      if (kb + 32 < D) load_k(kb + 32);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        T wf[8];
        frag_load<DT>(sW1 + (16 * t + li) * PW + kb + 8 * g, wf);
#pragma unroll
        for (int pt = 0; pt < PT; ++pt) acc[pt][t] = frag_mma<DT>(wf, op[pt], acc[pt][t]);
      }
    }
    // ---- epilogue: h = ReLU(acc + U_i + V_j) for outputs 16t + 4g + rr of pair li
    // (in groups of 3 tiles: the scheduler would otherwise hoist every load of the epilogue at once)
#pragma unroll
    for (int pt = 0; pt < PT; ++pt) {
      const float* U = a.UV + ra[pt] * 2 * D + 4 * g;
      const float* V = a.UV + rb[pt] * 2 * D + D + 4 * g;
#pragma unroll
      for (int t0 = 0; t0 < NT; t0 += 3) {
#pragma unroll
        for (int t = t0; t < t0 + 3 && t < NT; ++t) {
          const float4 u4 = *reinterpret_cast<const float4*>(U + 16 * t);
          const float4 v4 = *reinterpret_cast<const float4*>(V + 16 * t);
          acc[pt][t][0] = fmaxf(acc[pt][t][0] + u4.x + v4.x, 0.f);
          acc[pt][t][1] = fmaxf(acc[pt][t][1] + u4.y + v4.y, 0.f);
          acc[pt][t][2] = fmaxf(acc[pt][t][2] + u4.z + v4.z, 0.f);
          acc[pt][t][3] = fmaxf(acc[pt][t][3] + u4.w + v4.w, 0.f);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // ---- second layer: k-block kb takes tiles 2kb (k = 32kb + 4g + e) and 2kb + 1 (32kb + 16 + 4g + e)
    f32x4 acc2[PT][NT2];
#pragma unroll
    for (int pt = 0; pt < PT; ++pt)
#pragma unroll
      for (int t = 0; t < NT2; ++t) acc2[pt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      T hb[PT][8];
#pragma unroll
      for (int pt = 0; pt < PT; ++pt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          hb[pt][e] = A::fromf(acc[pt][2 * kb][e]);
          hb[pt][4 + e] = A::fromf(acc[pt][2 * kb + 1][e]);
        }
#pragma unroll
      for (int t = 0; t < NT2; ++t) {
        T wf[8];
        frag_load<DT>(sW2 + (16 * t + li) * PW + 32 * kb + 8 * g, wf);
#pragma unroll
        for (int pt = 0; pt < PT; ++pt) acc2[pt][t] = frag_mma<DT>(wf, hb[pt], acc2[pt][t]);
      }
    }
    // ---- score of pair li: sum over the second layer's outputs 16t + 4g + rr, then over the 4 lane groups
#pragma unroll
    for (int pt = 0; pt < PT; ++pt) {
      float part = 0.f;
#pragma unroll
      for (int t = 0; t < NT2; ++t)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int o = 16 * t + 4 * g + rr;
          part = fmaf(fmaxf(acc2[pt][t][rr] + sb2[o], 0.f), sw3[o], part);
        }
      part = rows4_sum(part);
      const int64_t p = pw + 16 * pt + li;
      if (g == 0 && p < a.pairs) {
        float s = part + a.b3[0];
        if (a.alive_a) {
          s = s - (a.alive_a[ra[pt]] < 0.5f ? TRK_PENALTY : 0.f);
          s = s - (a.alive_b[rb[pt] - a.boff] < 0.5f ? TRK_PENALTY : 0.f);
        }
        a.cost[p] = -s;
      }
    }
  }
}

// y[r, k] = clamp(x[r, k], -50, 50) (NaN passes through, as torch.clamp); VW = 4: float4 units (n a multiple of
// 4, x and y 16-byte aligned)
__device__ __forceinline__ float trk_clamp1(float v) {
  return v < -TRK_SLOT_CLAMP ? -TRK_SLOT_CLAMP : (v > TRK_SLOT_CLAMP ? TRK_SLOT_CLAMP : v);
}
template <int VW>
__global__ void __launch_bounds__(256)
trk_clamp_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t n) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= n / VW) return;
  if constexpr (VW == 4) {
    float4 v = reinterpret_cast<const float4*>(x)[e];
    v.x = trk_clamp1(v.x); v.y = trk_clamp1(v.y); v.z = trk_clamp1(v.z); v.w = trk_clamp1(v.w);
    reinterpret_cast<float4*>(y)[e] = v;
  } else {
    y[e] = trk_clamp1(x[e]);
  }
}

// --------------------------------------------------------------------------------------------- Sinkhorn
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, true));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, true);
}

// max(m, x) without fmaxf's quieting of the operands: NaN is not a value the matching has to order
__device__ __forceinline__ float max_sel(float m, float x) { return x > m ? x : m; }

// log-sum-exp of a reduced (max, sum of exp(x - max)); a row or column of padding (max -inf) gives 0 so that
// it stays -inf.  The sum is at least 1: the hardware log2 needs no range handling.
__device__ __forceinline__ float lse_of(float m, float s) {
  return m == -INFINITY ? 0.f : fmaf(__builtin_amdgcn_logf(s), HCLSM_LN2, m);
}

// All-reduce over the 8 lanes of a row group (lane bits 0-2): quad xor 1, quad xor 2, half-row mirror.
__device__ __forceinline__ float group_max(float v) {
  v = max_sel(v, dpp_f<0xb1>(v));
  v = max_sel(v, dpp_f<0x4e>(v));
  return max_sel(v, dpp_f<0x141>(v));
}
__device__ __forceinline__ float group_sum(float v) {
  v += dpp_f<0xb1>(v);
  v += dpp_f<0x4e>(v);
  return v + dpp_f<0x141>(v);
}

// The N x N log_alpha of one frame lives in LDS (sL, row pitch SkTile::P) and is normalised in place, as
// the reference does.  W = CPL waves of 64 lanes; lane 8 rg + cg of wave w handles line w 8 + rg of the
// half-step (a row in the row step, a column in the column step) and its CPL entries cg CPL + c, so both
// reductions are CPL values in the lane plus three DPP steps over the 8 lanes of the line, with one
// barrier between half-steps.  The pitch makes the column reads of a wave hit 64 (or 32) distinct banks.
template <int CPL>
struct SkTile {
  static constexpr int W = CPL, NC = 8 * CPL, NTH = 64 * CPL;
  static constexpr int P = CPL == 2 ? NC + 4 : CPL == 4 ? NC + 2 : NC + 1;
};

template <int CPL>
__device__ __forceinline__ void lse_line(float (&v)[CPL]) {
  float m = v[0];
#pragma unroll
  for (int c = 1; c < CPL; ++c) m = max_sel(m, v[c]);
  m = group_max(m);
  float s = __expf(v[0] - m);
#pragma unroll
  for (int c = 1; c < CPL; ++c) s += __expf(v[c] - m);
  s = group_sum(s);
  const float l = lse_of(m, s);
#pragma unroll
  for (int c = 0; c < CPL; ++c) v[c] -= l;
}

// n_iters rounds of row then column log-sum-exp normalisation of sL in place.  Entries at -inf (padding)
// stay -inf.  Every thread of the workgroup calls it; sL must be complete (a barrier after its writes).
template <int CPL>
__device__ __forceinline__ void sinkhorn_lds(float* sL, int n_iters, int line, int cg) {
  constexpr int P = SkTile<CPL>::P;
  float v[CPL];
  for (int it = 0; it < n_iters; ++it) {
    float* r = sL + line * P + cg * CPL;          // row `line`, columns cg CPL + c
#pragma unroll
    for (int c = 0; c < CPL; ++c) v[c] = r[c];
    lse_line<CPL>(v);
#pragma unroll
    for (int c = 0; c < CPL; ++c) r[c] = v[c];
    __syncthreads();
    float* k = sL + (cg * CPL) * P + line;        // column `line`, rows cg CPL + c
#pragma unroll
    for (int c = 0; c < CPL; ++c) v[c] = k[c * P];
    lse_line<CPL>(v);
#pragma unroll
    for (int c = 0; c < CPL; ++c) k[c * P] = v[c];
    __syncthreads();
  }
}

// Row `line`: (max over j < N of exp(log_alpha), its lowest j), in every lane of the row's group.  The index
// is always in [0, N): a row with no comparable entry (all NaN) gives index 0, value NaN.
template <int CPL>
__device__ __forceinline__ void argmax_row(const float* sL, int N, int line, int cg, float& bv, int& bi) {
  constexpr int P = SkTile<CPL>::P;
  const float* r = sL + line * P + cg * CPL;
  float v = -1.f;
  int id = 0;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const float e = expf(r[c]);
    if (cg * CPL + c < N && e > v) {
      v = e;
      id = cg * CPL + c;
    }
  }
  auto take = [&](float ov, int oi) {
    if (ov > v || (ov == v && oi < id)) {
      v = ov;
      id = oi;
    }
  };
  take(dpp_f<0xb1>(v), dpp_i<0xb1>(id));
  take(dpp_f<0x4e>(v), dpp_i<0x4e>(id));
  take(dpp_f<0x141>(v), dpp_i<0x141>(id));
  bv = v < 0.f ? __int_as_float(0x7fc00000) : v;
  bi = id;
}

// -log_alpha entry: clamp(cost, -1e4, 1e4) (NaN passes through), negated, times 1 / temperature
__device__ __forceinline__ float la_of(float c, float inv_t) {
  c = c < -TRK_COST_CLAMP ? -TRK_COST_CLAMP : (c > TRK_COST_CLAMP ? TRK_COST_CLAMP : c);
  return -c * inv_t;
}

// SlotTracker.forward after the cost (slot_tracker.py:122-135) for one frame per workgroup.
template <int CPL>
__global__ void __launch_bounds__(64 * CPL)
track_match_kernel(const float* __restrict__ cost, const float* __restrict__ alive_a,
                   const float* __restrict__ alive_b, int64_t* __restrict__ perm, float* __restrict__ matched,
                   float* __restrict__ conf, int N, int n_iters, float inv_t) {
  using S = SkTile<CPL>;
  __shared__ float sL[S::NC * S::P];
  const int64_t f = blockIdx.x;
  const int tid = threadIdx.x, line = (tid >> 6) * 8 + ((tid & 63) >> 3), cg = tid & 7;
  const float* cf = cost + f * N * N;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int j = cg * CPL + c;
    sL[line * S::P + j] = (line < N && j < N) ? la_of(cf[(size_t)line * N + j], inv_t) : -INFINITY;
  }
  __syncthreads();
  sinkhorn_lds<CPL>(sL, n_iters, line, cg);
  float bv;
  int bi;
  argmax_row<CPL>(sL, N, line, cg, bv, bi);
  if (cg == 0 && line < N) {
    const int64_t o = f * N + line;
    const float at = alive_a ? (alive_a[o] > 0.5f ? 1.f : 0.f) : 1.f;
    const float at1 = alive_b ? (alive_b[f * N + bi] > 0.5f ? 1.f : 0.f) : 1.f;
    perm[o] = bi;
    matched[o] = at * at1 * (bv > 0.3f ? 1.f : 0.f);
    if (conf) conf[o] = bv;
  }
}

// The matching half of the tracking loop (model.py:233-252) for one clip per workgroup.  C: cost between
// the unpermuted frames t-1 and t, [clip][T-1][N][N]; alive [clip][T][N] (null: all alive).  Writes, for
// t >= 1, perm32 / perm64 / matched / alive_out at [clip][t][i] (t = 0: identity, 0, alive of frame 0).
// The next frame pair's cost block is loaded into registers while the current step runs.
template <int CPL>
__global__ void __launch_bounds__(64 * CPL)
track_sequence_kernel(const float* __restrict__ C, const float* __restrict__ alive, int* __restrict__ perm32,
                      int64_t* __restrict__ perm64, float* __restrict__ matched, float* __restrict__ alive_out,
                      int T, int N, int n_iters, float inv_t) {
  using S = SkTile<CPL>;
  constexpr int NC = S::NC, P = S::P;
  __shared__ float sL[NC * P];     // log_alpha of the current step
  __shared__ float sC[NC * P];     // cost block of the current frame pair (rows of the unpermuted frame)
  __shared__ int sperm[NC];        // perm of the previous step (rows of the tracked frame t-1)
  __shared__ float salive[NC];     // alive of the tracked frame t-1
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x, line = (tid >> 6) * 8 + ((tid & 63) >> 3), cg = tid & 7;
  const int64_t base = b * T * N;
  if (cg == 0 && line < N) {
    const float al = alive ? alive[base + line] : 1.f;
    sperm[line] = line;
    salive[line] = al;
    perm32[base + line] = line;
    if (perm64) perm64[base + line] = line;
    matched[base + line] = 0.f;
    if (alive_out) alive_out[base + line] = al;
  }
  // this thread's slice of a cost block: row `line`, columns cg CPL + c
  float pf[CPL];
  auto prefetch = [&](int t) {
    const float* ct = C + (((size_t)b * (T - 1) + (t - 1)) * N + (line < N ? line : 0)) * N;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int j = cg * CPL + c;
      pf[c] = (line < N && j < N) ? ct[j] : 0.f;
    }
  };
  if (T > 1) prefetch(1);
  for (int t = 1; t < T; ++t) {
#pragma unroll
    for (int c = 0; c < CPL; ++c) sC[line * P + cg * CPL + c] = pf[c];
    __syncthreads();   // sC complete; the previous step's sperm / salive updates visible
    if (t + 1 < T) prefetch(t + 1);
    const float* src = sC + (line < N ? sperm[line] : 0) * P;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int j = cg * CPL + c;
      sL[line * P + j] = (line < N && j < N) ? la_of(src[j], inv_t) : -INFINITY;
    }
    __syncthreads();
    sinkhorn_lds<CPL>(sL, n_iters, line, cg);
    float bv;
    int bi;
    argmax_row<CPL>(sL, N, line, cg, bv, bi);
    __syncthreads();   // every lane has read sperm, sC and sL
    if (cg == 0 && line < N) {
      const int64_t o = base + (int64_t)t * N;
      const float a1 = alive ? alive[o + bi] : 1.f;
      perm32[o + line] = bi;
      if (perm64) perm64[o + line] = bi;
      matched[o + line] = (salive[line] > 0.5f ? 1.f : 0.f) * (a1 > 0.5f ? 1.f : 0.f) * (bv > 0.3f ? 1.f : 0.f);
      if (alive_out) alive_out[o + line] = a1;
      salive[line] = a1;
      sperm[line] = bi;
    }
  }
}

// ------------------------------------------------------------------------------------- reorder and GRU
// y[row, k] = x[frame * N + perm[row], k] with frame = row / N; an index outside [0, N) gives a NaN row.
// VW = 4: four consecutive k per thread (D a multiple of 4; x and y 16-byte aligned).
template <typename I, int VW>
__global__ void __launch_bounds__(256)
trk_gather_kernel(const float* __restrict__ x, const I* __restrict__ perm, float* __restrict__ y, int64_t rows,
                  int N, int D) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int DU = D / VW;
  if (e >= rows * DU) return;
  const int64_t row = e / DU;
  const int k = (int)(e - row * DU) * VW;
  const int64_t p = (int64_t)perm[row];
  const float nan = __int_as_float(0x7fc00000);
  const bool in = p >= 0 && p < N;
  const float* src = x + ((row / N) * N + (in ? p : 0)) * D + k;
  if constexpr (VW == 4) {
    *reinterpret_cast<float4*>(y + row * D + k) =
        in ? *reinterpret_cast<const float4*>(src) : make_float4(nan, nan, nan, nan);
  } else {
    y[row * D + k] = in ? *src : nan;
  }
}


// torch.nn.GRUCell gates and the matched blend of SlotTracker.reorder_and_update (slot_tracker.py:150-156)
// for rows (f, i), f < nf, i < N:
//   gi = GI[f * sgi + pi] (pi = perm[f * sp + i], or i when perm is null), gh = GH[f * N + i] ([r; z; n]);
//   h' = n + z (h - n), n = tanh(gi_n + r gh_n);  out = m h' + (1 - m) re, m = matched[f * sm + i],
//   re = RE[f * sre + i], h = H[f * N + i].  In place (out == H) is allowed.
__global__ void __launch_bounds__(256)
trk_gru_gate_kernel(const float* __restrict__ GI, int64_t sgi, const int* __restrict__ perm, int64_t sp,
                    const float* __restrict__ GH, const float* __restrict__ matched, int64_t sm,
                    const float* __restrict__ RE, int64_t sre, const float* H, float* out, int64_t nf, int N,
                    int D) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= nf * N * D) return;
  const int64_t row = e / D;
  const int k = (int)(e - row * D);
  const int64_t f = row / N;
  const int i = (int)(row - f * N);
  const int pi = perm ? perm[f * sp + i] : i;
  const float* gi = GI + (f * sgi + pi) * 3 * D;
  const float* gh = GH + row * 3 * D;
  const float r = 1.f / (1.f + expf(-(gi[k] + gh[k])));
  const float z = 1.f / (1.f + expf(-(gi[D + k] + gh[D + k])));
  const float n = tanhf(gi[2 * D + k] + r * gh[2 * D + k]);
  const float h1 = n + z * (H[e] - n);
  const float m = matched[f * sm + i];
  out[e] = m * h1 + (1.f - m) * RE[(f * sre + i) * D + k];
}

// ------------------------------------------------------------------------------------------------ host
static unsigned blocks256(int64_t n) { return (unsigned)((n + 255) / 256); }

template <typename I>
static void launch_gather(const float* x, const I* perm, float* y, int64_t rows, int64_t N, int64_t D,
                          hipStream_t st) {
  if (D % 4 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)y & 15) == 0)
    hipLaunchKernelGGL((trk_gather_kernel<I, 4>), dim3(blocks256(rows * D / 4)), dim3(256), 0, st, x, perm, y, rows,
                       (int)N, (int)D);
  else
    hipLaunchKernelGGL((trk_gather_kernel<I, 1>), dim3(blocks256(rows * D)), dim3(256), 0, st, x, perm, y, rows,
                       (int)N, (int)D);
}

template <int DT, int NW, int KC>
static size_t cost_lds(int D) {
  return ((size_t)16 * NW * (D + 8) + (size_t)D * (KC + 8)) * sizeof(typename MM<DT>::T);
}

constexpr size_t TRK_LDS_MAX = 160 * 1024;

template <int DT, int NW, int KC>
static int launch_cost_kc(const TrackCostArgs& a, hipStream_t st) {
  const size_t lds = cost_lds<DT, NW, KC>(a.D);
  static std::atomic<int> setup[HCLSM_MAX_DEVICES];   // more than the default 64 KB of dynamic LDS, per device
  int unused;
  const int se = device_launch_setup(reinterpret_cast<const void*>(&track_cost_kernel<DT, NW, KC>), 64 * NW, lds,
                                     (int)TRK_LDS_MAX, setup, &unused);
  if (se) return se;
  const int64_t tiles = (a.pairs + 16 * NW - 1) / (16 * NW);
  hipLaunchKernelGGL((track_cost_kernel<DT, NW, KC>), dim3((unsigned)tiles), dim3(64 * NW), lds, st, a);
  HCLSM_LAUNCH_CHECK();
  return 0;
}

template <int DT, int D, int NW>
static int launch_cost_res(const TrackCostArgs& a, hipStream_t st) {
  using T = typename MM<DT>::T;
  constexpr size_t lds = ((size_t)D * (D + 8) + (size_t)(D / 4) * (D + 8)) * sizeof(T) + (size_t)(D / 4) * 8;
  static std::atomic<int> setup[HCLSM_MAX_DEVICES];   // resident workgroups per device (persistent kernel)
  int grid = 0;
  const int se = device_launch_setup(reinterpret_cast<const void*>(&track_cost_res_kernel<DT, D, NW>), 64 * NW, lds,
                                     (int)TRK_LDS_MAX, setup, &grid);
  if (se) return se;
  const int64_t nblk = (a.pairs + 32 * NW - 1) / (32 * NW);
  const unsigned g = (unsigned)(nblk < grid ? nblk : grid);
  hipLaunchKernelGGL((track_cost_res_kernel<DT, D, NW>), dim3(g), dim3(64 * NW), lds, st, a);
  HCLSM_LAUNCH_CHECK();
  return 0;
}

// 16-bit operands: the weight-resident kernel for D <= 192; otherwise 128 pairs per workgroup with weight
// chunks of 64 columns (32 when the LDS would overflow).  fp32: 64 pairs, chunks of 16.
template <int DT>
static int launch_cost(const TrackCostArgs& a, hipStream_t st) {
  if (a.pairs == 0) return 0;
  if constexpr (DT == HCLSM_F32) {
    return launch_cost_kc<DT, 4, 16>(a, st);
  } else {
    if (a.D == 64) return launch_cost_res<DT, 64, 8>(a, st);
    if (a.D == 128) return launch_cost_res<DT, 128, 8>(a, st);
    if (a.D == 192) return launch_cost_res<DT, 192, 8>(a, st);
    if (cost_lds<DT, 8, 64>(a.D) <= TRK_LDS_MAX) return launch_cost_kc<DT, 8, 64>(a, st);
    return launch_cost_kc<DT, 8, 32>(a, st);
  }
}

static int launch_cost_dt(int dtype, const TrackCostArgs& a, hipStream_t st) {
  switch (dtype) {
    case HCLSM_BF16: return launch_cost<HCLSM_BF16>(a, st);
    case HCLSM_F16: return launch_cost<HCLSM_F16>(a, st);
    default: return launch_cost<HCLSM_F32>(a, st);
  }
}

static int clamp_rows(const float* x, float* y, int64_t n, hipStream_t st) {
  if (n == 0) return 0;
  if (n % 4 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)y & 15) == 0)
    hipLaunchKernelGGL(trk_clamp_kernel<4>, dim3(blocks256(n / 4)), dim3(256), 0, st, x, y, n);
  else
    hipLaunchKernelGGL(trk_clamp_kernel<1>, dim3(blocks256(n)), dim3(256), 0, st, x, y, n);
  HCLSM_LAUNCH_CHECK();
  return 0;
}

// Sinkhorn tile for N: CPL columns per lane and CPL waves (8 CPL >= N)
template <typename F>
static int with_tile(int64_t N, F&& fn) {
  using std::integral_constant;
  if (N <= 16) return fn(integral_constant<int, 2>{});
  if (N <= 32) return fn(integral_constant<int, 4>{});
  if (N <= 64) return fn(integral_constant<int, 8>{});
  return fn(integral_constant<int, 16>{});
}

constexpr int64_t TRK_MAX_SLOTS = 128;

// D a multiple of 64 (so D/4 fills 16-wide MFMA tiles) and at most 384 (24 accumulator tiles); the pair
// tile of the widest supported D fits the LDS with 32-column chunks for every operand type.
static int track_check(int64_t N, int64_t D, int dtype) {
  if (N < 0 || D <= 0) return HCLSM_ERR_SHAPE;
  if (dtype != HCLSM_F32 && dtype != HCLSM_BF16 && dtype != HCLSM_F16) return HCLSM_ERR_DTYPE;
  if (D % 64 || D > 384) return HCLSM_ERR_UNSUPPORTED;
  return 0;
}

static float inv_temperature(float temperature) { return 1.f / (temperature > 1e-6f ? temperature : 1e-6f); }

static size_t al256t(size_t v) { return (v + 255) / 256 * 256; }

struct SeqWs {
  size_t s, uv, c, perm, matched, gi, gh, total;
};

static SeqWs seq_ws(int64_t B, int64_t T, int64_t N, int64_t D, bool hidden) {
  SeqWs w{};
  const size_t R = (size_t)B * T * N;
  size_t o = 0;
  w.s = o; o += al256t(R * D * 4);
  w.uv = o; o += al256t(R * 2 * D * 4);
  w.c = o; o += al256t((size_t)B * (T > 0 ? T - 1 : 0) * N * N * 4);
  w.perm = o; o += al256t(R * 4);
  w.matched = o; o += al256t(R * 4);
  if (hidden) {
    w.gi = o; o += al256t(R * 3 * D * 4);
    w.gh = o; o += al256t((size_t)B * N * 3 * D * 4);
  }
  w.total = o;
  return w;
}

}  // namespace hclsm

using namespace hclsm;

// ----------------------------------------------------------------------------------------------- C ABI
extern "C" int64_t hclsm_slot_track_cost_workspace(int64_t frames, int64_t N, int64_t D, int dtype) {
  if (frames < 0) return HCLSM_ERR_SHAPE;
  const int c = track_check(N, D, dtype);
  if (c) return c;
  const size_t R = (size_t)2 * frames * N;
  return (int64_t)(al256t(R * D * 4) + al256t(R * 2 * D * 4));
}

// params: match_mlp.0.weight, .0.bias, match_mlp.2.weight, .2.bias, match_mlp.4.weight, .4.bias
extern "C" int hclsm_slot_track_cost(const float* slots_t, const float* slots_t1, const float* alive_t,
                                     const float* alive_t1, float* cost, int64_t frames, int64_t N, int64_t D,
                                     const void* const* params, int dtype, void* workspace, int64_t workspace_bytes,
                                     void* stream) {
  if (frames < 0) return HCLSM_ERR_SHAPE;
  const int chk = track_check(N, D, dtype);
  if (chk) return chk;
  if (frames * N * N > 0x7fffffffLL * 64) return HCLSM_ERR_SHAPE;
  if (frames == 0 || N == 0) return 0;
  if (!slots_t || !slots_t1 || !cost || !params || !workspace) return HCLSM_ERR_NULL;
  if ((alive_t == nullptr) != (alive_t1 == nullptr)) return HCLSM_ERR_NULL;
  for (int i = 0; i < 6; ++i)
    if (!params[i]) return HCLSM_ERR_NULL;
  if (workspace_bytes < hclsm_slot_track_cost_workspace(frames, N, D, dtype)) return HCLSM_ERR_SHAPE;
  hipStream_t st = (hipStream_t)stream;
  const int64_t FN = frames * N, R = 2 * FN;
  char* ws = reinterpret_cast<char*>(workspace);
  float* S = reinterpret_cast<float*>(ws);
  float* UV = reinterpret_cast<float*>(ws + al256t((size_t)R * D * 4));
  int rc;
  if ((rc = clamp_rows(slots_t, S, FN * D, st))) return rc;
  if ((rc = clamp_rows(slots_t1, S + FN * D, FN * D, st))) return rc;
  const int es = dtype == HCLSM_F32 ? 4 : 2;
  const char* W1 = reinterpret_cast<const char*>(params[0]);
  const float* b1 = reinterpret_cast<const float*>(params[1]);
  // U over the earlier frame's rows (with b1), V over the later frame's rows
  if ((rc = linear_rows(S, D, HCLSM_F32, W1, 3 * D, b1, nullptr, 0, UV, 2 * D, HCLSM_F32, FN, D, D, 0, 0, nullptr,
                        nullptr, 0.f, nullptr, 0, nullptr, 1, dtype, st)))
    return rc;
  if ((rc = linear_rows(S + FN * D, D, HCLSM_F32, W1 + (size_t)D * es, 3 * D, nullptr, nullptr, 0,
                        UV + FN * 2 * D + D, 2 * D, HCLSM_F32, FN, D, D, 0, 0, nullptr, nullptr, 0.f, nullptr, 0,
                        nullptr, 1, dtype, st)))
    return rc;
  TrackCostArgs a{};
  a.S = S; a.UV = UV; a.W1 = params[0]; a.W2 = params[2];
  a.b2 = reinterpret_cast<const float*>(params[3]);
  a.w3 = reinterpret_cast<const float*>(params[4]);
  a.b3 = reinterpret_cast<const float*>(params[5]);
  a.alive_a = alive_t;
  a.alive_b = alive_t1;
  a.boff = FN;
  a.cost = cost;
  a.pairs = frames * N * N;
  a.N = (int)N; a.D = (int)D;
  a.nt = (int)frames; a.tstride = 0; a.fboff = (int)frames;
  return launch_cost_dt(dtype, a, st);
}

extern "C" int hclsm_slot_track_match(const float* cost, const float* alive_t, const float* alive_t1,
                                      int64_t* perm, float* matched, float* confidence, int64_t frames, int64_t N,
                                      int64_t n_iters, float temperature, void* stream) {
  if (frames < 0 || N < 0 || n_iters < 0) return HCLSM_ERR_SHAPE;
  if (N > TRK_MAX_SLOTS) return HCLSM_ERR_UNSUPPORTED;
  if (frames > 0x7fffffffLL || n_iters > 0x7fffffffLL) return HCLSM_ERR_SHAPE;
  if (frames == 0 || N == 0) return 0;
  if (!cost || !perm || !matched) return HCLSM_ERR_NULL;
  hipStream_t st = (hipStream_t)stream;
  const float inv_t = inv_temperature(temperature);
  return with_tile(N, [&](auto cpl) {
    constexpr int CPL = decltype(cpl)::value;
    hipLaunchKernelGGL((track_match_kernel<CPL>), dim3((unsigned)frames), dim3(64 * CPL), 0, st, cost, alive_t,
                       alive_t1, perm, matched, confidence, (int)N, (int)n_iters, inv_t);
    HCLSM_LAUNCH_CHECK();
    return 0;
  });
}

extern "C" int64_t hclsm_slot_track_reorder_update_workspace(int64_t frames, int64_t N, int64_t D, int dtype) {
  if (frames < 0) return HCLSM_ERR_SHAPE;
  const int c = track_check(N, D, dtype);
  if (c) return c;
  return (int64_t)(2 * al256t((size_t)frames * N * 3 * D * 4));
}

// params: hidden_gru.weight_ih, .weight_hh (operand dtype), .bias_ih, .bias_hh (fp32, nullable)
extern "C" int hclsm_slot_track_reorder_update(const float* slots_t1, const int64_t* perm, const float* hidden_t,
                                               const float* matched, float* reordered, float* hidden_t1,
                                               int64_t frames, int64_t N, int64_t D, const void* const* params,
                                               int dtype, void* workspace, int64_t workspace_bytes, void* stream) {
  if (frames < 0) return HCLSM_ERR_SHAPE;
  const int chk = track_check(N, D, dtype);
  if (chk) return chk;
  if (frames * N * 3 * D > 0x7fffffffLL * 64) return HCLSM_ERR_SHAPE;
  if (frames == 0 || N == 0) return 0;
  if (!slots_t1 || !perm || !hidden_t || !matched || !reordered || !hidden_t1 || !params || !workspace)
    return HCLSM_ERR_NULL;
  if (!params[0] || !params[1]) return HCLSM_ERR_NULL;
  if (workspace_bytes < hclsm_slot_track_reorder_update_workspace(frames, N, D, dtype)) return HCLSM_ERR_SHAPE;
  hipStream_t st = (hipStream_t)stream;
  const int64_t R = frames * N;
  char* ws = reinterpret_cast<char*>(workspace);
  float* GI = reinterpret_cast<float*>(ws);
  float* GH = reinterpret_cast<float*>(ws + al256t((size_t)R * 3 * D * 4));
  const float* b_ih = reinterpret_cast<const float*>(params[2]);
  const float* b_hh = reinterpret_cast<const float*>(params[3]);
  launch_gather<int64_t>(slots_t1, perm, reordered, R, N, D, st);
  HCLSM_LAUNCH_CHECK();
  int rc;
  if ((rc = linear_rows(reordered, D, HCLSM_F32, params[0], D, b_ih, nullptr, 0, GI, 3 * D, HCLSM_F32, R, 3 * D, D, 0,
                        0, nullptr, nullptr, 0.f, nullptr, 0, nullptr, 1, dtype, st)))
    return rc;
  if ((rc = linear_rows(hidden_t, D, HCLSM_F32, params[1], D, b_hh, nullptr, 0, GH, 3 * D, HCLSM_F32, R, 3 * D, D, 0,
                        0, nullptr, nullptr, 0.f, nullptr, 0, nullptr, 1, dtype, st)))
    return rc;
  hipLaunchKernelGGL(trk_gru_gate_kernel, dim3(blocks256(R * D)), dim3(256), 0, st, GI, (int64_t)N, nullptr,
                     (int64_t)0, GH, matched, (int64_t)N, reordered, (int64_t)N, hidden_t, hidden_t1, frames, (int)N,
                     (int)D);
  HCLSM_LAUNCH_CHECK();
  return 0;
}

extern "C" int64_t hclsm_slot_track_sequence_workspace(int64_t batch, int64_t T, int64_t N, int64_t D,
                                                       int with_hidden, int dtype) {
  if (batch < 0 || T < 0) return HCLSM_ERR_SHAPE;
  const int c = track_check(N, D, dtype);
  if (c) return c;
  if (N > TRK_MAX_SLOTS) return HCLSM_ERR_UNSUPPORTED;
  return (int64_t)seq_ws(batch, T, N, D, with_hidden != 0).total;
}

// params: the six match_mlp tensors, then hidden_gru.weight_ih, .weight_hh, .bias_ih, .bias_hh (only read
// when hidden is wanted).
extern "C" int hclsm_slot_track_sequence(const float* slots, const float* alive, float* tracked, float* alive_out,
                                         int64_t* perm, float* matched, float* hidden, int64_t batch, int64_t T,
                                         int64_t N, int64_t D, int64_t n_iters, float temperature,
                                         const void* const* params, int dtype, void* workspace,
                                         int64_t workspace_bytes, void* stream) {
  if (batch < 0 || T < 0 || n_iters < 0) return HCLSM_ERR_SHAPE;
  const int chk = track_check(N, D, dtype);
  if (chk) return chk;
  if (N > TRK_MAX_SLOTS) return HCLSM_ERR_UNSUPPORTED;
  if (batch > 0x7fffffffLL || T > 0x7fffffffLL || n_iters > 0x7fffffffLL) return HCLSM_ERR_SHAPE;
  if (batch * T * N * 3 * D > 0x7fffffffLL * 64) return HCLSM_ERR_SHAPE;
  if (batch == 0 || T == 0 || N == 0) return 0;
  if (!slots || !tracked || !params || !workspace) return HCLSM_ERR_NULL;
  for (int i = 0; i < 6; ++i)
    if (!params[i]) return HCLSM_ERR_NULL;
  if (hidden && (!params[6] || !params[7])) return HCLSM_ERR_NULL;
  const SeqWs L = seq_ws(batch, T, N, D, hidden != nullptr);
  if (workspace_bytes < (int64_t)L.total) return HCLSM_ERR_SHAPE;
  hipStream_t st = (hipStream_t)stream;
  char* ws = reinterpret_cast<char*>(workspace);
  float* S = reinterpret_cast<float*>(ws + L.s);
  float* UV = reinterpret_cast<float*>(ws + L.uv);
  float* C = reinterpret_cast<float*>(ws + L.c);
  int* P = reinterpret_cast<int*>(ws + L.perm);
  float* M = matched ? matched : reinterpret_cast<float*>(ws + L.matched);
  const int64_t R = batch * T * N;
  const int es = dtype == HCLSM_F32 ? 4 : 2;
  int rc;
  if (T > 1) {
    // pair MLP over every (t-1, t) frame pair: U = W1a s + b1 and V = W1b s for every node row
    if ((rc = clamp_rows(slots, S, R * D, st))) return rc;
    const char* W1 = reinterpret_cast<const char*>(params[0]);
    if ((rc = linear_rows(S, D, HCLSM_F32, W1, 3 * D, reinterpret_cast<const float*>(params[1]), nullptr, 0, UV,
                          2 * D, HCLSM_F32, R, D, D, 0, 0, nullptr, nullptr, 0.f, nullptr, 0, nullptr, 1, dtype, st)))
      return rc;
    if ((rc = linear_rows(S, D, HCLSM_F32, W1 + (size_t)D * es, 3 * D, nullptr, nullptr, 0, UV + D, 2 * D, HCLSM_F32,
                          R, D, D, 0, 0, nullptr, nullptr, 0.f, nullptr, 0, nullptr, 1, dtype, st)))
      return rc;
    TrackCostArgs a{};
    a.S = S; a.UV = UV; a.W1 = params[0]; a.W2 = params[2];
    a.b2 = reinterpret_cast<const float*>(params[3]);
    a.w3 = reinterpret_cast<const float*>(params[4]);
    a.b3 = reinterpret_cast<const float*>(params[5]);
    a.alive_a = alive;
    a.alive_b = alive;
    a.boff = 0;
    a.cost = C;
    a.pairs = batch * (T - 1) * N * N;
    a.N = (int)N; a.D = (int)D;
    a.nt = (int)(T - 1); a.tstride = (int)T; a.fboff = 1;
    if ((rc = launch_cost_dt(dtype, a, st))) return rc;
  }
  const float inv_t = inv_temperature(temperature);
  rc = with_tile(N, [&](auto cpl) {
    constexpr int CPL = decltype(cpl)::value;
    hipLaunchKernelGGL((track_sequence_kernel<CPL>), dim3((unsigned)batch), dim3(64 * CPL), 0, st, C, alive, P, perm,
                       M, alive_out, (int)T, (int)N, (int)n_iters, inv_t);
    HCLSM_LAUNCH_CHECK();
    return 0;
  });
  if (rc) return rc;
  launch_gather<int>(slots, P, tracked, R, N, D, st);
  HCLSM_LAUNCH_CHECK();
  if (!hidden) return 0;
  // GRU carry (slot_tracker.py:150-156): hidden_0 = 0; for t >= 1 hidden_t = blend(GRU(tracked_t, hidden_{t-1}))
  float* GI = reinterpret_cast<float*>(ws + L.gi);
  float* GH = reinterpret_cast<float*>(ws + L.gh);
  const float* b_ih = reinterpret_cast<const float*>(params[8]);
  const float* b_hh = reinterpret_cast<const float*>(params[9]);
  if ((rc = zero_fill_f32(hidden, batch * N * D, st))) return rc;
  if (T < 2) return 0;
  if ((rc = linear_rows(slots, D, HCLSM_F32, params[6], D, b_ih, nullptr, 0, GI, 3 * D, HCLSM_F32, R, 3 * D, D, 0, 0,
                        nullptr, nullptr, 0.f, nullptr, 0, nullptr, 1, dtype, st)))
    return rc;
  const int64_t BN = batch * N;
  for (int64_t t = 1; t < T; ++t) {
    if ((rc = linear_rows(hidden, D, HCLSM_F32, params[7], D, b_hh, nullptr, 0, GH, 3 * D, HCLSM_F32, BN, 3 * D, D,
                          0, 0, nullptr, nullptr, 0.f, nullptr, 0, nullptr, 1, dtype, st)))
      return rc;
    hipLaunchKernelGGL(trk_gru_gate_kernel, dim3(blocks256(BN * D)), dim3(256), 0, st, GI + t * N * 3 * D, T * N,
                       P + t * N, T * N, GH, M + t * N, T * N, tracked + t * N * D, T * N, hidden, hidden, batch,
                       (int)N, (int)D);
    HCLSM_LAUNCH_CHECK();
  }
  return 0;
}
