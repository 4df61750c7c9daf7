// Relation graph (GNN over object slots) for gfx950: RelationGraph.forward of
// hclsm/objects/relation_graph.py:68-193 without materialising the (frames, N, N, 4D) pair tensor.
//
// Edge features of pair (i, j) of a frame: e = ReLU(W2 ReLU(W1 LN(p) + b1) + b2) with
// p = [n_i; n_j; n_i - n_j; n_i * n_j] (4D) and LN the pair LayerNorm (weight gamma, bias beta).
// Since LN(p) = (p - mu) rstd * gamma + beta with per-pair scalars mu, rstd, the first layer is
//   W1 LN(p) + b1 = rstd (P_i + Q_j + A4 (n_i * n_j) - mu r) + c
// with, per node, P_i = (W1_1 + W1_3) G n_i and Q_j = (W1_2 - W1_3) G n_j (W1_k the k-th D-column block
// of W1, G = diag(gamma)), A4 = W1_4 G, r = W1 gamma, c = W1 beta + b1; and per pair
//   mu = (2 s_i + g_ij) / 4D,   E[p^2] = (2 q_i + 2 q_j - 2 g_ij + h_ij) / 4D,
// s = sum n, q = sum n^2, g_ij = sum n_i n_j, h_ij = sum (n_i n_j)^2.  So the per-pair contraction is
// only A4 (n_i * n_j) (K = D instead of 4D), and P, Q are one GEMM over the nodes.
//
// gnn_prep_kernel   derives [P-weights; Q-weights] (4E x D), A4 (2E x D), r, c from the module's W1, b1,
//                   gamma, beta (once per call).
// gnn_edge_kernel   one workgroup per (frame, 16*NW consecutive pairs of whole i-rows); each wave a
//                   16-pair MFMA row tile:
//                   A  Hadamard GEMM A4 (n_i * n_j) with g, h, s, q accumulated while the operand is
//                      formed; epilogue adds P_i + Q_j, normalises, + c, ReLU -> H1 in LDS
//                   B  H1 W2^T + b2, ReLU -> edge features in LDS; edge weight
//                      w = sigmoid(we . e + be) * alive_i * alive_j
//                   C  (messages) ReLU(e Wm^T + bm) * w summed over j -> agg[i]  (per-wave partial sums
//                      in LDS, added in a fixed order: deterministic)
//                   D  (causal) sigmoid(c2 . ReLU(e C1^T + d1) + d2) * alive_i * alive_j -> causal[i, j]
// The node update nodes += U2 ReLU(U1 [nodes; agg] + c1) + c2 runs on the MFMA linear kernels.
#include "internal.h"
#include "pair_tile.h"

#include <utility>

namespace hclsm {

struct GnnArgs {
  const float* X;      // node features, row stride ldx
  int64_t ldx;
  const float* PQ;     // [F*N, 4E] fp32: P (first 2E), Q (next 2E)
  const void* A4;      // [2E, D] operand dtype
  const float* r;      // [2E]
  const float* c;      // [2E]
  const void* W2;      // [E, 2E]
  const float* b2;     // [E]
  const float* we;     // [E]
  const float* be;     // [1]
  const void* Wm;      // [D, E]
  const float* bm;     // [D]
  const void* C1;      // [E/2, E]
  const float* d1;     // [E/2]
  const float* cc2;    // [E/2]
  const float* d2;     // [1]
  const float* alive;  // [F, N] or null
  float* agg;          // messages summed over j, row stride ldagg (null: not wanted)
  int64_t ldagg;
  float* causal;       // [F, N, N] or null
  float* edges;        // [F, N, enj, E] fp32 edge features of the targets j in [ej0, ej0 + enj), or null
  int ej0, enj;
  int F, N, NP, D, E;  // NP = N rounded up to 16 (pairs of a padded i-row)
  int norm;            // 1: pair LayerNorm folded in (RelationGraph); 0: no pair norm (gnn_message_pass)
  float eps;
};

// Weight chunks are staged in LDS (shared by the workgroup's waves): KC columns of every output row
// (KC a multiple of the fragment block KB; smaller KC when the widest layer would not fit).

template <int DT, int NW, int KC>
__global__ void __launch_bounds__(64 * NW)
gnn_edge_kernel(GnnArgs a) {
  using A = MM<DT>;
  using T = typename A::T;
  constexpr int KE = GFrag<DT>::KE, KB = GFrag<DT>::KB, PW = KC + 8;
  static_assert(KC % KB == 0, "chunk of whole fragment blocks");
  constexpr int ROWS = 16 * NW, NTH = 64 * NW;
  extern __shared__ __align__(16) unsigned char smem[];
  const int N = a.N, NP = a.NP, D = a.D, E = a.E, H1 = 2 * E;
  const int LH = H1 + 8, LE = E + 8;     // LDS row pitches (elements)
  const int WR = (H1 > D ? H1 : D);      // most weight rows staged at once
  T* sH = reinterpret_cast<T*>(smem);                                                  // [ROWS][LH], then [ROWS][LE]
  T* sW = sH + (size_t)ROWS * LH;                                                      // [WR][PW] weight chunk
  float* sw = reinterpret_cast<float*>(sW + (size_t)WR * PW);                          // [ROWS] edge weights
  float* sst = sw + ROWS;                                                              // [ROWS][2] mu, rstd
  float* sagg = sst + 2 * ROWS;                                                        // [NW][D] message sums
  const int G = ROWS / NP;                                                             // i-rows per workgroup
  const int tiles_f = (N + G - 1) / G;
  const int f = blockIdx.x / tiles_f;
  const int i0 = (blockIdx.x - f * tiles_f) * G;
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63, g = lane >> 4, li = lane & 15;
  auto row_pair = [&](int row, int& i, int& j) {
    const int il = row / NP;
    i = i0 + il;
    j = row - il * NP;
    return il < G && i < N && j < N;
  };
  const float* Xf = a.X + (size_t)f * N * a.ldx;
  const float* alive = a.alive ? a.alive + (size_t)f * N : nullptr;
  auto pair_mask = [&](int i, int j) { return alive ? alive[i] * alive[j] : 1.f; };
  auto gemm = [&](auto& acc, int NT, const T* W, int K, auto a_frag) {
    tile_gemm<DT, KC, NTH>(acc, NT, W, K, K, sW, tid, a_frag);
  };

  // ---- A: Hadamard GEMM + pair statistics -> H1
  {
    const int row = wid * 16 + li;
    int ia, ja;
    const bool okA = row_pair(row, ia, ja);
    const float* xi = Xf + (size_t)(okA ? ia : 0) * a.ldx;
    const float* xj = Xf + (size_t)(okA ? ja : 0) * a.ldx;
    float gs = 0.f, hs = 0.f, si = 0.f, qi = 0.f, qj = 0.f;
    const int NT = H1 / 16;
    f32x4 acc[24];
#pragma unroll
    for (int t = 0; t < 24; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    gemm(acc, NT, reinterpret_cast<const T*>(a.A4), D, [&](int k, T* op) {
      float vi[KE], vj[KE];
#pragma unroll
      for (int e = 0; e < KE; e += 4) {
        const float4 x4 = *reinterpret_cast<const float4*>(xi + k + e);
        const float4 y4 = *reinterpret_cast<const float4*>(xj + k + e);
        vi[e] = x4.x; vi[e + 1] = x4.y; vi[e + 2] = x4.z; vi[e + 3] = x4.w;
        vj[e] = y4.x; vj[e + 1] = y4.y; vj[e + 2] = y4.z; vj[e + 3] = y4.w;
      }
#pragma unroll
      for (int e = 0; e < KE; ++e) {
        const float pr = vi[e] * vj[e];
        gs += pr;
        hs = fmaf(pr, pr, hs);
        si += vi[e];
        qi = fmaf(vi[e], vi[e], qi);
        qj = fmaf(vj[e], vj[e], qj);
        op[e] = A::fromf(pr);
      }
    });
    // row sums over the four lane groups sharing the row
#pragma unroll
    for (int m = 16; m < 64; m <<= 1) {
      gs += __shfl_xor(gs, m, 64);
      hs += __shfl_xor(hs, m, 64);
      si += __shfl_xor(si, m, 64);
      qi += __shfl_xor(qi, m, 64);
      qj += __shfl_xor(qj, m, 64);
    }
    if (g == 0) {
      const float inv = 1.f / (4.f * (float)D);
      const float mu = (2.f * si + gs) * inv;
      const float m2 = (2.f * qi + 2.f * qj - 2.f * gs + hs) * inv;
      sst[2 * row] = a.norm ? mu : 0.f;
      sst[2 * row + 1] = a.norm ? 1.f / sqrtf(fmaxf(m2 - mu * mu, 0.f) + a.eps) : 1.f;
    }
    __syncthreads();   // statistics of every row are in LDS
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int orow = wid * 16 + 4 * g + rr;
      int i, j;
      const bool ok = row_pair(orow, i, j);
      const float mu = sst[2 * orow], rs = sst[2 * orow + 1];
      const float* P = a.PQ + ((size_t)f * N + (ok ? i : 0)) * 2 * H1;
      const float* Q = a.PQ + ((size_t)f * N + (ok ? j : 0)) * 2 * H1 + H1;
#pragma unroll
      for (int t = 0; t < 24; ++t) {
        if (t < NT) {
          const int o = t * 16 + li;
          const float v = fmaf(P[o] + Q[o] + acc[t][rr] - mu * a.r[o], rs, a.c[o]);
          sH[(size_t)orow * LH + o] = A::fromf(ok ? fmaxf(v, 0.f) : 0.f);
        }
      }
    }
  }

  // ---- B: H1 W2^T + b2, ReLU -> edge features (written over H1 after everyone has read it)
  {
    const int NT = E / 16;
    f32x4 acc[12];
#pragma unroll
    for (int t = 0; t < 12; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    const T* hrow = sH + (size_t)(wid * 16 + li) * LH;
    gemm(acc, NT, reinterpret_cast<const T*>(a.W2), H1, [&](int k, T* op) { frag_load<DT>(hrow + k, op); });
    __syncthreads();   // H1 fully consumed
#pragma unroll
    for (int t = 0; t < 12; ++t) {
      if (t < NT) {
        const int o = t * 16 + li;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          sH[(size_t)(wid * 16 + 4 * g + rr) * LE + o] = A::fromf(fmaxf(acc[t][rr] + a.b2[o], 0.f));
      }
    }
  }
  __syncthreads();
  const T* sE = sH;
  const T* erow = sE + (size_t)(wid * 16 + li) * LE;
  if (a.edges) {   // edge features of the output window, as the next layers see them
    for (int e = tid; e < ROWS * E; e += NTH) {
      const int row = e / E, o = e - row * E;
      int i, j;
      if (row_pair(row, i, j) && j >= a.ej0 && j < a.ej0 + a.enj)
        a.edges[(((size_t)f * N + i) * a.enj + (j - a.ej0)) * E + o] = A::tof(sE[(size_t)row * LE + o]);
    }
  }
  // edge weight per row
  for (int row = tid; row < ROWS; row += NTH) {
    int i, j;
    const bool ok = row_pair(row, i, j);
    float s = a.be[0];
    for (int o = 0; o < E; ++o) s = fmaf(A::tof(sE[(size_t)row * LE + o]), a.we[o], s);
    sw[row] = ok ? pair_mask(i, j) / (1.f + __expf(-s)) : 0.f;
  }
  // (the first chunk staging of the next GEMM begins with a barrier: sw is complete before it is read)

  // ---- C: messages, summed over the wave's 16 pairs (one i-row: NP is a multiple of 16)
  if (a.agg) {
    const int NTALL = D / 16;
    const T* Wm = reinterpret_cast<const T*>(a.Wm);
    for (int t0 = 0; t0 < NTALL; t0 += 12) {
      const int NT = NTALL - t0 < 12 ? NTALL - t0 : 12;
      f32x4 acc[12];
#pragma unroll
      for (int t = 0; t < 12; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
      gemm(acc, NT, Wm + (size_t)t0 * 16 * E, E, [&](int k, T* op) { frag_load<DT>(erow + k, op); });
#pragma unroll
      for (int t = 0; t < 12; ++t) {
        if (t < NT) {
          const int o = (t0 + t) * 16 + li;
          float sacc = 0.f;
#pragma unroll
          for (int rr = 0; rr < 4; ++rr)
            sacc = fmaf(fmaxf(acc[t][rr] + a.bm[o], 0.f), sw[wid * 16 + 4 * g + rr], sacc);
          sacc = rows4_sum(sacc);
          if (g == 0) sagg[wid * D + o] = sacc;
        }
      }
    }
    __syncthreads();
    // agg[i] = sum of the partials of the NP/16 waves of row i, in wave order
    const int wpr = NP / 16;
    for (int e = tid; e < G * D; e += NTH) {
      const int il = e / D, o = e - il * D;
      const int i = i0 + il;
      if (i < N) {
        float sacc = 0.f;
        for (int w = 0; w < wpr; ++w) sacc += sagg[(il * wpr + w) * D + o];
        a.agg[((size_t)f * N + i) * a.ldagg + o] = sacc;
      }
    }
  }

  // ---- D: causal edge probabilities
  if (a.causal) {
    const int NT = E / 32;
    f32x4 acc[6];
#pragma unroll
    for (int t = 0; t < 6; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    gemm(acc, NT, reinterpret_cast<const T*>(a.C1), E, [&](int k, T* op) { frag_load<DT>(erow + k, op); });
    float part[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 6; ++t) {
      if (t < NT) {
        const int o = t * 16 + li;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) part[rr] = fmaf(fmaxf(acc[t][rr] + a.d1[o], 0.f), a.cc2[o], part[rr]);
      }
    }
#pragma unroll
    for (int rr = 0; rr < 4; ++rr)
#pragma unroll
      for (int m = 1; m < 16; m <<= 1) part[rr] += __shfl_xor(part[rr], m, 64);
    if (li == 0) {
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        int i, j;
        if (row_pair(wid * 16 + 4 * g + rr, i, j))
          a.causal[((size_t)f * N + i) * N + j] = pair_mask(i, j) / (1.f + __expf(-(part[rr] + a.d2[0])));
      }
    }
  }
}

// Weight-resident edge kernel for 16-bit operands at the preset shapes (D, E) = (64, 32), (128, 64), (192, 96).
// A persistent workgroup stages A4, W2 and Wm (messages) and / or C1 (causal head) in LDS once; each wave then
// owns whole source rows i (frame f), 32 targets j per chunk as two 16-pair MFMA tiles.
//   A  A4 (n_i * n_j) with the weights as the A operand: lane (g, li) holds outputs 4g .. 4g+3 of each
//      16-wide tile for pair li, so the pair statistics, P_i + Q_j and the normalisation stay in the lane.
//   B  W2 H1: H1 is the B operand straight from A's accumulators (W2's columns stored in the matching order:
//      positions 8g .. 8g+7 of a 32-wide block hold k = 4g .. 4g+3 and 16 + 4g .. 16 + 4g+3); edge weight.
//   C  messages with the edge features as the A operand (pairs as rows), so the sum over j is four pairs in
//      the lane, then the two tiles, then over the lane groups; Wm's columns in the same order as W2's.
//   D  causal head with C1 as the A operand, the score reduced over the lane groups.
// Node sums s, q come precomputed (nstat); only g = sum n_i n_j and h = sum (n_i n_j)^2 are per pair.
template <typename T>
__device__ __forceinline__ uint32_t pack2(T lo, T hi) {
  return (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
}

template <int D, int E, bool MSG, bool CAUS>
struct GnnRes {
  static constexpr int H1 = 2 * E, PA = D + 8, PB = H1 + 8, PC = E + 8;
  static constexpr size_t a4 = 0;
  static constexpr size_t w2 = a4 + (size_t)H1 * PA * 2;
  static constexpr size_t wm = w2 + (size_t)E * PB * 2;
  static constexpr size_t c1 = wm + (MSG ? (size_t)D * PC * 2 : 0);
  static constexpr size_t vec = c1 + (CAUS ? (size_t)(E / 2) * PC * 2 : 0);
  // fp32 vectors: r, c [H1]; b2, we [E]; bm [D]; d1, cc2 [E/2]
  static constexpr size_t r = vec, c = r + H1 * 4, b2 = c + H1 * 4, we = b2 + E * 4, bm = we + E * 4;
  static constexpr size_t d1 = bm + (MSG ? D * 4 : 0), cc2 = d1 + (CAUS ? (E / 2) * 4 : 0);
  static constexpr size_t total = cc2 + (CAUS ? (E / 2) * 4 : 0);
};

// rows x KC of W (row stride ldw) into sW (pitch P) with the columns of every 32-wide block permuted so that
// positions 8g .. 8g+7 hold k = 4g .. 4g+3 and 16 + 4g .. 16 + 4g+3
template <typename T, int NTH>
__device__ __forceinline__ void stage_permuted(const T* __restrict__ W, int ldw, int rows, int K, T* sW, int P,
                                               int tid) {
  for (int u = tid; u < rows * (K / 8); u += NTH) {
    const int rr = u / (K / 8), q = (u - rr * (K / 8)) * 8;
    const int kb = q & ~31, gg = (q & 31) >> 3;
    const uint2 lo = *reinterpret_cast<const uint2*>(W + (size_t)rr * ldw + kb + 4 * gg);
    const uint2 hi = *reinterpret_cast<const uint2*>(W + (size_t)rr * ldw + kb + 16 + 4 * gg);
    *reinterpret_cast<uint4*>(sW + rr * P + q) = make_uint4(lo.x, lo.y, hi.x, hi.y);
  }
}

template <int DT, int D, int E, int NW, bool MSG, bool CAUS, bool MP>
__global__ void __launch_bounds__(64 * NW)
gnn_edge_res_kernel(GnnArgs a, const float* __restrict__ nstat) {
  using A = MM<DT>;
  using T = typename A::T;
  using L = GnnRes<D, E, MSG, CAUS>;
  static_assert(DT != HCLSM_F32 && D % 32 == 0 && E % 32 == 0, "16-bit operands, D and E multiples of 32");
  constexpr int NTH = 64 * NW, H1 = L::H1, PA = L::PA, PB = L::PB, PC = L::PC;
  constexpr int NT1 = H1 / 16, NT2 = E / 16, NT3 = D / 16, NT4 = E / 32;
  extern __shared__ __align__(16) unsigned char smem[];
  T* sA4 = reinterpret_cast<T*>(smem + L::a4);
  T* sW2 = reinterpret_cast<T*>(smem + L::w2);
  T* sWm = reinterpret_cast<T*>(smem + L::wm);
  T* sC1 = reinterpret_cast<T*>(smem + L::c1);
  float* sr = reinterpret_cast<float*>(smem + L::r);
  float* sc = reinterpret_cast<float*>(smem + L::c);
  float* sb2 = reinterpret_cast<float*>(smem + L::b2);
  float* swe = reinterpret_cast<float*>(smem + L::we);
  float* sbm = reinterpret_cast<float*>(smem + L::bm);
  float* sd1 = reinterpret_cast<float*>(smem + L::d1);
  float* scc2 = reinterpret_cast<float*>(smem + L::cc2);
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63, g = lane >> 4, li = lane & 15;
  {
    const T* A4 = reinterpret_cast<const T*>(a.A4);
    for (int u = tid; u < H1 * (D / 8); u += NTH) {
      const int rr = u / (D / 8), q = (u - rr * (D / 8)) * 8;
      *reinterpret_cast<uint4*>(sA4 + rr * PA + q) = *reinterpret_cast<const uint4*>(A4 + (size_t)rr * D + q);
    }
    stage_permuted<T, NTH>(reinterpret_cast<const T*>(a.W2), H1, E, H1, sW2, PB, tid);
    if constexpr (MSG) stage_permuted<T, NTH>(reinterpret_cast<const T*>(a.Wm), E, D, E, sWm, PC, tid);
    if constexpr (CAUS) stage_permuted<T, NTH>(reinterpret_cast<const T*>(a.C1), E, E / 2, E, sC1, PC, tid);
    for (int u = tid; u < H1; u += NTH) {
      sr[u] = a.r[u];
      sc[u] = a.c[u];
    }
    for (int u = tid; u < E; u += NTH) {
      sb2[u] = a.b2[u];
      swe[u] = a.we[u];
    }
    if constexpr (MSG)
      for (int u = tid; u < D; u += NTH) sbm[u] = a.bm[u];
    if constexpr (CAUS)
      for (int u = tid; u < E / 2; u += NTH) {
        sd1[u] = a.d1[u];
        scc2[u] = a.cc2[u];
      }
  }
  __syncthreads();
  const int N = a.N;
  const int64_t units = (int64_t)a.F * N;
  const float inv4d = 1.f / (4.f * (float)D);
  for (int64_t unit = (int64_t)blockIdx.x * NW + wid; unit < units; unit += (int64_t)gridDim.x * NW) {
    const int64_t f = unit / N;
    const int i = (int)(unit - f * N);
    const int64_t rowi = f * N + i;
    const float* xi = a.X + rowi * a.ldx;
    const float ali = a.alive ? a.alive[rowi] : 1.f;
    const float si = nstat[2 * rowi], qi = nstat[2 * rowi + 1];
    float aggp[NT3];   // message partial sums for outputs 16t + li over this lane's pairs
#pragma unroll
    for (int t = 0; t < NT3; ++t) aggp[t] = 0.f;
    for (int j0 = 0; j0 < N; j0 += 32) {
      int jj[2];
      const float* xj[2];
#pragma unroll
      for (int pt = 0; pt < 2; ++pt) {
        const int j = j0 + 16 * pt + li;
        jj[pt] = j;
        xj[pt] = a.X + (f * N + (j < N ? j : N - 1)) * a.ldx;
      }
      // ---- A: Hadamard GEMM, pair statistics
      f32x4 acc[2][NT1];
#pragma unroll
      for (int pt = 0; pt < 2; ++pt)
#pragma unroll
        for (int t = 0; t < NT1; ++t) acc[pt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
      float gs[2] = {0.f, 0.f}, hs[2] = {0.f, 0.f};
      float4 xr[6];
      auto load_k = [&](int kb) {
        xr[0] = *reinterpret_cast<const float4*>(xi + kb + 8 * g);
        xr[1] = *reinterpret_cast<const float4*>(xi + kb + 8 * g + 4);
#pragma unroll
        for (int pt = 0; pt < 2; ++pt) {
          xr[2 + 2 * pt] = *reinterpret_cast<const float4*>(xj[pt] + kb + 8 * g);
          xr[3 + 2 * pt] = *reinterpret_cast<const float4*>(xj[pt] + kb + 8 * g + 4);
        }
      };
      load_k(0);
#pragma unroll 1
      for (int kb = 0; kb < D; kb += 32) {
        T op[2][8];
        const float vi[8] = {xr[0].x, xr[0].y, xr[0].z, xr[0].w, xr[1].x, xr[1].y, xr[1].z, xr[1].w};
#pragma unroll
        for (int pt = 0; pt < 2; ++pt) {
          const float vj[8] = {xr[2 + 2 * pt].x, xr[2 + 2 * pt].y, xr[2 + 2 * pt].z, xr[2 + 2 * pt].w,
                               xr[3 + 2 * pt].x, xr[3 + 2 * pt].y, xr[3 + 2 * pt].z, xr[3 + 2 * pt].w};
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float pr = vi[e] * vj[e];
            gs[pt] += pr;
            hs[pt] = fmaf(pr, pr, hs[pt]);
            op[pt][e] = A::fromf(pr);
          }
        }
        if (kb + 32 < D) load_k(kb + 32);
#pragma unroll
        for (int t = 0; t < NT1; ++t) {
          T wf[8];
          frag_load<DT>(sA4 + (16 * t + li) * PA + kb + 8 * g, wf);
#pragma unroll
          for (int pt = 0; pt < 2; ++pt) acc[pt][t] = frag_mma<DT>(wf, op[pt], acc[pt][t]);
        }
      }
      // normalise: v = rstd (P_i + Q_j + acc - mu r) + c, ReLU (outputs 16t + 4g + rr of pair li)
      const float* P = a.PQ + rowi * 2 * H1 + 4 * g;
#pragma unroll
      for (int pt = 0; pt < 2; ++pt) {
        float gg = gs[pt], hh = hs[pt];
        gg = rows4_sum(gg);
        hh = rows4_sum(hh);
        const int64_t rowj = f * N + (jj[pt] < N ? jj[pt] : N - 1);
        const float qj = nstat[2 * rowj + 1];
        const float mu = MP ? 0.f : (2.f * si + gg) * inv4d;
        const float m2 = (2.f * qi + 2.f * qj - 2.f * gg + hh) * inv4d;
        const float rs = MP ? 1.f : 1.f / sqrtf(fmaxf(m2 - mu * mu, 0.f) + a.eps);
        const float* Q = a.PQ + rowj * 2 * H1 + H1 + 4 * g;
#pragma unroll
        for (int t0 = 0; t0 < NT1; t0 += 3) {
#pragma unroll
          for (int t = t0; t < t0 + 3 && t < NT1; ++t) {
            const float4 p4 = *reinterpret_cast<const float4*>(P + 16 * t);
            const float4 q4 = *reinterpret_cast<const float4*>(Q + 16 * t);
            const float4 r4 = *reinterpret_cast<const float4*>(sr + 16 * t + 4 * g);
            const float4 c4 = *reinterpret_cast<const float4*>(sc + 16 * t + 4 * g);
            acc[pt][t][0] = fmaxf(fmaf(p4.x + q4.x + acc[pt][t][0] - mu * r4.x, rs, c4.x), 0.f);
            acc[pt][t][1] = fmaxf(fmaf(p4.y + q4.y + acc[pt][t][1] - mu * r4.y, rs, c4.y), 0.f);
            acc[pt][t][2] = fmaxf(fmaf(p4.z + q4.z + acc[pt][t][2] - mu * r4.z, rs, c4.z), 0.f);
            acc[pt][t][3] = fmaxf(fmaf(p4.w + q4.w + acc[pt][t][3] - mu * r4.w, rs, c4.w), 0.f);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      // ---- B: edge features e = ReLU(W2 H1 + b2), rounded to the operand type as the next layers see them
      f32x4 acc2[2][NT2];
#pragma unroll
      for (int pt = 0; pt < 2; ++pt)
#pragma unroll
        for (int t = 0; t < NT2; ++t) acc2[pt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < H1 / 32; ++kb) {
        T hb[2][8];
#pragma unroll
        for (int pt = 0; pt < 2; ++pt)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            hb[pt][e] = A::fromf(acc[pt][2 * kb][e]);
            hb[pt][4 + e] = A::fromf(acc[pt][2 * kb + 1][e]);
          }
#pragma unroll
        for (int t = 0; t < NT2; ++t) {
          T wf[8];
          frag_load<DT>(sW2 + (16 * t + li) * PB + 32 * kb + 8 * g, wf);
#pragma unroll
          for (int pt = 0; pt < 2; ++pt) acc2[pt][t] = frag_mma<DT>(wf, hb[pt], acc2[pt][t]);
        }
      }
      // edge features of pair li, outputs 16t + 4g + rr, as packed operand pairs (rr = 0,1 | 2,3)
      uint32_t ebp[2][NT2][2];
      float wgt[2];      // edge weight of pair li
#pragma unroll
      for (int pt = 0; pt < 2; ++pt) {
        float s = 0.f;
#pragma unroll
        for (int t = 0; t < NT2; ++t) {
          T ev[4];
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) {
            const int o = 16 * t + 4 * g + rr;
            ev[rr] = A::fromf(fmaxf(acc2[pt][t][rr] + sb2[o], 0.f));
            s = fmaf(A::tof(ev[rr]), swe[o], s);
          }
          ebp[pt][t][0] = pack2<T>(ev[0], ev[1]);
          ebp[pt][t][1] = pack2<T>(ev[2], ev[3]);
          const int je = jj[pt] - a.ej0;
          if (MP && a.edges && jj[pt] < N && je >= 0 && je < a.enj)
            *reinterpret_cast<float4*>(a.edges + (rowi * a.enj + je) * E + 16 * t + 4 * g) =
                make_float4(A::tof(ev[0]), A::tof(ev[1]), A::tof(ev[2]), A::tof(ev[3]));
        }
        s = rows4_sum(s);
        const int j = jj[pt];
        const float alj = j < N ? (a.alive ? a.alive[f * N + j] : 1.f) : 0.f;
        wgt[pt] = ali * alj / (1.f + __expf(-(s + a.be[0])));
      }
      // k-block kb of the edge features as an MFMA operand (tiles 2kb and 2kb + 1, in the permuted k order)
      auto e_op = [&](int pt, int kb) {
        return __builtin_bit_cast(typename A::Op, make_uint4(ebp[pt][2 * kb][0], ebp[pt][2 * kb][1],
                                                            ebp[pt][2 * kb + 1][0], ebp[pt][2 * kb + 1][1]));
      };
      // ---- C: messages ReLU(Wm e + bm) * w summed over the pairs (outputs in two halves)
      if constexpr (MSG) {
        constexpr int HT = (NT3 + 1) / 2;
#pragma unroll
        for (int pt = 0; pt < 2; ++pt) {
          float wr[4];   // weights of pairs 4g + rr of this tile
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) wr[rr] = __shfl(wgt[pt], 4 * g + rr, 64);
#pragma unroll
          for (int h0 = 0; h0 < NT3; h0 += HT) {
            f32x4 acc3[HT];
#pragma unroll
            for (int t = 0; t < HT; ++t) acc3[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kb = 0; kb < E / 32; ++kb) {
              const typename A::Op ea = e_op(pt, kb);
#pragma unroll
              for (int t = 0; t < HT; ++t) {
                if (h0 + t < NT3)
                  acc3[t] = A::mfma(ea, A::load(sWm + (16 * (h0 + t) + li) * PC + 32 * kb + 8 * g), acc3[t]);
              }
            }
#pragma unroll
            for (int t = 0; t < HT; ++t) {
              if (h0 + t < NT3) {
                const float bmo = sbm[16 * (h0 + t) + li];
#pragma unroll
                for (int rr = 0; rr < 4; ++rr)
                  aggp[h0 + t] = fmaf(fmaxf(acc3[t][rr] + bmo, 0.f), wr[rr], aggp[h0 + t]);
              }
            }
          }
        }
      }
      // ---- D: causal edges
      if constexpr (CAUS) {
#pragma unroll
        for (int pt = 0; pt < 2; ++pt) {
          f32x4 acc4[NT4];
#pragma unroll
          for (int t = 0; t < NT4; ++t) acc4[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kb = 0; kb < E / 32; ++kb) {
            const typename A::Op hb = e_op(pt, kb);
#pragma unroll
            for (int t = 0; t < NT4; ++t)
              acc4[t] = A::mfma(A::load(sC1 + (16 * t + li) * PC + 32 * kb + 8 * g), hb, acc4[t]);
          }
          float s = 0.f;
#pragma unroll
          for (int t = 0; t < NT4; ++t)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
              const int o = 16 * t + 4 * g + rr;
              s = fmaf(fmaxf(acc4[t][rr] + sd1[o], 0.f), scc2[o], s);
            }
          s = rows4_sum(s);
          const int j = jj[pt];
          if (g == 0 && j < N) {
            const float alj = a.alive ? a.alive[f * N + j] : 1.f;
            a.causal[rowi * N + j] = ali * alj / (1.f + __expf(-(s + a.d2[0])));
          }
        }
      }
    }
    if constexpr (MSG) {
#pragma unroll
      for (int t = 0; t < NT3; ++t) {
        float v = aggp[t];
        v = rows4_sum(v);
        if (g == 0) a.agg[rowi * a.ldagg + 16 * t + li] = v;
      }
    }
  }
}

// Chunk-streamed edge kernel for 16-bit operands at the base preset's shape (D, E) = (256, 128), whose weights
// exceed the LDS: the same register-chained phases as gnn_edge_res_kernel, with one 16-pair tile per wave, and all
// weights streamed through a double-buffered LDS ring in 64-column chunks (A4, then W2, then Wm and / or C1;
// the schedule repeats every step, so the next chunk's global loads are always in flight while the current one
// is multiplied; one barrier per chunk).  A workgroup owns NW consecutive source rows (one per wave) and steps
// through the targets 16 at a time; the messages of a row are summed over the steps in registers.
template <int D, int E, bool MSG, bool CAUS>
struct GnnStr {
  static constexpr int H1 = 2 * E, KS = 64, PS = KS + 8;
  static constexpr int RMAX = H1 > D ? H1 : D;
  static constexpr int NA = D / KS, NB = H1 / KS, NC = MSG ? E / KS : 0, ND = CAUS ? E / KS : 0;
  static constexpr int NCH = NA + NB + NC + ND;
  static constexpr size_t buf = (size_t)RMAX * PS * 2;   // one chunk buffer (bytes)
  // fp32 vectors first: their offsets fit the 16-bit immediate of LDS reads
  static constexpr size_t r = 0, c = r + H1 * 4, b2 = c + H1 * 4, we = b2 + E * 4, bm = we + E * 4;
  static constexpr size_t d1 = bm + D * 4, cc2 = d1 + (E / 2) * 4;
  static constexpr size_t buf0 = (cc2 + (E / 2) * 4 + 255) / 256 * 256, buf1 = buf0 + buf, total = buf1 + buf;
};

template <int N_, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  [&]<int... I>(std::integer_sequence<int, I...>) { (f(std::integral_constant<int, I>{}), ...); }
  (std::make_integer_sequence<int, N_>{});
}

template <int DT, int D, int E, int NW, bool MSG, bool CAUS, bool MP>
__global__ void __launch_bounds__(64 * NW)
gnn_edge_str_kernel(GnnArgs a, const float* __restrict__ nstat) {
  using A = MM<DT>;
  using T = typename A::T;
  using L = GnnStr<D, E, MSG, CAUS>;
  static_assert(DT != HCLSM_F32 && D % 64 == 0 && E % 64 == 0, "16-bit operands, D and E multiples of 64");
  constexpr int NTH = 64 * NW, H1 = L::H1, KS = L::KS, PS = L::PS, NCH = L::NCH;
  constexpr int NA = L::NA, NB = L::NB, NC = L::NC;
  constexpr int NT1 = H1 / 16, NT2 = E / 16, NT3 = D / 16, NT4 = E / 32;
  constexpr int UPT = (L::RMAX * (KS / 8) + NTH - 1) / NTH;   // 16-byte units per thread per chunk
  extern __shared__ __align__(16) unsigned char smem[];
  T* sbuf0 = reinterpret_cast<T*>(smem + L::buf0);
  T* sbuf1 = reinterpret_cast<T*>(smem + L::buf1);
  float* sr = reinterpret_cast<float*>(smem + L::r);
  float* sc = reinterpret_cast<float*>(smem + L::c);
  float* sb2 = reinterpret_cast<float*>(smem + L::b2);
  float* swe = reinterpret_cast<float*>(smem + L::we);
  float* sbm = reinterpret_cast<float*>(smem + L::bm);
  float* sd1 = reinterpret_cast<float*>(smem + L::d1);
  float* scc2 = reinterpret_cast<float*>(smem + L::cc2);
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63, g = lane >> 4, li = lane & 15;
  for (int u = tid; u < H1; u += NTH) {
    sr[u] = a.r[u];
    sc[u] = a.c[u];
  }
  for (int u = tid; u < E; u += NTH) {
    sb2[u] = a.b2[u];
    swe[u] = a.we[u];
  }
  for (int u = tid; u < D; u += NTH) sbm[u] = MSG ? a.bm[u] : 0.f;
  for (int u = tid; u < E / 2; u += NTH) {
    sd1[u] = CAUS ? a.d1[u] : 0.f;
    scc2[u] = CAUS ? a.cc2[u] : 0.f;
  }
  // chunk ch of the periodic schedule: weight rows, their row stride, the first column, permuted or not
  auto chunk_src = [&](int ch, const T*& W, int& rows, int& ld, int& k0, bool& perm) {
    if (ch < NA) { W = reinterpret_cast<const T*>(a.A4); rows = H1; ld = D; k0 = ch * KS; perm = false; }
    else if (ch < NA + NB) { W = reinterpret_cast<const T*>(a.W2); rows = E; ld = H1; k0 = (ch - NA) * KS; perm = true; }
    else if (ch < NA + NB + NC) { W = reinterpret_cast<const T*>(a.Wm); rows = D; ld = E; k0 = (ch - NA - NB) * KS; perm = true; }
    else { W = reinterpret_cast<const T*>(a.C1); rows = E / 2; ld = E; k0 = (ch - NA - NB - NC) * KS; perm = true; }
  };
  uint4 stg[UPT];
  // The staging addresses are recomputed at every chunk from a copy of tid the compiler cannot see through:
  // hoisted out of the loops, the addresses of every chunk of the schedule would stay live in registers.
  auto opaque_tid = [&]() {
    int t = tid;
    asm volatile("" : "+v"(t));
    return t;
  };
  auto load_chunk = [&](int ch) {
    const T* W;
    int rows, ld, k0;
    bool perm;
    chunk_src(ch, W, rows, ld, k0, perm);
    const int t0 = opaque_tid();
#pragma unroll
    for (int q = 0; q < UPT; ++q) {
      const int u = t0 + q * NTH, rr = u / (KS / 8), p = (u - rr * (KS / 8)) * 8;
      if (rr < rows) {
        const T* src = W + (size_t)rr * ld + k0;
        if (perm) {
          const int kb = p & ~31, gg = (p & 31) >> 3;
          const uint2 lo = *reinterpret_cast<const uint2*>(src + kb + 4 * gg);
          const uint2 hi = *reinterpret_cast<const uint2*>(src + kb + 16 + 4 * gg);
          stg[q] = make_uint4(lo.x, lo.y, hi.x, hi.y);
        } else {
          stg[q] = *reinterpret_cast<const uint4*>(src + p);
        }
      }
    }
  };
  auto store_chunk = [&](int ch, T* buf) {
    const T* W;
    int rows, ld, k0;
    bool perm;
    chunk_src(ch, W, rows, ld, k0, perm);
    const int t0 = opaque_tid();
#pragma unroll
    for (int q = 0; q < UPT; ++q) {
      const int u = t0 + q * NTH, rr = u / (KS / 8), p = (u - rr * (KS / 8)) * 8;
      if (rr < rows) *reinterpret_cast<uint4*>(buf + rr * PS + p) = stg[q];
    }
  };
  const int N = a.N;
  const int64_t rows_all = (int64_t)a.F * N;
  const int64_t groups = (rows_all + NW - 1) / NW;
  const int steps = (N + 15) / 16;
  const float inv4d = 1.f / (4.f * (float)D);
  // prologue: chunk 0 of the schedule into buffer 0
  load_chunk(0);
  store_chunk(0, sbuf0);
  __syncthreads();
  int cur = 0;   // buffer holding the chunk about to be used (the schedule restarts with chunk 0 each step)
  for (int64_t grp = blockIdx.x; grp < groups; grp += gridDim.x) {
    const int64_t rowi_raw = grp * NW + wid;
    const bool live_row = rowi_raw < rows_all;
    const int64_t rowi = live_row ? rowi_raw : rows_all - 1;
    const int64_t f = rowi / N;
    const float* xi = a.X + rowi * a.ldx;
    const float ali = a.alive ? a.alive[rowi] : 1.f;
    const float si = nstat[2 * rowi], qi = nstat[2 * rowi + 1];
    float aggp[NT3];
#pragma unroll
    for (int t = 0; t < NT3; ++t) aggp[t] = 0.f;
    for (int st = 0; st < steps; ++st) {
      const int j = st * 16 + li;
      const int64_t rowj = f * N + (j < N ? j : N - 1);
      const float* xj = a.X + rowj * a.ldx;
      // accumulators of the four phases; each is cleared at its phase's first chunk (disjoint live ranges)
      f32x4 acc[NT1], acc2[NT2], acc3[NT3], acc4[NT4];
      float gs = 0.f, hs = 0.f, wgt = 0.f;
      uint32_t ebp[NT2][2];
      // node rows of the current A chunk (this lane's 2 x 8 columns of x_i and x_j), loaded one chunk ahead
      float4 xr[8], xn[8];
      auto load_x = [&](int kc, float4 (&d)[8]) {
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const int k = kc * KS + 32 * s2 + 8 * g;
          d[4 * s2] = *reinterpret_cast<const float4*>(xi + k);
          d[4 * s2 + 1] = *reinterpret_cast<const float4*>(xi + k + 4);
          d[4 * s2 + 2] = *reinterpret_cast<const float4*>(xj + k);
          d[4 * s2 + 3] = *reinterpret_cast<const float4*>(xj + k + 4);
        }
      };
      load_x(0, xr);
      auto e_op = [&](int kb) {
        return __builtin_bit_cast(typename A::Op, make_uint4(ebp[2 * kb][0], ebp[2 * kb][1], ebp[2 * kb + 1][0],
                                                            ebp[2 * kb + 1][1]));
      };
      static_for<NCH>([&](auto chc) {
        constexpr int ch = decltype(chc)::value;
        const T* sb = cur ? sbuf1 : sbuf0;
        load_chunk(ch + 1 < NCH ? ch + 1 : 0);   // the next chunk of the schedule, in flight
        if constexpr (ch < NA) {
          // ---- A: Hadamard GEMM over columns [64 ch, 64 ch + 64)
          if constexpr (ch == 0) {
#pragma unroll
            for (int t = 0; t < NT1; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
          }
          if constexpr (ch + 1 < NA) load_x(ch + 1, xn);
#pragma unroll
          for (int s = 0; s < 2; ++s) {
            const float4 x0 = xr[4 * s], x1 = xr[4 * s + 1], y0 = xr[4 * s + 2], y1 = xr[4 * s + 3];
            const float vi[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            const float vj[8] = {y0.x, y0.y, y0.z, y0.w, y1.x, y1.y, y1.z, y1.w};
            T op[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const float pr = vi[e] * vj[e];
              gs += pr;
              hs = fmaf(pr, pr, hs);
              op[e] = A::fromf(pr);
            }
            const typename A::Op opv = A::load(op);
#pragma unroll
            for (int t = 0; t < NT1; ++t) {
              acc[t] = A::mfma(A::load(sb + (16 * t + li) * PS + 32 * s + 8 * g), opv, acc[t]);
              if ((t & 3) == 3) __builtin_amdgcn_sched_barrier(0);   // at most 4 fragments in flight
            }
          }
          if constexpr (ch + 1 < NA) {
#pragma unroll
            for (int q = 0; q < 8; ++q) xr[q] = xn[q];
          }
          if constexpr (ch == NA - 1) {
            // normalise: v = rstd (P_i + Q_j + acc - mu r) + c, ReLU (outputs 16t + 4g + rr of pair li)
            gs = rows4_sum(gs);
            hs = rows4_sum(hs);
            const float qj = nstat[2 * rowj + 1];
            const float mu = MP ? 0.f : (2.f * si + gs) * inv4d;
            const float m2 = (2.f * qi + 2.f * qj - 2.f * gs + hs) * inv4d;
            const float rs = MP ? 1.f : 1.f / sqrtf(fmaxf(m2 - mu * mu, 0.f) + a.eps);
            const float* P = a.PQ + rowi * 2 * H1 + 4 * g;
            const float* Q = a.PQ + rowj * 2 * H1 + H1 + 4 * g;
#pragma unroll
            for (int t0 = 0; t0 < NT1; t0 += 4) {
#pragma unroll
              for (int t = t0; t < t0 + 4 && t < NT1; ++t) {
                const float4 p4 = *reinterpret_cast<const float4*>(P + 16 * t);
                const float4 q4 = *reinterpret_cast<const float4*>(Q + 16 * t);
                const float4 r4 = *reinterpret_cast<const float4*>(sr + 16 * t + 4 * g);
                const float4 c4 = *reinterpret_cast<const float4*>(sc + 16 * t + 4 * g);
                acc[t][0] = fmaxf(fmaf(p4.x + q4.x + acc[t][0] - mu * r4.x, rs, c4.x), 0.f);
                acc[t][1] = fmaxf(fmaf(p4.y + q4.y + acc[t][1] - mu * r4.y, rs, c4.y), 0.f);
                acc[t][2] = fmaxf(fmaf(p4.z + q4.z + acc[t][2] - mu * r4.z, rs, c4.z), 0.f);
                acc[t][3] = fmaxf(fmaf(p4.w + q4.w + acc[t][3] - mu * r4.w, rs, c4.w), 0.f);
              }
              __builtin_amdgcn_sched_barrier(0);
            }
          }
        } else if constexpr (ch < NA + NB) {
          // ---- B: W2 H1 over H1 columns [64 (ch - NA), +64): k-blocks kb take acc tiles 2kb, 2kb + 1
          constexpr int cb = ch - NA;
          if constexpr (cb == 0) {
#pragma unroll
            for (int t = 0; t < NT2; ++t) acc2[t] = f32x4{0.f, 0.f, 0.f, 0.f};
          }
#pragma unroll
          for (int s = 0; s < 2; ++s) {
            const int kb = 2 * cb + s;
            T hb[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              hb[e] = A::fromf(acc[2 * kb][e]);
              hb[4 + e] = A::fromf(acc[2 * kb + 1][e]);
            }
            const typename A::Op hv = A::load(hb);
#pragma unroll
            for (int t = 0; t < NT2; ++t) {
              acc2[t] = A::mfma(A::load(sb + (16 * t + li) * PS + 32 * s + 8 * g), hv, acc2[t]);
              if ((t & 3) == 3) __builtin_amdgcn_sched_barrier(0);
            }
          }
          if constexpr (ch == NA + NB - 1) {
            float sw = 0.f;
#pragma unroll
            for (int t = 0; t < NT2; ++t) {
              T ev[4];
#pragma unroll
              for (int rr = 0; rr < 4; ++rr) {
                const int o = 16 * t + 4 * g + rr;
                ev[rr] = A::fromf(fmaxf(acc2[t][rr] + sb2[o], 0.f));
                sw = fmaf(A::tof(ev[rr]), swe[o], sw);
              }
              ebp[t][0] = pack2<T>(ev[0], ev[1]);
              ebp[t][1] = pack2<T>(ev[2], ev[3]);
              const int je = j - a.ej0;
              if (MP && a.edges && live_row && j < N && je >= 0 && je < a.enj)
                *reinterpret_cast<float4*>(a.edges + (rowi * a.enj + je) * E + 16 * t + 4 * g) =
                    make_float4(A::tof(ev[0]), A::tof(ev[1]), A::tof(ev[2]), A::tof(ev[3]));
            }
            sw = rows4_sum(sw);
            const float alj = j < N ? (a.alive ? a.alive[rowj] : 1.f) : 0.f;
            wgt = ali * alj / (1.f + __expf(-(sw + a.be[0])));
          }
        } else if constexpr (ch < NA + NB + NC) {
          // ---- C: messages over edge-feature columns [64 (ch - NA - NB), +64); pairs as the A operand
          constexpr int cc = ch - NA - NB;
          if constexpr (cc == 0) {
#pragma unroll
            for (int t = 0; t < NT3; ++t) acc3[t] = f32x4{0.f, 0.f, 0.f, 0.f};
          }
#pragma unroll
          for (int s = 0; s < 2; ++s) {
            const typename A::Op ea = e_op(2 * cc + s);
#pragma unroll
            for (int t = 0; t < NT3; ++t) {
              acc3[t] = A::mfma(ea, A::load(sb + (16 * t + li) * PS + 32 * s + 8 * g), acc3[t]);
              if ((t & 3) == 3) __builtin_amdgcn_sched_barrier(0);
            }
          }
          if constexpr (ch == NA + NB + NC - 1) {
            float wr[4];   // weights of pairs 4g + rr
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) wr[rr] = __shfl(wgt, 4 * g + rr, 64);
#pragma unroll
            for (int t = 0; t < NT3; ++t) {
              const float bmo = sbm[16 * t + li];
#pragma unroll
              for (int rr = 0; rr < 4; ++rr) aggp[t] = fmaf(fmaxf(acc3[t][rr] + bmo, 0.f), wr[rr], aggp[t]);
            }
          }
        } else {
          // ---- D: causal head over edge-feature columns [64 (ch - NA - NB - NC), +64)
          constexpr int cd = ch - NA - NB - NC;
          if constexpr (cd == 0) {
#pragma unroll
            for (int t = 0; t < NT4; ++t) acc4[t] = f32x4{0.f, 0.f, 0.f, 0.f};
          }
#pragma unroll
          for (int s = 0; s < 2; ++s) {
            const typename A::Op hb = e_op(2 * cd + s);
#pragma unroll
            for (int t = 0; t < NT4; ++t) {
              acc4[t] = A::mfma(A::load(sb + (16 * t + li) * PS + 32 * s + 8 * g), hb, acc4[t]);
              if ((t & 3) == 3) __builtin_amdgcn_sched_barrier(0);
            }
          }
          if constexpr (ch == NCH - 1) {
            float s = 0.f;
#pragma unroll
            for (int t = 0; t < NT4; ++t)
#pragma unroll
              for (int rr = 0; rr < 4; ++rr) {
                const int o = 16 * t + 4 * g + rr;
                s = fmaf(fmaxf(acc4[t][rr] + sd1[o], 0.f), scc2[o], s);
              }
            s = rows4_sum(s);
            if (g == 0 && j < N && live_row) {
              const float alj = a.alive ? a.alive[rowj] : 1.f;
              a.causal[rowi * N + j] = ali * alj / (1.f + __expf(-(s + a.d2[0])));
            }
          }
        }
        // the other buffer was last read in the previous chunk, before the barrier that ended it
        store_chunk(ch + 1 < NCH ? ch + 1 : 0, cur ? sbuf0 : sbuf1);
        __syncthreads();
        cur ^= 1;
      });
    }
    if constexpr (MSG) {
#pragma unroll
      for (int t = 0; t < NT3; ++t) {
        float v = aggp[t];
        v = rows4_sum(v);
        if (g == 0 && live_row) a.agg[rowi * a.ldagg + 16 * t + li] = v;
      }
    }
  }
}

// s = sum_k x[row, k], q = sum_k x[row, k]^2 for every row (one wave per row); float4 loads, all of a lane's
// in flight at once, when vec (D and ldx multiples of 4, x 16-byte aligned)
__global__ void __launch_bounds__(256)
gnn_node_stats_kernel(const float* __restrict__ x, int64_t ldx, float* __restrict__ st, int64_t rows, int D,
                      int vec) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  float s = 0.f, q = 0.f;
  if (vec) {
    const float4* xr = reinterpret_cast<const float4*>(x + row * ldx);
#pragma unroll 4
    for (int u = lane; u < D / 4; u += 64) {
      const float4 v = xr[u];
      s += (v.x + v.y) + (v.z + v.w);
      q = fmaf(v.x, v.x, fmaf(v.y, v.y, fmaf(v.z, v.z, fmaf(v.w, v.w, q))));
    }
  } else {
    for (int k = lane; k < D; k += 64) {
      const float v = x[row * ldx + k];
      s += v;
      q = fmaf(v, v, q);
    }
  }
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) {
    s += __shfl_xor(s, m, 64);
    q += __shfl_xor(q, m, 64);
  }
  if (lane == 0) {
    st[2 * row] = s;
    st[2 * row + 1] = q;
  }
}

// [P-weights; Q-weights] (4E x D), A4 (2E x D) in the operand dtype, r and c (2E) in fp32, from W1 (2E x 4D,
// operand dtype), b1, gamma, beta.  Grid: one workgroup per output row o < 2E.
template <int DT>
__global__ void __launch_bounds__(256)
gnn_prep_kernel(const typename MM<DT>::T* __restrict__ W1, const float* __restrict__ b1,
                const float* __restrict__ gam, const float* __restrict__ bet, typename MM<DT>::T* __restrict__ WPQ,
                typename MM<DT>::T* __restrict__ A4, float* __restrict__ r, float* __restrict__ c, int D, int E) {
  using A = MM<DT>;
  const int o = blockIdx.x, H1 = 2 * E;
  const typename A::T* w = W1 + (size_t)o * 4 * D;
  float sr = 0.f, sc = 0.f;
  for (int k = threadIdx.x; k < D; k += blockDim.x) {
    auto gm = [&](int i) { return gam ? gam[i] : 1.f; };   // no pair norm: gamma 1, beta 0
    const float w1 = A::tof(w[k]) * gm(k), w2 = A::tof(w[D + k]) * gm(D + k);
    const float w3 = A::tof(w[2 * D + k]) * gm(2 * D + k), w4 = A::tof(w[3 * D + k]) * gm(3 * D + k);
    WPQ[(size_t)o * D + k] = A::fromf(w1 + w3);
    WPQ[(size_t)(H1 + o) * D + k] = A::fromf(w2 - w3);
    A4[(size_t)o * D + k] = A::fromf(w4);
    sr += w1 + w2 + w3 + w4;
#pragma unroll
    for (int q = 0; q < 4; ++q) sc = fmaf(A::tof(w[q * D + k]), bet ? bet[q * D + k] : 0.f, sc);
  }
  __shared__ float red[2][256];
  red[0][threadIdx.x] = sr;
  red[1][threadIdx.x] = sc;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) {
      red[0][threadIdx.x] += red[0][threadIdx.x + s];
      red[1][threadIdx.x] += red[1][threadIdx.x + s];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    r[o] = red[0][0];
    c[o] = red[1][0] + (b1 ? b1[o] : 0.f);
  }
}

// y[row * ldy + k] = x[row * ldx + k] * alive[row] for k < D (alive nullable); VW = 4: float4 units (D, ldx,
// ldy multiples of 4, x and y 16-byte aligned).
template <int VW>
__global__ void __launch_bounds__(256)
gnn_copy_rows_kernel(const float* __restrict__ x, int64_t ldx, const float* __restrict__ alive,
                     float* __restrict__ y, int64_t ldy, int64_t rows, int D) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int DU = D / VW;
  if (e >= rows * DU) return;
  const int64_t row = e / DU, k = (e - row * DU) * VW;
  const float a = alive ? alive[row] : 1.f;
  if constexpr (VW == 4) {
    float4 v = *reinterpret_cast<const float4*>(x + row * ldx + k);
    v.x *= a; v.y *= a; v.z *= a; v.w *= a;
    *reinterpret_cast<float4*>(y + row * ldy + k) = v;
  } else {
    y[row * ldy + k] = x[row * ldx + k] * a;
  }
}

struct GnnWs {
  size_t wpq, a4, r, c, pq, xa, u, nstat, total;
};

static size_t al256g(size_t v) { return (v + 255) / 256 * 256; }

static GnnWs gnn_ws(int64_t F, int64_t N, int64_t D, int64_t E, int es) {
  GnnWs w;
  size_t o = 0;
  const size_t R = (size_t)F * N;
  w.wpq = o; o += al256g((size_t)4 * E * D * es);
  w.a4 = o; o += al256g((size_t)2 * E * D * es);
  w.r = o; o += al256g((size_t)2 * E * 4);
  w.c = o; o += al256g((size_t)2 * E * 4);
  w.pq = o; o += al256g(R * 4 * E * 4);
  w.xa = o; o += al256g(R * 2 * D * 4);
  w.u = o; o += al256g(R * D * es);
  w.nstat = o; o += al256g(R * 2 * 4);
  w.total = o;
  return w;
}

template <int DT, int NW, int KC>
static size_t edge_lds(const GnnArgs& a) {
  using T = typename MM<DT>::T;
  const int WR = 2 * a.E > a.D ? 2 * a.E : a.D;
  return ((size_t)16 * NW * (2 * a.E + 8) + (size_t)WR * (KC + 8)) * sizeof(T) + (size_t)16 * NW * 3 * 4 +
         (size_t)NW * a.D * 4;
}

template <int DT, int NW, int KC>
static int launch_edges_kc(const GnnArgs& a, hipStream_t st) {
  const int G = 16 * NW / a.NP;
  const int64_t tiles = (int64_t)a.F * ((a.N + G - 1) / G);
  const size_t lds = edge_lds<DT, NW, KC>(a);
  static std::atomic<int> setup[HCLSM_MAX_DEVICES];   // more than the default 64 KB of dynamic LDS, per device
  int unused;
  const int se = device_launch_setup(reinterpret_cast<const void*>(&gnn_edge_kernel<DT, NW, KC>), 64 * NW, lds,
                                     160 * 1024, setup, &unused);
  if (se) return se;
  hipLaunchKernelGGL((gnn_edge_kernel<DT, NW, KC>), dim3((unsigned)tiles), dim3(64 * NW), lds, st, a);
  HCLSM_LAUNCH_CHECK();
  return 0;
}

// 16-bit operands: 128 pairs per workgroup, weight chunks of 64 columns (32 if the LDS would overflow);
// fp32: 64 pairs, chunks of 16.
constexpr size_t GNN_LDS_MAX = 160 * 1024;

template <int DT>
static bool edges_fit(const GnnArgs& a) {
  if constexpr (DT == HCLSM_F32) return edge_lds<DT, 4, 16>(a) <= GNN_LDS_MAX;
  else return edge_lds<DT, 8, 32>(a) <= GNN_LDS_MAX;
}

template <int DT, int D, int E, bool MSG, bool CAUS, bool MP = false>
static int launch_edges_res(const GnnArgs& a, const float* nstat, hipStream_t st) {
  constexpr int NW = 8;
  constexpr size_t lds = GnnRes<D, E, MSG, CAUS>::total;
  static_assert(lds <= GNN_LDS_MAX, "resident weights exceed the LDS");
  static std::atomic<int> setup[HCLSM_MAX_DEVICES];   // resident workgroups per device (persistent kernel)
  int grid = 0;
  const int se = device_launch_setup(reinterpret_cast<const void*>(&gnn_edge_res_kernel<DT, D, E, NW, MSG, CAUS, MP>),
                                     64 * NW, lds, (int)GNN_LDS_MAX, setup, &grid);
  if (se) return se;
  const int64_t units = (int64_t)a.F * a.N;
  const int64_t need = (units + NW - 1) / NW;
  const unsigned g = (unsigned)(need < grid ? need : grid);
  hipLaunchKernelGGL((gnn_edge_res_kernel<DT, D, E, NW, MSG, CAUS, MP>), dim3(g), dim3(64 * NW), lds, st, a, nstat);
  HCLSM_LAUNCH_CHECK();
  return 0;
}

// The resident kernel for the preset shapes (messages and causal head in one pass when both fit the LDS,
// otherwise one pass each over the same edges); 1 on a shape it does not cover.
template <int DT, int D, int E>
static int edges_res_shape(const GnnArgs& a, const float* nstat, hipStream_t st) {
  const bool msg = a.agg != nullptr, caus = a.causal != nullptr;
  // gnn_message_pass (no pair norm, edge-feature output, messages without the causal head) is an instantiation
  // of its own: with the norm switch and the edge stores as run-time branches the other variants spill.
  if (!a.norm) return msg && !caus ? launch_edges_res<DT, D, E, true, false, true>(a, nstat, st) : 1;
  if (msg && caus) {
    if constexpr (GnnRes<D, E, true, true>::total <= GNN_LDS_MAX) {
      return launch_edges_res<DT, D, E, true, true>(a, nstat, st);
    } else {
      GnnArgs m = a, c = a;
      m.causal = nullptr;
      c.agg = nullptr;
      const int rc = launch_edges_res<DT, D, E, true, false>(m, nstat, st);
      return rc ? rc : launch_edges_res<DT, D, E, false, true>(c, nstat, st);
    }
  }
  if (msg) return launch_edges_res<DT, D, E, true, false>(a, nstat, st);
  if (caus) return launch_edges_res<DT, D, E, false, true>(a, nstat, st);
  return 0;
}

template <int DT, int D, int E, bool MSG, bool CAUS, bool MP = false>
static int launch_edges_str(const GnnArgs& a, const float* nstat, hipStream_t st) {
  constexpr int NW = 4;   // one wave per SIMD: the accumulators can use the AGPRs
  constexpr size_t lds = GnnStr<D, E, MSG, CAUS>::total;
  static_assert(lds <= GNN_LDS_MAX, "chunk buffers exceed the LDS");
  static std::atomic<int> setup[HCLSM_MAX_DEVICES];   // resident workgroups per device (persistent kernel)
  int grid = 0;
  const int se = device_launch_setup(reinterpret_cast<const void*>(&gnn_edge_str_kernel<DT, D, E, NW, MSG, CAUS, MP>),
                                     64 * NW, lds, (int)GNN_LDS_MAX, setup, &grid);
  if (se) return se;
  const int64_t groups = ((int64_t)a.F * a.N + NW - 1) / NW;
  const unsigned g = (unsigned)(groups < grid ? groups : grid);
  hipLaunchKernelGGL((gnn_edge_str_kernel<DT, D, E, NW, MSG, CAUS, MP>), dim3(g), dim3(64 * NW), lds, st, a, nstat);
  HCLSM_LAUNCH_CHECK();
  return 0;
}

template <int DT, int D, int E>
static int edges_str_shape(const GnnArgs& a, const float* nstat, hipStream_t st) {
  const bool msg = a.agg != nullptr, caus = a.causal != nullptr;
  if (!a.norm) return msg && !caus ? launch_edges_str<DT, D, E, true, false, true>(a, nstat, st) : 1;
  if (msg && caus) return launch_edges_str<DT, D, E, true, true>(a, nstat, st);
  if (msg) return launch_edges_str<DT, D, E, true, false>(a, nstat, st);
  if (caus) return launch_edges_str<DT, D, E, false, true>(a, nstat, st);
  return 0;
}

template <int DT>
static int launch_edges_resident(const GnnArgs& a, const float* nstat, hipStream_t st) {
  if (a.D == 256 && a.E == 128) return edges_str_shape<DT, 256, 128>(a, nstat, st);
  if (a.D == 64 && a.E == 32) return edges_res_shape<DT, 64, 32>(a, nstat, st);
  if (a.D == 128 && a.E == 64) return edges_res_shape<DT, 128, 64>(a, nstat, st);
  if (a.D == 192 && a.E == 96) return edges_res_shape<DT, 192, 96>(a, nstat, st);
  return 1;
}

template <int DT>
static int launch_edges(const GnnArgs& a, hipStream_t st) {
  if constexpr (DT == HCLSM_F32) {
    if (edge_lds<DT, 4, 16>(a) > GNN_LDS_MAX) return HCLSM_ERR_UNSUPPORTED;
    return launch_edges_kc<DT, 4, 16>(a, st);
  } else {
    if (edge_lds<DT, 8, 64>(a) <= GNN_LDS_MAX) return launch_edges_kc<DT, 8, 64>(a, st);
    if (edge_lds<DT, 8, 32>(a) <= GNN_LDS_MAX) return launch_edges_kc<DT, 8, 32>(a, st);
    return HCLSM_ERR_UNSUPPORTED;
  }
}

static int copy_rows(const float* x, int64_t ldx, const float* alive, float* y, int64_t ldy, int64_t rows, int64_t D,
                     hipStream_t st) {
  const int64_t n = rows * D;
  if (n == 0) return 0;
  const bool vec = D % 4 == 0 && ldx % 4 == 0 && ldy % 4 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)y & 15) == 0;
  if (vec)
    hipLaunchKernelGGL(gnn_copy_rows_kernel<4>, dim3((unsigned)((n / 4 + 255) / 256)), dim3(256), 0, st, x, ldx, alive,
                       y, ldy, rows, (int)D);
  else
    hipLaunchKernelGGL(gnn_copy_rows_kernel<1>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, ldx, alive, y,
                       ldy, rows, (int)D);
  HCLSM_LAUNCH_CHECK();
  return 0;
}

static GnnArgs a0_shape(int64_t F, int64_t N, int64_t D, int64_t E) {
  GnnArgs a{};
  a.F = (int)F; a.N = (int)N; a.NP = (int)((N + 15) / 16 * 16); a.D = (int)D; a.E = (int)E;
  return a;
}

// One GNN call's workspace views and the steps shared by RelationGraph.forward and gnn_message_pass: the node
// projections P | Q, the edge pass (messages and / or causal edges and / or edge features), the node update.
template <int DT>
struct GnnRun {
  using T = typename MM<DT>::T;
  GnnArgs a{};
  T* WPQ;
  T* A4;
  float* r;
  float* c;
  float* PQ;
  float* XA;      // [F*N, 2D]: nodes | messages
  void* U;        // [F*N, D] hidden layer of the node update
  float* nstat;   // [F*N][2] node sums and sums of squares
  int64_t R, D, E, ld;
  const void* u1;
  const float* c1;
  const void* u2;
  const float* c2;
  hipStream_t st;

  GnnRun(char* ws, const GnnWs& L, int64_t F, int64_t N, int64_t D_, int64_t E_, const float* alive, hipStream_t s)
      : WPQ(reinterpret_cast<T*>(ws + L.wpq)), A4(reinterpret_cast<T*>(ws + L.a4)),
        r(reinterpret_cast<float*>(ws + L.r)), c(reinterpret_cast<float*>(ws + L.c)),
        PQ(reinterpret_cast<float*>(ws + L.pq)), XA(reinterpret_cast<float*>(ws + L.xa)), U(ws + L.u),
        nstat(reinterpret_cast<float*>(ws + L.nstat)), R(F * N), D(D_), E(E_), ld(2 * D_), st(s) {
    a.X = XA; a.ldx = ld; a.PQ = PQ; a.A4 = A4; a.r = r; a.c = c;
    a.alive = alive; a.ldagg = ld;
    a.F = (int)F; a.N = (int)N; a.NP = (int)((N + 15) / 16 * 16); a.D = (int)D_; a.E = (int)E_;
  }
  // W1 = edge_mlp.0.weight [2E, 4D] folded into P | Q weights, A4, r, c (gamma / beta null: no pair norm)
  int prep(const void* W1, const float* b1, const float* gam, const float* bet) {
    hipLaunchKernelGGL((gnn_prep_kernel<DT>), dim3((unsigned)(2 * E)), dim3(256), 0, st, (const T*)W1, b1, gam, bet,
                       WPQ, A4, r, c, (int)D, (int)E);
    HCLSM_LAUNCH_CHECK();
    return 0;
  }
  int edges(bool msg, float* causal, float* edges_out) {
    int e = linear_rows(XA, ld, HCLSM_F32, WPQ, D, nullptr, nullptr, 0, PQ, 4 * E, HCLSM_F32, R, 4 * E, D, 0, 0,
                        nullptr, nullptr, a.eps, nullptr, 0, nullptr, 1, DT, st);
    if (e) return e;
    a.agg = msg ? XA + D : nullptr;
    a.causal = causal;
    a.edges = edges_out;
    if constexpr (DT != HCLSM_F32) {
      const int vec = D % 4 == 0 && ld % 4 == 0 && ((uintptr_t)XA & 15) == 0;
      hipLaunchKernelGGL(gnn_node_stats_kernel, dim3((unsigned)((R + 3) / 4)), dim3(256), 0, st, XA, ld, nstat, R,
                         (int)D, vec);
      HCLSM_LAUNCH_CHECK();
      e = launch_edges_resident<DT>(a, nstat, st);
      if (e != 1) return e;
    }
    return launch_edges<DT>(a, st);
  }
  // nodes += U2 ReLU(U1 [nodes; agg] + c1) + c2, in place in XA
  int update() {
    int e = linear_rows(XA, ld, HCLSM_F32, u1, 2 * D, c1, nullptr, 0, U, D, DT, R, D, 2 * D, 0, 1, nullptr, nullptr,
                        a.eps, nullptr, 0, nullptr, 1, DT, st);
    if (e) return e;
    return linear_rows(U, D, DT, u2, D, c2, XA, ld, XA, ld, HCLSM_F32, R, D, D, 0, 0, nullptr, nullptr, a.eps, nullptr,
                       0, nullptr, 1, DT, st);
  }
};

#define HCLSM_TRY(call) \
  do {                  \
    const int rc_ = (call); \
    if (rc_) return rc_;    \
  } while (0)

// params (module order): 0 pair_norm.w, 1 pair_norm.b, 2 edge_mlp.0.w, 3 edge_mlp.0.b, 4 edge_mlp.2.w,
// 5 edge_mlp.2.b, 6 edge_weight.w, 7 edge_weight.b, 8 msg_mlp.0.w, 9 msg_mlp.0.b, 10 update_mlp.0.w,
// 11 update_mlp.0.b, 12 update_mlp.2.w, 13 update_mlp.2.b, 14 causal_mlp.0.w, 15 causal_mlp.0.b,
// 16 causal_mlp.2.w, 17 causal_mlp.2.b
template <int DT>
static int gnn_forward(const float* nodes, const float* alive, float* nodes_out, float* causal, int64_t F, int64_t N,
                       int64_t D, int64_t E, int64_t rounds, int chunked, const void* const* p, float eps,
                       char* ws, const GnnWs& L, hipStream_t st) {
  auto Pf = [&](int i) { return reinterpret_cast<const float*>(p[i]); };
  GnnRun<DT> g(ws, L, F, N, D, E, alive, st);
  g.a.W2 = p[4]; g.a.b2 = Pf(5); g.a.we = Pf(6); g.a.be = Pf(7); g.a.Wm = p[8]; g.a.bm = Pf(9);
  g.a.C1 = p[14]; g.a.d1 = Pf(15); g.a.cc2 = Pf(16); g.a.d2 = Pf(17);
  g.a.eps = eps;
  g.a.norm = 1;
  g.u1 = p[10]; g.c1 = Pf(11); g.u2 = p[12]; g.c2 = Pf(13);
  HCLSM_TRY(g.prep(p[2], Pf(3), Pf(0), Pf(1)));
  HCLSM_TRY(copy_rows(nodes, D, nullptr, g.XA, g.ld, g.R, D, st));
  // Round structure (relation_graph.py:150-188): the all-pairs path (N <= 32) computes the edges of the
  // input nodes, recomputes them after a round only when rounds > 1, and takes the causal edges from the
  // last edges computed; the chunked path recomputes the edges every round and takes the causal edges
  // from the final nodes.  Both coincide except for rounds == 1.
  if (rounds == 0) {
    HCLSM_TRY(g.edges(false, causal, nullptr));
  } else {
    HCLSM_TRY(g.edges(true, rounds == 1 && !chunked ? causal : nullptr, nullptr));
    for (int64_t rd = 0; rd < rounds; ++rd) {
      HCLSM_TRY(g.update());
      if (rd + 1 < rounds) HCLSM_TRY(g.edges(true, nullptr, nullptr));
    }
    if (rounds > 1 || chunked) HCLSM_TRY(g.edges(false, causal, nullptr));
  }
  HCLSM_TRY(copy_rows(g.XA, g.ld, alive, nodes_out, D, g.R, D, st));
  return 0;
}

// gnn_message_pass (hclsm/kernels/gnn_message_pass.py:38-100): no pair norm, no causal head; every round
// computes the edges of the current nodes, the messages and the update, and the last round's edge features of
// the targets [ej0, ej0 + enj) are written out.  params: 0 edge_mlp.0.w [2E, 4D], 1 edge_mlp.0.b, 2 edge_mlp.2.w
// [E, 2E], 3 edge_mlp.2.b, 4 edge_weight.w [E], 5 edge_weight.b [1], 6 msg_mlp.0.w [D, E], 7 msg_mlp.0.b,
// 8 update_mlp.0.w [D, 2D], 9 update_mlp.0.b, 10 update_mlp.2.w [D, D], 11 update_mlp.2.b
template <int DT>
static int gnn_mp_forward(const float* nodes, const float* alive, float* nodes_out, float* edges_out, int64_t F,
                          int64_t N, int64_t D, int64_t E, int64_t rounds, int64_t ej0, int64_t enj,
                          const void* const* p, char* ws, const GnnWs& L, hipStream_t st) {
  auto Pf = [&](int i) { return reinterpret_cast<const float*>(p[i]); };
  GnnRun<DT> g(ws, L, F, N, D, E, alive, st);
  g.a.W2 = p[2]; g.a.b2 = Pf(3); g.a.we = Pf(4); g.a.be = Pf(5); g.a.Wm = p[6]; g.a.bm = Pf(7);
  g.a.norm = 0;
  g.a.ej0 = (int)ej0;
  g.a.enj = (int)enj;
  g.u1 = p[8]; g.c1 = Pf(9); g.u2 = p[10]; g.c2 = Pf(11);
  HCLSM_TRY(g.prep(p[0], Pf(1), nullptr, nullptr));
  HCLSM_TRY(copy_rows(nodes, D, nullptr, g.XA, g.ld, g.R, D, st));
  for (int64_t rd = 0; rd < rounds; ++rd) {
    HCLSM_TRY(g.edges(true, nullptr, rd + 1 == rounds && enj > 0 ? edges_out : nullptr));
    HCLSM_TRY(g.update());
  }
  HCLSM_TRY(copy_rows(g.XA, g.ld, alive, nodes_out, D, g.R, D, st));
  return 0;
}
#undef HCLSM_TRY

}  // namespace hclsm

using namespace hclsm;

// HCLSM_ERR_UNSUPPORTED for shapes outside the fused kernel: D, E multiples of 32, E <= 192, N <= 128
// (64 for fp32 operands), and the workgroup's LDS tiles within 160 KB.
static int gnn_check(int64_t N, int64_t D, int64_t E, int dtype) {
  if (N < 0 || D <= 0 || E <= 0) return HCLSM_ERR_SHAPE;
  if (dtype != HCLSM_F32 && dtype != HCLSM_BF16 && dtype != HCLSM_F16) return HCLSM_ERR_DTYPE;
  const int NW = dtype == HCLSM_F32 ? 4 : 8;
  if (D % 32 || E % 32 || E > 192 || N > 16 * NW) return HCLSM_ERR_UNSUPPORTED;
  const GnnArgs a = a0_shape(1, N, D, E);
  const bool fit = dtype == HCLSM_F32 ? edges_fit<HCLSM_F32>(a) : edges_fit<HCLSM_BF16>(a);
  return fit ? 0 : HCLSM_ERR_UNSUPPORTED;
}

extern "C" int64_t hclsm_relation_graph_workspace(int64_t frames, int64_t N, int64_t D, int64_t E, int dtype) {
  if (frames < 0) return HCLSM_ERR_SHAPE;
  const int c = gnn_check(N, D, E, dtype);
  if (c) return c;
  return (int64_t)gnn_ws(frames, N, D, E, dtype == HCLSM_F32 ? 4 : 2).total;
}

extern "C" int hclsm_relation_graph_forward(const float* nodes, const float* alive, float* nodes_out, float* causal,
                                            int64_t frames, int64_t N, int64_t D, int64_t E, int64_t rounds,
                                            int chunked, const void* const* params, float ln_eps, int dtype,
                                            void* workspace, int64_t workspace_bytes, void* stream) {
  if (frames < 0 || rounds < 0) return HCLSM_ERR_SHAPE;
  const int chk = gnn_check(N, D, E, dtype);
  if (chk) return chk;
  if (frames * N > 0x7fffffffLL) return HCLSM_ERR_SHAPE;
  if (frames == 0 || N == 0) return 0;
  if (!nodes || !nodes_out || !causal || !params || !workspace) return HCLSM_ERR_NULL;
  for (int i = 0; i < 18; ++i)
    if (!params[i]) return HCLSM_ERR_NULL;
  const int es = dtype == HCLSM_F32 ? 4 : 2;
  const GnnWs L = gnn_ws(frames, N, D, E, es);
  if (workspace_bytes < (int64_t)L.total) return HCLSM_ERR_SHAPE;
  char* ws = reinterpret_cast<char*>(workspace);
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case HCLSM_BF16:
      return gnn_forward<HCLSM_BF16>(nodes, alive, nodes_out, causal, frames, N, D, E, rounds, chunked, params, ln_eps,
                                     ws, L, st);
    case HCLSM_F16:
      return gnn_forward<HCLSM_F16>(nodes, alive, nodes_out, causal, frames, N, D, E, rounds, chunked, params, ln_eps,
                                    ws, L, st);
    default:
      return gnn_forward<HCLSM_F32>(nodes, alive, nodes_out, causal, frames, N, D, E, rounds, chunked, params, ln_eps,
                                    ws, L, st);
  }
}

// HCLSM_ERR_UNSUPPORTED outside the message-pass kernels: D, E multiples of 16 (fp32) or 32 (16-bit operands),
// E <= 192, N <= 64 (fp32) or 128, and the workgroup's LDS tiles within 160 KB.
static int gnn_mp_check(int64_t N, int64_t D, int64_t E, int dtype) {
  if (N < 0 || D <= 0 || E <= 0) return HCLSM_ERR_SHAPE;
  if (dtype != HCLSM_F32 && dtype != HCLSM_BF16 && dtype != HCLSM_F16) return HCLSM_ERR_DTYPE;
  const int NW = dtype == HCLSM_F32 ? 4 : 8, mult = dtype == HCLSM_F32 ? 16 : 32;
  if (D % mult || E % mult || E > 192 || N > 16 * NW) return HCLSM_ERR_UNSUPPORTED;
  const GnnArgs a = a0_shape(1, N, D, E);
  const bool fit = dtype == HCLSM_F32 ? edges_fit<HCLSM_F32>(a) : edges_fit<HCLSM_BF16>(a);
  return fit ? 0 : HCLSM_ERR_UNSUPPORTED;
}

extern "C" int64_t hclsm_gnn_message_pass_workspace(int64_t frames, int64_t N, int64_t D, int64_t E, int dtype) {
  if (frames < 0) return HCLSM_ERR_SHAPE;
  const int c = gnn_mp_check(N, D, E, dtype);
  if (c) return c;
  return (int64_t)gnn_ws(frames, N, D, E, dtype == HCLSM_F32 ? 4 : 2).total;
}

extern "C" int hclsm_gnn_message_pass(const float* nodes, const float* alive, float* nodes_out, float* edges_out,
                                      int64_t frames, int64_t N, int64_t D, int64_t E, int64_t rounds, int64_t ej0,
                                      int64_t enj, const void* const* params, int dtype, void* workspace,
                                      int64_t workspace_bytes, void* stream) {
  if (frames < 0 || rounds < 0 || ej0 < 0 || enj < 0 || ej0 + enj > N) return HCLSM_ERR_SHAPE;
  const int chk = gnn_mp_check(N, D, E, dtype);
  if (chk) return chk;
  if (frames * N > 0x7fffffffLL || frames * N * (enj > 0 ? enj : 1) * E > (1LL << 40)) return HCLSM_ERR_SHAPE;
  if (frames == 0 || N == 0) return 0;
  if (!nodes || !nodes_out || !params || !workspace || (enj > 0 && rounds > 0 && !edges_out)) return HCLSM_ERR_NULL;
  for (int i = 0; i < 12; ++i)
    if (!params[i]) return HCLSM_ERR_NULL;
  const GnnWs L = gnn_ws(frames, N, D, E, dtype == HCLSM_F32 ? 4 : 2);
  if (workspace_bytes < (int64_t)L.total) return HCLSM_ERR_SHAPE;
  char* ws = reinterpret_cast<char*>(workspace);
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case HCLSM_BF16:
      return gnn_mp_forward<HCLSM_BF16>(nodes, alive, nodes_out, edges_out, frames, N, D, E, rounds, ej0, enj, params,
                                        ws, L, st);
    case HCLSM_F16:
      return gnn_mp_forward<HCLSM_F16>(nodes, alive, nodes_out, edges_out, frames, N, D, E, rounds, ej0, enj, params,
                                       ws, L, st);
    default:
      return gnn_mp_forward<HCLSM_F32>(nodes, alive, nodes_out, edges_out, frames, N, D, E, rounds, ej0, enj, params,
                                       ws, L, st);
  }
}
