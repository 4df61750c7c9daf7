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
  int F, N, NP, D, E;  // NP = N rounded up to 16 (pairs of a padded i-row)
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
      sst[2 * row] = mu;
      sst[2 * row + 1] = 1.f / sqrtf(fmaxf(m2 - mu * mu, 0.f) + a.eps);
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
          sacc += __shfl_xor(sacc, 16, 64);
          sacc += __shfl_xor(sacc, 32, 64);
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
    const float w1 = A::tof(w[k]) * gam[k], w2 = A::tof(w[D + k]) * gam[D + k];
    const float w3 = A::tof(w[2 * D + k]) * gam[2 * D + k], w4 = A::tof(w[3 * D + k]) * gam[3 * D + k];
    WPQ[(size_t)o * D + k] = A::fromf(w1 + w3);
    WPQ[(size_t)(H1 + o) * D + k] = A::fromf(w2 - w3);
    A4[(size_t)o * D + k] = A::fromf(w4);
    sr += w1 + w2 + w3 + w4;
#pragma unroll
    for (int q = 0; q < 4; ++q) sc = fmaf(A::tof(w[q * D + k]), bet[q * D + k], sc);
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

// y[row * ldy + k] = x[row * ldx + k] * alive[row] for k < D (alive nullable).
__global__ void __launch_bounds__(256)
gnn_copy_rows_kernel(const float* __restrict__ x, int64_t ldx, const float* __restrict__ alive,
                     float* __restrict__ y, int64_t ldy, int64_t rows, int D) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= rows * D) return;
  const int64_t row = e / D, k = e - row * D;
  y[row * ldy + k] = x[row * ldx + k] * (alive ? alive[row] : 1.f);
}

struct GnnWs {
  size_t wpq, a4, r, c, pq, xa, u, total;
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
  static bool big_lds = false;   // allow more than the default 64 KB of dynamic LDS (idempotent)
  if (!big_lds) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gnn_edge_kernel<DT, NW, KC>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e != hipSuccess) return (int)e;
    big_lds = true;
  }
  const size_t lds = edge_lds<DT, NW, KC>(a);
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
  hipLaunchKernelGGL(gnn_copy_rows_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, ldx, alive, y, ldy,
                     rows, (int)D);
  HCLSM_LAUNCH_CHECK();
  return 0;
}

static GnnArgs a0_shape(int64_t F, int64_t N, int64_t D, int64_t E) {
  GnnArgs a{};
  a.F = (int)F; a.N = (int)N; a.NP = (int)((N + 15) / 16 * 16); a.D = (int)D; a.E = (int)E;
  return a;
}

// params (module order): 0 pair_norm.w, 1 pair_norm.b, 2 edge_mlp.0.w, 3 edge_mlp.0.b, 4 edge_mlp.2.w,
// 5 edge_mlp.2.b, 6 edge_weight.w, 7 edge_weight.b, 8 msg_mlp.0.w, 9 msg_mlp.0.b, 10 update_mlp.0.w,
// 11 update_mlp.0.b, 12 update_mlp.2.w, 13 update_mlp.2.b, 14 causal_mlp.0.w, 15 causal_mlp.0.b,
// 16 causal_mlp.2.w, 17 causal_mlp.2.b
template <int DT>
static int gnn_forward(const float* nodes, const float* alive, float* nodes_out, float* causal, int64_t F, int64_t N,
                       int64_t D, int64_t E, int64_t rounds, int chunked, const void* const* p, float eps,
                       char* ws, const GnnWs& L, hipStream_t st) {
  using T = typename MM<DT>::T;
  T* WPQ = reinterpret_cast<T*>(ws + L.wpq);
  T* A4 = reinterpret_cast<T*>(ws + L.a4);
  float* r = reinterpret_cast<float*>(ws + L.r);
  float* c = reinterpret_cast<float*>(ws + L.c);
  float* PQ = reinterpret_cast<float*>(ws + L.pq);
  float* XA = reinterpret_cast<float*>(ws + L.xa);   // [F*N, 2D]: nodes | messages
  void* U = ws + L.u;                                // [F*N, D] hidden layer of the node update
  const int64_t R = F * N, ld = 2 * D;
  auto P = [&](int i) { return p[i]; };
  auto Pf = [&](int i) { return reinterpret_cast<const float*>(p[i]); };
  int rc;
#define HCLSM_TRY(call) \
  do {                  \
    rc = (call);        \
    if (rc) return rc;  \
  } while (0)
  hipLaunchKernelGGL((gnn_prep_kernel<DT>), dim3((unsigned)(2 * E)), dim3(256), 0, st, (const T*)P(2), Pf(3), Pf(0),
                     Pf(1), WPQ, A4, r, c, (int)D, (int)E);
  HCLSM_LAUNCH_CHECK();
  HCLSM_TRY(copy_rows(nodes, D, nullptr, XA, ld, R, D, st));
  GnnArgs a{};
  a.X = XA; a.ldx = ld; a.PQ = PQ; a.A4 = A4; a.r = r; a.c = c;
  a.W2 = P(4); a.b2 = Pf(5); a.we = Pf(6); a.be = Pf(7); a.Wm = P(8); a.bm = Pf(9);
  a.C1 = P(14); a.d1 = Pf(15); a.cc2 = Pf(16); a.d2 = Pf(17);
  a.alive = alive; a.ldagg = ld;
  a.F = (int)F; a.N = (int)N; a.NP = (int)((N + 15) / 16 * 16); a.D = (int)D; a.E = (int)E; a.eps = eps;
  auto edges = [&](bool msg, bool caus) -> int {
    int e = linear_rows(XA, ld, HCLSM_F32, WPQ, D, nullptr, nullptr, 0, PQ, 4 * E, HCLSM_F32, R, 4 * E, D, 0, 0,
                        nullptr, nullptr, eps, nullptr, 0, nullptr, 1, DT, st);
    if (e) return e;
    a.agg = msg ? XA + D : nullptr;
    a.causal = caus ? causal : nullptr;
    return launch_edges<DT>(a, st);
  };
  auto update = [&]() -> int {   // nodes += U2 ReLU(U1 [nodes; agg] + c1) + c2, in place in XA
    int e = linear_rows(XA, ld, HCLSM_F32, P(10), 2 * D, Pf(11), nullptr, 0, U, D, DT, R, D, 2 * D, 0, 1, nullptr,
                        nullptr, eps, nullptr, 0, nullptr, 1, DT, st);
    if (e) return e;
    return linear_rows(U, D, DT, P(12), D, Pf(13), XA, ld, XA, ld, HCLSM_F32, R, D, D, 0, 0, nullptr, nullptr, eps,
                       nullptr, 0, nullptr, 1, DT, st);
  };
  // Round structure (relation_graph.py:150-188): the all-pairs path (N <= 32) computes the edges of the
  // input nodes, recomputes them after a round only when rounds > 1, and takes the causal edges from the
  // last edges computed; the chunked path recomputes the edges every round and takes the causal edges
  // from the final nodes.  Both coincide except for rounds == 1.
  if (rounds == 0) {
    HCLSM_TRY(edges(false, true));
  } else {
    HCLSM_TRY(edges(true, rounds == 1 && !chunked));
    for (int64_t rd = 0; rd < rounds; ++rd) {
      HCLSM_TRY(update());
      if (rd + 1 < rounds) HCLSM_TRY(edges(true, false));
    }
    if (rounds > 1 || chunked) HCLSM_TRY(edges(false, true));
  }
  HCLSM_TRY(copy_rows(XA, ld, alive, nodes_out, D, R, D, st));
#undef HCLSM_TRY
  return 0;
}

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
