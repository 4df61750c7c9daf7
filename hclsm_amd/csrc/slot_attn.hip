// Slot attention on gfx950: the attention core and the slot-attention iteration.
//
// Every dense contraction runs on v_mfma_f32_16x16x32_{bf16,f16} (fp32 inputs: 16x16x4 f32).
// The contraction dimension is walked in 32-wide blocks (lane group g = lane/16 takes
// elements 8g..8g+7 of a block, one 16-byte load per operand row).
//
// linear_kernel   one workgroup per 32x32 output tile, its 4 waves splitting the K blocks
//                 (block s goes to wave s % 4); partial tiles are summed through LDS, then
//                 the epilogue adds bias, ReLU, residual, clamp.  Optional LayerNorm
//                 prologue: row statistics from the same split (sums shifted by the row's
//                 first element), then normalised operands are formed on the fly.
// gru_kernel      the six gate products of torch.nn.GRUCell for a 32x16 tile of h', same
//                 split-K scheme, gates and (1-z) n + z h in the epilogue.
// core_logits     grid (frame, 64-token block): each wave forms a 16-token x N-slot logit
//                 tile, softmax over the slot axis in registers (two xor shuffles cover the
//                 four lane groups), writes attn and per-slot partial sums over its tokens.
// core_update     grid (frame, 64-column block of D): attn (A operand, row-major in HBM) times
//                 v staged transposed through LDS in 32-token chunks; optional
//                 renormalisation (attn + eps) / sum_m (attn + eps) folded into the epilogue.
#include <mutex>

#include "mfma.h"
#include "internal.h"

namespace hclsm {

template <typename T> struct Cvt;
template <> struct Cvt<float> { static __device__ __forceinline__ float f(float v) { return v; } };
template <> struct Cvt<uint16_t> { static __device__ __forceinline__ float f(uint16_t v) { return bf16_bits_to_f32(v); } };
template <> struct Cvt<_Float16> { static __device__ __forceinline__ float f(_Float16 v) { return (float)v; } };

// Eight consecutive elements as floats with 16-byte loads (p 16-byte aligned for 16-bit XT, 32-byte for float).
template <typename XT>
__device__ __forceinline__ void load8f(const XT* p, float* o) {
  if constexpr (std::is_same_v<XT, float>) {
    const float4 u = reinterpret_cast<const float4*>(p)[0], v = reinterpret_cast<const float4*>(p)[1];
    o[0] = u.x; o[1] = u.y; o[2] = u.z; o[3] = u.w; o[4] = v.x; o[5] = v.y; o[6] = v.z; o[7] = v.w;
  } else {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    const XT* e = reinterpret_cast<const XT*>(&u);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = Cvt<XT>::f(e[i]);
  }
}

// Operand of one 32-wide K block for this lane (8 elements at k0 + 8g), converted to DT.
template <int DT, typename XT>
__device__ __forceinline__ typename MM<DT>::Op load_op(const XT* p) {
  using A = MM<DT>;
  if constexpr (std::is_same_v<XT, typename A::T>) {
    return A::load(p);
  } else {
    if constexpr (A::KPL == 8) {
      typename A::T e[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) e[i] = A::fromf(Cvt<XT>::f(p[i]));
      return __builtin_bit_cast(typename A::Op, *reinterpret_cast<uint4*>(e));
    } else {
      return Cvt<XT>::f(p[0]);
    }
  }
}

// LayerNorm-transformed operand: (x - mean) * rstd * w + b, converted to DT.
template <int DT, typename XT>
__device__ __forceinline__ typename MM<DT>::Op load_op_ln(const XT* p, int k, float mean, float rstd,
                                                          const float* __restrict__ w, const float* __restrict__ b) {
  using A = MM<DT>;
  constexpr int KPL = A::KPL;
  float x[KPL];
#pragma unroll
  for (int i = 0; i < KPL; ++i) {
    float t = (Cvt<XT>::f(p[i]) - mean) * rstd;
    if (w) t *= w[k + i];
    if (b) t += b[k + i];
    x[i] = t;
  }
  if constexpr (KPL == 8) {
    typename A::T e[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) e[i] = A::fromf(x[i]);
    return __builtin_bit_cast(typename A::Op, *reinterpret_cast<uint4*>(e));
  } else {
    return x[0];
  }
}

// Row statistics for the LayerNorm prologue: rows r0 + li and r0 + 16 + li, this wave's K blocks,
// reduced across lane groups and the 4 waves through LDS.  Uses sums of (x - c) with c = row's x[0].
template <typename XT, int KPL>
__device__ __forceinline__ void ln_stats(const XT* const pa[2], int64_t K, int wid, int g, int li, float eps,
                                         float* lds, float mean[2], float rstd[2]) {
  const int BLK = 4 * KPL;
  const int nblk = (int)(K / BLK);
  float s1[2] = {0.f, 0.f}, s2[2] = {0.f, 0.f};
  float c[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) c[t] = Cvt<XT>::f(pa[t][-(int64_t)(KPL * g)]);  // x[row][0]
  for (int s = wid; s < nblk; s += 4) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int i = 0; i < KPL; ++i) {
        const float d = Cvt<XT>::f(pa[t][(int64_t)s * BLK + i]) - c[t];
        s1[t] += d;
        s2[t] += d * d;
      }
  }
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    s1[t] = rows4_sum(s1[t]);
    s2[t] = rows4_sum(s2[t]);
  }
  // lds layout: [wave][row 0..31][2]
  if (g == 0) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      lds[(wid * 32 + 16 * t + li) * 2 + 0] = s1[t];
      lds[(wid * 32 + 16 * t + li) * 2 + 1] = s2[t];
    }
  }
  __syncthreads();
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    float a1 = 0.f, a2 = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      a1 += lds[(w * 32 + 16 * t + li) * 2 + 0];
      a2 += lds[(w * 32 + 16 * t + li) * 2 + 1];
    }
    const float m1 = a1 / (float)K;
    const float var = fmaxf(a2 / (float)K - m1 * m1, 0.f);
    mean[t] = c[t] + m1;
    rstd[t] = 1.f / sqrtf(var + eps);
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------
// Optional split of a linear layer's output: columns >= col go, transposed per frame of
// frame_rows rows, to yt[frame][col - split][row % frame_rows] (row stride ldyt, frame stride
// bstride) instead of Y.  Used to emit v^T next to k from one [W_k; W_v] projection.
struct OutSplit {
  int64_t col, frame_rows, ldyt, bstride;
  void* yt;
};

// Optional extras of a linear layer:
// - a device-side row count: rows = min(M, *m_dev * m_mul), read at kernel start, so a launch sized
//   for a capacity does only the rows a preceding kernel produced (workgroups past them exit);
// - a gated-linear epilogue: val = silu(glu[row, col]) * val (glu in the operand type), applied after
//   bias / ReLU and before the residual.
// - LayerNorm statistics of the output rows (linear_dma_kernel, fp32 output): pst[row * N / 64 + b] = (mean, centred
//   sum of squares) of the row's 64 columns 64 b .. 64 b + 63;
// - a LayerNorm folded into the weights (linear_lds_kernel, linear_lds128_kernel): with W = W0 diag(gamma),
//   fsum[j] = sum of row j of W and fbias[j] = (W0 beta)[j] + b[j], the output is rstd (acc - mean fsum[j]) + fbias[j]
//   with the row's mean and rstd combined from fparts such 64-column partials fst[row * fparts ..] (eps feps); for
//   a (w1, w3) pair fsum and fbias hold the w1 columns, then the w3 columns.
struct LinExt {
  const int32_t* m_dev;
  int64_t m_mul;
  const void* glu;
  int64_t ldg;
  const void* w3;   // paired gated-linear GEMM (LDS kernels): see w_row
  float2* pst = nullptr;
  const float2* fst = nullptr;
  int64_t fparts = 0;
  const float* fsum = nullptr;
  const float* fbias = nullptr;
  float feps = 0.f;
};
constexpr LinExt kNoLinExt{nullptr, 1, nullptr, 0, nullptr};

// (mean, rstd) of a row from its 64-column partials (mean_p, M2_p), parts <= FOLD_MAX_PARTS: every partial requested
// at once, then M2 = sum M2_p + 64 sum (mean_p - mean)^2.
__device__ __forceinline__ float2 fold_row_stats(const float2* __restrict__ p, int64_t parts, float eps) {
  // two rounds of at most 8 requests (8 partials in registers at a time); the partial means enter shifted by the
  // first, sum (m_p - m_0) and sum (m_p - m_0)^2, so that an offset of the row's values cancels exactly
  float m0 = 0.f, s1 = 0.f, s2 = 0.f, m2 = 0.f;
#pragma unroll
  for (int h = 0; h < FOLD_MAX_PARTS; h += 8) {
    if (h >= parts) break;
    float2 v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = h + i < parts ? p[h + i] : make_float2(0.f, 0.f);
    if (h == 0) m0 = v[0].x;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float dv = h + i < parts ? v[i].x - m0 : 0.f;
      s1 += dv;
      s2 += dv * dv;
      m2 += v[i].y;
    }
  }
  const float inv = __builtin_amdgcn_rcpf((float)parts);
  const float d = s1 * inv;   // mean - m_0
  m2 += 64.f * fmaxf(s2 - s1 * d, 0.f);
  return make_float2(m0 + d, rsqrtf(m2 * (inv * (1.f / 64.f)) + eps));
}

// Prologue of a folded-LayerNorm consumer (ROWS x 128 or 64 x 64 tile): threads 0 .. ROWS-1 form the (mean, rstd) of
// the tile's rows, threads ROWS .. ROWS+COLS-1 stage fsum / fbias of its COLS weight columns (jc of column c).
template <int ROWS, int COLS>
__device__ __forceinline__ void fold_prologue(const LinExt& e, int tid, int64_t row0, int64_t M, int64_t col0,
                                              int64_t N, float2 (&rst)[ROWS], float2 (&cst)[COLS]) {
  if (tid < ROWS) {
    const int64_t row = row0 + tid < M ? row0 + tid : M - 1;
    rst[tid] = fold_row_stats(e.fst + row * e.fparts, e.fparts, e.feps);
  } else if (tid < ROWS + COLS) {
    const int c = tid - ROWS;
    const int64_t col = col0 + c;
    if (col < N) {
      const int64_t jc = e.w3 == nullptr ? col : (col >> 5) * 16 + (col & 15) + ((col & 16) ? N / 2 : 0);
      cst[c] = make_float2(e.fsum[jc], e.fbias[jc]);
    }
  }
}

// The folded LayerNorm on one accumulator of columns c .. c + 3 of the tile (cst) and row statistics st.
__device__ __forceinline__ void fold_acc4(f32x4& acc, float2 st, const float2* cst) {
#pragma unroll
  for (int r = 0; r < 4; ++r) acc[r] = st.y * (acc[r] - st.x * cst[r].x) + cst[r].y;
}

// Weight row of GEMM column j.  With e.w3 set (LDS kernels) the GEMM is 2H columns wide and its 16-column tiles alternate
// between W (= w1) and e.w3: column j is row 16 (j / 32) + j % 16 of w1 for j % 32 < 16, of w3 otherwise.  A
// wave's tile pair (2u, 2u + 1) then holds h1 and h3 of the same 16 outputs, and the epilogue writes
// silu(h1) * h3 to output columns 16u .. 16u + 15 (SwiGLU without h1 ever leaving the registers).
template <typename T>
__device__ __forceinline__ const T* w_row(const T* W, const LinExt& e, int64_t j, int64_t ldw) {
  if (e.w3 == nullptr) return W + j * ldw;
  const int64_t r = ((j >> 5) << 4) + (j & 15);
  return ((j & 16) ? reinterpret_cast<const T*>(e.w3) : W) + r * ldw;
}

// Epilogue of a (w1, w3) tile pair: four consecutive outputs col .. col+3 of one row, col a multiple of 4 in
// the H-wide output.
template <int DT, int OT>
__device__ __forceinline__ void glu_pair_epilogue(const f32x4& h1, const f32x4& h3, int64_t row, int64_t col,
                                                  int64_t H, const float* resid, int64_t ldr,
                                                  typename MM<OT>::T* Y, int64_t ldy, typename MM<DT>::T* Y2,
                                                  int64_t ldy2, bool vec);

__device__ __forceinline__ int64_t ext_rows(const LinExt& e, int64_t M) {
  if (e.m_dev == nullptr) return M;
  const int64_t md = (int64_t)(*e.m_dev) * e.m_mul;
  return md < M ? md : M;
}
template <int DT>
__device__ __forceinline__ float ext_glu(const LinExt& e, int64_t row, int64_t col, float val) {
  if (e.glu == nullptr) return val;
  return silu_f(Cvt<typename MM<DT>::T>::f(reinterpret_cast<const typename MM<DT>::T*>(e.glu)[row * e.ldg + col])) * val;
}

// 64x64 output tile per workgroup, each wave a 32x32 quadrant over the full K (large M x N).
// 64x64 output tile per workgroup, 16-bit operands: the tile's A rows and W rows are staged in LDS in
// K chunks of 128 (each global byte read once per workgroup), the next chunk's global loads in flight
// while the current chunk is multiplied; each wave computes a 32x32 quadrant from LDS.  34 KB of LDS,
// so several workgroups share a CU.
// Workgroup -> tile order that keeps consecutive tiles (which share rows of X) on one XCD: the dispatcher
// deals workgroups to the 8 XCDs in turn, so XCD x receives blocks x, x + 8, ...; they take the x-th contiguous
// share of the tiles (the first G % 8 XCDs one tile more).
__device__ __forceinline__ int64_t xcd_tile(int64_t bid, int64_t G) {
  constexpr int64_t NX = 8;
  const int64_t x = bid % NX, k = bid / NX, per = G / NX, r = G % NX;
  return x * per + (x < r ? x : r) + k;
}

// Workgroup -> tile order for a launch whose live tiles are the leading ones (a device-side row count): row
// block b of the tiles (tiles_n tiles sharing 128 or 64 rows of X) goes to XCD b % 8, in groups of eight row
// blocks, so the tiles that read the same rows of X meet in one L2 and the leading row blocks still spread
// over all XCDs.  Taken for narrow outputs (tiles_n <= 8: measured faster on the Level-1 N = 384 layers); wider
// ones, and the last, partial group, keep the identity order (the wide SwiGLU layer measured slower with it).
__device__ __forceinline__ int64_t xcd_rowblock_tile(int64_t bid, int64_t tiles_n, int64_t G) {
  constexpr int64_t NX = 8;
  const int64_t grp = NX * tiles_n;
  if (tiles_n > 8 || bid >= G / grp * grp) return bid;
  const int64_t x = bid % NX, k = bid / NX;
  return (k / tiles_n) * grp + x * tiles_n + k % tiles_n;
}

// Epilogue of four consecutive output columns col .. col+3 of one row (columns past N skipped):
// val = acc + bias, ReLU, gated-linear factor, + resid, clamp; stored to Y (and Y2).  With vec, every
// row of Y / Y2 / resid / glu starts 16-byte aligned and the four columns are in range: one vector access each.
template <int DT, int OT>
__device__ __forceinline__ bool lin_vec4_ok(const void* Y, int64_t ldy, const void* Y2, int64_t ldy2,
                                            const float* resid, int64_t ldr, const LinExt& e) {
  auto al = [](const void* p, int64_t ld, int es) {
    return p == nullptr || ((((uintptr_t)p) & 15) == 0 && (ld * es) % 16 == 0);
  };
  return al(Y, ldy, (int)sizeof(typename MM<OT>::T)) && al(Y2, ldy2, (int)sizeof(typename MM<DT>::T)) &&
         al(resid, ldr, 4) && al(e.glu, e.ldg, (int)sizeof(typename MM<DT>::T));
}

// acc is left holding the values stored (before their rounding to the output type).
template <int DT, int OT>
__device__ __forceinline__ void lin_epilogue4(f32x4& acc, const float (&bv)[4], int64_t row, int64_t col,
                                              int64_t N, int relu, float clamp_v, const float* __restrict__ resid,
                                              int64_t ldr, typename MM<OT>::T* __restrict__ Y, int64_t ldy,
                                              typename MM<DT>::T* __restrict__ Y2, int64_t ldy2, const LinExt& e,
                                              bool vec) {
  using TD = typename MM<DT>::T;
  using TO = typename MM<OT>::T;
  float v[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    v[r] = acc[r] + bv[r];
    if (relu) v[r] = fmaxf(v[r], 0.f);
  }
  if (vec && col + 3 < N) {
    if (e.glu) {
      TD gv[4];
      const TD* gp = reinterpret_cast<const TD*>(e.glu) + row * e.ldg + col;
      if constexpr (sizeof(TD) == 4) *reinterpret_cast<float4*>(gv) = *reinterpret_cast<const float4*>(gp);
      else *reinterpret_cast<uint2*>(gv) = *reinterpret_cast<const uint2*>(gp);
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = silu_f(Cvt<TD>::f(gv[r])) * v[r];
    }
    if (resid) {
      const float4 rv = *reinterpret_cast<const float4*>(resid + row * ldr + col);
      v[0] += rv.x; v[1] += rv.y; v[2] += rv.z; v[3] += rv.w;
    }
    if (clamp_v > 0.f) {
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = fminf(fmaxf(v[r], -clamp_v), clamp_v);
    }
    TO o[4] = {MM<OT>::fromf(v[0]), MM<OT>::fromf(v[1]), MM<OT>::fromf(v[2]), MM<OT>::fromf(v[3])};
    if constexpr (sizeof(TO) == 4) *reinterpret_cast<float4*>(Y + row * ldy + col) = *reinterpret_cast<float4*>(o);
    else *reinterpret_cast<uint2*>(Y + row * ldy + col) = *reinterpret_cast<uint2*>(o);
    if (Y2) {
      TD o2[4] = {MM<DT>::fromf(v[0]), MM<DT>::fromf(v[1]), MM<DT>::fromf(v[2]), MM<DT>::fromf(v[3])};
      if constexpr (sizeof(TD) == 4) *reinterpret_cast<float4*>(Y2 + row * ldy2 + col) = *reinterpret_cast<float4*>(o2);
      else *reinterpret_cast<uint2*>(Y2 + row * ldy2 + col) = *reinterpret_cast<uint2*>(o2);
    }
    acc = f32x4{v[0], v[1], v[2], v[3]};
    return;
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    if (col + r >= N) break;
    float val = ext_glu<DT>(e, row, col + r, v[r]);
    if (resid) val += resid[row * ldr + col + r];
    if (clamp_v > 0.f) val = fminf(fmaxf(val, -clamp_v), clamp_v);
    Y[row * ldy + col + r] = MM<OT>::fromf(val);
    if (Y2) Y2[row * ldy2 + col + r] = MM<DT>::fromf(val);
    acc[r] = val;
  }
}

template <int DT, int OT>
__device__ __forceinline__ void glu_pair_epilogue(const f32x4& h1, const f32x4& h3, int64_t row, int64_t col,
                                                  int64_t H, const float* resid, int64_t ldr,
                                                  typename MM<OT>::T* Y, int64_t ldy, typename MM<DT>::T* Y2,
                                                  int64_t ldy2, bool vec) {
  f32x4 v;
#pragma unroll
  for (int r = 0; r < 4; ++r) v[r] = silu_f(h1[r]) * h3[r];
  const float zero[4] = {0.f, 0.f, 0.f, 0.f};
  lin_epilogue4<DT, OT>(v, zero, row, col, H, 0, 0.f, resid, ldr, Y, ldy, Y2, ldy2, kNoLinExt, vec);
}

// One 16-byte LDS unit (8 operand elements) of the A operand: loaded as is for 16-bit X, or as 8 fp32 values
// rounded to the operand type when it is stored (fp32 X).
template <int DT, typename XT>
struct AUnit {
  uint4 v;
  __device__ __forceinline__ void load(const XT* p) { v = *reinterpret_cast<const uint4*>(p); }
  __device__ __forceinline__ void zero() { v = make_uint4(0u, 0u, 0u, 0u); }
  __device__ __forceinline__ uint4 get() const { return v; }
};
template <int DT>
struct AUnit<DT, float> {
  float4 lo, hi;
  __device__ __forceinline__ void load(const float* p) {
    lo = *reinterpret_cast<const float4*>(p);
    hi = *reinterpret_cast<const float4*>(p + 4);
  }
  __device__ __forceinline__ void zero() { lo = hi = make_float4(0.f, 0.f, 0.f, 0.f); }
  __device__ __forceinline__ uint4 get() const {
    using A = MM<DT>;
    typename A::T e[8] = {A::fromf(lo.x), A::fromf(lo.y), A::fromf(lo.z), A::fromf(lo.w),
                          A::fromf(hi.x), A::fromf(hi.y), A::fromf(hi.z), A::fromf(hi.w)};
    return *reinterpret_cast<const uint4*>(e);
  }
};

constexpr int LT_KC = 128;

// KC: the K chunk staged per round (128, or 64 for half the LDS: twice the workgroups resident per CU)
template <int DT, int OT, typename XT = typename MM<DT>::T, bool FOLD = false, int KC = LT_KC>
__global__ void __launch_bounds__(256)
linear_lds_kernel(const XT* __restrict__ X, int64_t ldx, const typename MM<DT>::T* __restrict__ W,
                  int64_t ldw, const float* __restrict__ bias, const float* __restrict__ resid, int64_t ldr,
                  typename MM<OT>::T* __restrict__ Y, int64_t ldy, typename MM<DT>::T* __restrict__ Y2,
                  int64_t ldy2, int64_t M, int64_t N, int64_t K, int relu, float clamp_v, OutSplit os, LinExt ext) {
  using A = MM<DT>;
  using T = typename A::T;
  static_assert(A::KPL == 8, "16-bit operands");
  static_assert(KC == 64 || KC == 128, "K chunk");
  constexpr int LT_LD = KC + 8;      // LDS row pitch (elements): spreads the 16 rows of an operand over banks
  constexpr int UPR = KC / 8;        // 16-byte units per row of a chunk
  constexpr int NU = 64 * UPR / 256; // units per thread and operand
  __shared__ __align__(16) T As[64 * LT_LD];
  __shared__ __align__(16) T Bs[64 * LT_LD];
  const int64_t tiles_n = (N + 63) / 64;
  // (a device-side row count leaves only the leading tiles live: keep them spread over the XCDs)
  const int64_t tile = ext.m_dev ? xcd_rowblock_tile(blockIdx.x, tiles_n, gridDim.x) : xcd_tile(blockIdx.x, gridDim.x);
  const int64_t tm = tile / tiles_n, tn = tile - tm * tiles_n;
  M = ext_rows(ext, M);
  if (tm * 64 >= M) return;   // the whole workgroup, before any barrier
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63, g = lane >> 4, li = lane & 15;
  const int wr = wid >> 1, wc = wid & 1;
  // staging map: 64 rows x (KC / 8) 16-byte units per operand, NU per thread
  const XT* pa[NU];
  const T* pb[NU];
  int soff[NU], ucol[NU];
#pragma unroll
  for (int i = 0; i < NU; ++i) {
    const int u = tid + 256 * i, r = u / UPR;
    ucol[i] = (u % UPR) * 8;
    int64_t ra = tm * 64 + r, rb = tn * 64 + r;
    ra = ra < M ? ra : M - 1;
    rb = rb < N ? rb : N - 1;
    pa[i] = X + ra * ldx + ucol[i];
    pb[i] = w_row(W, ext, rb, ldw) + ucol[i];
    soff[i] = r * LT_LD + ucol[i];
  }
  AUnit<DT, XT> ra_[NU];
  uint4 rb_[NU];
  auto fetch = [&](int64_t k0, int kc) {
#pragma unroll
    for (int i = 0; i < NU; ++i) {
      const bool in = ucol[i] < kc;
      if (in) ra_[i].load(pa[i] + k0);
      else ra_[i].zero();
      rb_[i] = in ? *reinterpret_cast<const uint4*>(pb[i] + k0) : make_uint4(0u, 0u, 0u, 0u);
    }
  };
  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  fetch(0, (int)(K < KC ? K : KC));
  // FOLD: (mean, rstd) of the tile's rows and (fsum, fbias) of its columns, read after the loop's barriers
  __shared__ float2 rst[FOLD ? 64 : 1], cst[FOLD ? 64 : 1];
  if constexpr (FOLD) fold_prologue<64, 64>(ext, tid, tm * 64, M, tn * 64, N, rst, cst);
  for (int64_t k0 = 0; k0 < K; k0 += KC) {
    const int kc = (int)(K - k0 < KC ? K - k0 : KC);
    __syncthreads();   // the previous chunk is consumed
#pragma unroll
    for (int i = 0; i < NU; ++i) {
      *reinterpret_cast<uint4*>(As + soff[i]) = ra_[i].get();
      *reinterpret_cast<uint4*>(Bs + soff[i]) = rb_[i];
    }
    __syncthreads();
    if (k0 + KC < K) fetch(k0 + KC, (int)(K - k0 - KC < KC ? K - k0 - KC : KC));
    for (int s = 0; s < kc / 32; ++s) {
      const typename A::Op a0 = A::load(As + (wr * 32 + li) * LT_LD + s * 32 + 8 * g);
      const typename A::Op a1 = A::load(As + (wr * 32 + 16 + li) * LT_LD + s * 32 + 8 * g);
      const typename A::Op b0 = A::load(Bs + (wc * 32 + li) * LT_LD + s * 32 + 8 * g);
      const typename A::Op b1 = A::load(Bs + (wc * 32 + 16 + li) * LT_LD + s * 32 + 8 * g);
      // weights as the A operand: acc[ti][tj][r] = out[row 16 ti + li][col 16 tj + 4g + r]
      acc[0][0] = A::mfma(b0, a0, acc[0][0]);
      acc[0][1] = A::mfma(b1, a0, acc[0][1]);
      acc[1][0] = A::mfma(b0, a1, acc[1][0]);
      acc[1][1] = A::mfma(b1, a1, acc[1][1]);
    }
  }
  const int64_t r0 = tm * 64 + 32 * wr, c0 = tn * 64 + 32 * wc;
  if constexpr (FOLD) {   // folded LayerNorm (host: no output split, N a multiple of 4)
#pragma unroll
    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
      for (int tj = 0; tj < 2; ++tj)
        fold_acc4(acc[ti][tj], rst[32 * wr + 16 * ti + li], cst + 32 * wc + 16 * tj + 4 * g);
  }
  if (os.yt != nullptr && Y2 == nullptr && os.col % 64 == 0 && tn * 64 >= os.col) {
    // a tile of the transposed half: transpose through LDS so that consecutive threads write
    // consecutive rows (tokens) of yt
    constexpr int TP = 66;   // pitch of the transposed tile (elements)
    static_assert(64 * TP <= 64 * LT_LD, "the transposed tile fits As");
    T* Ts = As;
    __syncthreads();   // the last chunk is consumed
#pragma unroll
    for (int tj = 0; tj < 2; ++tj)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t col = c0 + 16 * tj + 4 * g + r;
        const float bv = (bias && col < N) ? bias[col] : 0.f;
#pragma unroll
        for (int ti = 0; ti < 2; ++ti) {
          const int64_t row = r0 + 16 * ti + li;
          float val = acc[ti][tj][r] + bv;
          if (relu) val = fmaxf(val, 0.f);
          if (resid && row < M && col < N) val += resid[row * ldr + col];
          if (clamp_v > 0.f) val = fminf(fmaxf(val, -clamp_v), clamp_v);
          Ts[(32 * wc + 16 * tj + 4 * g + r) * TP + 32 * wr + 16 * ti + li] = MM<OT>::fromf(val);
        }
      }
    __syncthreads();
    typename MM<OT>::T* yt = reinterpret_cast<typename MM<OT>::T*>(os.yt);
    for (int i = tid; i < 64 * 64; i += 256) {
      const int c = i >> 6, rl = i & 63;
      const int64_t row = tm * 64 + rl, col = tn * 64 + c;
      if (row < M && col < N) {
        const int64_t fr = row / os.frame_rows, rr = row - fr * os.frame_rows;
        yt[fr * os.bstride + (col - os.col) * os.ldyt + rr] = Ts[c * TP + rl];
      }
    }
    return;
  }
  if (ext.w3 != nullptr) {   // (w1, w3) tile pair: the wave's two column tiles (c0 a multiple of 32)
    const int64_t H = N / 2, col = c0 / 2 + 4 * g;
    const bool v4 = lin_vec4_ok<DT, OT>(Y, ldy, Y2, ldy2, resid, ldr, kNoLinExt);
#pragma unroll
    for (int ti = 0; ti < 2; ++ti) {
      const int64_t row = r0 + 16 * ti + li;
      if (row < M && col < H)
        glu_pair_epilogue<DT, OT>(acc[ti][0], acc[ti][1], row, col, H, resid, ldr, Y, ldy, Y2, ldy2, v4);
    }
    return;
  }
  const bool vec = os.yt == nullptr && lin_vec4_ok<DT, OT>(Y, ldy, Y2, ldy2, resid, ldr, ext);
#pragma unroll
  for (int tj = 0; tj < 2; ++tj) {
    const int64_t col = c0 + 16 * tj + 4 * g;
    float bv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) bv[r] = (bias && col + r < N) ? bias[col + r] : 0.f;
#pragma unroll
    for (int ti = 0; ti < 2; ++ti) {
      const int64_t row = r0 + 16 * ti + li;
      if (row >= M || col >= N) continue;
      if (os.yt == nullptr) {
        lin_epilogue4<DT, OT>(acc[ti][tj], bv, row, col, N, relu, clamp_v, resid, ldr, Y, ldy, Y2, ldy2, ext, vec);
        continue;
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t cr = col + r;
        if (cr >= N) break;
        float val = acc[ti][tj][r] + bv[r];
        if (relu) val = fmaxf(val, 0.f);
        val = ext_glu<DT>(ext, row, cr, val);
        if (resid) val += resid[row * ldr + cr];
        if (clamp_v > 0.f) val = fminf(fmaxf(val, -clamp_v), clamp_v);
        if (cr >= os.col) {
          const int64_t fr = row / os.frame_rows, rr = row - fr * os.frame_rows;
          reinterpret_cast<typename MM<OT>::T*>(os.yt)[fr * os.bstride + (cr - os.col) * os.ldyt + rr] =
              MM<OT>::fromf(val);
        } else {
          Y[row * ldy + cr] = MM<OT>::fromf(val);
        }
        if (Y2) Y2[row * ldy2 + cr] = A::fromf(val);
      }
    }
  }
}

// 128x128 output tile per workgroup, 16-bit operands, for wide layers (N >= 768) with many rows: the tile's
// A and W rows staged in LDS in K chunks of 64 (next chunk's global loads in flight), each wave a 64x64
// quadrant (4 x 4 MFMA tiles), so every LDS fragment feeds four MFMAs and each staged byte eight times the
// FLOPs of the 64x64 tile.  37 KB of LDS.
constexpr int LB_KC = 64;
constexpr int LB_LD = LB_KC + 8;   // pitch 144 B: the 16 rows of a fragment read hit distinct banks

template <int DT, int OT, typename XT = typename MM<DT>::T, bool FOLD = false>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(FOLD ? 3 : 1)))
// (FOLD: three waves per SIMD, as the plain form has; the folded epilogue would otherwise take two)
linear_lds128_kernel(const XT* __restrict__ X, int64_t ldx, const typename MM<DT>::T* __restrict__ W,
                     int64_t ldw, const float* __restrict__ bias, const float* __restrict__ resid, int64_t ldr,
                     typename MM<OT>::T* __restrict__ Y, int64_t ldy, typename MM<DT>::T* __restrict__ Y2,
                     int64_t ldy2, int64_t M, int64_t N, int64_t K, int relu, float clamp_v, LinExt ext) {
  using A = MM<DT>;
  using T = typename A::T;
  static_assert(A::KPL == 8, "16-bit operands");
  __shared__ __align__(16) T As[128 * LB_LD];
  __shared__ __align__(16) T Bs[128 * LB_LD];
  const int64_t tiles_n = (N + 127) / 128;
  // (a device-side row count leaves only the leading tiles live: keep them spread over the XCDs)
  const int64_t tile = ext.m_dev ? xcd_rowblock_tile(blockIdx.x, tiles_n, gridDim.x) : xcd_tile(blockIdx.x, gridDim.x);
  const int64_t tm = tile / tiles_n, tn = tile - tm * tiles_n;
  M = ext_rows(ext, M);
  if (tm * 128 >= M) return;   // the whole workgroup, before any barrier
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63, g = lane >> 4, li = lane & 15;
  const int wr = wid >> 1, wc = wid & 1;
  // staging map: 128 rows x (KC / 8) 16-byte units = 1024 units per operand, 4 per thread
  const XT* pa[4];
  const T* pb[4];
  int soff[4], ucol[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int u = tid + 256 * i, r = u >> 3;
    ucol[i] = (u & 7) * 8;
    int64_t ra = tm * 128 + r, rb = tn * 128 + r;
    ra = ra < M ? ra : M - 1;
    rb = rb < N ? rb : N - 1;
    pa[i] = X + ra * ldx + ucol[i];
    pb[i] = w_row(W, ext, rb, ldw) + ucol[i];
    soff[i] = r * LB_LD + ucol[i];
  }
  AUnit<DT, XT> ra_[4];
  uint4 rb_[4];
  auto fetch = [&](int64_t k0, int kc) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool in = ucol[i] < kc;
      if (in) ra_[i].load(pa[i] + k0);
      else ra_[i].zero();
      rb_[i] = in ? *reinterpret_cast<const uint4*>(pb[i] + k0) : make_uint4(0u, 0u, 0u, 0u);
    }
  };
  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  fetch(0, (int)(K < LB_KC ? K : LB_KC));
  // FOLD: (mean, rstd) of the tile's rows and (fsum, fbias) of its columns, read after the loop's barriers
  __shared__ float2 rst[FOLD ? 128 : 1], cst[FOLD ? 128 : 1];
  if constexpr (FOLD) fold_prologue<128, 128>(ext, tid, tm * 128, M, tn * 128, N, rst, cst);
  for (int64_t k0 = 0; k0 < K; k0 += LB_KC) {
    const int kc = (int)(K - k0 < LB_KC ? K - k0 : LB_KC);
    __syncthreads();   // the previous chunk is consumed
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *reinterpret_cast<uint4*>(As + soff[i]) = ra_[i].get();
      *reinterpret_cast<uint4*>(Bs + soff[i]) = rb_[i];
    }
    __syncthreads();
    if (k0 + LB_KC < K) fetch(k0 + LB_KC, (int)(K - k0 - LB_KC < LB_KC ? K - k0 - LB_KC : LB_KC));
    for (int s = 0; s < kc / 32; ++s) {
      typename A::Op a[4], b[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        a[t] = A::load(As + (wr * 64 + 16 * t + li) * LB_LD + s * 32 + 8 * g);
        b[t] = A::load(Bs + (wc * 64 + 16 * t + li) * LB_LD + s * 32 + 8 * g);
      }
      // weights as the A operand: acc[ti][tj][r] = out[row 16 ti + li][col 16 tj + 4g + r], so a lane's four
      // values are consecutive columns of one row (vector epilogue)
#pragma unroll
      for (int ti = 0; ti < 4; ++ti)
#pragma unroll
        for (int tj = 0; tj < 4; ++tj) acc[ti][tj] = A::mfma(b[tj], a[ti], acc[ti][tj]);
    }
  }
  const int64_t r0 = tm * 128 + 64 * wr, c0 = tn * 128 + 64 * wc;
  // FOLD (host: N a multiple of 4): the folded LayerNorm on each accumulator right before its epilogue, so that
  // few folded values are live at a time
  auto fold = [&](int ti, int tj) {
    if constexpr (FOLD) {
      asm volatile("" ::: "memory");   // keeps the LDS reads here instead of all hoisted to the epilogue's start
      fold_acc4(acc[ti][tj], rst[64 * wr + 16 * ti + li], cst + 64 * wc + 16 * tj + 4 * g);
    }
  };
  if (ext.w3 != nullptr) {   // (w1, w3) tile pairs (0, 1) and (2, 3) of the wave's 64 columns
    const int64_t H = N / 2;
    const bool v4 = lin_vec4_ok<DT, OT>(Y, ldy, Y2, ldy2, resid, ldr, kNoLinExt);
#pragma unroll
    for (int tj = 0; tj < 4; tj += 2) {
      const int64_t col = (c0 + 16 * tj) / 2 + 4 * g;
#pragma unroll
      for (int ti = 0; ti < 4; ++ti) {
        const int64_t row = r0 + 16 * ti + li;
        fold(ti, tj);
        fold(ti, tj + 1);
        if (row < M && col < H)
          glu_pair_epilogue<DT, OT>(acc[ti][tj], acc[ti][tj + 1], row, col, H, resid, ldr, Y, ldy, Y2, ldy2, v4);
      }
    }
    return;
  }
  const bool vec = lin_vec4_ok<DT, OT>(Y, ldy, Y2, ldy2, resid, ldr, ext);
#pragma unroll
  for (int tj = 0; tj < 4; ++tj) {
    const int64_t col = c0 + 16 * tj + 4 * g;
    float bv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) bv[r] = (bias && col + r < N) ? bias[col + r] : 0.f;
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
      const int64_t row = r0 + 16 * ti + li;
      fold(ti, tj);
      if (row >= M || col >= N) continue;
      lin_epilogue4<DT, OT>(acc[ti][tj], bv, row, col, N, relu, clamp_v, resid, ldr, Y, ldy, Y2, ldy2, ext, vec);
    }
  }
}

// 128x128 output tiles, 16-bit X and W, K a multiple of 64: the operands go from global memory straight into
// LDS (global_load_lds_dwordx4: each lane's 16 bytes land at lane * 16 of a wave-uniform LDS base, so no VGPRs
// stage them and no ds_write issues), two 32 KB stages of 64-wide K chunks, one barrier per chunk: chunk k + 1
// is requested into the other stage as soon as every wave has finished chunk k - 1, and is in flight while
// chunk k is multiplied.  64 KB of LDS: two workgroups per CU.  Each wave computes a 64x64 quadrant (4 x 4 MFMA
// tiles) as linear_lds128_kernel does, with the same instruction order, so the two give identical results.
// LDS layout per stage and operand: row r's eight 16-byte chunks at r * 8 + (c ^ (r & 7)); a fragment read
// (16 rows, one chunk) then touches eight distinct chunk slots of the bank rows.
constexpr int LD_KC = 64;
constexpr int LD_CPR = LD_KC / 8;                 // 16-byte chunks per row and chunk of K
constexpr int LD_OPB = 128 * LD_CPR * 16;         // bytes of one operand per stage (16 KB)

typedef __attribute__((address_space(3))) void lds_void_t;

// s_waitcnt with only the vector-memory count bounded (gfx9 encoding: vmcnt bits 3:0 and 15:14; expcnt and
// lgkmcnt at their maxima)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

template <int DT, int OT, bool STATS = false>
__global__ void __launch_bounds__(256)
linear_dma_kernel(const typename MM<DT>::T* __restrict__ X, int64_t ldx, const typename MM<DT>::T* __restrict__ W,
                  int64_t ldw, const float* __restrict__ bias, const float* __restrict__ resid, int64_t ldr,
                  typename MM<OT>::T* __restrict__ Y, int64_t ldy, typename MM<DT>::T* __restrict__ Y2,
                  int64_t ldy2, int64_t M, int64_t N, int64_t K, int relu, float clamp_v, OutSplit os, LinExt ext) {
  using A = MM<DT>;
  using T = typename A::T;
  static_assert(A::KPL == 8, "16-bit operands");
  __shared__ __align__(16) unsigned char smem[2 * 2 * LD_OPB];
  const int64_t tiles_n = (N + 127) / 128;
  const int64_t tile = ext.m_dev ? xcd_rowblock_tile(blockIdx.x, tiles_n, gridDim.x) : xcd_tile(blockIdx.x, gridDim.x);
  const int64_t tm = tile / tiles_n, tn = tile - tm * tiles_n;
  M = ext_rows(ext, M);
  if (tm * 128 >= M) return;   // the whole workgroup, before any barrier
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63, g = lane >> 4, li = lane & 15;
  const int wr = wid >> 1, wc = wid & 1;
  const int wu = __builtin_amdgcn_readfirstlane(wid);
  const int nk = (int)(K / LD_KC);
  // load map: unit u = 256 i + tid of an operand is LDS slot u (row u / 8, slot u % 8), which holds the row's
  // chunk (u % 8) ^ (row & 7); rows past M / N repeat the last row (their outputs are not stored)
  const T* pa[4];
  const T* pb[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int u = 256 * i + tid, r = u / LD_CPR, c = (u % LD_CPR) ^ (r & (LD_CPR - 1));
    int64_t ra = tm * 128 + r, rb = tn * 128 + r;
    ra = ra < M ? ra : M - 1;
    rb = rb < N ? rb : N - 1;
    pa[i] = X + ra * ldx + 8 * c;
    pb[i] = w_row(W, ext, rb, ldw) + 8 * c;
  }
  auto request = [&](int kc) {   // chunk kc into stage kc & 1: eight 16-byte loads per lane
    unsigned char* st = smem + (kc & 1) * 2 * LD_OPB;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      __builtin_amdgcn_global_load_lds((const void*)(pa[i] + (int64_t)kc * LD_KC),
                                       (lds_void_t*)(st + (256 * i + 64 * wu) * 16), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((const void*)(pb[i] + (int64_t)kc * LD_KC),
                                       (lds_void_t*)(st + LD_OPB + (256 * i + 64 * wu) * 16), 16, 0, 0);
    }
  };
  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  request(0);
  for (int kc = 0; kc < nk; ++kc) {
    wait_vmcnt<0>();   // this lane's part of chunk kc is in LDS
    __syncthreads();   // ... every lane's, and chunk kc - 1 is consumed by every wave (the fences also keep the
                       // compiler from moving LDS reads across the barrier)
    if (kc + 1 < nk) request(kc + 1);
    const T* As = reinterpret_cast<const T*>(smem + (kc & 1) * 2 * LD_OPB);
    const T* Bs = reinterpret_cast<const T*>(smem + (kc & 1) * 2 * LD_OPB + LD_OPB);
#pragma unroll
    for (int s = 0; s < LD_KC / 32; ++s) {
      typename A::Op a[4], b[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int ra = wr * 64 + 16 * t + li, rb = wc * 64 + 16 * t + li, c = 4 * s + g;
        a[t] = A::load(As + (ra * LD_CPR + (c ^ (ra & (LD_CPR - 1)))) * 8);
        b[t] = A::load(Bs + (rb * LD_CPR + (c ^ (rb & (LD_CPR - 1)))) * 8);
      }
      // weights as the A operand: acc[ti][tj][r] = out[row 16 ti + li][col 16 tj + 4g + r]
#pragma unroll
      for (int ti = 0; ti < 4; ++ti)
#pragma unroll
        for (int tj = 0; tj < 4; ++tj) acc[ti][tj] = A::mfma(b[tj], a[ti], acc[ti][tj]);
    }
  }
  const int64_t r0 = tm * 128 + 64 * wr, c0 = tn * 128 + 64 * wc;
  using TO = typename MM<OT>::T;
  if (sizeof(TO) == 2 && os.yt != nullptr && tn * 128 >= os.col) {
    // a tile of the transposed part (16-bit output, os.col a multiple of 128): transpose through LDS so that
    // consecutive threads write consecutive rows (tokens) of yt
    constexpr int TP = 130;   // pitch of the transposed tile (elements)
    TO* Ts = reinterpret_cast<TO*>(smem);
    static_assert(sizeof(TO) != 2 || 128 * TP * sizeof(TO) <= sizeof(smem), "transposed tile fits the stages");
    __syncthreads();   // the last chunk is consumed
#pragma unroll
    for (int tj = 0; tj < 4; ++tj)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t col = c0 + 16 * tj + 4 * g + r;
        const float bv = (bias && col < N) ? bias[col] : 0.f;
#pragma unroll
        for (int ti = 0; ti < 4; ++ti) {
          const int64_t row = r0 + 16 * ti + li;
          float val = acc[ti][tj][r] + bv;
          if (relu) val = fmaxf(val, 0.f);
          if (resid && row < M && col < N) val += resid[row * ldr + col];
          if (clamp_v > 0.f) val = fminf(fmaxf(val, -clamp_v), clamp_v);
          Ts[(64 * wc + 16 * tj + 4 * g + r) * TP + 64 * wr + 16 * ti + li] = MM<OT>::fromf(val);
        }
      }
    __syncthreads();
    TO* yt = reinterpret_cast<TO*>(os.yt);
    for (int i = tid; i < 128 * 128; i += 256) {
      const int c = i >> 7, rl = i & 127;
      const int64_t row = tm * 128 + rl, col = tn * 128 + c;
      if (row < M && col < N) {
        const int64_t fr = row / os.frame_rows, rr = row - fr * os.frame_rows;
        yt[fr * os.bstride + (col - os.col) * os.ldyt + rr] = Ts[c * TP + rl];
      }
    }
    return;
  }
  if (ext.w3 != nullptr) {   // (w1, w3) tile pairs (0, 1) and (2, 3) of the wave's 64 columns
    const int64_t H = N / 2;
    const bool v4 = lin_vec4_ok<DT, OT>(Y, ldy, Y2, ldy2, resid, ldr, kNoLinExt);
#pragma unroll
    for (int tj = 0; tj < 4; tj += 2) {
      const int64_t col = (c0 + 16 * tj) / 2 + 4 * g;
#pragma unroll
      for (int ti = 0; ti < 4; ++ti) {
        const int64_t row = r0 + 16 * ti + li;
        if (row < M && col < H)
          glu_pair_epilogue<DT, OT>(acc[ti][tj], acc[ti][tj + 1], row, col, H, resid, ldr, Y, ldy, Y2, ldy2, v4);
      }
    }
    return;
  }
  const bool vec = lin_vec4_ok<DT, OT>(Y, ldy, Y2, ldy2, resid, ldr, ext);
#pragma unroll
  for (int tj = 0; tj < 4; ++tj) {
    const int64_t col = c0 + 16 * tj + 4 * g;
    float bv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) bv[r] = (bias && col + r < N) ? bias[col + r] : 0.f;
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
      const int64_t row = r0 + 16 * ti + li;
      if (row >= M || col >= N) continue;
      lin_epilogue4<DT, OT>(acc[ti][tj], bv, row, col, N, relu, clamp_v, resid, ldr, Y, ldy, STATS ? nullptr : Y2,
                            ldy2, ext, vec);
    }
  }
  if (STATS && c0 < N) {
    // the 16-bit copy through LDS, in the stage the last chunk did not use (8 KB per wave; no other wave reads it
    // after the last chunk's barrier), so that each store writes 8 whole 128-byte rows of the quadrant: row r's
    // 16-byte chunk c at r * 64 + 8 (c ^ (r & 7)) elements
    if (Y2 != nullptr) {
      T* tb = reinterpret_cast<T*>(smem + (nk & 1) * 2 * LD_OPB) + wid * 64 * 64;
#pragma unroll
      for (int ti = 0; ti < 4; ++ti)
#pragma unroll
        for (int tj = 0; tj < 4; ++tj) {
          const int rl = 16 * ti + li, ch = (2 * tj + (g >> 1)) ^ (rl & 7);
          T e4[4] = {A::fromf(acc[ti][tj][0]), A::fromf(acc[ti][tj][1]), A::fromf(acc[ti][tj][2]),
                     A::fromf(acc[ti][tj][3])};
          *reinterpret_cast<uint2*>(tb + rl * 64 + 8 * ch + 4 * (g & 1)) = *reinterpret_cast<const uint2*>(e4);
        }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // the wave's stores are in LDS before any lane reads
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int rl = 8 * k + (lane >> 3), ch = lane & 7;
        const uint4 v = *reinterpret_cast<const uint4*>(tb + rl * 64 + 8 * (ch ^ (rl & 7)));
        const int64_t row = r0 + rl, col = c0 + 8 * ch;
        if (row < M && col < N) *reinterpret_cast<uint4*>(Y2 + row * ldy2 + col) = v;
      }
    }
    // LayerNorm partials of the stored rows over the wave's 64 columns (host: N a multiple of 64): each lane's mean
    // and centred sum of squares of its 16 values, combined over the 4 lane groups of the row
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
      float s1 = 0.f;
#pragma unroll
      for (int tj = 0; tj < 4; ++tj)
#pragma unroll
        for (int r = 0; r < 4; ++r) s1 += acc[ti][tj][r];
      const float ml = s1 * (1.f / 16.f);
      float m2 = 0.f;
#pragma unroll
      for (int tj = 0; tj < 4; ++tj)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float dv = acc[ti][tj][r] - ml;
          m2 += dv * dv;
        }
      const float m = rows4_sum(ml) * 0.25f;
      const float dg = ml - m;
      m2 = rows4_sum(m2 + 16.f * dg * dg);
      const int64_t row = r0 + 16 * ti + li;
      if (g == 0 && row < M) ext.pst[row * (N / 64) + c0 / 64] = make_float2(m, m2);
    }
  }
}

// Level-1 QKV projection and slot attention of one head in one launch (level1_event.py:37-52 for N = 32 slots and
// 64-wide heads, 16-bit operands).  Workgroup = (block of 128 rows = 4 events, head h); wave w owns event 4 b + w:
//   GEMM  its 32 rows x the head's 192 projection columns (q_h, k_h, v_h: rows h*64.., d + h*64.., 2d + h*64.. of
//         in_proj) over K = d_model, X and W chunks loaded straight into LDS as in linear_dma_kernel (two 40 KB
//         stages, one barrier per chunk);
//   attention  S^T = K Q^T and O^T = V^T P^T on v_mfma_f32_16x16x16 with the online softmax of event_attn_kernel
//         (mode 2: keys of dead slots excluded through obj_mask[ev_rows[e]], a query with every key excluded gives
//         NaN).  The GEMM accumulators hold row li, columns 4g .. 4g+3 of each 16-column block: for q and k that is
//         exactly the 16x16x16 operand layout (lane group g supplies head dims 16c + 4g .. +3 of MFMA c), so they
//         become operands by a rounding to the 16-bit type (the rounding the unfused QKV output takes); V is
//         transposed through LDS.
// q / k / v never reach HBM.  Output rows e*32 + i, columns h*64 .. h*64+63 of O (row stride ldo).
constexpr int QA_KC = 64;
constexpr int QA_VP = 72;   // LDS pitch of a wave's V rows (elements)

template <int DT>
__device__ __forceinline__ float qa_out(float acc, float inv) {
  float y = acc * inv;
  asm volatile("" : "+v"(y));   // as event_attn_kernel: the product rounded on its own, then converted
  return y;
}

// FOLD: LN1 folded into the weights (LinExt fst / fsum / fbias of linear_fold_rows, in_proj rows as the columns): each
// lane requests its two rows' partials and its 48 columns' (fsum, fbias) before the K loop (the LDS is full; the
// registers are not: two workgroups per CU leave 256 per lane) and folds the accumulators after it.
template <int DT, bool FOLD = false>
__global__ void __launch_bounds__(256, 2)
qkv_attn_kernel(const typename MM<DT>::T* __restrict__ X, int64_t ldx, const typename MM<DT>::T* __restrict__ W,
                typename MM<DT>::T* __restrict__ O, int64_t ldo, const int32_t* __restrict__ n_events, int64_t cap_rows,
                int64_t d, int H, const float* __restrict__ obj_mask, const int32_t* __restrict__ ev_rows,
                float scale_log2, LinExt fx) {
  using A = MM<DT>;
  using T = typename A::T;
  typedef short s16x4v __attribute__((ext_vector_type(4)));
  typedef _Float16 f16x4v __attribute__((ext_vector_type(4)));
  constexpr int CPR = QA_KC / 8;          // 16-byte chunks per row and chunk of K
  constexpr int XB = 128 * CPR * 16;      // X bytes per stage (16 KB)
  constexpr int WB = 192 * CPR * 16;      // W bytes per stage (24 KB)
  __shared__ __align__(16) unsigned char smem[2 * (XB + WB)];
  static_assert(4 * 32 * QA_VP * 2 <= sizeof(smem), "V rows fit the stages");
  const int64_t tile = xcd_rowblock_tile(blockIdx.x, H, gridDim.x);
  const int64_t rb = tile / H;
  const int h = (int)(tile - rb * H);
  int64_t M = (int64_t)(*n_events) * 32;
  M = M < cap_rows ? M : cap_rows;
  if (rb * 128 >= M) return;   // the whole workgroup, before any barrier
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63, g = lane >> 4, li = lane & 15;
  const int wu = __builtin_amdgcn_readfirstlane(wid);
  const int nk = (int)(d / QA_KC);
  // load maps (as linear_dma_kernel): unit u = 256 i + tid is LDS slot u (row u / 8, slot u % 8), which holds the
  // row's chunk (u % 8) ^ (row & 7); X rows past M repeat the last row (their outputs are not stored)
  const T* pa[4];
  const T* pb[6];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int u = 256 * i + tid, r = u / CPR, c = (u % CPR) ^ (r & (CPR - 1));
    int64_t ra = rb * 128 + r;
    ra = ra < M ? ra : M - 1;
    pa[i] = X + ra * ldx + 8 * c;
  }
#pragma unroll
  for (int i = 0; i < 6; ++i) {
    const int u = 256 * i + tid, r = u / CPR, c = (u % CPR) ^ (r & (CPR - 1));
    const int64_t wr = (int64_t)(r >> 6) * d + (int64_t)h * 64 + (r & 63);   // q, k or v row of head h
    pb[i] = W + wr * d + 8 * c;
  }
  auto request = [&](int kc) {
    unsigned char* st = smem + (kc & 1) * (XB + WB);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(pa[i] + (int64_t)kc * QA_KC),
                                       (lds_void_t*)(st + (256 * i + 64 * wu) * 16), 16, 0, 0);
#pragma unroll
    for (int i = 0; i < 6; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(pb[i] + (int64_t)kc * QA_KC),
                                       (lds_void_t*)(st + XB + (256 * i + 64 * wu) * 16), 16, 0, 0);
  };
  f32x4 acc[2][12];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int j = 0; j < 12; ++j) acc[t][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  request(0);
  float2 rs[2];          // FOLD: (mean, rstd) of rows 16 t + li of this wave's event
  float4 fc[12], fb[12];  // FOLD: fsum / fbias of columns 16 j + 4 g .. +3 of the head's 192
  if constexpr (FOLD) {
#pragma unroll
    for (int j = 0; j < 12; ++j) {
      const int64_t wr = (int64_t)(j >> 2) * d + (int64_t)h * 64 + 16 * (j & 3) + 4 * g;
      fc[j] = *reinterpret_cast<const float4*>(fx.fsum + wr);
      fb[j] = *reinterpret_cast<const float4*>(fx.fbias + wr);
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      int64_t row = rb * 128 + 32 * wid + 16 * t + li;
      row = row < M ? row : M - 1;
      rs[t] = fold_row_stats(fx.fst + row * fx.fparts, fx.fparts, fx.feps);
    }
  }
  for (int kc = 0; kc < nk; ++kc) {
    wait_vmcnt<0>();   // this lane's part of chunk kc is in LDS
    __syncthreads();   // every lane's, and chunk kc - 1 is consumed by every wave
    if (kc + 1 < nk) request(kc + 1);
    const T* Xs = reinterpret_cast<const T*>(smem + (kc & 1) * (XB + WB));
    const T* Ws = reinterpret_cast<const T*>(smem + (kc & 1) * (XB + WB) + XB);
#pragma unroll
    for (int s = 0; s < QA_KC / 32; ++s) {
      const int c = 4 * s + g;
      typename A::Op a[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int ra = 32 * wid + 16 * t + li;
        a[t] = A::load(Xs + (ra * CPR + (c ^ (ra & (CPR - 1)))) * 8);
      }
#pragma unroll
      for (int j = 0; j < 12; ++j) {
        const int rw = 16 * j + li;
        const typename A::Op b = A::load(Ws + (rw * CPR + (c ^ (rw & (CPR - 1)))) * 8);
        // weights as the A operand: acc[t][j][r] = out[row 16 t + li][col 16 j + 4 g + r]
#pragma unroll
        for (int t = 0; t < 2; ++t) acc[t][j] = A::mfma(b, a[t], acc[t][j]);
      }
    }
  }
  __syncthreads();   // every wave is done with the stages: they take the V rows now
  if constexpr (FOLD) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int j = 0; j < 12; ++j) {
        const float c[4] = {fc[j].x, fc[j].y, fc[j].z, fc[j].w}, b[4] = {fb[j].x, fb[j].y, fb[j].z, fb[j].w};
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[t][j][r] = rs[t].y * (acc[t][j][r] - rs[t].x * c[r]) + b[r];
      }
  }
  // this wave's event; q / k as 16x16x16 operands (dims 16 c + 4 g .. +3 of row 16 t + li), V to LDS
  const int64_t e = rb * 4 + wid;
  const bool live = e * 32 < M;
  s16x4v qo[2][4], ko[2][4];
  T* sv = reinterpret_cast<T*>(smem) + wid * 32 * QA_VP;
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        qo[t][c][r] = __builtin_bit_cast(short, A::fromf(acc[t][c][r]));   // the element's bits
        ko[t][c][r] = __builtin_bit_cast(short, A::fromf(acc[t][4 + c][r]));
      }
      T vv[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) vv[r] = A::fromf(acc[t][8 + c][r]);
      *reinterpret_cast<uint2*>(sv + (16 * t + li) * QA_VP + 16 * c + 4 * g) = *reinterpret_cast<const uint2*>(vv);
    }
  __syncthreads();   // (a wave reads only its own V rows; the barrier orders the LDS stores before the reads)
  if (!live) return;
  const float* om = obj_mask ? obj_mask + (int64_t)ev_rows[e] * 32 : nullptr;
  bool kok[2][4];
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int r = 0; r < 4; ++r) kok[kt][r] = om == nullptr || om[16 * kt + 4 * g + r] > 0.5f;
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    float m = -INFINITY, l = 0.f;
    float oacc[4][4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) oacc[r][nt] = 0.f;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      // V operand: keys 16 kt + 4 g + r, head columns 4 li .. 4 li + 3
      T ve[4][4];
#pragma unroll
      for (int r = 0; r < 4; ++r)
        *reinterpret_cast<uint2*>(ve[r]) = *reinterpret_cast<const uint2*>(sv + (16 * kt + 4 * g + r) * QA_VP + 4 * li);
      f32x4 s4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if constexpr (DT == HCLSM_BF16)
          s4 = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ko[kt][c], qo[qt][c], s4, 0, 0, 0);
        else
          s4 = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4v, ko[kt][c]),
                                                     __builtin_bit_cast(f16x4v, qo[qt][c]), s4, 0, 0, 0);
      }
      // s4[r] = S[query 16 qt + li][key 16 kt + 4 g + r]
      float sc[4];
      float tmax = -INFINITY;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sc[r] = kok[kt][r] ? s4[r] * scale_log2 : -INFINITY;
        tmax = fmaxf(tmax, sc[r]);
      }
      tmax = rows4_max(tmax);
      const float m_new = fmaxf(m, tmax);
      float pr[4], psum = 0.f;
      float alpha = 1.f;
      if (m_new != -INFINITY) {
        alpha = fast_exp2(m - m_new);
#pragma unroll
        for (int r = 0; r < 4; ++r) { pr[r] = fast_exp2(sc[r] - m_new); psum += pr[r]; }
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) pr[r] = 0.f;
      }
      psum = rows4_sum(psum);
      l = l * alpha + psum;
      m = m_new;
      s16x4v pb4;
#pragma unroll
      for (int r = 0; r < 4; ++r) pb4[r] = __builtin_bit_cast(short, A::fromf(pr[r]));
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        f32x4 o4 = {oacc[0][nt] * alpha, oacc[1][nt] * alpha, oacc[2][nt] * alpha, oacc[3][nt] * alpha};
        s16x4v av;
#pragma unroll
        for (int r = 0; r < 4; ++r) av[r] = __builtin_bit_cast(short, ve[r][nt]);
        if constexpr (DT == HCLSM_BF16)
          o4 = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(av, pb4, o4, 0, 0, 0);
        else
          o4 = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4v, av), __builtin_bit_cast(f16x4v, pb4),
                                                     o4, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) oacc[r][nt] = o4[r];
      }
    }
    // O[query 16 qt + li][dims 16 g + 4 r + nt]; l == 0 (every key excluded) -> NaN, as softmax over all -inf
    const float inv = 1.f / l;
    T ov[16];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) ov[4 * r + nt] = A::fromf(qa_out<DT>(oacc[r][nt], inv));
    T* dst = O + (e * 32 + 16 * qt + li) * ldo + (int64_t)h * 64 + 16 * g;
    *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(ov);
    *reinterpret_cast<uint4*>(dst + 8) = *reinterpret_cast<const uint4*>(ov + 8);
  }
}

// fp32 operands: the same 64x64 tile with A and W rows staged in LDS in K chunks of 64 floats (the next
// chunk in flight), each wave a 32x32 quadrant of v_mfma_f32_16x16x4_f32.  The contraction is permuted
// so that a lane's operands are float4 reads: in a 16-wide k block, lane group g owns k = 4g .. 4g+3 and
// MFMA j of the block contracts k = 4g + j across the four groups.
constexpr int LF_KC = 64;
constexpr int LF_LD = LF_KC + 4;   // LDS row pitch (floats)

template <int OT>
__global__ void __launch_bounds__(256)
linear_lds_f32_kernel(const float* __restrict__ X, int64_t ldx, const float* __restrict__ W, int64_t ldw,
                      const float* __restrict__ bias, const float* __restrict__ resid, int64_t ldr,
                      typename MM<OT>::T* __restrict__ Y, int64_t ldy, float* __restrict__ Y2, int64_t ldy2,
                      int64_t M, int64_t N, int64_t K, int relu, float clamp_v, LinExt ext) {
  __shared__ __align__(16) float As[64 * LF_LD];
  __shared__ __align__(16) float Bs[64 * LF_LD];
  const int64_t tiles_n = (N + 63) / 64;
  // (a device-side row count leaves only the leading tiles live: keep them spread over the XCDs; the row-block
  // order of the 16-bit kernels measured slower here)
  const int64_t tile = ext.m_dev ? (int64_t)blockIdx.x : xcd_tile(blockIdx.x, gridDim.x);
  const int64_t tm = tile / tiles_n, tn = tile - tm * tiles_n;
  M = ext_rows(ext, M);
  if (tm * 64 >= M) return;   // the whole workgroup, before any barrier
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63, g = lane >> 4, li = lane & 15;
  const int wr = wid >> 1, wc = wid & 1;
  // staging map: 64 rows x (KC / 4) float4 units = 1024 units per operand, 4 per thread
  const float* pa[4];
  const float* pb[4];
  int soff[4], ucol[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int u = tid + 256 * i, r = u >> 4;
    ucol[i] = (u & 15) * 4;
    int64_t ra = tm * 64 + r, rb = tn * 64 + r;
    ra = ra < M ? ra : M - 1;
    rb = rb < N ? rb : N - 1;
    pa[i] = X + ra * ldx + ucol[i];
    pb[i] = w_row(W, ext, rb, ldw) + ucol[i];
    soff[i] = r * LF_LD + ucol[i];
  }
  float4 ra_[4], rb_[4];
  auto fetch = [&](int64_t k0, int kc) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool in = ucol[i] < kc;
      ra_[i] = in ? *reinterpret_cast<const float4*>(pa[i] + k0) : make_float4(0.f, 0.f, 0.f, 0.f);
      rb_[i] = in ? *reinterpret_cast<const float4*>(pb[i] + k0) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  fetch(0, (int)(K < LF_KC ? K : LF_KC));
  for (int64_t k0 = 0; k0 < K; k0 += LF_KC) {
    const int kc = (int)(K - k0 < LF_KC ? K - k0 : LF_KC);
    __syncthreads();   // the previous chunk is consumed
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *reinterpret_cast<float4*>(As + soff[i]) = ra_[i];
      *reinterpret_cast<float4*>(Bs + soff[i]) = rb_[i];
    }
    __syncthreads();
    if (k0 + LF_KC < K) fetch(k0 + LF_KC, (int)(K - k0 - LF_KC < LF_KC ? K - k0 - LF_KC : LF_KC));
    for (int kb = 0; kb < (kc + 15) / 16; ++kb) {   // zero-padded past kc
      float4 a[2], b[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        a[t] = *reinterpret_cast<const float4*>(As + (wr * 32 + 16 * t + li) * LF_LD + kb * 16 + 4 * g);
        b[t] = *reinterpret_cast<const float4*>(Bs + (wc * 32 + 16 * t + li) * LF_LD + kb * 16 + 4 * g);
      }
#pragma unroll
      for (int ti = 0; ti < 2; ++ti)
#pragma unroll
        for (int tj = 0; tj < 2; ++tj) {
          // weights as the A operand: acc[ti][tj][r] = out[row 16 ti + li][col 16 tj + 4g + r]
          acc[ti][tj] = __builtin_amdgcn_mfma_f32_16x16x4f32(b[tj].x, a[ti].x, acc[ti][tj], 0, 0, 0);
          acc[ti][tj] = __builtin_amdgcn_mfma_f32_16x16x4f32(b[tj].y, a[ti].y, acc[ti][tj], 0, 0, 0);
          acc[ti][tj] = __builtin_amdgcn_mfma_f32_16x16x4f32(b[tj].z, a[ti].z, acc[ti][tj], 0, 0, 0);
          acc[ti][tj] = __builtin_amdgcn_mfma_f32_16x16x4f32(b[tj].w, a[ti].w, acc[ti][tj], 0, 0, 0);
        }
    }
  }
  const int64_t r0 = tm * 64 + 32 * wr, c0 = tn * 64 + 32 * wc;
  if (ext.w3 != nullptr) {   // (w1, w3) tile pair: the wave's two column tiles (c0 a multiple of 32)
    const int64_t H = N / 2, col = c0 / 2 + 4 * g;
    const bool v4 = lin_vec4_ok<HCLSM_F32, OT>(Y, ldy, Y2, ldy2, resid, ldr, kNoLinExt);
#pragma unroll
    for (int ti = 0; ti < 2; ++ti) {
      const int64_t row = r0 + 16 * ti + li;
      if (row < M && col < H)
        glu_pair_epilogue<HCLSM_F32, OT>(acc[ti][0], acc[ti][1], row, col, H, resid, ldr, Y, ldy, Y2, ldy2, v4);
    }
    return;
  }
  const bool vec = lin_vec4_ok<HCLSM_F32, OT>(Y, ldy, Y2, ldy2, resid, ldr, ext);
#pragma unroll
  for (int tj = 0; tj < 2; ++tj) {
    const int64_t col = c0 + 16 * tj + 4 * g;
    float bv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) bv[r] = (bias && col + r < N) ? bias[col + r] : 0.f;
#pragma unroll
    for (int ti = 0; ti < 2; ++ti) {
      const int64_t row = r0 + 16 * ti + li;
      if (row >= M || col >= N) continue;
      lin_epilogue4<HCLSM_F32, OT>(acc[ti][tj], bv, row, col, N, relu, clamp_v, resid, ldr, Y, ldy, Y2, ldy2, ext,
                                   vec);
    }
  }
}

template <int DT, int OT>
__global__ void __launch_bounds__(256)
linear_quad_kernel(const typename MM<DT>::T* __restrict__ X, int64_t ldx, const typename MM<DT>::T* __restrict__ W,
                   int64_t ldw, const float* __restrict__ bias, const float* __restrict__ resid, int64_t ldr,
                   typename MM<OT>::T* __restrict__ Y, int64_t ldy, typename MM<DT>::T* __restrict__ Y2,
                   int64_t ldy2, int64_t M, int64_t N, int64_t K, int relu, float clamp_v, OutSplit os, LinExt ext) {
  using A = MM<DT>;
  constexpr int KPL = A::KPL;
  constexpr int BLK = 4 * KPL;
  const int64_t tiles_n = (N + 63) / 64;
  const int64_t tm = blockIdx.x / tiles_n, tn = blockIdx.x - tm * tiles_n;
  M = ext_rows(ext, M);
  if (tm * 64 >= M) return;
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63, g = lane >> 4, li = lane & 15;
  const int64_t r0 = tm * 64 + 32 * (wid >> 1), c0 = tn * 64 + 32 * (wid & 1);
  const typename A::T* pa[2];
  const typename A::T* pb[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    int64_t r = r0 + 16 * t + li;
    r = r < M ? r : M - 1;
    pa[t] = X + r * ldx + KPL * g;
    int64_t c = c0 + 16 * t + li;
    c = c < N ? c : N - 1;
    pb[t] = W + c * ldw + KPL * g;
  }
  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int nblk = (int)(K / BLK);
#pragma unroll 4
  for (int s = 0; s < nblk; ++s) {
    const int64_t k0 = (int64_t)s * BLK;
    const typename A::Op a0 = A::load(pa[0] + k0), a1 = A::load(pa[1] + k0);
    const typename A::Op b0 = A::load(pb[0] + k0), b1 = A::load(pb[1] + k0);
    acc[0][0] = A::mfma(a0, b0, acc[0][0]);
    acc[0][1] = A::mfma(a0, b1, acc[0][1]);
    acc[1][0] = A::mfma(a1, b0, acc[1][0]);
    acc[1][1] = A::mfma(a1, b1, acc[1][1]);
  }
#pragma unroll
  for (int tj = 0; tj < 2; ++tj) {
    const int64_t col = c0 + 16 * tj + li;
    if (col >= N) continue;
    const float bv = bias ? bias[col] : 0.f;
#pragma unroll
    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t row = r0 + 16 * ti + 4 * g + r;
        if (row >= M) continue;
        float val = acc[ti][tj][r] + bv;
        if (relu) val = fmaxf(val, 0.f);
        val = ext_glu<DT>(ext, row, col, val);
        if (resid) val += resid[row * ldr + col];
        if (clamp_v > 0.f) val = fminf(fmaxf(val, -clamp_v), clamp_v);
        if (os.yt != nullptr && col >= os.col) {
          const int64_t fr = row / os.frame_rows, rr = row - fr * os.frame_rows;
          reinterpret_cast<typename MM<OT>::T*>(os.yt)[fr * os.bstride + (col - os.col) * os.ldyt + rr] =
              MM<OT>::fromf(val);
        } else {
          Y[row * ldy + col] = MM<OT>::fromf(val);
        }
        if (Y2) Y2[row * ldy2 + col] = A::fromf(val);
      }
  }
}

template <int DT, int OT, typename XT, bool LN>
__global__ void __launch_bounds__(256)
linear_kernel(const XT* __restrict__ X, int64_t ldx, const typename MM<DT>::T* __restrict__ W, int64_t ldw,
              const float* __restrict__ bias, const float* __restrict__ resid, int64_t ldr,
              typename MM<OT>::T* __restrict__ Y, int64_t ldy, typename MM<DT>::T* __restrict__ Y2, int64_t ldy2,
              int64_t M, int64_t N, int64_t K, int relu, float clamp_v, const float* __restrict__ lnw,
              const float* __restrict__ lnb, float ln_eps, LinExt ext) {
  using A = MM<DT>;
  constexpr int KPL = A::KPL;
  constexpr int BLK = 4 * KPL;
  __shared__ float red[4][2][2][4][64];   // [wave][ti][tj][r][lane]: 16 KB
  const int64_t tiles_n = (N + 31) / 32;
  const int64_t tm = blockIdx.x / tiles_n, tn = blockIdx.x - tm * tiles_n;
  M = ext_rows(ext, M);
  if (tm * 32 >= M) return;   // the whole workgroup, before any barrier
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63, g = lane >> 4, li = lane & 15;
  const XT* pa[2];
  const typename A::T* pb[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    int64_t r = tm * 32 + 16 * t + li;
    r = r < M ? r : M - 1;
    pa[t] = X + r * ldx + KPL * g;
    int64_t c = tn * 32 + 16 * t + li;
    c = c < N ? c : N - 1;
    pb[t] = W + c * ldw + KPL * g;
  }
  float mean[2] = {0.f, 0.f}, rstd[2] = {1.f, 1.f};
  if constexpr (LN) ln_stats<XT, KPL>(pa, K, wid, g, li, ln_eps, &red[0][0][0][0][0], mean, rstd);
  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int nblk = (int)(K / BLK);
#pragma unroll 2
  for (int s = wid; s < nblk; s += 4) {
    const int64_t k0 = (int64_t)s * BLK;
    typename A::Op a0, a1;
    if constexpr (LN) {
      a0 = load_op_ln<DT, XT>(pa[0] + k0, (int)k0 + KPL * g, mean[0], rstd[0], lnw, lnb);
      a1 = load_op_ln<DT, XT>(pa[1] + k0, (int)k0 + KPL * g, mean[1], rstd[1], lnw, lnb);
    } else {
      a0 = load_op<DT, XT>(pa[0] + k0);
      a1 = load_op<DT, XT>(pa[1] + k0);
    }
    const typename A::Op b0 = A::load(pb[0] + k0), b1 = A::load(pb[1] + k0);
    acc[0][0] = A::mfma(a0, b0, acc[0][0]);
    acc[0][1] = A::mfma(a0, b1, acc[0][1]);
    acc[1][0] = A::mfma(a1, b0, acc[1][0]);
    acc[1][1] = A::mfma(a1, b1, acc[1][1]);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[wid][i][j][r][lane] = acc[i][j][r];
  __syncthreads();
  // 1024 outputs, 4 per thread: thread -> (ti, tj) = wave index, lane, all four r
  {
    const int ti = wid >> 1, tj = wid & 1;
    const int64_t col = tn * 32 + 16 * tj + li;
    if (col < N) {
      const float bv = bias ? bias[col] : 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t row = tm * 32 + 16 * ti + 4 * g + r;
        if (row >= M) continue;
        float val = red[0][ti][tj][r][lane] + red[1][ti][tj][r][lane] + red[2][ti][tj][r][lane] +
                    red[3][ti][tj][r][lane] + bv;
        if (relu) val = fmaxf(val, 0.f);
        val = ext_glu<DT>(ext, row, col, val);
        if (resid) val += resid[row * ldr + col];
        if (clamp_v > 0.f) val = fminf(fmaxf(val, -clamp_v), clamp_v);
        Y[row * ldy + col] = MM<OT>::fromf(val);
        if (Y2) Y2[row * ldy2 + col] = A::fromf(val);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Small-M linear layer (16-bit operands) with every K block of a wave requested at once: the 4 waves
// of a 32 x 32 output tile split K in blocks of 32 (wave w: blocks w, w + 4, ...; KB per wave), each
// lane holding its 8 elements of every block for two rows and two columns, so the loads take one
// latency round instead of one per block.  With LN the row statistics of X come from the same
// registers (mean, then the centred sum of squares: two passes, two barriers) and the operands are
// normalised in place: LN(X) W^T with no separate LayerNorm launch.  xout (nullable): the workgroups
// of column tile 0 also store X rounded to DT.
// FOLD: LayerNorm folded into the weights instead.  With W = W0 diag(gamma) (rounded to DT), fsum[n] = the sum of
// row n of W (its rounded entries, in fp32) and bias = W0 beta (+ the layer's bias),
//   LN(x) W0^T + b = rstd (x W^T - mean fsum) + bias,
// so the operands go to the MFMAs as loaded and the row statistics (two passes over the same registers, while the
// products run) enter only the epilogue.  x (16-bit) is exact as given, and x W^T - mean fsum is the sum of
// (x - mean) W over the rounded entries, so nothing cancels beyond the fp32 accumulation.
template <int DT, int OT, typename XT, bool LN, int KB, bool FOLD = false>
__global__ void __launch_bounds__(256)
linear_kreg_kernel(const XT* __restrict__ X, int64_t ldx, const typename MM<DT>::T* __restrict__ W, int64_t ldw,
                   const float* __restrict__ bias, const float* __restrict__ resid, int64_t ldr,
                   typename MM<OT>::T* __restrict__ Y, int64_t ldy, typename MM<DT>::T* __restrict__ Y2,
                   int64_t ldy2, int64_t M, int64_t N, int64_t K, int relu, float clamp_v,
                   const float* __restrict__ lnw, const float* __restrict__ lnb, float ln_eps,
                   typename MM<DT>::T* __restrict__ xout, int64_t ldxo, const float* __restrict__ fsum) {
  using A = MM<DT>;
  constexpr int KPL = A::KPL;
  constexpr int BLK = 4 * KPL;
  static_assert(KPL == 8, "16-bit operands");
  static_assert(!(LN && FOLD), "one LayerNorm form");
  __shared__ float red[4][2][2][4][64];   // 16 KB
  __shared__ float stat[2][4][2][16];     // [pass][wave][row tile][li]
  __shared__ float2 fstat[FOLD ? 4 : 1][2][16];   // FOLD: (mean, centred sum of squares) [wave][row tile][li]
  const int64_t tiles_n = (N + 31) / 32;
  const int64_t tm = blockIdx.x / tiles_n, tn = blockIdx.x - tm * tiles_n;
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63, g = lane >> 4, li = lane & 15;
  const int nblk = (int)(K / BLK);
  const XT* pa[2];
  const typename A::T* pb[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    int64_t r = tm * 32 + 16 * t + li;
    r = r < M ? r : M - 1;
    pa[t] = X + r * ldx + KPL * g;
    int64_t c = tn * 32 + 16 * t + li;
    c = c < N ? c : N - 1;
    pb[t] = W + c * ldw + KPL * g;
  }
  // 0. the epilogue's bias and residual values of this thread's four outputs, requested first so that their
  // latency overlaps the operand loads instead of following the reduction
  const int ti = wid >> 1, tj = wid & 1;
  const int64_t col = tn * 32 + 16 * tj + li;
  float bv = 0.f, rv[4] = {0.f, 0.f, 0.f, 0.f}, fs = 0.f;
  if (col < N) {
    if (bias) bv = bias[col];
    if constexpr (FOLD) fs = fsum[col];
    if (resid) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t row = tm * 32 + 16 * ti + 4 * g + r;
        if (row < M) rv[r] = resid[row * ldr + col];
      }
    }
  }
  // 1. every operand of this wave's blocks (block index clamped; blocks past nblk are skipped below)
  float xa[LN ? KB : 1][2][KPL];
  typename A::Op ao[LN ? 1 : KB][2], bo[KB][2];
  float lw[LN ? KB : 1][KPL], lb[LN ? KB : 1][KPL];
#pragma unroll
  for (int i = 0; i < KB; ++i) {
    const int sb = wid + 4 * i < nblk ? wid + 4 * i : nblk - 1;
    const int64_t k0 = (int64_t)sb * BLK;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      if constexpr (LN) {
        load8f<XT>(pa[t] + k0, xa[i][t]);
      } else {
        ao[i][t] = load_op<DT, XT>(pa[t] + k0);
      }
      bo[i][t] = A::load(pb[t] + k0);
    }
    if constexpr (LN) {
      if (lnw) load8f<float>(lnw + k0 + KPL * g, lw[i]);
      else
#pragma unroll
        for (int e = 0; e < KPL; ++e) lw[i][e] = 1.f;
      if (lnb) load8f<float>(lnb + k0 + KPL * g, lb[i]);
      else
#pragma unroll
        for (int e = 0; e < KPL; ++e) lb[i][e] = 0.f;
    }
  }
  float mean[2] = {0.f, 0.f}, rstd[2] = {1.f, 1.f};
  if constexpr (LN) {
    // 2. row mean, then the centred sum of squares, over this lane's values, the 4 lane groups and the waves
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        float sacc = 0.f;
#pragma unroll
        for (int i = 0; i < KB; ++i) {
          if (wid + 4 * i >= nblk) continue;
#pragma unroll
          for (int e = 0; e < KPL; ++e) {
            const float dv = pass == 0 ? xa[i][t][e] : xa[i][t][e] - mean[t];
            sacc += pass == 0 ? dv : dv * dv;
          }
        }
        sacc = rows4_sum(sacc);
        if (g == 0) stat[pass][wid][t][li] = sacc;
      }
      __syncthreads();
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const float tot = stat[pass][0][t][li] + stat[pass][1][t][li] + stat[pass][2][t][li] + stat[pass][3][t][li];
        if (pass == 0) mean[t] = tot / (float)K;
        else rstd[t] = rsqrtf(tot / (float)K + ln_eps);
      }
    }
    if (xout != nullptr && tn == 0) {   // X in DT, rows of this tile
#pragma unroll
      for (int i = 0; i < KB; ++i) {
        if (wid + 4 * i >= nblk) continue;
        const int64_t k0 = (int64_t)(wid + 4 * i) * BLK + KPL * g;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int64_t row = tm * 32 + 16 * t + li;
          if (row >= M) continue;
          typename A::T e8[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) e8[e] = A::fromf(xa[i][t][e]);
          *reinterpret_cast<uint4*>(xout + row * ldxo + k0) = *reinterpret_cast<uint4*>(e8);
        }
      }
    }
  }
  // 3. the products
  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < KB; ++i) {
    if (wid + 4 * i >= nblk) continue;
    typename A::Op a[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      if constexpr (LN) {
        typename A::T e8[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) e8[e] = A::fromf((xa[i][t][e] - mean[t]) * rstd[t] * lw[i][e] + lb[i][e]);
        a[t] = __builtin_bit_cast(typename A::Op, *reinterpret_cast<uint4*>(e8));
      } else {
        a[t] = ao[i][t];
      }
    }
    acc[0][0] = A::mfma(a[0], bo[i][0], acc[0][0]);
    acc[0][1] = A::mfma(a[0], bo[i][1], acc[0][1]);
    acc[1][0] = A::mfma(a[1], bo[i][0], acc[1][0]);
    acc[1][1] = A::mfma(a[1], bo[i][1], acc[1][1]);
  }
  // FOLD: the row statistics of this lane's rows 16 t + li over the wave's part of K, with no barrier: the mean
  // and centred sum of squares of the lane's own values, combined over the 4 lane groups (equal counts) by
  // M2 = sum M2_g + n_g sum (m_g - m)^2; the waves' parts are combined the same way in the epilogue
  if constexpr (FOLD) {
    const int kbw = nblk > wid ? (nblk - 1 - wid) / 4 + 1 : 0;   // blocks of this wave
    const float ng = (float)(KPL * kbw), inv = kbw > 0 ? __builtin_amdgcn_rcpf(ng) : 0.f;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      float xs[KB][KPL];
      float s1 = 0.f;
#pragma unroll
      for (int i = 0; i < KB; ++i) {
        typename A::T e8[8];
        *reinterpret_cast<uint4*>(e8) = __builtin_bit_cast(uint4, ao[i][t]);
#pragma unroll
        for (int e = 0; e < KPL; ++e) {
          xs[i][e] = A::tof(e8[e]);
          if (wid + 4 * i < nblk) s1 += xs[i][e];
        }
      }
      const float mg = s1 * inv;
      float m2 = 0.f;
#pragma unroll
      for (int i = 0; i < KB; ++i) {
        if (wid + 4 * i >= nblk) continue;
#pragma unroll
        for (int e = 0; e < KPL; ++e) {
          const float dv = xs[i][e] - mg;
          m2 += dv * dv;
        }
      }
      const float mw = rows4_sum(mg) * 0.25f;
      const float dg = mg - mw;
      m2 = rows4_sum(m2 + ng * dg * dg);
      if (g == 0) fstat[wid][t][li] = make_float2(mw, m2);
    }
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[wid][i][j][r][lane] = acc[i][j][r];
  __syncthreads();
  // 1024 outputs, 4 per thread: thread -> (ti, tj) = wave index, lane, all four r
  if (col >= N) return;
  float fmu[4], frs[4];   // FOLD: mean and rstd of this thread's rows 16 ti + 4 g + r
  if constexpr (FOLD) {
    // the waves' parts: wave w holds 32 x (its block count) of the row's K values
    float2 p[4][4];
    const float invk = __builtin_amdgcn_rcpf((float)K);
#pragma unroll
    for (int w = 0; w < 4; ++w)
#pragma unroll
      for (int r = 0; r < 4; ++r) p[w][r] = fstat[w][ti][4 * g + r];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float nw[4], mu = 0.f, m2 = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        nw[w] = (float)(BLK * (nblk > w ? (nblk - 1 - w) / 4 + 1 : 0));
        mu += nw[w] * p[w][r].x;
      }
      mu *= invk;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float dw = p[w][r].x - mu;
        m2 += p[w][r].y + nw[w] * dw * dw;
      }
      fmu[r] = mu;
      frs[r] = rsqrtf(m2 * invk + ln_eps);
    }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t row = tm * 32 + 16 * ti + 4 * g + r;
    if (row >= M) continue;
    float val = red[0][ti][tj][r][lane] + red[1][ti][tj][r][lane] + red[2][ti][tj][r][lane] +
                red[3][ti][tj][r][lane];
    if constexpr (FOLD) {
      val = frs[r] * (val - fmu[r] * fs) + bv;
    } else {
      val += bv;
    }
    if (relu) val = fmaxf(val, 0.f);
    if (resid) val += rv[r];
    if (clamp_v > 0.f) val = fminf(fmaxf(val, -clamp_v), clamp_v);
    Y[row * ldy + col] = MM<OT>::fromf(val);
    if (Y2) Y2[row * ldy2 + col] = A::fromf(val);
  }
}

// ---------------------------------------------------------------------------
// GH: the hidden-side products come precomputed in gh ([M][3H] fp32, row stride ldgh, without b_hh); Hb and Whh
// are not read.
template <int DT, bool GH>
__global__ void __launch_bounds__(256)
gru_kernel(const typename MM<DT>::T* __restrict__ X, int64_t ldx, const typename MM<DT>::T* __restrict__ Hb,
           int64_t ldhb, const float* __restrict__ Hf, int64_t ldh, const typename MM<DT>::T* __restrict__ Wih,
           const typename MM<DT>::T* __restrict__ Whh, const float* __restrict__ bih, const float* __restrict__ bhh,
           float* __restrict__ out, int64_t ldo, typename MM<DT>::T* __restrict__ out2, int64_t ldo2, int64_t M,
           int64_t H, int64_t Kx, const float* __restrict__ gh, int64_t ldgh) {
  using A = MM<DT>;
  constexpr int KPL = A::KPL;
  constexpr int BLK = 4 * KPL;
  constexpr int NQ = GH ? 3 : 6;         // products formed here
  __shared__ float red[4][2][NQ][4][64];  // 48 KB (24 KB with GH)
  const int64_t tiles_n = (H + 15) / 16;
  const int64_t tm = blockIdx.x / tiles_n, tn = blockIdx.x - tm * tiles_n;
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63, g = lane >> 4, li = lane & 15;
  int64_t colr = tn * 16 + li;
  colr = colr < H ? colr : H - 1;
  int64_t rows[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int64_t r = tm * 32 + 16 * t + li;
    rows[t] = r < M ? r : M - 1;
  }
  // the epilogue's biases and previous hidden state for this thread's two outputs, requested first
  const int64_t col = tn * 16 + li;
  const int t_e = wid >> 1;
  float bir = 0.f, biz = 0.f, bin = 0.f, bhr = 0.f, bhz = 0.f, bhn = 0.f, hv[2] = {0.f, 0.f};
  float ghv[2][3] = {{0.f, 0.f, 0.f}, {0.f, 0.f, 0.f}};
  if (col < H) {
    if (bih) { bir = bih[col]; biz = bih[H + col]; bin = bih[2 * H + col]; }
    if (bhh) { bhr = bhh[col]; bhz = bhh[H + col]; bhn = bhh[2 * H + col]; }
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      const int64_t row = tm * 32 + 16 * t_e + 4 * g + 2 * (wid & 1) + rr;
      if (row < M) {
        hv[rr] = Hf[row * ldh + col];
        if constexpr (GH) {
#pragma unroll
          for (int q = 0; q < 3; ++q) ghv[rr][q] = gh[row * ldgh + q * H + col];
        }
      }
    }
  }
  f32x4 acc[2][NQ];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < NQ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  {
    const typename A::T* pa[2] = {X + rows[0] * ldx + KPL * g, X + rows[1] * ldx + KPL * g};
    const typename A::T* pw[3] = {Wih + colr * Kx + KPL * g, Wih + (H + colr) * Kx + KPL * g,
                                  Wih + (2 * H + colr) * Kx + KPL * g};
    const int nblk = (int)(Kx / BLK);
    for (int s = wid; s < nblk; s += 4) {
      const int64_t k0 = (int64_t)s * BLK;
      const typename A::Op a0 = A::load(pa[0] + k0), a1 = A::load(pa[1] + k0);
#pragma unroll
      for (int q = 0; q < 3; ++q) {
        const typename A::Op bq = A::load(pw[q] + k0);
        acc[0][q] = A::mfma(a0, bq, acc[0][q]);
        acc[1][q] = A::mfma(a1, bq, acc[1][q]);
      }
    }
  }
  if constexpr (!GH) {
    const typename A::T* pa[2] = {Hb + rows[0] * ldhb + KPL * g, Hb + rows[1] * ldhb + KPL * g};
    const typename A::T* pw[3] = {Whh + colr * H + KPL * g, Whh + (H + colr) * H + KPL * g,
                                  Whh + (2 * H + colr) * H + KPL * g};
    const int nblk = (int)(H / BLK);
    for (int s = wid; s < nblk; s += 4) {
      const int64_t k0 = (int64_t)s * BLK;
      const typename A::Op a0 = A::load(pa[0] + k0), a1 = A::load(pa[1] + k0);
#pragma unroll
      for (int q = 0; q < 3; ++q) {
        const typename A::Op bq = A::load(pw[q] + k0);
        acc[0][3 + q] = A::mfma(a0, bq, acc[0][3 + q]);
        acc[1][3 + q] = A::mfma(a1, bq, acc[1][3 + q]);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int q = 0; q < NQ; ++q)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[wid][t][q][r][lane] = acc[t][q][r];
  __syncthreads();
  // 512 outputs (32 rows x 16 cols): thread -> (t = wid >> 1, r pair = 2 * (wid & 1) .. +1), lane
  if (col >= H) return;
  const int t = t_e;
#pragma unroll
  for (int rr = 0; rr < 2; ++rr) {
    const int r = 2 * (wid & 1) + rr;
    const int64_t row = tm * 32 + 16 * t + 4 * g + r;
    if (row >= M) continue;
    float gsum[6];
#pragma unroll
    for (int q = 0; q < NQ; ++q)
      gsum[q] = red[0][t][q][r][lane] + red[1][t][q][r][lane] + red[2][t][q][r][lane] + red[3][t][q][r][lane];
    if constexpr (GH) {
#pragma unroll
      for (int q = 0; q < 3; ++q) gsum[3 + q] = ghv[rr][q];
    }
    const float rg = sigmoid_f(gsum[0] + bir + gsum[3] + bhr);
    const float zg = sigmoid_f(gsum[1] + biz + gsum[4] + bhz);
    const float ng = tanh_f(gsum[2] + bin + rg * (gsum[5] + bhn));
    const float o = (1.f - zg) * ng + zg * hv[rr];
    out[row * ldo + col] = o;
    if (out2) out2[row * ldo2 + col] = A::fromf(o);
  }
}

// ---------------------------------------------------------------------------
// Slot-attention core.
struct CoreArgs {
  int64_t ldq, ldk, ldv, ldo, qb, kb, vb, ob;  // row strides and frame strides (elements)
  int N, M, D, NT, MT;                          // NT = ceil(N/16), MT = ceil(M/16)
  float scale, denom_eps, logit_clamp, renorm_eps;
};

constexpr int CORE_MAX_NT = 8;  // up to 128 slots

// P: [B][N][Mp] (Mp = 32 * ceil(M/32)) softmax in DT, zero for m >= M.  part: [B][MT][N] fp32.
// Grid (frame, 16-token tile); the 4 waves split the D blocks, partial logits meet in LDS and
// wave 0 finishes the softmax over slots.
// NWL waves split the contraction (8 for fp32 on a grid that fills few CUs: half the blocks per wave).
template <int DT, int AT, int NWL = 4>
__global__ void __launch_bounds__(64 * NWL)
core_logits_kernel(const typename MM<DT>::T* __restrict__ q, const typename MM<DT>::T* __restrict__ k,
                   typename MM<DT>::T* __restrict__ P, int64_t Mp, float* __restrict__ part,
                   typename MM<AT>::T* __restrict__ attn_out, CoreArgs a) {
  using A = MM<DT>;
  constexpr int KPL = A::KPL;
  constexpr int BLK = 4 * KPL;
  __shared__ float red[NWL][CORE_MAX_NT][4][64];   // 32 KB (64 KB with eight waves)
  const int64_t b = blockIdx.x;
  const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, li = lane & 15;
  const int mt = blockIdx.y;
  const int m = mt * 16 + li;                  // this lane's token (column)
  const bool mvalid = m < a.M;
  const typename A::T* kp = k + b * a.kb + (int64_t)(mvalid ? m : a.M - 1) * a.ldk + KPL * g;
  f32x4 acc[CORE_MAX_NT];
#pragma unroll
  for (int nt = 0; nt < CORE_MAX_NT; ++nt) acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int nblk = a.D / BLK;
  const typename A::T* qrow[CORE_MAX_NT];
#pragma unroll
  for (int nt = 0; nt < CORE_MAX_NT; ++nt) {
    int n = nt * 16 + li;
    n = n < a.N ? n : a.N - 1;
    qrow[nt] = q + b * a.qb + (int64_t)n * a.ldq + KPL * g;
  }
#pragma unroll 2
  for (int s = wid; s < nblk; s += NWL) {
    const typename A::Op kb_ = A::load(kp + (int64_t)s * BLK);
#pragma unroll
    for (int nt = 0; nt < CORE_MAX_NT; ++nt) {
      if (nt < a.NT) {
        const typename A::Op qa = A::load(qrow[nt] + (int64_t)s * BLK);
        acc[nt] = A::mfma(qa, kb_, acc[nt]);   // acc[nt][r] = logit[n = 16nt + 4g + r][m]
      }
    }
  }
#pragma unroll
  for (int nt = 0; nt < CORE_MAX_NT; ++nt)
    if (nt < a.NT)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[wid][nt][r][lane] = acc[nt][r];
  __syncthreads();
  if (wid != 0) return;
#pragma unroll
  for (int nt = 0; nt < CORE_MAX_NT; ++nt)
    if (nt < a.NT)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float t = 0.f;
#pragma unroll
        for (int w = 0; w < NWL; ++w) t += red[w][nt][r][lane];
        acc[nt][r] = t;
      }
  // softmax over slots for column m: values over (nt, r) in-lane and over g across lanes
  float mx = -INFINITY;
#pragma unroll
  for (int nt = 0; nt < CORE_MAX_NT; ++nt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int n = nt * 16 + 4 * g + r;
      float s = acc[nt][r] * a.scale;
      if (a.logit_clamp > 0.f) s = fminf(fmaxf(s, -a.logit_clamp), a.logit_clamp);
      s = (nt < a.NT && n < a.N) ? s : -INFINITY;
      acc[nt][r] = s;
      mx = fmaxf(mx, s);
    }
  mx = rows4_max(mx);
  float sum = 0.f;
#pragma unroll
  for (int nt = 0; nt < CORE_MAX_NT; ++nt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float e = (nt < a.NT) ? __expf(acc[nt][r] - mx) : 0.f;
      acc[nt][r] = e;
      sum += e;
    }
  sum = rows4_sum(sum);
  const float inv = 1.f / (sum + a.denom_eps);
#pragma unroll
  for (int nt = 0; nt < CORE_MAX_NT; ++nt) {
    if (nt >= a.NT) break;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int n = nt * 16 + 4 * g + r;
      const float p = mvalid ? acc[nt][r] * inv : 0.f;
      float ps = p;   // partial sum over this tile's 16 tokens, for the renormalisation
      ps += __shfl_xor(ps, 1, 64);
      ps += __shfl_xor(ps, 2, 64);
      ps += __shfl_xor(ps, 4, 64);
      ps += __shfl_xor(ps, 8, 64);
      if (n < a.N) {
        P[(b * a.N + n) * Mp + m] = A::fromf(p);
        if (attn_out && mvalid) attn_out[(b * a.N + n) * (int64_t)a.M + m] = MM<AT>::fromf(p);
        if (li == 0 && part && mt < a.MT) part[(b * a.MT + mt) * a.N + n] = ps;
      }
    }
  }
}

// attn . v with v given transposed per frame: vt[b][d][Mp] (rows of Mp tokens, m >= M ignored).
// Grid (frame, 64-column block); wave w owns 16 columns; no LDS.
template <int DT>
__global__ void __launch_bounds__(256)
core_update_t_kernel(const typename MM<DT>::T* __restrict__ P, int64_t Mp, const float* __restrict__ part,
                     const typename MM<DT>::T* __restrict__ vt, typename MM<DT>::T* __restrict__ out, CoreArgs a) {
  using A = MM<DT>;
  using TT = typename A::T;
  constexpr int KPL = A::KPL;
  __shared__ float rinv_s[CORE_MAX_NT * 16];
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63, g = lane >> 4, li = lane & 15;
  const int d = blockIdx.y * 64 + wid * 16 + li;
  const int dc = d < a.D ? d : a.D - 1;
  const bool renorm = a.renorm_eps >= 0.f;
  if (tid < a.NT * 16) {   // 1 / sum_m (attn + eps) per slot, from the per-tile partial sums
    float s = 1.f;
    if (renorm && tid < a.N) {
      float t = 0.f;
      for (int j = 0; j < a.MT; ++j) t += part[(b * a.MT + j) * a.N + tid];
      s = 1.f / (t + (float)a.M * a.renorm_eps);
    }
    rinv_s[tid] = s;
  }
  __syncthreads();
  const TT* pv = vt + b * a.vb + (int64_t)dc * Mp;
  const TT* prow[CORE_MAX_NT];
#pragma unroll
  for (int nt = 0; nt < CORE_MAX_NT; ++nt) {
    int n = nt * 16 + li;
    n = n < a.N ? n : a.N - 1;
    prow[nt] = P + (b * a.N + n) * Mp;
  }
  f32x4 acc[CORE_MAX_NT];
#pragma unroll
  for (int nt = 0; nt < CORE_MAX_NT; ++nt) acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float cs = 0.f;
#pragma unroll 2
  for (int m0 = 0; m0 < (int)Mp; m0 += 32) {
    if constexpr (KPL == 8) {
      typename A::Op bv = A::load(pv + m0 + 8 * g);
      if (m0 + 32 > a.M) {   // tokens past M: v rows are not initialised, zero them
        TT e[8];
        *reinterpret_cast<uint4*>(e) = __builtin_bit_cast(uint4, bv);
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (m0 + 8 * g + i >= a.M) e[i] = A::fromf(0.f);
        bv = __builtin_bit_cast(typename A::Op, *reinterpret_cast<uint4*>(e));
      }
      if (renorm) {
        TT e[8];
        *reinterpret_cast<uint4*>(e) = __builtin_bit_cast(uint4, bv);
#pragma unroll
        for (int i = 0; i < 8; ++i) cs += A::tof(e[i]);
      }
#pragma unroll
      for (int nt = 0; nt < CORE_MAX_NT; ++nt)
        if (nt < a.NT) acc[nt] = A::mfma(A::load(prow[nt] + m0 + 8 * g), bv, acc[nt]);
    } else {
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const int mm = m0 + 4 * s + g;
        float bv = mm < a.M ? pv[mm] : 0.f;
        if (renorm) cs += bv;
#pragma unroll
        for (int nt = 0; nt < CORE_MAX_NT; ++nt)
          if (nt < a.NT) acc[nt] = A::mfma(prow[nt][mm], bv, acc[nt]);
      }
    }
  }
  cs = rows4_sum(cs);
  if (d >= a.D) return;
  const float epsv = renorm ? a.renorm_eps * cs : 0.f;
#pragma unroll
  for (int nt = 0; nt < CORE_MAX_NT; ++nt) {
    if (nt >= a.NT) break;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int n = nt * 16 + 4 * g + r;
      if (n < a.N) out[b * a.ob + (int64_t)n * a.ldo + d] = A::fromf((acc[nt][r] + epsv) * rinv_s[n]);
    }
  }
}

constexpr int CORE_DB = 64;          // output columns per workgroup
constexpr int CORE_MAXM = 256;       // tokens staged in LDS at once (longer inputs loop)

template <int DT>
__global__ void __launch_bounds__(256)
core_update_kernel(const typename MM<DT>::T* __restrict__ P, int64_t Mp, const float* __restrict__ part,
                   const typename MM<DT>::T* __restrict__ v, typename MM<DT>::T* __restrict__ out, CoreArgs a) {
  using A = MM<DT>;
  using TT = typename A::T;
  constexpr int KPL = A::KPL;
  constexpr int VLD = CORE_MAXM + 8;   // row stride of the transposed chunk (elements)
  __shared__ __align__(16) TT VT[CORE_DB * VLD];
  __shared__ float colsum[CORE_DB];
  __shared__ float rinv[CORE_MAX_NT * 16];
  const int64_t b = blockIdx.x;
  const int d0 = blockIdx.y * CORE_DB;
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63, g = lane >> 4, li = lane & 15;
  const bool renorm = a.renorm_eps >= 0.f;
  if (tid < a.NT * 16) {
    float s = 1.f;
    if (renorm && tid < a.N) {
      float t = 0.f;
      for (int j = 0; j < a.MT; ++j) t += part[(b * a.MT + j) * a.N + tid];
      s = 1.f / (t + (float)a.M * a.renorm_eps);
    }
    rinv[tid] = s;
  }
  const int dt = wid;   // wave -> 16-column tile of the 64-column block
  f32x4 acc[CORE_MAX_NT];
#pragma unroll
  for (int nt = 0; nt < CORE_MAX_NT; ++nt) acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
  const TT* vb = v + b * a.vb;
  float cs = 0.f;
  for (int m0 = 0; m0 < (int)Mp; m0 += CORE_MAXM) {
    const int mc = ((int)Mp - m0) < CORE_MAXM ? ((int)Mp - m0) : CORE_MAXM;   // multiple of 32
    __syncthreads();
    // one pass: thread i loads v[m0 + ml][d0 + dl] for all (ml, dl) of the chunk
    for (int i = tid; i < mc * CORE_DB; i += 256) {
      const int ml = i / CORE_DB, dl = i - ml * CORE_DB;
      const int m = m0 + ml, d = d0 + dl;
      VT[dl * VLD + ml] = (m < a.M && d < a.D) ? vb[(int64_t)m * a.ldv + d] : A::fromf(0.f);
    }
    __syncthreads();
    if (renorm && tid < CORE_DB)
      for (int ml = 0; ml < mc; ++ml) cs += A::tof(VT[tid * VLD + ml]);
    const TT* pv = VT + (dt * 16 + li) * VLD;
    for (int mm = 0; mm < mc; mm += 32) {
#pragma unroll
      for (int nt = 0; nt < CORE_MAX_NT; ++nt) {
        if (nt < a.NT) {
          int n = nt * 16 + li;
          n = n < a.N ? n : a.N - 1;
          const TT* pp = P + (b * a.N + n) * Mp + m0 + mm;
          if constexpr (KPL == 8) {
            acc[nt] = A::mfma(A::load(pp + 8 * g), A::load(pv + mm + 8 * g), acc[nt]);
          } else {
#pragma unroll
            for (int s = 0; s < 8; ++s)
              acc[nt] = A::mfma(A::load(pp + 4 * s + g), A::load(pv + mm + 4 * s + g), acc[nt]);
          }
        }
      }
    }
  }
  if (tid < CORE_DB) colsum[tid] = cs;
  __syncthreads();
  const int d = d0 + dt * 16 + li;
  if (d >= a.D) return;
  const float epsv = renorm ? a.renorm_eps * colsum[dt * 16 + li] : 0.f;
#pragma unroll
  for (int nt = 0; nt < CORE_MAX_NT; ++nt) {
    if (nt >= a.NT) break;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int n = nt * 16 + 4 * g + r;
      if (n < a.N) out[b * a.ob + (int64_t)n * a.ldo + d] = A::fromf((acc[nt][r] + epsv) * rinv[n]);
    }
  }
}

// attn @ v for fp32 operands on a narrow grid (few frames): grid (frame, 16-column tile), the 4 waves splitting the
// token steps (4 tokens per 16x16x4 product, step t to wave t % 4) and meeting in LDS.  v is read in place: for
// fp32 a lane's B operand is one element, v[m][d], and the 16 lanes of a lane group read 16 consecutive columns.
// Same output as core_update_kernel: (sum_m attn v + renorm_eps sum_m v) / (sum_m attn + M renorm_eps) when
// renormalising.
__global__ void __launch_bounds__(256)
core_update_narrow_kernel(const float* __restrict__ P, int64_t Mp, const float* __restrict__ part,
                          const float* __restrict__ v, float* __restrict__ out, CoreArgs a) {
  using A = MM<HCLSM_F32>;
  __shared__ float red[4][CORE_MAX_NT][4][64];   // 32 KB
  __shared__ float csum[4][16];
  __shared__ float rinv[CORE_MAX_NT * 16];
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63, g = lane >> 4, li = lane & 15;
  const int d = blockIdx.y * 16 + li;
  const int dc = d < a.D ? d : a.D - 1;
  const bool renorm = a.renorm_eps >= 0.f;
  if (tid < a.NT * 16) {
    float sr = 1.f;
    if (renorm && tid < a.N) {
      float t = 0.f;
      for (int j = 0; j < a.MT; ++j) t += part[(b * a.MT + j) * a.N + tid];
      sr = 1.f / (t + (float)a.M * a.renorm_eps);
    }
    rinv[tid] = sr;
  }
  f32x4 acc[CORE_MAX_NT];
#pragma unroll
  for (int nt = 0; nt < CORE_MAX_NT; ++nt) acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
  const float* vb = v + b * a.vb + dc;
  const float* pb = P + b * (int64_t)a.N * Mp;
  int prow[CORE_MAX_NT];
#pragma unroll
  for (int nt = 0; nt < CORE_MAX_NT; ++nt) {
    const int n = nt * 16 + li;
    prow[nt] = n < a.N ? n : a.N - 1;
  }
  float cs = 0.f;
  const int steps = (int)(Mp / 4);
  for (int t0 = wid; t0 < steps; t0 += 8) {   // two steps per round, both loads issued first
    float vv[2], pv[2][CORE_MAX_NT];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int t = t0 + 4 * u;
      const int m = 4 * t + g;
      const bool live = t < steps && m < a.M;
      vv[u] = live ? vb[(int64_t)m * a.ldv] : 0.f;
#pragma unroll
      for (int nt = 0; nt < CORE_MAX_NT; ++nt)
        pv[u][nt] = (nt < a.NT && t < steps) ? pb[(int64_t)prow[nt] * Mp + m] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      cs += vv[u];
#pragma unroll
      for (int nt = 0; nt < CORE_MAX_NT; ++nt)
        if (nt < a.NT) acc[nt] = A::mfma(pv[u][nt], vv[u], acc[nt]);
    }
  }
  cs = rows4_sum(cs);
  if (g == 0) csum[wid][li] = cs;
#pragma unroll
  for (int nt = 0; nt < CORE_MAX_NT; ++nt)
    if (nt < a.NT)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[wid][nt][r][lane] = acc[nt][r];
  __syncthreads();
  if (d >= a.D) return;
  const float epsv = renorm ? a.renorm_eps * (csum[0][li] + csum[1][li] + csum[2][li] + csum[3][li]) : 0.f;
  // outputs (slot n, column d): wave w takes slot tiles w, w + 4, ...
  for (int nt = wid; nt < a.NT; nt += 4) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int n = nt * 16 + 4 * g + r;
      if (n < a.N) {
        const float sacc = red[0][nt][r][lane] + red[1][nt][r][lane] + red[2][nt][r][lane] + red[3][nt][r][lane];
        out[b * a.ob + (int64_t)n * a.ldo + d] = (sacc + epsv) * rinv[n];
      }
    }
  }
}

// Fused attention core for the iteration (16-bit operands, v given transposed per frame: vt[b][d][Mp]), one launch
// per iteration: grid (frame, column block of D / NCB columns), 8 waves.  Each column block of a frame recomputes
// the frame's logits and softmax (k is read from L2 by the frame's NCB workgroups), so the probabilities never leave
// the workgroup and no second launch or global round trip is needed.  Every global load of the kernel is issued at
// its start -- the wave's k tiles, its v^T column tiles and q (staged in LDS) -- so the kernel waits on memory once:
// measured on MI355X, each dependent round of global loads costs ~1.5 us here, more than the arithmetic.
//   phase 1 wave w: token tiles w and w + 8: S = q k^T as NT MFMA tiles (slots as rows, 16 tokens as columns),
//           softmax over the slots of each token column in registers (the NT*4 values of a lane, then the four lane
//           groups), P (zero for tokens m >= M) to LDS, per-slot sums of P for the renormalisation.
//   phase 2 wave w: column tiles w, w + 8, ... of the block for every slot: P (A operand, LDS) times the v^T rows
//           held in registers (tokens m >= M zeroed); epilogue (acc + eps sum_m v) / (sum_m P + M eps).
// Limits: M <= 256 (two token tiles per wave, eight 32-token blocks of v^T).
constexpr int CF_WAVES = 8;
constexpr int CF_MAXM = 256;

//
// With LNQ the query side is formed in the kernel: `q` is unused, the workgroup reads its frame's fp32 slot rows
// (ln.s), takes their LayerNorm (two-pass mean and variance over a wave per row) into the LDS tile that holds q
// otherwise, and `k` holds k Wq (the keys already multiplied by the query weight): (LN(s) Wq^T) k^T = LN(s) (k Wq)^T,
// so the iteration needs no q projection.  ln.sb_out (nullable) receives the slot rows in the operand type (the
// column-block-0 workgroup of each frame writes them).
struct LnqArgs {
  const float* s;        // [B][N][D] slot rows: row stride ld, frame stride fb
  int64_t ld, fb;
  const float* w;        // LayerNorm gamma / beta (nullable)
  const float* b;
  float eps;
  void* sb_out;          // [B][N][D] in the operand type: row stride ldsb, frame stride sbb (nullable)
  int64_t ldsb, sbb;
  const void* whh;       // GH: GRU hidden weights [3D][D] (operand type)
  float* gh;             // GH: s W_hh^T, [B][N][3D] fp32 (row stride 3D), without the bias
};

// With GH (LNQ only) the workgroup also forms the GRU's hidden-side product for its frame's rows and its column
// block of each of the three gates, s W_hh^T with s the slot rows in the operand type (the same operand the GRU
// would multiply): phase 3, after attn.V, from the slot rows written to the q tile once the logits are done.
template <int DT, int NT, int DD, int NCB, bool LNQ, bool GH>
__global__ void __launch_bounds__(64 * CF_WAVES)
core_fused_t_kernel(const typename MM<DT>::T* __restrict__ q, const typename MM<DT>::T* __restrict__ k,
                    const typename MM<DT>::T* __restrict__ vt, int64_t Mp, typename MM<DT>::T* __restrict__ out,
                    CoreArgs a, LnqArgs ln) {
  using A = MM<DT>;
  using TT = typename A::T;
  static_assert(A::KPL == 8 && DD % (16 * NCB) == 0, "16-bit operands, whole 16-column tiles per block");
  constexpr int NW = CF_WAVES, NKB = DD / 32, NS = NT * 16, QP = DD + 8, NCT = DD / NCB / 16;
  constexpr int CTW = (NCT + NW - 1) / NW, TPW = CF_MAXM / 16 / NW, VB = CF_MAXM / 32;
  extern __shared__ __align__(16) unsigned char smem[];
  TT* sq = reinterpret_cast<TT*>(smem);                                  // [NS][QP]
  TT* sp = sq + NS * QP;                                                 // [NS][Mp + 8] probabilities
  float* srs = reinterpret_cast<float*>(sp + (size_t)NS * (Mp + 8));     // [NW][NS] per-wave sums of P
  const int PP = (int)Mp + 8;
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63, g = lane >> 4, li = lane & 15;
  const int MT = (int)((a.M + 15) / 16), MPT = (int)(Mp / 16), NVB = (int)(Mp / 32);
  // ---- every global load first: k tiles, v^T column tiles, q
  const TT* kf = k + b * a.kb;
  uint4 kr[TPW][NKB];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int t = wid + NW * j;
    if (t < MT) {
      int m = t * 16 + li;
      m = m < a.M ? m : a.M - 1;
      const TT* kp = kf + (int64_t)m * a.ldk + 8 * g;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) kr[j][kb] = *reinterpret_cast<const uint4*>(kp + 32 * kb);
    }
  }
  uint4 vr[CTW][VB];
#pragma unroll
  for (int c = 0; c < CTW; ++c) {
    const int ct = wid + NW * c;
    if (ct < NCT) {
      const TT* vp = vt + b * a.vb + (int64_t)(blockIdx.y * (DD / NCB) + ct * 16 + li) * Mp + 8 * g;
#pragma unroll
      for (int i = 0; i < VB; ++i)
        if (i < NVB) vr[c][i] = *reinterpret_cast<const uint4*>(vp + 32 * i);
    }
  }
  static_assert(!GH || LNQ, "the hidden-side product takes the slot rows of the LNQ form");
  constexpr int EPL = DD / 64, RPW = NS / NW;
  TT xh[GH ? RPW : 1][GH ? EPL : 1];   // GH: the slot rows in the operand type, written to sq after phase 1
  if constexpr (LNQ) {
    // LayerNorm of the frame's slot rows into sq: wave w takes rows w, w + NW, ...; lane l holds elements
    // l + 64 e.  Rows n >= N repeat row N - 1 (their logits are masked).
    static_assert(DD % 64 == 0 && NS % NW == 0, "whole rows per wave");
    float xs[RPW][EPL];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const int n = wid + NW * r;
      const int nc = n < a.N ? n : a.N - 1;
      const float* sp_ = ln.s + b * ln.fb + (int64_t)nc * ln.ld + lane;
#pragma unroll
      for (int e = 0; e < EPL; ++e) xs[r][e] = sp_[64 * e];
    }
    float gw[EPL], gb[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      gw[e] = ln.w ? ln.w[lane + 64 * e] : 1.f;
      gb[e] = ln.b ? ln.b[lane + 64 * e] : 0.f;
    }
    TT* sbo = (ln.sb_out != nullptr && blockIdx.y == 0) ? reinterpret_cast<TT*>(ln.sb_out) + b * ln.sbb : nullptr;
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const int n = wid + NW * r;
      float s1 = 0.f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) s1 += xs[r][e];
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) s1 += __shfl_xor(s1, o, 64);
      const float mean = s1 * (1.f / (float)DD);
      float s2 = 0.f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const float dv = xs[r][e] - mean;
        s2 += dv * dv;
      }
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) s2 += __shfl_xor(s2, o, 64);
      const float rstd = 1.f / sqrtf(s2 * (1.f / (float)DD) + ln.eps);
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        sq[n * QP + lane + 64 * e] = A::fromf((xs[r][e] - mean) * rstd * gw[e] + gb[e]);
        if (sbo != nullptr && n < a.N) sbo[(int64_t)n * ln.ldsb + lane + 64 * e] = A::fromf(xs[r][e]);
        if constexpr (GH) xh[r][e] = A::fromf(xs[r][e]);
      }
    }
  } else {
    for (int u = tid; u < NS * (DD / 8); u += 64 * NW) {   // rows n >= N repeat row N - 1 (their logits are masked)
      const int n = u / (DD / 8), c = (u - n * (DD / 8)) * 8;
      const int nc = n < a.N ? n : a.N - 1;
      *reinterpret_cast<uint4*>(sq + n * QP + c) =
          *reinterpret_cast<const uint4*>(q + b * a.qb + (int64_t)nc * a.ldq + c);
    }
  }
  __syncthreads();
  // ---- phase 1: logits, softmax over slots, P to LDS
  float rs[NT][4];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int r = 0; r < 4; ++r) rs[nt][r] = 0.f;
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int t = wid + NW * j;
    if (t >= MPT) break;
    const int m = t * 16 + li;
    if (t >= MT) {   // the padding tile past the last token tile: zero probabilities
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int r = 0; r < 4; ++r) sp[(nt * 16 + 4 * g + r) * PP + m] = A::fromf(0.f);
      continue;
    }
    f32x4 acc[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      const typename A::Op kv = __builtin_bit_cast(typename A::Op, kr[j][kb]);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)   // acc[nt][r] = logit[n = 16nt + 4g + r][m]
        acc[nt] = A::mfma(A::load(sq + (nt * 16 + li) * QP + 32 * kb + 8 * g), kv, acc[nt]);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float sv = acc[nt][r] * a.scale;
        if (a.logit_clamp > 0.f) sv = fminf(fmaxf(sv, -a.logit_clamp), a.logit_clamp);
        sv = (nt * 16 + 4 * g + r < a.N) ? sv : -INFINITY;
        acc[nt][r] = sv;
        mx = fmaxf(mx, sv);
      }
    mx = rows4_max(mx);
    float sum = 0.f;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float e = __expf(acc[nt][r] - mx);
        acc[nt][r] = e;
        sum += e;
      }
    sum = rows4_sum(sum);
    const float inv = m < a.M ? 1.f / (sum + a.denom_eps) : 0.f;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float pv = acc[nt][r] * inv;
        rs[nt][r] += pv;
        sp[(nt * 16 + 4 * g + r) * PP + m] = A::fromf(pv);
      }
  }
  // per-slot sums over this wave's tokens (the 16 lanes of a lane group hold 16 tokens)
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v = rs[nt][r];
      v += __shfl_xor(v, 1, 64);
      v += __shfl_xor(v, 2, 64);
      v += __shfl_xor(v, 4, 64);
      v += __shfl_xor(v, 8, 64);
      if (li == 0) srs[wid * NS + nt * 16 + 4 * g + r] = v;
    }
  __syncthreads();
  // GH: the logits are done with sq; it now takes the slot rows, and the W_hh rows of this wave's gate column tiles
  // are requested before phase 2 so that they arrive while it runs.
  constexpr int GCB = DD / NCB, GT = GH ? 3 * GCB / 16 : 0, GPW = GH ? (GT + NW - 1) / NW : 1;
  uint4 wr[GPW][GH ? NKB : 1];
  if constexpr (GH) {
    static_assert((3 * GCB) % 16 == 0 && GCB % 16 == 0, "whole 16-column gate tiles");
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
      for (int e = 0; e < EPL; ++e) sq[(wid + NW * r) * QP + lane + 64 * e] = xh[r][e];
    const TT* whh = reinterpret_cast<const TT*>(ln.whh);
#pragma unroll
    for (int c = 0; c < GPW; ++c) {
      const int ct = wid + NW * c;
      if (ct < GT) {
        const int j = (ct / (GCB / 16)) * DD + blockIdx.y * GCB + (ct % (GCB / 16)) * 16 + li;
        const TT* wp = whh + (int64_t)j * DD + 8 * g;
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) wr[c][kb] = *reinterpret_cast<const uint4*>(wp + 32 * kb);
      }
    }
  }
  // ---- phase 2: this wave's column tiles
  const bool renorm = a.renorm_eps >= 0.f;
  float rinv[NT][4];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float t = (float)a.M * a.renorm_eps;
#pragma unroll
      for (int w = 0; w < NW; ++w) t += srs[w * NS + nt * 16 + 4 * g + r];
      rinv[nt][r] = renorm ? 1.f / t : 1.f;
    }
#pragma unroll
  for (int c = 0; c < CTW; ++c) {
    const int ct = wid + NW * c;
    if (ct >= NCT) break;
    const int d = blockIdx.y * (DD / NCB) + ct * 16 + li;
    f32x4 acc[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float cs = 0.f;
#pragma unroll
    for (int i = 0; i < VB; ++i) {
      if (i >= NVB) break;
      const int m0 = 32 * i;
      uint4 raw = vr[c][i];
      if (m0 + 32 > a.M) {   // tokens past M: v^T columns are not initialised, zero them
        TT e[8];
        *reinterpret_cast<uint4*>(e) = raw;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj)
          if (m0 + 8 * g + jj >= a.M) e[jj] = A::fromf(0.f);
        raw = *reinterpret_cast<uint4*>(e);
      }
      if (renorm) {
        TT e[8];
        *reinterpret_cast<uint4*>(e) = raw;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) cs += A::tof(e[jj]);
      }
      const typename A::Op bv = __builtin_bit_cast(typename A::Op, raw);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) acc[nt] = A::mfma(A::load(sp + (nt * 16 + li) * PP + m0 + 8 * g), bv, acc[nt]);
    }
    cs = rows4_sum(cs);
    const float epsv = renorm ? a.renorm_eps * cs : 0.f;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = nt * 16 + 4 * g + r;
        if (n < a.N) out[b * a.ob + (int64_t)n * a.ldo + d] = A::fromf((acc[nt][r] + epsv) * rinv[nt][r]);
      }
  }
  if constexpr (GH) {
    // ---- phase 3: gh[n][j] = sum_i s[n][i] W_hh[j][i] for this wave's gate column tiles
    __syncthreads();
#pragma unroll
    for (int c = 0; c < GPW; ++c) {
      const int ct = wid + NW * c;
      if (ct >= GT) break;
      const int j = (ct / (GCB / 16)) * DD + blockIdx.y * GCB + (ct % (GCB / 16)) * 16 + li;
      f32x4 acc[NT];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        const typename A::Op bq = __builtin_bit_cast(typename A::Op, wr[c][kb]);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[nt] = A::mfma(A::load(sq + (nt * 16 + li) * QP + 32 * kb + 8 * g), bq, acc[nt]);
      }
      float* ghf = ln.gh + b * (int64_t)a.N * (3 * DD);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int n = nt * 16 + 4 * g + r;
          if (n < a.N) ghf[(int64_t)n * (3 * DD) + j] = acc[nt][r];
        }
    }
  }
}

static size_t core_fused_lds(int NT, int64_t D, int64_t Mp, int esize) {
  return ((size_t)NT * 16 * (D + 8) + (size_t)NT * 16 * (Mp + 8)) * esize + (size_t)CF_WAVES * NT * 16 * 4;
}

static bool al16(const void* p) { return (((uintptr_t)p) & 15) == 0; }

static size_t core_ws_bytes(int64_t B, int64_t N, int64_t M, int esize) {
  const int64_t Mp = (M + 31) / 32 * 32, MT = (M + 15) / 16;
  size_t p = (size_t)B * N * Mp * esize;
  p = (p + 255) / 256 * 256;
  return p + (size_t)B * MT * N * 4;
}

// attn @ v with v in place (not transposed): the narrow-grid fp32 kernel when the 64-column grid would fill fewer
// than half of a 256-CU device, else core_update_kernel.
template <int DT>
static void launch_update_plain(const typename MM<DT>::T* P, int64_t Mp, const float* part, const typename MM<DT>::T* v,
                                typename MM<DT>::T* out, const CoreArgs& a, int64_t B, int64_t D, dim3 g2,
                                hipStream_t st) {
  if constexpr (DT == HCLSM_F32) {
    if (B * ((D + CORE_DB - 1) / CORE_DB) < 128) {
      hipLaunchKernelGGL(core_update_narrow_kernel, dim3((unsigned)B, (unsigned)((D + 15) / 16)), dim3(256), 0, st, P,
                         Mp, part, v, out, a);
      return;
    }
  }
  hipLaunchKernelGGL((core_update_kernel<DT>), g2, dim3(256), 0, st, P, Mp, part, v, out, a);
}

static int launch_core(const void* q, int64_t ldq, int64_t qbs, const void* k, int64_t ldk, int64_t kbs,
                       const void* v, int64_t ldv, int64_t vbs, void* out, int64_t ldo, int64_t obs, void* attn,
                       int attn_dtype, int64_t B, int64_t N, int64_t M, int64_t D, float scale, float denom_eps,
                       float logit_clamp, float renorm_eps, int dtype, void* ws, hipStream_t st,
                       bool v_transposed = false) {
  CoreArgs a;
  a.ldq = ldq; a.ldk = ldk; a.ldv = ldv; a.ldo = ldo;
  a.qb = qbs; a.kb = kbs; a.vb = vbs; a.ob = obs;
  a.N = (int)N; a.M = (int)M; a.D = (int)D;
  a.NT = (int)((N + 15) / 16);
  a.MT = (int)((M + 15) / 16);
  a.scale = scale; a.denom_eps = denom_eps; a.logit_clamp = logit_clamp; a.renorm_eps = renorm_eps;
  const int64_t Mp = (M + 31) / 32 * 32;
  const int esize = dtype == HCLSM_F32 ? 4 : 2;
  size_t poff = (size_t)B * N * Mp * esize;
  poff = (poff + 255) / 256 * 256;
  float* part = reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + poff);
  dim3 g1((unsigned)B, (unsigned)(Mp / 16));
  dim3 g2((unsigned)B, (unsigned)((D + CORE_DB - 1) / CORE_DB));
#define HCLSM_CORE(D_, A_)                                                                                   \
  if (dtype == D_ && (attn == nullptr ? A_ == D_ : attn_dtype == A_)) {                                      \
    if (D_ == HCLSM_F32 && B * (Mp / 16) < 128)                                                              \
      hipLaunchKernelGGL((core_logits_kernel<D_, A_, 8>), g1, dim3(512), 0, st, (const MM<D_>::T*)q,         \
                         (const MM<D_>::T*)k, (MM<D_>::T*)ws, Mp, part, (MM<A_>::T*)attn, a);                \
    else                                                                                                     \
      hipLaunchKernelGGL((core_logits_kernel<D_, A_>), g1, dim3(256), 0, st, (const MM<D_>::T*)q,           \
                         (const MM<D_>::T*)k, (MM<D_>::T*)ws, Mp, part, (MM<A_>::T*)attn, a);                \
    HCLSM_LAUNCH_CHECK();                                                                                    \
    if (v_transposed)                                                                                        \
      hipLaunchKernelGGL((core_update_t_kernel<D_>), g2, dim3(256), 0, st, (const MM<D_>::T*)ws, Mp, part,   \
                         (const MM<D_>::T*)v, (MM<D_>::T*)out, a);                                           \
    else                                                                                                     \
      launch_update_plain<D_>((const MM<D_>::T*)ws, Mp, part, (const MM<D_>::T*)v, (MM<D_>::T*)out, a, B, D, g2, st); \
    HCLSM_LAUNCH_CHECK();                                                                                    \
    return 0;                                                                                                \
  }
  HCLSM_CORE(HCLSM_BF16, HCLSM_BF16)
  HCLSM_CORE(HCLSM_BF16, HCLSM_F32)
  HCLSM_CORE(HCLSM_F16, HCLSM_F16)
  HCLSM_CORE(HCLSM_F16, HCLSM_F32)
  HCLSM_CORE(HCLSM_F32, HCLSM_F32)
#undef HCLSM_CORE
  return HCLSM_ERR_DTYPE;
}

// The fused core (16-bit operands, v transposed) when the shape fits its instantiations; 1 otherwise.  Column
// blocks per frame: eight 48-column blocks for D = 384 (config 2: 256 workgroups, one per CU; each block
// recomputes the frame's logits, and against three 128-column blocks the wider grid still wins by ~2.5 us per
// forward), 128-column blocks for D = 256, one block for D = 192 / 128.
// Column blocks per frame of the fused core for D (the launcher's instantiations).
static constexpr int cf_ncb(int64_t D) { return D == 384 ? 8 : D == 256 ? 2 : 1; }
// The GH form holds each wave's W_hh tiles in registers: at most two 16-column gate tiles per wave.
static constexpr bool cf_gh_fits(int64_t D, int ncb) { return (3 * D / ncb / 16 + CF_WAVES - 1) / CF_WAVES <= 2; }

static bool core_fused_fits(int64_t B, int64_t N, int64_t M, int64_t D, int dtype) {
  if (dtype != HCLSM_BF16 && dtype != HCLSM_F16) return false;
  if (N < 1 || N > 32 || M < 1 || M > CF_MAXM || (D != 128 && D != 192 && D != 256 && D != 384)) return false;
  if (B > 65535) return false;
  return core_fused_lds(N <= 16 ? 1 : 2, D, (M + 31) / 32 * 32, 2) <= 64 * 1024;
}

// lnq (nullable): the LNQ form (q formed in the kernel from the slot rows; k holds k Wq).
static int launch_core_fused(const void* q, int64_t ldq, int64_t qbs, const void* k, int64_t ldk, int64_t kbs,
                             const void* vt, int64_t vbs, void* out, int64_t ldo, int64_t obs, int64_t B, int64_t N,
                             int64_t M, int64_t D, float scale, float denom_eps, float logit_clamp, float renorm_eps,
                             int dtype, hipStream_t st, const LnqArgs* lnq = nullptr) {
  if (!core_fused_fits(B, N, M, D, dtype)) return 1;
  const int NT = N <= 16 ? 1 : 2;
  const int64_t Mp = (M + 31) / 32 * 32;
  const size_t lds = core_fused_lds(NT, D, Mp, 2);
  const LnqArgs ln = lnq ? *lnq : LnqArgs{nullptr, 0, 0, nullptr, nullptr, 0.f, nullptr, 0, 0, nullptr, nullptr};
  CoreArgs a;
  a.ldq = ldq; a.ldk = ldk; a.ldv = 0; a.ldo = ldo;
  a.qb = qbs; a.kb = kbs; a.vb = vbs; a.ob = obs;
  a.N = (int)N; a.M = (int)M; a.D = (int)D;
  a.NT = NT;
  a.MT = (int)((M + 15) / 16);
  a.scale = scale; a.denom_eps = denom_eps; a.logit_clamp = logit_clamp; a.renorm_eps = renorm_eps;
#define HCLSM_CF(DT_, NT_, DD_, NCB_)                                                                           \
  if (dtype == DT_ && NT == NT_ && D == DD_) {                                                                 \
    if (lnq && ln.gh) {                                                                                        \
      if constexpr (cf_gh_fits(DD_, NCB_))                                                                     \
        hipLaunchKernelGGL((core_fused_t_kernel<DT_, NT_, DD_, NCB_, true, true>), dim3((unsigned)B, NCB_),    \
                           dim3(64 * CF_WAVES), lds, st, (const MM<DT_>::T*)q, (const MM<DT_>::T*)k,          \
                           (const MM<DT_>::T*)vt, Mp, (MM<DT_>::T*)out, a, ln);                                \
      else                                                                                                     \
        return 1;                                                                                              \
    } else if (lnq)                                                                                            \
      hipLaunchKernelGGL((core_fused_t_kernel<DT_, NT_, DD_, NCB_, true, false>), dim3((unsigned)B, NCB_),     \
                         dim3(64 * CF_WAVES), lds, st, (const MM<DT_>::T*)q, (const MM<DT_>::T*)k,            \
                         (const MM<DT_>::T*)vt, Mp, (MM<DT_>::T*)out, a, ln);                                  \
    else                                                                                                       \
      hipLaunchKernelGGL((core_fused_t_kernel<DT_, NT_, DD_, NCB_, false, false>), dim3((unsigned)B, NCB_),    \
                         dim3(64 * CF_WAVES), lds, st, (const MM<DT_>::T*)q, (const MM<DT_>::T*)k,            \
                         (const MM<DT_>::T*)vt, Mp, (MM<DT_>::T*)out, a, ln);                                  \
    HCLSM_LAUNCH_CHECK();                                                                                      \
    return 0;                                                                                                  \
  }
#define HCLSM_CF_D(DT_, NT_) \
  HCLSM_CF(DT_, NT_, 128, cf_ncb(128)) HCLSM_CF(DT_, NT_, 192, cf_ncb(192)) HCLSM_CF(DT_, NT_, 256, cf_ncb(256)) \
  HCLSM_CF(DT_, NT_, 384, cf_ncb(384))
  HCLSM_CF_D(HCLSM_BF16, 1) HCLSM_CF_D(HCLSM_BF16, 2)
  HCLSM_CF_D(HCLSM_F16, 1) HCLSM_CF_D(HCLSM_F16, 2)
#undef HCLSM_CF_D
#undef HCLSM_CF
  return 1;
}

static int check_core(const void* q, int64_t ldq, int64_t qbs, const void* k, int64_t ldk, int64_t kbs, int64_t B,
                      int64_t N, int64_t M, int64_t D, int dtype) {
  if (B < 0 || N < 0 || M < 0 || D < 0 || B > 65535 || M > (1 << 20)) return HCLSM_ERR_SHAPE;
  if (N > 16 * CORE_MAX_NT) return HCLSM_ERR_UNSUPPORTED;
  if (dtype != HCLSM_BF16 && dtype != HCLSM_F16 && dtype != HCLSM_F32) return HCLSM_ERR_DTYPE;
  const int kpl = dtype == HCLSM_F32 ? 1 : 8;
  if (D % (4 * kpl) || D % 16) return HCLSM_ERR_UNSUPPORTED;
  if (kpl == 8 && (!al16(q) || !al16(k) || ldq % 8 || ldk % 8 || qbs % 8 || kbs % 8)) return HCLSM_ERR_UNSUPPORTED;
  return 0;
}

template <int DT, int OT, typename XT>
static void launch_linear_quad(const void* x, int64_t ldx, const void* w, int64_t ldw, const float* bias,
                               const float* resid, int64_t ldr, void* y, int64_t ldy, void* y2, int64_t ldy2,
                               int64_t M, int64_t N, int64_t K, int relu, float clamp, hipStream_t st,
                               OutSplit os = OutSplit{0, 1, 0, 0, nullptr}, LinExt ext = kNoLinExt) {
  constexpr bool direct = std::is_same_v<XT, typename MM<DT>::T>;
  // fp32 X with 16-bit operands: the LDS kernels round X while staging it (callers check 16-byte rows)
  constexpr bool cvt = MM<DT>::KPL == 8 && std::is_same_v<XT, float>;
  if constexpr (direct || cvt) {
    const unsigned grid = (unsigned)(((M + 63) / 64) * ((N + 63) / 64));
    const int64_t tiles128 = ((M + 127) / 128) * ((N + 127) / 128);
    if constexpr (MM<DT>::KPL == 8) {
      // 16-bit X with 16-byte rows and K in 64-wide chunks: the direct-to-LDS kernel (a transposed part must
      // start on a 128-column tile)
      // narrow layers (N <= 512) behind a device-side row count: the direct-to-LDS kernel (measured faster there
      // than the 64x64 tiles; wider layers and host-side row counts measured no faster or slower with it)
      const bool dma = direct && ext.m_dev != nullptr && os.yt == nullptr && K % LD_KC == 0 && al16(x) &&
                       ldx % 8 == 0 && N >= 256 && N <= 512;
      if (dma) {
        if constexpr (direct)
          hipLaunchKernelGGL((linear_dma_kernel<DT, OT>), dim3((unsigned)tiles128), dim3(256), 0, st,
                             (const typename MM<DT>::T*)x, ldx, (const typename MM<DT>::T*)w, ldw, bias, resid, ldr,
                             (typename MM<OT>::T*)y, ldy, (typename MM<DT>::T*)y2, ldy2, M, N, K, relu, clamp, os,
                             ext);
      } else if (os.yt == nullptr && N >= 768 && tiles128 >= 512)
        hipLaunchKernelGGL((linear_lds128_kernel<DT, OT, XT>), dim3((unsigned)tiles128), dim3(256), 0, st,
                           (const XT*)x, ldx, (const typename MM<DT>::T*)w, ldw, bias, resid, ldr,
                           (typename MM<OT>::T*)y, ldy, (typename MM<DT>::T*)y2, ldy2, M, N, K, relu, clamp, ext);
      else
        hipLaunchKernelGGL((linear_lds_kernel<DT, OT, XT, false, 64>), dim3(grid), dim3(256), 0, st, (const XT*)x,
                           ldx, (const typename MM<DT>::T*)w, ldw, bias, resid, ldr, (typename MM<OT>::T*)y, ldy,
                           (typename MM<DT>::T*)y2, ldy2, M, N, K, relu, clamp, os, ext);
    } else if constexpr (direct) {
      if (os.yt == nullptr && al16(x) && al16(w) && ldx % 4 == 0 && ldw % 4 == 0)
        hipLaunchKernelGGL((linear_lds_f32_kernel<OT>), dim3(grid), dim3(256), 0, st, (const float*)x, ldx,
                           (const float*)w, ldw, bias, resid, ldr, (typename MM<OT>::T*)y, ldy, (float*)y2, ldy2, M,
                           N, K, relu, clamp, ext);
      else
        hipLaunchKernelGGL((linear_quad_kernel<DT, OT>), dim3(grid), dim3(256), 0, st, (const typename MM<DT>::T*)x,
                           ldx, (const typename MM<DT>::T*)w, ldw, bias, resid, ldr, (typename MM<OT>::T*)y, ldy,
                           (typename MM<DT>::T*)y2, ldy2, M, N, K, relu, clamp, os, ext);
    }
  }
}

// linear_kreg_kernel with KB = the smallest instantiated count of blocks per wave covering K; false
// (nothing launched) past the largest.
template <int DT, int OT, typename XT, bool LN, bool FOLD = false>
static bool launch_linear_kreg(const void* x, int64_t ldx, const void* w, int64_t ldw, const float* bias,
                               const float* resid, int64_t ldr, void* y, int64_t ldy, void* y2, int64_t ldy2,
                               int64_t M, int64_t N, int64_t K, int relu, float clamp, const float* lnw,
                               const float* lnb, float eps, void* xout, int64_t ldxo, hipStream_t st,
                               const float* fsum = nullptr) {
  const int64_t nblk = K / 32;
  const int need = (int)((nblk + 3) / 4);
  const unsigned grid = (unsigned)(((M + 31) / 32) * ((N + 31) / 32));
  using TT = typename MM<DT>::T;
#define HCLSM_KREG(KBV)                                                                                      \
  if (need <= KBV) {                                                                                         \
    hipLaunchKernelGGL((linear_kreg_kernel<DT, OT, XT, LN, KBV, FOLD>), dim3(grid), dim3(256), 0, st,        \
                       (const XT*)x, ldx, (const TT*)w, ldw, bias, resid, ldr, (typename MM<OT>::T*)y, ldy,   \
                       (TT*)y2, ldy2, M, N, K, relu, clamp, lnw, lnb, eps, (TT*)xout, ldxo, fsum);           \
    return true;                                                                                             \
  }
  HCLSM_KREG(1) HCLSM_KREG(2) HCLSM_KREG(3)
  if constexpr (!LN) {   // with LN the raw rows, gamma and beta stay in registers too: K <= 384 only
    HCLSM_KREG(4) HCLSM_KREG(6) HCLSM_KREG(8)
  }
#undef HCLSM_KREG
  return false;
}

template <int DT, int OT, typename XT>
static void launch_linear_t(bool ln, const void* x, int64_t ldx, const void* w, int64_t ldw, const float* bias,
                            const float* resid, int64_t ldr, void* y, int64_t ldy, void* y2, int64_t ldy2, int64_t M,
                            int64_t N, int64_t K, int relu, float clamp, const float* lnw, const float* lnb,
                            float eps, hipStream_t st, LinExt ext = kNoLinExt, void* xout = nullptr,
                            int64_t ldxo = 0) {
  const int64_t tiles32 = ((M + 31) / 32) * ((N + 31) / 32);
  constexpr bool cvt = MM<DT>::KPL == 8 && std::is_same_v<XT, float>;
  if (!ln && (std::is_same_v<XT, typename MM<DT>::T> || (cvt && al16(x) && ldx % 4 == 0)) && tiles32 >= 2048) {
    launch_linear_quad<DT, OT, XT>(x, ldx, w, ldw, bias, resid, ldr, y, ldy, y2, ldy2, M, N, K, relu, clamp, st,
                                   OutSplit{0, 1, 0, 0, nullptr}, ext);
    return;
  }
  // 16-bit operands, K <= 1024, no device-side row count or gate: every K block in flight at once
  if constexpr (MM<DT>::KPL == 8) {
    const bool xok = std::is_same_v<XT, float> ? (al16(x) && ldx % 4 == 0) : (al16(x) && ldx % 8 == 0);
    const bool lnok = !ln || ((lnw == nullptr || al16(lnw)) && (lnb == nullptr || al16(lnb)));
    const bool xo_ok = xout == nullptr || (ln && al16(xout) && ldxo % 8 == 0);
    if (ext.m_dev == nullptr && ext.glu == nullptr && K <= 1024 && xok && lnok && xo_ok) {
      const bool done = ln ? launch_linear_kreg<DT, OT, XT, true>(x, ldx, w, ldw, bias, resid, ldr, y, ldy, y2, ldy2, M,
                                                                 N, K, relu, clamp, lnw, lnb, eps, xout, ldxo, st)
                           : launch_linear_kreg<DT, OT, XT, false>(x, ldx, w, ldw, bias, resid, ldr, y, ldy, y2, ldy2,
                                                                  M, N, K, relu, clamp, lnw, lnb, eps, nullptr, 0, st);
      if (done) return;
    }
  }
  const unsigned grid = (unsigned)tiles32;
  if (ln)
    hipLaunchKernelGGL((linear_kernel<DT, OT, XT, true>), dim3(grid), dim3(256), 0, st, (const XT*)x, ldx,
                       (const typename MM<DT>::T*)w, ldw, bias, resid, ldr, (typename MM<OT>::T*)y, ldy,
                       (typename MM<DT>::T*)y2, ldy2, M, N, K, relu, clamp, lnw, lnb, eps, ext);
  else
    hipLaunchKernelGGL((linear_kernel<DT, OT, XT, false>), dim3(grid), dim3(256), 0, st, (const XT*)x, ldx,
                       (const typename MM<DT>::T*)w, ldw, bias, resid, ldr, (typename MM<OT>::T*)y, ldy,
                       (typename MM<DT>::T*)y2, ldy2, M, N, K, relu, clamp, lnw, lnb, eps, ext);
}

static int linear_impl(const void* x, int64_t ldx, int x_dtype, const void* w, int64_t ldw, const float* bias,
                       const float* resid, int64_t ldr, void* y, int64_t ldy, int y_dtype, void* y2, int64_t ldy2,
                       int64_t M, int64_t N, int64_t K, int relu, float clamp, int ln, const float* lnw,
                       const float* lnb, float ln_eps, int dtype, hipStream_t st, LinExt ext = kNoLinExt,
                       void* xout = nullptr, int64_t ldxo = 0) {
  if (M < 0 || N < 0 || K < 0) return HCLSM_ERR_SHAPE;
  if (M == 0 || N == 0) return 0;
  if (!x || !w || !y) return HCLSM_ERR_NULL;
  const int kpl = dtype == HCLSM_F32 ? 1 : 8;
  if (K % (4 * kpl) != 0 || K == 0) return HCLSM_ERR_UNSUPPORTED;
  if (kpl == 8 && (!al16(w) || ldw % 8)) return HCLSM_ERR_UNSUPPORTED;
  if (kpl == 8 && x_dtype == dtype && (!al16(x) || ldx % 8)) return HCLSM_ERR_UNSUPPORTED;
  const bool LNf = ln != 0;
#define HCLSM_LIN(D, O, XD, XT)                                                                              \
  if (dtype == D && y_dtype == O && x_dtype == XD) {                                                         \
    launch_linear_t<D, O, XT>(LNf, x, ldx, w, ldw, bias, resid, ldr, y, ldy, y2, ldy2, M, N, K, relu, clamp, lnw, \
                              lnb, ln_eps, st, ext, xout, ldxo);                                             \
    HCLSM_LAUNCH_CHECK();                                                                                    \
    return 0;                                                                                                \
  }
  HCLSM_LIN(HCLSM_BF16, HCLSM_BF16, HCLSM_BF16, uint16_t)
  HCLSM_LIN(HCLSM_BF16, HCLSM_F32, HCLSM_BF16, uint16_t)
  HCLSM_LIN(HCLSM_BF16, HCLSM_BF16, HCLSM_F32, float)
  HCLSM_LIN(HCLSM_BF16, HCLSM_F32, HCLSM_F32, float)
  HCLSM_LIN(HCLSM_F16, HCLSM_F16, HCLSM_F16, _Float16)
  HCLSM_LIN(HCLSM_F16, HCLSM_F32, HCLSM_F16, _Float16)
  HCLSM_LIN(HCLSM_F16, HCLSM_F16, HCLSM_F32, float)
  HCLSM_LIN(HCLSM_F16, HCLSM_F32, HCLSM_F32, float)
  HCLSM_LIN(HCLSM_F32, HCLSM_F32, HCLSM_F32, float)
#undef HCLSM_LIN
  return HCLSM_ERR_DTYPE;
}

// Linear layer with a device-side row count and an optional gated-linear epilogue, for composite
// entry points in other files (declared in internal.h).
int linear_rows(const void* x, int64_t ldx, int x_dtype, const void* w, int64_t ldw, const float* bias,
                const float* resid, int64_t ldr, void* y, int64_t ldy, int y_dtype, int64_t M, int64_t N, int64_t K,
                int ln, int relu, const float* ln_w, const float* ln_b, float ln_eps, const void* glu, int64_t ldg,
                const int32_t* m_dev, int64_t m_mul, int dtype, hipStream_t st) {
  if (glu && (x_dtype != dtype && x_dtype != HCLSM_F32)) return HCLSM_ERR_DTYPE;
  return linear_impl(x, ldx, x_dtype, w, ldw, bias, resid, ldr, y, ldy, y_dtype, nullptr, 0, M, N, K, relu, 0.f, ln,
                     ln_w, ln_b, ln_eps, dtype, st, LinExt{m_dev, m_mul, glu, ldg});
}

// Declared in internal.h.
int qkv_attn_rows(const void* x, const void* w, void* o, const int32_t* n_events, int64_t capacity, int64_t N,
                  int64_t d, int H, int dh, const float* obj_mask, const int32_t* ev_rows, float scale, int dtype,
                  hipStream_t st, const float* fsum, const float* fbias, const void* fst, int64_t fparts, float eps) {
  if ((dtype != HCLSM_BF16 && dtype != HCLSM_F16) || N != 32 || dh != 64 || H <= 0 || d != (int64_t)H * 64 ||
      d % QA_KC || !al16(x) || !al16(w) || !al16(o))
    return HCLSM_ERR_UNSUPPORTED;
  const bool fold = fst != nullptr;
  if (fold && (!fsum || !fbias || !al16(fsum) || !al16(fbias) || (((uintptr_t)fst) & 7) || fparts <= 0 ||
               fparts > FOLD_MAX_PARTS))
    return HCLSM_ERR_UNSUPPORTED;
  if (capacity <= 0) return 0;
  if (!x || !w || !o || !n_events || (obj_mask && !ev_rows)) return HCLSM_ERR_NULL;
  const int64_t rows = capacity * 32;
  const int64_t grid = (rows + 127) / 128 * H;
  if (grid > 0x7fffffffLL) return HCLSM_ERR_SHAPE;
  const float sl2 = scale * HCLSM_LOG2E;
  LinExt fx = kNoLinExt;
  fx.fst = reinterpret_cast<const float2*>(fst);
  fx.fparts = fparts;
  fx.fsum = fsum;
  fx.fbias = fbias;
  fx.feps = eps;
#define HCLSM_QA(D, TT, F)                                                                                   \
  hipLaunchKernelGGL((qkv_attn_kernel<D, F>), dim3((unsigned)grid), dim3(256), 0, st, (const TT*)x, d,        \
                     (const TT*)w, (TT*)o, d, n_events, rows, d, H, obj_mask, ev_rows, sl2, fx)
  if (dtype == HCLSM_BF16) {
    if (fold) HCLSM_QA(HCLSM_BF16, uint16_t, true);
    else HCLSM_QA(HCLSM_BF16, uint16_t, false);
  } else {
    if (fold) HCLSM_QA(HCLSM_F16, _Float16, true);
    else HCLSM_QA(HCLSM_F16, _Float16, false);
  }
#undef HCLSM_QA
  HCLSM_LAUNCH_CHECK();
  return 0;
}

// Y[M, N] = X W^T + resid (fp32) on linear_dma_kernel, with Y rounded to dtype in y2 and the LayerNorm partials of
// Y's rows in pst (LinExt pst).  Declared in internal.h.
int linear_stats_rows(const void* x, int64_t ldx, const void* w, int64_t ldw, const float* resid, int64_t ldr,
                      float* y, int64_t ldy, void* y2, int64_t ldy2, void* pst, int64_t M, int64_t N, int64_t K,
                      const int32_t* m_dev, int64_t m_mul, int dtype, hipStream_t st) {
  if (M < 0 || N < 0 || K < 0) return HCLSM_ERR_SHAPE;
  if ((dtype != HCLSM_BF16 && dtype != HCLSM_F16) || K == 0 || K % LD_KC || N % 64 || !al16(x) || ldx % 8 ||
      !al16(w) || ldw % 8 || !al16(y) || ldy % 4 || !al16(y2) || ldy2 % 8 || !al16(resid) || ldr % 4 || !m_dev)
    return HCLSM_ERR_UNSUPPORTED;
  if (M == 0 || N == 0) return 0;
  if (!x || !w || !y || !y2 || !pst) return HCLSM_ERR_NULL;
  LinExt ext{m_dev, m_mul, nullptr, 0, nullptr};
  ext.pst = reinterpret_cast<float2*>(pst);
  const int64_t tiles128 = ((M + 127) / 128) * ((N + 127) / 128);
  if (tiles128 > 0x7fffffffLL) return HCLSM_ERR_SHAPE;
#define HCLSM_ST(D)                                                                                          \
  if (dtype == D)                                                                                            \
    hipLaunchKernelGGL((linear_dma_kernel<D, HCLSM_F32, true>), dim3((unsigned)tiles128), dim3(256), 0, st,  \
                       (const MM<D>::T*)x, ldx, (const MM<D>::T*)w, ldw, nullptr, resid, ldr, y, ldy,         \
                       (MM<D>::T*)y2, ldy2, M, N, K, 0, 0.f, OutSplit{0, 1, 0, 0, nullptr}, ext);
  HCLSM_ST(HCLSM_BF16)
  HCLSM_ST(HCLSM_F16)
#undef HCLSM_ST
  HCLSM_LAUNCH_CHECK();
  return 0;
}

// Y = LN(X) W0^T with the LayerNorm folded into the weights (LinExt fst / fsum / fbias): w = W0 diag(gamma), x the
// 16-bit rows whose partials fst [M][fparts] linear_stats_rows wrote.  With w3 the SwiGLU input layer over N = 2 H
// interleaved columns (Y [M, H], linear_lds128_kernel), else Y [M, N] (linear_lds_kernel).  Declared in
// internal.h.
int linear_fold_rows(const void* x, int64_t ldx, const void* w, const void* w3, int64_t ldw, const float* fsum,
                     const float* fbias, const void* fst, int64_t fparts, float eps, void* y, int64_t ldy, int y_dtype,
                     int64_t M, int64_t N, int64_t K, const int32_t* m_dev, int64_t m_mul, int dtype, hipStream_t st) {
  if (M < 0 || N < 0 || K < 0 || fparts <= 0) return HCLSM_ERR_SHAPE;
  if (fparts > FOLD_MAX_PARTS) return HCLSM_ERR_UNSUPPORTED;
  if ((dtype != HCLSM_BF16 && dtype != HCLSM_F16) || (y_dtype != dtype && y_dtype != HCLSM_F32)) return HCLSM_ERR_DTYPE;
  if (K == 0 || K % 32 || N % (w3 ? 32 : 4) || !al16(x) || ldx % 8 || !al16(w) || !al16(w3) || ldw % 8 ||
      !al16(fsum) || !al16(fbias) || (((uintptr_t)fst) & 7))
    return HCLSM_ERR_UNSUPPORTED;
  if (M == 0 || N == 0) return 0;
  if (!x || !w || !fsum || !fbias || !fst || !y) return HCLSM_ERR_NULL;
  LinExt ext{m_dev, m_mul, nullptr, 0, w3};
  ext.fst = reinterpret_cast<const float2*>(fst);
  ext.fparts = fparts;
  ext.fsum = fsum;
  ext.fbias = fbias;
  ext.feps = eps;
  const int64_t tiles128 = ((M + 127) / 128) * ((N + 127) / 128), tiles64 = ((M + 63) / 64) * ((N + 63) / 64);
  if (tiles64 > 0x7fffffffLL) return HCLSM_ERR_SHAPE;
#define HCLSM_FO(D, O)                                                                                       \
  if (dtype == D && y_dtype == O) {                                                                          \
    if (w3)                                                                                                  \
      hipLaunchKernelGGL((linear_lds128_kernel<D, O, MM<D>::T, true>), dim3((unsigned)tiles128), dim3(256), 0,  \
                         st,                                                                                 \
                         (const MM<D>::T*)x, ldx, (const MM<D>::T*)w, ldw, nullptr, nullptr, 0, (MM<O>::T*)y,  \
                         ldy, nullptr, 0, M, N, K, 0, 0.f, ext);                                              \
    else                                                                                                     \
      hipLaunchKernelGGL((linear_lds_kernel<D, O, MM<D>::T, true>), dim3((unsigned)tiles64), dim3(256), 0, st, \
                         (const MM<D>::T*)x, ldx, (const MM<D>::T*)w, ldw, nullptr, nullptr, 0, (MM<O>::T*)y,  \
                         ldy, nullptr, 0, M, N, K, 0, 0.f, OutSplit{0, 1, 0, 0, nullptr}, ext);             \
  }
  HCLSM_FO(HCLSM_BF16, HCLSM_BF16)
  HCLSM_FO(HCLSM_BF16, HCLSM_F32)
  HCLSM_FO(HCLSM_F16, HCLSM_F16)
  HCLSM_FO(HCLSM_F16, HCLSM_F32)
#undef HCLSM_FO
  HCLSM_LAUNCH_CHECK();
  return 0;
}

// SwiGLU input layer Y[M, H] = silu(X . w1^T) * (X . w3^T) as one GEMM over 2H interleaved columns (w_row) on
// the LDS kernels (HCLSM_ERR_UNSUPPORTED for shapes or alignments they do not take: the caller runs two GEMMs).
// Declared in internal.h.
int linear_glu_rows(const void* x, int64_t ldx, int x_dtype, const void* w1, const void* w3, int64_t ldw, void* y,
                    int64_t ldy, int y_dtype, int64_t M, int64_t H, int64_t K, const int32_t* m_dev, int64_t m_mul,
                    int dtype, hipStream_t st) {
  if (M < 0 || H < 0 || K < 0) return HCLSM_ERR_SHAPE;
  if (M == 0 || H == 0) return 0;
  if (!x || !w1 || !w3 || !y) return HCLSM_ERR_NULL;
  if (H % 16 != 0 || K == 0) return HCLSM_ERR_UNSUPPORTED;
  if (dtype == HCLSM_F32) {   // the fp32 LDS kernel: 16-byte rows
    if (x_dtype != HCLSM_F32 || K % 4 || !al16(x) || !al16(w1) || !al16(w3) || ldx % 4 || ldw % 4)
      return HCLSM_ERR_UNSUPPORTED;
  } else {
    if (K % 32 != 0 || !al16(w1) || !al16(w3) || ldw % 8) return HCLSM_ERR_UNSUPPORTED;
    if (x_dtype == dtype ? (!al16(x) || ldx % 8) : (x_dtype != HCLSM_F32 || !al16(x) || ldx % 4))
      return HCLSM_ERR_UNSUPPORTED;
  }
  const LinExt ext{m_dev, m_mul, nullptr, 0, w3};
  const int64_t N = 2 * H;
#define HCLSM_GLU2(D, O, XD, XT)                                                                             \
  if (dtype == D && y_dtype == O && x_dtype == XD) {                                                         \
    launch_linear_quad<D, O, XT>(x, ldx, w1, ldw, nullptr, nullptr, 0, y, ldy, nullptr, 0, M, N, K, 0, 0.f, st, \
                                 OutSplit{0, 1, 0, 0, nullptr}, ext);                                        \
    HCLSM_LAUNCH_CHECK();                                                                                    \
    return 0;                                                                                                \
  }
  HCLSM_GLU2(HCLSM_BF16, HCLSM_BF16, HCLSM_BF16, uint16_t)
  HCLSM_GLU2(HCLSM_BF16, HCLSM_F32, HCLSM_BF16, uint16_t)
  HCLSM_GLU2(HCLSM_BF16, HCLSM_BF16, HCLSM_F32, float)
  HCLSM_GLU2(HCLSM_F16, HCLSM_F16, HCLSM_F16, _Float16)
  HCLSM_GLU2(HCLSM_F16, HCLSM_F32, HCLSM_F16, _Float16)
  HCLSM_GLU2(HCLSM_F16, HCLSM_F16, HCLSM_F32, float)
  HCLSM_GLU2(HCLSM_F32, HCLSM_F32, HCLSM_F32, float)
#undef HCLSM_GLU2
  return HCLSM_ERR_DTYPE;
}

// gh (nullable): the hidden-side products s W_hh^T precomputed ([M][3H] fp32, row stride ldgh); hb and w_hh are
// then not read.
static int gru_impl(const void* x, int64_t ldx, const void* hb, int64_t ldhb, const float* h, int64_t ldh,
                    const void* w_ih, const void* w_hh, const float* b_ih, const float* b_hh, float* out, int64_t ldo,
                    void* out2, int64_t ldo2, int64_t M, int64_t H, int64_t Kx, int dtype, hipStream_t st,
                    const float* gh = nullptr, int64_t ldgh = 0) {
  if (M < 0 || H < 0 || Kx < 0) return HCLSM_ERR_SHAPE;
  if (M == 0 || H == 0) return 0;
  if (!x || (!hb && !gh) || !h || !w_ih || (!w_hh && !gh) || !out) return HCLSM_ERR_NULL;
  const int kpl = dtype == HCLSM_F32 ? 1 : 8;
  if (Kx % (4 * kpl) || H % (4 * kpl)) return HCLSM_ERR_UNSUPPORTED;
  if (kpl == 8 && (!al16(x) || !al16(w_ih) || ldx % 8)) return HCLSM_ERR_UNSUPPORTED;
  if (kpl == 8 && !gh && (!al16(hb) || !al16(w_hh) || ldhb % 8)) return HCLSM_ERR_UNSUPPORTED;
  const unsigned grid = (unsigned)(((M + 31) / 32) * ((H + 15) / 16));
#define HCLSM_GRU(D)                                                                                        \
  if (dtype == D) {                                                                                         \
    if (gh)                                                                                                 \
      hipLaunchKernelGGL((gru_kernel<D, true>), dim3(grid), dim3(256), 0, st, (const MM<D>::T*)x, ldx,       \
                         (const MM<D>::T*)hb, ldhb, h, ldh, (const MM<D>::T*)w_ih, (const MM<D>::T*)w_hh, b_ih, \
                         b_hh, out, ldo, (MM<D>::T*)out2, ldo2, M, H, Kx, gh, ldgh);                        \
    else                                                                                                    \
      hipLaunchKernelGGL((gru_kernel<D, false>), dim3(grid), dim3(256), 0, st, (const MM<D>::T*)x, ldx,      \
                         (const MM<D>::T*)hb, ldhb, h, ldh, (const MM<D>::T*)w_ih, (const MM<D>::T*)w_hh, b_ih, \
                         b_hh, out, ldo, (MM<D>::T*)out2, ldo2, M, H, Kx, gh, ldgh);                        \
    HCLSM_LAUNCH_CHECK();                                                                                   \
    return 0;                                                                                               \
  }
  HCLSM_GRU(HCLSM_BF16)
  HCLSM_GRU(HCLSM_F16)
  HCLSM_GRU(HCLSM_F32)
#undef HCLSM_GRU
  return HCLSM_ERR_DTYPE;
}

// ---------------------------------------------------------------------------
// LayerNorm kernel (standalone entry point): one wave per row, values kept in registers.
template <int DTI, int DTO>
__global__ void __launch_bounds__(256)
layer_norm_kernel(const typename MM<DTI>::T* __restrict__ x, int64_t ldx, const float* __restrict__ w,
                  const float* __restrict__ b, typename MM<DTO>::T* __restrict__ y, int64_t ldy, int64_t M,
                  int D, float eps, LinExt ext) {
  constexpr int MAXPL = 16;  // elements per lane held in registers (D <= 1024); larger D re-reads
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  M = ext_rows(ext, M);
  if (row >= M) return;
  const typename MM<DTI>::T* xr = x + row * ldx;
  float vals[MAXPL];
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < MAXPL; ++j) {
    const int i = lane + 64 * j;
    vals[j] = i < D ? MM<DTI>::tof(xr[i]) : 0.f;
    s += vals[j];
  }
  for (int i = lane + 64 * MAXPL; i < D; i += 64) s += MM<DTI>::tof(xr[i]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
  const float mean = s / (float)D;
  float v = 0.f;
#pragma unroll
  for (int j = 0; j < MAXPL; ++j) {
    const int i = lane + 64 * j;
    const float d = vals[j] - mean;
    v += i < D ? d * d : 0.f;
  }
  for (int i = lane + 64 * MAXPL; i < D; i += 64) {
    const float d = MM<DTI>::tof(xr[i]) - mean;
    v += d * d;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  const float rstd = 1.f / sqrtf(v / (float)D + eps);
  typename MM<DTO>::T* yr = y + row * ldy;
#pragma unroll
  for (int j = 0; j < MAXPL; ++j) {
    const int i = lane + 64 * j;
    if (i < D) {
      float t = (vals[j] - mean) * rstd;
      if (w) t *= w[i];
      if (b) t += b[i];
      yr[i] = MM<DTO>::fromf(t);
    }
  }
  for (int i = lane + 64 * MAXPL; i < D; i += 64) {
    float t = (MM<DTI>::tof(xr[i]) - mean) * rstd;
    if (w) t *= w[i];
    if (b) t += b[i];
    yr[i] = MM<DTO>::fromf(t);
  }
}

// 4 consecutive elements as fp32 (one 16-byte load for fp32, 8 bytes for 16-bit types) and back
template <int DT>
__device__ __forceinline__ float4 ln_load4(const typename MM<DT>::T* p) {
  if constexpr (DT == HCLSM_F32) {
    return *reinterpret_cast<const float4*>(p);
  } else {
    typename MM<DT>::T e[4];
    *reinterpret_cast<uint2*>(e) = *reinterpret_cast<const uint2*>(p);
    return make_float4(MM<DT>::tof(e[0]), MM<DT>::tof(e[1]), MM<DT>::tof(e[2]), MM<DT>::tof(e[3]));
  }
}
template <int DT>
__device__ __forceinline__ void ln_store4(typename MM<DT>::T* p, float4 v) {
  if constexpr (DT == HCLSM_F32) {
    *reinterpret_cast<float4*>(p) = v;
  } else {
    typename MM<DT>::T e[4] = {MM<DT>::fromf(v.x), MM<DT>::fromf(v.y), MM<DT>::fromf(v.z), MM<DT>::fromf(v.w)};
    *reinterpret_cast<uint2*>(p) = *reinterpret_cast<const uint2*>(e);
  }
}

// LayerNorm for rows of D = 4u elements (u <= LPR * VPL 4-element units) starting 16-byte (fp32) / 8-byte aligned:
// LPR lanes per row (64: a wave per row; 32: two rows per wave, one per half), lane l of a row holding units
// l, l + LPR, ... in registers, every load issued before the reductions.  Same two-pass statistics as
// layer_norm_kernel.  With xc the input rows are also written, in the output type, to xc (row stride ldy).
template <int DTI, int DTO, int VPL, int LPR = 64>
__global__ void __launch_bounds__(256)
layer_norm_vec_kernel(const typename MM<DTI>::T* __restrict__ x, int64_t ldx, const float* __restrict__ w,
                      const float* __restrict__ b, typename MM<DTO>::T* __restrict__ y, int64_t ldy, int64_t M,
                      int D, float eps, LinExt ext, typename MM<DTO>::T* __restrict__ xc) {
  static_assert(LPR == 64 || LPR == 32, "a row per wave or per half-wave");
  constexpr int RPW = 64 / LPR;   // rows per wave
  const int lane = threadIdx.x & 63, ll = lane % LPR;
  M = ext_rows(ext, M);
  const int U = D >> 2;
  // rows walked with the grid's stride (the grid may be smaller than M / (4 RPW) with a device-side row count)
  for (int64_t row = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW + lane / LPR; row < M;
       row += (int64_t)gridDim.x * 4 * RPW) {
    const typename MM<DTI>::T* xr = x + row * ldx;
    float4 v[VPL];
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const int u = ll + LPR * j;
      v[j] = u < U ? ln_load4<DTI>(xr + 4 * u) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int j = 0; j < VPL; ++j) s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    const float mean = s / (float)D;
    float q = 0.f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      if (ll + LPR * j < U) {
        const float a = v[j].x - mean, c = v[j].y - mean, d = v[j].z - mean, e = v[j].w - mean;
        q += (a * a + c * c) + (d * d + e * e);
      }
    }
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) q += __shfl_xor(q, o, 64);
    const float rstd = 1.f / sqrtf(q / (float)D + eps);
    typename MM<DTO>::T* yr = y + row * ldy;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const int u = ll + LPR * j;
      if (u < U) {
        float4 t = make_float4((v[j].x - mean) * rstd, (v[j].y - mean) * rstd, (v[j].z - mean) * rstd,
                               (v[j].w - mean) * rstd);
        if (w) {
          const float4 wv = *reinterpret_cast<const float4*>(w + 4 * u);
          t.x *= wv.x; t.y *= wv.y; t.z *= wv.z; t.w *= wv.w;
        }
        if (b) {
          const float4 bv = *reinterpret_cast<const float4*>(b + 4 * u);
          t.x += bv.x; t.y += bv.y; t.z += bv.z; t.w += bv.w;
        }
        ln_store4<DTO>(yr + 4 * u, t);
        if (xc) ln_store4<DTO>(xc + row * ldy + 4 * u, v[j]);   // the input row itself, in the output type
      }
    }
  }
}

template <int DT>
__global__ void __launch_bounds__(256)
convert_f32_kernel(const float* __restrict__ src, typename MM<DT>::T* __restrict__ dst, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = MM<DT>::fromf(src[i]);
}

static int convert_f32(const float* src, void* dst, int64_t n, int dtype, hipStream_t st) {
  if (n <= 0) return 0;
  int64_t g = (n + 255) / 256;
  g = g > 4096 ? 4096 : g;
  if (dtype == HCLSM_BF16)
    hipLaunchKernelGGL(convert_f32_kernel<HCLSM_BF16>, dim3((unsigned)g), dim3(256), 0, st, src, (uint16_t*)dst, n);
  else if (dtype == HCLSM_F16)
    hipLaunchKernelGGL(convert_f32_kernel<HCLSM_F16>, dim3((unsigned)g), dim3(256), 0, st, src, (_Float16*)dst, n);
  else
    hipLaunchKernelGGL(convert_f32_kernel<HCLSM_F32>, dim3((unsigned)g), dim3(256), 0, st, src, (float*)dst, n);
  HCLSM_LAUNCH_CHECK();
  return 0;
}

// LayerNorm of M rows; with xc (fp32 input rows with ldx == D only) the input is also copied to xc in the output
// type, in the same pass where the vector kernel runs.
static int ln_impl(const void* x, int64_t ldx, const float* w, const float* b, void* y, int64_t ldy, int64_t M,
                   int64_t D, float eps, int in_dtype, int out_dtype, hipStream_t st, LinExt ext = kNoLinExt,
                   void* xc = nullptr) {
  if (M < 0 || D < 0 || D > 0x7fffffff) return HCLSM_ERR_SHAPE;
  if (M == 0 || D == 0) return 0;
  if (!x || !y) return HCLSM_ERR_NULL;
  if (xc && (in_dtype != HCLSM_F32 || ldx != D || ldy != D || ext.m_dev)) return HCLSM_ERR_UNSUPPORTED;
  const unsigned grid = (unsigned)((M + 3) / 4);
  // vector kernel: D a multiple of 4 up to 1024, rows and weights aligned for 4-element accesses
  const int ies = in_dtype == HCLSM_F32 ? 4 : 2, oes = out_dtype == HCLSM_F32 ? 4 : 2;
  const bool vec = D % 4 == 0 && D <= 1024 && ((uintptr_t)x % (4 * ies)) == 0 && ((uintptr_t)y % (4 * oes)) == 0 &&
                   (ldx * ies) % (4 * ies) == 0 && (ldy * oes) % (4 * oes) == 0 && ((uintptr_t)w % 16) == 0 &&
                   ((uintptr_t)b % 16) == 0;
  // Rows of up to 128 units walked over more rows than one round of the grid covers (a device-side row count,
  // or many rows): a half-wave per row (1 .. 4 units per lane), half the waves per row; otherwise a wave per row
  // (up to 4 units per lane), which is faster when every row gets a wave of its own (measured: Level-1 step
  // -1.5% with half-wave rows, the 1024- and 6272-row slot-attention LayerNorms +0.3 us each).
  const int U = (int)(D / 4);
  const bool half = U <= 128 && (ext.m_dev != nullptr || M > 8192);
  const int vpl = half ? (U + 31) / 32 : (U + 63) / 64;
  const unsigned hgrid = half ? (unsigned)((M + 7) / 8) : grid;
  // device row count: at most what the device holds at once (the vector kernel walks the rows); every
  // instantiation has the same occupancy, so one of each width stands for all element types
  unsigned vgrid = hgrid;
  if (vec && ext.m_dev) {
    static std::atomic<int> cache[8][HCLSM_MAX_DEVICES];
    const void* fns[8] = {(const void*)layer_norm_vec_kernel<HCLSM_F32, HCLSM_BF16, 1, 64>,
                          (const void*)layer_norm_vec_kernel<HCLSM_F32, HCLSM_BF16, 2, 64>,
                          (const void*)layer_norm_vec_kernel<HCLSM_F32, HCLSM_BF16, 3, 64>,
                          (const void*)layer_norm_vec_kernel<HCLSM_F32, HCLSM_BF16, 4, 64>,
                          (const void*)layer_norm_vec_kernel<HCLSM_F32, HCLSM_BF16, 1, 32>,
                          (const void*)layer_norm_vec_kernel<HCLSM_F32, HCLSM_BF16, 2, 32>,
                          (const void*)layer_norm_vec_kernel<HCLSM_F32, HCLSM_BF16, 3, 32>,
                          (const void*)layer_norm_vec_kernel<HCLSM_F32, HCLSM_BF16, 4, 32>};
    const int fi = (half ? 4 : 0) + vpl - 1;
    int slots = 0;
    if (device_launch_setup(fns[fi], 256, 0, 0, cache[fi], &slots) == 0 && slots > 0 && (unsigned)slots < hgrid)
      vgrid = (unsigned)slots;
  }
#define HCLSM_LN_V(I, O, V, P)                                                                             \
  hipLaunchKernelGGL((layer_norm_vec_kernel<I, O, V, P>), dim3(vgrid), dim3(256), 0, st, (const MM<I>::T*)x,   \
                     ldx, w, b, (MM<O>::T*)y, ldy, M, (int)D, eps, ext, (MM<O>::T*)xc)
#define HCLSM_LN(I, O)                                                                                     \
  if (in_dtype == I && out_dtype == O) {                                                                   \
    if (vec && half) {                                                                                     \
      if (vpl == 1) HCLSM_LN_V(I, O, 1, 32);                                                               \
      else if (vpl == 2) HCLSM_LN_V(I, O, 2, 32);                                                          \
      else if (vpl == 3) HCLSM_LN_V(I, O, 3, 32);                                                          \
      else HCLSM_LN_V(I, O, 4, 32);                                                                        \
    } else if (vec) {                                                                                      \
      if (vpl == 1) HCLSM_LN_V(I, O, 1, 64);                                                               \
      else if (vpl == 2) HCLSM_LN_V(I, O, 2, 64);                                                          \
      else if (vpl == 3) HCLSM_LN_V(I, O, 3, 64);                                                          \
      else HCLSM_LN_V(I, O, 4, 64);                                                                        \
    } else {                                                                                               \
      hipLaunchKernelGGL((layer_norm_kernel<I, O>), dim3(grid), dim3(256), 0, st, (const MM<I>::T*)x, ldx, w, \
                         b, (MM<O>::T*)y, ldy, M, (int)D, eps, ext);                                       \
    }                                                                                                      \
    HCLSM_LAUNCH_CHECK();                                                                                  \
    if (xc && !vec) return convert_f32((const float*)x, xc, M * D, out_dtype, st);                         \
    return 0;                                                                                              \
  }
  HCLSM_LN(HCLSM_F32, HCLSM_F32)
  HCLSM_LN(HCLSM_F32, HCLSM_BF16)
  HCLSM_LN(HCLSM_BF16, HCLSM_BF16)
  HCLSM_LN(HCLSM_BF16, HCLSM_F32)
  HCLSM_LN(HCLSM_F32, HCLSM_F16)
  HCLSM_LN(HCLSM_F16, HCLSM_F16)
#undef HCLSM_LN
#undef HCLSM_LN_V
  return HCLSM_ERR_DTYPE;
}

int layer_norm_rows(const void* x, int64_t ldx, const float* w, const float* b, void* y, int64_t ldy, int64_t M,
                    int64_t D, float eps, int in_dtype, int out_dtype, const int32_t* m_dev, int64_t m_mul,
                    hipStream_t st) {
  return ln_impl(x, ldx, w, b, y, ldy, M, D, eps, in_dtype, out_dtype, st, LinExt{m_dev, m_mul, nullptr, 0});
}

}  // namespace hclsm

using namespace hclsm;

extern "C" int hclsm_layer_norm(const void* x, int64_t ldx, const float* w, const float* b, void* y, int64_t ldy,
                                int64_t M, int64_t D, float eps, int in_dtype, int out_dtype, void* stream) {
  return ln_impl(x, ldx, w, b, y, ldy, M, D, eps, in_dtype, out_dtype, (hipStream_t)stream);
}

extern "C" int hclsm_linear(const void* x, int64_t ldx, int x_dtype, const void* w, int64_t ldw, const float* bias,
                            const float* resid, int64_t ldr, void* y, int64_t ldy, int y_dtype, void* y2,
                            int64_t ldy2, int64_t M, int64_t N, int64_t K, int relu, float clamp, int ln,
                            const float* ln_w, const float* ln_b, float ln_eps, int dtype, void* stream) {
  return linear_impl(x, ldx, x_dtype, w, ldw, bias, resid, ldr, y, ldy, y_dtype, y2, ldy2, M, N, K, relu, clamp, ln,
                     ln_w, ln_b, ln_eps, dtype, (hipStream_t)stream);
}

extern "C" int hclsm_gru_cell(const void* x, int64_t ldx, const void* hb, int64_t ldhb, const float* h, int64_t ldh,
                              const void* w_ih, const void* w_hh, const float* b_ih, const float* b_hh, float* out,
                              int64_t ldo, void* out2, int64_t ldo2, int64_t M, int64_t H, int64_t Kx, int dtype,
                              void* stream) {
  return gru_impl(x, ldx, hb, ldhb, h, ldh, w_ih, w_hh, b_ih, b_hh, out, ldo, out2, ldo2, M, H, Kx, dtype,
                  (hipStream_t)stream);
}

extern "C" int64_t hclsm_slot_attn_core_workspace(int64_t B, int64_t N, int64_t M, int dtype) {
  if (B < 0 || N < 0 || M < 0) return HCLSM_ERR_SHAPE;
  return (int64_t)core_ws_bytes(B, N, M, dtype == HCLSM_F32 ? 4 : 2);
}

extern "C" int hclsm_slot_attn_core(const void* q, int64_t ldq, int64_t q_bstride, const void* k, int64_t ldk,
                                    int64_t k_bstride, const void* v, int64_t ldv, int64_t v_bstride, void* out,
                                    int64_t ldo, int64_t o_bstride, void* attn, int attn_dtype, int64_t B, int64_t N,
                                    int64_t M, int64_t D, float scale, float denom_eps, float logit_clamp,
                                    float renorm_eps, int dtype, void* workspace, int64_t workspace_bytes,
                                    void* stream) {
  const int c = check_core(q, ldq, q_bstride, k, ldk, k_bstride, B, N, M, D, dtype);
  if (c) return c;
  if (B == 0 || N == 0 || D == 0) return 0;
  if (M == 0) return HCLSM_ERR_SHAPE;
  if (!q || !k || !v || !out || !workspace) return HCLSM_ERR_NULL;
  if (attn && attn_dtype != HCLSM_F32 && attn_dtype != dtype) return HCLSM_ERR_DTYPE;
  if (workspace_bytes < (int64_t)core_ws_bytes(B, N, M, dtype == HCLSM_F32 ? 4 : 2)) return HCLSM_ERR_SHAPE;
  if (!al16(workspace)) return HCLSM_ERR_UNSUPPORTED;
  return launch_core(q, ldq, q_bstride, k, ldk, k_bstride, v, ldv, v_bstride, out, ldo, o_bstride, attn, attn_dtype, B,
                     N, M, D, scale, denom_eps, logit_clamp, renorm_eps, dtype, workspace, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------
// Whole iterations: the sequence of launches above, on one stream, out of one workspace.

static size_t al256(size_t x) { return (x + 255) / 256 * 256; }

// dst[c][r] = src[r][c] for 16-bit elements, 32 x 32 tiles through LDS.
__global__ void __launch_bounds__(256) transpose16_kernel(const uint16_t* __restrict__ src, int64_t lds,
                                                          uint16_t* __restrict__ dst, int64_t ldd, int64_t R,
                                                          int64_t C) {
  __shared__ uint16_t tile[32][34];
  const int64_t c0 = (int64_t)blockIdx.x * 32, r0 = (int64_t)blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int i = ty; i < 32; i += 8)
    if (r0 + i < R && c0 + tx < C) tile[i][tx] = src[(r0 + i) * lds + c0 + tx];
  __syncthreads();
  for (int i = ty; i < 32; i += 8)
    if (c0 + i < C && r0 + tx < R) dst[(c0 + i) * ldd + r0 + tx] = tile[tx][i];
}

static int transpose_16(const void* src, int64_t lds, void* dst, int64_t ldd, int64_t R, int64_t C, hipStream_t st) {
  if (R <= 0 || C <= 0) return 0;
  if ((R + 31) / 32 > 65535) return HCLSM_ERR_SHAPE;
  hipLaunchKernelGGL(transpose16_kernel, dim3((unsigned)((C + 31) / 32), (unsigned)((R + 31) / 32)), dim3(256), 0, st,
                     (const uint16_t*)src, lds, (uint16_t*)dst, ldd, R, C);
  HCLSM_LAUNCH_CHECK();
  return 0;
}

struct SlotWs {
  size_t q, core, upd, h, sb, m1, sfa, kv, vt, xn, xin, kq, wqt, gh, total;
  bool has_kq;
};

static SlotWs slot_ws_layout(int64_t B, int64_t N, int64_t M, int64_t d, int64_t hidden, int esize, bool with_kv,
                             int64_t d_in = 0) {
  SlotWs w;
  size_t o = 0;
  const size_t rows = (size_t)B * N;
  w.xn = o; o += al256(rows * d * esize);
  w.xin = o; o += with_kv ? al256((size_t)B * M * (d_in > 0 ? d_in : d) * esize) : 0;
  w.q = o; o += al256(rows * d * esize);
  w.core = o; o += al256(core_ws_bytes(B, N, M, esize));
  w.upd = o; o += al256(rows * d * esize);
  w.h = o; o += al256(rows * d * 4);
  w.sb = o; o += al256(rows * d * esize);
  w.m1 = o; o += al256(rows * hidden * esize);
  w.sfa = o; o += al256(rows * d * 4);
  w.kv = o; o += with_kv ? al256((size_t)B * M * d * esize) : 0;
  w.vt = o; o += with_kv ? al256((size_t)B * d * ((M + 31) / 32 * 32) * esize) : 0;
  // 16-bit forward: k Wq (the keys times the query weight) and Wq^T, for the fused core's LNQ form
  const bool kq = with_kv && esize == 2;
  w.has_kq = kq;
  w.kq = o; o += kq ? al256((size_t)B * M * d * esize) : 0;
  w.wqt = o; o += kq ? al256((size_t)d * d * esize) : 0;
  w.gh = o; o += kq ? al256(rows * 3 * d * 4) : 0;   // the GRU's hidden-side products, formed by the fused core
  w.total = o;
  return w;
}

extern "C" int64_t hclsm_slot_attention_workspace(int64_t B, int64_t N, int64_t M, int64_t d_in, int64_t d,
                                                  int64_t hidden, int dtype) {
  if (B < 0 || N < 0 || M < 0 || d_in < 0 || d < 0 || hidden < 0) return HCLSM_ERR_SHAPE;
  return (int64_t)slot_ws_layout(B, N, M, d, hidden, dtype == HCLSM_F32 ? 4 : 2, true, d_in).total;
}


// One iteration (dynamic_slots.py:98-131).  slots_in fp32 and sb (the same slots in `dtype`) are
// read; slots_out (may alias slots_in: it is written by the last launch, after every read) and
// sb (rewritten with the new slots in `dtype`) are produced.
// LN(x) W^T (+ bias) (ReLU) for fp32 x in one launch (linear_kreg_kernel: row statistics from the registers
// holding the rows); xout (nullable) receives x rounded to dtype.  *taken = false, launching nothing, when
// the shapes do not fit it: 16-bit dtype, K <= 384 a multiple of 32, 16-byte aligned rows and LN weights.
static int linear_ln_fold(const float* x, int64_t ldx, const void* w, int64_t ldw, const float* bias, void* y,
                          int64_t ldy, int64_t M, int64_t N, int64_t K, int relu, const float* lnw, const float* lnb,
                          float eps, void* xout, int64_t ldxo, int dtype, hipStream_t st, bool* taken) {
  *taken = false;
  // the LN variant keeps the rows, gamma and beta in registers (two workgroups per CU): taken only when the
  // tiles fit one such round on the device, where it beats a LayerNorm launch plus the linear layer
  const int64_t tiles = ((M + 31) / 32) * ((N + 31) / 32);
  int cus = 0;
  if (device_cus(&cus) != 0 || cus <= 0) return 0;
  if (tiles > 2 * (int64_t)cus) return 0;
  if ((dtype != HCLSM_BF16 && dtype != HCLSM_F16) || M <= 0 || N <= 0 || K <= 0 || K % 32 || K > 384 || !al16(x) ||
      ldx % 4 || !al16(w) || ldw % 8 || (lnw && !al16(lnw)) || (lnb && !al16(lnb)) ||
      (xout && (!al16(xout) || ldxo % 8)) || !al16(y) || ldy % 8)
    return 0;
  *taken = true;
  if (dtype == HCLSM_BF16)
    launch_linear_kreg<HCLSM_BF16, HCLSM_BF16, float, true>(x, ldx, w, ldw, bias, nullptr, 0, y, ldy, nullptr, 0, M, N,
                                                            K, relu, 0.f, lnw, lnb, eps, xout, ldxo, st);
  else
    launch_linear_kreg<HCLSM_F16, HCLSM_F16, float, true>(x, ldx, w, ldw, bias, nullptr, 0, y, ldy, nullptr, 0, M, N,
                                                          K, relu, 0.f, lnw, lnb, eps, xout, ldxo, st);
  HCLSM_LAUNCH_CHECK();
  return 0;
}

// norm_slots folded into W1 by the caller's weights (16-bit, K = d within the linear_kreg_kernel instantiations).
static bool norm_fold_fits(const HclsmSlotWeights* W, int64_t d, int64_t hidden, int dtype) {
  return (dtype == HCLSM_BF16 || dtype == HCLSM_F16) && W->w1_n != nullptr && W->w1_n_sum != nullptr &&
         W->w1_n_bias != nullptr && d % 32 == 0 && d <= 1024 && hidden > 0;
}

// y = act(rstd (x w_n^T - mean w_sum) + bias) for 16-bit x: LN(x) w^T + b with the LayerNorm folded into
// w_n = w diag(gamma), w_sum (row sums of w_n) and bias = w beta + b (linear_kreg_kernel, FOLD).
static int linear_norm_folded(const void* x, int64_t ldx, const void* w_n, const float* w_sum, const float* bias,
                              void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, int relu, float eps, int dtype,
                              hipStream_t st) {
  if (!al16(x) || ldx % 8 || !al16(w_n) || K % 32 || ldy % 8) return HCLSM_ERR_UNSUPPORTED;
  bool ok = false;
  if (dtype == HCLSM_BF16)
    ok = launch_linear_kreg<HCLSM_BF16, HCLSM_BF16, uint16_t, false, true>(x, ldx, w_n, K, bias, nullptr, 0, y, ldy,
                                                                         nullptr, 0, M, N, K, relu, 0.f, nullptr,
                                                                         nullptr, eps, nullptr, 0, st, w_sum);
  else if (dtype == HCLSM_F16)
    ok = launch_linear_kreg<HCLSM_F16, HCLSM_F16, _Float16, false, true>(x, ldx, w_n, K, bias, nullptr, 0, y, ldy,
                                                                        nullptr, 0, M, N, K, relu, 0.f, nullptr,
                                                                        nullptr, eps, nullptr, 0, st, w_sum);
  if (!ok) return HCLSM_ERR_UNSUPPORTED;
  HCLSM_LAUNCH_CHECK();
  return 0;
}

// kq (nullable; v transposed, shapes the fused core takes): k Wq with the same strides as k, and the iteration
// runs no q projection (the fused core's LNQ form).
static int slot_iteration_impl(const HclsmSlotWeights* W, const float* slots_in, void* sb, bool make_sb,
                               const void* k, int64_t ldk, int64_t k_bstride, const void* v, int64_t ldv,
                               int64_t v_bstride, bool v_transposed, float* slots_out, int64_t B, int64_t N, int64_t M,
                               int64_t d, int64_t hidden, float scale, float logit_clamp, float renorm_eps,
                               float slot_clamp, int dtype, char* ws, const SlotWs& L, hipStream_t st,
                               const void* kq = nullptr) {
  const int64_t rows = B * N;
  void* q = ws + L.q;
  void* upd = ws + L.upd;
  float* h = reinterpret_cast<float*>(ws + L.h);
  void* m1 = ws + L.m1;
  void* xn = ws + L.xn;
  bool folded = false;
  int rc = 1;
  // GH: the fused core also forms the GRU's hidden-side products (then no iteration needs the slots in dtype)
  float* gh = (kq != nullptr && cf_gh_fits(d, cf_ncb(d))) ? reinterpret_cast<float*>(ws + L.gh) : nullptr;
  if (kq != nullptr) {
    // updates = core(LN_pre(slots), k Wq, v^T); with make_sb the core also writes sb (the slots in dtype)
    const LnqArgs ln{slots_in, d,       N * d, W->ln_pre_w, W->ln_pre_b, 1e-5f, (make_sb && !gh) ? sb : nullptr,
                     d,        N * d,   W->w_hh, gh};
    rc = launch_core_fused(nullptr, d, N * d, kq, ldk, k_bstride, v, v_bstride, upd, d, N * d, B, N, M, d, scale, 0.f,
                           logit_clamp, renorm_eps, dtype, st, &ln);
    if (rc == 1) return HCLSM_ERR_UNSUPPORTED;   // the caller checked core_fused_fits
  } else {
    // q = LN_pre(slots) W_q^T; with make_sb the same pass writes sb (the slots in dtype)
    rc = linear_ln_fold(slots_in, d, W->w_q, d, nullptr, q, d, rows, d, d, 0, W->ln_pre_w, W->ln_pre_b, 1e-5f,
                        make_sb ? sb : nullptr, d, dtype, st, &folded);
    if (rc) return rc;
    if (!folded) {
      rc = ln_impl(slots_in, d, W->ln_pre_w, W->ln_pre_b, xn, d, rows, d, 1e-5f, HCLSM_F32, dtype, st, kNoLinExt,
                   make_sb ? sb : nullptr);
      if (rc) return rc;
      rc = linear_impl(xn, d, dtype, W->w_q, d, nullptr, nullptr, 0, q, d, dtype, nullptr, 0, rows, d, d, 0, 0.f, 0,
                       nullptr, nullptr, 0.f, dtype, st);
      if (rc) return rc;
    }
    // updates = attention core (logits, softmax over slots, [renorm], attn v): one fused launch when v is transposed
    rc = v_transposed ? launch_core_fused(q, d, N * d, k, ldk, k_bstride, v, v_bstride, upd, d, N * d, B, N, M, d,
                                          scale, 0.f, logit_clamp, renorm_eps, dtype, st)
                      : 1;
  }
  if (rc == 1)
    rc = launch_core(q, d, N * d, k, ldk, k_bstride, v, ldv, v_bstride, upd, d, N * d, nullptr, dtype, B, N, M, d,
                     scale, 0.f, logit_clamp, renorm_eps, dtype, ws + L.core, st, v_transposed);
  if (rc) return rc;
  // norm_slots folded into W1 (the caller's w1 diag(gamma), its row sums and w1 beta + b1): the GRU also writes h in
  // dtype, and W1 forms the row statistics itself
  const bool nfold = norm_fold_fits(W, d, hidden, dtype);
  // h = GRUCell(updates, slots)
  rc = gru_impl(upd, d, sb, d, slots_in, d, W->w_ih, W->w_hh, W->b_ih, W->b_hh, h, d, nfold ? xn : nullptr, d, rows, d,
                d, dtype, st, gh, 3 * d);
  if (rc) return rc;
  // m1 = ReLU(LN_mlp(h) W1^T + b1)
  if (nfold) {
    rc = linear_norm_folded(xn, d, W->w1_n, W->w1_n_sum, W->w1_n_bias, m1, hidden, rows, hidden, d, 1, 1e-5f, dtype,
                            st);
    if (rc) return rc;
    folded = true;
  } else {
    rc = linear_ln_fold(h, d, W->w1, d, W->b1, m1, hidden, rows, hidden, d, 1, W->ln_mlp_w, W->ln_mlp_b, 1e-5f,
                        nullptr, 0, dtype, st, &folded);
  }
  if (rc) return rc;
  if (!folded) {
    rc = ln_impl(h, d, W->ln_mlp_w, W->ln_mlp_b, xn, d, rows, d, 1e-5f, HCLSM_F32, dtype, st);
    if (rc) return rc;
    rc = linear_impl(xn, d, dtype, W->w1, d, W->b1, nullptr, 0, m1, hidden, dtype, nullptr, 0, rows, hidden, d, 1, 0.f,
                     0, nullptr, nullptr, 0.f, dtype, st);
    if (rc) return rc;
  }
  // slots_out = clamp(h + m1 W2^T + b2); sb = the same in dtype
  return linear_impl(m1, hidden, dtype, W->w2, hidden, W->b2, h, d, slots_out, d, HCLSM_F32, gh ? nullptr : sb, d, rows,
                     d, hidden, 0, slot_clamp, 0, nullptr, nullptr, 0.f, dtype, st);
}

// The 16-bit forward forms kq = k W_q (and its iterations run the fused core's LNQ form).
static bool kq_formed(const SlotWs& L, int64_t B, int64_t N, int64_t M, int64_t d, int dtype) {
  return L.has_kq && core_fused_fits(B, N, M, d, dtype);
}

static int check_slot_args(const HclsmSlotWeights* W, int64_t B, int64_t N, int64_t M, int64_t d, int64_t hidden,
                           int dtype, void* workspace, int64_t workspace_bytes, bool with_kv, SlotWs* L,
                           int64_t d_in = 0) {
  if (!W || !workspace) return HCLSM_ERR_NULL;
  if (!W->w_q || !W->w_ih || !W->w_hh || !W->w1 || !W->w2 || (with_kv && !W->w_kv)) return HCLSM_ERR_NULL;
  if (B < 0 || N < 0 || M < 1 || d < 1 || hidden < 1) return HCLSM_ERR_SHAPE;
  if (dtype != HCLSM_BF16 && dtype != HCLSM_F16 && dtype != HCLSM_F32) return HCLSM_ERR_DTYPE;
  const int kpl = dtype == HCLSM_F32 ? 1 : 8;
  if (d % 16 || d % (4 * kpl) || hidden % (4 * kpl)) return HCLSM_ERR_UNSUPPORTED;
  if (N > 16 * CORE_MAX_NT || B > 65535) return HCLSM_ERR_UNSUPPORTED;
  // 16-bit weights are read with 16-byte loads (the GEMMs, the GRU and the fused core's W_hh tiles)
  if (dtype != HCLSM_F32 && (!al16(W->w_q) || !al16(W->w_ih) || !al16(W->w_hh) || !al16(W->w1) || !al16(W->w2) ||
                             !al16(W->w1_n) || (with_kv && (!al16(W->w_kv) || !al16(W->w_qkv)))))
    return HCLSM_ERR_UNSUPPORTED;
  *L = slot_ws_layout(B, N, M, d, hidden, dtype == HCLSM_F32 ? 4 : 2, with_kv, d_in);
  if (workspace_bytes < (int64_t)L->total) return HCLSM_ERR_SHAPE;
  if (!al16(workspace)) return HCLSM_ERR_UNSUPPORTED;
  return 0;
}

extern "C" int hclsm_slot_attention_iteration(const HclsmSlotWeights* W, const float* slots_in, const void* k,
                                              const void* v, int64_t ldkv, int64_t kv_bstride, float* slots_out,
                                              int64_t B, int64_t N, int64_t M, int64_t d, int64_t hidden, float scale,
                                              float logit_clamp, float renorm_eps, float slot_clamp, int dtype,
                                              void* workspace, int64_t workspace_bytes, void* stream) {
  SlotWs L;
  int rc = check_slot_args(W, B, N, M, d, hidden, dtype, workspace, workspace_bytes, false, &L);
  if (rc) return rc;
  if (!slots_in || !k || !v || !slots_out) return HCLSM_ERR_NULL;
  rc = check_core(k, ldkv, kv_bstride, k, ldkv, kv_bstride, B, N, M, d, dtype);
  if (rc) return rc;
  if (B == 0 || N == 0) return 0;
  hipStream_t st = (hipStream_t)stream;
  char* ws = reinterpret_cast<char*>(workspace);
  return slot_iteration_impl(W, slots_in, ws + L.sb, true, k, ldkv, kv_bstride, v, ldkv, kv_bstride, false, slots_out,
                             B, N, M, d, hidden, scale, logit_clamp, renorm_eps, slot_clamp, dtype, ws, L, st);
}

static int slot_forward_impl(const HclsmSlotWeights* W, const float* inputs, int64_t d_in, const float* slots0,
                             float* slots_out, int64_t B, int64_t N, int64_t M, int64_t d, int64_t hidden,
                             int64_t n_iter, float scale, float logit_clamp, float renorm_eps, float slot_clamp,
                             int dtype, void* workspace, int64_t workspace_bytes, void* stream) {
  SlotWs L;
  int rc = check_slot_args(W, B, N, M, d, hidden, dtype, workspace, workspace_bytes, true, &L, d_in);
  if (rc) return rc;
  if (B * M > 0x7fffffffLL) return HCLSM_ERR_SHAPE;
  if (!inputs || (N > 0 && (!slots0 || !slots_out))) return HCLSM_ERR_NULL;   // no slots: empty slot tensors
  if (d_in < 1 || n_iter < 0) return HCLSM_ERR_SHAPE;
  if (d_in % (4 * (dtype == HCLSM_F32 ? 1 : 8))) return HCLSM_ERR_UNSUPPORTED;
  if (B == 0) return 0;   // (with no slots the keys are still formed: callers read them for slot birth)
  hipStream_t st = (hipStream_t)stream;
  char* ws = reinterpret_cast<char*>(workspace);
  const int esize = dtype == HCLSM_F32 ? 4 : 2;
  void* kv = ws + L.kv;
  // The iterations run the fused core's LNQ form (queries as LN_pre(slots) (k W_q)^T): with the caller's
  // [W_q^T W_k; W_v] the projection writes kq = k W_q itself, and k is not formed.
  const bool qkv = W->w_qkv != nullptr && kq_formed(L, B, N, M, d, dtype);
  // k | v = LN_in(inputs) [W_k; W_v]^T     (dynamic_slots.py:152-154), or kq | v
  void* xin = ws + L.xin;
  rc = ln_impl(inputs, d_in, W->ln_in_w, W->ln_in_b, xin, d_in, B * M, d_in, 1e-5f, HCLSM_F32, dtype, st);
  if (rc) return rc;
  // k rows [B*M][d]; v written transposed per frame: vt[b][d][Mp]
  const int64_t Mp = (M + 31) / 32 * 32;
  void* vt = ws + L.vt;
  {
    const OutSplit os{d, M, Mp, d * Mp, vt};
#define HCLSM_KV(D_, XT_)                                                                                    \
    if (dtype == D_)                                                                                         \
      launch_linear_quad<D_, D_, XT_>(xin, d_in, qkv ? W->w_qkv : W->w_kv, d_in, nullptr, nullptr, 0,         \
                                      qkv ? ws + L.kq : kv, d, nullptr, 0, B * M, 2 * d, d_in, 0, 0.f, st, os);
    HCLSM_KV(HCLSM_BF16, uint16_t)
    HCLSM_KV(HCLSM_F16, _Float16)
    HCLSM_KV(HCLSM_F32, float)
#undef HCLSM_KV
    HCLSM_LAUNCH_CHECK();
  }
  (void)esize;
  const void* k = kv;
  if (N == 0) return 0;
  if (n_iter == 0) return (int)hipMemcpyAsync(slots_out, slots0, (size_t)B * N * d * 4, hipMemcpyDeviceToDevice, st);
  // k Wq = k (Wq^T)^T once per call (unless the projection formed it), so that no iteration projects the
  // slots to queries
  const void* kq = qkv ? ws + L.kq : nullptr;
  if (!qkv && kq_formed(L, B, N, M, d, dtype)) {
    const void* wqt = W->w_qt;   // the caller's copy, formed once per weight set, or one formed here
    if (wqt == nullptr || !al16(wqt)) {
      rc = transpose_16(W->w_q, d, ws + L.wqt, d, d, d, st);
      if (rc) return rc;
      wqt = ws + L.wqt;
    }
    rc = linear_impl(kv, d, dtype, wqt, d, nullptr, nullptr, 0, ws + L.kq, d, dtype, nullptr, 0, B * M, d, d,
                     0, 0.f, 0, nullptr, nullptr, 0.f, dtype, st);
    if (rc) return rc;
    kq = ws + L.kq;
  }
  for (int64_t it = 0; it < n_iter; ++it) {
    rc = slot_iteration_impl(W, it == 0 ? slots0 : slots_out, ws + L.sb, it == 0, k, d, M * d, vt, Mp, d * Mp, true,
                             slots_out, B, N, M, d, hidden, scale, logit_clamp, renorm_eps, slot_clamp, dtype, ws, L,
                             st, kq);
    if (rc) return rc;
  }
  return 0;
}

extern "C" int64_t hclsm_slot_attention_k_offset(int64_t B, int64_t N, int64_t M, int64_t d_in, int64_t d,
                                                 int64_t hidden, int dtype) {
  if (B < 0 || N < 0 || M < 1 || d < 1 || hidden < 1 || d_in < 1) return HCLSM_ERR_SHAPE;
  if (dtype != HCLSM_BF16 && dtype != HCLSM_F16 && dtype != HCLSM_F32) return HCLSM_ERR_DTYPE;
  return (int64_t)slot_ws_layout(B, N, M, d, hidden, dtype == HCLSM_F32 ? 4 : 2, true, d_in).kv;
}

extern "C" int64_t hclsm_slot_attention_kq_offset(int64_t B, int64_t N, int64_t M, int64_t d_in, int64_t d,
                                                  int64_t hidden, int dtype) {
  if (B < 0 || N < 0 || M < 1 || d < 1 || hidden < 1 || d_in < 1) return HCLSM_ERR_SHAPE;
  if (dtype != HCLSM_BF16 && dtype != HCLSM_F16 && dtype != HCLSM_F32) return HCLSM_ERR_DTYPE;
  const SlotWs L = slot_ws_layout(B, N, M, d, hidden, dtype == HCLSM_F32 ? 4 : 2, true, d_in);
  return kq_formed(L, B, N, M, d, dtype) ? (int64_t)L.kq : (int64_t)HCLSM_ERR_UNSUPPORTED;
}

extern "C" int hclsm_slot_attention_forward(const HclsmSlotWeights* W, const float* inputs, int64_t d_in,
                                            const float* slots0, float* slots_out, int64_t B, int64_t N, int64_t M,
                                            int64_t d, int64_t hidden, int64_t n_iter, float scale, float logit_clamp,
                                            float renorm_eps, float slot_clamp, int dtype, void* workspace,
                                            int64_t workspace_bytes, void* stream) {
  return slot_forward_impl(W, inputs, d_in, slots0, slots_out, B, N, M, d, hidden, n_iter, scale, logit_clamp,
                           renorm_eps, slot_clamp, dtype, workspace, workspace_bytes, stream);
}

// ---------------------------------------------------------------------------
// Allocation-free forward: the same launches, with the workspace in a static device array.
//
// `scratch` is a file-scope device array: every GPU the library runs on holds its own copy, at its
// own address, from the code object's load until the process ends.  Its host-side name is not a device
// address, so host code only ever passes scratch_ptr[dev], the address hipGetSymbolAddress returns with
// that device current.  The forward needs no zeroed memory (every workspace region is written before it
// is read), so nothing is cleared between calls.  Calls that overlap on one GPU share the array and race.

static __device__ __align__(256) unsigned char scratch[HCLSM_SLOT_NOALLOC_SCRATCH_BYTES];

static std::mutex scratch_mu;
static void* scratch_ptr[HCLSM_MAX_DEVICES];

// Device address of the current device's scratch array, looked up once per device.
static int current_scratch(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= HCLSM_MAX_DEVICES) return HCLSM_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (p == nullptr) return HCLSM_ERR_NULL;
    scratch_ptr[dev] = p;
  }
  *out = scratch_ptr[dev];
  return 0;
}

extern "C" int hclsm_slot_attention_forward_noalloc(const HclsmSlotWeights* W, const float* inputs, int64_t d_in,
                                                    const float* slots0, float* slots_out, int64_t B, int64_t N,
                                                    int64_t M, int64_t d, int64_t hidden, int64_t n_iter, float scale,
                                                    float logit_clamp, float renorm_eps, float slot_clamp, int dtype,
                                                    void* stream) {
  if (B < 0 || N < 0 || M < 0 || d_in < 0 || d < 0 || hidden < 0) return HCLSM_ERR_SHAPE;
  const int64_t need = (int64_t)slot_ws_layout(B, N, M, d, hidden, dtype == HCLSM_F32 ? 4 : 2, true, d_in).total;
  if (need > HCLSM_SLOT_NOALLOC_SCRATCH_BYTES) return HCLSM_ERR_SCRATCH;
  void* ws = nullptr;
  const int rc = current_scratch(&ws);
  if (rc) return rc;
  return slot_forward_impl(W, inputs, d_in, slots0, slots_out, B, N, M, d, hidden, n_iter, scale, logit_clamp,
                           renorm_eps, slot_clamp, dtype, ws, HCLSM_SLOT_NOALLOC_SCRATCH_BYTES, stream);
}
