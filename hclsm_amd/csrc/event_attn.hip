// Variable-length event attention for gfx950 (MFMA).
//
// A "segment" p is a list of rows of a [P, T, H, dh] tensor given by int32
// offsets/indices (the event index): rows (p, indices[offsets[p] + i]), i < L_p.
//   TRACK_CAUSAL: query i attends keys j <= i of its segment (benchmark config 3/4).
//   SLOTS:        query i attends every key j of its segment not flagged in
//                 key_pad[p, j] (the N x N attention of Level-1, level1_event.py:37-52).
//
// One wave owns one (segment, head) and walks 16-row query tiles x 16-row key
// tiles with an online softmax.  Scores are formed transposed, S^T = K Q^T, and the
// output as O^T = V^T P^T, both with v_mfma_f32_16x16x16_{bf16,f16} (or the
// 16x16x4 f32 form for fp32 inputs).  With that orientation every lane owns one
// query row (i = lane % 16) in all three tiles:
//   S^T tile  : lane holds keys j = 4g + r (g = lane / 16, r = 0..3) of its query,
//   P^T       : those same values are exactly the B operand of the O^T product,
//   O^T tile  : lane holds dh/4 contiguous output columns of its query row.
// The head dimension inside the K.Q^T contraction is permuted so that a lane's
// K and Q operands are dh/4 contiguous elements of one row, and the output
// columns are permuted so that the lane's V operand is dh/16 contiguous elements
// per key and its output is dh/4 contiguous elements: every global access of the
// kernel is a contiguous per-lane vector, and no LDS or barrier is needed.
// Softmax statistics (max, sum) are per query: reduced over r in-lane and over
// the four lanes {i, i+16, i+32, i+48} with the row-swap permutes (rows4_max / rows4_sum).
#include "internal.h"

namespace hclsm {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Element-type traits: KPL = k-values per lane per MFMA (K = 4*KPL).
template <int DT> struct AttnT;
template <> struct AttnT<HCLSM_BF16> {
  using T = uint16_t;
  static constexpr int KPL = 4;
  using Op = s16x4;
  static __device__ __forceinline__ float f(T v) { return bf16_bits_to_f32(v); }
  static __device__ __forceinline__ T from(float v) { return f32_to_bf16_bits(v); }
  static __device__ __forceinline__ Op pack(const T* e) {
    Op o;
    o[0] = (short)e[0]; o[1] = (short)e[1]; o[2] = (short)e[2]; o[3] = (short)e[3];
    return o;
  }
  static __device__ __forceinline__ Op pack_f(const float* x) {
    T e[4] = {from(x[0]), from(x[1]), from(x[2]), from(x[3])};
    return pack(e);
  }
  static __device__ __forceinline__ f32x4 mfma(Op a, Op b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
  }
};
template <> struct AttnT<HCLSM_F16> {
  using T = _Float16;
  static constexpr int KPL = 4;
  using Op = f16x4;
  static __device__ __forceinline__ float f(T v) { return (float)v; }
  static __device__ __forceinline__ T from(float v) { return (_Float16)v; }
  static __device__ __forceinline__ Op pack(const T* e) {
    Op o;
    o[0] = e[0]; o[1] = e[1]; o[2] = e[2]; o[3] = e[3];
    return o;
  }
  static __device__ __forceinline__ Op pack_f(const float* x) {
    Op o;
    o[0] = (_Float16)x[0]; o[1] = (_Float16)x[1]; o[2] = (_Float16)x[2]; o[3] = (_Float16)x[3];
    return o;
  }
  static __device__ __forceinline__ f32x4 mfma(Op a, Op b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
  }
};
template <> struct AttnT<HCLSM_F32> {
  using T = float;
  static constexpr int KPL = 1;
  using Op = float;
  static __device__ __forceinline__ float f(T v) { return v; }
  static __device__ __forceinline__ T from(float v) { return v; }
  static __device__ __forceinline__ Op pack(const T* e) { return e[0]; }
  static __device__ __forceinline__ Op pack_f(const float* x) { return x[0]; }
  static __device__ __forceinline__ f32x4 mfma(Op a, Op b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
};

constexpr int ATTN_WAVES = 4;

// Output element acc / l: a rounded fp32 product, then the conversion.  The empty asm statement keeps the
// compiler from fusing the two into one mixed-precision FMA (a single rounding) in some kernels and not in
// others, so every kernel here writes the same bits for the same tile.
template <typename A>
__device__ __forceinline__ typename A::T attn_out(float acc, float inv) {
  float y = acc * inv;
  asm volatile("" : "+v"(y));
  return A::from(y);
}

// Load n contiguous elements (n a compile-time constant) from p into e[].
template <typename T, int N>
__device__ __forceinline__ void load_row(const T* __restrict__ p, T* e) {
#pragma unroll
  for (int i = 0; i < N; ++i) e[i] = p[i];
}

// MODE 2 (uniform segments, the packed Level-1 layout): segment p < *nseg_dev is rows p*T .. p*T+T-1 of
// q / k / v (row stride ldi elements) and of out_packed (row stride ldo); key j of segment p is live iff
// obj_mask is null or obj_mask[seg_rows[p] * T + j] > 0.5.  Unused by modes 0 / 1.
struct AttnExt {
  const int32_t* nseg_dev;
  int64_t ldi, ldo;
  const float* obj_mask;
  const int32_t* seg_rows;
};

// MODE 3 (track-causal, packed output, index built in the launch): track p's events are read from row p of
// the mask (rule as hclsm_event_index), its packed offset is the sum of counts[0, p) (row counts from an
// earlier launch), and the head-0 wave of each track writes the track's part of the index tables
// (offsets, indices, rows, slot_of); wave 0 also writes stats {total, largest count} and offsets[nseg].
struct AttnIdx {
  const void* mask;
  int mask_dtype, rule;
  const int32_t* counts;
  int32_t *offsets, *indices, *rows, *slot_of, *stats;
};
constexpr int ATTN_IDX_TMAX = 1024;   // MODE 3: timesteps per track held in LDS
// MODE 3: every wave sums the counts of the tracks before its own (P^2 H / 2 loads over a launch), so it is taken
// only up to this many tracks; more take the index build (one prefix per workgroup of rows) and mode 0.
constexpr int64_t ATTN_IDX_MAX_TRACKS = 4096;

template <int DT, int DH, int MODE>
__global__ void __launch_bounds__(64 * ATTN_WAVES)
event_attn_kernel(const typename AttnT<DT>::T* __restrict__ q, const typename AttnT<DT>::T* __restrict__ k,
                  const typename AttnT<DT>::T* __restrict__ v, typename AttnT<DT>::T* __restrict__ out_packed,
                  typename AttnT<DT>::T* __restrict__ out_grid, const int32_t* __restrict__ offsets,
                  const int32_t* __restrict__ indices, const uint8_t* __restrict__ key_pad,
                  int64_t nseg, int64_t T, int H, int64_t capacity, float scale_log2, AttnExt ex,
                  AttnIdx ix) {
  using A = AttnT<DT>;
  using TT = typename A::T;
  constexpr int QD = DH / 4;          // contiguous head columns per lane
  constexpr int NT = DH / 16;         // output tiles of 16 columns
  constexpr int KPL = A::KPL;
  constexpr int NCH = QD / KPL;       // MFMAs per 16x16 score tile
  static_assert(DH % 16 == 0, "head dim must be a multiple of 16");

  const int64_t wave = (int64_t)blockIdx.x * ATTN_WAVES + (threadIdx.x >> 6);
  __shared__ int32_t s_idx[MODE == 3 ? ATTN_WAVES * ATTN_IDX_TMAX : 1];
  if (wave >= nseg * H) return;  // whole wave exits
  const int64_t p = wave / H;
  const int h = (int)(wave - p * H);
  const int lane = threadIdx.x & 63, g = lane >> 4, li = lane & 15;
  int64_t base;
  int L;
  int32_t* sidx = s_idx + (MODE == 3 ? (threadIdx.x >> 6) * ATTN_IDX_TMAX : 0);
  if constexpr (MODE == 3) {
    // events of row p, ascending, into this wave's LDS list (the head-0 wave also fills the tables)
    const bool hw = h == 0;
    int run = 0;
    for (int64_t t0 = 0; t0 < T; t0 += 64) {
      const int64_t t = t0 + lane;
      const bool ev = t < T && is_event(ix.mask, ix.mask_dtype, p * T + (t < T ? t : T - 1), ix.rule);
      const uint64_t bal = __ballot(ev);
      const int r = run + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                        __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
      if (ev) sidx[r] = (int32_t)t;
      if (hw && t < T && ix.slot_of) ix.slot_of[p * T + t] = ev ? r : -1;
      run += __popcll(bal);
    }
    // packed offset: events of rows 0 .. p-1
    int32_t pre = 0;
    for (int64_t i0 = lane; i0 < p; i0 += 64 * 8) {
      int32_t c[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) c[u] = i0 + 64 * u < p ? ix.counts[i0 + 64 * u] : 0;
#pragma unroll
      for (int u = 0; u < 8; ++u) pre += c[u];
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) pre += __shfl_xor(pre, o, 64);
    base = pre;
    L = run;
    __builtin_amdgcn_wave_barrier();   // the list is read back by other lanes of this wave
    if (hw) {
      for (int e = lane; e < L; e += 64) {
        ix.indices[pre + e] = sidx[e];
        if (ix.rows) ix.rows[pre + e] = (int32_t)p;
      }
      if (lane == 0) {
        ix.offsets[p] = pre;
        if (p == nseg - 1) ix.offsets[nseg] = pre + L;
      }
    }
    if (wave == 0) {   // totals over every row
      int32_t tot = 0, mx = 0;
      for (int64_t i0 = lane; i0 < nseg; i0 += 64 * 8) {
        int32_t c[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) c[u] = i0 + 64 * u < nseg ? ix.counts[i0 + 64 * u] : 0;
#pragma unroll
        for (int u = 0; u < 8; ++u) { tot += c[u]; mx = c[u] > mx ? c[u] : mx; }
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        tot += __shfl_xor(tot, o, 64);
        const int u = __shfl_xor(mx, o, 64);
        mx = u > mx ? u : mx;
      }
      if (lane == 0) { ix.stats[0] = tot; ix.stats[1] = mx; }
    }
  } else if constexpr (MODE == 2) {
    if (p >= *ex.nseg_dev) return;
    base = p * T;
    L = (int)T;
  } else {
    base = offsets[p];
    L = offsets[p + 1] - (int32_t)base;
  }
  if (L <= 0) return;
  const int64_t rstride = (int64_t)H * DH;
  const int64_t ldi = MODE == 2 ? ex.ldi : rstride, ldo = MODE == 2 ? ex.ldo : rstride;
  auto row_ptr = [&](const TT* t, int i) -> const TT* {
    const int ic = i < L ? i : L - 1;  // clamp: always a valid row of this segment
    if constexpr (MODE == 2) return t + (base + ic) * ldi + (int64_t)h * DH;
    int64_t tr = MODE == 3 ? sidx[ic] : indices[base + ic];
    tr = tr < 0 ? 0 : (tr >= T ? T - 1 : tr);
    return t + ((int64_t)p * T + tr) * rstride + (int64_t)h * DH;
  };
  const float* om = MODE == 2 && ex.obj_mask ? ex.obj_mask + (int64_t)ex.seg_rows[p] * T : nullptr;

  const int nqt = (L + 15) >> 4;
  for (int qt = 0; qt < nqt; ++qt) {
    const int i = qt * 16 + li;
    TT qe[QD];
    load_row<TT, QD>(row_ptr(q, i) + g * QD, qe);
    float m = -INFINITY, l = 0.f;
    float acc[4][NT];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) acc[r][nt] = 0.f;

    const int kt_end = (MODE == 0 || MODE == 3) ? qt : nqt - 1;   // MODE 0 / 3 = track-causal
    for (int kt = 0; kt <= kt_end; ++kt) {
      // the tile's K and V rows are requested together, so their latencies overlap (segments here are
      // short: one key tile is the common case)
      TT ke[QD];
      load_row<TT, QD>(row_ptr(k, kt * 16 + li) + g * QD, ke);
      // V operand: keys j = kt*16 + 4g + r, columns NT*li .. NT*li + NT - 1
      TT ve[4][NT];
#pragma unroll
      for (int r = 0; r < 4; ++r) load_row<TT, NT>(row_ptr(v, kt * 16 + 4 * g + r) + NT * li, ve[r]);
      f32x4 s4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NCH; ++c) s4 = A::mfma(A::pack(ke + c * KPL), A::pack(qe + c * KPL), s4);
      // s4[r] = S[query i][key j = kt*16 + 4g + r]
      float s[4];
      float tmax = -INFINITY;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = kt * 16 + 4 * g + r;
        bool ok = (i < L) && (j < L);
        if (MODE == 0 || MODE == 3) ok = ok && (j <= i);
        else if (MODE == 2) ok = ok && (om == nullptr || om[j < L ? j : L - 1] > 0.5f);
        else if (key_pad != nullptr) {
          int64_t tj = indices[base + (j < L ? j : L - 1)];
          tj = tj < 0 ? 0 : (tj >= T ? T - 1 : tj);
          ok = ok && (key_pad[p * T + tj] == 0);
        }
        s[r] = ok ? s4[r] * scale_log2 : -INFINITY;
        tmax = fmaxf(tmax, s[r]);
      }
      tmax = rows4_max(tmax);
      const float m_new = fmaxf(m, tmax);
      float pr[4], psum = 0.f;
      float alpha = 1.f;
      if (m_new != -INFINITY) {
        alpha = fast_exp2(m - m_new);   // m == -inf -> 0
#pragma unroll
        for (int r = 0; r < 4; ++r) { pr[r] = fast_exp2(s[r] - m_new); psum += pr[r]; }
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) pr[r] = 0.f;
      }
      psum = rows4_sum(psum);
      l = l * alpha + psum;
      m = m_new;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        f32x4 o4 = {acc[0][nt] * alpha, acc[1][nt] * alpha, acc[2][nt] * alpha, acc[3][nt] * alpha};
        if constexpr (KPL == 4) {
          TT a_e[4] = {ve[0][nt], ve[1][nt], ve[2][nt], ve[3][nt]};
          o4 = A::mfma(A::pack(a_e), A::pack_f(pr), o4);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) o4 = A::mfma(ve[r][nt], pr[r], o4);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r][nt] = o4[r];
      }
    }
    if (i < L) {
      const float inv = 1.f / l;   // l == 0 (every key padded) -> NaN output, as softmax over all -inf
      TT o[QD];
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) o[r * NT + nt] = attn_out<A>(acc[r][nt], inv);
      if (out_packed && base + i < capacity) {
        TT* dst = out_packed + (base + i) * ldo + (int64_t)h * DH + g * QD;
#pragma unroll
        for (int e = 0; e < QD; ++e) dst[e] = o[e];
      }
      if (MODE < 2 && out_grid) {
        int64_t tr = indices[base + i];
        tr = tr < 0 ? 0 : (tr >= T ? T - 1 : tr);
        TT* dst = out_grid + ((int64_t)p * T + tr) * rstride + (int64_t)h * DH + g * QD;
#pragma unroll
        for (int e = 0; e < QD; ++e) dst[e] = o[e];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Track-causal attention over long tracks (T > ATTN_PAIR_MIN_T) from a prebuilt index (mode 0, packed output),
// with the K/V rows that get re-read staged in LDS.
//
// One workgroup holds two (track, head) units, each served by a pair of waves.  A track of n 16-row query
// tiles reads key tile kt once for every query tile qt >= kt; tiles 0 .. n-2 are read again, the last tile
// only once.  The pair therefore first copies rows 0 .. 16(n-1) - 1 of its unit's K and V (at most CAP rows)
// from HBM into LDS, once, then both waves take their share of the query tiles and read those key tiles from
// LDS; the last key tile, and any past CAP, come from global memory as in event_attn_kernel.  Every K/V row
// then crosses HBM once (n(n+1)/2 tile reads per track otherwise, of which L2 keeps about half at config 4).
// The two waves split the query tiles so that their key-tile counts match: counting tiles back from the last
// one, a wave takes those at positions 0 and 3 (mod 4), the other those at 1 and 2 (n = 4: tiles 3, 0 against
// 2, 1, 5 key tiles each).  Per tile the arithmetic is event_attn_kernel's, in the same order, so the outputs
// are identical.
//
// LDS rows are stored swizzled (pair_swz), so that the K operand reads (16 rows, the same two chunks each) and
// the V operand reads (four rows of consecutive chunks) spread over the banks.
constexpr int ATTN_PAIR_MIN_T = 64;     // tracks of at most 64 steps (<= 4 query tiles) stay on event_attn_kernel
constexpr int PAIR_KV_BYTES = 6144;     // per unit and tensor: 48 rows of a 64-column 16-bit head

// Chunk index of (row, chunk) in a unit's LDS rows.  The chunk is XORed with the row's low bits, and rows 2m, 2m+1
// trade places when bits 2 and 3 of the row differ, so that in one 256-byte bank cycle the K reads (rows R and R+8,
// same chunks) and the V reads (rows R and R+4, whole rows) fall in different halves of the banks.
__device__ __forceinline__ int pair_swz(int row, int chunk, int cpr) {
  const int prow = row ^ (((row >> 2) ^ (row >> 3)) & 1);
  return prow * cpr + (chunk ^ (row & (cpr - 1)));
}
template <int NB> struct LdsWord;
template <> struct LdsWord<4> { using T = uint32_t; };
template <> struct LdsWord<8> { using T = uint2; };
template <> struct LdsWord<16> { using T = uint4; };

template <int DT, int DH>
__global__ void __launch_bounds__(256, 5)
event_attn_pair_kernel(const typename AttnT<DT>::T* __restrict__ q, const typename AttnT<DT>::T* __restrict__ k,
                       const typename AttnT<DT>::T* __restrict__ v, typename AttnT<DT>::T* __restrict__ out_packed,
                       const int32_t* __restrict__ offsets, const int32_t* __restrict__ indices, int64_t nseg,
                       int64_t T, int H, int64_t capacity, float scale_log2) {
  using A = AttnT<DT>;
  using TT = typename A::T;
  constexpr int QD = DH / 4;
  constexpr int NT = DH / 16;
  constexpr int KPL = A::KPL;
  constexpr int NCH = QD / KPL;
  constexpr int ROWB = DH * (int)sizeof(TT);          // bytes of one head row
  constexpr int CPR = ROWB / 16;                        // 16-byte chunks per row
  constexpr int CAP = PAIR_KV_BYTES / ROWB;             // rows staged per unit
  static_assert((CPR & (CPR - 1)) == 0, "chunks per row: a power of two");
  static_assert(CAP % 2 == 0, "pair_swz trades rows in pairs");
  static_assert(QD * (int)sizeof(TT) % 16 == 0 && 16 % (NT * (int)sizeof(TT)) == 0, "operand widths");

  __shared__ __attribute__((aligned(16))) uint8_t s_kv[2][2][PAIR_KV_BYTES];   // [unit][K, V]

  const int wv = threadIdx.x >> 6, pr = wv >> 1, half = wv & 1;
  const int lane = threadIdx.x & 63, g = lane >> 4, li = lane & 15;
  const int64_t unit = (int64_t)blockIdx.x * 2 + pr;
  const bool live = unit < nseg * H;
  const int64_t p = live ? unit / H : 0;
  const int h = live ? (int)(unit - p * H) : 0;
  int64_t base = 0;
  int L = 0;
  if (live) {
    base = offsets[p];
    L = offsets[p + 1] - (int32_t)base;
  }

  const int64_t rstride = (int64_t)H * DH;
  auto row_of = [&](int i) -> int64_t {   // time step of the segment's row i (clamped to a valid row)
    const int ic = i < L ? i : L - 1;
    const int64_t tr = indices[base + ic];
    return tr < 0 ? 0 : (tr >= T ? T - 1 : tr);
  };
  auto gptr = [&](const TT* t, int i) -> const TT* { return t + (p * T + row_of(i)) * rstride + (int64_t)h * DH; };

  // stage rows 0 .. Ls - 1 of K and V, 16-byte chunks over the pair's 128 lanes: at most CAP rows, and not
  // the last key tile, which only the last query tile reads
  const int nqt = (L + 15) >> 4;
  const int Ls = (nqt - 1) * 16 < CAP ? (nqt - 1) * 16 : CAP;
  {
    const int lt = half * 64 + lane;
    uint8_t* sk = s_kv[pr][0];
    uint8_t* sv = s_kv[pr][1];
    auto gchunk = [&](const TT* t, int c) -> uint4 {
      const int row = c / CPR, ch = c - row * CPR;
      const int64_t go = (p * T + row_of(row)) * rstride + (int64_t)h * DH;
      return *reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(t + go) + ch * 16);
    };
    auto put = [&](uint8_t* dst, int c, uint4 w) {
      const int row = c / CPR, ch = c - row * CPR;
      *reinterpret_cast<uint4*>(dst + pair_swz(row, ch, CPR) * 16) = w;
    };
    const int nch = Ls * CPR;
    for (int c0 = lt; c0 < nch; c0 += 256) {   // two chunks of K and of V in flight per lane
      const int c1 = c0 + 128;
      const bool two = c1 < nch;
      const uint4 k0 = gchunk(k, c0), v0 = gchunk(v, c0);
      const uint4 k1 = gchunk(k, two ? c1 : c0), v1 = gchunk(v, two ? c1 : c0);
      put(sk, c0, k0);
      put(sv, c0, v0);
      if (two) {
        put(sk, c1, k1);
        put(sv, c1, v1);
      }
    }
  }
  __syncthreads();   // staged rows of both units
  if (!live || L <= 0) return;

  const uint8_t* sk = s_kv[pr][0];
  const uint8_t* sv = s_kv[pr][1];
  constexpr int EPC = 16 / (int)sizeof(TT);   // elements per 16-byte chunk
  using VW = typename LdsWord<NT * (int)sizeof(TT)>::T;
  // K operand (QD elements of row i from element e0) and V operand (NT elements of row i from element e0,
  // inside one chunk).  A key tile whose rows all lie below CAP reads LDS, any other tile global memory (the
  // choice is uniform over the wave).
  auto ld_k = [&](bool lds, int i, int e0, TT* e) {
    if (lds) {
      const int ic = i < L ? i : L - 1;
#pragma unroll
      for (int c = 0; c < QD / EPC; ++c) {
        const uint4 w = *reinterpret_cast<const uint4*>(sk + pair_swz(ic, e0 / EPC + c, CPR) * 16);
        __builtin_memcpy(e + c * EPC, &w, 16);
      }
    } else {
      load_row<TT, QD>(gptr(k, i) + e0, e);
    }
  };
  auto ld_v = [&](bool lds, int i, int e0, TT* e) {
    if (lds) {
      const int ic = i < L ? i : L - 1;
      const VW w = *reinterpret_cast<const VW*>(sv + pair_swz(ic, e0 / EPC, CPR) * 16 + (e0 % EPC) * (int)sizeof(TT));
      __builtin_memcpy(e, &w, sizeof(VW));
    } else {
      load_row<TT, NT>(gptr(v, i) + e0, e);
    }
  };

  for (int back = 0; back < nqt; ++back) {
    const int pos = back & 3;
    if (((pos == 0 || pos == 3) ? 0 : 1) != half) continue;
    const int qt = nqt - 1 - back;
    const int i = qt * 16 + li;
    TT qe[QD];
    load_row<TT, QD>(gptr(q, i) + g * QD, qe);
    float m = -INFINITY, l = 0.f;
    float acc[4][NT];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) acc[r][nt] = 0.f;
    for (int kt = 0; kt <= qt; ++kt) {
      const bool lds = (kt + 1) * 16 <= Ls;
      TT ke[QD];
      ld_k(lds, kt * 16 + li, g * QD, ke);
      TT ve[4][NT];
#pragma unroll
      for (int r = 0; r < 4; ++r) ld_v(lds, kt * 16 + 4 * g + r, NT * li, ve[r]);
      f32x4 s4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NCH; ++c) s4 = A::mfma(A::pack(ke + c * KPL), A::pack(qe + c * KPL), s4);
      float s[4];
      float tmax = -INFINITY;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = kt * 16 + 4 * g + r;
        const bool ok = (i < L) && (j < L) && (j <= i);
        s[r] = ok ? s4[r] * scale_log2 : -INFINITY;
        tmax = fmaxf(tmax, s[r]);
      }
      tmax = rows4_max(tmax);
      const float m_new = fmaxf(m, tmax);
      float prb[4], psum = 0.f;
      float alpha = 1.f;
      if (m_new != -INFINITY) {
        alpha = fast_exp2(m - m_new);
#pragma unroll
        for (int r = 0; r < 4; ++r) { prb[r] = fast_exp2(s[r] - m_new); psum += prb[r]; }
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) prb[r] = 0.f;
      }
      psum = rows4_sum(psum);
      l = l * alpha + psum;
      m = m_new;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        f32x4 o4 = {acc[0][nt] * alpha, acc[1][nt] * alpha, acc[2][nt] * alpha, acc[3][nt] * alpha};
        if constexpr (KPL == 4) {
          TT a_e[4] = {ve[0][nt], ve[1][nt], ve[2][nt], ve[3][nt]};
          o4 = A::mfma(A::pack(a_e), A::pack_f(prb), o4);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) o4 = A::mfma(ve[r][nt], prb[r], o4);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r][nt] = o4[r];
      }
    }
    if (i < L && base + i < capacity) {
      const float inv = 1.f / l;
      TT o[QD];
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) o[r * NT + nt] = attn_out<A>(acc[r][nt], inv);
      TT* dst = out_packed + (base + i) * rstride + (int64_t)h * DH + g * QD;
#pragma unroll
      for (int e = 0; e < QD; ++e) dst[e] = o[e];
    }
  }
}

// The staged-K/V kernel takes 16-bit heads of 32..128 columns and fp32 heads of 16..64, with 16-byte aligned
// q / k / v (each row's head slice is then a whole number of 16-byte chunks).
template <int DT, int DH>
constexpr bool pair_ok() {
  return DT == HCLSM_F32 ? (DH >= 16 && DH <= 64) : (DH >= 32 && DH <= 128);
}
static inline bool al16(const void* a) { return (((uintptr_t)a) & 15) == 0; }

template <int DT, int DH>
static int launch_attn_pair(const void* q, const void* k, const void* v, void* outp, const int32_t* offsets,
                            const int32_t* indices, int64_t nseg, int64_t T, int H, int64_t cap, float scale,
                            hipStream_t st) {
  using TT = typename AttnT<DT>::T;
  const unsigned grid = (unsigned)((nseg * H + 1) / 2);
  hipLaunchKernelGGL((event_attn_pair_kernel<DT, DH>), dim3(grid), dim3(256), 0, st, (const TT*)q, (const TT*)k,
                     (const TT*)v, (TT*)outp, offsets, indices, nseg, T, H, cap, scale * HCLSM_LOG2E);
  HCLSM_LAUNCH_CHECK();
  return 0;
}

template <int DT, int DH>
static int launch_attn(int mode, const void* q, const void* k, const void* v, void* outp, void* outg,
                       const int32_t* offsets, const int32_t* indices, const uint8_t* kp, int64_t nseg,
                       int64_t T, int H, int64_t cap, float scale, hipStream_t st) {
  using TT = typename AttnT<DT>::T;
  const int64_t waves = nseg * H;
  const unsigned grid = (unsigned)((waves + ATTN_WAVES - 1) / ATTN_WAVES);
  const float sl2 = scale * HCLSM_LOG2E;
  if constexpr (pair_ok<DT, DH>()) {
    if (mode == HCLSM_ATTN_TRACK_CAUSAL && T > ATTN_PAIR_MIN_T && outp && !outg && al16(q) && al16(k) && al16(v) &&
        al16(outp))
      return launch_attn_pair<DT, DH>(q, k, v, outp, offsets, indices, nseg, T, H, cap, scale, st);
  }
  if (mode == HCLSM_ATTN_TRACK_CAUSAL)
    hipLaunchKernelGGL((event_attn_kernel<DT, DH, 0>), dim3(grid), dim3(64 * ATTN_WAVES), 0, st, (const TT*)q,
                       (const TT*)k, (const TT*)v, (TT*)outp, (TT*)outg, offsets, indices, kp, nseg, T, H, cap, sl2,
                       AttnExt{}, AttnIdx{});
  else
    hipLaunchKernelGGL((event_attn_kernel<DT, DH, 1>), dim3(grid), dim3(64 * ATTN_WAVES), 0, st, (const TT*)q,
                       (const TT*)k, (const TT*)v, (TT*)outp, (TT*)outg, offsets, indices, kp, nseg, T, H, cap, sl2,
                       AttnExt{}, AttnIdx{});
  HCLSM_LAUNCH_CHECK();
  return 0;
}

// MODE 3 launch (track-causal, packed, index built in the launch; T <= ATTN_PAIR_MIN_T).
template <int DT, int DH>
static int launch_attn_idx(const void* q, const void* k, const void* v, void* outp, int64_t nseg, int64_t T, int H,
                           int64_t cap, float scale, const AttnIdx& ix, hipStream_t st) {
  using TT = typename AttnT<DT>::T;
  const unsigned grid = (unsigned)((nseg * H + ATTN_WAVES - 1) / ATTN_WAVES);
  hipLaunchKernelGGL((event_attn_kernel<DT, DH, 3>), dim3(grid), dim3(64 * ATTN_WAVES), 0, st, (const TT*)q,
                     (const TT*)k, (const TT*)v, (TT*)outp, (TT*)nullptr, nullptr, nullptr, nullptr, nseg, T, H, cap,
                     scale * HCLSM_LOG2E, AttnExt{}, ix);
  HCLSM_LAUNCH_CHECK();
  return 0;
}

template <int DT>
static int dispatch_idx(int dh, const void* q, const void* k, const void* v, void* outp, int64_t nseg, int64_t T,
                        int H, int64_t cap, float scale, const AttnIdx& ix, hipStream_t st) {
  switch (dh) {
    case 16: return launch_attn_idx<DT, 16>(q, k, v, outp, nseg, T, H, cap, scale, ix, st);
    case 32: return launch_attn_idx<DT, 32>(q, k, v, outp, nseg, T, H, cap, scale, ix, st);
    case 64: return launch_attn_idx<DT, 64>(q, k, v, outp, nseg, T, H, cap, scale, ix, st);
    case 128: return launch_attn_idx<DT, 128>(q, k, v, outp, nseg, T, H, cap, scale, ix, st);
    default: return HCLSM_ERR_UNSUPPORTED;
  }
}

template <int DT>
static int dispatch_dh(int dh, int mode, const void* q, const void* k, const void* v, void* outp, void* outg,
                       const int32_t* offsets, const int32_t* indices, const uint8_t* kp, int64_t nseg,
                       int64_t T, int H, int64_t cap, float scale, hipStream_t st) {
  switch (dh) {
    case 16: return launch_attn<DT, 16>(mode, q, k, v, outp, outg, offsets, indices, kp, nseg, T, H, cap, scale, st);
    case 32: return launch_attn<DT, 32>(mode, q, k, v, outp, outg, offsets, indices, kp, nseg, T, H, cap, scale, st);
    case 64: return launch_attn<DT, 64>(mode, q, k, v, outp, outg, offsets, indices, kp, nseg, T, H, cap, scale, st);
    case 128: return launch_attn<DT, 128>(mode, q, k, v, outp, outg, offsets, indices, kp, nseg, T, H, cap, scale, st);
    default: return HCLSM_ERR_UNSUPPORTED;
  }
}

// Packed Level-1 attention (MODE 2), for composite entry points in other files (declared in internal.h):
// cap segments of N rows, the first *nseg_dev of them live; q / k / v rows with stride ldi, out rows ldo.
int attn_slots_packed(const void* q, const void* k, const void* v, int64_t ldi, void* out, int64_t ldo,
                      const int32_t* nseg_dev, int64_t cap, int64_t N, int H, int dh, const float* obj_mask,
                      const int32_t* seg_rows, float scale, int dtype, hipStream_t st) {
  if (cap < 0 || N <= 0 || H <= 0 || cap * N > 0x7fffffffLL) return HCLSM_ERR_SHAPE;
  if (cap == 0) return 0;
  if (!q || !k || !v || !out || !nseg_dev || (obj_mask && !seg_rows)) return HCLSM_ERR_NULL;
  const float sl2 = scale * HCLSM_LOG2E;
  const unsigned grid = (unsigned)((cap * H + ATTN_WAVES - 1) / ATTN_WAVES);
  const AttnExt ex{nseg_dev, ldi, ldo, obj_mask, seg_rows};
#define HCLSM_SP(DT_, DH_)                                                                                   \
  if (dtype == DT_ && dh == DH_) {                                                                           \
    using TT = typename AttnT<DT_>::T;                                                                       \
    hipLaunchKernelGGL((event_attn_kernel<DT_, DH_, 2>), dim3(grid), dim3(64 * ATTN_WAVES), 0, st, (const TT*)q, \
                       (const TT*)k, (const TT*)v, (TT*)out, (TT*)nullptr, nullptr, nullptr, nullptr, cap, N, H,   \
                       cap * N, sl2, ex, AttnIdx{});                                                         \
    HCLSM_LAUNCH_CHECK();                                                                                    \
    return 0;                                                                                                \
  }
#define HCLSM_SP_DT(DT_) HCLSM_SP(DT_, 16) HCLSM_SP(DT_, 32) HCLSM_SP(DT_, 64) HCLSM_SP(DT_, 128)
  HCLSM_SP_DT(HCLSM_BF16)
  HCLSM_SP_DT(HCLSM_F16)
  HCLSM_SP_DT(HCLSM_F32)
#undef HCLSM_SP_DT
#undef HCLSM_SP
  return (dh == 16 || dh == 32 || dh == 64 || dh == 128) ? HCLSM_ERR_DTYPE : HCLSM_ERR_UNSUPPORTED;
}

}  // namespace hclsm

extern "C" int hclsm_event_attention(const void* q, const void* k, const void* v, void* out_packed, void* out_grid,
                                     const int32_t* offsets, const int32_t* indices, const uint8_t* key_pad,
                                     int64_t nseg, int64_t T, int64_t H, int64_t dh, int64_t capacity,
                                     float scale, int dtype, int mode, void* stream) {
  using namespace hclsm;
  if (nseg < 0 || T < 0 || H < 0 || dh < 0 || capacity < 0 || nseg * T > 0x7fffffffLL) return HCLSM_ERR_SHAPE;
  if (mode != HCLSM_ATTN_TRACK_CAUSAL && mode != HCLSM_ATTN_SLOTS) return HCLSM_ERR_MODE;
  if (dtype != HCLSM_F32 && dtype != HCLSM_BF16 && dtype != HCLSM_F16) return HCLSM_ERR_DTYPE;
  if (dh != 16 && dh != 32 && dh != 64 && dh != 128) return HCLSM_ERR_UNSUPPORTED;
  if (nseg == 0 || H == 0 || T == 0) return 0;
  if (!out_grid && capacity == 0) return 0;   // a packed output of no rows: nothing to write
  if (!q || !k || !v || !offsets || !indices || (!out_packed && !out_grid)) return HCLSM_ERR_NULL;
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case HCLSM_BF16:
      return dispatch_dh<HCLSM_BF16>((int)dh, mode, q, k, v, out_packed, out_grid, offsets, indices, key_pad, nseg, T, (int)H, capacity, scale, st);
    case HCLSM_F16:
      return dispatch_dh<HCLSM_F16>((int)dh, mode, q, k, v, out_packed, out_grid, offsets, indices, key_pad, nseg, T, (int)H, capacity, scale, st);
    default:
      return dispatch_dh<HCLSM_F32>((int)dh, mode, q, k, v, out_packed, out_grid, offsets, indices, key_pad, nseg, T, (int)H, capacity, scale, st);
  }
}

// Index build and per-track causal attention in one call, on `stream`.  For T <= ATTN_PAIR_MIN_T and at most
// ATTN_IDX_MAX_TRACKS tracks (with heads and a packed output to write) two launches: the row counts, then the attention, whose waves read their
// track's events straight from the mask, take the packed offset from the counts and fill the index tables as
// they go.  Longer tracks: hclsm_event_index, then hclsm_event_attention over its tables, which stages the
// re-read K/V rows in LDS (event_attn_pair_kernel); there every head of a track would otherwise rank the same
// mask row again.
extern "C" int hclsm_track_causal_attention(const void* mask, int mask_dtype, int rule, const void* q,
                                            const void* k, const void* v, void* out_packed, int64_t B,
                                            int64_t T, int64_t H, int64_t dh, int64_t capacity, float scale,
                                            int dtype, int32_t* tables, void* stream) {
  using namespace hclsm;
  if (B < 0 || T < 0 || H < 0 || dh < 0 || capacity < 0 || B * T > 0x7fffffffLL) return HCLSM_ERR_SHAPE;
  if (mask_dtype < HCLSM_F32 || mask_dtype > HCLSM_U8) return HCLSM_ERR_DTYPE;
  if (dtype != HCLSM_F32 && dtype != HCLSM_BF16 && dtype != HCLSM_F16) return HCLSM_ERR_DTYPE;
  if (rule != HCLSM_EVENT_GT_HALF && rule != HCLSM_EVENT_NONZERO) return HCLSM_ERR_MODE;
  if (dh != 16 && dh != 32 && dh != 64 && dh != 128) return HCLSM_ERR_UNSUPPORTED;
  if (!tables) return HCLSM_ERR_NULL;
  const int64_t cap = B * T > 1 ? B * T : 1;
  int32_t* stats = tables;
  int32_t* counts = stats + 2;
  int32_t* offsets = counts + B;
  int32_t* indices = offsets + B + 1;
  int32_t* rows = indices + cap;
  int32_t* slot_of = rows + cap;
  if (B > 0 && T > 0 && T <= ATTN_PAIR_MIN_T && B <= ATTN_IDX_MAX_TRACKS && H > 0 && capacity > 0) {
    if (!mask || !q || !k || !v || !out_packed) return HCLSM_ERR_NULL;
    hipStream_t st = (hipStream_t)stream;
    int rc = event_counts(mask, mask_dtype, B, T, rule, counts, st);
    if (rc) return rc;
    const AttnIdx ix{mask, mask_dtype, rule, counts, offsets, indices, rows, slot_of, stats};
    switch (dtype) {
      case HCLSM_BF16: return dispatch_idx<HCLSM_BF16>((int)dh, q, k, v, out_packed, B, T, (int)H, capacity, scale, ix, st);
      case HCLSM_F16: return dispatch_idx<HCLSM_F16>((int)dh, q, k, v, out_packed, B, T, (int)H, capacity, scale, ix, st);
      default: return dispatch_idx<HCLSM_F32>((int)dh, q, k, v, out_packed, B, T, (int)H, capacity, scale, ix, st);
    }
  }
  const int rc = hclsm_event_index(mask, mask_dtype, B, T, rule, counts, offsets, indices, rows, slot_of, stats, stream);
  if (rc) return rc;
  return hclsm_event_attention(q, k, v, out_packed, nullptr, offsets, indices, nullptr, B, T, H, dh, capacity, scale,
                               dtype, HCLSM_ATTN_TRACK_CAUSAL, stream);
}
