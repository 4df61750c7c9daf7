// Selective SSM scan, backward (reverse scan) for gfx950.
//
// Gradients of L = sum(gy * y) for y_t[d] = sum_s C_t[s] h_t[d,s] (+ D[d] x_t[d]) with
// h_t = exp(dt A) h_{t-1} + dt B_t x_t:
//   gh_t   = gy_t C_t + exp(dt_{t+1} A) gh_{t+1}
//   gx_t   = dt sum_s gh_t B_t + D gy_t              gdt_t = sum_s g_arg A + x sum_s gh_t B_t
//   gB_t[s] = sum_d gh_t dt x                        gC_t[s] = sum_d gy_t h_t
//   gA[d,s] = sum_{n,t} g_arg dt   with g_arg = gh_t h_{t-1} exp(dt A)
// (model mode: each clamp passes gradient only inside its closed interval).
//
// Mapping: one lane owns channel d of sequence n and SG <= 16 of its states (G = d_state/SG lanes
// per channel, adjacent); a workgroup holds up to 384 lanes of one sequence's channels.  Pass 1
// recomputes h forward and writes the state at every chunk start (chunks of K = 32/SG steps) to a
// checkpoint buffer.  Pass 2 walks the chunks backwards: it recomputes the chunk's states into
// registers, then runs the reverse recurrence step by step.  B_t / C_t rows are staged in LDS as fp32,
// 64 steps at a time.  Sums over the state axis (gx, gdt) are DPP sums inside the G-lane group; sums
// over the channel axis (gB, gC) are a recursive-halving reduce-scatter across the wave's channels
// followed by a cross-wave sum through LDS once per chunk, one part per channel block.  One tail launch
// then reduces the per-sequence partials of gA_log and gD, and adds the blocks' gB / gC parts and casts.
#include "internal.h"

namespace hclsm {

// States per lane: all of a channel's states up to 16 (G = SP / SG adjacent lanes per channel for
// d_state 32 / 64 / 128).  Chunks of K = 64 / SG steps: the chunk's recomputed states (64 floats) stay in
// registers.
constexpr int bwd_sg(int SP) { return SP < 16 ? SP : 16; }
constexpr int bwd_k(int SP) { return 64 / bwd_sg(SP); }
// Lanes per workgroup: two waves, so whole workgroups fill the four SIMDs of a CU evenly.
constexpr int BWD_MAX_THREADS = 128;

// Channels per workgroup and workgroups per sequence: the channels of a sequence split evenly.
struct BwdGrid { int DW, nblk; };
static inline BwdGrid bwd_grid(int64_t Dn, int G) {
  const int64_t nblk = (Dn * G + BWD_MAX_THREADS - 1) / BWD_MAX_THREADS;
  const int64_t nb = nblk < 1 ? 1 : nblk;
  return BwdGrid{(int)((Dn + nb - 1) / nb), (int)nb};
}

// Value of the partner lane across bit M for the reduce-scatter steps below 16 lanes.  The partner only
// has to differ in bit M and agree in the bits above it; when every bit below M is reduced later too
// (MASK_LO == 1) the DPP mirrors are used (lane ^ 15, lane ^ 7 inside a row), else exact xor partners.
template <int M, int MASK_LO>
__device__ __forceinline__ float rs_partner(float v) {
  const int b = __float_as_int(v);
  if constexpr (M == 8) {
    return __int_as_float(MASK_LO == 1 ? __builtin_amdgcn_update_dpp(0, b, 0x140, 0xf, 0xf, true)     // row_mirror
                                       : __builtin_amdgcn_update_dpp(0, b, 0x128, 0xf, 0xf, true));   // row_ror:8
  } else if constexpr (M == 4) {
    if constexpr (MASK_LO == 1)
      return __int_as_float(__builtin_amdgcn_update_dpp(0, b, 0x141, 0xf, 0xf, true));   // row_half_mirror
    else
      return __shfl_xor(v, 4, 64);
  } else if constexpr (M == 2) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, b, 0x4e, 0xf, 0xf, true));      // quad_perm 2,3,0,1
  } else {
    static_assert(M == 1, "rs_partner: M in {1, 2, 4, 8}");
    return __int_as_float(__builtin_amdgcn_update_dpp(0, b, 0xb1, 0xf, 0xf, true));      // quad_perm 1,0,3,2
  }
}

// (lo, hi) -> lo summed over the lane pair for the lower lane, hi summed for the upper lane, where the
// pair differs in bit 5 (M == 32) or bit 4 (M == 16): one gfx950 permlane swap exchanges the halves.
template <int M>
__device__ __forceinline__ float rs_swap_sum(float lo, float hi) {
  if constexpr (M == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(lo), __float_as_uint(hi), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  } else {
    static_assert(M == 16, "rs_swap_sum: M in {16, 32}");
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(lo), __float_as_uint(hi), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
}

// Sum over the G adjacent lanes of a channel (G a power of two <= 8), every lane gets the total.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (G >= 2) v += rs_partner<1, 1>(v);
  if constexpr (G >= 4) v += rs_partner<2, 1>(v);
  if constexpr (G >= 8) v += rs_partner<4, 1>(v);   // lane ^ 7: the other quad of the 8-lane group
  static_assert(G <= 8, "group_sum: at most 8 lanes");
  return v;
}

template <int V, int MASK_LO>
struct RS {
  // Reduce-scatter V values across the lanes that differ in bits [MASK_LO, 32] of the lane id.
  // On return v[0 .. V/2^h) holds sums for value indices starting at `off` (h = halving steps).
  template <int CNT, int M>
  static __device__ __forceinline__ void step(float* v, int lane, int& off) {
    if constexpr (M >= MASK_LO) {
      if constexpr (CNT > 1) {
        const bool upper = (lane & M) != 0;
#pragma unroll
        for (int i = 0; i < CNT / 2; ++i) {
          if constexpr (M >= 16) {
            v[i] = rs_swap_sum<M>(v[i], v[i + CNT / 2]);
          } else {
            const float keep = upper ? v[i + CNT / 2] : v[i];
            const float send = upper ? v[i] : v[i + CNT / 2];
            v[i] = keep + rs_partner<M, MASK_LO>(send);
          }
        }
        if (upper) off += CNT / 2;
        step<CNT / 2, M / 2>(v, lane, off);
      } else {
        if constexpr (M >= 16) v[0] = rs_swap_sum<M>(v[0], v[0]);
        else v[0] += rs_partner<M, MASK_LO>(v[0]);
        step<1, M / 2>(v, lane, off);
      }
    }
  }
  static __device__ __forceinline__ int run(float* v, int lane) {
    int off = 0;
    step<V, 32>(v, lane, off);
    return off;
  }
};

template <int N_, int MASK_LO> struct RSCount {  // values left per lane after RS
  static constexpr int h(int cnt, int m) { return (m < MASK_LO || cnt <= 1) ? cnt : h(cnt / 2, m / 2); }
  static constexpr int value = h(N_, 32);
};

struct BwdArgs {
  int T, Dn, S, nchunk, nck, DW;   // nck = checkpoints per sequence = ceil(nchunk / BWD_CKR)
  int64_t ld_ck;  // floats per (n, checkpoint) slab = Dn * SP, state-major: state s of channel d at s * Dn + d
  int have_ck;    // the checkpoints are already in ckpt (written by the forward): no pass 1
};

// Steps of B / C rows staged in LDS at a time (a multiple of every chunk length K).
constexpr int BWD_WT = 64;
// Chunks per checkpoint: pass 1 stores the state at the start of every BWD_CKR-th chunk, and pass 2 steps
// forward from there to the start of the chunks in between.  Checkpoints are the largest HBM stream of the
// backward (16 fp32 states per channel per chunk, written and read back); every other chunk halves it for
// one extra forward chunk in two.  The chunks of a checkpoint share one B / C window.
constexpr int BWD_CKR = 2;

template <int DT, int SP, int MODE>
__global__ void __launch_bounds__(BWD_MAX_THREADS)
ssm_scan_bwd_kernel(const typename Elem<DT>::T* __restrict__ x, const typename Elem<DT>::T* __restrict__ dt,
                    const float* __restrict__ A_log, const typename Elem<DT>::T* __restrict__ Bm,
                    const typename Elem<DT>::T* __restrict__ Cm, const float* __restrict__ Dskip,
                    const typename Elem<DT>::T* __restrict__ gy, typename Elem<DT>::T* __restrict__ gx,
                    typename Elem<DT>::T* __restrict__ gdt, float* __restrict__ ckpt, float* __restrict__ gbc,
                    float* __restrict__ gA_part, float* __restrict__ gD_part, BwdArgs a) {
  constexpr int ES = (int)sizeof(typename Elem<DT>::T);
  constexpr int SG = bwd_sg(SP);
  constexpr int G = SP / SG;
  constexpr int K = bwd_k(SP);
  constexpr int VL = RSCount<SG, G>::value;       // values per lane after reduce-scattering gB (then gC)
  constexpr int WMAX = BWD_MAX_THREADS / 64;
  static_assert(BWD_WT % K == 0, "an LDS window holds whole chunks");
  static_assert((BWD_WT / K) % BWD_CKR == 0, "the chunks of a checkpoint share one LDS window");
  __shared__ float red[K][WMAX][2 * SP];           // per-chunk wave partials of gB | gC
  __shared__ __align__(16) float sB[BWD_WT][SP];   // B / C rows of the current window, fp32; states >= S
  __shared__ __align__(16) float sC[BWD_WT][SP];   // and steps >= T are zero
  __shared__ float sH0[SG][BWD_MAX_THREADS];       // the chunk's starting state, read back at its first step
  const int n = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6, nw = blockDim.x >> 6;
  const int dl = tid / G, gi = tid - dl * G;
  const int d = blockIdx.y * a.DW + dl;
  const bool act = d < a.Dn && dl < a.DW;
  const int dd = act ? d : 0;
  const int s0 = gi * SG;
  const int T = a.T, Dn = a.Dn, S = a.S;

  float a2[SG];   // A * log2(e) for this lane's states (padded states: 0); A = a2 * ln 2 where needed
#pragma unroll
  for (int j = 0; j < SG; ++j) {
    const int s = s0 + j;
    const float e = expf(A_log[(size_t)dd * S + (s < S ? s : S - 1)]);
    const float ec = (MODE != HCLSM_SCAN_RAW) ? fminf(fmaxf(e, 1e-6f), 1.0f) : e;
    a2[j] = (s < S) ? -ec * HCLSM_LOG2E : 0.f;
  }
  const float dsk = Dskip ? Dskip[dd] : 0.f;

  // Per-sequence buffer resources, byte offset = lane part + step * pitch.  Steps at or past T read 0
  // (so a chunk's missing steps have dt = x = gy = 0 and B = C = 0: the state passes through unchanged)
  // and stores there are dropped; lanes without a channel store past the slab.
  const size_t row0 = (size_t)n * T;
  const unsigned pitch = (unsigned)Dn * ES;
  const int slab = (int)(T * pitch);               // < 2^31: checked by the entry point
  const auto rx = __builtin_amdgcn_make_buffer_rsrc((void*)(x + row0 * Dn), 0, slab, kRawBufferWord3);
  const auto rdt = __builtin_amdgcn_make_buffer_rsrc((void*)(dt + row0 * Dn), 0, slab, kRawBufferWord3);
  const auto rgy = __builtin_amdgcn_make_buffer_rsrc((void*)(gy + row0 * Dn), 0, slab, kRawBufferWord3);
  const auto rgx = __builtin_amdgcn_make_buffer_rsrc((void*)(gx + row0 * Dn), 0, slab, kRawBufferWord3);
  const auto rgdt = __builtin_amdgcn_make_buffer_rsrc((void*)(gdt + row0 * Dn), 0, slab, kRawBufferWord3);
  const auto rb = __builtin_amdgcn_make_buffer_rsrc((void*)(Bm + row0 * S), 0, T * S * ES, kRawBufferWord3);
  const auto rc = __builtin_amdgcn_make_buffer_rsrc((void*)(Cm + row0 * S), 0, T * S * ES, kRawBufferWord3);
  const int vo = dd * ES;
  const int vo_st = (act && gi == 0) ? d * ES : 0x7ffffff0;

  if (S < SP)
    for (int e = tid; e < BWD_WT * SP; e += blockDim.x)
      if (e % SP >= S) { (&sB[0][0])[e] = 0.f; (&sC[0][0])[e] = 0.f; }
  // rows [w0, w0 + BWD_WT) of B (and C) as fp32; rows past T read as zero
  auto stage = [&](int w0, bool with_c) {
    for (int e = tid; e < BWD_WT * S; e += blockDim.x) {
      const int r = e / S, s = e - r * S;
      const int off = (w0 * S + e) * ES;
      sB[r][s] = buf_ld<DT>(rb, off, 0);
      if (with_c) sC[r][s] = buf_ld<DT>(rc, off, 0);
    }
  };
  auto row = [&](const float (*src)[SP], int r, float* o) {
#pragma unroll
    for (int j = 0; j < SG; ++j) o[j] = src[r][s0 + j];
  };
  // dt as the recurrence uses it; 0 for a missing step (its raw dt reads 0, which the model clamp
  // would lift to 1e-3).  BLOCK mode: dt = clamp(softplus(input)) in fp32, as the block forward.
  auto dt_of = [&](float v, bool live) {
    if constexpr (MODE == HCLSM_SCAN_MODEL) return live ? fminf(fmaxf(v, 1e-3f), 1.0f) : 0.f;
    else if constexpr (MODE == HCLSM_SCAN_BLOCK) return live ? fminf(fmaxf(softplus_f(v), 1e-3f), 1.0f) : 0.f;
    else return v;
  };
  auto ld_chunk = [&](int c, float* xo, float* dto) {
#pragma unroll
    for (int i = 0; i < K; ++i) {
      const int so = (int)((unsigned)(c * K + i) * pitch);   // past the slab for steps >= T: reads 0
      xo[i] = buf_ld<DT>(rx, vo, so);
      dto[i] = buf_ld<DT>(rdt, vo, so);
    }
  };
  // this lane's states in the checkpoint slabs: state s0 + j of channel dd at (s0 + j) * Dn + dd, so that a wave's
  // channels read and write whole lines
  float* ck = ckpt + (size_t)n * a.nck * a.ld_ck + (size_t)s0 * Dn + dd;

  // ---- pass 1: forward recompute, checkpoint at every chunk start; the next chunk's x / dt are in
  // flight while a chunk is stepped (skipped when the forward wrote the checkpoints)
  if (!a.have_ck) {
    float h[SG];
#pragma unroll
    for (int j = 0; j < SG; ++j) h[j] = 0.f;
    float xc[K], dc[K];
    ld_chunk(0, xc, dc);
    int wcur = -1;
    for (int c = 0; c < a.nchunk; ++c) {
      const int t0 = c * K, len = (t0 + K < T ? t0 + K : T) - t0;
      const int w0 = t0 / BWD_WT * BWD_WT;
      if (w0 != wcur) {
        __syncthreads();
        stage(w0, false);
        __syncthreads();
        wcur = w0;
      }
      float xn[K], dn[K];
      ld_chunk(c + 1, xn, dn);
      if (act && c % BWD_CKR == 0 && c > 0)   // (checkpoint 0 is the zero initial state: never stored)
#pragma unroll
        for (int j = 0; j < SG; ++j) ck[(size_t)(c / BWD_CKR) * a.ld_ck + (size_t)j * Dn] = h[j];
#pragma unroll
      for (int i = 0; i < K; ++i) {
        const float dtv = dt_of(dc[i], i < len);
        const float u = dtv * xc[i];
        float bv[SG];
        row(sB, t0 + i - w0, bv);
#pragma unroll
        for (int j = 0; j < SG; ++j) h[j] = fmaf(fast_exp2(dtv * a2[j]), h[j], u * bv[j]);
      }
#pragma unroll
      for (int i = 0; i < K; ++i) { xc[i] = xn[i]; dc[i] = dn[i]; }
    }
  }
  __syncthreads();   // pass 1's reads of the window are done before pass 2 restages it

  // ---- pass 2: reverse, one chunk at a time
  float gh[SG], gA[SG];
#pragma unroll
  for (int j = 0; j < SG; ++j) { gh[j] = 0.f; gA[j] = 0.f; }
  float gD = 0.f;
  int wcur = -1;
  for (int c = a.nchunk - 1; c >= 0; --c) {
    const int t0 = c * K, len = (t0 + K < T ? t0 + K : T) - t0;
    const int w0 = t0 / BWD_WT * BWD_WT;
    float hc[SG], xs[K], ds[K], gs[K];
#pragma unroll
    for (int j = 0; j < SG; ++j) hc[j] = (act && c >= BWD_CKR) ? ck[(size_t)(c / BWD_CKR) * a.ld_ck + (size_t)j * Dn] : 0.f;
    ld_chunk(c, xs, ds);
#pragma unroll
    for (int i = 0; i < K; ++i) {
      const float v = buf_ld<DT>(rgy, vo, (int)((unsigned)(t0 + i) * pitch));
      gs[i] = act ? v : 0.f;
    }
    if (w0 != wcur) {   // the previous chunk ended on a barrier: no lane still reads the old window
      stage(w0, true);
      __syncthreads();
      wcur = w0;
    }
    // from the checkpoint to this chunk's start: the chunks in between, forward (full chunks, same window)
    for (int cc = c - c % BWD_CKR; cc < c; ++cc) {
      float xr[K], dr[K];
      ld_chunk(cc, xr, dr);
#pragma unroll
      for (int i = 0; i < K; ++i) {
        const float dtv = dt_of(dr[i], true);
        const float u = dtv * xr[i];
        float bv[SG];
        row(sB, cc * K + i - w0, bv);
#pragma unroll
        for (int j = 0; j < SG; ++j) hc[j] = fmaf(fast_exp2(dtv * a2[j]), hc[j], u * bv[j]);
      }
    }
    // recompute the chunk's states h_{t0+i} into hk (registers; the starting state goes to LDS) and
    // reduce gC_t = sum_d gy_t h_t over the wave's channels on the way (gy = 0 on inactive lanes and
    // missing steps); lanes that differ only in bits below the last halving hold identical copies
#pragma unroll
    for (int j = 0; j < SG; ++j) sH0[j][tid] = hc[j];
    float hk[K - 1][SG];
#pragma unroll
    for (int i = 0; i < K; ++i) {
      const float dtv = dt_of(ds[i], i < len);
      const float u = dtv * xs[i];
      float bv[SG], w[SG];
      row(sB, t0 + i - w0, bv);
#pragma unroll
      for (int j = 0; j < SG; ++j) {
        hc[j] = fmaf(fast_exp2(dtv * a2[j]), hc[j], u * bv[j]);
        if (i < K - 1) hk[i < K - 1 ? i : 0][j] = hc[j];
        w[j] = gs[i] * hc[j];
      }
      const int off = RS<SG, G>::run(w, lane);
#pragma unroll
      for (int e = 0; e < VL; ++e) red[i][wid][SP + s0 + off + e] = w[e];
    }
    // the reverse steps recompute the gates and reread the rows instead of keeping the recompute's
    // K * SG values live (registers are the occupancy limit): hide both from CSE
    asm volatile("" ::: "memory");
#pragma unroll
    for (int i = K - 1; i >= 0; --i) {
      const int t = t0 + i;
      const float draw = ds[i];
      float dtv = dt_of(draw, i < len);
      asm volatile("" : "+v"(dtv));
      const float xv = xs[i];
      const float gyv = gs[i];
      const float um = act ? dtv * xv : 0.f;   // gy is zero on inactive lanes, so gh is too; um zeroes their gB terms
      float bv[SG], cv[SG], hp[SG];
      row(sB, t - w0, bv);
      row(sC, t - w0, cv);
#pragma unroll
      for (int j = 0; j < SG; ++j) hp[j] = (i > 0) ? hk[i > 0 ? i - 1 : 0][j] : sH0[j][tid];   // h_{t-1}
      float w[SG];
      float q = 0.f, gda2 = 0.f;   // gda2 = sum garg * A * log2(e); times ln 2 below
#pragma unroll
      for (int j = 0; j < SG; ++j) {
        gh[j] = fmaf(gyv, cv[j], gh[j]);
        q = fmaf(gh[j], bv[j], q);
        w[j] = gh[j] * um;                           // -> gB
        gh[j] *= fast_exp2(dtv * a2[j]);             // carried to step t-1
        const float garg = gh[j] * hp[j];            // gh_t h_{t-1} exp(dt A)
        gda2 = fmaf(garg, a2[j], gda2);
        gA[j] = fmaf(garg, dtv, gA[j]);
      }
      q = group_sum<G>(q);
      gda2 = group_sum<G>(gda2);
      float gdv = fmaf(gda2, HCLSM_LN2, q * xv);
      if (MODE == HCLSM_SCAN_MODEL && !(draw >= 1e-3f && draw <= 1.0f)) gdv = 0.f;
      if constexpr (MODE == HCLSM_SCAN_BLOCK) {   // through the clamp (closed interval) and softplus
        const float sp = softplus_f(draw);
        gdv = (sp >= 1e-3f && sp <= 1.0f) ? gdv * __builtin_amdgcn_rcpf(1.f + __expf(-draw)) : 0.f;
      }
      const int so = (i < len) ? (int)((unsigned)t * pitch) : slab;   // a missing step stores nothing
      buf_st<DT>(fmaf(q, dtv, dsk * gyv), rgx, vo_st, so);
      buf_st<DT>(gdv, rgdt, vo_st, so);
      gD = fmaf(gyv, xv, gD);
      // gB_t = sum over the wave's channels (as for gC above)
      const int off = RS<SG, G>::run(w, lane);
#pragma unroll
      for (int e = 0; e < VL; ++e) red[i][wid][s0 + off + e] = w[e];
    }
    __syncthreads();
    // sum the chunk's wave partials: K steps x 2*SP values
    for (int e = tid; e < K * 2 * SP; e += blockDim.x) {
      const int i = e / (2 * SP), v = e - i * 2 * SP;
      if (i < len) {
        float sacc = 0.f;
        for (int w = 0; w < nw; ++w) sacc += red[i][w][v];
        gbc[(((size_t)blockIdx.y * gridDim.x + n) * T + t0 + i) * 2 * SP + v] = sacc;   // this block's part
      }
    }
    __syncthreads();
  }
  if (act) {
#pragma unroll
    for (int j = 0; j < SG; ++j) gA_part[((size_t)n * SP + s0 + j) * Dn + d] = gA[j];   // state-major: whole lines
    if (gi == 0) gD_part[(size_t)n * Dn + d] = gD;
  }
}

// The backward's tail in one launch: blocks [0, nga) reduce the per-sequence gA partials over the sequences and
// write gA_log[d, s] = sum * dA/dA_log; blocks [nga, nga + ngd) reduce the gD partials; the remaining blocks add
// the channel blocks' gB / gC parts in block order and cast.  The three parts are independent.  Each reducing
// block sums 64 columns in 16 row groups (fixed order: deterministic).
template <int DT, int SP, int MODE>
__global__ void __launch_bounds__(1024)
ssm_scan_bwd_tail(const float* __restrict__ ga_part, const float* __restrict__ gd_part, const float* __restrict__ gbc,
                  const float* __restrict__ A_log, typename Elem<DT>::T* __restrict__ gB,
                  typename Elem<DT>::T* __restrict__ gC, float* __restrict__ gA_log, float* __restrict__ gD,
                  int64_t N, int T, int Dn, int S, int nblk, int nga, int ngd) {
  using E = Elem<DT>;
  __shared__ float red[16][64];
  const int bx = blockIdx.x;
  if (bx < nga + ngd) {
    const bool is_a = bx < nga;
    const int64_t ncols = is_a ? (int64_t)Dn * SP : Dn;
    const float* part = is_a ? ga_part : gd_part;
    const int c = threadIdx.x & 63, rg = threadIdx.x >> 6;
    const int64_t col = (int64_t)(is_a ? bx : bx - nga) * 64 + c;
    float acc = 0.f;
    if (col < ncols) {
#pragma unroll 8
      for (int64_t n = rg; n < N; n += 16) acc += part[n * ncols + col];
    }
    red[rg][c] = acc;
    __syncthreads();
    if (rg == 0 && col < ncols) {
      float t = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) t += red[r][c];
      if (is_a) {   // the gA partials are state-major: column s * Dn + d
        const int64_t s = col / Dn, dd = col - s * Dn;
        if (s < S) {   // (padded states carry no gradient)
          const int64_t i = dd * S + s;
          const float e = expf(A_log[i]);
          float dadl = -e;                          // d(-exp(A_log))/dA_log
          if (MODE != HCLSM_SCAN_RAW && !(e >= 1e-6f && e <= 1.0f)) dadl = 0.f;
          gA_log[i] = t * dadl;
        }
      } else {
        gD[col] = t;
      }
    }
    return;
  }
  const int64_t stride = (int64_t)(gridDim.x - nga - ngd) * blockDim.x;
  const int64_t nbc = N * T * S;
  const int64_t part = N * T * 2 * SP;   // floats per channel block's partial
  for (int64_t i = (int64_t)(bx - nga - ngd) * blockDim.x + threadIdx.x; i < nbc; i += stride) {
    const int64_t r = i / S, s = i - r * S;
    float b = 0.f, c = 0.f;
    for (int k = 0; k < nblk; ++k) {   // fixed order: deterministic
      b += gbc[k * part + r * 2 * SP + s];
      c += gbc[k * part + r * 2 * SP + SP + s];
    }
    E::st(gB + i, b);
    E::st(gC + i, c);
  }
}

static int64_t sp_of(int64_t S) {
  return S <= 4 ? 4 : S <= 8 ? 8 : S <= 16 ? 16 : S <= 32 ? 32 : S <= 64 ? 64 : 128;
}

struct BwdWs {
  size_t ck, gbc, ga, gd, total;
  int nchunk, nck;
  BwdGrid grid;
};

static BwdWs bwd_ws(int64_t N, int64_t T, int64_t Dn, int64_t S) {
  const int64_t SP = sp_of(S);
  const int64_t SG = bwd_sg((int)SP);
  const int64_t K = bwd_k((int)SP);
  BwdWs w;
  w.nchunk = (int)((T + K - 1) / K);
  w.grid = bwd_grid(Dn, (int)(SP / SG));
  auto al = [](size_t v) { return (v + 255) / 256 * 256; };
  size_t o = 0;
  w.nck = (w.nchunk + BWD_CKR - 1) / BWD_CKR;
  w.ck = o; o += al((size_t)N * w.nck * Dn * SP * 4);
  w.gbc = o; o += al((size_t)w.grid.nblk * N * T * 2 * SP * 4);
  w.ga = o; o += al((size_t)N * Dn * SP * 4);
  w.gd = o; o += al((size_t)N * Dn * 4);
  w.total = o;
  return w;
}

template <int DT, int SP, int MODE>
static int launch_bwd(const void* x, const void* dt, const float* A_log, const void* B, const void* C,
                      const float* Dskip, const void* gy, void* gx, void* gdt, float* gA_log, void* gB, void* gC,
                      float* gD, char* ws, const BwdWs& L, int64_t N, int64_t T, int64_t Dn, int64_t S,
                      bool have_ck, hipStream_t st) {
  using TT = typename Elem<DT>::T;
  constexpr int SG = bwd_sg(SP);
  constexpr int G = SP / SG;
  const int DW = L.grid.DW, nblk_d = L.grid.nblk;
  int threads = DW * G;
  threads = (threads + 63) / 64 * 64;
  BwdArgs a;
  a.T = (int)T; a.Dn = (int)Dn; a.S = (int)S; a.nchunk = L.nchunk; a.nck = L.nck; a.DW = DW;
  a.ld_ck = Dn * SP;
  a.have_ck = have_ck ? 1 : 0;
  float* gbc = reinterpret_cast<float*>(ws + L.gbc);
  hipLaunchKernelGGL((ssm_scan_bwd_kernel<DT, SP, MODE>), dim3((unsigned)N, (unsigned)nblk_d), dim3(threads), 0, st,
                     (const TT*)x, (const TT*)dt, A_log, (const TT*)B, (const TT*)C, Dskip, (const TT*)gy, (TT*)gx,
                     (TT*)gdt, reinterpret_cast<float*>(ws + L.ck), gbc, reinterpret_cast<float*>(ws + L.ga),
                     reinterpret_cast<float*>(ws + L.gd), a);
  HCLSM_LAUNCH_CHECK();
  // the tail: gA_log and gD reductions and the gB / gC block sums, one launch
  const int nga = (int)((Dn * SP + 63) / 64), ngd = gD ? (int)((Dn + 63) / 64) : 0;
  int64_t g = (N * T * S + 1023) / 1024;
  g = g < 1 ? 1 : (g > 1024 ? 1024 : g);
  hipLaunchKernelGGL((ssm_scan_bwd_tail<DT, SP, MODE>), dim3((unsigned)(nga + ngd + g)), dim3(1024), 0, st,
                     reinterpret_cast<const float*>(ws + L.ga), reinterpret_cast<const float*>(ws + L.gd), gbc, A_log,
                     (TT*)gB, (TT*)gC, gA_log, gD, N, (int)T, (int)Dn, (int)S, nblk_d, nga, ngd);
  HCLSM_LAUNCH_CHECK();
  return 0;
}

}  // namespace hclsm

using namespace hclsm;

extern "C" int64_t hclsm_ssm_scan_bwd_workspace(int64_t batch, int64_t T, int64_t d_inner, int64_t d_state) {
  if (batch < 0 || T < 0 || d_inner < 0 || d_state < 1 || d_state > 128) return HCLSM_ERR_SHAPE;
  return (int64_t)bwd_ws(batch, T, d_inner, d_state).total;
}

static int scan_bwd_entry(const void* x, const void* dt, const float* A_log, const void* B, const void* C,
                          const float* Dskip, const void* gy, void* gx, void* gdt, float* gA_log, void* gB, void* gC,
                          float* gD, int64_t batch, int64_t T, int64_t d_inner, int64_t d_state, int dtype, int mode,
                          void* workspace, int64_t workspace_bytes, bool have_ck, void* stream) {
  if (batch < 0 || T < 0 || d_inner < 0 || d_state < 1) return HCLSM_ERR_SHAPE;
  if (batch > 0x7fffffffLL || T > 0x7fffffffLL || d_inner > 0x7fffffffLL) return HCLSM_ERR_SHAPE;
  if (d_state > 128) return HCLSM_ERR_UNSUPPORTED;
  // per-sequence slabs are addressed through 32-bit buffer offsets
  if (T * d_inner * (dtype == HCLSM_F32 ? 4 : 2) >= (1LL << 31)) return HCLSM_ERR_UNSUPPORTED;
  if (mode != HCLSM_SCAN_RAW && mode != HCLSM_SCAN_MODEL && mode != HCLSM_SCAN_BLOCK) return HCLSM_ERR_MODE;
  if (dtype != HCLSM_F32 && dtype != HCLSM_BF16 && dtype != HCLSM_F16) return HCLSM_ERR_DTYPE;
  hipStream_t st = (hipStream_t)stream;
  if (batch == 0 || T == 0 || d_inner == 0) {
    // no products: every gradient is zero
    if (gA_log && d_inner > 0) { int rc = zero_fill_f32(gA_log, d_inner * d_state, st); if (rc) return rc; }
    if (gD && d_inner > 0) { int rc = zero_fill_f32(gD, d_inner, st); if (rc) return rc; }
    const int64_t es = dtype == HCLSM_F32 ? 4 : 2;
    if (gB && batch * T > 0) { int rc = zero_fill_bytes(gB, batch * T * d_state * es, st); if (rc) return rc; }
    if (gC && batch * T > 0) { int rc = zero_fill_bytes(gC, batch * T * d_state * es, st); if (rc) return rc; }
    return 0;
  }
  if (!x || !dt || !A_log || !B || !C || !gy || !gx || !gdt || !gA_log || !gB || !gC || !workspace)
    return HCLSM_ERR_NULL;
  const BwdWs L = bwd_ws(batch, T, d_inner, d_state);
  if (workspace_bytes < (int64_t)L.total) return HCLSM_ERR_SHAPE;
  char* ws = reinterpret_cast<char*>(workspace);
#define HCLSM_BWD(DT_, SP_)                                                                                  \
  if (sp_of(d_state) == SP_) {                                                                               \
    if (mode == HCLSM_SCAN_RAW)                                                                              \
      return launch_bwd<DT_, SP_, HCLSM_SCAN_RAW>(x, dt, A_log, B, C, Dskip, gy, gx, gdt, gA_log, gB, gC, gD, ws, L, \
                                                  batch, T, d_inner, d_state, have_ck, st);                  \
    if (mode == HCLSM_SCAN_BLOCK)                                                                            \
      return launch_bwd<DT_, SP_, HCLSM_SCAN_BLOCK>(x, dt, A_log, B, C, Dskip, gy, gx, gdt, gA_log, gB, gC, gD, ws, \
                                                    L, batch, T, d_inner, d_state, have_ck, st);             \
    return launch_bwd<DT_, SP_, HCLSM_SCAN_MODEL>(x, dt, A_log, B, C, Dskip, gy, gx, gdt, gA_log, gB, gC, gD, ws, L, \
                                                  batch, T, d_inner, d_state, have_ck, st);                  \
  }
#define HCLSM_BWD_DT(DT_) \
  HCLSM_BWD(DT_, 4) HCLSM_BWD(DT_, 8) HCLSM_BWD(DT_, 16) HCLSM_BWD(DT_, 32) HCLSM_BWD(DT_, 64) HCLSM_BWD(DT_, 128)
  if (dtype == HCLSM_F32) { HCLSM_BWD_DT(HCLSM_F32) }
  if (dtype == HCLSM_BF16) { HCLSM_BWD_DT(HCLSM_BF16) }
  if (dtype == HCLSM_F16) { HCLSM_BWD_DT(HCLSM_F16) }
#undef HCLSM_BWD_DT
#undef HCLSM_BWD
  return HCLSM_ERR_UNSUPPORTED;
}

extern "C" int hclsm_ssm_scan_bwd(const void* x, const void* dt, const float* A_log, const void* B, const void* C,
                                  const float* Dskip, const void* gy, void* gx, void* gdt, float* gA_log, void* gB,
                                  void* gC, float* gD, int64_t batch, int64_t T, int64_t d_inner, int64_t d_state,
                                  int dtype, int mode, void* workspace, int64_t workspace_bytes, void* stream) {
  return scan_bwd_entry(x, dt, A_log, B, C, Dskip, gy, gx, gdt, gA_log, gB, gC, gD, batch, T, d_inner, d_state, dtype,
                        mode, workspace, workspace_bytes, false, stream);
}

// The checkpointing forward writes the state before steps 8, 16, ... into the backward workspace's checkpoint
// slab (offset 0): exactly what pass 1 of the backward would write for d_state 16 (4-step chunks, a checkpoint
// every second chunk).
static_assert(bwd_k(16) * BWD_CKR == 8, "the checkpointing forward stores the state before every 8th step");
static bool ckpt_shape_ok(int64_t d_state, int dtype) { return dtype == HCLSM_BF16 && d_state == 16; }

extern "C" int hclsm_ssm_scan_fwd_ckpt(const void* x, const void* dt, const float* A_log, const void* B,
                                       const void* C, const float* Dskip, void* y, float* h_final, int64_t batch,
                                       int64_t T, int64_t d_inner, int64_t d_state, int dtype, int mode,
                                       void* workspace, int64_t workspace_bytes, void* stream) {
  if (mode != HCLSM_SCAN_RAW && mode != HCLSM_SCAN_MODEL) return HCLSM_ERR_MODE;
  if (batch < 0 || T < 0 || d_inner < 0 || d_state < 1) return HCLSM_ERR_SHAPE;
  if (!ckpt_shape_ok(d_state, dtype)) return HCLSM_ERR_UNSUPPORTED;
  if (batch == 0 || T == 0 || d_inner == 0)   // no steps, no checkpoints: the plain forward's empty case
    return hclsm_ssm_scan_fwd(x, dt, A_log, B, C, Dskip, y, h_final, batch, T, d_inner, d_state, dtype, mode, stream);
  if (!workspace) return HCLSM_ERR_NULL;
  const BwdWs L = bwd_ws(batch, T, d_inner, d_state);
  if (workspace_bytes < (int64_t)L.total) return HCLSM_ERR_SHAPE;
  return scan_fwd_ckpt(mode, x, dt, A_log, B, C, Dskip, y, h_final, batch, T, d_inner, d_state, dtype, nullptr,
                       nullptr, reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + L.ck),
                       (hipStream_t)stream);
}

extern "C" int hclsm_ssm_block_scan_fwd_ckpt(const void* z, const void* dt_in, const float* A_log, const void* B,
                                             const void* C, const void* gate, void* y, void* y_pre, float* h_final,
                                             int64_t batch, int64_t T, int64_t d_inner, int64_t d_state, int dtype,
                                             void* workspace, int64_t workspace_bytes, void* stream) {
  if (batch < 0 || T < 0 || d_inner < 0 || d_state < 1) return HCLSM_ERR_SHAPE;
  if (!ckpt_shape_ok(d_state, dtype)) return HCLSM_ERR_UNSUPPORTED;
  if (batch == 0 || T == 0 || d_inner == 0)
    return hclsm_ssm_block_scan_fwd(z, dt_in, A_log, B, C, gate, y, y_pre, h_final, batch, T, d_inner, d_state, dtype,
                                    stream);
  if (!workspace || !gate) return HCLSM_ERR_NULL;
  const BwdWs L = bwd_ws(batch, T, d_inner, d_state);
  if (workspace_bytes < (int64_t)L.total) return HCLSM_ERR_SHAPE;
  return scan_fwd_ckpt(HCLSM_SCAN_BLOCK, z, dt_in, A_log, B, C, nullptr, y, h_final, batch, T, d_inner, d_state,
                       dtype, gate, y_pre, reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + L.ck),
                       (hipStream_t)stream);
}

extern "C" int hclsm_ssm_scan_bwd_ckpt(const void* x, const void* dt, const float* A_log, const void* B,
                                       const void* C, const float* Dskip, const void* gy, void* gx, void* gdt,
                                       float* gA_log, void* gB, void* gC, float* gD, int64_t batch, int64_t T,
                                       int64_t d_inner, int64_t d_state, int dtype, int mode, void* workspace,
                                       int64_t workspace_bytes, void* stream) {
  if (batch < 0 || T < 0 || d_inner < 0 || d_state < 1) return HCLSM_ERR_SHAPE;
  if (!ckpt_shape_ok(d_state, dtype)) return HCLSM_ERR_UNSUPPORTED;
  // (an empty problem has no checkpoints: the plain backward's zero gradients)
  const bool empty = batch == 0 || T == 0 || d_inner == 0;
  return scan_bwd_entry(x, dt, A_log, B, C, Dskip, gy, gx, gdt, gA_log, gB, gC, gD, batch, T, d_inner, d_state, dtype,
                        mode, workspace, workspace_bytes, !empty, stream);
}
