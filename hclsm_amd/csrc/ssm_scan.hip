// Selective SSM scan forward for gfx950.
//
// Mapping: one lane owns one (sequence n, channel d) pair and keeps its d_state
// recurrent states in fp32 registers for the whole sequence; the time loop is
// serial inside the lane.  A workgroup covers a contiguous block of channels of
// one sequence, so every lane of the group reads the same B_t / C_t row, which the
// compiler turns into scalar (SGPR) loads; x/dt/y rows are read and written as
// contiguous 128 B (bf16) or 256 B (fp32) wave-wide segments.  Time steps are
// processed in chunks of TCHUNK with the next chunk's x/dt loads issued before the
// current chunk's arithmetic, which keeps HBM requests in flight while the VALU
// works.
//
// Per state update the lane does: mul (dt*A*log2e), v_exp_f32, mul (dt*x*B),
// fma (gate*h + ...), fma (y += h*C).  The loop is bound by VALU issue, not HBM.
// For bf16 I/O with d_state 16 the rank-1 input term dt*x*B and its add into h
// run on the matrix core instead (ssm_scan_fwd_mfma_kernel below), which leaves
// mul, exp, mul, fma per state update on the VALU.
#include "internal.h"

namespace hclsm {

// Internal mode of hclsm_ssm_block_scan_fwd: the MODEL clamps, dt = softplus(dt input) before
// its clamp, and the output multiplied by silu(gate) -- the SimplifiedSSMBlock epilogues
// (level0_ssm.py:73, :76, :103) fused into the scan.
constexpr int SCAN_BLOCK = HCLSM_SCAN_BLOCK;
struct ScanEpi {
  const void* gate;   // [batch][T][d_inner], I/O type; required in SCAN_BLOCK
  void* y_pre;        // optional: the scan output before gating (kept for the backward)
  float* ck;          // checkpointing launches only: [batch][ceil(T / 8)][16][d_inner] fp32, the state
                      // before steps 8, 16, ... (the backward's checkpoint slab; entry 0, the zero initial
                      // state, is not stored)
};


template <int MODE>
__device__ __forceinline__ float scan_dt(float v) {
  if constexpr (MODE == SCAN_BLOCK) v = softplus_f(v);
  if constexpr (MODE != HCLSM_SCAN_RAW) v = fminf(fmaxf(v, 1e-3f), 1.0f);
  return v;
}


constexpr int SCAN_TCHUNK = 8;
constexpr int SCAN_MAX_BLOCK = 256;
// Generic kernel: one lane per channel holds up to 32 states; larger d_state splits a channel's
// states over 2 or 4 adjacent lanes (64 / 128 padded states), whose output partials are summed by
// lane exchange, so no lane keeps more than 32 states and 32 gate exponents in registers.
constexpr int scan_lanes_per_channel(int SP) { return SP > 32 ? SP / 32 : 1; }

template <int DT, int SP, int MODE>
__global__ void __launch_bounds__(SCAN_MAX_BLOCK)
ssm_scan_fwd_kernel(const typename Elem<DT>::T* __restrict__ x,
                    const typename Elem<DT>::T* __restrict__ dt,
                    const float* __restrict__ A_log,
                    const typename Elem<DT>::T* __restrict__ Bm,
                    const typename Elem<DT>::T* __restrict__ Cm,
                    const float* __restrict__ Dskip,
                    typename Elem<DT>::T* __restrict__ y,
                    float* __restrict__ h_final,
                    int T, int Dn, int S, ScanEpi epi) {
  using E = Elem<DT>;
  using TT = typename E::T;
  constexpr int TC = SCAN_TCHUNK;
  constexpr int LPC = scan_lanes_per_channel(SP);   // adjacent lanes sharing one channel
  constexpr int SPL = SP / LPC;                      // states per lane
  // B_t / C_t rows of the current and the next chunk, fp32, zero-padded to SP.
  __shared__ float4 sB[2][TC][SP / 4];
  __shared__ float4 sC[2][TC][SP / 4];

  const int n = blockIdx.x;
  const int lt = blockIdx.y * blockDim.x + threadIdx.x;
  const int d = lt / LPC;
  const int sbase = (lt % LPC) * SPL;   // this lane's first state
  const bool act = d < Dn;
  const bool writer = act && sbase == 0;   // one lane per channel stores y
  const int dd = act ? d : 0;  // inactive lanes read a valid address and store nothing

  // gate exponent per state in log2 units: A[d,s] * log2(e); padded states get 0
  float a2[SPL];
#pragma unroll
  for (int i = 0; i < SPL; ++i) {
    const int s = sbase + i;
    float a = 0.f;
    {
      // unconditional load of a valid element, then select: no divergent branch
      float e = expf(A_log[(size_t)dd * S + (s < S ? s : S - 1)]);
      if (MODE != HCLSM_SCAN_RAW) e = fminf(fmaxf(e, 1e-6f), 1.0f);
      a = (s < S) ? -e * HCLSM_LOG2E : 0.f;
    }
    a2[i] = a;
  }
  const bool has_d = Dskip != nullptr;
  const float dsk = has_d ? Dskip[dd] : 0.f;

  float h[SPL];
#pragma unroll
  for (int i = 0; i < SPL; ++i) h[i] = 0.f;

  const size_t row0 = (size_t)n * T;
  const TT* xp = x + row0 * Dn + dd;
  const TT* dp = dt + row0 * Dn + dd;
  TT* yp = y + row0 * Dn + dd;
  const TT* bp = Bm + row0 * S;
  const TT* cp = Cm + row0 * S;

  // Cooperative staging of B/C for chunk starting at t0: element i of the
  // [TC][SP] tile is (tt = i / SP, s = i % SP).  Each lane handles at most
  // ceil(TC*SP / blockDim) elements; values are held in registers across the
  // arithmetic of the current chunk and written to LDS afterwards.
  constexpr int STAGE_MAX = (TC * SP + 63) / 64;  // blockDim >= 64
  float stB[STAGE_MAX], stC[STAGE_MAX];
  auto stage_load = [&](int t0) {
#pragma unroll
    for (int k = 0; k < STAGE_MAX; ++k) {
      const int i = threadIdx.x + k * blockDim.x;
      const int ii = i < TC * SP ? i : 0;
      const int tt = ii / SP, s = ii % SP, t = t0 + tt;
      const bool ok = (i < TC * SP) && (t < T) && (s < S);
      const int tc = t < T ? t : T - 1, sc = s < S ? s : S - 1;
      const float bv = E::ld(bp + (size_t)tc * S + sc);
      const float cv = E::ld(cp + (size_t)tc * S + sc);
      stB[k] = ok ? bv : 0.f;
      stC[k] = ok ? cv : 0.f;
    }
  };
  auto stage_store = [&](int buf) {
    float* fb = reinterpret_cast<float*>(&sB[buf][0][0]);
    float* fc = reinterpret_cast<float*>(&sC[buf][0][0]);
#pragma unroll
    for (int k = 0; k < STAGE_MAX; ++k) {
      const int i = threadIdx.x + k * blockDim.x;
      if (i < TC * SP) { fb[i] = stB[k]; fc[i] = stC[k]; }
    }
  };

  float xv[TC], dv[TC];
  auto xd_load = [&](int t0, float* xo, float* dO) {
#pragma unroll
    for (int j = 0; j < TC; ++j) {
      const int t = t0 + j < T ? t0 + j : T - 1;  // clamped: always a valid address
      xo[j] = E::ld(xp + (size_t)t * Dn);
      dO[j] = E::ld(dp + (size_t)t * Dn);
    }
  };

  auto store_y = [&](int t, float yv) {
    if constexpr (MODE == SCAN_BLOCK) {
      const size_t o = row0 * Dn + dd + (size_t)t * Dn;
      if (epi.y_pre) E::st(reinterpret_cast<TT*>(epi.y_pre) + o, yv);
      yv *= silu_f(E::ld(reinterpret_cast<const TT*>(epi.gate) + o));
    }
    E::st(yp + (size_t)t * Dn, yv);
  };

  auto step = [&](int buf, int j, float xval, float dval) -> float {
    float dtv = dval;
    dtv = scan_dt<MODE>(dtv);
    // In MODEL mode |dt*A| <= 1*1 < 20, so the clamp of dt*A to [-20, 0]
    // (ssm_scan_kernel.py:77) can never bind and is not applied.
    const float u = dtv * xval;
    float y0 = 0.f, y1 = 0.f;
#pragma unroll
    for (int q = 0; q < SPL / 4; ++q) {
      const float4 b4 = sB[buf][j][sbase / 4 + q];
      const float4 c4 = sC[buf][j][sbase / 4 + q];
      const float bb[4] = {b4.x, b4.y, b4.z, b4.w};
      const float cc[4] = {c4.x, c4.y, c4.z, c4.w};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 4 * q + r;
        const float g = fast_exp2(dtv * a2[i]);
        h[i] = fmaf(g, h[i], u * bb[r]);
        if (r & 1) y1 = fmaf(h[i], cc[r], y1); else y0 = fmaf(h[i], cc[r], y0);
      }
    }
    float yv = y0 + y1;
    if constexpr (LPC >= 2) yv += __shfl_xor(yv, 1, 64);   // sum over the channel's lanes
    if constexpr (LPC >= 4) yv += __shfl_xor(yv, 2, 64);
    if (has_d) yv = fmaf(dsk, xval, yv);
    return yv;
  };

  xd_load(0, xv, dv);
  stage_load(0);
  stage_store(0);
  __syncthreads();

  const int nchunk = (T + TC - 1) / TC;
  for (int c = 0; c < nchunk; ++c) {
    const int t0 = c * TC;
    const int buf = c & 1;
    float xn[TC], dn[TC];
    const bool more = (c + 1) < nchunk;
    if (more) {
      xd_load(t0 + TC, xn, dn);
      stage_load(t0 + TC);
    }
    if (t0 + TC <= T) {
#pragma unroll
      for (int j = 0; j < TC; ++j) {
        const float yv = step(buf, j, xv[j], dv[j]);
        if (writer) store_y(t0 + j, yv);
      }
    } else {
      for (int j = 0; j < T - t0; ++j) {
        float xj = 0.f, dj = 0.f;
#pragma unroll
        for (int k = 0; k < TC; ++k) if (k == j) { xj = xv[k]; dj = dv[k]; }
        const float yv = step(buf, j, xj, dj);
        if (writer) store_y(t0 + j, yv);
      }
    }
    if (more) {
      stage_store(buf ^ 1);
#pragma unroll
      for (int j = 0; j < TC; ++j) { xv[j] = xn[j]; dv[j] = dn[j]; }
    }
    __syncthreads();
  }

  if (h_final != nullptr && act) {
    float* hp = h_final + ((size_t)n * Dn + d) * S;
#pragma unroll
    for (int i = 0; i < SPL; ++i)
      if (sbase + i < S) hp[sbase + i] = h[i];
  }
}

// ---------------------------------------------------------------------------
// Fast path: d_state == SP, B/C rows small enough to live in SGPRs.
//
// B_t and C_t are the same for every lane of the workgroup, so they are fetched
// with scalar loads (s_load_dwordx*) one step ahead and unpacked by the scalar
// ALU; the VALU then reads them as SGPR operands.  No LDS and no barriers.  Each
// lane owns DPL adjacent channels (DPL=2 gives 32-bit bf16 pair loads/stores and
// shares the scalar unpack between two channels).  x/dt for the next TC steps are
// loaded (clamped addresses, unconditional) before the current TC steps compute.
template <int DT, int SP, int MODE, int DPL, int TC>
__global__ void __launch_bounds__(64)
ssm_scan_fwd_sgpr_kernel(const typename Elem<DT>::T* __restrict__ x,
                         const typename Elem<DT>::T* __restrict__ dt,
                         const float* __restrict__ A_log,
                         const typename Elem<DT>::T* __restrict__ Bm,
                         const typename Elem<DT>::T* __restrict__ Cm,
                         const float* __restrict__ Dskip,
                         typename Elem<DT>::T* __restrict__ y,
                         float* __restrict__ h_final,
                         int T, int Dn, ScanEpi epi) {
  using E = Elem<DT>;
  using TT = typename E::T;
  constexpr int NW = SP * (int)sizeof(TT) / 4;  // 32-bit words per B/C row
  static_assert(NW >= 1, "row must be at least one word");

  const int n = blockIdx.x;
  const int lane_d = (blockIdx.y * 64 + threadIdx.x) * DPL;  // first channel of this lane
  const bool act = lane_d < Dn;
  const int d0 = act ? lane_d : 0;

  float a2[DPL][SP];
#pragma unroll
  for (int k = 0; k < DPL; ++k)
#pragma unroll
    for (int s = 0; s < SP; ++s) {
      float e = expf(A_log[(size_t)(d0 + k) * SP + s]);
      if (MODE != HCLSM_SCAN_RAW) e = fminf(fmaxf(e, 1e-6f), 1.0f);
      a2[k][s] = -e * HCLSM_LOG2E;
    }
  const bool has_d = Dskip != nullptr;
  float dsk[DPL];
#pragma unroll
  for (int k = 0; k < DPL; ++k) dsk[k] = has_d ? Dskip[d0 + k] : 0.f;

  float h[DPL][SP];
#pragma unroll
  for (int k = 0; k < DPL; ++k)
#pragma unroll
    for (int s = 0; s < SP; ++s) h[k][s] = 0.f;

  const size_t row0 = (size_t)n * T;
  const TT* xp = x + row0 * Dn + d0;
  const TT* dp = dt + row0 * Dn + d0;
  TT* yp = y + row0 * Dn + d0;
  const uint32_t* bw0 = reinterpret_cast<const uint32_t*>(Bm + row0 * SP);
  const uint32_t* cw0 = reinterpret_cast<const uint32_t*>(Cm + row0 * SP);

  auto ld_pair = [&](const TT* p, float* o) {
    if constexpr (DPL == 2 && DT == HCLSM_BF16) {
      const uint32_t w = *reinterpret_cast<const uint32_t*>(p);
      o[0] = __uint_as_float(w << 16);
      o[1] = __uint_as_float(w & 0xffff0000u);
    } else if constexpr (DPL == 2 && DT == HCLSM_F32) {
      const float2 v = *reinterpret_cast<const float2*>(p);
      o[0] = v.x;
      o[1] = v.y;
    } else {
#pragma unroll
      for (int k = 0; k < DPL; ++k) o[k] = E::ld(p + k);
    }
  };
  auto st_pair = [&](TT* p, const float* v) {
    if constexpr (DPL == 2 && DT == HCLSM_BF16) {
      const uint32_t w = pack_bf16x2(v[0], v[1]);
      *reinterpret_cast<uint32_t*>(p) = w;
    } else if constexpr (DPL == 2 && DT == HCLSM_F32) {
      *reinterpret_cast<float2*>(p) = make_float2(v[0], v[1]);
    } else {
#pragma unroll
      for (int k = 0; k < DPL; ++k) E::st(p + k, v[k]);
    }
  };
  auto unpack = [&](const uint32_t (&w)[NW], float (&v)[SP]) {
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      if constexpr (DT == HCLSM_BF16) {
        v[2 * i] = __uint_as_float(w[i] << 16);
        v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
      } else {
        v[i] = __uint_as_float(w[i]);
      }
    }
  };

  float xv[TC][DPL], dv[TC][DPL];
  auto xd_load = [&](int t0, float (*xo)[DPL], float (*dO)[DPL]) {
#pragma unroll
    for (int j = 0; j < TC; ++j) {
      const int t = t0 + j < T ? t0 + j : T - 1;  // clamped: always a valid address
      ld_pair(xp + (size_t)t * Dn, xo[j]);
      ld_pair(dp + (size_t)t * Dn, dO[j]);
    }
  };

  uint32_t bw[NW], cw[NW];
#pragma unroll
  for (int i = 0; i < NW; ++i) { bw[i] = bw0[i]; cw[i] = cw0[i]; }

  auto step = [&](int t, const float* xs, const float* ds) {
    // fetch next step's rows first (uniform address -> scalar loads)
    const int tn = t + 1 < T ? t + 1 : T - 1;
    uint32_t bwn[NW], cwn[NW];
#pragma unroll
    for (int i = 0; i < NW; ++i) { bwn[i] = bw0[(size_t)tn * NW + i]; cwn[i] = cw0[(size_t)tn * NW + i]; }
    float bv[SP], cv[SP];
    unpack(bw, bv);
    unpack(cw, cv);
    float yo[DPL];
#pragma unroll
    for (int k = 0; k < DPL; ++k) {
      float dtv = ds[k];
      dtv = scan_dt<MODE>(dtv);
      // MODEL mode: |dt*A| <= 1 < 20, so the [-20, 0] clamp of ssm_scan_kernel.py:77 never binds.
      const float u = dtv * xs[k];
      float y0 = 0.f, y1 = 0.f;
#pragma unroll
      for (int s = 0; s < SP; ++s) {
        const float g = fast_exp2(dtv * a2[k][s]);
        h[k][s] = fmaf(g, h[k][s], u * bv[s]);
        if (s & 1) y1 = fmaf(h[k][s], cv[s], y1); else y0 = fmaf(h[k][s], cv[s], y0);
      }
      float yv = y0 + y1;
      if (has_d) yv = fmaf(dsk[k], xs[k], yv);
      yo[k] = yv;
    }
    if constexpr (MODE == SCAN_BLOCK) {
      const size_t o = row0 * Dn + d0 + (size_t)t * Dn;
      if (epi.y_pre && act) st_pair(reinterpret_cast<TT*>(epi.y_pre) + o, yo);
      float gv[DPL];
      ld_pair(reinterpret_cast<const TT*>(epi.gate) + o, gv);
#pragma unroll
      for (int k = 0; k < DPL; ++k) yo[k] *= silu_f(gv[k]);
    }
    if (act) st_pair(yp + (size_t)t * Dn, yo);
#pragma unroll
    for (int i = 0; i < NW; ++i) { bw[i] = bwn[i]; cw[i] = cwn[i]; }
  };

  xd_load(0, xv, dv);
  const int tfull = T - T % TC;
  for (int t0 = 0; t0 < tfull; t0 += TC) {
    float xn[TC][DPL], dn[TC][DPL];
    xd_load(t0 + TC, xn, dn);
#pragma unroll
    for (int j = 0; j < TC; ++j) step(t0 + j, xv[j], dv[j]);
#pragma unroll
    for (int j = 0; j < TC; ++j)
#pragma unroll
      for (int k = 0; k < DPL; ++k) { xv[j][k] = xn[j][k]; dv[j][k] = dn[j][k]; }
  }
  // tail (T % TC steps): xv/dv already hold them
#pragma unroll
  for (int j = 0; j < TC - 1; ++j)
    if (tfull + j < T) step(tfull + j, xv[j], dv[j]);

  if (h_final != nullptr && act) {
#pragma unroll
    for (int k = 0; k < DPL; ++k) {
      float* hp = h_final + ((size_t)n * Dn + d0 + k) * SP;
#pragma unroll
      for (int s = 0; s < SP; ++s) hp[s] = h[k][s];
    }
  }
}

template <int DT, int SP, int MODE, int DPL, int TC>
static int launch_scan_sgpr(const void* x, const void* dt, const float* A_log, const void* B,
                            const void* C, const float* Dskip, void* y, float* h_final,
                            int64_t batch, int64_t T, int64_t Dn, hipStream_t st, ScanEpi epi) {
  using TT = typename Elem<DT>::T;
  const int64_t lanes = (Dn + DPL - 1) / DPL;
  dim3 grid((unsigned)batch, (unsigned)((lanes + 63) / 64));
  hipLaunchKernelGGL((ssm_scan_fwd_sgpr_kernel<DT, SP, MODE, DPL, TC>), grid, dim3(64), 0, st,
                     (const TT*)x, (const TT*)dt, A_log, (const TT*)B, (const TT*)C, Dskip,
                     (TT*)y, h_final, (int)T, (int)Dn, epi);
  HCLSM_LAUNCH_CHECK();
  return 0;
}

// ---------------------------------------------------------------------------
// bf16 I/O, d_state == 16: the rank-1 input term on the matrix core.
//
// Per step the state update is h[d][s] = g[d][s] * h[d][s] + u[d] * b[s] with
// g = exp2(dt[d] * a2[d][s]) and u = dt * x.  One v_mfma_f32_32x32x8_bf16 per
// wave and step computes D = A * B + C over a 32 x 32 tile whose accumulator
// layout gives lane l the 16 rows i = 8*(r/4) + 4*(l/32) + r%4 (r = 0..15) of
// column j = l%32.  Rows are read as (state s = r, half c = l/32), columns as
// j, so lane l holds exactly the 16 states of channel c*32 + j = l, in register
// order r = s: the y contraction stays an in-lane fp32 FMA chain and the
// per-lane decay g * h is an elementwise VALU product fed as the accumulator C.
// The product u * b enters through the k dimension:
//   B operand (lane l: k = 4*(l/32) .. +3 of column l%32) = (u_hi, u_lo, 0, 0)
//   of the lane's own channel, where u = u_hi + u_lo exactly: dt and x are
//   bf16, so u has at most 16 significant bits; u_hi is u truncated to bf16 and
//   the remainder has at most 8 (in MODEL mode a clamped dt can leave a
//   remainder below 2^-16 of u, which is dropped);
//   A operand (lane l: k = 4*(l/32) .. +3 of row l%32) = (b_s, b_s, 0, 0) with
//   s = s(row), when the row's half c(row) matches the lane's k half, else 0.
// Both products are exact in fp32, so the state keeps fp32 accuracy; the
// matrix core replaces one multiply and turns the FMA into a multiply.  Each
// lane needs b_s for a lane-dependent s, so the B row is read with a per-lane
// 2-byte load (lanes whose row belongs to the other k half load from past the
// buffer's range, which reads 0); the C row is uniform and goes through scalar
// loads, unpacked on the scalar unit.
//
// The loop is bound by VALU issue: per state update one multiply for the
// exponent, one v_exp_f32 (two FMA issue slots on gfx950), one multiply for
// the decay and one FMA for the readout.  The gates of step t+1
// are computed between the state update of step t and its readout, so the
// exponentials cover the matrix-core latency and no exp result is consumed
// by the next instruction.  Moving the readout onto the matrix core (bf16 h,
// two 16x16x32 products per channel) issues fewer VALU instructions but ran
// slower here, as did one barrier-synchronised workgroup per CU.
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2v __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

template <int MODE, int TC, int DPL, bool CK = false>
__global__ void __launch_bounds__(64)
ssm_scan_fwd_mfma_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ dt,
                         const float* __restrict__ A_log, const uint16_t* __restrict__ Bm,
                         const uint16_t* __restrict__ Cm, const float* __restrict__ Dskip,
                         uint16_t* __restrict__ y, float* __restrict__ h_final, int T, int Dn, ScanEpi epi) {
  constexpr int SP = 16;
  const int n = blockIdx.x;
  const int l = threadIdx.x;
  const int c0 = (blockIdx.y * 64 + l) * DPL;          // this lane's first channel
  const bool act = c0 < Dn;
  const int d0 = act ? c0 : Dn - DPL;                  // Dn % DPL == 0 (checked by the dispatcher)
  const int ii = l & 31;                               // A-operand row of this lane
  const bool a_on = (((ii >> 2) & 1) == (l >> 5));     // row half == lane's k half
  const int s_row = (ii & 3) + 4 * (ii >> 3);          // state of that row

  float a2[DPL][SP];
  float dsk[DPL];
#pragma unroll
  for (int k = 0; k < DPL; ++k) {
#pragma unroll
    for (int s = 0; s < SP; ++s) {
      float e = fast_exp2(A_log[(size_t)(d0 + k) * SP + s] * HCLSM_LOG2E);
      if (MODE != HCLSM_SCAN_RAW) e = fminf(fmaxf(e, 1e-6f), 1.0f);
      a2[k][s] = -e * HCLSM_LOG2E;
    }
    dsk[k] = Dskip != nullptr ? Dskip[d0 + k] : 0.f;
  }

  f32x16_t h[DPL];
#pragma unroll
  for (int k = 0; k < DPL; ++k)
#pragma unroll
    for (int s = 0; s < SP; ++s) h[k][s] = 0.f;

  // Per-sequence buffer resources: byte offsets are (lane constant) + (step * row pitch, uniform).
  const size_t row0 = (size_t)n * T;
  const int slab = T * Dn * 2;                         // < 2^31 (checked by the dispatcher)
  const auto rx = __builtin_amdgcn_make_buffer_rsrc((void*)(x + row0 * Dn), 0, slab, kRawBufferWord3);
  const auto rd = __builtin_amdgcn_make_buffer_rsrc((void*)(dt + row0 * Dn), 0, slab, kRawBufferWord3);
  const auto ry = __builtin_amdgcn_make_buffer_rsrc((void*)(y + row0 * Dn), 0, slab, kRawBufferWord3);
  const auto rb = __builtin_amdgcn_make_buffer_rsrc((void*)(Bm + row0 * SP), 0, T * SP * 2, kRawBufferWord3);
  // SCAN_BLOCK: gate read like x; the optional pre-gate output through a resource of 0 records when
  // it is not wanted, so its stores are dropped without a branch
  const auto rg = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(MODE == SCAN_BLOCK ? reinterpret_cast<const uint16_t*>(epi.gate) + row0 * Dn : x + row0 * Dn), 0, slab,
      kRawBufferWord3);
  const auto rp = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(epi.y_pre ? reinterpret_cast<uint16_t*>(epi.y_pre) + row0 * Dn : y + row0 * Dn), 0,
      epi.y_pre ? slab : 0, kRawBufferWord3);
  const int vo = d0 * 2;
  const int vo_st = act ? vo : 0x7ffffff0;             // past num_records: the store is dropped
  const int vo_b = a_on ? s_row * 2 : 0x7ffffff0;   // rows of the other k half read 0 (past num_records)
  const int pitch = Dn * 2;
  const uint32_t* cw0 = reinterpret_cast<const uint32_t*>(Cm + row0 * SP);

  constexpr int GC = MODE == SCAN_BLOCK ? TC : 1;   // gate words prefetched with x / dt in SCAN_BLOCK
  uint32_t xv[TC], dv[TC], gv[GC];
  uint16_t bv[TC];
  auto load = [&](int t0, uint32_t* xo, uint32_t* dO, uint16_t* bO, uint32_t* gO) {
#pragma unroll
    for (int j = 0; j < TC; ++j) {
      const int t = t0 + j < T ? t0 + j : T - 1;
      if constexpr (DPL == 2) {
        xo[j] = __builtin_amdgcn_raw_buffer_load_b32(rx, vo, t * pitch, 0);
        dO[j] = __builtin_amdgcn_raw_buffer_load_b32(rd, vo, t * pitch, 0);
        if constexpr (MODE == SCAN_BLOCK) gO[j] = __builtin_amdgcn_raw_buffer_load_b32(rg, vo, t * pitch, 0);
      } else {
        xo[j] = __builtin_amdgcn_raw_buffer_load_b16(rx, vo, t * pitch, 0);
        dO[j] = __builtin_amdgcn_raw_buffer_load_b16(rd, vo, t * pitch, 0);
        if constexpr (MODE == SCAN_BLOCK) gO[j] = __builtin_amdgcn_raw_buffer_load_b16(rg, vo, t * pitch, 0);
      }
      bO[j] = __builtin_amdgcn_raw_buffer_load_b16(rb, vo_b, t * (SP * 2), 0);
    }
  };

  uint32_t cw[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) cw[i] = cw0[i];

  // Gates are computed one step ahead, between the state update of step t and its readout, so the
  // exponentials fill the matrix-core latency of the update and each exp result is consumed a step later.
  float gt[DPL][SP];
  float dtc[DPL];
  auto gates = [&](uint32_t dw) {
#pragma unroll
    for (int k = 0; k < DPL; ++k) {
      dtc[k] = scan_dt<MODE>(__uint_as_float(k == 0 ? dw << 16 : dw & 0xffff0000u));
#pragma unroll
      for (int s = 0; s < SP; ++s) gt[k][s] = dtc[k] * a2[k][s];
#pragma unroll
      for (int s = 0; s < SP; ++s) gt[k][s] = fast_exp2(gt[k][s]);
    }
  };

  // MFMA operands: only the low halves change per step; the zero halves stay in their registers (built once, so
  // no per-step copies of zeros)
  s16x4_t aop = {0, 0, 0, 0};
  s16x4_t bop[DPL];
#pragma unroll
  for (int k = 0; k < DPL; ++k) bop[k] = s16x4_t{0, 0, 0, 0};
  auto step = [&](int t, uint32_t xw, uint32_t dw_next, uint16_t bb, uint32_t gw) {
    if constexpr (CK) {   // the state before steps 8, 16, ..., for the backward (before step 0 it is zero)
      // state-major slabs (state s of channel d at s * Dn + d): one store per state writes the wave's channels,
      // whole lines
      if ((t & 7) == 0 && t > 0 && act) {
        float* cp = epi.ck + ((size_t)n * ((T + 7) >> 3) + (t >> 3)) * Dn * SP + d0;
#pragma unroll
        for (int s = 0; s < SP; ++s) {
          if constexpr (DPL == 2)
            *reinterpret_cast<f32x2v*>(cp + (size_t)s * Dn) = f32x2v{h[0][s], h[1][s]};
          else
            cp[(size_t)s * Dn] = h[0][s];
        }
      }
    }
    const int tn = t + 1 < T ? t + 1 : T - 1;
    uint32_t cwn[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) cwn[i] = cw0[(size_t)tn * 8 + i];
    aop.x = (short)bb;
    aop.y = (short)bb;
    float xs[DPL];
#pragma unroll
    for (int k = 0; k < DPL; ++k) {
      xs[k] = __uint_as_float(k == 0 ? xw << 16 : xw & 0xffff0000u);
      const float u = dtc[k] * xs[k];
      const uint32_t uhi = __float_as_uint(u) & 0xffff0000u;
      const float ulo = u - __uint_as_float(uhi);
      bop[k].x = (short)(uhi >> 16);
      bop[k].y = (short)(__float_as_uint(ulo) >> 16);
#pragma unroll
      for (int s = 0; s < SP; ++s) h[k][s] *= gt[k][s];
      h[k] = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(aop, bop[k], h[k], 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    gates(dw_next);
    __builtin_amdgcn_sched_barrier(0);
    float yo[DPL];
#pragma unroll
    for (int k = 0; k < DPL; ++k) {
      float y0 = 0.f, y1 = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        y0 = fmaf(h[k][2 * i], __uint_as_float(cw[i] << 16), y0);
        y1 = fmaf(h[k][2 * i + 1], __uint_as_float(cw[i] & 0xffff0000u), y1);
      }
      yo[k] = fmaf(dsk[k], xs[k], y0 + y1);
    }
    if constexpr (MODE == SCAN_BLOCK) {
      if constexpr (DPL == 2)
        __builtin_amdgcn_raw_buffer_store_b32(pack_bf16x2(yo[0], yo[1]), rp, vo_st, t * pitch, 0);
      else
        __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16_bits(yo[0]), rp, vo_st, t * pitch, 0);
#pragma unroll
      for (int k = 0; k < DPL; ++k) yo[k] *= silu_f(__uint_as_float(k == 0 ? gw << 16 : gw & 0xffff0000u));
    }
    if constexpr (DPL == 2)
      __builtin_amdgcn_raw_buffer_store_b32(pack_bf16x2(yo[0], yo[1]), ry, vo_st, t * pitch, 0);
    else
      __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16_bits(yo[0]), ry, vo_st, t * pitch, 0);
#pragma unroll
    for (int i = 0; i < 8; ++i) cw[i] = cwn[i];
  };

  load(0, xv, dv, bv, gv);
  gates(dv[0]);
  const int tfull = T - T % TC;
  for (int t0 = 0; t0 < tfull; t0 += TC) {
    // Issue priority falls with progress, by quarters of T.  The waves of a SIMD start together; with
    // equal priorities the sequencer issues oldest-first, so they would run almost one after another.  A
    // wave that gets a quarter ahead now yields to the others, and they finish closer together (same-box
    // A/B on MI355X: 69.0 -> 65.6 us per launch at config 1).
    {
      const int pr = (4 * t0) / T;
      if (pr == 0) __builtin_amdgcn_s_setprio(3);
      else if (pr == 1) __builtin_amdgcn_s_setprio(2);
      else if (pr == 2) __builtin_amdgcn_s_setprio(1);
      else __builtin_amdgcn_s_setprio(0);
    }
    uint32_t xn[TC], dn[TC], gn[GC];
    uint16_t bn[TC];
    load(t0 + TC, xn, dn, bn, gn);
#pragma unroll
    for (int j = 0; j < TC; ++j) step(t0 + j, xv[j], j + 1 < TC ? dv[j + 1] : dn[0], bv[j], gv[j < GC ? j : 0]);
#pragma unroll
    for (int j = 0; j < TC; ++j) { xv[j] = xn[j]; dv[j] = dn[j]; bv[j] = bn[j]; }
#pragma unroll
    for (int j = 0; j < GC; ++j) gv[j] = gn[j];
  }
#pragma unroll
  for (int j = 0; j < TC - 1; ++j)
    if (tfull + j < T) step(tfull + j, xv[j], dv[j + 1], bv[j], gv[j < GC ? j : 0]);

  if (h_final != nullptr && act) {
#pragma unroll
    for (int k = 0; k < DPL; ++k) {
      float* hp = h_final + ((size_t)n * Dn + d0 + k) * SP;
#pragma unroll
      for (int s = 0; s < SP; ++s) hp[s] = h[k][s];
    }
  }
}

template <int MODE, int TC, int DPL, bool CK = false>
static int launch_scan_mfma(const void* x, const void* dt, const float* A_log, const void* B,
                            const void* C, const float* Dskip, void* y, float* h_final,
                            int64_t batch, int64_t T, int64_t Dn, hipStream_t st, ScanEpi epi) {
  const int64_t lanes = Dn / DPL;
  dim3 grid((unsigned)batch, (unsigned)((lanes + 63) / 64));
  hipLaunchKernelGGL((ssm_scan_fwd_mfma_kernel<MODE, TC, DPL, CK>), grid, dim3(64), 0, st,
                     (const uint16_t*)x, (const uint16_t*)dt, A_log, (const uint16_t*)B,
                     (const uint16_t*)C, Dskip, (uint16_t*)y, h_final, (int)T, (int)Dn, epi);
  HCLSM_LAUNCH_CHECK();
  return 0;
}

static inline bool aligned(const void* p, uintptr_t a) { return (((uintptr_t)p) & (a - 1)) == 0; }

// Returns 1 if no fast kernel applies (caller falls back to the generic kernel).
template <int DT, int MODE>
static int try_scan_sgpr(const void* x, const void* dt, const float* A_log, const void* B,
                         const void* C, const float* Dskip, void* y, float* h_final,
                         int64_t batch, int64_t T, int64_t Dn, int64_t S, hipStream_t st, ScanEpi epi) {
  constexpr int ES = (int)sizeof(typename Elem<DT>::T);
  if (!aligned(B, 4) || !aligned(C, 4)) return 1;
  const bool pair = (Dn % 2 == 0) && aligned(x, 2 * ES) && aligned(dt, 2 * ES) && aligned(y, 2 * ES) &&
                    (!epi.gate || aligned(epi.gate, 2 * ES)) && (!epi.y_pre || aligned(epi.y_pre, 2 * ES));
#define HCLSM_SCAN_SGPR(SPV)                                                                      \
  if (S == SPV) {                                                                                  \
    if (pair) return launch_scan_sgpr<DT, SPV, MODE, 2, 4>(x, dt, A_log, B, C, Dskip, y, h_final, batch, T, Dn, st, epi); \
    return launch_scan_sgpr<DT, SPV, MODE, 1, 8>(x, dt, A_log, B, C, Dskip, y, h_final, batch, T, Dn, st, epi); \
  }
  if constexpr (DT == HCLSM_BF16) {
    if (S == 16 && T * Dn * 2 < 0x7fffffffLL) {
      // Steps per prefetched chunk: 4 while the grid is at most one round of three waves per SIMD (131 VGPRs,
      // three waves fit); past that 2 (120 VGPRs: four waves per SIMD, fewer rounds).  Measured on MI355X
      // (same-run A/B against 8-step chunks): config 1 (three waves per SIMD) 65.7 -> 64.2 us with 4, 65.5 with
      // 2; config 4 (six per SIMD) 1833 -> 1795 us with 2, 1822 with 4.
      if constexpr (MODE == SCAN_BLOCK) {   // the gate prefetch costs registers: 4-step chunks throughout
        if (pair) return launch_scan_mfma<MODE, 4, 2>(x, dt, A_log, B, C, Dskip, y, h_final, batch, T, Dn, st, epi);
        return launch_scan_mfma<MODE, 4, 1>(x, dt, A_log, B, C, Dskip, y, h_final, batch, T, Dn, st, epi);
      } else {
        int cus = 0;
        const int rc = device_cus(&cus);
        if (rc) return rc;
        const int64_t waves = batch * ((Dn / (pair ? 2 : 1) + 63) / 64);
        const bool many = waves > 3 * 4 * (int64_t)cus;   // more than three waves per SIMD
        if (pair && many) return launch_scan_mfma<MODE, 2, 2>(x, dt, A_log, B, C, Dskip, y, h_final, batch, T, Dn, st, epi);
        if (pair) return launch_scan_mfma<MODE, 4, 2>(x, dt, A_log, B, C, Dskip, y, h_final, batch, T, Dn, st, epi);
        if (many) return launch_scan_mfma<MODE, 2, 1>(x, dt, A_log, B, C, Dskip, y, h_final, batch, T, Dn, st, epi);
        return launch_scan_mfma<MODE, 4, 1>(x, dt, A_log, B, C, Dskip, y, h_final, batch, T, Dn, st, epi);
      }
    }
    HCLSM_SCAN_SGPR(4)
    HCLSM_SCAN_SGPR(8)
  } else if constexpr (DT == HCLSM_F32) {
    HCLSM_SCAN_SGPR(4)
    HCLSM_SCAN_SGPR(8)
    HCLSM_SCAN_SGPR(16)
  }
#undef HCLSM_SCAN_SGPR
  return 1;
}

template <int DT, int SP, int MODE>
static int launch_scan(const void* x, const void* dt, const float* A_log, const void* B,
                       const void* C, const float* Dskip, void* y, float* h_final,
                       int64_t batch, int64_t T, int64_t Dn, int64_t S, hipStream_t st, ScanEpi epi) {
  using TT = typename Elem<DT>::T;
  const int64_t lanes = Dn * scan_lanes_per_channel(SP);
  const int block = (lanes % 256 == 0) ? 256 : (lanes % 128 == 0 ? 128 : 64);
  dim3 grid((unsigned)batch, (unsigned)((lanes + block - 1) / block));
  hipLaunchKernelGGL((ssm_scan_fwd_kernel<DT, SP, MODE>), grid, dim3(block), 0, st,
                     (const TT*)x, (const TT*)dt, A_log, (const TT*)B, (const TT*)C, Dskip,
                     (TT*)y, h_final, (int)T, (int)Dn, (int)S, epi);
  HCLSM_LAUNCH_CHECK();
  return 0;
}

template <int DT, int SP, int MODE>
static int dispatch_one(const void* x, const void* dt, const float* A_log, const void* B, const void* C,
                        const float* Dskip, void* y, float* h_final, int64_t batch, int64_t T, int64_t Dn,
                        int64_t S, hipStream_t st, ScanEpi epi) {
  if constexpr (DT == HCLSM_BF16 || DT == HCLSM_F32) {
    if (SP == S) {
      const int r = try_scan_sgpr<DT, MODE>(x, dt, A_log, B, C, Dskip, y, h_final, batch, T, Dn, S, st, epi);
      if (r != 1) return r;
    }
  }
  return launch_scan<DT, SP, MODE>(x, dt, A_log, B, C, Dskip, y, h_final, batch, T, Dn, S, st, epi);
}

template <int DT, int SP>
static int dispatch_mode(int mode, const void* x, const void* dt, const float* A_log, const void* B,
                         const void* C, const float* Dskip, void* y, float* h_final,
                         int64_t batch, int64_t T, int64_t Dn, int64_t S, hipStream_t st, ScanEpi epi) {
  if (mode == HCLSM_SCAN_RAW)
    return dispatch_one<DT, SP, HCLSM_SCAN_RAW>(x, dt, A_log, B, C, Dskip, y, h_final, batch, T, Dn, S, st, epi);
  if (mode == HCLSM_SCAN_MODEL)
    return dispatch_one<DT, SP, HCLSM_SCAN_MODEL>(x, dt, A_log, B, C, Dskip, y, h_final, batch, T, Dn, S, st, epi);
  return dispatch_one<DT, SP, SCAN_BLOCK>(x, dt, A_log, B, C, Dskip, y, h_final, batch, T, Dn, S, st, epi);
}

template <int DT>
static int dispatch_sp(int mode, const void* x, const void* dt, const float* A_log, const void* B,
                       const void* C, const float* Dskip, void* y, float* h_final,
                       int64_t batch, int64_t T, int64_t Dn, int64_t S, hipStream_t st, ScanEpi epi) {
  if (S <= 4) return dispatch_mode<DT, 4>(mode, x, dt, A_log, B, C, Dskip, y, h_final, batch, T, Dn, S, st, epi);
  if (S <= 8) return dispatch_mode<DT, 8>(mode, x, dt, A_log, B, C, Dskip, y, h_final, batch, T, Dn, S, st, epi);
  if (S <= 16) return dispatch_mode<DT, 16>(mode, x, dt, A_log, B, C, Dskip, y, h_final, batch, T, Dn, S, st, epi);
  if (S <= 32) return dispatch_mode<DT, 32>(mode, x, dt, A_log, B, C, Dskip, y, h_final, batch, T, Dn, S, st, epi);
  if (S <= 64) return dispatch_mode<DT, 64>(mode, x, dt, A_log, B, C, Dskip, y, h_final, batch, T, Dn, S, st, epi);
  return dispatch_mode<DT, 128>(mode, x, dt, A_log, B, C, Dskip, y, h_final, batch, T, Dn, S, st, epi);
}

static int scan_entry(int mode, const void* x, const void* dt, const float* A_log, const void* B, const void* C,
                      const float* Dskip, void* y, float* h_final, int64_t batch, int64_t T, int64_t d_inner,
                      int64_t d_state, int dtype, hipStream_t st, ScanEpi epi) {
  if (batch < 0 || T < 0 || d_inner < 0 || d_state < 1) return HCLSM_ERR_SHAPE;
  if (batch > 0x7fffffffLL || T > 0x7fffffffLL || d_inner > 0x7fffffffLL) return HCLSM_ERR_SHAPE;
  if ((d_inner * 4 + 63) / 64 > 65535) return HCLSM_ERR_SHAPE;
  if (d_state > 128) return HCLSM_ERR_UNSUPPORTED;
  if (dtype != HCLSM_F32 && dtype != HCLSM_BF16 && dtype != HCLSM_F16) return HCLSM_ERR_DTYPE;
  if (batch == 0 || T == 0 || d_inner == 0) {
    // nothing to scan; h_final (if any) is the zero initial state
    if (h_final && batch > 0 && d_inner > 0) return zero_fill_f32(h_final, batch * d_inner * d_state, st);
    return 0;
  }
  if (!x || !dt || !A_log || !B || !C || !y) return HCLSM_ERR_NULL;
  switch (dtype) {
    case HCLSM_F32:
      return dispatch_sp<HCLSM_F32>(mode, x, dt, A_log, B, C, Dskip, y, h_final, batch, T, d_inner, d_state, st, epi);
    case HCLSM_BF16:
      return dispatch_sp<HCLSM_BF16>(mode, x, dt, A_log, B, C, Dskip, y, h_final, batch, T, d_inner, d_state, st, epi);
    default:
      return dispatch_sp<HCLSM_F16>(mode, x, dt, A_log, B, C, Dskip, y, h_final, batch, T, d_inner, d_state, st, epi);
  }
}

// The forward that also writes the backward's checkpoints (epi.ck): the bf16, d_state 16 matrix-core kernel
// only, with the chunking the plain forward picks.  HCLSM_ERR_UNSUPPORTED where that kernel does not apply.
int scan_fwd_ckpt(int mode, const void* x, const void* dt, const float* A_log, const void* B, const void* C,
                  const float* Dskip, void* y, float* h_final, int64_t batch, int64_t T, int64_t Dn, int64_t S,
                  int dtype, const void* gate, void* y_pre, float* ck, hipStream_t st) {
  const ScanEpi epi{gate, y_pre, ck};
  if (batch < 1 || T < 1 || Dn < 1 || batch > 0x7fffffffLL || T > 0x7fffffffLL || (Dn * 4 + 63) / 64 > 65535)
    return HCLSM_ERR_SHAPE;
  if (dtype != HCLSM_BF16 || S != 16 || T * Dn * 2 >= 0x7fffffffLL) return HCLSM_ERR_UNSUPPORTED;
  if (!x || !dt || !A_log || !B || !C || !y || !epi.ck) return HCLSM_ERR_NULL;
  if (mode == SCAN_BLOCK && !epi.gate) return HCLSM_ERR_NULL;
  if (!aligned(B, 4) || !aligned(C, 4) || !aligned(epi.ck, 16)) return HCLSM_ERR_UNSUPPORTED;
  const bool pair = (Dn % 2 == 0) && aligned(x, 4) && aligned(dt, 4) && aligned(y, 4) &&
                    (!epi.gate || aligned(epi.gate, 4)) && (!epi.y_pre || aligned(epi.y_pre, 4));
  int cus = 0;
  const int rc = device_cus(&cus);
  if (rc) return rc;
  const bool many = batch * ((Dn / (pair ? 2 : 1) + 63) / 64) > 3 * 4 * (int64_t)cus;
#define HCLSM_CK(MODE_)                                                                                       \
  if constexpr (MODE_ == SCAN_BLOCK) {                                                                        \
    if (pair) return launch_scan_mfma<MODE_, 4, 2, true>(x, dt, A_log, B, C, Dskip, y, h_final, batch, T, Dn, st, epi); \
    return launch_scan_mfma<MODE_, 4, 1, true>(x, dt, A_log, B, C, Dskip, y, h_final, batch, T, Dn, st, epi); \
  } else {                                                                                                    \
    if (pair && many) return launch_scan_mfma<MODE_, 2, 2, true>(x, dt, A_log, B, C, Dskip, y, h_final, batch, T, Dn, st, epi); \
    if (pair) return launch_scan_mfma<MODE_, 4, 2, true>(x, dt, A_log, B, C, Dskip, y, h_final, batch, T, Dn, st, epi); \
    if (many) return launch_scan_mfma<MODE_, 2, 1, true>(x, dt, A_log, B, C, Dskip, y, h_final, batch, T, Dn, st, epi); \
    return launch_scan_mfma<MODE_, 4, 1, true>(x, dt, A_log, B, C, Dskip, y, h_final, batch, T, Dn, st, epi); \
  }
  if (mode == HCLSM_SCAN_RAW) { HCLSM_CK(HCLSM_SCAN_RAW) }
  if (mode == HCLSM_SCAN_MODEL) { HCLSM_CK(HCLSM_SCAN_MODEL) }
  if (mode == SCAN_BLOCK) { HCLSM_CK(SCAN_BLOCK) }
#undef HCLSM_CK
  return HCLSM_ERR_MODE;
}

}  // namespace hclsm

extern "C" int hclsm_ssm_scan_fwd(const void* x, const void* dt, const float* A_log,
                                  const void* B, const void* C, const float* Dskip,
                                  void* y, float* h_final,
                                  int64_t batch, int64_t T, int64_t d_inner, int64_t d_state,
                                  int dtype, int mode, void* stream) {
  if (mode != HCLSM_SCAN_RAW && mode != HCLSM_SCAN_MODEL) return HCLSM_ERR_MODE;
  return hclsm::scan_entry(mode, x, dt, A_log, B, C, Dskip, y, h_final, batch, T, d_inner, d_state, dtype,
                           (hipStream_t)stream, hclsm::ScanEpi{nullptr, nullptr});
}

extern "C" int hclsm_ssm_block_scan_fwd(const void* z, const void* dt_in, const float* A_log, const void* B,
                                        const void* C, const void* gate, void* y, void* y_pre, float* h_final,
                                        int64_t batch, int64_t T, int64_t d_inner, int64_t d_state, int dtype,
                                        void* stream) {
  if (batch > 0 && T > 0 && d_inner > 0 && !gate) return HCLSM_ERR_NULL;
  return hclsm::scan_entry(hclsm::SCAN_BLOCK, z, dt_in, A_log, B, C, nullptr, y, h_final, batch, T, d_inner,
                           d_state, dtype, (hipStream_t)stream, hclsm::ScanEpi{gate, y_pre});
}
