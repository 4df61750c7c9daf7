// Slot attention on gfx950: the attention core and the building blocks of the
// slot-attention iteration (LayerNorm, MFMA linear layers, fused GRU cell).
//
// slot_core_kernel (one workgroup per frame b, 4 waves):
//   phase 1  logits[n][m] = scale * q[n] . k[m]          MFMA, tiles of 16 slots x 16 tokens,
//                                                         fp32 into LDS
//   phase 2  softmax over the slot axis for every token  (optional logit clamp, optional
//            +denom_eps in the denominator), optional renormalisation over tokens
//            (attn + eps) / sum_m (attn + eps); attn written to global if asked
//   phase 3  updates[n] = sum_m attn[n][m] v[m]           MFMA over 32-token chunks of v,
//            each chunk staged transposed in LDS so both operands are contiguous
// linear_kernel: Y = X W^T (+ bias) (ReLU) (+ residual) (clamp), X / W K-contiguous, one
//   wave per 32x32 output tile, lane group g streaming its quarter of K.
// gru_kernel: the six gate products of torch.nn.GRUCell for a 32x16 tile of h', with the
//   gate nonlinearities and the (1-z) n + z h blend in the epilogue.
#include "mfma.h"

namespace hclsm {

// ---------------------------------------------------------------------------
// LayerNorm over the last dim: one wave per row, two-pass mean / variance in fp32.
template <int DTI, int DTO>
__global__ void __launch_bounds__(256)
layer_norm_kernel(const typename MM<DTI>::T* __restrict__ x, int64_t ldx, const float* __restrict__ w,
                  const float* __restrict__ b, typename MM<DTO>::T* __restrict__ y, int64_t ldy, int64_t M,
                  int D, float eps) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= M) return;
  const typename MM<DTI>::T* xr = x + row * ldx;
  float s = 0.f;
  for (int i = lane; i < D; i += 64) s += MM<DTI>::tof(xr[i]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
  const float mean = s / (float)D;
  float v = 0.f;
  for (int i = lane; i < D; i += 64) {
    const float d = MM<DTI>::tof(xr[i]) - mean;
    v += d * d;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  const float rstd = 1.f / sqrtf(v / (float)D + eps);
  typename MM<DTO>::T* yr = y + row * ldy;
  for (int i = lane; i < D; i += 64) {
    float t = (MM<DTI>::tof(xr[i]) - mean) * rstd;
    if (w) t *= w[i];
    if (b) t += b[i];
    yr[i] = MM<DTO>::fromf(t);
  }
}

// ---------------------------------------------------------------------------
// Linear layer, NT: Y[M][N] = X[M][K] . W[N][K]^T
template <int DT, int OT>
__global__ void __launch_bounds__(256)
linear_kernel(const typename MM<DT>::T* __restrict__ X, int64_t ldx, const typename MM<DT>::T* __restrict__ W,
              int64_t ldw, const float* __restrict__ bias, const float* __restrict__ resid, int64_t ldr,
              typename MM<OT>::T* __restrict__ Y, int64_t ldy, typename MM<DT>::T* __restrict__ Y2, int64_t ldy2,
              int64_t M, int64_t N, int64_t K, int relu, float clamp_v) {
  using A = MM<DT>;
  constexpr int KPL = A::KPL;
  const int64_t wave = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t tiles_n = (N + 31) / 32;
  if (wave >= ((M + 31) / 32) * tiles_n) return;
  const int64_t tm = wave / tiles_n, tn = wave - tm * tiles_n;
  const int lane = threadIdx.x & 63, g = lane >> 4, li = lane & 15;
  const int64_t K4 = K / 4;
  const typename A::T* pa[2];
  const typename A::T* pb[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    int64_t r = tm * 32 + 16 * t + li;
    r = r < M ? r : M - 1;
    pa[t] = X + r * ldx + g * K4;
    int64_t c = tn * 32 + 16 * t + li;
    c = c < N ? c : N - 1;
    pb[t] = W + c * ldw + g * K4;
  }
  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 2
  for (int64_t c = 0; c < K4; c += KPL) {
    const typename A::Op a0 = A::load(pa[0] + c), a1 = A::load(pa[1] + c);
    const typename A::Op b0 = A::load(pb[0] + c), b1 = A::load(pb[1] + c);
    acc[0][0] = A::mfma(a0, b0, acc[0][0]);
    acc[0][1] = A::mfma(a0, b1, acc[0][1]);
    acc[1][0] = A::mfma(a1, b0, acc[1][0]);
    acc[1][1] = A::mfma(a1, b1, acc[1][1]);
  }
#pragma unroll
  for (int tj = 0; tj < 2; ++tj) {
    const int64_t col = tn * 32 + 16 * tj + li;
    if (col >= N) continue;
    const float bv = bias ? bias[col] : 0.f;
#pragma unroll
    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t row = tm * 32 + 16 * ti + 4 * g + r;
        if (row >= M) continue;
        float val = acc[ti][tj][r] + bv;
        if (relu) val = fmaxf(val, 0.f);
        if (resid) val += resid[row * ldr + col];
        if (clamp_v > 0.f) val = fminf(fmaxf(val, -clamp_v), clamp_v);
        Y[row * ldy + col] = MM<OT>::fromf(val);
        if (Y2) Y2[row * ldy2 + col] = A::fromf(val);
      }
  }
}

// ---------------------------------------------------------------------------
// torch.nn.GRUCell: h' = (1 - z) * n + z * h with
//   r = sig(x Wir^T + bir + h Whr^T + bhr), z = sig(x Wiz^T + biz + h Whz^T + bhz),
//   n = tanh(x Win^T + bin + r * (h Whn^T + bhn)); weight rows ordered [r; z; n].
template <int DT>
__global__ void __launch_bounds__(256)
gru_kernel(const typename MM<DT>::T* __restrict__ X, int64_t ldx, const typename MM<DT>::T* __restrict__ Hb,
           int64_t ldhb, const float* __restrict__ Hf, int64_t ldh, const typename MM<DT>::T* __restrict__ Wih,
           const typename MM<DT>::T* __restrict__ Whh, const float* __restrict__ bih, const float* __restrict__ bhh,
           float* __restrict__ out, int64_t ldo, typename MM<DT>::T* __restrict__ out2, int64_t ldo2, int64_t M,
           int64_t H, int64_t Kx) {
  using A = MM<DT>;
  constexpr int KPL = A::KPL;
  const int64_t wave = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t tiles_n = (H + 15) / 16;
  if (wave >= ((M + 31) / 32) * tiles_n) return;
  const int64_t tm = wave / tiles_n, tn = wave - tm * tiles_n;
  const int lane = threadIdx.x & 63, g = lane >> 4, li = lane & 15;
  int64_t colr = tn * 16 + li;
  colr = colr < H ? colr : H - 1;
  f32x4 acc[2][6];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 6; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  int64_t rows[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int64_t r = tm * 32 + 16 * t + li;
    rows[t] = r < M ? r : M - 1;
  }
  {  // input gates: x . W_ih^T
    const int64_t K4 = Kx / 4;
    const typename A::T* pa[2] = {X + rows[0] * ldx + g * K4, X + rows[1] * ldx + g * K4};
    const typename A::T* pw[3] = {Wih + colr * Kx + g * K4, Wih + (H + colr) * Kx + g * K4,
                                  Wih + (2 * H + colr) * Kx + g * K4};
    for (int64_t c = 0; c < K4; c += KPL) {
      const typename A::Op a0 = A::load(pa[0] + c), a1 = A::load(pa[1] + c);
#pragma unroll
      for (int q = 0; q < 3; ++q) {
        const typename A::Op bq = A::load(pw[q] + c);
        acc[0][q] = A::mfma(a0, bq, acc[0][q]);
        acc[1][q] = A::mfma(a1, bq, acc[1][q]);
      }
    }
  }
  {  // hidden gates: h . W_hh^T
    const int64_t K4 = H / 4;
    const typename A::T* pa[2] = {Hb + rows[0] * ldhb + g * K4, Hb + rows[1] * ldhb + g * K4};
    const typename A::T* pw[3] = {Whh + colr * H + g * K4, Whh + (H + colr) * H + g * K4,
                                  Whh + (2 * H + colr) * H + g * K4};
    for (int64_t c = 0; c < K4; c += KPL) {
      const typename A::Op a0 = A::load(pa[0] + c), a1 = A::load(pa[1] + c);
#pragma unroll
      for (int q = 0; q < 3; ++q) {
        const typename A::Op bq = A::load(pw[q] + c);
        acc[0][3 + q] = A::mfma(a0, bq, acc[0][3 + q]);
        acc[1][3 + q] = A::mfma(a1, bq, acc[1][3 + q]);
      }
    }
  }
  const int64_t col = tn * 16 + li;
  if (col >= H) return;
  const float bir = bih ? bih[col] : 0.f, biz = bih ? bih[H + col] : 0.f, bin = bih ? bih[2 * H + col] : 0.f;
  const float bhr = bhh ? bhh[col] : 0.f, bhz = bhh ? bhh[H + col] : 0.f, bhn = bhh ? bhh[2 * H + col] : 0.f;
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t row = tm * 32 + 16 * t + 4 * g + r;
      if (row >= M) continue;
      const float rg = sigmoid_f(acc[t][0][r] + bir + acc[t][3][r] + bhr);
      const float zg = sigmoid_f(acc[t][1][r] + biz + acc[t][4][r] + bhz);
      const float ng = tanh_f(acc[t][2][r] + bin + rg * (acc[t][5][r] + bhn));
      const float hv = Hf[row * ldh + col];
      const float o = (1.f - zg) * ng + zg * hv;
      out[row * ldo + col] = o;
      if (out2) out2[row * ldo2 + col] = A::fromf(o);
    }
}

// ---------------------------------------------------------------------------
// Slot-attention core, one workgroup per frame.
struct CoreArgs {
  int64_t ldq, ldk, ldv, ldo, qb, kb, vb, ob;  // row strides and frame strides (elements)
  int N, M, D, NP, MP;                          // NP, MP: N, M rounded up to 16
  float scale, denom_eps, logit_clamp, renorm_eps;
};

constexpr int CORE_VCHUNK = 32;   // tokens of v staged per phase-3 step
constexpr int CORE_VPAD = 8;      // LDS row padding (elements) of the transposed v chunk
constexpr int CORE_MAX_TILES = 16;  // output tiles per wave per phase-3 pass

template <int DT, int AT>
__global__ void __launch_bounds__(256)
slot_core_kernel(const typename MM<DT>::T* __restrict__ q, const typename MM<DT>::T* __restrict__ k,
                 const typename MM<DT>::T* __restrict__ v, typename MM<DT>::T* __restrict__ out,
                 typename MM<AT>::T* __restrict__ attn_out, CoreArgs a) {
  using A = MM<DT>;
  using TT = typename A::T;
  constexpr int KPL = A::KPL;
  extern __shared__ __align__(16) unsigned char smem[];
  float* S = reinterpret_cast<float*>(smem);                          // [NP][MP] fp32
  TT* P = reinterpret_cast<TT*>(S + (size_t)a.NP * a.MP);             // [NP][MP] operand copy
  float* rs = reinterpret_cast<float*>(P + (size_t)a.NP * a.MP);       // [NP]
  TT* VT = reinterpret_cast<TT*>(rs + a.NP + 4);                       // [D][VCHUNK + VPAD]
  const int VLD = CORE_VCHUNK + CORE_VPAD;

  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63, g = lane >> 4, li = lane & 15;
  const TT* qb = q + b * a.qb;
  const TT* kb = k + b * a.kb;
  const TT* vb = v + b * a.vb;

  // ---- phase 1: logits
  {
    const int nt_n = a.NP / 16, nt_m = a.MP / 16;
    const int D4 = a.D / 4;
    for (int tile = wid; tile < nt_n * nt_m; tile += 4) {
      const int tn = tile / nt_m, tmm = tile - tn * nt_m;
      int rn = tn * 16 + li;
      rn = rn < a.N ? rn : a.N - 1;
      int rm = tmm * 16 + li;
      rm = rm < a.M ? rm : a.M - 1;
      const TT* pq = qb + (int64_t)rn * a.ldq + g * D4;
      const TT* pk = kb + (int64_t)rm * a.ldk + g * D4;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      for (int c = 0; c < D4; c += KPL) acc = A::mfma(A::load(pq + c), A::load(pk + c), acc);
#pragma unroll
      for (int r = 0; r < 4; ++r) S[(tn * 16 + 4 * g + r) * a.MP + tmm * 16 + li] = acc[r] * a.scale;
    }
  }
  __syncthreads();

  // ---- phase 2: softmax over slots per token (+ optional renorm over tokens)
  for (int m = tid; m < a.MP; m += 256) {
    if (m < a.M) {
      float mx = -INFINITY;
      for (int n = 0; n < a.N; ++n) {
        float s = S[n * a.MP + m];
        if (a.logit_clamp > 0.f) s = fminf(fmaxf(s, -a.logit_clamp), a.logit_clamp);
        S[n * a.MP + m] = s;
        mx = fmaxf(mx, s);
      }
      float sum = 0.f;
      for (int n = 0; n < a.N; ++n) {
        const float e = __expf(S[n * a.MP + m] - mx);
        S[n * a.MP + m] = e;
        sum += e;
      }
      const float inv = 1.f / (sum + a.denom_eps);
      for (int n = 0; n < a.N; ++n) {
        const float p = S[n * a.MP + m] * inv;
        S[n * a.MP + m] = p;
        if (attn_out) attn_out[b * (int64_t)a.N * a.M + (int64_t)n * a.M + m] = MM<AT>::fromf(p);
      }
      for (int n = a.N; n < a.NP; ++n) S[n * a.MP + m] = 0.f;
    } else {
      for (int n = 0; n < a.NP; ++n) S[n * a.MP + m] = 0.f;
    }
  }
  __syncthreads();
  const bool renorm = a.renorm_eps >= 0.f;
  if (renorm) {
    for (int n = wid; n < a.N; n += 4) {
      float s = 0.f;
      for (int m = lane; m < a.M; m += 64) s += S[n * a.MP + m] + a.renorm_eps;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
      if (lane == 0) rs[n] = 1.f / s;
    }
    __syncthreads();
  }
  for (int i = tid; i < a.NP * a.MP; i += 256) {
    const int n = i / a.MP, m = i - n * a.MP;
    float p = S[i];
    if (renorm) p = (n < a.N && m < a.M) ? (p + a.renorm_eps) * rs[n] : 0.f;
    P[i] = A::fromf(p);
  }
  __syncthreads();

  // ---- phase 3: updates = attn . v, 32 tokens at a time, v chunk transposed in LDS
  const int nt_n = a.NP / 16, nt_d = a.D / 16;
  const int ntiles = nt_n * nt_d;
  for (int tbase = 0; tbase < ntiles; tbase += 4 * CORE_MAX_TILES) {
    f32x4 acc[CORE_MAX_TILES];
#pragma unroll
    for (int i = 0; i < CORE_MAX_TILES; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int m0 = 0; m0 < a.MP; m0 += CORE_VCHUNK) {
      // stage v[m0 .. m0+31][0 .. D) transposed: VT[d][ml]; rows past M are zero
      for (int i = tid; i < CORE_VCHUNK * a.D; i += 256) {
        const int ml = i / a.D, d = i - ml * a.D;
        const int m = m0 + ml;
        VT[d * VLD + ml] = (m < a.M) ? vb[(int64_t)m * a.ldv + d] : A::fromf(0.f);
      }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < CORE_MAX_TILES; ++i) {
        const int tile = tbase + wid + 4 * i;
        if (tile < ntiles) {
          const int tn = tile / nt_d, td = tile - tn * nt_d;
          const TT* pp = P + (tn * 16 + li) * a.MP + m0;
          const TT* pv = VT + (td * 16 + li) * VLD;
          if constexpr (KPL == 8) {
            // one MFMA: lane group g covers tokens m0 + 8g .. 8g+7
            acc[i] = A::mfma(A::load(pp + 8 * g), A::load(pv + 8 * g), acc[i]);
          } else {
#pragma unroll
            for (int s = 0; s < CORE_VCHUNK / 4; ++s)
              acc[i] = A::mfma(A::load(pp + 4 * s + g), A::load(pv + 4 * s + g), acc[i]);
          }
        }
      }
      __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < CORE_MAX_TILES; ++i) {
      const int tile = tbase + wid + 4 * i;
      if (tile < ntiles) {
        const int tn = tile / nt_d, td = tile - tn * nt_d;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int n = tn * 16 + 4 * g + r;
          if (n < a.N) out[b * a.ob + (int64_t)n * a.ldo + td * 16 + li] = A::fromf(acc[i][r]);
        }
      }
    }
  }
}

static size_t core_smem(int NP, int MP, int D, int esize) {
  return (size_t)NP * MP * 4 + (size_t)NP * MP * esize + (size_t)(NP + 4) * 4 +
         (size_t)D * (CORE_VCHUNK + CORE_VPAD) * esize;
}

static bool al16(const void* p) { return (((uintptr_t)p) & 15) == 0; }

}  // namespace hclsm

using namespace hclsm;

extern "C" int hclsm_layer_norm(const void* x, int64_t ldx, const float* w, const float* b, void* y, int64_t ldy,
                                int64_t M, int64_t D, float eps, int in_dtype, int out_dtype, void* stream) {
  if (M < 0 || D < 0 || D > 0x7fffffff) return HCLSM_ERR_SHAPE;
  if (M == 0 || D == 0) return 0;
  if (!x || !y) return HCLSM_ERR_NULL;
  hipStream_t st = (hipStream_t)stream;
  const unsigned grid = (unsigned)((M + 3) / 4);
#define HCLSM_LN(I, O)                                                                                     \
  if (in_dtype == I && out_dtype == O) {                                                                   \
    hipLaunchKernelGGL((layer_norm_kernel<I, O>), dim3(grid), dim3(256), 0, st, (const MM<I>::T*)x, ldx, w, b, \
                       (MM<O>::T*)y, ldy, M, (int)D, eps);                                                 \
    HCLSM_LAUNCH_CHECK();                                                                                  \
    return 0;                                                                                              \
  }
  HCLSM_LN(HCLSM_F32, HCLSM_F32)
  HCLSM_LN(HCLSM_F32, HCLSM_BF16)
  HCLSM_LN(HCLSM_BF16, HCLSM_BF16)
  HCLSM_LN(HCLSM_BF16, HCLSM_F32)
  HCLSM_LN(HCLSM_F32, HCLSM_F16)
  HCLSM_LN(HCLSM_F16, HCLSM_F16)
#undef HCLSM_LN
  return HCLSM_ERR_DTYPE;
}

extern "C" int hclsm_linear(const void* x, int64_t ldx, const void* w, int64_t ldw, const float* bias,
                            const float* resid, int64_t ldr, void* y, int64_t ldy, int y_dtype, void* y2,
                            int64_t ldy2, int64_t M, int64_t N, int64_t K, int relu, float clamp, int dtype,
                            void* stream) {
  if (M < 0 || N < 0 || K < 0) return HCLSM_ERR_SHAPE;
  if (M == 0 || N == 0) return 0;
  if (!x || !w || !y) return HCLSM_ERR_NULL;
  const int kpl = dtype == HCLSM_F32 ? 1 : 8;
  if (K % (4 * kpl) != 0) return HCLSM_ERR_UNSUPPORTED;
  if (kpl == 8 && (!al16(x) || !al16(w) || ldx % 8 || ldw % 8)) return HCLSM_ERR_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  const int64_t waves = ((M + 31) / 32) * ((N + 31) / 32);
  const unsigned grid = (unsigned)((waves + 3) / 4);
#define HCLSM_LIN(D, O)                                                                                    \
  if (dtype == D && y_dtype == O) {                                                                        \
    hipLaunchKernelGGL((linear_kernel<D, O>), dim3(grid), dim3(256), 0, st, (const MM<D>::T*)x, ldx,        \
                       (const MM<D>::T*)w, ldw, bias, resid, ldr, (MM<O>::T*)y, ldy, (MM<D>::T*)y2, ldy2, M,  \
                       N, K, relu, clamp);                                                                 \
    HCLSM_LAUNCH_CHECK();                                                                                  \
    return 0;                                                                                              \
  }
  HCLSM_LIN(HCLSM_BF16, HCLSM_BF16)
  HCLSM_LIN(HCLSM_BF16, HCLSM_F32)
  HCLSM_LIN(HCLSM_F16, HCLSM_F16)
  HCLSM_LIN(HCLSM_F16, HCLSM_F32)
  HCLSM_LIN(HCLSM_F32, HCLSM_F32)
#undef HCLSM_LIN
  return HCLSM_ERR_DTYPE;
}

extern "C" int hclsm_gru_cell(const void* x, int64_t ldx, const void* hb, int64_t ldhb, const float* h, int64_t ldh,
                              const void* w_ih, const void* w_hh, const float* b_ih, const float* b_hh, float* out,
                              int64_t ldo, void* out2, int64_t ldo2, int64_t M, int64_t H, int64_t Kx, int dtype,
                              void* stream) {
  if (M < 0 || H < 0 || Kx < 0) return HCLSM_ERR_SHAPE;
  if (M == 0 || H == 0) return 0;
  if (!x || !hb || !h || !w_ih || !w_hh || !out) return HCLSM_ERR_NULL;
  const int kpl = dtype == HCLSM_F32 ? 1 : 8;
  if (Kx % (4 * kpl) || H % (4 * kpl)) return HCLSM_ERR_UNSUPPORTED;
  if (kpl == 8 && (!al16(x) || !al16(hb) || !al16(w_ih) || !al16(w_hh) || ldx % 8 || ldhb % 8))
    return HCLSM_ERR_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  const int64_t waves = ((M + 31) / 32) * ((H + 15) / 16);
  const unsigned grid = (unsigned)((waves + 3) / 4);
#define HCLSM_GRU(D)                                                                                        \
  if (dtype == D) {                                                                                         \
    hipLaunchKernelGGL((gru_kernel<D>), dim3(grid), dim3(256), 0, st, (const MM<D>::T*)x, ldx,               \
                       (const MM<D>::T*)hb, ldhb, h, ldh, (const MM<D>::T*)w_ih, (const MM<D>::T*)w_hh, b_ih, \
                       b_hh, out, ldo, (MM<D>::T*)out2, ldo2, M, H, Kx);                                    \
    HCLSM_LAUNCH_CHECK();                                                                                   \
    return 0;                                                                                               \
  }
  HCLSM_GRU(HCLSM_BF16)
  HCLSM_GRU(HCLSM_F16)
  HCLSM_GRU(HCLSM_F32)
#undef HCLSM_GRU
  return HCLSM_ERR_DTYPE;
}

extern "C" int hclsm_slot_attn_core(const void* q, int64_t ldq, int64_t q_bstride, const void* k, int64_t ldk,
                                    int64_t k_bstride, const void* v, int64_t ldv, int64_t v_bstride, void* out,
                                    int64_t ldo, int64_t o_bstride, void* attn, int attn_dtype, int64_t B, int64_t N,
                                    int64_t M, int64_t D, float scale, float denom_eps, float logit_clamp,
                                    float renorm_eps, int dtype, void* stream) {
  if (B < 0 || N < 0 || M < 0 || D < 0 || B > 0x7fffffff || N > 4096 || M > 0x7fffffff) return HCLSM_ERR_SHAPE;
  if (B == 0 || N == 0) return 0;
  if (!q || !k || !v || !out) return HCLSM_ERR_NULL;
  if (dtype != HCLSM_BF16 && dtype != HCLSM_F16 && dtype != HCLSM_F32) return HCLSM_ERR_DTYPE;
  if (attn && attn_dtype != HCLSM_F32 && attn_dtype != dtype) return HCLSM_ERR_DTYPE;
  const int kpl = dtype == HCLSM_F32 ? 1 : 8;
  if (D % 16 || D % (4 * kpl)) return HCLSM_ERR_UNSUPPORTED;
  if (kpl == 8 && (!al16(q) || !al16(k) || ldq % 8 || ldk % 8 || q_bstride % 8 || k_bstride % 8))
    return HCLSM_ERR_UNSUPPORTED;
  CoreArgs a;
  a.ldq = ldq; a.ldk = ldk; a.ldv = ldv; a.ldo = ldo;
  a.qb = q_bstride; a.kb = k_bstride; a.vb = v_bstride; a.ob = o_bstride;
  a.N = (int)N; a.M = (int)M; a.D = (int)D;
  a.NP = (int)((N + 15) / 16 * 16);
  a.MP = (int)((M + 31) / 32 * 32);
  a.scale = scale; a.denom_eps = denom_eps; a.logit_clamp = logit_clamp; a.renorm_eps = renorm_eps;
  const int esize = dtype == HCLSM_F32 ? 4 : 2;
  const size_t smem = core_smem(a.NP, a.MP, a.D, esize);
  if (smem > 160 * 1024) return HCLSM_ERR_UNSUPPORTED;
  if (M == 0) return HCLSM_ERR_SHAPE;
  hipStream_t st = (hipStream_t)stream;
#define HCLSM_CORE(D_, A_)                                                                                  \
  if (dtype == D_ && (attn == nullptr ? A_ == D_ : attn_dtype == A_)) {                                     \
    if (smem > 64 * 1024)                                                                                   \
      hipFuncSetAttribute((const void*)slot_core_kernel<D_, A_>, hipFuncAttributeMaxDynamicSharedMemorySize, \
                          (int)smem);                                                                       \
    hipLaunchKernelGGL((slot_core_kernel<D_, A_>), dim3((unsigned)B), dim3(256), smem, st, (const MM<D_>::T*)q, \
                       (const MM<D_>::T*)k, (const MM<D_>::T*)v, (MM<D_>::T*)out, (MM<A_>::T*)attn, a);      \
    HCLSM_LAUNCH_CHECK();                                                                                   \
    return 0;                                                                                               \
  }
  HCLSM_CORE(HCLSM_BF16, HCLSM_BF16)
  HCLSM_CORE(HCLSM_BF16, HCLSM_F32)
  HCLSM_CORE(HCLSM_F16, HCLSM_F16)
  HCLSM_CORE(HCLSM_F16, HCLSM_F32)
  HCLSM_CORE(HCLSM_F32, HCLSM_F32)
#undef HCLSM_CORE
  return HCLSM_ERR_DTYPE;
}
