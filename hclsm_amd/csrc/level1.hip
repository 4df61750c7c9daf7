// Level-1 event dynamics on packed events, for gfx950.
//
// Level1EventDynamics.forward (hclsm/dynamics/level1_event.py:57-133) for the live events of a packed
// layout: event e < *n_events is rows e*N .. e*N+N-1 (its N slots).  Every launch is sized for the
// capacity and reads the live count on the device, so nothing here waits on the host:
//
//   x   = ev . proj_in^T                                  (fp32 residual stream)        :102-107
//   per layer (EventTransformerBlock, :31-54):
//     xn  = LN1(x)                                        (operand dtype)
//     qkv = xn . in_proj^T
//     o   = softmax(q k^T / sqrt(dh), keys of dead slots excluded) v, per event and head   :49-51
//           (16-bit, 32 slots, 64-wide heads: both in one launch, q / k / v kept on chip: qkv_attn_rows)
//     x  += o . out_proj^T                                (residual in the GEMM epilogue)
//     xn  = LN2(x)
//     g   = silu(xn . w1^T) * (xn . w3^T)                 (one GEMM over interleaved w1 / w3 rows whose
//                                                          epilogue pairs the products)                   :17-28
//     x  += g . w2^T
//   out = LN(x) . proj_out^T                                                                 :124-128
//
// 16-bit with the caller's folded weights (fold): the out-projection also writes x in dtype and x's LayerNorm
// partials per 64 columns (linear_stats_rows), and the SwiGLU input takes LN2 from them through
// w1 diag(gamma2), w3 diag(gamma2), their row sums and w1 beta2 | w3 beta2 (linear_fold_rows): no LN2 launch.  W2
// does the same for the next layer's LN1 (folded into the fused QKV attention, where it applies) and, in the last
// layer, for the final LayerNorm, folded into proj_out.
//
// GEMMs are the MFMA linear kernels of slot_attn.hip (64x64 LDS-staged tiles for 16-bit operands at
// these sizes), LayerNorm its one-wave-per-row kernel, the attention the uniform-segment mode of the
// varlen event-attention kernel (event_attn.hip).  The reference's event_pad_mask multiply (:130-131)
// has nothing to do here: packed rows are all real events.
#include "internal.h"

namespace hclsm {

struct L1Ws {
  size_t x, xn, qkv, o, h1, g, st, total;
};

static size_t al256(size_t v) { return (v + 255) / 256 * 256; }
static bool al16(const void* p) { return (((uintptr_t)p) & 15) == 0; }

static L1Ws l1_ws(int64_t cap, int64_t N, int64_t dm, int64_t hid, int es) {
  const size_t R = (size_t)cap * N;
  L1Ws w;
  size_t o = 0;
  w.x = o; o += al256(R * dm * 4);
  w.xn = o; o += al256(R * dm * es);
  w.qkv = o; o += al256(R * 3 * dm * es);
  w.o = o; o += al256(R * dm * es);
  w.h1 = o; o += al256(R * hid * es);
  w.g = o; o += al256(R * hid * es);
  w.st = o; o += al256(R * ((dm + 63) / 64) * 8);   // LayerNorm partials of x's rows (folded LayerNorms)
  w.total = o;
  return w;
}

}  // namespace hclsm

using namespace hclsm;

extern "C" int64_t hclsm_level1_forward_workspace(int64_t capacity, int64_t N, int64_t d_model, int64_t hidden,
                                                  int dtype) {
  if (capacity < 0 || N < 0 || d_model < 0 || hidden < 0) return HCLSM_ERR_SHAPE;
  if (dtype != HCLSM_F32 && dtype != HCLSM_BF16 && dtype != HCLSM_F16) return HCLSM_ERR_DTYPE;
  return (int64_t)l1_ws(capacity, N, d_model, hidden, dtype == HCLSM_F32 ? 4 : 2).total;
}

extern "C" int hclsm_level1_forward(const void* ev, int ev_dtype, void* out, int out_dtype, const int32_t* n_events,
                                    int64_t capacity, int64_t N, const int32_t* ev_rows, const float* obj_mask,
                                    int64_t d_slot, int64_t d_model, int64_t n_heads, int64_t hidden,
                                    int64_t n_layers, const void* const* params, const void* const* fold,
                                    float ln_eps, int dtype, void* workspace, int64_t workspace_bytes,
                                    void* stream) {
  if (capacity < 0 || N < 0 || d_slot <= 0 || d_model <= 0 || n_heads <= 0 || hidden <= 0 || n_layers < 0)
    return HCLSM_ERR_SHAPE;
  if (capacity * N > 0x7fffffffLL || d_model % n_heads) return HCLSM_ERR_SHAPE;
  if (dtype != HCLSM_F32 && dtype != HCLSM_BF16 && dtype != HCLSM_F16) return HCLSM_ERR_DTYPE;
  if ((ev_dtype != HCLSM_F32 && ev_dtype != dtype) || (out_dtype != HCLSM_F32 && out_dtype != dtype))
    return HCLSM_ERR_DTYPE;
  const int64_t dh = d_model / n_heads;
  if (dh != 16 && dh != 32 && dh != 64 && dh != 128) return HCLSM_ERR_UNSUPPORTED;
  const int64_t kmul = dtype == HCLSM_F32 ? 4 : 32;   // GEMM contraction granule of the linear kernels
  if (d_slot % kmul || d_model % kmul || hidden % kmul) return HCLSM_ERR_UNSUPPORTED;
  if (capacity == 0 || N == 0) return 0;
  if (!ev || !out || !n_events || !params || !workspace || (obj_mask && !ev_rows)) return HCLSM_ERR_NULL;
  const int es = dtype == HCLSM_F32 ? 4 : 2;
  const L1Ws L = l1_ws(capacity, N, d_model, hidden, es);
  if (workspace_bytes < (int64_t)L.total) return HCLSM_ERR_SHAPE;
  for (int64_t i = 0; i < 4 + 9 * n_layers; ++i)
    if (params[i] == nullptr) return HCLSM_ERR_NULL;
  // the LayerNorms before the SwiGLU inputs and proj_out folded into those layers' weights: 16-bit, the
  // out-projection and the last W2 writing x's LayerNorm partials (d_model a multiple of 64)
  // (shapes or alignments the fold's kernels do not take: the LayerNorm launches instead)
  bool folded = fold != nullptr && dtype != HCLSM_F32 && d_model % 64 == 0 && d_model <= 64 * FOLD_MAX_PARTS &&
                hidden % 64 == 0 && d_slot % 4 == 0 && n_layers > 0;
  if (fold != nullptr && dtype != HCLSM_F32)
    for (int64_t i = 0; i < 3 + 7 * n_layers; ++i) {
      if (fold[i] == nullptr) return HCLSM_ERR_NULL;
      folded = folded && al16(fold[i]);
    }
  for (int64_t l = 0; folded && l < n_layers; ++l) folded = al16(params[4 + 9 * l + 3]) && al16(params[4 + 9 * l + 8]);
  hipStream_t st = (hipStream_t)stream;
  char* ws = reinterpret_cast<char*>(workspace);
  float* x = reinterpret_cast<float*>(ws + L.x);
  void* xn = ws + L.xn;
  char* qkv = ws + L.qkv;
  void* o = ws + L.o;
  void* h1 = ws + L.h1;
  void* g = ws + L.g;
  void* st_part = ws + L.st;
  const int64_t R = capacity * N, dm = d_model;
  auto P = [&](int64_t i) { return params[i]; };
  auto Pf = [&](int64_t i) { return reinterpret_cast<const float*>(params[i]); };
  int rc;
#define HCLSM_TRY(call) \
  do {                  \
    rc = (call);        \
    if (rc) return rc;  \
  } while (0)
  // GEMM Y[R, n] = X[R, k] . W^T (+ resid) (gated by glu), rows of the live events only
  auto gemm = [&](const void* X, int xdt, const void* W, int64_t n, int64_t k, const float* resid, void* Y, int ydt,
                  const void* glu) {
    return linear_rows(X, k, xdt, W, k, nullptr, resid, n, Y, n, ydt, R, n, k, 0, 0, nullptr, nullptr, ln_eps, glu, n,
                       n_events, N, dtype, st);
  };
  auto norm = [&](const float* w, const float* b) {
    return layer_norm_rows(x, dm, w, b, xn, dm, R, dm, ln_eps, HCLSM_F32, dtype, n_events, N, st);
  };
  HCLSM_TRY(gemm(ev, ev_dtype, P(0), dm, d_slot, nullptr, x, HCLSM_F32, nullptr));   // x = ev . proj_in^T
  const float scale = 1.f / sqrtf((float)dh);
  // with the fold, LN1 of layers after the first is folded into the fused QKV attention (from the previous W2's
  // partials) where that launch applies (the shapes qkv_attn_rows takes: 32 slots, 64-wide heads, d_model = 64 H)
  const bool qkv_fold = folded && N == 32 && dh == 64 && dm == 64 * n_heads && al16(xn);
  for (int64_t l = 0; l < n_layers; ++l) {
    const int64_t b = 4 + 9 * l;   // ln1_w, ln1_b, in_proj, out_proj, ln2_w, ln2_b, w1, w3, w2
    const int64_t f = 3 + 7 * l;   // fold: in_proj diag(g1), its row sums, in_proj b1, w1 / w3 diag(g2), sums, biases
    if (qkv_fold && l > 0) {
      // xn holds x in dtype and st_part its partials (the previous layer's W2)
      HCLSM_TRY(qkv_attn_rows(xn, fold[f], o, n_events, capacity, N, dm, (int)n_heads, (int)dh, obj_mask, ev_rows,
                              scale, dtype, st, reinterpret_cast<const float*>(fold[f + 1]),
                              reinterpret_cast<const float*>(fold[f + 2]), st_part, dm / 64, ln_eps));
      rc = 0;
    } else {
      HCLSM_TRY(norm(Pf(b), Pf(b + 1)));
      // o = attention over q | k | v = xn . in_proj^T: one fused launch (q / k / v stay on chip) where it applies
      rc = qkv_attn_rows(xn, P(b + 2), o, n_events, capacity, N, dm, (int)n_heads, (int)dh, obj_mask, ev_rows, scale,
                         dtype, st);
    }
    if (rc == HCLSM_ERR_UNSUPPORTED) {
      HCLSM_TRY(gemm(xn, dtype, P(b + 2), 3 * dm, dm, nullptr, qkv, dtype, nullptr));
      HCLSM_TRY(attn_slots_packed(qkv, qkv + dm * es, qkv + 2 * dm * es, 3 * dm, o, dm, n_events, capacity, N,
                                  (int)n_heads, (int)dh, obj_mask, ev_rows, scale, dtype, st));
    } else if (rc) {
      return rc;
    }
    if (folded) {
      // x += o . out_proj^T, x also in dtype (into xn) with its LayerNorm partials; g = SwiGLU(LN2 x) with LN2
      // folded into w1 / w3: fold[f + 3 ..] = w1 diag(g2), w3 diag(g2), their row sums, w1 b2 | w3 b2
      HCLSM_TRY(linear_stats_rows(o, dm, P(b + 3), dm, x, dm, x, dm, xn, dm, st_part, R, dm, dm, n_events, N, dtype,
                                  st));
      HCLSM_TRY(linear_fold_rows(xn, dm, fold[f + 3], fold[f + 4], dm, reinterpret_cast<const float*>(fold[f + 5]),
                                 reinterpret_cast<const float*>(fold[f + 6]), st_part, dm / 64, ln_eps, g, hidden,
                                 dtype, R, 2 * hidden, dm, n_events, N, dtype, st));
      if (l + 1 < n_layers && !qkv_fold) {
        HCLSM_TRY(gemm(g, dtype, P(b + 8), dm, hidden, x, x, HCLSM_F32, nullptr));
      } else {   // W2 also writes the partials of the next LayerNorm: the next layer's LN1 or the final one
        HCLSM_TRY(linear_stats_rows(g, hidden, P(b + 8), hidden, x, dm, x, dm, xn, dm, st_part, R, dm, hidden,
                                    n_events, N, dtype, st));
      }
      continue;
    }
    HCLSM_TRY(gemm(o, dtype, P(b + 3), dm, dm, x, x, HCLSM_F32, nullptr));
    HCLSM_TRY(norm(Pf(b + 4), Pf(b + 5)));
    // g = silu(xn . w1^T) * (xn . w3^T): one paired GEMM, or two GEMMs through h1 where it does not apply
    rc = linear_glu_rows(xn, dm, dtype, P(b + 6), P(b + 7), dm, g, hidden, dtype, R, hidden, dm, n_events, N, dtype,
                         st);
    if (rc == HCLSM_ERR_UNSUPPORTED) {
      HCLSM_TRY(gemm(xn, dtype, P(b + 6), hidden, dm, nullptr, h1, dtype, nullptr));
      HCLSM_TRY(gemm(xn, dtype, P(b + 7), hidden, dm, nullptr, g, dtype, h1));
    } else if (rc) {
      return rc;
    }
    HCLSM_TRY(gemm(g, dtype, P(b + 8), dm, hidden, x, x, HCLSM_F32, nullptr));
  }
  if (folded) {   // out = LN(x) . proj_out^T with the LayerNorm folded: fold[0 ..] = proj_out diag(g), sums, proj_out b
    HCLSM_TRY(linear_fold_rows(xn, dm, fold[0], nullptr, dm, reinterpret_cast<const float*>(fold[1]),
                               reinterpret_cast<const float*>(fold[2]), st_part, dm / 64, ln_eps, out, d_slot,
                               out_dtype, R, d_slot, dm, n_events, N, dtype, st));
    return 0;
  }
  HCLSM_TRY(norm(Pf(1), Pf(2)));
  HCLSM_TRY(gemm(xn, dtype, P(3), d_slot, dm, nullptr, out, out_dtype, nullptr));   // out = LN(x) . proj_out^T
#undef HCLSM_TRY
  return 0;
}
