// Launchers shared between the translation units of libhclsm_amd (not part of the C ABI).
#pragma once

#include "common.h"

namespace hclsm {

// Event rule of mask element i (mask dtype mdt: F32 / BF16 / F16 / U8): GT_HALF is v > 0.5, NONZERO
// v != 0 (NaN counts, as torch.nonzero); U8 masks: any nonzero byte.
__device__ __forceinline__ bool is_event(const void* mask, int mdt, int64_t i, int rule) {
  float v;
  switch (mdt) {
    case HCLSM_F32: v = reinterpret_cast<const float*>(mask)[i]; break;
    case HCLSM_BF16: v = bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(mask)[i]); break;
    case HCLSM_F16: v = (float)reinterpret_cast<const _Float16*>(mask)[i]; break;
    default: return reinterpret_cast<const uint8_t*>(mask)[i] != 0;
  }
  if (rule == HCLSM_EVENT_GT_HALF) return v > 0.5f;
  return !(v == 0.0f);  // NaN counts as an event, like torch.nonzero
}

// Event flags of U blocks of 64 steps of mask row `row` (step t0 + 64u + lane of block u; steps past T are not
// events), by the rule of is_event.  Every load is issued before any flag is formed, so a row of up to 64 U
// steps costs one memory round trip instead of one per block.
template <int U>
__device__ __forceinline__ void mask_events(const void* mask, int mdt, int64_t row, int64_t T, int64_t t0, int lane,
                                            int rule, bool* ev) {
  float v[U];
  const int64_t base = row * T;
  switch (mdt) {
    case HCLSM_F32: {
      const float* m = reinterpret_cast<const float*>(mask) + base;
#pragma unroll
      for (int u = 0; u < U; ++u) { const int64_t t = t0 + 64 * u + lane; v[u] = t < T ? m[t] : 0.f; }
      break;
    }
    case HCLSM_BF16: {
      const uint16_t* m = reinterpret_cast<const uint16_t*>(mask) + base;
#pragma unroll
      for (int u = 0; u < U; ++u) { const int64_t t = t0 + 64 * u + lane; v[u] = t < T ? bf16_bits_to_f32(m[t]) : 0.f; }
      break;
    }
    case HCLSM_F16: {
      const _Float16* m = reinterpret_cast<const _Float16*>(mask) + base;
#pragma unroll
      for (int u = 0; u < U; ++u) { const int64_t t = t0 + 64 * u + lane; v[u] = t < T ? (float)m[t] : 0.f; }
      break;
    }
    default: {   // U8: any nonzero byte is an event, whatever the rule
      const uint8_t* m = reinterpret_cast<const uint8_t*>(mask) + base;
#pragma unroll
      for (int u = 0; u < U; ++u) { const int64_t t = t0 + 64 * u + lane; v[u] = (t < T && m[t] != 0) ? 1.f : 0.f; }
      break;
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const bool in = t0 + 64 * u + lane < T;
    ev[u] = in && (rule == HCLSM_EVENT_GT_HALF && mdt != HCLSM_U8 ? v[u] > 0.5f : !(v[u] == 0.0f));
  }
}
constexpr int MASK_BLOCKS = 16;   // blocks of 64 steps per mask_events call in the index kernels


// Y[M, N] = A . W^T (+ bias) (ReLU if relu) (+ resid) with A = X or LayerNorm(X) rows (ln != 0), the
// row count taken as min(M, *m_dev * m_mul) when m_dev is set (read on the device), and, when glu is
// set, the gated-linear epilogue val = silu(glu[row, col]) * val (glu in `dtype`, row stride ldg) before
// the residual.  Defined in slot_attn.hip.
int linear_rows(const void* x, int64_t ldx, int x_dtype, const void* w, int64_t ldw, const float* bias,
                const float* resid, int64_t ldr, void* y, int64_t ldy, int y_dtype, int64_t M, int64_t N, int64_t K,
                int ln, int relu, const float* ln_w, const float* ln_b, float ln_eps, const void* glu, int64_t ldg,
                const int32_t* m_dev, int64_t m_mul, int dtype, hipStream_t st);

// SwiGLU input layer Y[M, H] = silu(X . w1^T) * (X . w3^T) (w1, w3 [H, K] with row stride ldw) as one GEMM
// whose epilogue pairs the two products; row count as linear_rows.  HCLSM_ERR_UNSUPPORTED for shapes it does not
// take (H % 16; K % 32 for 16-bit operands, K % 4 for fp32; 16-byte alignment), where the caller runs two GEMMs.
// Defined in slot_attn.hip.
int linear_glu_rows(const void* x, int64_t ldx, int x_dtype, const void* w1, const void* w3, int64_t ldw, void* y,
                    int64_t ldy, int y_dtype, int64_t M, int64_t H, int64_t K, const int32_t* m_dev, int64_t m_mul,
                    int dtype, hipStream_t st);

// Y[M, N] (fp32) = X . W^T + resid for 16-bit X, also writing Y rounded to dtype into y2 and, per row and 64-column
// block b, the LayerNorm partial pst[row * N / 64 + b] = (mean, centred sum of squares) as float2 (device row count
// as linear_rows, required).  HCLSM_ERR_UNSUPPORTED unless K % 64 == 0, N % 64 == 0 and 16-byte alignment.
// Defined in slot_attn.hip.
int linear_stats_rows(const void* x, int64_t ldx, const void* w, int64_t ldw, const float* resid, int64_t ldr,
                      float* y, int64_t ldy, void* y2, int64_t ldy2, void* pst, int64_t M, int64_t N, int64_t K,
                      const int32_t* m_dev, int64_t m_mul, int dtype, hipStream_t st);

// Most 64-column LayerNorm partials a folded row may have (rows of up to 1024 columns): linear_fold_rows and
// qkv_attn_rows refuse more (HCLSM_ERR_UNSUPPORTED).
constexpr int FOLD_MAX_PARTS = 16;

// Y = LN(X) . W0^T for the rows of a linear_stats_rows output: x its 16-bit copy, fst its partials (fparts per row),
// w = W0 diag(gamma) in dtype, fsum[j] = sum of row j of w (fp32), fbias[j] = (W0 beta)[j]; the output is
// rstd (x w^T - mean fsum) + fbias.  With w3 (rows of W0 diag(gamma) for the gate's second factor, N = 2 H):
// Y[M, H] = silu(h1) * h3 with fsum / fbias holding the w columns, then the w3 columns.  HCLSM_ERR_UNSUPPORTED
// unless 16-bit, K % 32 == 0, N % 4 == 0 (% 32 with w3) and 16-byte alignment.  Defined in slot_attn.hip.
int linear_fold_rows(const void* x, int64_t ldx, const void* w, const void* w3, int64_t ldw, const float* fsum,
                     const float* fbias, const void* fst, int64_t fparts, float eps, void* y, int64_t ldy, int y_dtype,
                     int64_t M, int64_t N, int64_t K, const int32_t* m_dev, int64_t m_mul, int dtype, hipStream_t st);

// LayerNorm of M rows (row count min(M, *m_dev * m_mul) when m_dev is set), as hclsm_layer_norm.
// Defined in slot_attn.hip.
int layer_norm_rows(const void* x, int64_t ldx, const float* w, const float* b, void* y, int64_t ldy, int64_t M,
                    int64_t D, float eps, int in_dtype, int out_dtype, const int32_t* m_dev, int64_t m_mul,
                    hipStream_t st);

// event_count_kernel over a [B, T] mask: counts[b] = events of row b (events.hip).
int event_counts(const void* mask, int mdt, int64_t B, int64_t T, int rule, int32_t* counts, hipStream_t st);

// Attention among the N rows of each of cap uniform segments (the first *nseg_dev live): rows p*N + i
// of q / k / v (row stride ldi) and out (row stride ldo), H heads of dh columns; key j of segment p is
// excluded when obj_mask[seg_rows[p] * N + j] <= 0.5 (obj_mask nullable).  Defined in event_attn.hip.
int attn_slots_packed(const void* q, const void* k, const void* v, int64_t ldi, void* out, int64_t ldo,
                      const int32_t* nseg_dev, int64_t cap, int64_t N, int H, int dh, const float* obj_mask,
                      const int32_t* seg_rows, float scale, int dtype, hipStream_t st);

// Level-1 QKV projection and slot attention in one launch: o[e*32 + i, h*64 ..] = attention of event e's 32 rows
// (head h, keys excluded as attn_slots_packed) over q | k | v = x . w^T (w = in_proj [3d, d], x / o row stride d),
// for the first *n_events of capacity events.  HCLSM_ERR_UNSUPPORTED unless 16-bit, N = 32, dh = 64, d = 64 H,
// 16-byte aligned x / w / o; the caller then runs the GEMM and attn_slots_packed.  Defined in slot_attn.hip.
// fst (nullable): x is the 16-bit copy of a linear_stats_rows output and LN1 is folded into w as in
// linear_fold_rows (fsum / fbias per in_proj row, fparts partials per row of x).
int qkv_attn_rows(const void* x, const void* w, void* o, const int32_t* n_events, int64_t capacity, int64_t N,
                  int64_t d, int H, int dh, const float* obj_mask, const int32_t* ev_rows, float scale, int dtype,
                  hipStream_t st, const float* fsum = nullptr, const float* fbias = nullptr,
                  const void* fst = nullptr, int64_t fparts = 0, float eps = 0.f);

// Forward scan that also writes the backward's checkpoint slab ck ([batch][ceil(T / 8)][16][d_inner] fp32, the
// state before steps 8, 16, ...; entry 0, the zero initial state, is not stored): the bf16, d_state 16
// matrix-core kernel; HCLSM_ERR_UNSUPPORTED elsewhere.
// mode: HCLSM_SCAN_RAW / _MODEL, or HCLSM_SCAN_BLOCK with gate (and optional y_pre).  Defined in ssm_scan.hip.
int scan_fwd_ckpt(int mode, const void* x, const void* dt, const float* A_log, const void* B, const void* C,
                  const float* Dskip, void* y, float* h_final, int64_t batch, int64_t T, int64_t Dn, int64_t S,
                  int dtype, const void* gate, void* y_pre, float* ck, hipStream_t st);

}  // namespace hclsm

#include <atomic>

namespace hclsm {

constexpr int HCLSM_MAX_DEVICES = 64;

// Once per device and call site: raise the kernel's dynamic-LDS limit to max_lds (when max_lds > 0) and find how
// many workgroups of `threads` threads using `lds` bytes the device holds at once (multiprocessors x occupancy).
// cache: the call site's per-device slots (0 = not set up).  *grid gets the count.  Defined in launch.hip.
int device_launch_setup(const void* fn, int threads, size_t lds, int max_lds, std::atomic<int>* cache, int* grid);
// Compute units of the current device (cached per device).  Defined in launch.hip.
int device_cus(int* cus);

}  // namespace hclsm
