/*
 * hclsm_amd.h -- C ABI of libhclsm_amd.so, the MI355X (gfx950) hot path of
 * RightNow-AI/hclsm's hclsm/kernels package.
 *
 * Conventions shared by every entry point:
 *   - Pointers are device pointers (HBM), row-major and contiguous in the shapes
 *     stated per function.  Nullable pointers say so.
 *   - Sizes are int64_t element counts.
 *   - `stream` is a hipStream_t passed as void* (NULL = the default stream).
 *     Every call is asynchronous on that stream; nothing here synchronises the
 *     device, allocates or frees memory, or keeps per-call host state, so calls
 *     are re-entrant across host threads and streams.
 *   - Return value: 0 on success; a positive hipError_t from the launch; or a
 *     negative HCLSM_ERR_* code for an argument the library rejects before any
 *     launch.  hclsm_strerror() names both kinds.
 *   - The reference (RightNow-AI/hclsm) is Python/Triton with no C ABI; each
 *     entry point cites the reference function whose behaviour it replaces.
 */
#ifndef HCLSM_AMD_H
#define HCLSM_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HCLSM_ABI_VERSION 1

/* element types of floating-point tensors */
#define HCLSM_F32  0
#define HCLSM_BF16 1
#define HCLSM_F16  2

/* SSM scan clamp modes */
#define HCLSM_SCAN_RAW   0  /* A=-exp(A_log), no clamps: ssm_scan_kernel.py:191, :255 */
#define HCLSM_SCAN_MODEL 1  /* clamps of ssm_scan_kernel.py:63,68,77 and level0_ssm.py:76,82,96 */

/* argument errors (negative) */
#define HCLSM_ERR_NULL        (-1) /* a required pointer is NULL */
#define HCLSM_ERR_SHAPE       (-2) /* a size is negative, zero where not allowed, or too large */
#define HCLSM_ERR_DTYPE       (-3) /* unknown element-type code */
#define HCLSM_ERR_UNSUPPORTED (-4) /* valid but not implemented (e.g. d_state > 64) */
#define HCLSM_ERR_MODE        (-5) /* unknown mode code */

/* Version of this ABI (HCLSM_ABI_VERSION of the built library). */
int hclsm_abi_version(void);

/* Static string for a return code of any entry point. */
const char* hclsm_strerror(int code);

/*
 * Selective SSM scan, forward.
 *   h_t[d,s] = exp(dt_t[d]*A[d,s]) * h_{t-1}[d,s] + dt_t[d]*B_t[s]*x_t[d],  h_{-1} = 0
 *   y_t[d]   = sum_s C_t[s]*h_t[d,s]  (+ Dskip[d]*x_t[d] when Dskip != NULL)
 * with A = -exp(A_log) (RAW) or the clamped model form (MODEL).
 *   x, dt, y : [batch, T, d_inner]   element type `dtype`
 *   B, C     : [batch, T, d_state]   element type `dtype`
 *   A_log    : [d_inner, d_state]    float32
 *   Dskip    : [d_inner]             float32, nullable
 *   h_final  : [batch, d_inner, d_state] float32, nullable (state after the last step)
 * State and arithmetic are float32; 1 <= d_state <= 64.
 * Replaces: ssm_scan_fn / fused_ssm_scan_triton / _TritonSSMScan.forward
 *   (hclsm/kernels/ssm_scan_kernel.py:394-421, :379-387, :294-319) in RAW mode and
 *   sequential_ssm_scan (ssm_scan_kernel.py:42-86) in MODEL mode.
 */
int hclsm_ssm_scan_fwd(const void* x, const void* dt, const float* A_log,
                       const void* B, const void* C, const float* Dskip,
                       void* y, float* h_final,
                       int64_t batch, int64_t T, int64_t d_inner, int64_t d_state,
                       int dtype, int mode, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HCLSM_AMD_H */
