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

/* 2: HclsmSlotWeights gained w_qkv (a caller built against version 1 passes a shorter struct and must be rebuilt)
 * 3: HclsmSlotWeights gained w1_n, w1_n_sum, w1_n_bias (the same holds for a caller built against version 2), and
 *    hclsm_level1_forward the fold argument */
#define HCLSM_ABI_VERSION 3

/* element types of floating-point tensors */
#define HCLSM_F32  0
#define HCLSM_BF16 1
#define HCLSM_F16  2
#define HCLSM_U8   3  /* event masks only: bool / uint8 */

/* event rules for masks */
#define HCLSM_EVENT_GT_HALF 0 /* mask > 0.5: hierarchy_manager.py:61, sparse_event_attn.py:124 */
#define HCLSM_EVENT_NONZERO 1 /* mask != 0 (NaN is an event): sparse_event_attn.py:65 */

/* event attention modes */
#define HCLSM_ATTN_TRACK_CAUSAL 0 /* causal over the events of one track (benchmark configs 3/4) */
#define HCLSM_ATTN_SLOTS        1 /* all rows of a segment, key padding (level1_event.py:37-52) */

/* SSM scan clamp modes */
#define HCLSM_SCAN_RAW   0  /* A=-exp(A_log), no clamps: ssm_scan_kernel.py:191, :255 */
#define HCLSM_SCAN_MODEL 1  /* clamps of ssm_scan_kernel.py:63,68,77 and level0_ssm.py:76,82,96 */
#define HCLSM_SCAN_BLOCK 2  /* hclsm_ssm_scan_bwd only: MODEL with dt = clamp(softplus(dt input), 1e-3, 1) inside
                               the kernel, as hclsm_ssm_block_scan_fwd computes it (level0_ssm.py:76) */

/* argument errors (negative) */
#define HCLSM_ERR_NULL        (-1) /* a required pointer is NULL */
#define HCLSM_ERR_SHAPE       (-2) /* a size is negative, zero where not allowed, or too large */
#define HCLSM_ERR_DTYPE       (-3) /* unknown element-type code */
#define HCLSM_ERR_UNSUPPORTED (-4) /* valid but not implemented (e.g. d_state > 128) */
#define HCLSM_ERR_MODE        (-5) /* unknown mode code */
#define HCLSM_ERR_SCRATCH     (-6) /* the call needs more than an allocation-free entry point's static scratch */

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
 * State and arithmetic are float32; 1 <= d_state <= 128.
 * Replaces: ssm_scan_fn / fused_ssm_scan_triton / _TritonSSMScan.forward
 *   (hclsm/kernels/ssm_scan_kernel.py:394-421, :379-387, :294-319) in RAW mode and
 *   sequential_ssm_scan (ssm_scan_kernel.py:42-86) in MODEL mode.
 */
int hclsm_ssm_scan_fwd(const void* x, const void* dt, const float* A_log,
                       const void* B, const void* C, const float* Dskip,
                       void* y, float* h_final,
                       int64_t batch, int64_t T, int64_t d_inner, int64_t d_state,
                       int dtype, int mode, void* stream);

/*
 * The scan of SimplifiedSSMBlock with its elementwise epilogues fused
 * (hclsm/dynamics/level0_ssm.py:72-103):
 *   dt    = clamp(softplus(dt_in), 1e-3, 1)           (:76, softplus threshold 20 as in torch)
 *   y_pre = clamped selective scan of z with dt, A_log, B, C   (MODEL mode, :82-101)
 *   y     = y_pre * silu(gate)                        (:73, :103)
 * z, dt_in, gate, y, y_pre: [batch][T][d_inner] in `dtype`; B, C: [batch][T][d_state]; A_log fp32.
 * y_pre (kept for the backward) and h_final are nullable.  No skip term.
 * Replaces: the softplus / clamp of dt, the inline scan, F.silu(gate) and the gating product of
 *   SimplifiedSSMBlock.forward.
 */
int hclsm_ssm_block_scan_fwd(const void* z, const void* dt_in, const float* A_log, const void* B,
                             const void* C, const void* gate, void* y, void* y_pre, float* h_final,
                             int64_t batch, int64_t T, int64_t d_inner, int64_t d_state, int dtype,
                             void* stream);

/* Workspace bytes for hclsm_ssm_scan_bwd. */
int64_t hclsm_ssm_scan_bwd_workspace(int64_t batch, int64_t T, int64_t d_inner, int64_t d_state);

/*
 * Selective SSM scan, backward: gradients of sum(gy * y) for the forward of hclsm_ssm_scan_fwd with the
 * same arguments and mode.  gy, gx, gdt [batch, T, d_inner] and gB, gC [batch, T, d_state] in `dtype`;
 * gA_log [d_inner, d_state] float32; gD [d_inner] float32 (nullable; Dskip nullable as in the forward).
 * MODEL mode passes gradient through each clamp only inside its closed interval.  BLOCK mode takes the
 * block's dt input (before softplus) as `dt`, recomputes dt = clamp(softplus(dt), 1e-3, 1) in fp32 exactly as
 * the fused block forward does, and returns in gdt the gradient with respect to that input (through the clamp,
 * closed interval, and softplus).  Chunk checkpoints and
 * partial sums live in `workspace` (>= hclsm_ssm_scan_bwd_workspace bytes).  Two launches.
 * Deterministic (no float atomics).  One sequence's [T, d_inner] slab must be < 2^31 bytes
 * (HCLSM_ERR_UNSUPPORTED otherwise).
 * Replaces: _TritonSSMScan.backward (hclsm/kernels/ssm_scan_kernel.py:321-377) and the autograd of
 *   sequential_ssm_scan (:42-86) / the inline scan of SimplifiedSSMBlock (dynamics/level0_ssm.py:82-101).
 */
int hclsm_ssm_scan_bwd(const void* x, const void* dt, const float* A_log, const void* B, const void* C,
                       const float* Dskip, const void* gy, void* gx, void* gdt, float* gA_log, void* gB,
                       void* gC, float* gD, int64_t batch, int64_t T, int64_t d_inner, int64_t d_state,
                       int dtype, int mode, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Training pair: a forward that also leaves the backward's chunk checkpoints in `workspace`, and a backward
 * that starts from them instead of recomputing them (its first pass).  bf16 I/O with d_state 16 only (the
 * matrix-core forward); HCLSM_ERR_UNSUPPORTED otherwise, and the caller uses the plain pair.
 *   hclsm_ssm_scan_fwd_ckpt:       hclsm_ssm_scan_fwd's arguments (RAW or MODEL) plus the backward workspace
 *                                  (>= hclsm_ssm_scan_bwd_workspace bytes); y and h_final as hclsm_ssm_scan_fwd.
 *   hclsm_ssm_block_scan_fwd_ckpt: the same for hclsm_ssm_block_scan_fwd (its backward runs in BLOCK mode).
 *   hclsm_ssm_scan_bwd_ckpt:       hclsm_ssm_scan_bwd's arguments; `workspace` must hold the checkpoints a
 *                                  *_fwd_ckpt call wrote for the same inputs and mode, unmodified since.
 * The gradients equal hclsm_ssm_scan_bwd's within fp32 rounding of the recomputed states.
 * Replaces: the saved-for-backward split of _TritonSSMScan (hclsm/kernels/ssm_scan_kernel.py:294-377); the
 *   reference's forward saves its inputs, this one also saves the states the backward restarts from.
 */
int hclsm_ssm_scan_fwd_ckpt(const void* x, const void* dt, const float* A_log, const void* B, const void* C,
                            const float* Dskip, void* y, float* h_final, int64_t batch, int64_t T,
                            int64_t d_inner, int64_t d_state, int dtype, int mode, void* workspace,
                            int64_t workspace_bytes, void* stream);
int hclsm_ssm_block_scan_fwd_ckpt(const void* z, const void* dt_in, const float* A_log, const void* B,
                                  const void* C, const void* gate, void* y, void* y_pre, float* h_final,
                                  int64_t batch, int64_t T, int64_t d_inner, int64_t d_state, int dtype,
                                  void* workspace, int64_t workspace_bytes, void* stream);
int hclsm_ssm_scan_bwd_ckpt(const void* x, const void* dt, const float* A_log, const void* B, const void* C,
                            const float* Dskip, const void* gy, void* gx, void* gdt, float* gA_log, void* gB,
                            void* gC, float* gD, int64_t batch, int64_t T, int64_t d_inner, int64_t d_state,
                            int dtype, int mode, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Event index of a [B, T] mask, built on the device with no host synchronisation.
 *   counts  [B]      int32  events per row
 *   offsets [B+1]    int32  exclusive prefix sum of counts; offsets[B] = total
 *   indices [B*T]    int32  capacity; first `total` hold the event timesteps, ascending
 *                           within each row, rows concatenated
 *   rows    [B*T]    int32  capacity, nullable; rows[e] = row of packed event e
 *   slot_of [B, T]   int32  nullable; rank of t among row b's events, or -1
 *   stats   [2]      int32  {total, max count}
 * mask_dtype: HCLSM_F32 / BF16 / F16 / U8; rule: HCLSM_EVENT_GT_HALF / NONZERO (U8 masks: any nonzero).
 * Replaces the index construction of HierarchyManager.gather_events (hierarchy_manager.py:59-67),
 *   _vectorized_gather (sparse_event_attn.py:104-120) and the nonzero loop of
 *   naive_sparse_event_attention (sparse_event_attn.py:64-70), and removes their .item() syncs
 *   (hierarchy_manager.py:63, sparse_event_attn.py:56,173).
 */
int hclsm_event_index(const void* mask, int mask_dtype, int64_t B, int64_t T, int rule,
                      int32_t* counts, int32_t* offsets, int32_t* indices, int32_t* rows,
                      int32_t* slot_of, int32_t* stats, void* stream);

/*
 * Padded gather: dst[b, k, :] = src[b, indices[offsets[b]+k], :] for k < counts[b], zero bytes for
 * counts[b] <= k < K.  src [B, T, row_bytes], dst [B, K, row_bytes]; any element type (byte copy).
 * Replaces the gathers of HierarchyManager.gather_events (hierarchy_manager.py:69-75),
 *   _vectorized_gather (sparse_event_attn.py:121-128) and the naive loop (:64-70); never launched
 *   Triton _sparse_gather_kernel (:197-235).
 */
int hclsm_event_gather(const void* src, void* dst, int64_t row_bytes, int64_t B, int64_t T, int64_t K,
                       const int32_t* counts, const int32_t* offsets, const int32_t* indices,
                       void* stream);

/*
 * Packed gather: dst[e, :] = src[rows[e], indices[e], :] for e < min(stats[0], capacity); rows
 * beyond the device-side total are left untouched.  dst [capacity, row_bytes].
 * (No reference counterpart: the packed, sync-free layout of the event segments.)
 */
int hclsm_event_gather_packed(const void* src, void* dst, int64_t row_bytes, int64_t B, int64_t T,
                              int64_t capacity, const int32_t* rows, const int32_t* indices,
                              const int32_t* stats, void* stream);

/*
 * Padded scatter: out[b, t, :] = updates[b, s, :] where 0 <= s = slot_of[b, t] < K, else base[b, t, :].
 * base / updates may be NULL (read as zero bytes); out may alias base.
 * Replaces HierarchyManager.scatter_events (hierarchy_manager.py:79-118), _vectorized_scatter
 *   (sparse_event_attn.py:134-150) and the naive scatter loop (:78-84).
 */
int hclsm_event_scatter(const void* base, const void* updates, void* out, int64_t row_bytes,
                        int64_t B, int64_t T, int64_t K, const int32_t* slot_of, void* stream);

/*
 * Packed scatter: out[b, t, :] = packed[offsets[b] + s, :] where s = slot_of[b, t] >= 0, else base.
 * base / packed may be NULL (zeros); out may alias base.  (Packed counterpart of the above.)
 */
int hclsm_event_scatter_packed(const void* base, const void* packed, void* out, int64_t row_bytes,
                               int64_t B, int64_t T, const int32_t* offsets, const int32_t* slot_of,
                               void* stream);

/*
 * Hierarchy manager output step: HierarchyManager.forward (hierarchy_manager.py:120-162) after the
 * Level-1 pass, fused.  All states fp32, rows of D floats, 16-byte aligned:
 *   level0  [B, T, N, D]; events: the Level-1 rows, packed [capacity, N, D] at offsets[b] + slot_of[b, t]
 *   (kpad == 0) or padded [B, kpad, N, D] at slot_of[b, t] < kpad (kpad > 0; later events keep level0).
 *   combined = event row at events, level0 elsewhere (the scatter, :143).
 *   With level2_context [B, S2, DL2] (nullable):
 *     l2 = W_l2 mean_s(level2_context)   (W_l2 = l2_to_l1.weight [D, DL2], :147-152)
 *     gate = sigmoid(W_gate [combined; l2] + b_gate)   (W_gate [D, 2D], b_gate [D] nullable, :153-154)
 *     combined = gate * l2 + (1 - gate) * combined   (:155)
 *   the gate GEMM runs in `dtype` (f32 / bf16 / f16 operands, fp32 accumulation) on W_gate_x, a copy of
 *   W_gate[:, :D] in that type with row stride ldw (for f32 it may be W_gate itself, ldw = 2D); l2 and the
 *   Level-2 half of the gate are fp32.
 *   out = combined * obj_mask[b, n] (obj_mask [B, N] nullable, :159-160).  out may alias level0.
 * ws: hclsm_event_top_down_workspace(B, D) bytes, 16-byte aligned (needed with a level2_context).
 * D a multiple of 32 up to 384, DL2 up to 16384 (HCLSM_ERR_UNSUPPORTED otherwise).
 */
int64_t hclsm_event_top_down_workspace(int64_t B, int64_t D);
int hclsm_event_top_down(const float* level0, const float* events, const int32_t* offsets,
                         const int32_t* slot_of, int64_t kpad, const float* level2_context, int64_t S2,
                         int64_t DL2, const float* W_l2, const float* W_gate, const float* b_gate,
                         const void* W_gate_x, int64_t ldw, const float* obj_mask, float* out, int64_t B,
                         int64_t T, int64_t N, int64_t D, int dtype, void* ws, int64_t ws_bytes,
                         void* stream);

/*
 * Variable-length attention over event segments, on MFMA.
 *   q, k, v   [nseg, T, H, dh]  element type `dtype` (bf16 / f16 / f32), contiguous
 *   offsets   [nseg+1], indices [>= offsets[nseg]]  int32 (an event index: segment p is the rows
 *             (p, indices[offsets[p] + i]), i < offsets[p+1] - offsets[p], in that order)
 *   key_pad   [nseg, T] uint8, nullable; SLOTS mode ignores keys whose row is flagged nonzero
 *   out_packed [capacity, H, dh], nullable: row offsets[p] + i = output of query i of segment p
 *             (rows at or past `capacity` are not written)
 *   out_grid   [nseg, T, H, dh], nullable: output written at the query's own row; other rows untouched
 * mode TRACK_CAUSAL: query i attends keys j <= i; mode SLOTS: all unpadded keys of the segment.
 * softmax in fp32 with `scale` applied to q.k; dh in {16, 32, 64, 128}.  A query whose keys are all
 * padded produces NaN, as softmax over an all -inf row does in the reference.
 * Replaces: the attention core of nn.MultiheadAttention in EventTransformerBlock
 *   (dynamics/level1_event.py:37-52, SLOTS mode) and the per-track causal event attention of the
 *   benchmark configuration (TRACK_CAUSAL), fed by the event index instead of the padded
 *   gather of hierarchy_manager.py:42-77.
 */
int hclsm_event_attention(const void* q, const void* k, const void* v, void* out_packed, void* out_grid,
                          const int32_t* offsets, const int32_t* indices, const uint8_t* key_pad,
                          int64_t nseg, int64_t T, int64_t H, int64_t dh, int64_t capacity,
                          float scale, int dtype, int mode, void* stream);

/*
 * hclsm_event_index of a [B, T] mask followed by hclsm_event_attention in HCLSM_ATTN_TRACK_CAUSAL mode
 * with a packed output ([capacity, H, dh]), in one call on one stream.  `tables` is one int32 buffer
 * holding the index in this order: stats [2], counts [B], offsets [B+1], indices [max(B*T,1)],
 * rows [max(B*T,1)], slot_of [B*T]; it is left filled for later gathers and scatters.
 * Replaces: the index construction and attention of the per-track causal event attention of the
 *   benchmark configuration (sparse_event_attn.py:153-188, hierarchy_manager.py:42-77) as one host call.
 */
int hclsm_track_causal_attention(const void* mask, int mask_dtype, int rule, const void* q, const void* k,
                                 const void* v, void* out_packed, int64_t B, int64_t T, int64_t H, int64_t dh,
                                 int64_t capacity, float scale, int dtype, int32_t* tables, void* stream);

/*
 * LayerNorm over the last dimension of a [M, D] row-major tensor (row strides ldx / ldy):
 *   y = (x - mean) / sqrt(var + eps) * w + b, population variance, fp32 statistics.
 * w, b: [D] float32, nullable (then 1 / 0).  (in, out) dtype pairs: (F32,F32) (F32,BF16) (BF16,BF16)
 * (BF16,F32) (F32,F16) (F16,F16).
 * Replaces: nn.LayerNorm of DynamicSlotAttention (objects/dynamic_slots.py:72-73,111,128,152),
 *   SimplifiedSSMBlock (dynamics/level0_ssm.py:59,68) and EventTransformerBlock (level1_event.py:36,40).
 */
int hclsm_layer_norm(const void* x, int64_t ldx, const float* w, const float* b, void* y, int64_t ldy,
                     int64_t M, int64_t D, float eps, int in_dtype, int out_dtype, void* stream);

/*
 * Linear layer on MFMA: Y[M, N] = A[M, K] . W[N, K]^T (+ bias[N]) (ReLU if relu) (+ resid[M, N] fp32)
 *   (clamped to +-clamp if clamp > 0), where A = X, or A = LayerNorm(X) rows (ln != 0; ln_w / ln_b
 *   [K] float32 nullable, eps ln_eps) formed on the fly.  X: x_dtype (F32, or = dtype); W: `dtype`
 *   (BF16 / F16: 16-byte aligned rows, K % 32 == 0; F32: K % 4 == 0); Y: y_dtype (F32 or dtype);
 *   y2 (nullable): a second copy of Y in `dtype`.  Row strides in elements.  One workgroup per
 *   32x32 output tile, K split across its four waves.
 * Replaces: the nn.Linear layers (with their preceding nn.LayerNorm) of the slot iteration
 *   (objects/dynamic_slots.py:51-53,64-73,111-112,128,152-154).
 */
int hclsm_linear(const void* x, int64_t ldx, int x_dtype, const void* w, int64_t ldw, const float* bias,
                 const float* resid, int64_t ldr, void* y, int64_t ldy, int y_dtype, void* y2,
                 int64_t ldy2, int64_t M, int64_t N, int64_t K, int relu, float clamp, int ln,
                 const float* ln_w, const float* ln_b, float ln_eps, int dtype, void* stream);

/*
 * torch.nn.GRUCell on MFMA for M rows: x [M, Kx] and h (both as `dtype` hb [M, H] for the products
 * and as float32 h [M, H] for the blend), w_ih [3H, Kx], w_hh [3H, H] (`dtype`, rows [r; z; n]),
 * b_ih, b_hh [3H] float32 nullable.  out [M, H] float32 = (1 - z) * n + z * h; out2 (nullable) the
 * same in `dtype`.  Kx, H multiples of 32 (16-bit types) or 4 (F32).
 * Replaces: self.gru of DynamicSlotAttention._iteration_step (objects/dynamic_slots.py:55-60,123-126).
 */
int hclsm_gru_cell(const void* x, int64_t ldx, const void* hb, int64_t ldhb, const float* h, int64_t ldh,
                   const void* w_ih, const void* w_hh, const float* b_ih, const float* b_hh, float* out,
                   int64_t ldo, void* out2, int64_t ldo2, int64_t M, int64_t H, int64_t Kx, int dtype,
                   void* stream);

/*
 * Slot-attention core for B frames:
 *   logits = scale * q k^T (clamped to +-logit_clamp if logit_clamp > 0);
 *   attn = softmax over the N slots for each of the M tokens, denominator + denom_eps;
 *   if renorm_eps >= 0: attn = (attn + renorm_eps) / sum over tokens (attn + renorm_eps);
 *   out = attn v.
 * q [B][N][D], k, v [B][M][D], out [B][N][D]: `dtype` with row strides ldq/ldk/ldv/ldo and frame
 * strides *_bstride (elements); attn (nullable) [B, N, M] contiguous, attn_dtype F32 or `dtype`, holds
 * the softmax (before renormalisation).  N <= 128; D % 16 == 0 (and % 32 for 16-bit types).
 * workspace: >= hclsm_slot_attn_core_workspace(B, N, M, dtype) bytes, 16-byte aligned.
 * Two launches: logits + softmax over (frame, 64-token block); attn . v over (frame, 64-column block).
 * Replaces: slot_attention_fn / naive_slot_attention / compiled_slot_attention / the two Triton
 *   kernels (hclsm/kernels/slot_attention_kernel.py:43-355; denom_eps 1e-8 is the Triton form, :126)
 *   and the attention part of DynamicSlotAttention._iteration_step (objects/dynamic_slots.py:115-121).
 */
int64_t hclsm_slot_attn_core_workspace(int64_t B, int64_t N, int64_t M, int dtype);
int hclsm_slot_attn_core(const void* q, int64_t ldq, int64_t q_bstride, const void* k, int64_t ldk,
                         int64_t k_bstride, const void* v, int64_t ldv, int64_t v_bstride, void* out,
                         int64_t ldo, int64_t o_bstride, void* attn, int attn_dtype, int64_t B, int64_t N,
                         int64_t M, int64_t D, float scale, float denom_eps, float logit_clamp,
                         float renorm_eps, int dtype, void* workspace, int64_t workspace_bytes,
                         void* stream);

/* Parameters of one DynamicSlotAttention (objects/dynamic_slots.py:47-82).  Matrices in the compute
 * dtype, row-major as torch stores nn.Linear / nn.GRUCell weights; vectors float32 (nullable = 0 bias,
 * unit LayerNorm weight). */
typedef struct HclsmSlotWeights {
  const void* w_q;     /* [d, d]          project_q.weight */
  const void* w_kv;    /* [2d, d_in]      [project_k.weight; project_v.weight] (forward only) */
  const void* w_ih;    /* [3d, d]         gru.weight_ih (rows r, z, n) */
  const void* w_hh;    /* [3d, d]         gru.weight_hh */
  const void* w1;      /* [hidden, d]     mlp[0].weight */
  const void* w2;      /* [d, hidden]     mlp[2].weight */
  const float* b_ih;   /* [3d] */
  const float* b_hh;   /* [3d] */
  const float* b1;     /* [hidden] */
  const float* b2;     /* [d] */
  const float* ln_in_w;  const float* ln_in_b;   /* [d_in] norm_input */
  const float* ln_pre_w; const float* ln_pre_b;  /* [d]    norm_pre_attn */
  const float* ln_mlp_w; const float* ln_mlp_b;  /* [d]    norm_slots */
  const void* w_qt;    /* [d, d] w_q transposed, nullable: formed once per weight set by the caller; when NULL a
                          16-bit forward forms it in its workspace on every call (one more launch) */
  const void* w_qkv;   /* [2d, d_in] [w_q^T w_k; w_v], nullable: formed once per weight set by the caller (the
                          product in fp32, then rounded).  A 16-bit forward whose iterations run the fused core
                          (hclsm_slot_attention_kq_offset >= 0) then projects the inputs straight to kq = k w_q
                          and v, with no kq GEMM per call, and forms no k */
  const void* w1_n;        /* [hidden, d] w1 diag(ln_mlp_w) in dtype, nullable (then w1_n_sum and w1_n_bias are not
                              read): formed once per weight set by the caller.  A 16-bit iteration then folds
                              norm_slots into the W1 launch, ReLU(rstd (h w1_n^T - mean w1_n_sum) + w1_n_bias) with
                              mean and rstd of h's rows in dtype formed there, and runs no LayerNorm launch for it */
  const float* w1_n_sum;   /* [hidden] row sums of w1_n (its entries in dtype, summed in fp32) */
  const float* w1_n_bias;  /* [hidden] w1 ln_mlp_b + b1 */
} HclsmSlotWeights;

/* Workspace bytes for hclsm_slot_attention_iteration / _forward (16-byte aligned buffer). */
int64_t hclsm_slot_attention_workspace(int64_t B, int64_t N, int64_t M, int64_t d_in, int64_t d, int64_t hidden,
                                       int dtype);

/*
 * Byte offset, inside the workspace of hclsm_slot_attention_forward, of the token keys it computed:
 * k = LN_in(inputs) W_k^T as [B*M, d] row-major in `dtype`, valid after the forward until the workspace is
 * reused (or a negative error code).  Lets a caller reuse the keys (slot birth, dynamic_slots.py:170-177)
 * instead of recomputing norm_input + project_k.
 */
int64_t hclsm_slot_attention_k_offset(int64_t B, int64_t N, int64_t M, int64_t d_in, int64_t d, int64_t hidden,
                                      int dtype);

/*
 * Byte offset, inside the workspace of hclsm_slot_attention_forward, of kq = k w_q ([B*M, d] row-major in
 * `dtype`), which a 16-bit forward forms for shapes whose iterations run the fused attention core; a negative
 * code (HCLSM_ERR_UNSUPPORTED) for shapes and dtypes that form none.  The logits are then
 * LN_pre(slots) kq^T scale, so slot birth (dynamic_slots.py:180-186) can take its attention from kq without
 * project_q.  When W->w_qkv is given and this offset is valid, the forward forms kq and no k: the keys at
 * hclsm_slot_attention_k_offset are then not written.
 */
int64_t hclsm_slot_attention_kq_offset(int64_t B, int64_t N, int64_t M, int64_t d_in, int64_t d, int64_t hidden,
                                       int dtype);

/*
 * One slot-attention iteration (objects/dynamic_slots.py:98-131) for B frames of N slots:
 *   q = LN_pre(slots) W_q^T; attention core (logit clamp, renorm as above); GRUCell; slots + MLP(LN(.));
 *   clamp to +-slot_clamp if slot_clamp > 0.  slots_in / slots_out [B, N, d] float32 (may alias);
 *   k, v rows of `dtype` with row stride ldkv and frame stride kv_bstride.  Eight launches, no host sync.
 */
int hclsm_slot_attention_iteration(const HclsmSlotWeights* W, const float* slots_in, const void* k,
                                   const void* v, int64_t ldkv, int64_t kv_bstride, float* slots_out,
                                   int64_t B, int64_t N, int64_t M, int64_t d, int64_t hidden, float scale,
                                   float logit_clamp, float renorm_eps, float slot_clamp, int dtype,
                                   void* workspace, int64_t workspace_bytes, void* stream);

/*
 * DynamicSlotAttention forward up to the iterations (objects/dynamic_slots.py:149-164): k | v =
 * LN_in(inputs) [W_k; W_v]^T for inputs [B, M, d_in] float32, then n_iter iterations from slots0
 * [B, N, d] float32 into slots_out.  The slot initialisation draw (:86-96), existence head and slot
 * birth (:166-199) stay with the caller.  With N == 0 only the keys k are formed (slots0 / slots_out may be
 * NULL, W->w_qkv is not used); birth reads them at hclsm_slot_attention_k_offset in the workspace.  16-bit
 * weight matrices must be 16-byte aligned (HCLSM_ERR_UNSUPPORTED before any launch otherwise).
 */
int hclsm_slot_attention_forward(const HclsmSlotWeights* W, const float* inputs, int64_t d_in,
                                 const float* slots0, float* slots_out, int64_t B, int64_t N, int64_t M,
                                 int64_t d, int64_t hidden, int64_t n_iter, float scale, float logit_clamp,
                                 float renorm_eps, float slot_clamp, int dtype, void* workspace,
                                 int64_t workspace_bytes, void* stream);

/*
 * Allocation-free variant of hclsm_slot_attention_forward: the same arguments and launches, with the workspace
 * taken from a static device array of HCLSM_SLOT_NOALLOC_SCRATCH_BYTES in the library (one copy per GPU, held
 * until the process ends) instead of a caller buffer.  No allocation, free or synchronisation, so the call may
 * run under HIP graph capture once a first call has run on the device (it looks the array's address up and
 * sets up its launch tables): tests/test_zz_no_alloc.py captures it and replays it on new inputs.  A shape whose hclsm_slot_attention_workspace exceeds the array returns
 * HCLSM_ERR_SCRATCH before any launch (config 2, B=32 M=196 d=384 bf16, needs about 33 MB).  Calls that overlap
 * on one GPU (two streams, two threads) share the array and race; serialise them.
 * No counterpart in the reference: it is for callers that cannot allocate device memory (graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).
 */
#define HCLSM_SLOT_NOALLOC_SCRATCH_BYTES (64LL << 20)
int hclsm_slot_attention_forward_noalloc(const HclsmSlotWeights* W, const float* inputs, int64_t d_in,
                                         const float* slots0, float* slots_out, int64_t B, int64_t N, int64_t M,
                                         int64_t d, int64_t hidden, int64_t n_iter, float scale, float logit_clamp,
                                         float renorm_eps, float slot_clamp, int dtype, void* stream);

/* Workspace bytes for hclsm_level1_forward. */
int64_t hclsm_level1_forward_workspace(int64_t capacity, int64_t N, int64_t d_model, int64_t hidden, int dtype);

/*
 * Level1EventDynamics.forward on packed events, without host synchronisation.  Event e < *n_events
 * (a device-side count, e.g. the event index's stats[0]) is rows e*N .. e*N+N-1 of ev [capacity*N, d_slot]
 * (ev_dtype: F32 or dtype); the same rows of out [capacity*N, d_slot] (out_dtype: F32 or dtype) receive
 *   x = ev proj_in^T; per layer x += MHA over the event's N slots (LN1 first; keys j with
 *   obj_mask[ev_rows[e], j] <= 0.5 excluded; obj_mask [B, N] float32 nullable) and x += SwiGLU(LN2 x);
 *   out = LN(x) proj_out^T.
 * Rows of later events are untouched.  GEMM operands in `dtype` (F32 / BF16 / F16) with fp32
 * accumulation; the residual stream is fp32.  d_model / n_heads in {16, 32, 64, 128}; d_slot, d_model,
 * hidden multiples of 32 (4 for F32).  params: host array of 4 + 9 * n_layers device pointers:
 *   proj_in [d_model, d_slot], norm_w [d_model], norm_b [d_model], proj_out [d_slot, d_model], then per
 *   layer ln1_w, ln1_b [d_model], in_proj [3 d_model, d_model], out_proj [d_model, d_model], ln2_w,
 *   ln2_b [d_model], w1 [hidden, d_model], w3 [hidden, d_model], w2 [d_model, hidden]
 * (LayerNorm weights float32, the rest in `dtype`; no biases, as in the reference).  A query whose keys
 * are all excluded gives NaN, as torch's softmax over all -inf does.
 * fold (nullable; read for 16-bit dtypes): host array of 3 + 7 * n_layers device pointers, formed once per
 * weight set, with which the LayerNorms inside the stack are folded into the next layer (LN(x) W^T =
 * rstd (x (W diag g)^T - mean s) + W b, s the row sums of W diag g): no launch for the final LayerNorm and each
 * block's LN2, nor for LN1 of the blocks after the first where the QKV projection and the attention are one
 * launch (N = 32, 64-wide heads).  proj_out diag(norm_w) [d_slot, d_model] (dtype), its row sums [d_slot],
 * proj_out norm_b [d_slot]; then per layer in_proj diag(ln1_w) [3 d_model, d_model] (dtype), its row sums,
 * in_proj ln1_b [3 d_model], w1 diag(ln2_w), w3 diag(ln2_w) [hidden, d_model] (dtype), their row sums
 * [2 hidden] (w1 rows, then w3 rows), w1 ln2_b | w3 ln2_b [2 hidden] (float32 where not dtype); 16-byte aligned,
 * else (or for d_model or hidden not multiples of 64) the LayerNorms run as launches.
 * Replaces: Level1EventDynamics.forward with EventTransformerBlock and SwiGLUFFN
 *   (hclsm/dynamics/level1_event.py:17-133) on the events gathered by HierarchyManager.gather_events.
 */
int hclsm_level1_forward(const void* ev, int ev_dtype, void* out, int out_dtype, const int32_t* n_events,
                         int64_t capacity, int64_t N, const int32_t* ev_rows, const float* obj_mask,
                         int64_t d_slot, int64_t d_model, int64_t n_heads, int64_t hidden, int64_t n_layers,
                         const void* const* params, const void* const* fold, float ln_eps, int dtype,
                         void* workspace, int64_t workspace_bytes, void* stream);

/* Workspace bytes for hclsm_relation_graph_forward, or HCLSM_ERR_UNSUPPORTED for a shape outside it. */
int64_t hclsm_relation_graph_workspace(int64_t frames, int64_t N, int64_t D, int64_t E, int dtype);

/*
 * RelationGraph.forward (GNN over object slots) for `frames` frames of N slots:
 *   per round: edge features e_ij = ReLU(W2 ReLU(W1 LN([n_i; n_j; n_i - n_j; n_i * n_j]) + b1) + b2),
 *   weights w_ij = sigmoid(we . e_ij + be) * alive_i * alive_j, agg_i = sum_j ReLU(Wm e_ij + bm) w_ij,
 *   n_i += U2 ReLU(U1 [n_i; agg_i] + c1) + c2; causal_ij = sigmoid(c2' . ReLU(C1 e_ij + d1) + d2) * alive_i
 *   * alive_j; finally nodes_out = n * alive.
 * chunked != 0 gives the reference's N > 32 path semantics: edges recomputed from the current nodes every
 * round and the causal edges from the final nodes; chunked == 0 the all-pairs path (causal edges from the
 * last edges computed, which for n_rounds == 1 are those of the input nodes).
 * nodes, nodes_out [frames, N, D], alive [frames, N] (nullable), causal [frames, N, N]: float32.
 * params: host array of 18 device pointers in the module's parameter order (pair_norm.weight/bias [4D],
 *   edge_mlp.0.weight [2E, 4D] / bias, edge_mlp.2.weight [E, 2E] / bias, edge_weight.weight [E] / bias [1],
 *   msg_mlp.0.weight [D, E] / bias, update_mlp.0.weight [D, 2D] / bias, update_mlp.2.weight [D, D] / bias,
 *   causal_mlp.0.weight [E/2, E] / bias, causal_mlp.2.weight [E/2] / bias [1]); matrices in `dtype`
 *   (F32 / BF16 / F16), vectors float32.  D, E multiples of 32, E <= 192, N <= 128 (64 for F32), and the
 *   workgroup tiles within 160 KB of LDS (hclsm_relation_graph_workspace says HCLSM_ERR_UNSUPPORTED otherwise).
 * Replaces: RelationGraph.forward (hclsm/objects/relation_graph.py:68-193), called by the model on the
 *   tracked slots (model.py:255-266).
 */
int hclsm_relation_graph_forward(const float* nodes, const float* alive, float* nodes_out, float* causal,
                                 int64_t frames, int64_t N, int64_t D, int64_t E, int64_t n_rounds, int chunked,
                                 const void* const* params, float ln_eps, int dtype, void* workspace,
                                 int64_t workspace_bytes, void* stream);

/* Workspace bytes for hclsm_gnn_message_pass, or HCLSM_ERR_UNSUPPORTED for a shape outside it. */
int64_t hclsm_gnn_message_pass_workspace(int64_t frames, int64_t N, int64_t D, int64_t E, int dtype);

/*
 * GNN message passing over the N slots of `frames` frames, n_rounds rounds of:
 *   e_ij = ReLU(W2 ReLU(W1 [n_i; n_j; n_i - n_j; n_i * n_j] + b1) + b2)      (no pair norm)
 *   w_ij = sigmoid(we . e_ij + be) * alive_i * alive_j
 *   agg_i = sum_j ReLU(Wm e_ij + bm) w_ij,   n_i += U2 ReLU(U1 [n_i; agg_i] + c1) + c2
 * then nodes_out = n * alive.  The last round's edge features of the targets j in [ej0, ej0 + enj) go to
 * edges_out [frames, N, enj, E] float32 (as the next layer sees them: rounded to `dtype` for 16-bit operands).
 * nodes, nodes_out [frames, N, D], alive [frames, N] (nullable): float32.  params: host array of 12 device
 * pointers edge_mlp.0.weight [2E, 4D] / .bias, edge_mlp.2.weight [E, 2E] / .bias, edge_weight.weight [E] /
 * .bias [1], msg_mlp.0.weight [D, E] / .bias, update_mlp.0.weight [D, 2D] / .bias, update_mlp.2.weight [D, D] /
 * .bias; matrices in `dtype` (F32 / BF16 / F16), vectors float32, none nullable.  D, E multiples of 16 (F32) or 32,
 * E <= 192, N <= 64 (F32) or 128.
 * Replaces: naive_gnn_message_pass / optimized_gnn_message_pass (all pairs, enj = N) and
 *   chunked_gnn_message_pass (edges of the last target chunk) of hclsm/kernels/gnn_message_pass.py:38-243.
 */
int hclsm_gnn_message_pass(const float* nodes, const float* alive, float* nodes_out, float* edges_out,
                           int64_t frames, int64_t N, int64_t D, int64_t E, int64_t n_rounds, int64_t ej0,
                           int64_t enj, const void* const* params, int dtype, void* workspace,
                           int64_t workspace_bytes, void* stream);

/* ---- slot tracker (hclsm/objects/slot_tracker.py, tracking loop of hclsm/model.py:229-252) ----
 * Shapes: D (d_slot) a multiple of 64 and at most 384; the Sinkhorn entries N <= 128.  The workspace
 * queries return HCLSM_ERR_UNSUPPORTED outside these.  Slots, alive flags, costs and hidden states are
 * float32; match_mlp.0.weight [D, 3D], match_mlp.2.weight [D/4, D], hidden_gru.weight_ih / weight_hh
 * [3D, D] in `dtype` (F32 / BF16 / F16); biases and match_mlp.4.weight [D/4] float32. */

/* Workspace bytes for hclsm_slot_track_cost. */
int64_t hclsm_slot_track_cost_workspace(int64_t frames, int64_t N, int64_t D, int dtype);

/*
 * Matching cost between frames t and t1 for `frames` frame pairs of N slots:
 *   cost_ij = -(w3 . ReLU(W2 ReLU(W1 [a_i; b_j; |a_i - b_j|] + b1) + b2) + b3
 *              - 1e4 [alive_t_i < 0.5] - 1e4 [alive_t1_j < 0.5]),  a, b = slots clamped to [-50, 50].
 * slots_t, slots_t1 [frames, N, D]; alive_t, alive_t1 [frames, N] (both NULL: no penalties); cost
 * [frames, N, N] (not clamped).  params: 6 device pointers match_mlp.0.weight, .0.bias, .2.weight,
 * .2.bias, .4.weight, .4.bias.
 * Replaces: SlotTracker.compute_cost_matrix (hclsm/objects/slot_tracker.py:74-107).
 */
int hclsm_slot_track_cost(const float* slots_t, const float* slots_t1, const float* alive_t, const float* alive_t1,
                          float* cost, int64_t frames, int64_t N, int64_t D, const void* const* params, int dtype,
                          void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Sinkhorn matching of `frames` N x N costs: log_alpha = -clamp(cost, -1e4, 1e4) * (1 / max(temperature,
 * 1e-6)), n_iters rounds of row then column log-sum-exp normalisation; perm [frames, N] int64 = argmax over
 * j of exp(log_alpha) (lowest index on ties), confidence [frames, N] (nullable) its value, matched
 * [frames, N] = [alive_t_i > 0.5] [alive_t1_perm_i > 0.5] [confidence > 0.3] (alive pointers nullable:
 * alive).  No workspace.  N <= 128.
 * Replaces: SlotTracker.forward after the cost (slot_tracker.py:122-135) and _sinkhorn_matching (:15-43).
 */
int hclsm_slot_track_match(const float* cost, const float* alive_t, const float* alive_t1, int64_t* perm,
                           float* matched, float* confidence, int64_t frames, int64_t N, int64_t n_iters,
                           float temperature, void* stream);

/* Workspace bytes for hclsm_slot_track_reorder_update. */
int64_t hclsm_slot_track_reorder_update_workspace(int64_t frames, int64_t N, int64_t D, int dtype);

/*
 * reordered[f, i] = slots_t1[f, perm[f, i]] (an index outside [0, N) gives a NaN row);
 * hidden_t1 = m * GRUCell(reordered, hidden_t) + (1 - m) * reordered, m = matched[f, i].
 * slots_t1, hidden_t, reordered, hidden_t1 [frames, N, D]; perm [frames, N] int64; matched [frames, N].
 * params: 4 device pointers hidden_gru.weight_ih, .weight_hh, .bias_ih, .bias_hh (biases nullable).
 * Replaces: SlotTracker.reorder_and_update (slot_tracker.py:137-158).
 */
int hclsm_slot_track_reorder_update(const float* slots_t1, const int64_t* perm, const float* hidden_t,
                                    const float* matched, float* reordered, float* hidden_t1, int64_t frames,
                                    int64_t N, int64_t D, const void* const* params, int dtype, void* workspace,
                                    int64_t workspace_bytes, void* stream);

/* Workspace bytes for hclsm_slot_track_sequence (with_hidden != 0: room for the GRU carry). */
int64_t hclsm_slot_track_sequence_workspace(int64_t batch, int64_t T, int64_t N, int64_t D, int with_hidden,
                                            int dtype);

/*
 * The tracking loop over `batch` clips of T frames: frame 0 is kept; for t >= 1 the tracked slots of frame
 * t-1 are matched against frame t (cost, Sinkhorn with n_iters / temperature, as the two entries above),
 * frame t's slots and alive flags are reordered by the perm, and, when hidden is non-NULL, the GRU state
 * is carried (hidden_0 = 0, blend as hclsm_slot_track_reorder_update).
 * slots, tracked [batch, T, N, D]; alive, alive_out [batch, T, N] (nullable: all alive / not written);
 * perm [batch, T, N] int64 and matched [batch, T, N] (nullable; frame 0: identity and 0); hidden
 * [batch, N, D] (nullable), the state after the last frame.  params: 10 device pointers, the six of
 * hclsm_slot_track_cost then the four of hclsm_slot_track_reorder_update (those only read when hidden is
 * wanted).  The matching costs of every (t-1, t) frame pair are computed in one launch (the previous perm
 * only reorders cost rows); one workgroup per clip runs the Sinkhorn steps in sequence.
 * Replaces: the frame loop of HCLSMWorldModel.forward (hclsm/model.py:229-252) over self.slot_tracker.
 */
int hclsm_slot_track_sequence(const float* slots, const float* alive, float* tracked, float* alive_out,
                              int64_t* perm, float* matched, float* hidden, int64_t batch, int64_t T, int64_t N,
                              int64_t D, int64_t n_iters, float temperature, const void* const* params, int dtype,
                              void* workspace, int64_t workspace_bytes, void* stream);

/*
 * VALU issue-rate probe (measurement support; no counterpart in the reference, whose kernels have no
 * roofline).  Launches `waves` one-wave workgroups; each runs `iters` iterations of a fixed block of
 * independent VALU instructions of one class on eight register chains:
 *   kind 0: 32 v_fma_f32;  kind 1: 32 v_exp_f32;
 *   kind 2: 32 v_exp_f32 + 96 v_fma_f32, one exp then three FMAs (the scan's essential mix per update);
 *   kind 3: the same 128 in blocks of 8 exps then 24 FMAs.
 * With waves = w x (4 x compute units), the launch time / (w x iters x instructions per iteration) is a
 * SIMD's time per instruction of that class at w waves per SIMD: the issue costs that price the scan's
 * instruction counts in the benchmark's VALU roofline.  sink: device float[waves x 64], never written for
 * the values the kernel computes (it keeps the chains live).  HCLSM_ERR_MODE for an unknown kind.
 */
int hclsm_issue_probe(int kind, int64_t waves, int iters, float* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HCLSM_AMD_H */
