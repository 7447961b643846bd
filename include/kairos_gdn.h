/*
 * kairos_gdn.h -- C ABI of the MI355X (gfx950) chunked GatedDeltaNet forward.
 *
 * Drop-in native backend for the op
 *     chunk_gated_delta_rule(q, k, v, g, beta, scale, initial_state,
 *                            output_final_state, use_qk_l2norm_in_kernel,
 *                            cu_seqlens) -> (o, final_state)
 * of flash-linear-attention 0.4.0 as vendored by Kairos
 * (kairos/third_party/fla/ops/gated_delta_rule/chunk.py:217-323).
 *
 * Conventions (all entry points):
 *  - Every tensor argument is a device pointer to a contiguous buffer in the
 *    reference layout: q, k [B, T, H, K]; v, o [B, T, H, V]; g, beta [B, T, H];
 *    initial_state / final_state [N, H, K, V].  Vector-loaded buffers (q, k, v,
 *    o and the stage intermediates) must be 16-byte aligned.
 *  - Variable length: pass cu_seqlens (device, int64 [n_seqs + 1], first entry
 *    0, last entry T, non-decreasing) with B == 1 and n_seqs >= 1; the chunk
 *    map is built on the device (no host synchronisation).  Fixed length:
 *    cu_seqlens == NULL and n_seqs == 0 (N = B sequences of length T).
 *  - dtype codes: KAIROS_GDN_F32, KAIROS_GDN_BF16, KAIROS_GDN_F8E4M3 (q/k only,
 *    with per-head fp32 dequantisation scales q_scale[H], k_scale[H]).
 *    bf16 q/k/v (or fp8 q/k with bf16 v) run the bf16 path; fp32 q/k/v the
 *    fp32 path.  g is fp32 or bf16; beta fp32 or bf16; initial_state fp32 or
 *    bf16; final_state is always fp32.
 *  - Supported head dims: K in {64, 128, 256}; V a multiple of 16, at most
 *    1024 (the Kairos 4B layer runs K = 256, V = 512).  bf16 with K, V in
 *    {64, 128} runs the segment-parallel fused kernels; every other shape runs
 *    the stage kernels in sequence.
 *  - Work is enqueued on `stream` (a hipStream_t; NULL = default stream) and
 *    is stream-ordered: no entry point synchronises or allocates.  Scratch
 *    memory comes from the caller's `workspace`.  Entry points are reentrant;
 *    concurrent calls must use distinct workspaces.  One exception in how the
 *    work is queued: the fixed-length K = 256 forward of kairos_gdn_chunk_fwd
 *    (and of the _gated_norm / _conv calls) runs in parts on library streams
 *    of the current device (two, three with the gated norm, which runs by
 *    parts beside the last recurrence part), shared by every caller in the process
 *    (created on first use, default priority, kept until exit, enqueued under
 *    one process-wide lock), joined to `stream` by events: work queued on
 *    `stream` after the call sees its results, but such calls issued from
 *    different caller streams run one after another on the library streams.
 *    Under graph capture, for varlen batches, in kairos_gdn_chunk_fwd_noalloc
 *    and with KAIROS_GDN_WIDE_PIPE=1 everything runs on `stream`.
 *  - Return value: KAIROS_GDN_OK or an error code; kairos_gdn_last_error()
 *    returns the message of the calling thread's last failure.  No exception
 *    crosses the ABI.
 */
#ifndef KAIROS_GDN_H
#define KAIROS_GDN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KAIROS_GDN_ABI_VERSION 2

#define KAIROS_GDN_F32 0
#define KAIROS_GDN_BF16 1
#define KAIROS_GDN_F8E4M3 2

#define KAIROS_GDN_OK 0
#define KAIROS_GDN_EINVAL 1       /* invalid argument: shape, pointer, alignment, dtype mix */
#define KAIROS_GDN_EUNSUPPORTED 2 /* head dims / dtype combination not built */
#define KAIROS_GDN_EWORKSPACE 3   /* workspace too small */
#define KAIROS_GDN_EHIP 4         /* HIP runtime error at launch */

int kairos_gdn_abi_version(void);
const char* kairos_gdn_last_error(void);

/* Upper bound on the number of 64-token chunks over all sequences (exact for
 * fixed length: B * ceil(T / 64); varlen: T / 64 + n_seqs).  Stage
 * intermediates indexed by chunk are sized with it. */
int64_t kairos_gdn_num_chunks_bound(int64_t B, int64_t T, int64_t n_seqs);

/* Bytes of workspace kairos_gdn_chunk_fwd needs for this problem. */
size_t kairos_gdn_chunk_fwd_workspace_size(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V,
                                           int64_t n_seqs, int qk_dtype, int v_dtype,
                                           int use_qk_l2norm);

/* Whole forward.  Replaces ChunkGatedDeltaRuleFunction.forward
 * (chunk.py:154-186: optional q/k L2 norm, then chunk_gated_delta_rule_fwd,
 * chunk.py:16-67).  o gets v's storage dtype.  final_state may be NULL
 * (output_final_state=False); initial_state may be NULL (zero state).
 * scale multiplies q.k and q.h (the reference defaults it to K^-0.5,
 * chunk.py:309-310; the caller passes the value). */
int kairos_gdn_chunk_fwd(const void* q, const void* k, const void* v, const void* g, const void* beta,
                         const float* q_scale, const float* k_scale, const void* initial_state, void* o,
                         float* final_state, const int64_t* cu_seqlens, int64_t n_seqs, int64_t B, int64_t T,
                         int64_t H, int64_t K, int64_t V, int qk_dtype, int v_dtype, int g_dtype,
                         int beta_dtype, int h0_dtype, float scale, int use_qk_l2norm, void* workspace,
                         size_t workspace_bytes, void* stream);

/* The forward followed by the layer's output norm: y = o_norm(o, gate) with
 * o = chunk_gated_delta_rule(q, k, v, g, beta, ...), replacing the pair of
 * calls at fla layers/gated_deltanet.py:275-311 (chunk_gated_delta_rule, then
 * FusedRMSNormGated, modules/fused_norm_gate.py:42-127, RMS path, no
 * residual; the norm is kairos_gdn_rms_norm_gated over rows of V).  The
 * forward's arguments are kairos_gdn_chunk_fwd's, with y (v's dtype) in place
 * of o; gate: [B*T, H, V] in gate_dtype (fp32 or bf16, 16-byte aligned);
 * norm_weight / norm_bias: [V] in norm_w_dtype or NULL; eps and activation as
 * kairos_gdn_rms_norm_gated.  V at most 512.  The workspace is
 * kairos_gdn_chunk_fwd_gated_norm_workspace_size()'s (a workspace of
 * kairos_gdn_chunk_fwd_workspace_size() bytes is also accepted: the norm then
 * runs as a pass of its own).  The norm is applied to o rounded to its storage
 * dtype, as the two reference calls do.  With a bf16 gate and head dims 64 /
 * 128 it is computed in the segment scan's output kernel (o never reaches
 * HBM); with the environment variable KAIROS_GDN_WIDE_NORM_FOLD=1 also in the
 * fused K = 256 kernel (V a multiple of 64), whose workgroups of one head
 * exchange per-token sums of squares through the workspace (off by default:
 * slower there than the norm kernel after the forward); otherwise the norm
 * kernel runs on y in place: for the pipelined K = 256 forward by parts, the
 * rows of every part but the last beside the last recurrence part
 * (KAIROS_GDN_NORM_PARTS=0: one pass after the forward), else after it. */
int kairos_gdn_chunk_fwd_gated_norm(const void* q, const void* k, const void* v, const void* g, const void* beta,
                                    const float* q_scale, const float* k_scale, const void* initial_state,
                                    const void* gate, const void* norm_weight, const void* norm_bias, void* y,
                                    float* final_state, const int64_t* cu_seqlens, int64_t n_seqs, int64_t B,
                                    int64_t T, int64_t H, int64_t K, int64_t V, int qk_dtype, int v_dtype,
                                    int g_dtype, int beta_dtype, int h0_dtype, int gate_dtype, int norm_w_dtype,
                                    float scale, int use_qk_l2norm, float eps, int activation, void* workspace,
                                    size_t workspace_bytes, void* stream);

/* Bytes of workspace kairos_gdn_chunk_fwd_gated_norm needs:
 * kairos_gdn_chunk_fwd_workspace_size() plus, when the norm is folded into
 * the fused K = 256 form (KAIROS_GDN_WIDE_NORM_FOLD=1), 4 KiB per (chunk,
 * head) for the exchanged sums of squares.  No counterpart in the reference
 * (its norm is a separate module). */
size_t kairos_gdn_chunk_fwd_gated_norm_workspace_size(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V,
                                                      int64_t n_seqs, int qk_dtype, int v_dtype,
                                                      int use_qk_l2norm);

/* kairos_gdn_chunk_fwd without a workspace argument: the call allocates
 * nothing (no hipMalloc / hipFree, no allocating library routine) and takes
 * its scratch memory from a static device array inside the library, of
 * kairos_gdn_chunk_fwd_noalloc_max_bytes() bytes (256 MiB) on every GPU the
 * library runs on, committed at the first call on a device (a process that
 * never calls it does not pay for it) and held until the process ends.  No
 * counterpart in the reference: it is for callers that cannot allocate (code
 * under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation).  A problem
 * whose kairos_gdn_chunk_fwd_workspace_size() exceeds the array is rejected
 * with KAIROS_GDN_EWORKSPACE.  Every call on one GPU shares that GPU's array:
 * calls that overlap on one GPU (concurrent streams or threads) race and must
 * be serialised by the caller.  Same results as kairos_gdn_chunk_fwd (same
 * kernels); calls made through it are not recorded by the timing hook. */
int kairos_gdn_chunk_fwd_noalloc(const void* q, const void* k, const void* v, const void* g, const void* beta,
                                 const float* q_scale, const float* k_scale, const void* initial_state, void* o,
                                 float* final_state, const int64_t* cu_seqlens, int64_t n_seqs, int64_t B,
                                 int64_t T, int64_t H, int64_t K, int64_t V, int qk_dtype, int v_dtype,
                                 int g_dtype, int beta_dtype, int h0_dtype, float scale, int use_qk_l2norm,
                                 void* stream);
size_t kairos_gdn_chunk_fwd_noalloc_max_bytes(void);

/* Chunks per segment that kairos_gdn_chunk_fwd uses for this problem (the
 * segment plan: sequences are cut into segments of this many 64-token chunks
 * so that (segment, head) work items fill the GPU; the environment variable
 * KAIROS_GDN_SEG_CHUNKS overrides it).  No counterpart in the reference. */
int kairos_gdn_segment_chunks(int64_t B, int64_t T, int64_t H, int64_t n_seqs);

/* The varlen maps every call builds on the device from cu_seqlens (exposed for
 * testing and for callers that precompute them): chunk_off[n] = index of the
 * first 64-token chunk of sequence n, chunk_off[n_seqs] = the chunk count --
 * prepare_chunk_offsets(cu_seqlens, 64) (fla ops/utils/index.py:122-127) as
 * int32 -- and seg_off[n] = index of the first segment of sequence n when
 * sequences are cut into segments of seg_chunks chunks (no counterpart in the
 * reference).  chunk_off, seg_off: device int32 [n_seqs + 1]. */
int kairos_gdn_varlen_maps(const int64_t* cu_seqlens, int64_t n_seqs, int64_t seg_chunks, int32_t* chunk_off,
                           int32_t* seg_off, void* stream);

/* ---- backward ---------------------------------------------------------------
 * Gradients of the forward above: replaces ChunkGatedDeltaRuleFunction.backward
 * (chunk.py:188-213: chunk_gated_delta_rule_bwd, chunk.py:70-146, then the
 * l2norm backward of q and k when use_qk_l2norm).  Takes the forward's own
 * inputs (q, k as given to the forward, i.e. before the in-op L2 norm) and
 * recomputes what the reference saves (the normalised q, k, gc and Ai) and
 * what it recomputes (w, u, the state snapshots h and v_new, chunk.py:84-101).
 * do [B, T, H, V] in v's dtype; dht [N, H, K, V] fp32 or NULL (zero).
 * Outputs: dq, dk [B, T, H, K] in q's dtype; dv [B, T, H, V] in v's dtype;
 * dg [B, T, H] fp32; dbeta [B, T, H] in beta's dtype; dh0 [N, H, K, V] fp32, or
 * NULL (must be NULL when initial_state is).  bf16 or fp32 q/k/v (fp8 is
 * forward-only); K in {64, 128, 256}, V a multiple of 64 (at most 512 in bf16;
 * K, V at most 128 in fp32).  Workspace: kairos_gdn_chunk_bwd_workspace_size(). */
size_t kairos_gdn_chunk_bwd_workspace_size(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V,
                                           int64_t n_seqs, int qk_dtype, int v_dtype, int use_qk_l2norm);
int kairos_gdn_chunk_bwd(const void* q, const void* k, const void* v, const void* g, const void* beta,
                         const void* initial_state, const void* do_, const float* dht, void* dq, void* dk, void* dv,
                         float* dg, void* dbeta, float* dh0, const int64_t* cu_seqlens, int64_t n_seqs, int64_t B,
                         int64_t T, int64_t H, int64_t K, int64_t V, int qk_dtype, int v_dtype, int g_dtype,
                         int beta_dtype, int h0_dtype, float scale, int use_qk_l2norm, void* workspace,
                         size_t workspace_bytes, void* stream);

/* ---- kernel timing (measurement hook, no counterpart in the reference) ----
 * kairos_gdn_profile_begin() makes every following kairos_gdn_chunk_fwd call
 * of the fused path record hipEvents on its stream around its four kernels
 * (seg_prep, seg_trans, seg_combine, seg_out).  kairos_gdn_profile_end() waits
 * for the recorded events, stops recording, writes the average milliseconds of
 * the four kernels per call into avg_ms[0..min(n,4)-1] and returns the number
 * of calls recorded, or -1 on a HIP error (message in kairos_gdn_last_error()).
 * A kernel the call did not need (seg_trans / seg_combine for single-segment
 * sequences) reports ~0 ms.  The staged fp32 K = 128 path records nothing. */
int kairos_gdn_profile_begin(void);
int kairos_gdn_profile_end(double* avg_ms, int n);

/* ---- stage entry points (parity testing and composition) ----------------
 * Each stage replaces one reference function.  Varlen stage calls need
 * kairos_gdn_stage_workspace_size(n_seqs) bytes of workspace (chunk map);
 * fixed-length calls accept workspace = NULL. */
size_t kairos_gdn_stage_workspace_size(int64_t n_seqs);

/* chunk_local_cumsum (fla ops/utils/cumsum.py:247-279, scalar gates, chunk 64):
 * gc [B, T, H] fp32. */
int kairos_gdn_chunk_local_cumsum(const void* g, int g_dtype, float* gc, const int64_t* cu_seqlens,
                                  int64_t n_seqs, int64_t B, int64_t T, int64_t H, void* workspace,
                                  size_t workspace_bytes, void* stream);

/* chunk_local_cumsum + chunk_scaled_dot_kkt_fwd + solve_tril + recompute_w_u_fwd
 * (cumsum.py:247-279, chunk_scaled_dot_kkt.py:76-124, solve_tril.py:334-382,
 * wy_fast.py:213-248), fused.  Outputs: gc [B,T,H] fp32; w [B,T,H,K];
 * uT [NCb, H, V, 64] (u of chunk c transposed, NCb = num_chunks_bound);
 * optional A [B,T,H,64] fp32 and Ai [B,T,H,64] (storage dtype) -- pass NULL to skip. */
int kairos_gdn_prepare_wy(const void* k, const void* v, const void* g, const void* beta, const float* k_scale,
                          float* gc, void* w, void* uT, float* A, void* Ai, const int64_t* cu_seqlens,
                          int64_t n_seqs, int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int k_dtype,
                          int v_dtype, int g_dtype, int beta_dtype, void* workspace, size_t workspace_bytes,
                          void* stream);

/* chunk_gated_delta_rule_fwd_h (fla ops/common/chunk_delta_h.py:454-500).
 * Outputs: hT [NCb, H, V, K] (state before chunk c, transposed per chunk);
 * vnT [NCb, H, V, 64] (ungated v_new of chunk c, transposed); final_state
 * [N, H, K, V] fp32 or NULL. */
int kairos_gdn_fwd_h(const void* k, const float* k_scale, const void* w, const void* uT, const float* gc,
                     const void* initial_state, void* hT, void* vnT, float* final_state,
                     const int64_t* cu_seqlens, int64_t n_seqs, int64_t B, int64_t T, int64_t H, int64_t K,
                     int64_t V, int k_dtype, int v_dtype, int h0_dtype, void* workspace,
                     size_t workspace_bytes, void* stream);

/* chunk_fwd_o (fla ops/common/chunk_o.py:498-535): o [B, T, H, V] in v's dtype. */
int kairos_gdn_fwd_o(const void* q, const void* k, const float* q_scale, const float* k_scale, const void* hT,
                     const void* vnT, const float* gc, void* o, float scale, const int64_t* cu_seqlens,
                     int64_t n_seqs, int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int qk_dtype,
                     int v_dtype, void* workspace, size_t workspace_bytes, void* stream);

/* ---- the same stages in the reference's layouts --------------------------
 * u and v_new [B, T, H, V] as recompute_w_u_fwd and chunk_gated_delta_rule_fwd_h
 * return them (wy_fast.py:213-248, chunk_delta_h.py:454-500); h [NCb, H, K, V],
 * the reference's h [B, NT, H, K, V] (varlen: [1, NT, H, K, V]) in its first
 * NT = number-of-real-chunks rows, zeros after them.  K and V multiples of 64.
 * Workspace: kairos_gdn_stage_tokens_workspace_size(..., dtype = v's dtype);
 * each call moves its operands between the two layouts at its boundary. */
size_t kairos_gdn_stage_tokens_workspace_size(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int64_t n_seqs,
                                              int dtype);

/* kairos_gdn_prepare_wy with u [B, T, H, V] (wy_fast.py:213-248 recompute_w_u_fwd's u). */
int kairos_gdn_prepare_wy_tokens(const void* k, const void* v, const void* g, const void* beta, const float* k_scale,
                                 float* gc, void* w, void* u, float* A, void* Ai, const int64_t* cu_seqlens,
                                 int64_t n_seqs, int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int k_dtype,
                                 int v_dtype, int g_dtype, int beta_dtype, void* workspace, size_t workspace_bytes,
                                 void* stream);

/* chunk_gated_delta_rule_fwd_h (chunk_delta_h.py:454-500) in its own layouts: u in, h and
 * v_new (ungated) out as above; final_state [N, H, K, V] fp32 or NULL. */
int kairos_gdn_fwd_h_tokens(const void* k, const float* k_scale, const void* w, const void* u, const float* gc,
                            const void* initial_state, void* h, void* v_new, float* final_state,
                            const int64_t* cu_seqlens, int64_t n_seqs, int64_t B, int64_t T, int64_t H, int64_t K,
                            int64_t V, int k_dtype, int v_dtype, int h0_dtype, void* workspace,
                            size_t workspace_bytes, void* stream);

/* chunk_fwd_o (chunk_o.py:498-535) in its own layouts: h [NCb, H, K, V], v_new [B, T, H, V]
 * in; o [B, T, H, V] in v's dtype. */
int kairos_gdn_fwd_o_tokens(const void* q, const void* k, const float* q_scale, const float* k_scale, const void* h,
                            const void* v_new, const float* gc, void* o, float scale, const int64_t* cu_seqlens,
                            int64_t n_seqs, int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int qk_dtype,
                            int v_dtype, void* workspace, size_t workspace_bytes, void* stream);

/* l2norm_fwd (fla modules/l2norm.py:157-196), y = x / sqrt(sum x^2 + 1e-6) over
 * the last dim D (multiple of 8, <= 512), in x's dtype (fp32 or bf16), and, if
 * rstd is not null, rstd = 1 / sqrt(sum x^2 + 1e-6) per row in fp32 (the
 * reference returns (y, rstd)). */
int kairos_gdn_l2norm_fwd(const void* x, void* y, float* rstd, int dtype, int64_t rows, int64_t D, void* stream);

/* ---- output epilogue -------------------------------------------------------
 * Gated RMSNorm of the GatedDeltaNet layer's output (o_norm = FusedRMSNormGated,
 * fla layers/gated_deltanet.py:197,311), replacing layer_norm_gated_fwd with
 * is_rms_norm=True (fla modules/fused_norm_gate.py:449-525, kernel :42-127)
 * without residual:
 *   rstd = 1 / sqrt(mean_d x^2 + eps);  y = x rstd weight [+ bias];
 *   y *= g sigmoid(g) (KAIROS_GDN_ACT_SWISH, 'swish' / 'silu') or
 *   y *= sigmoid(g)   (KAIROS_GDN_ACT_SIGMOID).
 * x, g: [rows, D] (fp32 or bf16 each; 16-byte aligned); weight, bias: [D] in
 * w_dtype (16-byte aligned), either may be NULL (no affine weight / no bias); y: [rows, D] in
 * x's dtype; rstd: [rows] fp32 or NULL.  D a multiple of 8, at most 512. */
#define KAIROS_GDN_ACT_SWISH 0
#define KAIROS_GDN_ACT_SIGMOID 1
int kairos_gdn_rms_norm_gated(const void* x, const void* g, const void* weight, const void* bias, void* y,
                              float* rstd, int x_dtype, int g_dtype, int w_dtype, int64_t rows, int64_t D,
                              float eps, int activation, void* stream);

/* ---- short-sequence mode -------------------------------------------------
 * Token-by-token gated delta rule in fp32, replacing
 * fused_recurrent_gated_delta_rule_fwd (fla ops/gated_delta_rule/fused_recurrent.py:138-185,
 * kernel :21-135), the layer's mode for q_len <= 64 (layers/gated_deltanet.py:220).
 * q, k [B, T, H, K] (fp32 or bf16, 16-byte aligned); v [B, T, HV, V] with HV a
 * multiple of H (q/k head i_hv / (HV / H) serves value head i_hv); optional
 * gates g [B, T, HV], gk [B, T, HV, K], gv [B, T, HV, V] (log space, fp32 or
 * bf16, NULL = absent); beta [B, T, HV] (beta_headwise = 1) or [B, T, HV, V]
 * (beta_headwise = 0), NULL = ones; initial_state [N, HV, K, V] (fp32 or bf16,
 * NULL = zeros); o [B, T, HV, V] in v's dtype; final_state [N, HV, K, V] fp32
 * or NULL.  K in {16, 32, 64, 128, 256}, V at most 4096.  No workspace. */
int kairos_gdn_fused_recurrent_fwd(const void* q, const void* k, const void* v, const void* g, const void* gk,
                                   const void* gv, const void* beta, const void* initial_state, void* o,
                                   float* final_state, const int64_t* cu_seqlens, int64_t n_seqs, int64_t B,
                                   int64_t T, int64_t H, int64_t HV, int64_t K, int64_t V, int qk_dtype,
                                   int v_dtype, int g_dtype, int gk_dtype, int gv_dtype, int beta_dtype,
                                   int beta_headwise, int h0_dtype, float scale, int use_qk_l2norm, void* stream);

/* ---- layer prologue --------------------------------------------------------
 * Short causal convolution of the q/k/v projections (ShortConvolution with
 * activation 'silu', fla layers/gated_deltanet.py:176-189,235-253), replacing
 * causal_conv1d_fwd and causal_conv1d_update_states (fla modules/convolution.py:410-458,
 * :539-602, Triton backend):
 *   y[t, d] = act( sum_{i<W} weight[d, i] x~[t - W + 1 + i, d] + bias[d] )
 * with x~ = x inside each sequence and, before its first token, initial_state
 * (the cache [N, D, W], slot W-1 the most recent input; NULL = zeros).
 * x, y: [B*T, D] fp32 or bf16 (16-byte aligned, D a multiple of 8); weight
 * [D, W] (16-byte aligned) and bias [D] (NULL = none) in w_dtype; initial_state / final_state
 * [N, D, W] in x's dtype, final_state = the last W entries of [cache, x] per
 * sequence (NULL = not wanted; must not alias initial_state).  W in 1..4.
 * activation_silu: y = z sigmoid(z).  l2norm_head_dim (0 = off, else 64, 128,
 * 256 or 512 dividing D): y, rounded to x's dtype, is then normalised per head,
 * y / sqrt(sum y^2 + 1e-6) (fla modules/l2norm.py:115-118) -- the q/k
 * normalisation the layer asks of the chunked op, fused here (no counterpart
 * in the reference as one kernel). */
int kairos_gdn_causal_conv1d_fwd(const void* x, const void* weight, const void* bias, const void* initial_state,
                                 void* y, void* final_state, const int64_t* cu_seqlens, int64_t n_seqs, int64_t B,
                                 int64_t T, int64_t D, int64_t W, int x_dtype, int w_dtype, int activation_silu,
                                 int l2norm_head_dim, void* stream);

/* The layer's prologue folded into the chunked forward: the q_conv1d / k_conv1d / v_conv1d
 * ShortConvolutions (kernel size 4, activation 'silu') of fla layers/gated_deltanet.py:234-253
 * followed by chunk_gated_delta_rule (:275-285), in one call that takes the projections
 * q_proj(h), k_proj(h), v_proj(h) instead of q, k, v.  Same result as
 * kairos_gdn_causal_conv1d_fwd on each projection, then kairos_gdn_chunk_fwd on the outputs
 * (use_qk_l2norm: q and k normalised as the op would).  At the Kairos layer's head dims
 * (K = 256, V a multiple of 64) the convolution runs where the forward stages its rows: k and q
 * in the prepare kernel, v in the recurrence's loader waves; q leaves prepare once, convolved
 * (and normalised), for the recurrence.  Other head dims convolve into the workspace first.
 * xq, xk: [B*T, H*K] bf16; xv: [B*T, H*V] bf16 (16-byte aligned); wq, wk: [H*K, 4],
 * wv: [H*V, 4] and biases bq, bk, bv ([D] or NULL) in w_dtype (fp32 or bf16); conv caches in
 * cq_in, ck_in, cv_in ([N, D, 4] bf16 or NULL = zeros) and out cq_out, ck_out, cv_out (the last
 * 4 entries of [cache, x] per sequence, NULL = not wanted, not aliasing the cache in).  The rest
 * as kairos_gdn_chunk_fwd with bf16 q/k/v; workspace from
 * kairos_gdn_chunk_fwd_conv_workspace_size.  No counterpart in the reference as one call: it
 * replaces the layer's three ShortConvolution calls and its chunk_gated_delta_rule call. */
size_t kairos_gdn_chunk_fwd_conv_workspace_size(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V,
                                                int64_t n_seqs, int use_qk_l2norm);
int kairos_gdn_chunk_fwd_conv(const void* xq, const void* xk, const void* xv, const void* wq, const void* wk,
                              const void* wv, const void* bq, const void* bk, const void* bv, const void* cq_in,
                              const void* ck_in, const void* cv_in, void* cq_out, void* ck_out, void* cv_out,
                              int w_dtype, const void* g, const void* beta, const void* initial_state, void* o,
                              float* final_state, const int64_t* cu_seqlens, int64_t n_seqs, int64_t B, int64_t T,
                              int64_t H, int64_t K, int64_t V, int g_dtype, int beta_dtype, int h0_dtype,
                              float scale, int use_qk_l2norm, void* workspace, size_t workspace_bytes,
                              void* stream);

/* Gates of the GatedDeltaNet layer (fla layers/gated_deltanet.py:265-271):
 * g = -exp(A_log) softplus(a + dt_bias) (fp32, softplus threshold 20) and
 * beta = sigmoid(b) in b's dtype, doubled when allow_neg_eigval.  a, b: [rows, HV]
 * (fp32 or bf16 each); A_log, dt_bias: [HV] in param_dtype; g: [rows, HV] fp32;
 * beta: [rows, HV] in b's dtype. */
int kairos_gdn_gates_fwd(const void* a, const void* b, const void* A_log, const void* dt_bias, float* g, void* beta,
                         int64_t rows, int64_t HV, int a_dtype, int b_dtype, int param_dtype, int allow_neg_eigval,
                         void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KAIROS_GDN_H */
