// Internal launch interface between the C-ABI layer (gdn_api.hip) and the
// kernel translation units.  Plain C++ structs of device pointers; no torch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kgdn {

enum : int { DT_F32 = 0, DT_BF16 = 1, DT_F8E4M3 = 2 };

// Shared addressing: fixed-length batches use (cu == nullptr, N = B, T = per-sequence
// length); varlen uses cu [N+1] (int64 token offsets) and chunk_off [N+1] (int32).
struct SeqArgs {
  const int64_t* cu;
  const int32_t* chunk_off;
  int N;
  int64_t T;
  int H;
};

constexpr int kConvW = 4;              // taps of the folded convolution (the layer's conv_size)

// A projection the op convolves (short causal convolution + SiLU, taps of width 4) as it stages its
// rows, the layer's prologue folded into the op's loads (gdn_conv.hpp): x [B*T, D] bf16 with D = H * Dh,
// taps w [D, 4] and bias b [D] (or nullptr) fp32 (the C ABI converts bf16 taps into its workspace),
// cache [N, D, 4] bf16 or nullptr.  x == nullptr: the op reads the tensor itself.
struct ConvIn {
  const void* x;
  const void* w;
  const void* b;
  const void* cache;
  int w_dtype;
  int D;
};

struct PrepareArgs {
  const void* k;          // [B*T, H, K]  k_dtype
  const void* v;          // [B*T, H, V]  compute dtype
  const void* g;          // [B*T, H]     g_dtype (0 fp32, 1 bf16)
  const void* beta;       // [B*T, H]     beta_dtype
  const float* k_scale;   // [H] dequant scale for fp8 k, else nullptr
  int g_dtype, beta_dtype;
  const int64_t* cu;
  const int32_t* chunk_off;
  int N;
  int64_t T;
  int H;
  float* gc;              // out [B*T, H] fp32
  void* w;                // out [B*T, H, K]
  void* uT;               // out [NC, H, V, 64]
  float* A_out;           // optional out [B*T, H, 64] fp32
  void* Ai_out;           // optional out [B*T, H, 64]
  const void* q;          // [B*T, H, K] (qk dtype), read only with aqk_out
  void* aqk_out;          // optional out [NC, H, 64, 64]: mask_{i>=j}(q k^T exp(gc_i - gc_j)) (compute dtype)
  float* beta_out;        // optional out [B*T, H] fp32 beta
  void* kT_out;           // optional out [NC, H, K, 64] k^T per chunk (compute dtype, zero past the chunk's end)
  void* wT_out;           // optional out [NC, H, K, 64] w^T per chunk (bf16 compute only, zero past the chunk's end)
  int64_t it0, it_span;   // it_span > 0 (cu == nullptr): only local chunks it0 .. it0 + it_span - 1 of each
                          // sequence, grid N * it_span (chunks past a sequence's end exit)
  // uT == nullptr: no u pass (v is not read)
  int l2;                 // the in-op L2 norm (the compact bf16 plan only): k rows normalised and rounded
                          // as they are staged, q rows of Aqk likewise
  float* qs_out;          // with l2 and aqk_out: out [B*T, H] fp32 rstd of each q row
  ConvIn ck, cq;          // with ck.x / cq.x (compact plan): k, q formed from their projections
  void* q_out;            // with cq.x: out [B*T, H, K] bf16 q as the recurrence reads it (convolved and, with
                          // l2, normalised)
};

struct FwdHArgs {
  const void* k;          // [B*T, H, K]  (k_dtype)
  const float* k_scale;   // [H] or nullptr
  const void* w;          // [B*T, H, K]
  const void* uT;         // [NC, H, V, 64]
  const float* gc;        // [B*T, H]
  const void* h0;         // [N, H, K, V] (h0_dtype) or nullptr
  int h0_dtype;
  const int64_t* cu;
  const int32_t* chunk_off;
  int N;
  int64_t T;
  int H;
  void* hT;               // out [NC, H, V, K] state snapshots (before each chunk)
  void* vnT;              // out [NC, H, V, 64] ungated v_new
  float* ht;              // out [N, H, K, V] fp32 or nullptr
  bool row_major;         // write the reference layouts instead: hT -> h [NC, H, K, V], vnT -> v_new [B*T, H, V]
};

struct FwdOArgs {
  const void* q;          // [B*T, H, K]  (qk_dtype)
  const void* k;
  const float* q_scale;   // [H] or nullptr
  const float* k_scale;
  const void* hT;         // [NC, H, V, K]
  const void* vnT;        // [NC, H, V, 64]
  const float* gc;        // [B*T, H]
  float scale;
  const int64_t* cu;
  const int32_t* chunk_off;
  int N;
  int64_t T;
  int H;
  void* o;                // out [B*T, H, V] compute dtype
};

// Fused recurrence + output for K = 256 (gdn_wide.hip), after launch_prepare without its u pass
// (gc, w, Ai, fp32 beta, Aqk and k^T); u = Ai bf16(beta v) is formed in the kernel.  bf16 q, k, w,
// u; V a multiple of 64.
struct WideFusedArgs {
  const void* q;          // [B*T, H, 256] bf16
  const void* kT;         // [NC, H, 256, 64] bf16 k^T per chunk (launch_prepare's kT_out)
  const void* v;          // [B*T, H, V] bf16
  const void* w;          // [B*T, H, 256] bf16
  const void* Ai;         // [B*T, H, 64] bf16 (I + A)^-1 rows (launch_prepare's Ai_out)
  const float* beta;      // [B*T, H] fp32 (launch_prepare's beta_out)
  const float* gc;        // [B*T, H]
  const void* aqk;        // [NC, H, 64, 64] bf16 (launch_prepare's aqk_out)
  const void* h0;         // [N, H, 256, V] (h0_dtype) or nullptr
  int h0_dtype;
  const int64_t* cu;
  const int32_t* chunk_off;
  int N;
  int64_t T;
  int H;
  float scale;
  void* o;                // out [B*T, H, V] bf16
  float* ht;              // out [N, H, 256, V] fp32 or nullptr
  int64_t it_begin, it_end;  // the chunks of each sequence to walk (it_end <= 0: to the end); h0 is the
                             // state before chunk it_begin, ht the one after the last chunk walked
  void* h_out;            // recompute mode (the backward's): out [NC, H, 256, V] bf16 state before each
                          // chunk, row-major; q, aqk and o are not used
  void* vn_out;           // recompute mode: out [B*T, H, V] bf16 v_new
  const float* qs;        // [B*T, H] fp32 rstd of the q rows (the in-op L2 norm: q is raw, k^T, w and Aqk
                          // come normalised from prepare), or nullptr
  ConvIn cv;              // with cv.x: v formed from its projection by the loader waves (v unused)
  // The layer's gated RMSNorm on o (fla modules/fused_norm_gate.py:42-127), with ngate: o is replaced
  // by y = bf16(o) rstd w [+ b] times g sigmoid(g) (or sigmoid(g)), rstd over the V columns of a token.
  // A token's row spans the V / 64 workgroups of its head, which exchange per-token sums of squares
  // through nss: entry ((chunk H + h) 64 + t) 8 + tile holds the sum in its low word and nepoch, the
  // call's tag, in its high word (no reset between calls; V <= 512).
  const void* ngate;      // [B*T, H, V] bf16, or nullptr (no norm)
  const void* nw;         // [V] in nw_dtype, or nullptr (ones)
  const void* nb;         // [V] in nw_dtype, or nullptr (zeros)
  int nw_dtype;
  float neps;
  int nsigmoid_only;
  unsigned long long* nss;  // [nss_chunks, H, 64, 8] tagged sums, then a 1 KB line that is written, never read
  int64_t nss_chunks;
  unsigned int nepoch;
};
// Bytes of WideFusedArgs::nss for nc chunks of H heads
inline size_t wide_norm_bytes(int64_t nc, int64_t H) { return (size_t)nc * H * 64 * 8 * 8 + 1024; }
bool wide_fused_supported(int compute_dtype, int qk_dtype, int K, int V);
int launch_wide_fused(const WideFusedArgs& a, int V, hipStream_t s);
// An empty one-workgroup kernel: a point in a stream's order that an event can mark.
int launch_marker(hipStream_t s);

// Per (chunk, head) record written by seg_prep and streamed by seg_trans and
// seg_out: the chunk inverse (I + A)^-1 rounded to bf16 [64][64] (row t holding
// columns in pcol order), then eight fp32 vectors of 64: gc, exp(gc) * scale,
// exp(gc), the update gate exp(gc_last - gc), beta, exp(gc_last) (repeated),
// and two unused.
constexpr int kSegRecordBytes = 64 * 64 * 2 + 8 * 64 * 4;

// Segment-parallel fused forward (gdn_seg.hip).  Sequences are cut into
// segments of L chunks; M is ns_grid * H blocks of K x K as a bf16 pair (hi, lo),
// R and s_init fp32 workspaces of ns_grid * H blocks of K x V.
struct SegFwdArgs {
  const void* q;          // [B*T, H, K]  (qk_dtype)
  const void* k;
  const void* v;          // [B*T, H, V]  compute dtype
  const void* g;          // [B*T, H]     g_dtype
  const void* beta;       // [B*T, H]     beta_dtype
  const float* q_scale;   // [H] (fp8 q/k) or nullptr
  const float* k_scale;
  int g_dtype, beta_dtype;
  const void* h0;         // [N, H, K, V] (h0_dtype) or nullptr
  int h0_dtype;
  const int64_t* cu;      // varlen: [N+1] token offsets, else nullptr
  const int32_t* chunk_off;
  const int32_t* seg_off; // varlen: [N+1] segment offsets
  int N;
  int64_t T;
  int H;
  int L;                  // chunks per segment
  int nseg_fixed;         // fixed length: segments per sequence
  int64_t ns_grid;        // number of segments (varlen: an upper bound)
  uint16_t* M;            // [ns_grid, H] blocks of K x K bf16 M_hi, then K x K bf16 M_lo (M = M_hi + M_lo)
  float* R;               // [ns_grid, H, K, V]
  float* s_init;          // [ns_grid, H, K, V]
  float scale;
  void* o;                // out [B*T, H, V]
  float* ht;              // out [N, H, K, V] or nullptr
  void* Ai;               // [nc_grid, H] chunk records of kSegRecordBytes (seg_prep -> seg_trans, seg_out)
  int64_t nc_grid;        // number of chunks (varlen: an upper bound)
  bool l2;                // the in-op L2 norm of q and k (bf16 q/k), folded into the kernels
  bool run_trans;         // some sequence has more than one segment
  bool run_combine;       // ... or final_state of empty sequences is needed
  bool skip_out;          // stop after the segment scan (s_init, M): the backward's recomputation
  hipEvent_t* events;     // optional [5]: recorded before seg_prep, seg_trans, seg_combine, seg_out and after seg_out
  // optional gated RMSNorm epilogue fused into the output (fla modules/fused_norm_gate.py:42-127, the
  // layer's o_norm): with gate set, o receives y = bf16(o) rstd w [+ b] times g sigmoid(g) (or sigmoid(g))
  const void* gate;       // [B*T, H, V] bf16, or nullptr (no epilogue)
  const void* nw;         // [V] (nw_dtype) or nullptr
  const void* nb;         // [V] (nw_dtype) or nullptr
  int nw_dtype;
  float eps;
  int sigmoid_only;
};

// Backward pass (gdn_bwd.hip), after the forward is recomputed by launch_prepare (gc, w, uT, Ai)
// and launch_fwd_h with row_major (h, v_new).  All token tensors are [B*T, H, *] in the compute
// dtype; q and k are the (normalised) operands the forward used.
struct BwdArgs {
  const void* q;          // [B*T, H, K]
  const void* k;          // [B*T, H, K]
  const void* v;          // [B*T, H, V]
  const float* gc;        // [B*T, H] chunk-local cumsum of g
  const void* beta;       // [B*T, H] beta_dtype
  int beta_dtype;
  const void* do_;        // [B*T, H, V] gradient of o
  const float* dht;       // [N, H, K, V] gradient of final_state, or nullptr (zero)
  const void* w;          // [B*T, H, K]
  const void* Ai;         // [B*T, H, 64] (I + A)^-1 rows
  const void* h;          // [NC, H, K, V] state snapshots
  const void* vn;         // [B*T, H, V] v_new
  void* dvl;              // [B*T, H, V] dv_local (scratch)
  void* dh;               // [NC, H, K, V] dh snapshots (scratch)
  void* dv2;              // [B*T, H, V] dv after the state recurrence (scratch)
  void* dw;               // [B*T, H, K] -dw as the reference stores it (scratch)
  void* dk1;              // [B*T, H, K] dk of chunk_bwd_dqkwg (scratch)
  float* dg1;             // [B*T, H] dg of chunk_bwd_dqkwg, before the cumsum (scratch)
  void* dq;               // out [B*T, H, K]
  void* dk;               // out [B*T, H, K]
  void* dv;               // out [B*T, H, V]
  float* dg;              // out [B*T, H]
  void* db;               // out [B*T, H] beta_dtype
  float* dh0;             // out [N, H, K, V] or nullptr
  void* qT;               // [NC, H, K, 64] q^T per chunk (zero past the chunk's end): written by the
                          // dv_local stage when set, read by the dh recurrence
  const void* wT;         // [NC, H, K, 64] w^T per chunk (zero past the chunk's end)
  // the in-op L2 norm's backward of q (l2norm.py:132-154) folded into the eight-wave dq / dk kernel:
  // rstd of each q row [B*T, H] from the forward norm pass, q above being the normalised rows; dq then
  // receives the gradient of the raw rows.  Null: dq is the gradient of the normalised rows.
  const float* rq;
  const int64_t* cu;
  const int32_t* chunk_off;
  int N;
  int64_t T;
  int H;
  float scale;
};
bool bwd_supported(int compute_dtype, int K, int V);
// whether the dq / dk / dw / dg stage runs the eight-wave kernel (the one that takes BwdArgs::rq)
bool bwd_dqk_wide(int compute_dtype, int K);
// stages: a mask of BWD_DVL (dv_local), BWD_DHU (the dh recurrence: dh, dv2, dh0; dh and dv2 may
// be null to skip their stores) and BWD_GRADS (dq, dk, dw, dg, then the WY backward: dq .. dbeta)
enum : int { BWD_DVL = 1, BWD_DHU = 2, BWD_GRADS = 4, BWD_ALL = 7 };
int launch_bwd(const BwdArgs& a, int compute_dtype, int K, int V, int64_t nc_grid, int stages, hipStream_t s);
// the dh recurrence for K = 256 in bf16 with 64 value columns per workgroup (needs qT, wT, dh and dv2)
bool wide_dhu_supported(int compute_dtype, int K, int V);
int launch_wide_dhu(const BwdArgs& a, int V, hipStream_t s);
// dq, dk, dw, dg for K = 128 or 256 in bf16, eight waves per (chunk, head) (V a multiple of 64)
int launch_wide_dqkwg(const BwdArgs& a, int K, int V, int64_t nc_grid, hipStream_t s);
int launch_l2norm_bwd(const void* x, const void* dy, void* dx, int dtype, int64_t rows, int D, hipStream_t s);

// Each returns 0 on success, -1 on a HIP launch error, -2 for an unsupported
// (dtype, K, V) combination.
int launch_prepare(const PrepareArgs& a, int compute_dtype, int k_dtype, int K, int V, int64_t nc_grid,
                   hipStream_t s);
int launch_fwd_h(const FwdHArgs& a, int compute_dtype, int k_dtype, int K, int V, hipStream_t s);
int launch_fwd_o(const FwdOArgs& a, int compute_dtype, int qk_dtype, int K, int V, int64_t nc_grid,
                 hipStream_t s);
bool seg_fwd_supported(int compute_dtype, int K, int V);
// Layout moves of the reference-layout stage entry points (gdn_layout.hip): token rows
// [B*T, H, D] <-> per-chunk transposed tiles [NCb, H, D, 64] (to_tiles selects the
// direction), and per-chunk states [NCb, H, R, S] -> [NCb, H, S, R].  D, R, S multiples of 64.
int launch_chunk_tiles(const void* src, void* dst, int to_tiles, int elem_bytes, const int64_t* cu,
                       const int32_t* chunk_off, int N, int64_t T, int H, int D, int64_t nc_grid, hipStream_t s);
int launch_state_tiles(const void* src, void* dst, int elem_bytes, const int64_t* cu, const int32_t* chunk_off, int N,
                       int64_t T, int H, int R, int S, int64_t nc_grid, hipStream_t s);
int launch_seg_fwd(const SegFwdArgs& a, int compute_dtype, int qk_dtype, int K, int V, hipStream_t s);
int launch_seg_map(const int64_t* cu, int N, int L, int32_t* chunk_off, int32_t* seg_off, hipStream_t s);
// Segments as sequences for the stage kernels (the backward), from the geometry fields of a
// SegFwdArgs (cu, chunk_off, seg_off, N, T, H, L, nseg_fixed, ns_grid, M):
// seg_cu [ns_grid + 1] token and seg_coff [ns_grid + 1] chunk offsets of the segments;
int launch_seg_seq_map(const SegFwdArgs& p, int64_t* seg_cu, int32_t* seg_coff, hipStream_t s);
// dst [ns_grid, H, K, V] fp32 = src [N, H, K, V] at the first (first_seg) or last segment of each
// sequence (src == nullptr: zeros), zeros at the other segments (left alone with first_seg);
int launch_seg_place(const SegFwdArgs& p, const void* src, int src_dtype, float* dst, int K, int V, bool first_seg,
                     hipStream_t s);
// the reverse scan of dh over segments with the transposed maps M_j^T: Bseg [ns_grid, H, K, V] holds
// each segment's dh recurrence from zero (the last segment's: from dht), dht [N, H, K, V] (or null)
// the final-state gradient; writes
// F [ns_grid, H, K, V], the dh each segment's last chunk starts from, and dh0 [N, H, K, V] (or null).
int launch_seg_bwd_combine(const SegFwdArgs& p, const float* Bseg, const float* dht, float* F, float* dh0, int K,
                           int V, hipStream_t s);
int launch_l2norm(const void* x, void* y, float* rstd, int dtype, int64_t rows, int D, hipStream_t s);
// the same for two tensors of equal shape in one launch (x1, y1 may be null), rstd of each row into
// r0 / r1 where not null
int launch_l2norm2(const void* x0, void* y0, const void* x1, void* y1, int dtype, int64_t rows, int D,
                   hipStream_t s, float* r0 = nullptr, float* r1 = nullptr);

// Gated RMSNorm (gdn_norm.hip): y = x rstd w [+ b] * act(g) per row of D.
struct NormArgs {
  const void* x;          // [rows, D] x_dtype
  const void* g;          // [rows, D] g_dtype
  const void* w;          // [D] w_dtype or nullptr
  const void* b;          // [D] w_dtype or nullptr
  void* y;                // [rows, D] x_dtype
  float* rstd;            // [rows] or nullptr
  int x_dtype, g_dtype, w_dtype;
  int64_t rows;
  int D;
  float eps;
  int sigmoid_only;       // 0: y *= g sigmoid(g) (swish / silu); 1: y *= sigmoid(g)
};
int launch_rmsnorm_gated(const NormArgs& a, hipStream_t s);

// Token-by-token gated delta rule (gdn_recurrent.hip), fused_recurrent.py:21-135.
struct RecArgs {
  const void* q;          // [B*T, H, K]  qk_dtype
  const void* k;
  const void* v;          // [B*T, HV, V] v_dtype
  const void* g;          // [B*T, HV] g_dtype or nullptr
  const void* gk;         // [B*T, HV, K] gk_dtype or nullptr
  const void* gv;         // [B*T, HV, V] gv_dtype or nullptr
  const void* beta;       // [B*T, HV] (headwise) or [B*T, HV, V], beta_dtype; nullptr = ones
  const void* h0;         // [N, HV, K, V] h0_dtype or nullptr
  void* o;                // out [B*T, HV, V] v_dtype
  float* ht;              // out [N, HV, K, V] fp32 or nullptr
  const int64_t* cu;      // varlen [N+1] or nullptr
  int64_t T;              // tokens per sequence (fixed length)
  int N, H, HV, K, V;
  int qk_dtype, v_dtype, g_dtype, gk_dtype, gv_dtype, beta_dtype, h0_dtype;
  int beta_headwise;
  int l2;
  float scale;
};
int launch_fused_recurrent(const RecArgs& a, hipStream_t s);

// Short causal convolution (gdn_prologue.hip), causal_conv1d_fwd of fla modules/convolution.py.
struct ConvArgs {
  const void* x;          // [B*T, D] x_dtype
  void* y;                // [B*T, D] x_dtype
  const void* w;          // [D, W] w_dtype
  const void* bias;       // [D] w_dtype or nullptr
  const void* h0;         // cache in [N, D, W] x_dtype or nullptr
  void* ht;               // cache out [N, D, W] x_dtype or nullptr
  const int64_t* cu;      // varlen [N+1] or nullptr
  int64_t T;              // tokens per sequence (fixed length)
  int64_t total_tokens;   // B*T
  int N, D, W;
  int x_dtype, w_dtype;
  int silu;               // apply y * sigmoid(y)
  int head_lanes;         // 0, or hd / 8: L2-normalise the rounded y per head of hd channels
};
int launch_conv1d(const ConvArgs& a, hipStream_t s);
int launch_conv_state(const ConvArgs& a, hipStream_t s);   // the final cache only
int launch_to_f32(const void* src, int dtype, float* dst, int64_t n, hipStream_t s);

// GatedDeltaNet gates (gdn_prologue.hip), layers/gated_deltanet.py:265-271.
struct GateArgs {
  const void* a;          // [rows, HV] a_dtype
  const void* b;          // [rows, HV] b_dtype
  const void* A_log;      // [HV] p_dtype
  const void* dt_bias;    // [HV] p_dtype
  float* g;               // out [rows, HV] fp32
  void* beta;             // out [rows, HV] b_dtype
  int64_t rows;
  int HV;
  int a_dtype, b_dtype, p_dtype;
  int neg_eigval;
};
int launch_gates(const GateArgs& a, hipStream_t s);
int launch_chunk_offsets(const int64_t* cu, int N, int32_t* chunk_off, hipStream_t s);
int launch_cumsum(const void* g, int g_dtype, float* gc, const int64_t* cu, const int32_t* chunk_off, int N,
                  int64_t T, int H, int64_t nc_grid, hipStream_t s);

}  // namespace kgdn
