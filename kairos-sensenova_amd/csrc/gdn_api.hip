// C ABI of the chunked GatedDeltaNet forward (declared in include/kairos_gdn.h):
// argument validation, workspace carving and kernel orchestration.
//
// kairos_gdn_chunk_fwd computes chunk_gated_delta_rule_fwd (fla
// ops/gated_delta_rule/chunk.py:16-67) with the segment-parallel fused kernels
// of gdn_seg.hip:
//   [l2norm q, k] -> [segment map] -> seg_trans (per-segment [M | R])
//                 -> seg_combine (segment initial states) -> seg_out (o, ht)
// The stage entry points (kairos_gdn_prepare_wy, _fwd_h, _fwd_o, ...) run
// one reference stage each with the stage kernels and the reference's
// intermediate tensors.
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <ctime>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/kairos_gdn.h"
#include "gdn_common.hpp"
#include "gdn_kernels.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return KAIROS_GDN_OK;
}

int from_launch(int rc, const char* what) {
  if (rc == 0) return KAIROS_GDN_OK;
  if (rc == -2) return fail(KAIROS_GDN_EUNSUPPORTED, "%s: dtype / head-dim combination is not built", what);
  return fail(KAIROS_GDN_EHIP, "%s: HIP launch failed: %s", what, hipGetErrorString(hipGetLastError()));
}

constexpr size_t kAlign = 256;
size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }
size_t dt_size(int dt) { return dt == KAIROS_GDN_F32 ? 4 : dt == KAIROS_GDN_BF16 ? 2 : 1; }
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int64_t chunks_bound(int64_t B, int64_t T, int64_t n_seqs) {
  if (n_seqs > 0) return T / kgdn::C + n_seqs;
  return B * ((T + kgdn::C - 1) / kgdn::C);
}

struct Geometry {
  int64_t B, T, H, K, V, n_seqs, N, nc;
  bool varlen;
};

int check_geometry(Geometry& G, const int64_t* cu, int64_t n_seqs, int64_t B, int64_t T, int64_t H, int64_t K,
                   int64_t V, const char* what) {
  if (B <= 0 || T < 0 || H <= 0 || K <= 0 || V <= 0)
    return fail(KAIROS_GDN_EINVAL, "%s: invalid shape B=%lld T=%lld H=%lld K=%lld V=%lld", what, (long long)B,
                (long long)T, (long long)H, (long long)K, (long long)V);
  if (K > 256) return fail(KAIROS_GDN_EINVAL, "%s: head dimension K=%lld is larger than 256", what, (long long)K);
  if ((cu == nullptr) != (n_seqs == 0))
    return fail(KAIROS_GDN_EINVAL, "%s: cu_seqlens and n_seqs must be given together", what);
  if (n_seqs < 0) return fail(KAIROS_GDN_EINVAL, "%s: n_seqs must be >= 0", what);
  if (cu && B != 1)
    return fail(KAIROS_GDN_EINVAL, "%s: the batch size is expected to be 1 rather than %lld when using cu_seqlens",
                what, (long long)B);
  if (H > 65535) return fail(KAIROS_GDN_EINVAL, "%s: H=%lld exceeds the grid limit", what, (long long)H);
  G.B = B; G.T = T; G.H = H; G.K = K; G.V = V;
  G.n_seqs = n_seqs;
  G.varlen = cu != nullptr;
  G.N = G.varlen ? n_seqs : B;
  G.nc = chunks_bound(B, T, n_seqs);
  if (G.nc > 0x7fffffff) return fail(KAIROS_GDN_EINVAL, "%s: too many chunks", what);
  return KAIROS_GDN_OK;
}

// compute dtype of a (q/k, v) pair: bf16 path for bf16 v with bf16/fp8 q,k; fp32 for all-fp32.
int compute_dtype(int qk_dtype, int v_dtype) {
  if (v_dtype == KAIROS_GDN_BF16 && (qk_dtype == KAIROS_GDN_BF16 || qk_dtype == KAIROS_GDN_F8E4M3))
    return KAIROS_GDN_BF16;
  if (v_dtype == KAIROS_GDN_F32 && qk_dtype == KAIROS_GDN_F32) return KAIROS_GDN_F32;
  return -1;
}

bool valid_scalar_dt(int dt) { return dt == KAIROS_GDN_F32 || dt == KAIROS_GDN_BF16; }

// Workspace carving helper.
struct Carver {
  char* base;
  size_t off = 0;
  void* take(size_t bytes) {
    void* p = base ? base + off : nullptr;
    off += align_up(bytes);
    return p;
  }
};

// Build the varlen chunk map into the workspace (no-op for fixed length).
int chunk_map(const Geometry& G, const int64_t* cu, Carver& cv, const int32_t** out, hipStream_t s) {
  *out = nullptr;
  if (!G.varlen) return KAIROS_GDN_OK;
  int32_t* off = static_cast<int32_t*>(cv.take(sizeof(int32_t) * (G.N + 1)));
  *out = off;
  return from_launch(kgdn::launch_chunk_offsets(cu, (int)G.N, off, s), "chunk map");
}

size_t stage_ws(int64_t n_seqs) { return n_seqs > 0 ? align_up(sizeof(int32_t) * (n_seqs + 1)) : 0; }

// Compute units of the current device (queried once; 256, the MI355X count, without a device).
int device_cus() {
  static int cached = 0;
  if (cached > 0) return cached;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
    (void)hipGetLastError();
    cus = 256;
  }
  cached = cus;
  return cached;
}

// Segment plan of the fused forward: L chunks per segment, chosen so that the
// (segment, head) work items of the longest-running kernels fill the compute
// units once (one 4-wave workgroup per CU).  KAIROS_GDN_SEG_CHUNKS overrides L.
struct SegPlan {
  int L;
  int nseg_fixed;     // fixed length: segments per sequence
  int64_t ns;         // segments (varlen: upper bound)
  bool trans, combine;
};

SegPlan plan_segments(int64_t B, int64_t T, int64_t H, int64_t n_seqs) {
  SegPlan P{1, 0, 0, false, false};
  const int64_t cus = device_cus();
  int64_t L_env = 0;
  if (const char* e = std::getenv("KAIROS_GDN_SEG_CHUNKS")) L_env = std::atoll(e);
  if (n_seqs == 0) {
    const int64_t nc = (T + kgdn::C - 1) / kgdn::C;
    if (nc == 0) {
      P.combine = true;         // final_state of empty sequences = initial_state
      return P;
    }
    int64_t L;
    if (L_env > 0) {
      L = L_env;
    } else {
      const int64_t target = std::max<int64_t>(1, cus / std::max<int64_t>(1, B * H));
      const int64_t nseg = std::min(nc, target);
      L = (nc + nseg - 1) / nseg;
    }
    P.L = (int)std::min<int64_t>(L, 1 << 20);
    P.nseg_fixed = (int)((nc + P.L - 1) / P.L);
    P.ns = B * P.nseg_fixed;
    P.trans = P.combine = P.nseg_fixed > 1;
    return P;
  }
  const int64_t cb = T / kgdn::C + n_seqs;       // bound on the total chunk count
  int64_t L;
  if (L_env > 0) {
    L = L_env;
  } else {
    const int64_t free_slots = std::max<int64_t>(cus - n_seqs * H, cus / 2);
    L = std::max<int64_t>(1, (cb * H + free_slots - 1) / free_slots);
  }
  P.L = (int)std::min<int64_t>(L, 1 << 20);
  P.ns = cb / P.L + n_seqs;                      // sum_n ceil(nc_n / L) <= cb / L + N
  P.trans = P.combine = true;
  return P;
}

size_t seg_ws(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int64_t n_seqs, const SegPlan& P) {
  size_t total = n_seqs > 0 ? 2 * align_up(sizeof(int32_t) * (n_seqs + 1)) : 0;
  // chunk records: bf16 inverse [64][64] + chunk vectors, per (chunk, head)
  total += align_up((size_t)chunks_bound(B, T, n_seqs) * H * kgdn::kSegRecordBytes);
  if (P.trans || P.combine) {
    const size_t blocks = (size_t)P.ns * H;
    total += align_up(blocks * K * K * sizeof(float));        // M
    total += align_up(blocks * K * V * sizeof(float));        // R
    total += align_up(blocks * K * V * sizeof(float));        // segment initial states
  }
  return total;
}

// Kernel timing of kairos_gdn_chunk_fwd (kairos_gdn_profile_begin / _end): while
// enabled, every fused call records kProfEvents hipEvents on its stream around
// its kProfKernels kernels (seg_prep, seg_trans, seg_combine, seg_out).
constexpr int kProfKernels = 4;
constexpr int kProfEvents = kProfKernels + 1;
struct Profile {
  std::mutex mu;
  bool on = false;
  std::vector<hipEvent_t> pool;   // kProfEvents per recorded call
  size_t used = 0;
};
Profile& profile() {
  static Profile p;
  return p;
}
// Next set of kProfEvents events while profiling is on, else nullptr.
hipEvent_t* profile_events() {
  Profile& P = profile();
  std::lock_guard<std::mutex> lk(P.mu);
  if (!P.on) return nullptr;
  if (P.used + kProfEvents > P.pool.size()) {
    for (int i = 0; i < kProfEvents; ++i) {
      hipEvent_t e;
      if (hipEventCreate(&e) != hipSuccess) return nullptr;
      P.pool.push_back(e);
    }
  }
  hipEvent_t* ev = P.pool.data() + P.used;
  P.used += kProfEvents;
  return ev;
}

// Whether the staged path runs the fused K = 256 recurrence + output (bf16 q/k, V a multiple of 64)
// instead of fwd_h + fwd_o.  KAIROS_GDN_WIDE_FUSED=0 keeps the two stage kernels.
bool use_wide_fused(int cdt, int qk_dtype, int64_t K, int64_t V) {
  if (!kgdn::wide_fused_supported(cdt, qk_dtype, (int)K, (int)V)) return false;
  const char* e = std::getenv("KAIROS_GDN_WIDE_FUSED");
  return !(e && e[0] == '0' && e[1] == 0);
}

// Workspace of the staged path (stage kernels with the reference's intermediates; the fused K = 256
// form keeps the state snapshots and v_new on chip and adds the per-chunk Aqk instead).
size_t staged_ws(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int64_t n_seqs, int cdt, bool wide,
                 bool l2) {
  const size_t es = cdt == KAIROS_GDN_F32 ? 4 : 2;
  const size_t nc = (size_t)chunks_bound(B, T, n_seqs);
  const size_t tok = (size_t)(B * T * H);
  size_t total = stage_ws(n_seqs);
  total += align_up(tok * sizeof(float));                 // gc
  total += align_up(tok * K * es);                        // w
  if (wide) {
    total += align_up(nc * H * kgdn::C * kgdn::C * es);   // Aqk
    total += align_up(tok * kgdn::C * es);                // Ai
    total += align_up(tok * sizeof(float));               // beta (fp32)
    total += align_up(nc * H * K * kgdn::C * es);         // k^T per chunk
    total += align_up((size_t)(n_seqs > 0 ? n_seqs : B) * H * K * V * sizeof(float));   // state between parts
    if (l2) total += align_up(tok * sizeof(float));       // rstd of the q rows (the in-op L2 norm, folded)
  } else {
    total += align_up(nc * H * V * kgdn::C * es);         // uT
    total += align_up(nc * H * V * K * es);               // hT
    total += align_up(nc * H * V * kgdn::C * es);         // vnT
  }
  return total;
}

// The backward's segment scan (bf16, K and V in {64, 128}, more than one segment somewhere): the
// recomputed states and the dh recurrence run per segment of the forward's plan, from the states a
// scan over segments supplies (the forward's segment maps M_j and, in reverse, their transposes), so
// the serial chains are L chunks long instead of a whole sequence.  KAIROS_GDN_BWD_SEG=0 keeps the
// sequence-long recurrences.
bool bwd_segmented(int cdt, int64_t K, int64_t V, const SegPlan& P) {
  if (!kgdn::seg_fwd_supported(cdt, (int)K, (int)V) || !P.trans || P.ns <= 0) return false;
  const char* e = std::getenv("KAIROS_GDN_BWD_SEG");
  return !(e && e[0] == '0' && e[1] == 0);
}

// The dh recurrence for K = 256 in bf16 with 64 value columns per workgroup (KAIROS_GDN_BWD_DHU_WIDE=0
// selects the 16-column form); it reads q^T and w^T per chunk from the workspace.
bool wide_dhu_on(int cdt, int64_t K, int64_t V) {
  if (!kgdn::wide_dhu_supported(cdt, (int)K, (int)V)) return false;
  const char* e = std::getenv("KAIROS_GDN_BWD_DHU_WIDE");
  return !(e && e[0] == '0' && e[1] == 0);
}

// The backward's recompute of h and v_new at K = 256 in bf16 by the fused forward kernel in its
// recompute mode (KAIROS_GDN_BWD_RC_WIDE=0 selects prepare's u pass and fwd_h): prepare then writes
// k^T per chunk (into the q^T buffer, which the dv_local stage fills later) and fp32 beta (into dg1,
// which the dq/dk stage fills later), and no u.
bool bwd_rc_wide(int cdt, int qk_dtype, int64_t K, int64_t V, bool segmented) {
  if (segmented || !kgdn::wide_fused_supported(cdt, qk_dtype, (int)K, (int)V)) return false;
  const char* e = std::getenv("KAIROS_GDN_BWD_RC_WIDE");
  return !(e && e[0] == '0' && e[1] == 0);
}

// Workspace of the backward: the recomputed forward (gc, w, u, Ai, h, v_new) and the
// backward's own intermediates (dv_local, dh, dv2, -dw, dk of the dq/dk stage, dg before the
// cumsum), plus the normalised q, k and their pre-norm gradients with the in-op L2 norm.  The
// segment scan adds the forward's chunk records and segment maps and states, and the segments'
// token and chunk offsets.
size_t bwd_ws(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int64_t n_seqs, int cdt, int qk_dtype,
              int use_l2) {
  const size_t es = cdt == KAIROS_GDN_F32 ? 4 : 2;
  const size_t nc = (size_t)chunks_bound(B, T, n_seqs);
  const size_t tok = (size_t)(B * T * H);
  size_t total = stage_ws(n_seqs);
  const SegPlan P = plan_segments(B, T, H, n_seqs);
  if (bwd_segmented(cdt, K, V, P)) {
    total += stage_ws(n_seqs);                                     // seg_off
    total += align_up(nc * H * kgdn::kSegRecordBytes);            // chunk records
    const size_t blocks = (size_t)P.ns * H;
    total += align_up(blocks * K * K * sizeof(float));            // M (bf16 hi, lo)
    total += 2 * align_up(blocks * K * V * sizeof(float));        // R, then F; s_init, then B
    total += align_up((P.ns + 1) * sizeof(int64_t)) + align_up((P.ns + 1) * sizeof(int32_t));
  }
  total += 2 * align_up(tok * sizeof(float));            // gc, dg1
  total += 3 * align_up(tok * K * es);                   // w, -dw, dk1
  const bool seg = bwd_segmented(cdt, K, V, P);
  const bool rc_wide = bwd_rc_wide(cdt, qk_dtype, K, V, seg);
  if (!rc_wide) total += align_up(nc * H * V * kgdn::C * es);   // uT
  total += align_up(tok * kgdn::C * es);                 // Ai
  total += 2 * align_up(nc * H * K * V * es);            // h, dh
  total += 3 * align_up(tok * V * es);                   // v_new, dv_local, dv2
  if (use_l2) {                                          // qn, kn, dkn, rstd of q, and dqn where the
    total += 3 * align_up(tok * K * es) + align_up(tok * sizeof(float));         // dq kernel does not
    if (!kgdn::bwd_dqk_wide(cdt, (int)K)) total += align_up(tok * K * es);      // take q's norm backward
  }
  if (!seg && kgdn::wide_dhu_supported(cdt, (int)K, (int)V))
    total += 2 * align_up(nc * H * K * kgdn::C * es);    // q^T (k^T first with rc_wide), w^T per chunk
  else if (rc_wide)
    total += align_up(nc * H * K * kgdn::C * es);        // k^T per chunk
  return total;
}

// Staged forward: prepare (gc, w, u) -> fwd_h (h, v_new, ht) -> fwd_o (o), the
// reference's stage order with its intermediates in the workspace.  Used for the
// shapes the fused kernels do not cover: fp32, and the Kairos model's head dims
// K = 256, V = 512 (any K in {64, 128, 256} with V a multiple of 16).
// The pipelined form of the fused K = 256 path: the chunks of every sequence are cut into P parts
// (4 by default, growing by 1.4 along the sequence);
// the prepare kernel of part p + 1 runs on a second stream while the recurrence walks part p (whose
// 64-column workgroups leave CUs idle: 160 of 256 at the Kairos layer shape), the state passing
// between parts through an fp32 buffer.  KAIROS_GDN_WIDE_PIPE sets P (1: one prepare, then one
// recurrence); fixed-length sequences only.  Part 0's prepare runs on the caller's stream (the whole
// GPU), the later prepares on a second stream and the recurrence parts on a third.  Prepare p + 1
// waits for an event recorded just before recurrence part p (wide_mark_mode), so the recurrence's
// workgroups are dispatched first and the prepare fills the CUs they leave (were both ready at once,
// the prepare's 10^4 workgroups could take every CU and hold the recurrence back).  The caller's
// stream waits for the last recurrence part.
constexpr int kMaxParts = 16;

int wide_pipe_parts() {
  const char* e = std::getenv("KAIROS_GDN_WIDE_PIPE");
  if (e == nullptr) return 4;
  const int p = std::atoi(e);
  return p < 1 ? 1 : p > kMaxParts ? kMaxParts : p;
}

// Part sizes grow by this factor (KAIROS_GDN_WIDE_PIPE_GROWTH; 1 = equal parts): part 0's prepare
// runs alone, so a smaller first part shortens the call as long as each later part's prepare, on
// the CUs the recurrence leaves, still finishes within the previous recurrence part.
double wide_pipe_growth() {
  const char* e = std::getenv("KAIROS_GDN_WIDE_PIPE_GROWTH");
  if (e == nullptr) return 1.4;
  const double g = std::atof(e);
  return g < 0.25 ? 0.25 : g > 4.0 ? 4.0 : g;
}

// Chunk boundaries of P parts of nt chunks with sizes growing by `growth`: b[0] = 0, b[P] = nt, every
// part at least one chunk (nt >= P)
void wide_pipe_bounds(int64_t nt, int P, double growth, int64_t* b) {
  double tot = 0.0, wsum = 0.0;
  for (int p = 0; p < P; ++p) tot += std::pow(growth, p);
  b[0] = 0;
  for (int p = 1; p < P; ++p) {
    wsum += std::pow(growth, p - 1);
    int64_t x = (int64_t)std::llround((double)nt * wsum / tot);
    x = std::max<int64_t>(x, b[p - 1] + 1);
    x = std::min<int64_t>(x, nt - (P - p));
    b[p] = x;
  }
  b[P] = nt;
}

std::mutex g_aux_mu;                                     // held while a pipelined call enqueues its work
hipStream_t g_aux_stream[64][4] = {};
hipEvent_t g_aux_events[64][3 * kMaxParts + 4] = {};   // + 4 join events

// What releases prepare p + 1 (KAIROS_GDN_WIDE_PIPE_MARK): 0, a one-workgroup marker kernel on the
// recurrence stream just before part p; 1, that marker on a stream of its own once recurrence part
// p - 1 has finished, beside the dispatch of part p; 2 (default), an event recorded on the
// recurrence stream just before part p (no kernel: the recurrence parts follow each other directly).
// At the Kairos layer shape 1 and 2 measure alike, 0 about 10 us slower per call.
int wide_mark_mode() {
  const char* e = std::getenv("KAIROS_GDN_WIDE_PIPE_MARK");
  if (e == nullptr) return 2;
  const int m = std::atoi(e);
  return m < 0 || m > 2 ? 2 : m;
}

// The four streams (prepares, recurrence parts, markers, the per-part gated norm) and the events of
// the current device, created on first use and kept until the process ends (a recorded event may be
// recorded again: waits already enqueued keep the record they saw).  Call with g_aux_mu held.
int aux_streams(hipStream_t* sp, hipStream_t* sr, hipStream_t* sm, hipStream_t* sn, hipEvent_t** events) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return -1;
  if (g_aux_events[dev][0] == nullptr) {
    for (int p = 0; p < 3 * kMaxParts + 4; ++p)
      if (hipEventCreateWithFlags(&g_aux_events[dev][p], hipEventDisableTiming) != hipSuccess) return -1;
  }
  *events = g_aux_events[dev];
  if (g_aux_stream[dev][0] == nullptr) {
    hipStream_t st[4] = {nullptr, nullptr, nullptr, nullptr};
    for (int j = 0; j < 4; ++j)
      if (hipStreamCreateWithFlags(&st[j], hipStreamNonBlocking) != hipSuccess) return -1;
    for (int j = 0; j < 4; ++j) g_aux_stream[dev][j] = st[j];
  }
  *sp = g_aux_stream[dev][0];
  *sr = g_aux_stream[dev][1];
  *sm = g_aux_stream[dev][2];
  *sn = g_aux_stream[dev][3];
  return 0;
}

// The layer's gated RMSNorm applied to the forward's output (kairos_gdn_chunk_fwd_gated_norm)
struct NormEpilogue {
  const void* gate;
  const void* w;
  const void* b;
  int gate_dtype;
  int w_dtype;
  float eps;
  int sigmoid_only;
};

// Rows [row0, row0 + rows) of y replaced by their gated RMSNorm, in place (each element is read and
// written by the same lane)
int norm_in_place(void* y, int y_dtype, const NormEpilogue& e, int64_t rows, int64_t D, hipStream_t s,
                  int64_t row0 = 0) {
  if (rows == 0) return 0;
  char* yp = static_cast<char*>(y) + row0 * D * (int64_t)dt_size(y_dtype);
  const char* gp = static_cast<const char*>(e.gate) + row0 * D * (int64_t)dt_size(e.gate_dtype);
  kgdn::NormArgs na{yp, gp, e.w, e.b, yp, nullptr, y_dtype, e.gate_dtype, e.w_dtype, rows, (int)D, e.eps,
                    e.sigmoid_only};
  return from_launch(kgdn::launch_rmsnorm_gated(na, s), "gated RMSNorm epilogue");
}

// Whether the pipelined K = 256 forward applies the gated norm by parts (KAIROS_GDN_NORM_PARTS=0: one
// pass over all rows after the forward): the rows of every part but the last on a library stream of
// their own beside the last recurrence part (when no prepare runs any more), the last part's after it.
// Measured at the Kairos layer shape with the in-op L2 norm: 1.83 against 1.88 ms; each part's rows
// released as soon as that part is done (competing with the prepares) 2.09 ms.
bool norm_parts_on() {
  const char* e = std::getenv("KAIROS_GDN_NORM_PARTS");
  return !(e && e[0] == '0' && e[1] == 0);
}

int run_staged(const Geometry& G, const void* q, const void* k, const void* v, const void* g, const void* beta,
               const float* q_scale, const float* k_scale, const void* h0, int h0_dtype, void* o, float* ht,
               const int64_t* cu_seqlens, int qk_dtype, int cdt, int g_dtype, int beta_dtype, float scale,
               Carver& cv, hipStream_t s, bool may_fork, bool l2 = false,
               const kgdn::ConvIn* conv3 = nullptr, const kgdn::WideFusedArgs* wnorm = nullptr,
               const NormEpilogue* epi = nullptr, int y_dtype = 0, bool* epi_done = nullptr) {
  const size_t es = cdt == KAIROS_GDN_F32 ? 4 : 2;
  const size_t tok = (size_t)(G.B * G.T * G.H);
  const int K = (int)G.K, V = (int)G.V, H = (int)G.H;
  const int32_t* chunk_off = nullptr;
  if (int rc = chunk_map(G, cu_seqlens, cv, &chunk_off, s)) return rc;
  float* gc = static_cast<float*>(cv.take(tok * sizeof(float)));
  void* w = cv.take(tok * K * es);
  const bool wide = use_wide_fused(cdt, qk_dtype, G.K, G.V);
  void* uT = nullptr;
  void* hT = nullptr;
  void* vnT = nullptr;
  void* aqk = nullptr;
  void* ai = nullptr;
  float* bf = nullptr;
  void* kt = nullptr;
  float* st = nullptr;
  if (wide) {
    aqk = cv.take((size_t)G.nc * H * kgdn::C * kgdn::C * es);
    ai = cv.take(tok * kgdn::C * es);
    bf = static_cast<float*>(cv.take(tok * sizeof(float)));
    kt = cv.take((size_t)G.nc * H * K * kgdn::C * es);
    st = static_cast<float*>(cv.take((size_t)G.N * H * K * V * sizeof(float)));
  } else if (l2) {
    return fail(KAIROS_GDN_EINVAL, "the in-op L2 norm is folded only into the fused K = 256 form");
  } else {
    uT = cv.take((size_t)G.nc * H * V * kgdn::C * es);
    hT = cv.take((size_t)G.nc * H * V * K * es);
    vnT = cv.take((size_t)G.nc * H * V * kgdn::C * es);
  }
  const int N = (int)G.N;
  kgdn::PrepareArgs pa{};
  pa.k = k; pa.v = v; pa.g = g; pa.beta = beta; pa.k_scale = k_scale;
  pa.g_dtype = g_dtype; pa.beta_dtype = beta_dtype;
  pa.cu = cu_seqlens; pa.chunk_off = chunk_off; pa.N = N; pa.T = G.T; pa.H = H;
  pa.gc = gc; pa.w = w; pa.uT = uT; pa.A_out = nullptr; pa.Ai_out = ai;
  pa.q = q; pa.aqk_out = aqk; pa.beta_out = bf;          // the fused K = 256 form: Aqk, Ai, beta, k^T, no u
  pa.kT_out = kt;
  // the in-op L2 norm folded into prepare; without the folded convolution the recurrence reads raw q
  // and scales q h by the rstd prepare records, with it prepare writes q normalised
  float* qs = (wide && l2 && conv3 == nullptr) ? static_cast<float*>(cv.take(tok * sizeof(float))) : nullptr;
  pa.l2 = wide && l2;
  pa.qs_out = qs;
  void* q_conv = nullptr;
  if (conv3) {                                            // the layer's prologue folded in (K = 256 form only)
    if (!wide) return fail(KAIROS_GDN_EINVAL, "the convolution is folded only into the fused K = 256 form");
    q_conv = cv.take(tok * K * es);
    pa.cq = conv3[0];
    pa.ck = conv3[1];
    pa.q_out = q_conv;
  }
  kgdn::WideFusedArgs fa{};
  fa.q = q; fa.kT = kt; fa.v = v; fa.w = w; fa.Ai = ai; fa.beta = bf; fa.gc = gc; fa.aqk = aqk;
  fa.h0 = h0; fa.h0_dtype = h0_dtype;
  fa.cu = cu_seqlens; fa.chunk_off = chunk_off; fa.N = N; fa.T = G.T; fa.H = H;
  fa.scale = scale; fa.o = o; fa.ht = ht;
  fa.qs = qs;
  if (conv3) {
    fa.q = q_conv;
    fa.cv = conv3[2];
  }
  if (wnorm) {                                            // the gated norm in place of the o stores
    if (!wide) return fail(KAIROS_GDN_EINVAL, "the gated norm is folded only into the fused K = 256 form");
    fa.ngate = wnorm->ngate; fa.nw = wnorm->nw; fa.nb = wnorm->nb; fa.nw_dtype = wnorm->nw_dtype;
    fa.neps = wnorm->neps; fa.nsigmoid_only = wnorm->nsigmoid_only; fa.nss = wnorm->nss; fa.nepoch = wnorm->nepoch;
    fa.nss_chunks = G.nc;
  }
  if (wide && G.nc > 0 && may_fork && cu_seqlens == nullptr) {
    const int64_t nt = (G.T + kgdn::C - 1) / kgdn::C;
    int P = wide_pipe_parts();
    if (nt < 2 * P) P = 1;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (P > 1 && (hipStreamIsCapturing(s, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone)) P = 1;
    std::unique_lock<std::mutex> lk(g_aux_mu, std::defer_lock);
    hipStream_t s2 = nullptr, s3 = nullptr, s4 = nullptr, s5 = nullptr;
    hipEvent_t* ev = nullptr;
    if (P > 1) {
      lk.lock();
      if (aux_streams(&s2, &s3, &s4, &s5, &ev) != 0) {
        lk.unlock();
        P = 1;
      }
    }
    if (P > 1) {
      const double growth = wide_pipe_growth();
      int64_t bnd[kMaxParts + 1];
      if (growth == 1.0) {
        const int64_t span = (nt + P - 1) / P;
        P = (int)((nt + span - 1) / span);                // no empty trailing part (13 chunks in 6: 5 parts of 3)
        for (int p = 0; p <= P; ++p) bnd[p] = std::min<int64_t>(p * span, nt);
      } else {
        wide_pipe_bounds(nt, P, growth, bnd);
      }
      int rc = KAIROS_GDN_OK;
      auto wait = [&](hipStream_t st, hipEvent_t e) {
        if (rc == KAIROS_GDN_OK && hipStreamWaitEvent(st, e, 0) != hipSuccess) rc = fail(KAIROS_GDN_EHIP, "hipStreamWaitEvent");
      };
      auto record = [&](hipEvent_t e, hipStream_t st) {
        if (rc == KAIROS_GDN_OK && hipEventRecord(e, st) != hipSuccess) rc = fail(KAIROS_GDN_EHIP, "hipEventRecord");
      };
      // ev[p]: prepare p done; ev[kMaxParts + p]: recurrence part p about to be dispatched (its
      // marker done); ev[2 kMaxParts + p]: recurrence part p done
      const int mark = wide_mark_mode();
      const bool beside = mark == 1;
      // the gated norm of part p's rows (per sequence: tokens [64 bnd[p], 64 bnd[p + 1]) of each)
      // on s5 once recurrence part p is done, beside the next part's recurrence
      const bool nparts = epi != nullptr && N <= 8 && norm_parts_on();
      auto norm_part = [&](int p) {
        const int64_t t0 = bnd[p] * kgdn::C, t1 = std::min<int64_t>(bnd[p + 1] * kgdn::C, G.T);
        for (int n = 0; n < N && rc == KAIROS_GDN_OK; ++n)
          rc = norm_in_place(o, y_dtype, *epi, (t1 - t0) * H, V, s5, ((int64_t)n * G.T + t0) * H);
      };
      auto prepare = [&](int p, hipStream_t sp) {
        pa.it0 = bnd[p];
        pa.it_span = bnd[p + 1] - bnd[p];
        if (rc == KAIROS_GDN_OK)
          rc = from_launch(kgdn::launch_prepare(pa, cdt, qk_dtype, K, V, (int64_t)N * pa.it_span, sp), "prepare");
        record(ev[p], sp);
      };
      prepare(0, s);
      for (int p = 0; p < P && rc == KAIROS_GDN_OK; ++p) {
        wait(s3, ev[p]);
        if (p + 1 < P) {
          if (beside) {                                   // the marker waits for what part p waits for
            wait(s4, ev[p]);
            if (p > 0) wait(s4, ev[2 * kMaxParts + p - 1]);
            if (rc == KAIROS_GDN_OK) rc = from_launch(kgdn::launch_marker(s4), "marker");
            record(ev[kMaxParts + p], s4);
          } else {
            if (mark == 0 && rc == KAIROS_GDN_OK) rc = from_launch(kgdn::launch_marker(s3), "marker");
            record(ev[kMaxParts + p], s3);
          }
        }
        kgdn::WideFusedArgs fp = fa;
        fp.it_begin = bnd[p];
        fp.it_end = bnd[p + 1];
        if (p > 0) {
          fp.h0 = st;
          fp.h0_dtype = KAIROS_GDN_F32;
        }
        if (p + 1 < P) fp.ht = st;
        if (rc == KAIROS_GDN_OK) rc = from_launch(kgdn::launch_wide_fused(fp, V, s3), "wide fused recurrence");
        if ((beside && p + 2 < P) || nparts) record(ev[2 * kMaxParts + p], s3);
        if (p + 1 < P) {
          wait(s2, ev[kMaxParts + p]);
          prepare(p + 1, s2);
        }
      }
      if (nparts) {                                         // parts 0 .. P - 2 once part P - 2 is done
        wait(s5, ev[2 * kMaxParts + P - 2]);
        for (int p = 0; p + 1 < P; ++p) norm_part(p);
        wait(s5, ev[2 * kMaxParts + P - 1]);
        norm_part(P - 1);
      }
      // Join, also after a failed launch or event call above: the caller's stream waits for all
      // that was queued on the library streams (prepares on s2, recurrence parts on s3, markers on
      // s4, norm parts on s5), so the caller may release the workspace once its own stream has passed
      // this point.  If the join itself cannot be enqueued, the library streams are drained on the host.
      const hipStream_t lib_streams[4] = {s2, s3, s4, s5};
      bool joined = true;
      for (int j = 0; j < 4; ++j) {
        if (j == 2 && !beside) continue;                    // s4 carries work only with markers beside
        if (j == 3 && !nparts) continue;                    // s5 only with the norm by parts
        const hipEvent_t e = ev[3 * kMaxParts + j];
        if (hipEventRecord(e, lib_streams[j]) != hipSuccess || hipStreamWaitEvent(s, e, 0) != hipSuccess)
          joined = false;
      }
      if (!joined) {
        for (int j = 0; j < 4; ++j) (void)hipStreamSynchronize(lib_streams[j]);
        if (rc == KAIROS_GDN_OK) rc = fail(KAIROS_GDN_EHIP, "joining the pipelined forward's streams failed");
      }
      if (epi_done) *epi_done = nparts && rc == KAIROS_GDN_OK;
      return rc;
    }
  }
  if (G.nc > 0) {
    if (int rc = from_launch(kgdn::launch_prepare(pa, cdt, qk_dtype, K, V, G.nc, s), "prepare")) return rc;
  }
  if (wide) return from_launch(kgdn::launch_wide_fused(fa, V, s), "wide fused recurrence");
  kgdn::FwdHArgs ha{};
  ha.k = k; ha.k_scale = k_scale; ha.w = w; ha.uT = uT; ha.gc = gc;
  ha.h0 = h0; ha.h0_dtype = h0_dtype;
  ha.cu = cu_seqlens; ha.chunk_off = chunk_off; ha.N = N; ha.T = G.T; ha.H = H;
  ha.hT = hT; ha.vnT = vnT; ha.ht = ht;
  if (int rc = from_launch(kgdn::launch_fwd_h(ha, cdt, qk_dtype, K, V, s), "fwd_h")) return rc;
  if (G.nc > 0) {
    kgdn::FwdOArgs oa{};
    oa.q = q; oa.k = k; oa.q_scale = q_scale; oa.k_scale = k_scale;
    oa.hT = hT; oa.vnT = vnT; oa.gc = gc; oa.scale = scale;
    oa.cu = cu_seqlens; oa.chunk_off = chunk_off; oa.N = N; oa.T = G.T; oa.H = H; oa.o = o;
    if (int rc = from_launch(kgdn::launch_fwd_o(oa, cdt, qk_dtype, K, V, G.nc, s), "fwd_o")) return rc;
  }
  return KAIROS_GDN_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// Static scratch of kairos_gdn_chunk_fwd_noalloc: a file-scope device array,
// one copy per GPU the library's code object is loaded on, held until the
// process ends.  Host code never uses the array's name as an address (on the
// host it is only a handle): the device address is looked up once per device
// with hipGetSymbolAddress and kept in g_scratch_ptr.
// ---------------------------------------------------------------------------
constexpr size_t kScratchBytes = size_t(256) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's scratch array (looked up on the first call per device).
int scratch_address(void** out, const char* what) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess)
    return fail(KAIROS_GDN_EHIP, "%s: hipGetDevice failed: %s", what, hipGetErrorString(hipGetLastError()));
  if (dev < 0 || dev >= kMaxDevices) return fail(KAIROS_GDN_EINVAL, "%s: device %d out of range", what, dev);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t rc = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (rc != hipSuccess || p == nullptr)
      return fail(KAIROS_GDN_EHIP, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", what, dev,
                  hipGetErrorString(rc));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return KAIROS_GDN_OK;
}

}  // namespace

extern "C" {

int kairos_gdn_abi_version(void) { return KAIROS_GDN_ABI_VERSION; }

const char* kairos_gdn_last_error(void) { return g_last_error.c_str(); }

int64_t kairos_gdn_num_chunks_bound(int64_t B, int64_t T, int64_t n_seqs) { return chunks_bound(B, T, n_seqs); }

size_t kairos_gdn_stage_workspace_size(int64_t n_seqs) { return stage_ws(n_seqs); }

size_t kairos_gdn_chunk_fwd_workspace_size(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int64_t n_seqs,
                                           int qk_dtype, int v_dtype, int use_qk_l2norm) {
  if (B <= 0 || T < 0 || H <= 0 || K <= 0 || V <= 0 || n_seqs < 0) return 0;
  const size_t tok = (size_t)(B * T * H);
  const int cdt = compute_dtype(qk_dtype, v_dtype);
  const bool seg = kgdn::seg_fwd_supported(cdt, (int)K, (int)V);
  const bool wide = !seg && use_wide_fused(cdt, qk_dtype, K, V);
  size_t total = seg ? seg_ws(B, T, H, K, V, n_seqs, plan_segments(B, T, H, n_seqs))
                     : staged_ws(B, T, H, K, V, n_seqs, cdt, wide, use_qk_l2norm != 0);
  // in-op L2 norm: the segment scan and the fused K = 256 form fold it into their kernels; the stage
  // kernels normalise q and k in a pass of their own
  if (use_qk_l2norm && !seg && !wide) total += 2 * align_up(tok * K * dt_size(qk_dtype));
  return total;
}


// The segment scan's output kernel takes the epilogue itself for a bf16 gate (KAIROS_GDN_FUSED_NORM=0
// selects the separate norm kernel instead)
static bool fused_norm_on(const NormEpilogue* epi) {
  if (epi == nullptr || epi->gate_dtype != KAIROS_GDN_BF16) return false;
  const char* e = std::getenv("KAIROS_GDN_FUSED_NORM");
  return !(e && e[0] == '0' && e[1] == 0);
}

// With KAIROS_GDN_WIDE_NORM_FOLD=1 the fused K = 256 form takes the epilogue in its loader waves (bf16
// gate, V a multiple of 64 up to 512) when the workspace also holds its exchange buffer
// (kairos_gdn_chunk_fwd_gated_norm_workspace_size counts it then).  Off by default: measured at the Kairos
// layer shape the folded norm makes the call slower than the forward followed by the norm kernel
// (3.04 against 1.90 ms): the fused kernel's step is bound by its loader waves, which share the SIMDs
// with the compute waves, and the norm adds its gate and o rows to their loads and its sigmoid and
// scaling to their VALU issue.
static bool wide_norm_on(const NormEpilogue* epi, int cdt, int qk_dtype, int64_t K, int64_t V) {
  const char* e = std::getenv("KAIROS_GDN_WIDE_NORM_FOLD");
  return e && e[0] == '1' && e[1] == 0 && fused_norm_on(epi) && !kgdn::seg_fwd_supported(cdt, (int)K, (int)V) &&
         use_wide_fused(cdt, qk_dtype, K, V) && V % 64 == 0 && V <= 512;
}

// Tag of one call's exchange entries: a per-process start (time and pid) plus a call count, never 0
static unsigned next_norm_epoch() {
  static std::atomic<unsigned> ctr{0};
  static const unsigned start = (unsigned)std::time(nullptr) * 2654435761u ^ (unsigned)getpid() * 40503u;
  unsigned e;
  do e = start + ctr.fetch_add(1, std::memory_order_relaxed); while (e == 0);
  return e;
}


// Body of kairos_gdn_chunk_fwd, kairos_gdn_chunk_fwd_noalloc and kairos_gdn_chunk_fwd_gated_norm:
// validation, workspace carving and the launches.  Allocates nothing; `profile` lets the call take part
// in kernel timing (which creates events); `epi` (or nullptr) is the gated norm applied to o.
static int chunk_fwd_impl(const char* what, bool profile, const void* q, const void* k, const void* v,
                          const void* g, const void* beta, const float* q_scale, const float* k_scale,
                          const void* initial_state, void* o, float* final_state, const int64_t* cu_seqlens,
                          int64_t n_seqs, int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int qk_dtype,
                          int v_dtype, int g_dtype, int beta_dtype, int h0_dtype, float scale, int use_qk_l2norm,
                          void* workspace, size_t workspace_bytes, void* stream,
                          const NormEpilogue* epi = nullptr) {
  Geometry G;
  if (int rc = check_geometry(G, cu_seqlens, n_seqs, B, T, H, K, V, what)) return rc;
  const int cdt = compute_dtype(qk_dtype, v_dtype);
  if (cdt < 0) return fail(KAIROS_GDN_EINVAL, "%s: unsupported dtype mix q/k=%d v=%d", what, qk_dtype, v_dtype);
  if (!valid_scalar_dt(g_dtype) || !valid_scalar_dt(beta_dtype) || (initial_state && !valid_scalar_dt(h0_dtype)))
    return fail(KAIROS_GDN_EINVAL, "%s: g, beta and initial_state must be fp32 or bf16", what);
  if (qk_dtype == KAIROS_GDN_F8E4M3 && (q_scale == nullptr || k_scale == nullptr))
    return fail(KAIROS_GDN_EINVAL, "%s: fp8 q/k need per-head q_scale and k_scale", what);
  if (qk_dtype == KAIROS_GDN_F8E4M3 && use_qk_l2norm)
    return fail(KAIROS_GDN_EUNSUPPORTED, "%s: the in-kernel L2 norm is not available for fp8 q/k", what);
  if (!(K == 64 || K == 128 || K == 256) || V % 16 != 0 || V > 1024)
    return fail(KAIROS_GDN_EUNSUPPORTED,
                "%s: head dims K=%lld V=%lld are not built (K in {64, 128, 256}, V a multiple of 16 up to 1024)",
                what, (long long)K, (long long)V);
  if (!std::isfinite(scale)) return fail(KAIROS_GDN_EINVAL, "%s: scale must be finite", what);
  const bool any_tokens = G.B * G.T > 0;
  if (any_tokens && (!q || !k || !v || !g || !beta || !o))
    return fail(KAIROS_GDN_EINVAL, "%s: null tensor pointer", what);
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
    return fail(KAIROS_GDN_EINVAL, "%s: q, k, v and o must be 16-byte aligned", what);
  const size_t need = kairos_gdn_chunk_fwd_workspace_size(B, T, H, K, V, n_seqs, qk_dtype, v_dtype, use_qk_l2norm);
  if (workspace_bytes < need)
    return fail(KAIROS_GDN_EWORKSPACE, "%s: workspace of %zu bytes is smaller than the %zu required", what,
                workspace_bytes, need);
  if (need && !aligned16(workspace)) return fail(KAIROS_GDN_EINVAL, "%s: workspace must be 16-byte aligned", what);

  hipStream_t s = static_cast<hipStream_t>(stream);
  const size_t tok = (size_t)(B * T * H);
  Carver cv{static_cast<char*>(workspace)};
  if (!kgdn::seg_fwd_supported(cdt, (int)K, (int)V)) {
    const bool wide = use_wide_fused(cdt, qk_dtype, K, V);
    // the gated norm in the fused K = 256 form, given room for its exchange buffer beyond `need`
    kgdn::WideFusedArgs wn{};
    const size_t nb = kgdn::wide_norm_bytes(G.nc, H);
    const bool wfold = any_tokens && wide_norm_on(epi, cdt, qk_dtype, K, V) && workspace_bytes >= need + nb;
    if (wfold) {
      wn.ngate = epi->gate; wn.nw = epi->w; wn.nb = epi->b; wn.nw_dtype = epi->w_dtype;
      wn.neps = epi->eps; wn.nsigmoid_only = epi->sigmoid_only;
      wn.nss = reinterpret_cast<unsigned long long*>(static_cast<char*>(workspace) + need);
      wn.nepoch = next_norm_epoch();
    }
    if (use_qk_l2norm && any_tokens && !wide) {
      void* qn = cv.take(tok * K * dt_size(qk_dtype));
      void* kn = cv.take(tok * K * dt_size(qk_dtype));
      if (int rc = from_launch(kgdn::launch_l2norm2(q, qn, k, kn, qk_dtype, (int64_t)tok, (int)K, s), "l2norm(q, k)"))
        return rc;
      q = qn;
      k = kn;
    }
    bool epi_done = false;
    if (int rc = run_staged(G, q, k, v, g, beta, q_scale, k_scale, initial_state, h0_dtype, o, final_state,
                            cu_seqlens, qk_dtype, cdt, g_dtype, beta_dtype, scale, cv, s, profile,
                            wide && use_qk_l2norm != 0, nullptr, wfold ? &wn : nullptr,
                            wfold ? nullptr : epi, v_dtype, &epi_done))
      return rc;
    if (epi && !wfold && !epi_done)
      if (int rc = norm_in_place(o, v_dtype, *epi, (int64_t)tok, V, s)) return rc;
    return ok();
  }
  const SegPlan P = plan_segments(B, T, H, n_seqs);
  const int32_t* chunk_off = nullptr;
  const int32_t* seg_off = nullptr;
  if (G.varlen) {
    int32_t* co = static_cast<int32_t*>(cv.take(sizeof(int32_t) * (G.N + 1)));
    int32_t* so = static_cast<int32_t*>(cv.take(sizeof(int32_t) * (G.N + 1)));
    if (int rc = from_launch(kgdn::launch_seg_map(cu_seqlens, (int)G.N, P.L, co, so, s), "segment map")) return rc;
    chunk_off = co;
    seg_off = so;
  }
  const int64_t nc_grid = chunks_bound(B, T, n_seqs);
  void* Ai = cv.take((size_t)nc_grid * H * kgdn::kSegRecordBytes);
  uint16_t* M = nullptr;
  float* R = nullptr;
  float* s_init = nullptr;
  if (P.trans || P.combine) {
    const size_t blocks = (size_t)P.ns * H;
    M = static_cast<uint16_t*>(cv.take(blocks * 2 * K * K * sizeof(uint16_t)));
    R = static_cast<float*>(cv.take(blocks * K * V * sizeof(float)));
    s_init = static_cast<float*>(cv.take(blocks * K * V * sizeof(float)));
  }
  if (P.ns > 0x7fffffff / 2) return fail(KAIROS_GDN_EINVAL, "%s: too many segments", what);

  kgdn::SegFwdArgs a{};
  a.q = q; a.k = k; a.v = v; a.g = g; a.beta = beta; a.q_scale = q_scale; a.k_scale = k_scale;
  a.g_dtype = g_dtype; a.beta_dtype = beta_dtype;
  a.h0 = initial_state; a.h0_dtype = h0_dtype;
  a.cu = cu_seqlens; a.chunk_off = chunk_off; a.seg_off = seg_off;
  a.N = (int)G.N; a.T = T; a.H = (int)H; a.L = P.L; a.nseg_fixed = P.nseg_fixed; a.ns_grid = P.ns;
  a.M = M; a.R = R; a.s_init = s_init; a.scale = scale; a.o = o; a.ht = final_state;
  a.Ai = Ai; a.nc_grid = nc_grid;
  a.l2 = use_qk_l2norm != 0;
  a.run_trans = P.trans && P.ns > 0;
  a.run_combine = P.combine;
  a.events = profile ? profile_events() : nullptr;
  const bool fuse = fused_norm_on(epi);
  if (fuse) {
    a.gate = epi->gate; a.nw = epi->w; a.nb = epi->b; a.nw_dtype = epi->w_dtype;
    a.eps = epi->eps; a.sigmoid_only = epi->sigmoid_only;
  }
  if (int rc = from_launch(kgdn::launch_seg_fwd(a, cdt, qk_dtype, (int)K, (int)V, s), "segment forward")) return rc;
  if (epi && !fuse)
    if (int rc = norm_in_place(o, v_dtype, *epi, (int64_t)tok, V, s)) return rc;
  return ok();
}

int kairos_gdn_chunk_fwd(const void* q, const void* k, const void* v, const void* g, const void* beta,
                         const float* q_scale, const float* k_scale, const void* initial_state, void* o,
                         float* final_state, const int64_t* cu_seqlens, int64_t n_seqs, int64_t B, int64_t T,
                         int64_t H, int64_t K, int64_t V, int qk_dtype, int v_dtype, int g_dtype, int beta_dtype,
                         int h0_dtype, float scale, int use_qk_l2norm, void* workspace, size_t workspace_bytes,
                         void* stream) {
  return chunk_fwd_impl("kairos_gdn_chunk_fwd", true, q, k, v, g, beta, q_scale, k_scale, initial_state, o,
                        final_state, cu_seqlens, n_seqs, B, T, H, K, V, qk_dtype, v_dtype, g_dtype, beta_dtype,
                        h0_dtype, scale, use_qk_l2norm, workspace, workspace_bytes, stream);
}

int kairos_gdn_chunk_fwd_gated_norm(const void* q, const void* k, const void* v, const void* g, const void* beta,
                                    const float* q_scale, const float* k_scale, const void* initial_state,
                                    const void* gate, const void* norm_weight, const void* norm_bias, void* y,
                                    float* final_state, const int64_t* cu_seqlens, int64_t n_seqs, int64_t B,
                                    int64_t T, int64_t H, int64_t K, int64_t V, int qk_dtype, int v_dtype,
                                    int g_dtype, int beta_dtype, int h0_dtype, int gate_dtype, int norm_w_dtype,
                                    float scale, int use_qk_l2norm, float eps, int activation, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  const char* what = "kairos_gdn_chunk_fwd_gated_norm";
  if (!valid_scalar_dt(gate_dtype)) return fail(KAIROS_GDN_EINVAL, "%s: gate must be fp32 or bf16", what);
  if ((norm_weight || norm_bias) && !valid_scalar_dt(norm_w_dtype))
    return fail(KAIROS_GDN_EINVAL, "%s: norm weight and bias must be fp32 or bf16", what);
  if (activation != KAIROS_GDN_ACT_SWISH && activation != KAIROS_GDN_ACT_SIGMOID)
    return fail(KAIROS_GDN_EINVAL, "%s: activation must be KAIROS_GDN_ACT_SWISH or KAIROS_GDN_ACT_SIGMOID", what);
  if (!(eps >= 0.f)) return fail(KAIROS_GDN_EINVAL, "%s: eps must be non-negative", what);
  if (V > 512)
    return fail(KAIROS_GDN_EUNSUPPORTED, "%s: the gated norm is built for V up to 512 (got %lld)", what,
                (long long)V);
  if (B > 0 && T > 0 && (!gate || !aligned16(gate)))
    return fail(KAIROS_GDN_EINVAL, "%s: gate must be non-null and 16-byte aligned", what);
  if ((norm_weight && !aligned16(norm_weight)) || (norm_bias && !aligned16(norm_bias)))
    return fail(KAIROS_GDN_EINVAL, "%s: norm weight and bias must be 16-byte aligned", what);
  const NormEpilogue epi{gate, norm_weight, norm_bias, gate_dtype, norm_w_dtype, eps,
                         activation == KAIROS_GDN_ACT_SIGMOID ? 1 : 0};
  return chunk_fwd_impl(what, true, q, k, v, g, beta, q_scale, k_scale, initial_state, y, final_state, cu_seqlens,
                        n_seqs, B, T, H, K, V, qk_dtype, v_dtype, g_dtype, beta_dtype, h0_dtype, scale,
                        use_qk_l2norm, workspace, workspace_bytes, stream, &epi);
}

size_t kairos_gdn_chunk_fwd_gated_norm_workspace_size(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V,
                                                      int64_t n_seqs, int qk_dtype, int v_dtype, int use_qk_l2norm) {
  const size_t need = kairos_gdn_chunk_fwd_workspace_size(B, T, H, K, V, n_seqs, qk_dtype, v_dtype, use_qk_l2norm);
  if (need == 0 && (B <= 0 || T < 0 || H <= 0 || K <= 0 || V <= 0 || n_seqs < 0)) return 0;
  const int cdt = compute_dtype(qk_dtype, v_dtype);
  const NormEpilogue probe{nullptr, nullptr, nullptr, KAIROS_GDN_BF16, KAIROS_GDN_F32, 0.f, 0};
  if (cdt < 0 || !wide_norm_on(&probe, cdt, qk_dtype, K, V)) return need;
  return need + kgdn::wide_norm_bytes(chunks_bound(B, T, n_seqs), H);
}

size_t kairos_gdn_chunk_fwd_noalloc_max_bytes(void) { return kScratchBytes; }

// ---------------------------------------------------------------------------
// The layer's prologue folded into the forward (kairos_gdn_chunk_fwd_conv)
// ---------------------------------------------------------------------------
// Where the fused K = 256 form runs (bf16, K = 256, V a multiple of 64), prepare forms k and q from
// their projections and the recurrence's loader waves form v: the convolved q, k, v never reach HBM
// but q once (normalised with the in-op L2 norm), which the recurrence's value tiles share.  Other head
// dims run the standalone convolution (with the per-head L2 norm) into the workspace and then the
// forward.
static bool conv_folded(int64_t K, int64_t V) {
  return K == 256 && use_wide_fused(KAIROS_GDN_BF16, KAIROS_GDN_BF16, K, V);
}

size_t kairos_gdn_chunk_fwd_conv_workspace_size(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V,
                                                int64_t n_seqs, int use_qk_l2norm) {
  if (B <= 0 || T < 0 || H <= 0 || K <= 0 || V <= 0 || n_seqs < 0) return 0;
  const size_t tok = (size_t)(B * T * H);
  size_t total = 2 * align_up((size_t)(H * K) * 5 * sizeof(float)) + align_up((size_t)(H * V) * 5 * sizeof(float));
  if (conv_folded(K, V))
    return total + staged_ws(B, T, H, K, V, n_seqs, KAIROS_GDN_BF16, true, false) + align_up(tok * K * 2);
  total += 2 * align_up(tok * K * 2) + align_up(tok * V * 2);
  return total + kairos_gdn_chunk_fwd_workspace_size(B, T, H, K, V, n_seqs, KAIROS_GDN_BF16, KAIROS_GDN_BF16, 0);
}

int kairos_gdn_chunk_fwd_conv(const void* xq, const void* xk, const void* xv, const void* wq, const void* wk,
                              const void* wv, const void* bq, const void* bk, const void* bv, const void* cq_in,
                              const void* ck_in, const void* cv_in, void* cq_out, void* ck_out, void* cv_out,
                              int w_dtype, const void* g, const void* beta, const void* initial_state, void* o,
                              float* final_state, const int64_t* cu_seqlens, int64_t n_seqs, int64_t B, int64_t T,
                              int64_t H, int64_t K, int64_t V, int g_dtype, int beta_dtype, int h0_dtype,
                              float scale, int use_qk_l2norm, void* workspace, size_t workspace_bytes,
                              void* stream) {
  const char* what = "kairos_gdn_chunk_fwd_conv";
  Geometry G;
  if (int rc = check_geometry(G, cu_seqlens, n_seqs, B, T, H, K, V, what)) return rc;
  if (!valid_scalar_dt(w_dtype)) return fail(KAIROS_GDN_EINVAL, "%s: conv weights must be fp32 or bf16", what);
  if (!valid_scalar_dt(g_dtype) || !valid_scalar_dt(beta_dtype) || (initial_state && !valid_scalar_dt(h0_dtype)))
    return fail(KAIROS_GDN_EINVAL, "%s: g, beta and initial_state must be fp32 or bf16", what);
  if (!(K == 64 || K == 128 || K == 256) || V % 16 != 0 || V > 1024)
    return fail(KAIROS_GDN_EUNSUPPORTED, "%s: head dims K=%lld V=%lld are not built", what, (long long)K,
                (long long)V);
  if (!std::isfinite(scale)) return fail(KAIROS_GDN_EINVAL, "%s: scale must be finite", what);
  const bool any_tokens = G.B * G.T > 0;
  if (any_tokens && (!xq || !xk || !xv || !wq || !wk || !wv || !g || !beta || !o))
    return fail(KAIROS_GDN_EINVAL, "%s: null tensor pointer", what);
  for (const void* p : {xq, xk, xv, wq, wk, wv, bq, bk, bv, static_cast<const void*>(o)})
    if (!aligned16(p)) return fail(KAIROS_GDN_EINVAL, "%s: projections, weights, biases and o must be 16-byte aligned",
                                   what);
  if ((cq_out && cq_out == cq_in) || (ck_out && ck_out == ck_in) || (cv_out && cv_out == cv_in))
    return fail(KAIROS_GDN_EINVAL, "%s: a conv cache out must not alias its cache in", what);
  const size_t need = kairos_gdn_chunk_fwd_conv_workspace_size(B, T, H, K, V, n_seqs, use_qk_l2norm);
  if (workspace_bytes < need)
    return fail(KAIROS_GDN_EWORKSPACE, "%s: workspace of %zu bytes is smaller than the %zu required", what,
                workspace_bytes, need);
  if (need && !aligned16(workspace)) return fail(KAIROS_GDN_EINVAL, "%s: workspace must be 16-byte aligned", what);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t DK = H * K, DV = H * V;
  Carver cv{static_cast<char*>(workspace)};
  // fp32 taps [D, 4] and biases [D] of the three projections
  const void* xs[3] = {xq, xk, xv};
  const void* ws3[3] = {wq, wk, wv};
  const void* bs3[3] = {bq, bk, bv};
  const void* cin[3] = {cq_in, ck_in, cv_in};
  void* cout[3] = {cq_out, ck_out, cv_out};
  const int64_t D3[3] = {DK, DK, DV};
  kgdn::ConvIn c3[3];
  for (int i = 0; i < 3; ++i) {
    float* tw = static_cast<float*>(cv.take((size_t)D3[i] * 5 * sizeof(float)));
    float* tb = bs3[i] ? tw + D3[i] * 4 : nullptr;
    if (any_tokens) {
      if (int rc = from_launch(kgdn::launch_to_f32(ws3[i], w_dtype, tw, D3[i] * 4, s), what)) return rc;
      if (tb)
        if (int rc = from_launch(kgdn::launch_to_f32(bs3[i], w_dtype, tb, D3[i], s), what)) return rc;
    }
    c3[i] = kgdn::ConvIn{xs[i], tw, tb, cin[i], KAIROS_GDN_F32, (int)D3[i]};
  }
  if (any_tokens) {
    if (conv_folded(K, V)) {
      if (int rc = run_staged(G, xq, xk, xv, g, beta, nullptr, nullptr, initial_state, h0_dtype, o, final_state,
                              cu_seqlens, KAIROS_GDN_BF16, KAIROS_GDN_BF16, g_dtype, beta_dtype, scale, cv, s, true,
                              use_qk_l2norm != 0, c3))
        return rc;
    } else {
      // the standalone convolution (the per-head L2 norm fused into it), then the forward
      void* y3[3];
      for (int i = 0; i < 3; ++i) {
        y3[i] = cv.take((size_t)(B * T) * D3[i] * 2);
        kgdn::ConvArgs ca{};
        ca.x = xs[i]; ca.y = y3[i]; ca.w = c3[i].w; ca.bias = c3[i].b; ca.h0 = cin[i]; ca.ht = nullptr;
        ca.cu = cu_seqlens; ca.T = T; ca.total_tokens = B * T; ca.N = (int)G.N; ca.D = (int)D3[i]; ca.W = kgdn::kConvW;
        ca.x_dtype = KAIROS_GDN_BF16; ca.w_dtype = KAIROS_GDN_F32; ca.silu = 1;
        ca.head_lanes = (use_qk_l2norm && i < 2) ? (int)(K / 8) : 0;
        if (int rc = from_launch(kgdn::launch_conv1d(ca, s), what)) return rc;
      }
      const size_t rest = workspace_bytes - cv.off;
      if (int rc = chunk_fwd_impl(what, false, y3[0], y3[1], y3[2], g, beta, nullptr, nullptr, initial_state, o,
                                  final_state, cu_seqlens, n_seqs, B, T, H, K, V, KAIROS_GDN_BF16, KAIROS_GDN_BF16,
                                  g_dtype, beta_dtype, h0_dtype, scale, 0, static_cast<char*>(workspace) + cv.off,
                                  rest, stream))
        return rc;
    }
  } else if (final_state) {
    // no tokens: the final state is the initial one (zeros without it)
    if (int rc = kairos_gdn_chunk_fwd(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, initial_state,
                                      nullptr, final_state, cu_seqlens, n_seqs, B, T, H, K, V, KAIROS_GDN_BF16,
                                      KAIROS_GDN_BF16, g_dtype, beta_dtype, h0_dtype, scale, 0, workspace,
                                      workspace_bytes, stream))
      return rc;
  }
  // the final caches, after every kernel that reads the caches in (stream order)
  for (int i = 0; i < 3; ++i) {
    if (!cout[i]) continue;
    kgdn::ConvArgs ca{};
    ca.x = xs[i]; ca.h0 = cin[i]; ca.ht = cout[i]; ca.cu = cu_seqlens; ca.T = T; ca.total_tokens = B * T;
    ca.N = (int)G.N; ca.D = (int)D3[i]; ca.W = kgdn::kConvW; ca.x_dtype = KAIROS_GDN_BF16;
    if (int rc = from_launch(kgdn::launch_conv_state(ca, s), what)) return rc;
  }
  return ok();
}

int kairos_gdn_chunk_fwd_noalloc(const void* q, const void* k, const void* v, const void* g, const void* beta,
                                 const float* q_scale, const float* k_scale, const void* initial_state, void* o,
                                 float* final_state, const int64_t* cu_seqlens, int64_t n_seqs, int64_t B,
                                 int64_t T, int64_t H, int64_t K, int64_t V, int qk_dtype, int v_dtype,
                                 int g_dtype, int beta_dtype, int h0_dtype, float scale, int use_qk_l2norm,
                                 void* stream) {
  const char* what = "kairos_gdn_chunk_fwd_noalloc";
  const size_t need = kairos_gdn_chunk_fwd_workspace_size(B, T, H, K, V, n_seqs, qk_dtype, v_dtype, use_qk_l2norm);
  if (need > kScratchBytes)
    return fail(KAIROS_GDN_EWORKSPACE,
                "%s: this problem needs %zu bytes of scratch, more than the library's static %zu-byte array; "
                "call kairos_gdn_chunk_fwd with a workspace instead", what, need, kScratchBytes);
  void* ws = nullptr;
  if (need > 0) {
    if (int rc = scratch_address(&ws, what)) return rc;
  }
  return chunk_fwd_impl(what, false, q, k, v, g, beta, q_scale, k_scale, initial_state, o, final_state, cu_seqlens,
                        n_seqs, B, T, H, K, V, qk_dtype, v_dtype, g_dtype, beta_dtype, h0_dtype, scale,
                        use_qk_l2norm, ws, kScratchBytes, stream);
}

size_t kairos_gdn_chunk_bwd_workspace_size(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int64_t n_seqs,
                                           int qk_dtype, int v_dtype, int use_qk_l2norm) {
  if (B <= 0 || T < 0 || H <= 0 || K <= 0 || V <= 0 || n_seqs < 0) return 0;
  const int cdt = compute_dtype(qk_dtype, v_dtype);
  if (cdt < 0) return 0;
  return bwd_ws(B, T, H, K, V, n_seqs, cdt, qk_dtype, use_qk_l2norm);
}

int kairos_gdn_chunk_bwd(const void* q, const void* k, const void* v, const void* g, const void* beta,
                         const void* initial_state, const void* do_, const float* dht, void* dq, void* dk, void* dv,
                         float* dg, void* dbeta, float* dh0, const int64_t* cu_seqlens, int64_t n_seqs, int64_t B,
                         int64_t T, int64_t H, int64_t K, int64_t V, int qk_dtype, int v_dtype, int g_dtype,
                         int beta_dtype, int h0_dtype, float scale, int use_qk_l2norm, void* workspace,
                         size_t workspace_bytes, void* stream) {
  const char* what = "kairos_gdn_chunk_bwd";
  Geometry G;
  if (int rc = check_geometry(G, cu_seqlens, n_seqs, B, T, H, K, V, what)) return rc;
  if (qk_dtype == KAIROS_GDN_F8E4M3)
    return fail(KAIROS_GDN_EUNSUPPORTED, "%s: the backward pass takes bf16 or fp32 q/k (not fp8)", what);
  const int cdt = compute_dtype(qk_dtype, v_dtype);
  if (cdt < 0) return fail(KAIROS_GDN_EINVAL, "%s: unsupported dtype mix q/k=%d v=%d", what, qk_dtype, v_dtype);
  if (!valid_scalar_dt(g_dtype) || !valid_scalar_dt(beta_dtype) || (initial_state && !valid_scalar_dt(h0_dtype)))
    return fail(KAIROS_GDN_EINVAL, "%s: g, beta and initial_state must be fp32 or bf16", what);
  if (!kgdn::bwd_supported(cdt, (int)K, (int)V))
    return fail(KAIROS_GDN_EUNSUPPORTED,
                "%s: head dims K=%lld V=%lld are not built for the backward (K in {64, 128, 256}, V a multiple of "
                "64: at most 512 in bf16, K and V at most 128 in fp32)", what, (long long)K, (long long)V);
  if (!std::isfinite(scale)) return fail(KAIROS_GDN_EINVAL, "%s: scale must be finite", what);
  const bool any_tokens = G.B * G.T > 0;
  if (any_tokens && (!q || !k || !v || !g || !beta || !do_ || !dq || !dk || !dv || !dg || !dbeta))
    return fail(KAIROS_GDN_EINVAL, "%s: null tensor pointer", what);
  if (initial_state == nullptr && dh0 != nullptr)
    return fail(KAIROS_GDN_EINVAL, "%s: dh0 needs the initial_state it is the gradient of", what);
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(do_) || !aligned16(dq) || !aligned16(dk) ||
      !aligned16(dv))
    return fail(KAIROS_GDN_EINVAL, "%s: q, k, v, do, dq, dk and dv must be 16-byte aligned", what);
  const size_t need = bwd_ws(B, T, H, K, V, n_seqs, cdt, qk_dtype, use_qk_l2norm);
  if (workspace_bytes < need)
    return fail(KAIROS_GDN_EWORKSPACE, "%s: workspace of %zu bytes is smaller than the %zu required", what,
                workspace_bytes, need);
  if (need && !aligned16(workspace)) return fail(KAIROS_GDN_EINVAL, "%s: workspace must be 16-byte aligned", what);

  hipStream_t s = static_cast<hipStream_t>(stream);
  const size_t es = cdt == KAIROS_GDN_F32 ? 4 : 2;
  const size_t tok = (size_t)(B * T * H);
  Carver cv{static_cast<char*>(workspace)};
  const SegPlan P = plan_segments(B, T, H, n_seqs);
  const bool segb = any_tokens && bwd_segmented(cdt, K, V, P);
  if (segb && P.ns > 0x7fffffff / 2) return fail(KAIROS_GDN_EINVAL, "%s: too many segments", what);
  const int32_t* chunk_off = nullptr;
  const int32_t* seg_off = nullptr;
  if (segb && G.varlen) {
    int32_t* co = static_cast<int32_t*>(cv.take(sizeof(int32_t) * (G.N + 1)));
    int32_t* so = static_cast<int32_t*>(cv.take(sizeof(int32_t) * (G.N + 1)));
    if (int rc = from_launch(kgdn::launch_seg_map(cu_seqlens, (int)G.N, P.L, co, so, s), "segment map")) return rc;
    chunk_off = co;
    seg_off = so;
  } else if (int rc = chunk_map(G, cu_seqlens, cv, &chunk_off, s)) {
    return rc;
  }
  float* gc = static_cast<float*>(cv.take(tok * sizeof(float)));
  float* dg1 = static_cast<float*>(cv.take(tok * sizeof(float)));
  void* w = cv.take(tok * K * es);
  void* dwb = cv.take(tok * K * es);
  void* dk1 = cv.take(tok * K * es);
  const bool rc_wide = !segb && bwd_rc_wide(cdt, qk_dtype, K, V, false);
  void* uT = rc_wide ? nullptr : cv.take((size_t)G.nc * H * V * kgdn::C * es);
  void* Ai = cv.take(tok * kgdn::C * es);
  void* hs = cv.take((size_t)G.nc * H * K * V * es);
  void* dhs = cv.take((size_t)G.nc * H * K * V * es);
  void* vn = cv.take(tok * V * es);
  void* dvl = cv.take(tok * V * es);
  void* dv2 = cv.take(tok * V * es);
  void* qT = nullptr;                           // with rc_wide it holds k^T until the dv_local stage
  void* wT = nullptr;
  const bool dhu_wide = !segb && wide_dhu_on(cdt, K, V);
  if (dhu_wide || rc_wide) qT = cv.take((size_t)G.nc * H * K * kgdn::C * es);
  if (dhu_wide) wT = cv.take((size_t)G.nc * H * K * kgdn::C * es);
  const void* qx = q;
  const void* kx = k;
  void* dq_k = dq;
  void* dk_k = dk;
  float* rq = nullptr;
  // the L2 norm's backward: q's folded into the eight-wave dq / dk kernel (from the rstd of each q row
  // the forward norm pass records), else a pass of its own (l2norm_bwd) like k's
  const bool l2q_fold = use_qk_l2norm && kgdn::bwd_dqk_wide(cdt, (int)K);
  if (use_qk_l2norm) {
    void* qn = cv.take(tok * K * es);
    void* kn = cv.take(tok * K * es);
    rq = static_cast<float*>(cv.take(tok * sizeof(float)));
    dk_k = cv.take(tok * K * es);
    if (!l2q_fold) dq_k = cv.take(tok * K * es);
    if (any_tokens) {
      if (int rc = from_launch(kgdn::launch_l2norm2(q, qn, k, kn, qk_dtype, (int64_t)tok, (int)K, s, rq, nullptr),
                               "l2norm(q, k)"))
        return rc;
    }
    qx = qn;
    kx = kn;
  }
  const int N = (int)G.N;
  if (G.nc > 0 && any_tokens) {
    kgdn::PrepareArgs pa{};
    pa.k = kx; pa.v = v; pa.g = g; pa.beta = beta; pa.k_scale = nullptr;
    pa.g_dtype = g_dtype; pa.beta_dtype = beta_dtype;
    pa.cu = cu_seqlens; pa.chunk_off = chunk_off; pa.N = N; pa.T = T; pa.H = (int)H;
    pa.gc = gc; pa.w = w; pa.uT = uT; pa.A_out = nullptr; pa.Ai_out = Ai; pa.wT_out = wT;
    if (rc_wide) {
      pa.kT_out = qT;
      pa.beta_out = dg1;
    }
    if (int rc = from_launch(kgdn::launch_prepare(pa, cdt, qk_dtype, (int)K, (int)V, G.nc, s), "prepare")) return rc;
  }
  kgdn::FwdHArgs ha{};
  ha.k = kx; ha.k_scale = nullptr; ha.w = w; ha.uT = uT; ha.gc = gc;
  ha.h0 = initial_state; ha.h0_dtype = h0_dtype;
  ha.cu = cu_seqlens; ha.chunk_off = chunk_off; ha.N = N; ha.T = T; ha.H = (int)H;
  ha.hT = hs; ha.vnT = vn; ha.ht = nullptr; ha.row_major = true;
  kgdn::BwdArgs ba{};
  ba.q = qx; ba.k = kx; ba.v = v; ba.gc = gc; ba.beta = beta; ba.beta_dtype = beta_dtype;
  ba.do_ = do_; ba.dht = dht; ba.w = w; ba.Ai = Ai; ba.h = hs; ba.vn = vn;
  ba.dvl = dvl; ba.dh = dhs; ba.dv2 = dv2; ba.dw = dwb; ba.dk1 = dk1; ba.dg1 = dg1;
  ba.dq = dq_k; ba.dk = dk_k; ba.dv = dv; ba.dg = dg; ba.db = dbeta; ba.dh0 = dh0;
  ba.rq = l2q_fold ? rq : nullptr;
  ba.cu = cu_seqlens; ba.chunk_off = chunk_off; ba.N = N; ba.T = T; ba.H = (int)H; ba.scale = scale;
  ba.qT = dhu_wide ? qT : nullptr;
  ba.wT = wT;
  const int64_t nc_b = any_tokens ? G.nc : 0;
  if (!segb) {
    if (G.nc > 0 && any_tokens && rc_wide) {
      kgdn::WideFusedArgs fa{};
      fa.kT = qT; fa.v = v; fa.w = w; fa.Ai = Ai; fa.beta = dg1; fa.gc = gc;
      fa.h0 = initial_state; fa.h0_dtype = h0_dtype;
      fa.cu = cu_seqlens; fa.chunk_off = chunk_off; fa.N = N; fa.T = T; fa.H = (int)H; fa.scale = scale;
      fa.h_out = hs; fa.vn_out = vn;
      if (int rc = from_launch(kgdn::launch_wide_fused(fa, (int)V, s), "fused recompute of h and v_new")) return rc;
    } else if (G.nc > 0 && any_tokens) {
      if (int rc = from_launch(kgdn::launch_fwd_h(ha, cdt, qk_dtype, (int)K, (int)V, s), "fwd_h (recompute)"))
        return rc;
    }
    if (int rc = from_launch(kgdn::launch_bwd(ba, cdt, (int)K, (int)V, nc_b, kgdn::BWD_ALL, s), what)) return rc;
  } else {
    // Segment scan.  The forward's segment kernels (prep, trans, combine) give each segment's start
    // state; h and v_new are recomputed per segment from it.  dh: pass 1 runs each segment's
    // recurrence from zero (its dh at the segment start, B_j), a reverse scan with the transposed
    // segment maps turns these into the dh each segment ends with, and pass 2 reruns the segments
    // from there, writing the dh snapshots and dv2 the gradient kernels read.
    const size_t blocks = (size_t)P.ns * H;
    void* rec = cv.take((size_t)G.nc * H * kgdn::kSegRecordBytes);
    uint16_t* M = static_cast<uint16_t*>(cv.take(blocks * 2 * K * K * sizeof(uint16_t)));
    float* R = static_cast<float*>(cv.take(blocks * K * V * sizeof(float)));
    float* s_init = static_cast<float*>(cv.take(blocks * K * V * sizeof(float)));
    int64_t* seg_cu = static_cast<int64_t*>(cv.take((P.ns + 1) * sizeof(int64_t)));
    int32_t* seg_coff = static_cast<int32_t*>(cv.take((P.ns + 1) * sizeof(int32_t)));
    kgdn::SegFwdArgs sa{};
    sa.q = qx; sa.k = kx; sa.v = v; sa.g = g; sa.beta = beta; sa.q_scale = nullptr; sa.k_scale = nullptr;
    sa.g_dtype = g_dtype; sa.beta_dtype = beta_dtype;
    sa.h0 = initial_state; sa.h0_dtype = h0_dtype;
    sa.cu = cu_seqlens; sa.chunk_off = chunk_off; sa.seg_off = seg_off;
    sa.N = N; sa.T = T; sa.H = (int)H; sa.L = P.L; sa.nseg_fixed = P.nseg_fixed; sa.ns_grid = P.ns;
    sa.M = M; sa.R = R; sa.s_init = s_init; sa.scale = scale; sa.o = nullptr; sa.ht = nullptr;
    sa.Ai = rec; sa.nc_grid = G.nc; sa.l2 = false;
    sa.run_trans = true; sa.run_combine = true; sa.skip_out = true; sa.events = nullptr;
    if (int rc = from_launch(kgdn::launch_seg_fwd(sa, cdt, qk_dtype, (int)K, (int)V, s), "segment scan (recompute)"))
      return rc;
    if (int rc = from_launch(kgdn::launch_seg_place(sa, initial_state, h0_dtype, s_init, (int)K, (int)V, true, s),
                             "segment start states"))
      return rc;
    if (int rc = from_launch(kgdn::launch_seg_seq_map(sa, seg_cu, seg_coff, s), "segment offsets")) return rc;
    // the stage kernels over segments: segments as sequences of a varlen batch (the last segment of
    // each sequence has no map; its dh pass starts from dht)
    const int NS = (int)P.ns;
    const int64_t T_all = B * T;
    kgdn::FwdHArgs hs_a = ha;
    hs_a.h0 = s_init; hs_a.h0_dtype = kgdn::DT_F32;
    hs_a.cu = seg_cu; hs_a.chunk_off = seg_coff; hs_a.N = NS; hs_a.T = T_all;
    if (int rc = from_launch(kgdn::launch_fwd_h(hs_a, cdt, qk_dtype, (int)K, (int)V, s), "fwd_h (recompute)"))
      return rc;
    kgdn::BwdArgs bs = ba;
    bs.cu = seg_cu; bs.chunk_off = seg_coff; bs.N = NS; bs.T = T_all;
    if (int rc = from_launch(kgdn::launch_bwd(bs, cdt, (int)K, (int)V, nc_b, kgdn::BWD_DVL, s), what)) return rc;
    float* Bseg = s_init;                       // free once h is recomputed
    float* F = R;                               // free once the forward scan is done
    kgdn::BwdArgs b1 = bs;
    b1.dht = nullptr; b1.dh = nullptr; b1.dv2 = nullptr; b1.dh0 = Bseg;
    if (dht) {                                  // the last segment of each sequence starts from dht
      if (int rc = from_launch(kgdn::launch_seg_place(sa, dht, kgdn::DT_F32, F, (int)K, (int)V, false, s),
                               "segment final-state gradients"))
        return rc;
      b1.dht = F;
    }
    if (int rc = from_launch(kgdn::launch_bwd(b1, cdt, (int)K, (int)V, nc_b, kgdn::BWD_DHU, s), what)) return rc;
    if (int rc = from_launch(kgdn::launch_seg_bwd_combine(sa, Bseg, dht, F, dh0, (int)K, (int)V, s),
                             "segment scan of dh"))
      return rc;
    kgdn::BwdArgs b2 = bs;
    b2.dht = F; b2.dh0 = nullptr;
    if (int rc = from_launch(kgdn::launch_bwd(b2, cdt, (int)K, (int)V, nc_b, kgdn::BWD_DHU, s), what)) return rc;
    if (int rc = from_launch(kgdn::launch_bwd(bs, cdt, (int)K, (int)V, nc_b, kgdn::BWD_GRADS, s), what)) return rc;
  }
  if (use_qk_l2norm && any_tokens) {
    if (!l2q_fold) {
      if (int rc = from_launch(kgdn::launch_l2norm_bwd(q, dq_k, dq, qk_dtype, (int64_t)tok, (int)K, s), "l2norm_bwd(q)"))
        return rc;
    }
    if (int rc = from_launch(kgdn::launch_l2norm_bwd(k, dk_k, dk, qk_dtype, (int64_t)tok, (int)K, s), "l2norm_bwd(k)"))
      return rc;
  }
  return ok();
}

int kairos_gdn_varlen_maps(const int64_t* cu_seqlens, int64_t n_seqs, int64_t seg_chunks, int32_t* chunk_off,
                           int32_t* seg_off, void* stream) {
  const char* what = "kairos_gdn_varlen_maps";
  if (n_seqs <= 0 || n_seqs > 0x7fffffff) return fail(KAIROS_GDN_EINVAL, "%s: n_seqs must be in [1, 2^31)", what);
  if (seg_chunks <= 0 || seg_chunks > (1 << 20))
    return fail(KAIROS_GDN_EINVAL, "%s: seg_chunks must be in [1, 2^20]", what);
  if (!cu_seqlens || !chunk_off || !seg_off) return fail(KAIROS_GDN_EINVAL, "%s: null pointer", what);
  if (int rc = from_launch(kgdn::launch_seg_map(cu_seqlens, (int)n_seqs, (int)seg_chunks, chunk_off, seg_off,
                                                static_cast<hipStream_t>(stream)), what))
    return rc;
  return ok();
}

int kairos_gdn_segment_chunks(int64_t B, int64_t T, int64_t H, int64_t n_seqs) {
  if (B <= 0 || T < 0 || H <= 0 || n_seqs < 0) return 0;
  return plan_segments(B, T, H, n_seqs).L;
}

int kairos_gdn_profile_begin(void) {
  Profile& P = profile();
  std::lock_guard<std::mutex> lk(P.mu);
  P.on = true;
  P.used = 0;
  return ok();
}

int kairos_gdn_profile_end(double* avg_ms, int n) {
  Profile& P = profile();
  std::lock_guard<std::mutex> lk(P.mu);
  P.on = false;
  const size_t calls = P.used / kProfEvents;
  double acc[kProfKernels] = {};
  for (size_t c = 0; c < calls; ++c) {
    hipEvent_t* e = P.pool.data() + kProfEvents * c;
    if (hipEventSynchronize(e[kProfKernels]) != hipSuccess) {
      fail(KAIROS_GDN_EHIP, "kairos_gdn_profile_end: %s", hipGetErrorString(hipGetLastError()));
      return -1;
    }
    for (int k = 0; k < kProfKernels; ++k) {
      float ms = 0.f;
      if (hipEventElapsedTime(&ms, e[k], e[k + 1]) != hipSuccess) {
        fail(KAIROS_GDN_EHIP, "kairos_gdn_profile_end: %s", hipGetErrorString(hipGetLastError()));
        return -1;
      }
      acc[k] += ms;
    }
  }
  for (int k = 0; k < kProfKernels && k < n; ++k) avg_ms[k] = calls ? acc[k] / (double)calls : 0.0;
  P.used = 0;
  g_last_error.clear();
  return (int)calls;
}

int kairos_gdn_chunk_local_cumsum(const void* g, int g_dtype, float* gc, const int64_t* cu_seqlens, int64_t n_seqs,
                                  int64_t B, int64_t T, int64_t H, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  const char* what = "kairos_gdn_chunk_local_cumsum";
  Geometry G;
  if (int rc = check_geometry(G, cu_seqlens, n_seqs, B, T, H, 64, 64, what)) return rc;
  if (!valid_scalar_dt(g_dtype)) return fail(KAIROS_GDN_EINVAL, "%s: g must be fp32 or bf16", what);
  if (workspace_bytes < stage_ws(n_seqs)) return fail(KAIROS_GDN_EWORKSPACE, "%s: workspace too small", what);
  if (G.nc == 0) return ok();
  if (!g || !gc) return fail(KAIROS_GDN_EINVAL, "%s: null tensor pointer", what);
  hipStream_t s = static_cast<hipStream_t>(stream);
  Carver cv{static_cast<char*>(workspace)};
  const int32_t* chunk_off = nullptr;
  if (int rc = chunk_map(G, cu_seqlens, cv, &chunk_off, s)) return rc;
  if (int rc = from_launch(kgdn::launch_cumsum(g, g_dtype, gc, cu_seqlens, chunk_off, (int)G.N, T, (int)H, G.nc, s),
                           what))
    return rc;
  return ok();
}

int kairos_gdn_prepare_wy(const void* k, const void* v, const void* g, const void* beta, const float* k_scale,
                          float* gc, void* w, void* uT, float* A, void* Ai, const int64_t* cu_seqlens, int64_t n_seqs,
                          int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int k_dtype, int v_dtype,
                          int g_dtype, int beta_dtype, void* workspace, size_t workspace_bytes, void* stream) {
  const char* what = "kairos_gdn_prepare_wy";
  Geometry G;
  if (int rc = check_geometry(G, cu_seqlens, n_seqs, B, T, H, K, V, what)) return rc;
  const int cdt = compute_dtype(k_dtype, v_dtype);
  if (cdt < 0) return fail(KAIROS_GDN_EINVAL, "%s: unsupported dtype mix k=%d v=%d", what, k_dtype, v_dtype);
  if (!valid_scalar_dt(g_dtype) || !valid_scalar_dt(beta_dtype))
    return fail(KAIROS_GDN_EINVAL, "%s: g and beta must be fp32 or bf16", what);
  if (k_dtype == KAIROS_GDN_F8E4M3 && !k_scale) return fail(KAIROS_GDN_EINVAL, "%s: fp8 k needs k_scale", what);
  if (workspace_bytes < stage_ws(n_seqs)) return fail(KAIROS_GDN_EWORKSPACE, "%s: workspace too small", what);
  if (G.nc == 0) return ok();
  if (!k || !v || !g || !beta || !gc || !w || !uT) return fail(KAIROS_GDN_EINVAL, "%s: null tensor pointer", what);
  if (!aligned16(k) || !aligned16(v) || !aligned16(w) || !aligned16(uT))
    return fail(KAIROS_GDN_EINVAL, "%s: k, v, w and uT must be 16-byte aligned", what);
  hipStream_t s = static_cast<hipStream_t>(stream);
  Carver cv{static_cast<char*>(workspace)};
  const int32_t* chunk_off = nullptr;
  if (int rc = chunk_map(G, cu_seqlens, cv, &chunk_off, s)) return rc;
  kgdn::PrepareArgs pa{};
  pa.k = k; pa.v = v; pa.g = g; pa.beta = beta; pa.k_scale = k_scale;
  pa.g_dtype = g_dtype; pa.beta_dtype = beta_dtype;
  pa.cu = cu_seqlens; pa.chunk_off = chunk_off; pa.N = (int)G.N; pa.T = T; pa.H = (int)H;
  pa.gc = gc; pa.w = w; pa.uT = uT; pa.A_out = A; pa.Ai_out = Ai;
  if (int rc = from_launch(kgdn::launch_prepare(pa, cdt, k_dtype, (int)K, (int)V, G.nc, s), what)) return rc;
  return ok();
}

int kairos_gdn_fwd_h(const void* k, const float* k_scale, const void* w, const void* uT, const float* gc,
                     const void* initial_state, void* hT, void* vnT, float* final_state, const int64_t* cu_seqlens,
                     int64_t n_seqs, int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int k_dtype, int v_dtype,
                     int h0_dtype, void* workspace, size_t workspace_bytes, void* stream) {
  const char* what = "kairos_gdn_fwd_h";
  Geometry G;
  if (int rc = check_geometry(G, cu_seqlens, n_seqs, B, T, H, K, V, what)) return rc;
  const int cdt = compute_dtype(k_dtype, v_dtype);
  if (cdt < 0) return fail(KAIROS_GDN_EINVAL, "%s: unsupported dtype mix k=%d v=%d", what, k_dtype, v_dtype);
  if (initial_state && !valid_scalar_dt(h0_dtype))
    return fail(KAIROS_GDN_EINVAL, "%s: initial_state must be fp32 or bf16", what);
  if (k_dtype == KAIROS_GDN_F8E4M3 && !k_scale) return fail(KAIROS_GDN_EINVAL, "%s: fp8 k needs k_scale", what);
  if (workspace_bytes < stage_ws(n_seqs)) return fail(KAIROS_GDN_EWORKSPACE, "%s: workspace too small", what);
  if (G.nc > 0 && (!k || !w || !uT || !gc || !hT || !vnT))
    return fail(KAIROS_GDN_EINVAL, "%s: null tensor pointer", what);
  hipStream_t s = static_cast<hipStream_t>(stream);
  Carver cv{static_cast<char*>(workspace)};
  const int32_t* chunk_off = nullptr;
  if (int rc = chunk_map(G, cu_seqlens, cv, &chunk_off, s)) return rc;
  kgdn::FwdHArgs ha{};
  ha.k = k; ha.k_scale = k_scale; ha.w = w; ha.uT = uT; ha.gc = gc;
  ha.h0 = initial_state; ha.h0_dtype = h0_dtype;
  ha.cu = cu_seqlens; ha.chunk_off = chunk_off; ha.N = (int)G.N; ha.T = T; ha.H = (int)H;
  ha.hT = hT; ha.vnT = vnT; ha.ht = final_state;
  if (int rc = from_launch(kgdn::launch_fwd_h(ha, cdt, k_dtype, (int)K, (int)V, s), what)) return rc;
  return ok();
}

int kairos_gdn_fwd_o(const void* q, const void* k, const float* q_scale, const float* k_scale, const void* hT,
                     const void* vnT, const float* gc, void* o, float scale, const int64_t* cu_seqlens,
                     int64_t n_seqs, int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int qk_dtype,
                     int v_dtype, void* workspace, size_t workspace_bytes, void* stream) {
  const char* what = "kairos_gdn_fwd_o";
  Geometry G;
  if (int rc = check_geometry(G, cu_seqlens, n_seqs, B, T, H, K, V, what)) return rc;
  const int cdt = compute_dtype(qk_dtype, v_dtype);
  if (cdt < 0) return fail(KAIROS_GDN_EINVAL, "%s: unsupported dtype mix q/k=%d v=%d", what, qk_dtype, v_dtype);
  if (qk_dtype == KAIROS_GDN_F8E4M3 && (!q_scale || !k_scale))
    return fail(KAIROS_GDN_EINVAL, "%s: fp8 q/k need q_scale and k_scale", what);
  if (workspace_bytes < stage_ws(n_seqs)) return fail(KAIROS_GDN_EWORKSPACE, "%s: workspace too small", what);
  if (G.nc == 0) return ok();
  if (!q || !k || !hT || !vnT || !gc || !o) return fail(KAIROS_GDN_EINVAL, "%s: null tensor pointer", what);
  if (!aligned16(q) || !aligned16(k) || !aligned16(hT) || !aligned16(vnT) || !aligned16(o))
    return fail(KAIROS_GDN_EINVAL, "%s: q, k, hT, vnT and o must be 16-byte aligned", what);
  hipStream_t s = static_cast<hipStream_t>(stream);
  Carver cv{static_cast<char*>(workspace)};
  const int32_t* chunk_off = nullptr;
  if (int rc = chunk_map(G, cu_seqlens, cv, &chunk_off, s)) return rc;
  kgdn::FwdOArgs oa{};
  oa.q = q; oa.k = k; oa.q_scale = q_scale; oa.k_scale = k_scale;
  oa.hT = hT; oa.vnT = vnT; oa.gc = gc; oa.scale = scale;
  oa.cu = cu_seqlens; oa.chunk_off = chunk_off; oa.N = (int)G.N; oa.T = T; oa.H = (int)H; oa.o = o;
  if (int rc = from_launch(kgdn::launch_fwd_o(oa, cdt, qk_dtype, (int)K, (int)V, G.nc, s), what)) return rc;
  return ok();
}

// ---- the same stages in the reference's layouts: u and v_new [B, T, H, V], h [NCb, H, K, V] ----
// Each converts at its boundary (gdn_layout.hip) and runs the stage above on its own layout in the
// workspace: [stage chunk map | uT | hT | vnT].
namespace {

size_t tokens_ws(const Geometry& G, int cdt) {
  const size_t es = dt_size(cdt);
  const size_t tiles = (size_t)G.nc * G.H * G.V * kgdn::C * es;
  return stage_ws(G.n_seqs) + 2 * align_up(tiles) + align_up((size_t)G.nc * G.H * G.K * G.V * es);
}

int check_tokens(const Geometry& G, int cdt, size_t workspace_bytes, const char* what) {
  if (G.K % 64 != 0 || G.V % 64 != 0)
    return fail(KAIROS_GDN_EINVAL, "%s: K and V must be multiples of 64", what);
  if (workspace_bytes < tokens_ws(G, cdt)) return fail(KAIROS_GDN_EWORKSPACE, "%s: workspace too small", what);
  return KAIROS_GDN_OK;
}

struct TokensWs {
  void *uT, *hT, *vnT;
};

TokensWs carve_tokens(const Geometry& G, int cdt, void* workspace) {
  const size_t es = dt_size(cdt);
  Carver cv{static_cast<char*>(workspace)};
  cv.take(stage_ws(G.n_seqs));
  TokensWs t;
  t.uT = cv.take((size_t)G.nc * G.H * G.V * kgdn::C * es);
  t.hT = cv.take((size_t)G.nc * G.H * G.K * G.V * es);
  t.vnT = cv.take((size_t)G.nc * G.H * G.V * kgdn::C * es);
  return t;
}

}  // namespace

size_t kairos_gdn_stage_tokens_workspace_size(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int64_t n_seqs,
                                              int dtype) {
  if (B <= 0 || T < 0 || H <= 0 || K <= 0 || V <= 0 || n_seqs < 0 || !valid_scalar_dt(dtype)) return 0;
  Geometry G{B, T, H, K, V, n_seqs, n_seqs > 0 ? n_seqs : B, chunks_bound(B, T, n_seqs), n_seqs > 0};
  return tokens_ws(G, dtype);
}

int kairos_gdn_prepare_wy_tokens(const void* k, const void* v, const void* g, const void* beta, const float* k_scale,
                                 float* gc, void* w, void* u, float* A, void* Ai, const int64_t* cu_seqlens,
                                 int64_t n_seqs, int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int k_dtype,
                                 int v_dtype, int g_dtype, int beta_dtype, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  const char* what = "kairos_gdn_prepare_wy_tokens";
  Geometry G;
  if (int rc = check_geometry(G, cu_seqlens, n_seqs, B, T, H, K, V, what)) return rc;
  const int cdt = compute_dtype(k_dtype, v_dtype);
  if (cdt < 0) return fail(KAIROS_GDN_EINVAL, "%s: unsupported dtype mix k=%d v=%d", what, k_dtype, v_dtype);
  if (int rc = check_tokens(G, cdt, workspace_bytes, what)) return rc;
  if (G.nc == 0) return ok();
  if (!u) return fail(KAIROS_GDN_EINVAL, "%s: null tensor pointer", what);
  const TokensWs t = carve_tokens(G, cdt, workspace);
  if (int rc = kairos_gdn_prepare_wy(k, v, g, beta, k_scale, gc, w, t.uT, A, Ai, cu_seqlens, n_seqs, B, T, H, K, V,
                                     k_dtype, v_dtype, g_dtype, beta_dtype, workspace, stage_ws(n_seqs), stream))
    return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int32_t* chunk_off = G.varlen ? static_cast<const int32_t*>(workspace) : nullptr;   // built by the stage
  if (int rc = from_launch(kgdn::launch_chunk_tiles(t.uT, u, 0, (int)dt_size(cdt), cu_seqlens, chunk_off, (int)G.N,
                                                    T, (int)H, (int)V, G.nc, s),
                           what))
    return rc;
  return ok();
}

int kairos_gdn_fwd_h_tokens(const void* k, const float* k_scale, const void* w, const void* u, const float* gc,
                            const void* initial_state, void* h, void* v_new, float* final_state,
                            const int64_t* cu_seqlens, int64_t n_seqs, int64_t B, int64_t T, int64_t H, int64_t K,
                            int64_t V, int k_dtype, int v_dtype, int h0_dtype, void* workspace,
                            size_t workspace_bytes, void* stream) {
  const char* what = "kairos_gdn_fwd_h_tokens";
  Geometry G;
  if (int rc = check_geometry(G, cu_seqlens, n_seqs, B, T, H, K, V, what)) return rc;
  const int cdt = compute_dtype(k_dtype, v_dtype);
  if (cdt < 0) return fail(KAIROS_GDN_EINVAL, "%s: unsupported dtype mix k=%d v=%d", what, k_dtype, v_dtype);
  if (int rc = check_tokens(G, cdt, workspace_bytes, what)) return rc;
  if (G.nc > 0 && (!u || !h || !v_new)) return fail(KAIROS_GDN_EINVAL, "%s: null tensor pointer", what);
  const TokensWs t = carve_tokens(G, cdt, workspace);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int es = (int)dt_size(cdt);
  if (G.nc > 0) {
    Carver cv{static_cast<char*>(workspace)};
    const int32_t* chunk_off = nullptr;
    if (int rc = chunk_map(G, cu_seqlens, cv, &chunk_off, s)) return rc;
    if (int rc = from_launch(kgdn::launch_chunk_tiles(u, t.uT, 1, es, cu_seqlens, chunk_off, (int)G.N, T, (int)H,
                                                      (int)V, G.nc, s),
                             what))
      return rc;
  }
  if (int rc = kairos_gdn_fwd_h(k, k_scale, w, t.uT, gc, initial_state, t.hT, t.vnT, final_state, cu_seqlens, n_seqs,
                                B, T, H, K, V, k_dtype, v_dtype, h0_dtype, workspace, stage_ws(n_seqs), stream))
    return rc;
  if (G.nc == 0) return ok();
  const int32_t* chunk_off = G.varlen ? static_cast<const int32_t*>(workspace) : nullptr;
  if (int rc = from_launch(kgdn::launch_state_tiles(t.hT, h, es, cu_seqlens, chunk_off, (int)G.N, T, (int)H, (int)V,
                                                    (int)K, G.nc, s),
                           what))
    return rc;
  if (int rc = from_launch(kgdn::launch_chunk_tiles(t.vnT, v_new, 0, es, cu_seqlens, chunk_off, (int)G.N, T, (int)H,
                                                    (int)V, G.nc, s),
                           what))
    return rc;
  return ok();
}

int kairos_gdn_fwd_o_tokens(const void* q, const void* k, const float* q_scale, const float* k_scale, const void* h,
                            const void* v_new, const float* gc, void* o, float scale, const int64_t* cu_seqlens,
                            int64_t n_seqs, int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int qk_dtype,
                            int v_dtype, void* workspace, size_t workspace_bytes, void* stream) {
  const char* what = "kairos_gdn_fwd_o_tokens";
  Geometry G;
  if (int rc = check_geometry(G, cu_seqlens, n_seqs, B, T, H, K, V, what)) return rc;
  const int cdt = compute_dtype(qk_dtype, v_dtype);
  if (cdt < 0) return fail(KAIROS_GDN_EINVAL, "%s: unsupported dtype mix q/k=%d v=%d", what, qk_dtype, v_dtype);
  if (int rc = check_tokens(G, cdt, workspace_bytes, what)) return rc;
  if (G.nc == 0) return ok();
  if (!h || !v_new) return fail(KAIROS_GDN_EINVAL, "%s: null tensor pointer", what);
  const TokensWs t = carve_tokens(G, cdt, workspace);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int es = (int)dt_size(cdt);
  Carver cv{static_cast<char*>(workspace)};
  const int32_t* chunk_off = nullptr;
  if (int rc = chunk_map(G, cu_seqlens, cv, &chunk_off, s)) return rc;
  if (int rc = from_launch(kgdn::launch_state_tiles(h, t.hT, es, cu_seqlens, chunk_off, (int)G.N, T, (int)H, (int)K,
                                                    (int)V, G.nc, s),
                           what))
    return rc;
  if (int rc = from_launch(kgdn::launch_chunk_tiles(v_new, t.vnT, 1, es, cu_seqlens, chunk_off, (int)G.N, T, (int)H,
                                                    (int)V, G.nc, s),
                           what))
    return rc;
  return kairos_gdn_fwd_o(q, k, q_scale, k_scale, t.hT, t.vnT, gc, o, scale, cu_seqlens, n_seqs, B, T, H, K, V,
                          qk_dtype, v_dtype, workspace, stage_ws(n_seqs), stream);
}

int kairos_gdn_l2norm_fwd(const void* x, void* y, float* rstd, int dtype, int64_t rows, int64_t D, void* stream) {
  const char* what = "kairos_gdn_l2norm_fwd";
  if (rows < 0 || D <= 0 || D % 8 != 0 || D > 512)
    return fail(KAIROS_GDN_EINVAL, "%s: D must be a positive multiple of 8, at most 512", what);
  if (!valid_scalar_dt(dtype)) return fail(KAIROS_GDN_EINVAL, "%s: dtype must be fp32 or bf16", what);
  if (rows == 0) return ok();
  if (!x || !y || !aligned16(x) || !aligned16(y))
    return fail(KAIROS_GDN_EINVAL, "%s: x and y must be non-null and 16-byte aligned", what);
  if (rstd != nullptr && reinterpret_cast<uintptr_t>(rstd) % 4 != 0)
    return fail(KAIROS_GDN_EINVAL, "%s: rstd must be 4-byte aligned", what);
  if (int rc = from_launch(kgdn::launch_l2norm(x, y, rstd, dtype, rows, (int)D, static_cast<hipStream_t>(stream)),
                           what))
    return rc;
  return ok();
}

int kairos_gdn_rms_norm_gated(const void* x, const void* g, const void* weight, const void* bias, void* y,
                              float* rstd, int x_dtype, int g_dtype, int w_dtype, int64_t rows, int64_t D,
                              float eps, int activation, void* stream) {
  const char* what = "kairos_gdn_rms_norm_gated";
  if (rows < 0 || D <= 0 || D % 8 != 0 || D > 512)
    return fail(KAIROS_GDN_EINVAL, "%s: D must be a positive multiple of 8, at most 512", what);
  if (!valid_scalar_dt(x_dtype) || !valid_scalar_dt(g_dtype))
    return fail(KAIROS_GDN_EINVAL, "%s: x and g must be fp32 or bf16", what);
  if ((weight || bias) && !valid_scalar_dt(w_dtype))
    return fail(KAIROS_GDN_EINVAL, "%s: weight and bias must be fp32 or bf16", what);
  if (activation != KAIROS_GDN_ACT_SWISH && activation != KAIROS_GDN_ACT_SIGMOID)
    return fail(KAIROS_GDN_EINVAL, "%s: activation must be KAIROS_GDN_ACT_SWISH or KAIROS_GDN_ACT_SIGMOID", what);
  if (!(eps >= 0.f)) return fail(KAIROS_GDN_EINVAL, "%s: eps must be non-negative", what);
  if (rows == 0) return ok();
  if (!x || !g || !y || !aligned16(x) || !aligned16(g) || !aligned16(y))
    return fail(KAIROS_GDN_EINVAL, "%s: x, g and y must be non-null and 16-byte aligned", what);
  if ((weight && !aligned16(weight)) || (bias && !aligned16(bias)))
    return fail(KAIROS_GDN_EINVAL, "%s: weight and bias must be 16-byte aligned", what);
  kgdn::NormArgs a{x, g, weight, bias, y, rstd, x_dtype, g_dtype, w_dtype, rows, (int)D, eps,
                   activation == KAIROS_GDN_ACT_SIGMOID ? 1 : 0};
  if (int rc = from_launch(kgdn::launch_rmsnorm_gated(a, static_cast<hipStream_t>(stream)), what)) return rc;
  return ok();
}

int kairos_gdn_fused_recurrent_fwd(const void* q, const void* k, const void* v, const void* g, const void* gk,
                                   const void* gv, const void* beta, const void* initial_state, void* o,
                                   float* final_state, const int64_t* cu_seqlens, int64_t n_seqs, int64_t B,
                                   int64_t T, int64_t H, int64_t HV, int64_t K, int64_t V, int qk_dtype, int v_dtype,
                                   int g_dtype, int gk_dtype, int gv_dtype, int beta_dtype, int beta_headwise,
                                   int h0_dtype, float scale, int use_qk_l2norm, void* stream) {
  const char* what = "kairos_gdn_fused_recurrent_fwd";
  Geometry G;
  if (int rc = check_geometry(G, cu_seqlens, n_seqs, B, T, HV, K, V, what)) return rc;
  if (H <= 0 || HV % H != 0)
    return fail(KAIROS_GDN_EINVAL, "%s: the value heads HV=%lld must be a multiple of the q/k heads H=%lld", what,
                (long long)HV, (long long)H);
  if (!(K == 16 || K == 32 || K == 64 || K == 128 || K == 256))
    return fail(KAIROS_GDN_EUNSUPPORTED, "%s: K=%lld is not built (K in {16, 32, 64, 128, 256})", what,
                (long long)K);
  if (V > 4096) return fail(KAIROS_GDN_EUNSUPPORTED, "%s: V=%lld is larger than 4096", what, (long long)V);
  if (!valid_scalar_dt(qk_dtype) || !valid_scalar_dt(v_dtype))
    return fail(KAIROS_GDN_EINVAL, "%s: q/k and v must be fp32 or bf16", what);
  if ((g && !valid_scalar_dt(g_dtype)) || (gk && !valid_scalar_dt(gk_dtype)) || (gv && !valid_scalar_dt(gv_dtype)) ||
      (beta && !valid_scalar_dt(beta_dtype)) || (initial_state && !valid_scalar_dt(h0_dtype)))
    return fail(KAIROS_GDN_EINVAL, "%s: g, gk, gv, beta and initial_state must be fp32 or bf16", what);
  if (!std::isfinite(scale)) return fail(KAIROS_GDN_EINVAL, "%s: scale must be finite", what);
  if (G.B * G.T > 0 && (!q || !k || !v || !o)) return fail(KAIROS_GDN_EINVAL, "%s: null tensor pointer", what);
  if (!aligned16(q) || !aligned16(k))
    return fail(KAIROS_GDN_EINVAL, "%s: q and k must be 16-byte aligned", what);
  kgdn::RecArgs a{};
  a.q = q; a.k = k; a.v = v; a.g = g; a.gk = gk; a.gv = gv; a.beta = beta; a.h0 = initial_state;
  a.o = o; a.ht = final_state; a.cu = cu_seqlens; a.T = T;
  a.N = (int)G.N; a.H = (int)H; a.HV = (int)HV; a.K = (int)K; a.V = (int)V;
  a.qk_dtype = qk_dtype; a.v_dtype = v_dtype; a.g_dtype = g_dtype; a.gk_dtype = gk_dtype; a.gv_dtype = gv_dtype;
  a.beta_dtype = beta_dtype; a.h0_dtype = h0_dtype; a.beta_headwise = beta_headwise ? 1 : 0;
  a.l2 = use_qk_l2norm ? 1 : 0; a.scale = scale;
  if (int rc = from_launch(kgdn::launch_fused_recurrent(a, static_cast<hipStream_t>(stream)), what)) return rc;
  return ok();
}

int kairos_gdn_causal_conv1d_fwd(const void* x, const void* weight, const void* bias, const void* initial_state,
                                 void* y, void* final_state, const int64_t* cu_seqlens, int64_t n_seqs, int64_t B,
                                 int64_t T, int64_t D, int64_t W, int x_dtype, int w_dtype, int activation_silu,
                                 int l2norm_head_dim, void* stream) {
  const char* what = "kairos_gdn_causal_conv1d_fwd";
  if (B <= 0 || T < 0 || D <= 0)
    return fail(KAIROS_GDN_EINVAL, "%s: invalid shape B=%lld T=%lld D=%lld", what, (long long)B, (long long)T,
                (long long)D);
  if ((cu_seqlens == nullptr) != (n_seqs == 0) || n_seqs < 0)
    return fail(KAIROS_GDN_EINVAL, "%s: cu_seqlens and n_seqs must be given together", what);
  if (cu_seqlens && B != 1)
    return fail(KAIROS_GDN_EINVAL, "%s: the batch size is expected to be 1 rather than %lld when using cu_seqlens",
                what, (long long)B);
  if (W < 1 || W > 4) return fail(KAIROS_GDN_EUNSUPPORTED, "%s: kernel size W=%lld is not built (1..4)", what,
                                  (long long)W);
  if (D % 8 != 0) return fail(KAIROS_GDN_EINVAL, "%s: D=%lld must be a multiple of 8", what, (long long)D);
  if (!valid_scalar_dt(x_dtype) || !valid_scalar_dt(w_dtype))
    return fail(KAIROS_GDN_EINVAL, "%s: x and weight must be fp32 or bf16", what);
  int head_lanes = 0;
  if (l2norm_head_dim) {
    const int64_t hd = l2norm_head_dim;
    if (!(hd == 64 || hd == 128 || hd == 256 || hd == 512) || D % hd != 0)
      return fail(KAIROS_GDN_EUNSUPPORTED, "%s: l2norm_head_dim=%lld must be 64, 128, 256 or 512 and divide D",
                  what, (long long)hd);
    head_lanes = (int)(hd / 8);
  }
  const int64_t N = cu_seqlens ? n_seqs : B;
  if (N > 0x7fffffff || D > 0x7fffffff) return fail(KAIROS_GDN_EINVAL, "%s: too many sequences or channels", what);
  if (B * T > 0 && (!x || !weight || !y)) return fail(KAIROS_GDN_EINVAL, "%s: null tensor pointer", what);
  if (!aligned16(x) || !aligned16(y) || !aligned16(weight))
    return fail(KAIROS_GDN_EINVAL, "%s: x, y and weight must be 16-byte aligned", what);
  if (final_state && final_state == initial_state)
    return fail(KAIROS_GDN_EINVAL, "%s: final_state must not alias initial_state", what);
  kgdn::ConvArgs a{};
  a.x = x; a.y = y; a.w = weight; a.bias = bias; a.h0 = initial_state; a.ht = final_state; a.cu = cu_seqlens;
  a.T = T; a.total_tokens = B * T; a.N = (int)N; a.D = (int)D; a.W = (int)W;
  a.x_dtype = x_dtype; a.w_dtype = w_dtype; a.silu = activation_silu ? 1 : 0; a.head_lanes = head_lanes;
  if (int rc = from_launch(kgdn::launch_conv1d(a, static_cast<hipStream_t>(stream)), what)) return rc;
  return ok();
}

int kairos_gdn_gates_fwd(const void* a, const void* b, const void* A_log, const void* dt_bias, float* g, void* beta,
                         int64_t rows, int64_t HV, int a_dtype, int b_dtype, int param_dtype, int allow_neg_eigval,
                         void* stream) {
  const char* what = "kairos_gdn_gates_fwd";
  if (rows < 0 || HV <= 0 || HV > 0x7fffffff) return fail(KAIROS_GDN_EINVAL, "%s: invalid shape", what);
  if (!valid_scalar_dt(a_dtype) || !valid_scalar_dt(b_dtype) || !valid_scalar_dt(param_dtype))
    return fail(KAIROS_GDN_EINVAL, "%s: a, b and the parameters must be fp32 or bf16", what);
  if (rows > 0 && (!a || !b || !A_log || !dt_bias || !g || !beta))
    return fail(KAIROS_GDN_EINVAL, "%s: null tensor pointer", what);
  kgdn::GateArgs ga{a, b, A_log, dt_bias, g, beta, rows, (int)HV, a_dtype, b_dtype, param_dtype,
                    allow_neg_eigval ? 1 : 0};
  if (int rc = from_launch(kgdn::launch_gates(ga, static_cast<hipStream_t>(stream)), what)) return rc;
  return ok();
}

}  // extern "C"
