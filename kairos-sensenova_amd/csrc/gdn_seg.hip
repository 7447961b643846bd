// Segment-parallel fused forward of the chunked GatedDeltaNet (the path behind
// kairos_gdn_chunk_fwd).  It computes what the reference's six stages compute
// (fla ops/gated_delta_rule/chunk.py:16-67: cumsum, K.K^T, solve_tril, w/u,
// chunk_fwd_h, chunk_fwd_o) without materialising any stage output in HBM.
//
// Every sequence is cut into segments of L consecutive 64-token chunks, so
// that (segment, head) work items fill the GPU even for one long sequence.
// Per chunk c the state recurrence is affine in the incoming state S:
//     S' = M_c S + R_c,   M_c = g I - k^T diag(gate) w,   R_c = k^T diag(gate) u,
// with g = exp(gc_last) and gate_t = exp(gc_last - gc_t) (chunk_delta_h.py:163-211).
//
//   seg_trans_kernel    (segment, head): recomputes the chunk-local WY
//                       representation and accumulates the segment's affine map
//                       [M | R] (K x (K+V), fp32) starting from [I | 0].
//   seg_combine_kernel  (sequence, head, 16 V columns): serial over segments,
//                       S_{j+1} = M_j S_j + R_j in fp32, from initial_state.
//   seg_out_kernel      (segment, head): recomputes the WY representation,
//                       runs the exact recurrence of chunk_delta_h.py from the
//                       segment's initial state and emits o (chunk_o.py:84-128)
//                       and, for the last segment, final_state.
//
// One workgroup = 4 waves.  Per chunk, the chunk's q, k (row-major and
// transposed) and v (transposed) are staged in LDS; the state tile of each
// wave (K rows x V/4 columns) lives in VGPRs in the MFMA accumulator layout
// for the whole segment.  The next chunk's inputs are loaded into registers
// while the current chunk computes.
//
// LDS operand layout.  All MFMA operands are read as one 8-element fragment
// per lane (16 bytes for bf16).  Lane l of a 16x16x32 product feeds the K
// indices {4(l/16)..+3} and {16+4(l/16)..+3} of a 32-wide step (the order in
// which an accumulator tile pair is converted into an operand), so every
// operand row stores each 32-column block permuted by pcol(): logical column
// 16*hh + 4*lg + j sits at 8*lg + 4*hh + j.  Rows are padded by 8 elements,
// so the 16 rows one fragment read touches fall on distinct banks; the
// transposing stores of k and v ([d][t], [v][t]) run with consecutive lanes on
// consecutive token pairs of one row, which is conflict-free as well.
#include <type_traits>

#include "gdn_common.hpp"
#include "gdn_kernels.h"

namespace kgdn {

namespace {

// Workgroup sizes: seg_out runs one wave per 16 V columns (V/16 waves), seg_trans
// one wave per 32 columns of [M | R] ((K+V)/32 waves), seg_combine 4 waves.
template <int K, int V> struct OutCfg { static constexpr int NW = V / 16, NT = 64 * NW; };
template <int K, int V> struct TransCfg { static constexpr int NW = (K + V) / 32, NT = 64 * NW; };
constexpr int NT_COMB = 256;
constexpr int NW_COMB = 4;

// Workgroup barrier that orders LDS only.  __syncthreads() also fences global
// memory, which makes every barrier wait for all outstanding vector memory
// operations -- the next chunk's prefetch and the output stores included.  The
// waves of a workgroup share nothing but LDS, so an LDS fence is sufficient.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ int pcol(int c) {
  return (c & ~31) | (((c >> 2) & 3) << 3) | (((c >> 4) & 1) << 2) | (c & 3);
}
// physical column of logical token t in a transposed [*][64] tile row
__device__ __forceinline__ int tcol(int, int t) { return pcol(t); }
// physical start of the 8-element fragment chunk `chunk8` (a multiple of 8, already in pcol order)
__device__ __forceinline__ int tchunk(int, int chunk8) { return chunk8; }

template <typename TC>
__device__ __forceinline__ Frag<TC> frag_at(const TC* p) {
  Frag<TC> f;
  if constexpr (sizeof(TC) == 2) {
    f.v = *reinterpret_cast<const bf16x8*>(p);
  } else {
    f.lo = *reinterpret_cast<const f32x4*>(p);
    f.hi = *reinterpret_cast<const f32x4*>(p + 4);
  }
  return f;
}
// two floats -> two bf16 (round to nearest even) packed in a dword, a in the low half
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
  bf16x2_t v = {(bf16)a, (bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}

// the two bf16 values packed in a dword, as floats
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// 8 consecutive LDS elements as floats
template <typename TC>
__device__ __forceinline__ void lds_get8(const TC* p, float (&x)[8]) {
  if constexpr (sizeof(TC) == 2) {
    const uint4 r = *reinterpret_cast<const uint4*>(p);
    x[0] = bf16_lo(r.x); x[1] = bf16_hi(r.x); x[2] = bf16_lo(r.y); x[3] = bf16_hi(r.y);
    x[4] = bf16_lo(r.z); x[5] = bf16_hi(r.z); x[6] = bf16_lo(r.w); x[7] = bf16_hi(r.w);
  } else {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p);
    const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[e] = a[e];
      x[4 + e] = b[e];
    }
  }
}
// operand fragment from 8 floats, rounded to TC
template <typename TC>
__device__ __forceinline__ Frag<TC> frag_pack(const float (&x)[8]) {
  Frag<TC> f;
  if constexpr (sizeof(TC) == 2) {
    bf16x8 v = {(bf16)x[0], (bf16)x[1], (bf16)x[2], (bf16)x[3], (bf16)x[4], (bf16)x[5], (bf16)x[6], (bf16)x[7]};
    f.v = v;
  } else {
    f.lo = f32x4{x[0], x[1], x[2], x[3]};
    f.hi = f32x4{x[4], x[5], x[6], x[7]};
  }
  return f;
}
// Operand fragment from two accumulator tiles (rows 4*lg+j of tile a, then of tile b), rounded to TC.
template <typename TC>
__device__ __forceinline__ Frag<TC> acc_frag(const f32x4& a, const f32x4& b) {
  Frag<TC> f;
  if constexpr (sizeof(TC) == 2) {
    bf16x8 v = {(bf16)a[0], (bf16)a[1], (bf16)a[2], (bf16)a[3], (bf16)b[0], (bf16)b[1], (bf16)b[2], (bf16)b[3]};
    f.v = v;
  } else {
    f.lo = a;
    f.hi = b;
  }
  return f;
}
// logical token index of element e of the fragment a lane of group lg holds for 32-step ks
__device__ __forceinline__ int frag_t(int ks, int lg, int e) { return 32 * ks + 16 * (e >> 2) + 4 * lg + (e & 3); }

// 2 consecutive storage elements
template <typename TC>
__device__ __forceinline__ void st2(TC* p, float a, float b) {
  if constexpr (sizeof(TC) == 2) {
    typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
    bf16x2 v = {(bf16)a, (bf16)b};
    *reinterpret_cast<bf16x2*>(p) = v;
  } else {
    f32x2 v = {a, b};
    *reinterpret_cast<f32x2*>(p) = v;
  }
}

// ---------------------------------------------------------------------------
// problem geometry shared by the three kernels
// ---------------------------------------------------------------------------
struct SegGeom {
  const int64_t* cu;          // varlen token offsets [N+1] or nullptr
  const int32_t* chunk_off;   // varlen chunk offsets [N+1]
  const int32_t* seg_off;     // varlen segment offsets [N+1]
  int N;
  int64_t T;                  // fixed length: per-sequence length
  int H;
  int L;                      // chunks per segment
  int nseg_fixed;             // fixed length: segments per sequence
};

struct SegLoc {
  int n, j, nseg;             // sequence, segment index within it, segments of the sequence
  int64_t bos, eos;           // token range of the sequence
  int64_t c0;                 // first chunk (within the sequence) of the segment
  int nch;                    // chunks in the segment
  bool ok;
};

__device__ __forceinline__ SegLoc locate_seg(int s, const SegGeom& G) {
  SegLoc r;
  r.ok = false;
  if (G.cu == nullptr) {
    if (s >= G.N * G.nseg_fixed) return r;
    r.n = s / G.nseg_fixed;
    r.j = s % G.nseg_fixed;
    r.nseg = G.nseg_fixed;
    r.bos = (int64_t)r.n * G.T;
    r.eos = r.bos + G.T;
  } else {
    if (s >= G.seg_off[G.N]) return r;
    int lo = 0, hi = G.N - 1;      // last n with seg_off[n] <= s
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (G.seg_off[mid] <= s) lo = mid; else hi = mid - 1;
    }
    r.n = lo;
    r.j = s - G.seg_off[lo];
    r.nseg = G.seg_off[lo + 1] - G.seg_off[lo];
    r.bos = G.cu[lo];
    r.eos = G.cu[lo + 1];
  }
  const int64_t nc = (r.eos - r.bos + C - 1) / C;
  r.c0 = (int64_t)r.j * G.L;
  r.nch = (int)min((int64_t)G.L, nc - r.c0);
  r.ok = r.nch > 0;
  return r;
}

// ---------------------------------------------------------------------------
// LDS layout of one workgroup
// ---------------------------------------------------------------------------
template <typename TC, int K, int V, bool WITH_Q>
struct SegLds {
  static constexpr int LDK = K + 8;        // row stride of [64][K] tiles (q, k, w)
  static constexpr int LDT = C + 8;        // row stride of [*][64] tiles (kT, vT, Ai, Aqk)
  static constexpr int LDA = C + 4;        // row stride of the fp32 solve workspace
  static constexpr size_t a16(size_t x) { return (x + 15) / 16 * 16; }
  static constexpr size_t k_bytes = sizeof(TC) * C * LDK;
  static constexpr size_t A_bytes = sizeof(float) * C * LDA;
  // s_k, later s_w (w is produced after the last read of k)
  static constexpr size_t off_k = 0;
  static constexpr size_t off_q = a16(off_k + k_bytes);
  static constexpr size_t off_kT = a16(off_q + (WITH_Q ? k_bytes : 0));
  static constexpr size_t off_vT = a16(off_kT + sizeof(TC) * K * LDT);
  static constexpr size_t off_A = a16(off_vT + sizeof(TC) * V * LDT);
  static constexpr size_t off_Ai = a16(off_A + A_bytes);
  static constexpr size_t off_Aqk = a16(off_Ai + sizeof(TC) * C * LDT);
  static constexpr size_t off_g = a16(off_Aqk + (WITH_Q ? sizeof(TC) * C * LDT : 0));
  static constexpr size_t vec_end = off_g + sizeof(float) * 4 * C;   // gc, exp(gc), beta, gate
  static constexpr size_t raw_off = a16(vec_end);                    // raw staging area of the next chunk
};

// ---------------------------------------------------------------------------
// chunk inputs held in registers between chunks (the prefetch), in storage format
// ---------------------------------------------------------------------------
template <typename T> struct Raw8;                    // 8 consecutive input elements, as loaded
template <> struct Raw8<bf16> { uint4 v; };
template <> struct Raw8<float> { f32x4 lo, hi; };
template <> struct Raw8<uint8_t> { uint2 v; };        // fp8 e4m3 codes

template <typename T>
__device__ __forceinline__ Raw8<T> raw_load(const T* p) {
  Raw8<T> r;
  if constexpr (sizeof(T) == 1) {
    r.v = *reinterpret_cast<const uint2*>(p);
  } else if constexpr (sizeof(T) == 2) {
    r.v = *reinterpret_cast<const uint4*>(p);
  } else {
    r.lo = *reinterpret_cast<const f32x4*>(p);
    r.hi = *reinterpret_cast<const f32x4*>(p + 4);
  }
  return r;
}
template <typename T>
__device__ __forceinline__ Raw8<T> raw_zero() {
  Raw8<T> r;
  if constexpr (sizeof(T) == 1) {
    r.v = make_uint2(0u, 0u);
  } else if constexpr (sizeof(T) == 2) {
    r.v = make_uint4(0u, 0u, 0u, 0u);
  } else {
    r.lo = f32x4{0.f, 0.f, 0.f, 0.f};
    r.hi = r.lo;
  }
  return r;
}
// the 8 elements as floats (fp8 codes are dequantised with the per-head scale)
template <typename T>
__device__ __forceinline__ void raw_get8(const Raw8<T>& r, float scale, float (&x)[8]) {
  if constexpr (sizeof(T) == 1) {
#pragma unroll
    for (int e = 0; e < 4; ++e) x[e] = fp8e4m3_to_f32((r.v.x >> (8 * e)) & 0xFF) * scale;
#pragma unroll
    for (int e = 0; e < 4; ++e) x[4 + e] = fp8e4m3_to_f32((r.v.y >> (8 * e)) & 0xFF) * scale;
  } else if constexpr (sizeof(T) == 2) {
    x[0] = bf16_lo(r.v.x); x[1] = bf16_hi(r.v.x); x[2] = bf16_lo(r.v.y); x[3] = bf16_hi(r.v.y);
    x[4] = bf16_lo(r.v.z); x[5] = bf16_hi(r.v.z); x[6] = bf16_lo(r.v.w); x[7] = bf16_hi(r.v.w);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[e] = r.lo[e];
      x[4 + e] = r.hi[e];
    }
  }
}

// Bytes of 8 input elements and how they are fetched by direct global->LDS loads
// (global_load_lds_dword / _dwordx4: lane L of a wave writes SIZE bytes at the
// wave's LDS base + L * SIZE).
template <typename T> struct GroupIO {
  static constexpr int G = 8 * (int)sizeof(T);
  static constexpr int SIZE = G >= 16 ? 16 : 4;
  static constexpr int N = G / SIZE;
};

// The next chunk's inputs, fetched while the current chunk computes.  On the
// bf16 path (DIRECT) q, k and v go straight to a raw staging area in LDS
// (no registers held, and no register wait can stall on them); the fp32 path,
// whose operand tiles leave no room for that area, holds them in registers.
template <typename TC, typename TQ, int K, int V, bool WITH_Q, int NT>
struct ChunkRegs {
  static constexpr int QU = C * (K / 8), KU = (C / 2) * (K / 8), VU = (C / 2) * (V / 8);   // work units
  static constexpr int QJ = (QU + NT - 1) / NT;     // 8-element row pieces of q per thread
  static constexpr int KJ = (KU + NT - 1) / NT;     // row-pair pieces of k per thread
  static constexpr int VJ = (VU + NT - 1) / NT;     // row-pair pieces of v per thread
  static constexpr bool DIRECT = sizeof(TC) == 2;
  // raw staging area: block b of a stream holds NT groups, wave w's 64 at (b * NT + 64 w) * G
  static constexpr size_t RAW_Q = WITH_Q ? (size_t)QJ * NT * GroupIO<TQ>::G : 0;
  static constexpr size_t RAW_K = (size_t)KJ * 2 * NT * GroupIO<TQ>::G;
  static constexpr size_t RAW_V = (size_t)VJ * 2 * NT * GroupIO<TC>::G;
  static constexpr size_t RAW = DIRECT ? RAW_Q + RAW_K + RAW_V : 0;
  Raw8<TQ> q[DIRECT ? 1 : (WITH_Q ? QJ : 1)];
  Raw8<TQ> k[DIRECT ? 1 : KJ][2];
  Raw8<TC> v[DIRECT ? 1 : VJ][2];
  uint32_t g, b;              // raw bits of g and beta of row tid (fp32, or bf16 in the low half)
};

typedef __attribute__((address_space(1))) void gmem_void;
typedef __attribute__((address_space(3))) void lmem_void;

// Direct loads of one group per lane (the wave's 64 groups land contiguously per load).
template <typename T>
__device__ __forceinline__ void group_to_lds(const T* src, unsigned char* blk) {
  using IO = GroupIO<T>;
  const unsigned char* p = reinterpret_cast<const unsigned char*>(src);
#pragma unroll
  for (int j = 0; j < IO::N; ++j) {
    // the builtin takes the size as a literal
    if constexpr (IO::SIZE == 16)
      __builtin_amdgcn_global_load_lds((gmem_void*)(p + j * 16), (lmem_void*)(blk + j * WAVE * 16), 16, 0, 0);
    else
      __builtin_amdgcn_global_load_lds((gmem_void*)(p + j * 4), (lmem_void*)(blk + j * WAVE * 4), 4, 0, 0);
  }
}
// This lane's group back from the staging area.
template <typename T>
__device__ __forceinline__ Raw8<T> group_from_lds(const unsigned char* blk) {
  using IO = GroupIO<T>;
  const int l = lane_id();
  Raw8<T> r;
  if constexpr (sizeof(T) == 1) {
    r.v.x = *reinterpret_cast<const uint32_t*>(blk + l * 4);
    r.v.y = *reinterpret_cast<const uint32_t*>(blk + WAVE * 4 + l * 4);
  } else if constexpr (sizeof(T) == 2) {
    r.v = *reinterpret_cast<const uint4*>(blk + l * 16);
  } else {
    r.lo = *reinterpret_cast<const f32x4*>(blk + l * 16);
    r.hi = *reinterpret_cast<const f32x4*>(blk + WAVE * 16 + l * 16);
  }
  return r;
}

// raw per-token scalar (fp32 or bf16 bits) -> float; converted only when staged, so
// that the loads of the next chunk stay in flight while the current one computes
__device__ __forceinline__ uint32_t ld_raw(const void* p, int64_t i, int dt) {
  return dt == DT_F32 ? reinterpret_cast<const uint32_t*>(p)[i] : (uint32_t)reinterpret_cast<const uint16_t*>(p)[i];
}
__device__ __forceinline__ float raw_to_f32(uint32_t r, int dt) {
  return dt == DT_F32 ? __uint_as_float(r) : __uint_as_float(r << 16);
}

template <typename TC, typename TQ, int K, int V, bool WITH_Q, int NT>
__device__ __forceinline__ void load_chunk(ChunkRegs<TC, TQ, K, V, WITH_Q, NT>& R, unsigned char* raw, const void* qp,
                                           const void* kp, const void* vp, const void* gp, const void* bp, int g_dt,
                                           int b_dt, int64_t t0, int nv, int h, int H) {
  using CR = ChunkRegs<TC, TQ, K, V, WITH_Q, NT>;
  const int tid = threadIdx.x;
  const int wid = tid / WAVE;
  const TQ* q = reinterpret_cast<const TQ*>(qp);
  const TQ* k = reinterpret_cast<const TQ*>(kp);
  const TC* v = reinterpret_cast<const TC*>(vp);
  if constexpr (CR::DIRECT) {
    // rows beyond nv read row 0 of the chunk (in bounds) and are zeroed when staged
    if constexpr (WITH_Q) {
#pragma unroll
      for (int i = 0; i < CR::QJ; ++i) {
        const int idx = tid + NT * i;
        if (CR::QJ * NT != CR::QU && idx >= CR::QU) break;        // uniform per wave
        const int r = idx / (K / 8), c8 = (idx % (K / 8)) * 8;
        const int rs = r < nv ? r : 0;
        group_to_lds<TQ>(q + ((t0 + rs) * H + h) * K + c8, raw + ((size_t)i * NT + WAVE * wid) * GroupIO<TQ>::G);
      }
    }
    unsigned char* rk = raw + CR::RAW_Q;
#pragma unroll
    for (int i = 0; i < CR::KJ; ++i) {
      const int idx = tid + NT * i;
      if (CR::KJ * NT != CR::KU && idx >= CR::KU) break;
      const int p = idx % (C / 2), c8 = (idx / (C / 2)) * 8;     // token pair fastest
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        const int r = 2 * p + rr;
        const int rs = r < nv ? r : 0;
        group_to_lds<TQ>(k + ((t0 + rs) * H + h) * K + c8,
                         rk + ((size_t)(2 * i + rr) * NT + WAVE * wid) * GroupIO<TQ>::G);
      }
    }
    unsigned char* rv = raw + CR::RAW_Q + CR::RAW_K;
#pragma unroll
    for (int i = 0; i < CR::VJ; ++i) {
      const int idx = tid + NT * i;
      if (CR::VJ * NT != CR::VU && idx >= CR::VU) break;
      const int p = idx % (C / 2), c8 = (idx / (C / 2)) * 8;
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        const int r = 2 * p + rr;
        const int rs = r < nv ? r : 0;
        group_to_lds<TC>(v + ((t0 + rs) * H + h) * V + c8,
                         rv + ((size_t)(2 * i + rr) * NT + WAVE * wid) * GroupIO<TC>::G);
      }
    }
  } else {
    if constexpr (WITH_Q) {
#pragma unroll
      for (int i = 0; i < CR::QJ; ++i) {
        const int idx = tid + NT * i;
        const int r = idx / (K / 8), c8 = (idx % (K / 8)) * 8;
        if (idx < CR::QU && r < nv) R.q[i] = raw_load<TQ>(q + ((t0 + r) * H + h) * K + c8);
        else R.q[i] = raw_zero<TQ>();
      }
    }
#pragma unroll
    for (int i = 0; i < CR::KJ; ++i) {
      const int idx = tid + NT * i;
      const int p = idx % (C / 2), c8 = (idx / (C / 2)) * 8;
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        const int r = 2 * p + rr;
        if (idx < CR::KU && r < nv) R.k[i][rr] = raw_load<TQ>(k + ((t0 + r) * H + h) * K + c8);
        else R.k[i][rr] = raw_zero<TQ>();
      }
    }
#pragma unroll
    for (int i = 0; i < CR::VJ; ++i) {
      const int idx = tid + NT * i;
      const int p = idx % (C / 2), c8 = (idx / (C / 2)) * 8;
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        const int r = 2 * p + rr;
        if (idx < CR::VU && r < nv) R.v[i][rr] = raw_load<TC>(v + ((t0 + r) * H + h) * V + c8);
        else R.v[i][rr] = raw_zero<TC>();
      }
    }
  }
  R.g = 0u;
  R.b = 0u;
  if (tid < C && tid < nv) {
    R.g = ld_raw(gp, (t0 + tid) * H + h, g_dt);
    R.b = ld_raw(bp, (t0 + tid) * H + h, b_dt);
  }
}

// Registers -> LDS.  Wave 0 also forms the chunk vectors: gc = chunk-local
// cumsum of g (fla ops/utils/cumsum.py:58-65), exp(gc), beta and the update
// gate exp(gc_last - gc) (0 beyond the valid rows, chunk_delta_h.py:163-169).
template <typename TC, typename TQ, int K, int V, bool WITH_Q, int NT>
__device__ __forceinline__ void stage_chunk(const ChunkRegs<TC, TQ, K, V, WITH_Q, NT>& R, const unsigned char* raw,
                                            unsigned char* smem, float qs, float ks, int nv, int g_dt, int b_dt) {
  using L = SegLds<TC, K, V, WITH_Q>;
  using CR = ChunkRegs<TC, TQ, K, V, WITH_Q, NT>;
  if constexpr (CR::DIRECT) {
    // the direct global->LDS loads of this wave have landed (the compiler does not
    // track them as a dependency of the LDS reads below)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  TC* s_k = reinterpret_cast<TC*>(smem + L::off_k);
  TC* s_q = reinterpret_cast<TC*>(smem + L::off_q);
  TC* s_kT = reinterpret_cast<TC*>(smem + L::off_kT);
  TC* s_vT = reinterpret_cast<TC*>(smem + L::off_vT);
  float* s_g = reinterpret_cast<float*>(smem + L::off_g);
  const int tid = threadIdx.x;
  if constexpr (WITH_Q) {
#pragma unroll
    for (int i = 0; i < CR::QJ; ++i) {
      const int idx = tid + NT * i;
      if (CR::QJ * NT != CR::QU && idx >= CR::QU) continue;
      const int r = idx / (K / 8), c8 = (idx % (K / 8)) * 8;
      float x[8];
      if constexpr (CR::DIRECT) {
        const Raw8<TQ> g8 = r < nv ? group_from_lds<TQ>(raw + ((size_t)i * NT + WAVE * (tid / WAVE)) * GroupIO<TQ>::G)
                                   : raw_zero<TQ>();
        raw_get8<TQ>(g8, qs, x);
      } else {
        raw_get8<TQ>(R.q[i], qs, x);
      }
      st4<TC>(s_q + r * L::LDK + pcol(c8), x[0], x[1], x[2], x[3]);
      st4<TC>(s_q + r * L::LDK + pcol(c8 + 4), x[4], x[5], x[6], x[7]);
    }
  }
#pragma unroll
  for (int i = 0; i < CR::KJ; ++i) {
    const int idx = tid + NT * i;
    if (CR::KJ * NT != CR::KU && idx >= CR::KU) continue;
    const int p = idx % (C / 2), c8 = (idx / (C / 2)) * 8;
    float x[2][8];
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      if constexpr (CR::DIRECT) {
        const Raw8<TQ> g8 =
            2 * p + rr < nv
                ? group_from_lds<TQ>(raw + CR::RAW_Q + ((size_t)(2 * i + rr) * NT + WAVE * (tid / WAVE)) * GroupIO<TQ>::G)
                : raw_zero<TQ>();
        raw_get8<TQ>(g8, ks, x[rr]);
      } else {
        raw_get8<TQ>(R.k[i][rr], ks, x[rr]);
      }
      TC* row = s_k + (2 * p + rr) * L::LDK;
      st4<TC>(row + pcol(c8), x[rr][0], x[rr][1], x[rr][2], x[rr][3]);
      st4<TC>(row + pcol(c8 + 4), x[rr][4], x[rr][5], x[rr][6], x[rr][7]);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int d = c8 + e;
      st2<TC>(s_kT + d * L::LDT + tcol(d, 2 * p), x[0][e], x[1][e]);
    }
  }
#pragma unroll
  for (int i = 0; i < CR::VJ; ++i) {
    const int idx = tid + NT * i;
    if (CR::VJ * NT != CR::VU && idx >= CR::VU) continue;
    const int p = idx % (C / 2), c8 = (idx / (C / 2)) * 8;
    float x0[8], x1[8];
    if constexpr (CR::DIRECT) {
      const unsigned char* rv = raw + CR::RAW_Q + CR::RAW_K;
      const Raw8<TC> a0 = 2 * p < nv ? group_from_lds<TC>(rv + ((size_t)(2 * i) * NT + WAVE * (tid / WAVE)) * GroupIO<TC>::G)
                                     : raw_zero<TC>();
      const Raw8<TC> a1 = 2 * p + 1 < nv
                              ? group_from_lds<TC>(rv + ((size_t)(2 * i + 1) * NT + WAVE * (tid / WAVE)) * GroupIO<TC>::G)
                              : raw_zero<TC>();
      raw_get8<TC>(a0, 1.f, x0);
      raw_get8<TC>(a1, 1.f, x1);
    } else {
      raw_get8<TC>(R.v[i][0], 1.f, x0);
      raw_get8<TC>(R.v[i][1], 1.f, x1);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int vv = c8 + e;
      st2<TC>(s_vT + vv * L::LDT + tcol(vv, 2 * p), x0[e], x1[e]);
    }
  }
  if (tid < WAVE) {
    float gv = raw_to_f32(R.g, g_dt);
#pragma unroll
    for (int off = 1; off < WAVE; off <<= 1) {
      const float o = __shfl_up(gv, off, WAVE);
      if (tid >= off) gv += o;
    }
    const float gl = __shfl(gv, nv - 1, WAVE);
    s_g[tid] = gv;                                         // gc
    s_g[C + tid] = gexp(gv);                               // exp(gc)
    s_g[2 * C + tid] = raw_to_f32(R.b, b_dt);              // beta
    s_g[3 * C + tid] = tid < nv ? gexp(gl - gv) : 0.f;     // gate
  }
}

// Zero the upper 16x16 tiles of Ai (and Aqk) that operand fragments read
// (col tile 2ks+1 of row tile 2ks): they are never written per chunk.
template <typename TC, int K, int V, bool WITH_Q, int NT>
__device__ __forceinline__ void zero_upper_tiles(unsigned char* smem) {
  using L = SegLds<TC, K, V, WITH_Q>;
  TC* s_Ai = reinterpret_cast<TC*>(smem + L::off_Ai);
  TC* s_Aqk = reinterpret_cast<TC*>(smem + L::off_Aqk);
  for (int idx = threadIdx.x; idx < 2 * 16 * 16; idx += NT) {
    const int tile = idx >> 8, r = (idx >> 4) & 15, c = idx & 15;
    const int row = 32 * tile + r, col = 32 * tile + 16 + c;
    s_Ai[row * L::LDT + pcol(col)] = from_f32<TC>(0.f);
    if constexpr (WITH_Q) s_Aqk[row * L::LDT + pcol(col)] = from_f32<TC>(0.f);
  }
}

// One 16-row block tm of A (beta_i exp(gc_i - gc_j) k_i.k_j, i > j; fp32 for the
// solve, chunk_scaled_dot_kkt.py:57-73) or of Aqk (exp(gc_i - gc_j) q_i.k_j,
// i >= j; rounded to TC, chunk_o.py:109-118).
template <typename TC, int K, int V, bool WITH_Q, bool IS_Q>
__device__ __forceinline__ void kkt_rowblock(unsigned char* smem, int tm) {
  using L = SegLds<TC, K, V, WITH_Q>;
  const TC* s_k = reinterpret_cast<const TC*>(smem + L::off_k);
  const TC* s_q = reinterpret_cast<const TC*>(smem + L::off_q);
  float* s_A = reinterpret_cast<float*>(smem + L::off_A);
  TC* s_Aqk = reinterpret_cast<TC*>(smem + L::off_Aqk);
  const float* s_g = reinterpret_cast<const float*>(smem + L::off_g);
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;
  const TC* asrc = IS_Q ? s_q : s_k;
  Frag<TC> a[K / 32];
#pragma unroll
  for (int ks = 0; ks < K / 32; ++ks) a[ks] = frag_at<TC>(asrc + (16 * tm + lc) * L::LDK + 32 * ks + 8 * lg);
  const int i0 = 16 * tm + 4 * lg;
  const f32x4 gi = *reinterpret_cast<const f32x4*>(s_g + i0);
  f32x4 bi = {1.f, 1.f, 1.f, 1.f};
  if constexpr (!IS_Q) bi = *reinterpret_cast<const f32x4*>(s_g + 2 * C + i0);
  for (int tn = 0; tn <= tm; ++tn) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < K / 32; ++ks) mma(acc, a[ks], frag_at<TC>(s_k + (16 * tn + lc) * L::LDK + 32 * ks + 8 * lg));
    const int j = 16 * tn + lc;
    const float gj = s_g[j];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int i = i0 + jj;
      const bool keep = IS_Q ? i >= j : i > j;
      const float val = keep ? acc[jj] * gexp(gi[jj] - gj) * bi[jj] : 0.f;
      if constexpr (IS_Q) s_Aqk[i * L::LDT + pcol(j)] = from_f32<TC>(val);
      else s_A[i * L::LDA + j] = val;
    }
  }
}

// A (and Aqk) row blocks over the waves: job order A0..A3, Q3..Q0 so that with
// 4 waves each wave gets one A block and the complementary Aqk block.
template <typename TC, int K, int V, bool WITH_Q, int NW>
__device__ __forceinline__ void kkt_phase(unsigned char* smem) {
  constexpr int NJ = WITH_Q ? 8 : 4;
  const int wid = threadIdx.x / WAVE;
  for (int j = wid; j < NJ; j += NW) {
    if (j < 4) kkt_rowblock<TC, K, V, WITH_Q, false>(smem, j);
    else kkt_rowblock<TC, K, V, WITH_Q, true>(smem, 7 - j);
  }
}

// (I + A)^-1 (solve_tril.py:184-331, fp32 throughout, rounded to TC once):
//   diag_solve:  the four 16x16 diagonal blocks D_i = (I + A_ii)^-1 by forward
//                substitution on one wave (lane = one column of one block), in
//                place in s_A, and rounded into s_Ai;
//   chain_solve: column block j of the inverse, X_ij = -D_i sum_{k=j}^{i-1} A_ik X_kj
//                for i = j+1..3, on one wave per j (j = 0, 1, 2); the X_kj stay in
//                registers as the B operand of the next product, so the three
//                chains need no barrier between their steps.
// Ai is stored [t][pcol(t')].
template <typename TC, int K, int V, bool WITH_Q>
__device__ __forceinline__ void diag_solve(unsigned char* smem) {
  using L = SegLds<TC, K, V, WITH_Q>;
  float* s_A = reinterpret_cast<float*>(smem + L::off_A);
  TC* s_Ai = reinterpret_cast<TC*>(smem + L::off_Ai);
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;
  float x[16];
  float* Xb = s_A + (16 * lg) * L::LDA + 16 * lg;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    float s = 0.f;
#pragma unroll
    for (int r = 0; r < i; ++r) s = fmaf(Xb[i * L::LDA + r], x[r], s);
    x[i] = (i == lc) ? 1.f : (i < lc ? 0.f : -s);
  }
  // same wave: the reads above are complete before these writes
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    Xb[i * L::LDA + lc] = x[i];
    s_Ai[(16 * lg + i) * L::LDT + pcol(16 * lg + lc)] = from_f32<TC>(x[i]);
  }
}

template <typename TC, int K, int V, bool WITH_Q>
__device__ __forceinline__ void chain_solve(unsigned char* smem, int j) {
  using L = SegLds<TC, K, V, WITH_Q>;
  const float* s_A = reinterpret_cast<const float*>(smem + L::off_A);
  TC* s_Ai = reinterpret_cast<TC*>(smem + L::off_Ai);
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;
  auto blk = [&](int r, int c) { return s_A + (16 * r) * L::LDA + 16 * c; };
  f32x4 X[3];                                   // X_{j+1,j}, X_{j+2,j}, X_{j+3,j}
  for (int i = j + 1; i < 4; ++i) {
    f32x4 t = {0.f, 0.f, 0.f, 0.f}, r = {0.f, 0.f, 0.f, 0.f};
    mma16_f32_lds(t, blk(i, j), L::LDA, blk(j, j), L::LDA);           // A_ij D_j
#pragma unroll
    for (int k = 1; k < 3; ++k)
      if (j + k < i) mma16_f32_lds_reg(t, blk(i, j + k), L::LDA, X[k - 1]);   // A_ik X_kj
    mma16_f32_lds_reg(r, blk(i, i), L::LDA, t);                       // D_i (...)
    r = -r;
#pragma unroll
    for (int k = 0; k < 3; ++k)
      if (k == i - j - 1) X[k] = r;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
      s_Ai[(16 * i + 4 * lg + jj) * L::LDT + pcol(16 * j + lc)] = from_f32<TC>(r[jj]);
  }
}

// kb^T fragments (kb = k beta exp(gc) with the reference's roundings, wy_fast.py:67-81)
// of the d tiles dt = wid + NW * n; independent of Ai.
template <typename TC, int K, int V, bool WITH_Q, int NW>
struct WFrags {
  static constexpr int ND = (K / 16 + NW - 1) / NW;
  Frag<TC> kb[ND][2];
};
template <typename TC, int K, int V, bool WITH_Q, int NW>
__device__ __forceinline__ void w_frags(const unsigned char* smem, bool beta_lowp, WFrags<TC, K, V, WITH_Q, NW>& F) {
  using L = SegLds<TC, K, V, WITH_Q>;
  const TC* s_kT = reinterpret_cast<const TC*>(smem + L::off_kT);
  const float* s_g = reinterpret_cast<const float*>(smem + L::off_g);
  const int wid = threadIdx.x / WAVE;
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;
#pragma unroll
  for (int n = 0; n < WFrags<TC, K, V, WITH_Q, NW>::ND; ++n) {
    const int dt = wid + NW * n;
    if (dt >= K / 16) break;
    const int d = 16 * dt + lc;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      float x[8];
      lds_get8<TC>(s_kT + d * L::LDT + tchunk(d, 32 * ks + 8 * lg), x);
      const f32x4 b0 = *reinterpret_cast<const f32x4*>(s_g + 2 * C + 32 * ks + 4 * lg);
      const f32x4 b1 = *reinterpret_cast<const f32x4*>(s_g + 2 * C + 32 * ks + 16 + 4 * lg);
      const f32x4 e0 = *reinterpret_cast<const f32x4*>(s_g + C + 32 * ks + 4 * lg);
      const f32x4 e1 = *reinterpret_cast<const f32x4*>(s_g + C + 32 * ks + 16 + 4 * lg);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float v = x[e] * (e < 4 ? b0[e] : b1[e - 4]);
        if (beta_lowp) v = round_to<TC>(v);
        x[e] = v * (e < 4 ? e0[e] : e1[e - 4]);
      }
      F.kb[n][ks] = frag_pack<TC>(x);
    }
  }
}
// w^T = kb^T Ai^T for this wave's d tiles -> s_w[t][pcol(d)]
template <typename TC, int K, int V, bool WITH_Q, int NW>
__device__ __forceinline__ void w_products(unsigned char* smem, const WFrags<TC, K, V, WITH_Q, NW>& F) {
  using L = SegLds<TC, K, V, WITH_Q>;
  TC* s_w = reinterpret_cast<TC*>(smem + L::off_k);
  const TC* s_Ai = reinterpret_cast<const TC*>(smem + L::off_Ai);
  const int wid = threadIdx.x / WAVE;
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;
#pragma unroll
  for (int n = 0; n < WFrags<TC, K, V, WITH_Q, NW>::ND; ++n) {
    const int dt = wid + NW * n;
    if (dt >= K / 16) break;
#pragma unroll
    for (int tn = 0; tn < 4; ++tn) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks <= tn / 2; ++ks)
        mma(acc, F.kb[n][ks], frag_at<TC>(s_Ai + (16 * tn + lc) * L::LDT + 32 * ks + 8 * lg));
      st4<TC>(s_w + (16 * tn + lc) * L::LDK + pcol(16 * dt + 4 * lg), acc[0], acc[1], acc[2], acc[3]);
    }
  }
}

// vb^T fragments (vb = v beta, wy_fast.py:61-65) of V columns v0..v0+15; independent of Ai
template <typename TC, int K, int V, bool WITH_Q>
__device__ __forceinline__ void u_frags(const unsigned char* smem, int v0, Frag<TC> (&vb)[2]) {
  using L = SegLds<TC, K, V, WITH_Q>;
  const TC* s_vT = reinterpret_cast<const TC*>(smem + L::off_vT);
  const float* s_b = reinterpret_cast<const float*>(smem + L::off_g) + 2 * C;
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;
  const int vv = v0 + lc;
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    float x[8];
    lds_get8<TC>(s_vT + vv * L::LDT + tchunk(vv, 32 * ks + 8 * lg), x);
    const f32x4 b0 = *reinterpret_cast<const f32x4*>(s_b + 32 * ks + 4 * lg);
    const f32x4 b1 = *reinterpret_cast<const f32x4*>(s_b + 32 * ks + 16 + 4 * lg);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] *= (e < 4 ? b0[e] : b1[e - 4]);
    vb[ks] = frag_pack<TC>(x);
  }
}
// u (64 rows x 16 columns) = Ai vb, rounded to TC, in accumulator tiles
template <typename TC, int K, int V, bool WITH_Q>
__device__ __forceinline__ void u_products(const unsigned char* smem, const Frag<TC> (&vb)[2], f32x4 (&u)[4]) {
  using L = SegLds<TC, K, V, WITH_Q>;
  const TC* s_Ai = reinterpret_cast<const TC*>(smem + L::off_Ai);
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;
#pragma unroll
  for (int tm = 0; tm < 4; ++tm) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks <= tm / 2; ++ks)
      mma(acc, frag_at<TC>(s_Ai + (16 * tm + lc) * L::LDT + 32 * ks + 8 * lg), vb[ks]);
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = round_to<TC>(acc[j]);
    u[tm] = acc;
  }
}

// S (K x 16*CT, accumulator tiles) <- gamma S + k^T vg, vg given as operand fragments
template <typename TC, int K, int V, bool WITH_Q, int CT>
__device__ __forceinline__ void state_update(f32x4 (&S)[K / 16][CT], const Frag<TC> (&vg)[2][CT],
                                             const unsigned char* smem, float gamma) {
  using L = SegLds<TC, K, V, WITH_Q>;
  const TC* s_kT = reinterpret_cast<const TC*>(smem + L::off_kT);
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;
#pragma unroll
  for (int tt = 0; tt < K / 16; ++tt) {
    const int d = 16 * tt + lc;
    const Frag<TC> a0 = frag_at<TC>(s_kT + d * L::LDT + tchunk(d, 8 * lg));
    const Frag<TC> a1 = frag_at<TC>(s_kT + d * L::LDT + tchunk(d, 32 + 8 * lg));
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      S[tt][ct] *= gamma;
      mma(S[tt][ct], a0, vg[0][ct]);
      mma(S[tt][ct], a1, vg[1][ct]);
    }
  }
}

// Y (64 x 16*CT) -= w X, X given as operand fragments of its K rows
template <typename TC, int K, int V, bool WITH_Q, int CT>
__device__ __forceinline__ void sub_wx(f32x4 (&Y)[4][CT], const Frag<TC> (&xb)[K / 32][CT], const unsigned char* smem) {
  using L = SegLds<TC, K, V, WITH_Q>;
  const TC* s_w = reinterpret_cast<const TC*>(smem + L::off_k);
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;
#pragma unroll
  for (int tm = 0; tm < 4; ++tm) {
    f32x4 p[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) p[ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < K / 32; ++ks) {
      const Frag<TC> a = frag_at<TC>(s_w + (16 * tm + lc) * L::LDK + 32 * ks + 8 * lg);
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) mma(p[ct], a, xb[ks][ct]);
    }
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) Y[tm][ct] -= p[ct];
  }
}

// operand fragments of the gated update input vg = Y * gate (rows t), rounded to TC
template <typename TC, int CT>
__device__ __forceinline__ void gate_frags(const f32x4 (&Y)[4][CT], const float* s_gate, Frag<TC> (&vg)[2][CT]) {
  const int lg = lane_id() >> 4;
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const f32x4 ga = *reinterpret_cast<const f32x4*>(s_gate + 32 * ks + 4 * lg);
    const f32x4 gb = *reinterpret_cast<const f32x4*>(s_gate + 32 * ks + 16 + 4 * lg);
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) vg[ks][ct] = acc_frag<TC>(Y[2 * ks][ct] * ga, Y[2 * ks + 1][ct] * gb);
  }
}

// The output tile of a wave (64 tokens x 16*CT columns, o^T accumulator layout:
// lane holds 4 consecutive columns of token 16*tn + lane%16), held in storage
// precision until it is stored.
template <typename TC, int CT>
struct OutPending {
  typedef typename std::conditional<sizeof(TC) == 2, uint2, f32x4>::type Piece;
  Piece v[4][CT];
  int64_t t0;
  int nv;                     // valid tokens; 0 = nothing pending
  __device__ __forceinline__ void set(int tn, int ct, const f32x4& r) {
    if constexpr (sizeof(TC) == 2) {
      v[tn][ct].x = pack_bf16x2(r[0], r[1]);
      v[tn][ct].y = pack_bf16x2(r[2], r[3]);
    } else {
      v[tn][ct] = r;
    }
  }
  __device__ __forceinline__ void store(TC* o, int H, int h, int V, int vw) {
    const int l = lane_id();
    const int lg = l >> 4, lc = l & 15;
#pragma unroll
    for (int tn = 0; tn < 4; ++tn) {
      const int t = 16 * tn + lc;
      if (t < nv) {
        TC* orow = o + ((t0 + t) * H + h) * V + vw + 4 * lg;
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) *reinterpret_cast<Piece*>(orow + 16 * ct) = v[tn][ct];
      }
    }
    nv = 0;
  }
};

// ---------------------------------------------------------------------------
// seg_out: exact recurrence + output over one segment
// ---------------------------------------------------------------------------
struct SegOutArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* g;
  const void* beta;
  const float* q_scale;
  const float* k_scale;
  int g_dtype, beta_dtype;
  const void* h0;             // [N, H, K, V] or nullptr
  int h0_dtype;
  const float* s_init;        // [NS, H, K, V] fp32 state at each segment start (j >= 1)
  float scale;
  void* o;                    // [B*T, H, V]
  float* ht;                  // [N, H, K, V] or nullptr
};

template <typename TC, typename TQ, int K, int V>
__global__ __launch_bounds__((OutCfg<K, V>::NT)) void seg_out_kernel(SegOutArgs a, SegGeom G) {
  using L = SegLds<TC, K, V, true>;
  constexpr int NW = OutCfg<K, V>::NW, NT = OutCfg<K, V>::NT;
  using CR = ChunkRegs<TC, TQ, K, V, true, NT>;
  constexpr int CT = 1;                 // 16-column tiles per wave
  constexpr int KT = K / 16;
  extern __shared__ __align__(16) unsigned char smem[];
  const TC* s_q = reinterpret_cast<const TC*>(smem + L::off_q);
  const TC* s_Aqk = reinterpret_cast<const TC*>(smem + L::off_Aqk);
  const float* s_g = reinterpret_cast<const float*>(smem + L::off_g);

  const int h = blockIdx.y;
  const int H = G.H;
  const SegLoc sl = locate_seg(blockIdx.x, G);
  if (!sl.ok) return;
  const int wid = threadIdx.x / WAVE;
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;
  const int vw = wid * 16 * CT;         // first V column of this wave
  const float qs = a.q_scale ? a.q_scale[h] : 1.f;
  const float ks_ = a.k_scale ? a.k_scale[h] : 1.f;
  const bool beta_lowp = a.beta_dtype == DT_BF16 && sizeof(TC) == 2;

  // ---- initial state of the segment (lane element (tt, ct, j): row 16*tt + 4*lg + j, column vw + 16*ct + lc)
  f32x4 S[KT][CT];
  {
    const int lane_off = 4 * lg * V + vw + lc;
    if (sl.j == 0 && a.h0 && a.h0_dtype == DT_F32) {
      const float* p = reinterpret_cast<const float*>(a.h0) + ((int64_t)sl.n * H + h) * K * V + lane_off;
#pragma unroll
      for (int tt = 0; tt < KT; ++tt)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
          for (int j = 0; j < 4; ++j) S[tt][ct][j] = p[(16 * tt + j) * V + 16 * ct];
    } else if (sl.j == 0 && a.h0) {
      const bf16* p = reinterpret_cast<const bf16*>(a.h0) + ((int64_t)sl.n * H + h) * K * V + lane_off;
#pragma unroll
      for (int tt = 0; tt < KT; ++tt)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
          for (int j = 0; j < 4; ++j) S[tt][ct][j] = (float)p[(16 * tt + j) * V + 16 * ct];
    } else if (sl.j > 0) {
      const float* p = a.s_init + ((int64_t)blockIdx.x * H + h) * K * V + lane_off;
#pragma unroll
      for (int tt = 0; tt < KT; ++tt)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
          for (int j = 0; j < 4; ++j) S[tt][ct][j] = p[(16 * tt + j) * V + 16 * ct];
    } else {
#pragma unroll
      for (int tt = 0; tt < KT; ++tt)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) S[tt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  zero_upper_tiles<TC, K, V, true, NT>(smem);

  CR cur;
  unsigned char* raw = smem + L::raw_off;
  int64_t t0 = sl.bos + sl.c0 * C;
  int nv = (int)min((int64_t)C, sl.eos - t0);
  load_chunk<TC, TQ, K, V, true, NT>(cur, raw, a.q, a.k, a.v, a.g, a.beta, a.g_dtype, a.beta_dtype, t0, nv, h, H);
  TC* o = reinterpret_cast<TC*>(a.o);
  OutPending<TC, CT> op;
  op.nv = 0;

  for (int ci = 0; ci < sl.nch; ++ci) {
    stage_chunk<TC, TQ, K, V, true, NT>(cur, raw, smem, qs, ks_, nv, a.g_dtype, a.beta_dtype);
    op.store(o, H, h, V, vw);
    lds_barrier();
    const int64_t t0c = t0;
    const int nvc = nv;
    if (ci + 1 < sl.nch) {
      t0 += C;
      nv = (int)min((int64_t)C, sl.eos - t0);
      load_chunk<TC, TQ, K, V, true, NT>(cur, raw, a.q, a.k, a.v, a.g, a.beta, a.g_dtype, a.beta_dtype, t0, nv, h, H);
    }
    kkt_phase<TC, K, V, true, NW>(smem);
    lds_barrier();

    // ---- h = S rounded (the snapshot of chunk_delta_h.py:129-139) as operand fragments
    Frag<TC> hb[K / 32][CT];
#pragma unroll
    for (int ks = 0; ks < K / 32; ++ks) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) hb[ks][ct] = acc_frag<TC>(S[2 * ks][ct], S[2 * ks + 1][ct]);
    }
    // ---- o1^T = h^T q^T (chunk_o.py:84-101)
    f32x4 o1[4][CT];
    auto inter_chunk_out = [&]() {
#pragma unroll
      for (int tn = 0; tn < 4; ++tn) {
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) o1[tn][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < K / 32; ++ks) {
          const Frag<TC> bq = frag_at<TC>(s_q + (16 * tn + lc) * L::LDK + 32 * ks + 8 * lg);
#pragma unroll
          for (int ct = 0; ct < CT; ++ct) mma(o1[tn][ct], hb[ks][ct], bq);
        }
      }
    };
    constexpr int W0 = NW - 1;            // the solver wave; waves W0, W0-1, W0-2 run the column chains
    const int role = W0 - wid;
    if (role == 0) diag_solve<TC, K, V, true>(smem);
    lds_barrier();   // diagonal blocks
    if (role < 3) chain_solve<TC, K, V, true>(smem, role);
    WFrags<TC, K, V, true, NW> wf;
    w_frags<TC, K, V, true, NW>(smem, beta_lowp, wf);
    Frag<TC> vb[CT][2];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) u_frags<TC, K, V, true>(smem, vw + 16 * ct, vb[ct]);
    lds_barrier();   // Ai complete

    w_products<TC, K, V, true, NW>(smem, wf);
    f32x4 Y[4][CT];
    {
      f32x4 u[4];
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        u_products<TC, K, V, true>(smem, vb[ct], u);
#pragma unroll
        for (int tm = 0; tm < 4; ++tm) Y[tm][ct] = u[tm];
      }
    }
    lds_barrier();   // w complete

    // ---- v' = u - w h                                   (chunk_delta_h.py:141-157)
    sub_wx<TC, K, V, true, CT>(Y, hb, smem);
    inter_chunk_out();

    // ---- o^T = scale (o1^T exp(gc) + v_new^T Aqk^T)     (chunk_o.py:102-128); stored
    //      after the next chunk is staged, so that no wait for loads covers the stores
    op.t0 = t0c;
    op.nv = nvc;
    Frag<TC> vn[2][CT];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) vn[ks][ct] = acc_frag<TC>(Y[2 * ks][ct], Y[2 * ks + 1][ct]);
    }
#pragma unroll
    for (int tn = 0; tn < 4; ++tn) {
      const int t = 16 * tn + lc;
      f32x4 o2[CT];
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) o2[ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        if (ks <= tn / 2) {
          const Frag<TC> ba = frag_at<TC>(s_Aqk + t * L::LDT + 32 * ks + 8 * lg);
#pragma unroll
          for (int ct = 0; ct < CT; ++ct) mma(o2[ct], vn[ks][ct], ba);
        }
      }
      const float eg = s_g[C + t] * a.scale;
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) op.set(tn, ct, o1[tn][ct] * eg + o2[ct] * a.scale);
    }

    // ---- S = exp(g_last) S + k^T (v' exp(g_last - gc))   (chunk_delta_h.py:163-211)
    Frag<TC> vg[2][CT];
    gate_frags<TC, CT>(Y, s_g + 3 * C, vg);
    state_update<TC, K, V, true, CT>(S, vg, smem, gexp(s_g[nvc - 1]));
    lds_barrier();   // LDS is restaged for the next chunk
  }

  op.store(o, H, h, V, vw);
  if (a.ht && sl.j == sl.nseg - 1) {
    float* p = a.ht + ((int64_t)sl.n * H + h) * K * V + 4 * lg * V + vw + lc;
#pragma unroll
    for (int tt = 0; tt < KT; ++tt)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int j = 0; j < 4; ++j) p[(16 * tt + j) * V + 16 * ct] = S[tt][ct][j];
  }
}

// ---------------------------------------------------------------------------
// seg_trans: affine map [M | R] of one segment (all but the last segment of a sequence)
// ---------------------------------------------------------------------------
struct SegTransArgs {
  const void* k;
  const void* v;
  const void* g;
  const void* beta;
  const float* k_scale;
  int g_dtype, beta_dtype;
  float* M;                   // [NS, H, K, K]
  float* R;                   // [NS, H, K, V]
};

template <typename TC, typename TQ, int K, int V>
__global__ __launch_bounds__((TransCfg<K, V>::NT)) void seg_trans_kernel(SegTransArgs a, SegGeom G) {
  using L = SegLds<TC, K, V, false>;
  constexpr int NW = TransCfg<K, V>::NW, NT = TransCfg<K, V>::NT;
  using CR = ChunkRegs<TC, TQ, K, V, false, NT>;
  constexpr int XC = K + V;             // columns of [M | R]
  static_assert(XC % 32 == 0, "K + V must be a multiple of 32");
  constexpr int CT = 2;                 // 16-column tiles per wave
  constexpr int KT = K / 16;
  extern __shared__ __align__(16) unsigned char smem[];
  const float* s_g = reinterpret_cast<const float*>(smem + L::off_g);

  const int h = blockIdx.y;
  const int H = G.H;
  const SegLoc sl = locate_seg(blockIdx.x, G);
  if (!sl.ok || sl.j == sl.nseg - 1) return;
  const int wid = threadIdx.x / WAVE;
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;
  const int xw = wid * 16 * CT;         // first column of [M | R] owned by this wave
  const float ks_ = a.k_scale ? a.k_scale[h] : 1.f;
  const bool beta_lowp = a.beta_dtype == DT_BF16 && sizeof(TC) == 2;

  f32x4 X[KT][CT];
#pragma unroll
  for (int tt = 0; tt < KT; ++tt) {
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
#pragma unroll
      for (int j = 0; j < 4; ++j) X[tt][ct][j] = (16 * tt + 4 * lg + j == xw + 16 * ct + lc) ? 1.f : 0.f;
    }
  }
  zero_upper_tiles<TC, K, V, false, NT>(smem);

  CR cur;
  unsigned char* raw = smem + L::raw_off;
  int64_t t0 = sl.bos + sl.c0 * C;
  int nv = (int)min((int64_t)C, sl.eos - t0);
  load_chunk<TC, TQ, K, V, false, NT>(cur, raw, nullptr, a.k, a.v, a.g, a.beta, a.g_dtype, a.beta_dtype, t0, nv, h,
                                      H);
  for (int ci = 0; ci < sl.nch; ++ci) {
    stage_chunk<TC, TQ, K, V, false, NT>(cur, raw, smem, 1.f, ks_, nv, a.g_dtype, a.beta_dtype);
    lds_barrier();
    const int nvc = nv;
    if (ci + 1 < sl.nch) {
      t0 += C;
      nv = (int)min((int64_t)C, sl.eos - t0);
      load_chunk<TC, TQ, K, V, false, NT>(cur, raw, nullptr, a.k, a.v, a.g, a.beta, a.g_dtype, a.beta_dtype, t0, nv,
                                          h, H);
    }
    kkt_phase<TC, K, V, false, NW>(smem);
    lds_barrier();
    constexpr int W0 = NW - 1;
    const int role = W0 - wid;
    if (role == 0) diag_solve<TC, K, V, false>(smem);
    lds_barrier();   // diagonal blocks
    if (role < 3) chain_solve<TC, K, V, false>(smem, role);
    WFrags<TC, K, V, false, NW> wf;
    w_frags<TC, K, V, false, NW>(smem, beta_lowp, wf);
    Frag<TC> vb[CT][2];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      const int c0 = xw + 16 * ct;
      if (c0 >= K) u_frags<TC, K, V, false>(smem, c0 - K, vb[ct]);
    }
    lds_barrier();   // Ai complete
    w_products<TC, K, V, false, NW>(smem, wf);
    f32x4 Y[4][CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      const int c0 = xw + 16 * ct;
      if (c0 >= K) {
        f32x4 u[4];
        u_products<TC, K, V, false>(smem, vb[ct], u);
#pragma unroll
        for (int tm = 0; tm < 4; ++tm) Y[tm][ct] = u[tm];
      } else {
#pragma unroll
        for (int tm = 0; tm < 4; ++tm) Y[tm][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
    lds_barrier();   // w complete
    __builtin_amdgcn_sched_barrier(0);
    Frag<TC> xb[K / 32][CT];
#pragma unroll
    for (int ks = 0; ks < K / 32; ++ks) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) xb[ks][ct] = acc_frag<TC>(X[2 * ks][ct], X[2 * ks + 1][ct]);
    }
    sub_wx<TC, K, V, false, CT>(Y, xb, smem);
    __builtin_amdgcn_sched_barrier(0);
    Frag<TC> yg[2][CT];
    gate_frags<TC, CT>(Y, s_g + 3 * C, yg);
    state_update<TC, K, V, false, CT>(X, yg, smem, gexp(s_g[nvc - 1]));
    lds_barrier();
  }

  const int64_t s = blockIdx.x;
  float* pm = a.M + (s * H + h) * K * K + 4 * lg * K + xw + lc;
  float* pr = a.R + (s * H + h) * K * V + 4 * lg * V + xw - K + lc;
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    if (xw + 16 * ct < K) {
#pragma unroll
      for (int tt = 0; tt < KT; ++tt)
#pragma unroll
        for (int j = 0; j < 4; ++j) pm[(16 * tt + j) * K + 16 * ct] = X[tt][ct][j];
    } else {
#pragma unroll
      for (int tt = 0; tt < KT; ++tt)
#pragma unroll
        for (int j = 0; j < 4; ++j) pr[(16 * tt + j) * V + 16 * ct] = X[tt][ct][j];
    }
  }
}

// ---------------------------------------------------------------------------
// seg_combine: S_{j+1} = M_j S_j + R_j over the segments of a sequence, 16 V
// columns per workgroup, fp32 (v_mfma_f32_16x16x4f32).  Also writes
// final_state of sequences without tokens.
// ---------------------------------------------------------------------------
struct SegCombineArgs {
  const float* M;
  const float* R;
  const void* h0;
  int h0_dtype;
  float* s_init;              // out [NS, H, K, V]
  float* ht;                  // final_state, written here only for empty sequences
  int V;
};

template <int K>
__global__ __launch_bounds__(NT_COMB) void seg_combine_kernel(SegCombineArgs a, SegGeom G, int total) {
  constexpr int RT = K / 16 / NW_COMB >= 1 ? K / 16 / NW_COMB : 1;   // row tiles per wave
  constexpr int NWA = K / 16 / RT;                          // active waves
  __shared__ __align__(16) float s_S[K][16];
  const int V = a.V;
  const int nvt = V / 16;
  // XCD-aware order: the V slices of one head run on one XCD and share M through its L2
  const int per_xcd = gridDim.x / 8;
  const int o_idx = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (o_idx >= total) return;
  const int unit = o_idx / nvt;
  const int v0 = (o_idx % nvt) * 16;
  const int H = G.H;
  const int n = unit / H, h = unit % H;
  const int wid = threadIdx.x / WAVE;
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;

  int nseg, s_first;
  if (G.cu == nullptr) {
    nseg = G.T > 0 ? G.nseg_fixed : 0;
    s_first = n * G.nseg_fixed;
  } else {
    nseg = G.seg_off[n + 1] - G.seg_off[n];
    s_first = G.seg_off[n];
  }
  for (int idx = threadIdx.x; idx < K * 16; idx += NT_COMB) {
    const int r = idx / 16, c = idx % 16;
    float x = 0.f;
    if (a.h0) {
      const int64_t off = (((int64_t)n * H + h) * K + r) * V + v0 + c;
      x = a.h0_dtype == DT_F32 ? reinterpret_cast<const float*>(a.h0)[off]
                               : (float)reinterpret_cast<const bf16*>(a.h0)[off];
    }
    s_S[r][c] = x;
  }
  if (nseg == 0) {
    if (a.ht) {
      __syncthreads();
      for (int idx = threadIdx.x; idx < K * 16; idx += NT_COMB) {
        const int r = idx / 16, c = idx % 16;
        a.ht[(((int64_t)n * H + h) * K + r) * V + v0 + c] = s_S[r][c];
      }
    }
    return;
  }
  __syncthreads();
  for (int j = 0; j + 1 < nseg; ++j) {
    const int64_t s = s_first + j;
    const float* Ms = a.M + (s * H + h) * K * K;
    const float* Rs = a.R + (s * H + h) * K * V;
    f32x4 acc[RT];
    if (wid < NWA) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const int r0 = 16 * (wid * RT + rt);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) acc[rt][jj] = Rs[(int64_t)(r0 + 4 * lg + jj) * V + v0 + lc];
#pragma unroll 4
        for (int kk = 0; kk < K / 16; ++kk) {
          const f32x4 m = *reinterpret_cast<const f32x4*>(Ms + (int64_t)(r0 + lc) * K + 16 * kk + 4 * lg);
#pragma unroll
          for (int qq = 0; qq < 4; ++qq)
            acc[rt] = __builtin_amdgcn_mfma_f32_16x16x4f32(m[qq], s_S[16 * kk + 4 * lg + qq][lc], acc[rt], 0, 0, 0);
        }
      }
    }
    __syncthreads();
    if (wid < NWA) {
      float* out = a.s_init + ((s + 1) * H + h) * K * V;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const int r0 = 16 * (wid * RT + rt);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int r = r0 + 4 * lg + jj;
          s_S[r][lc] = acc[rt][jj];
          out[(int64_t)r * V + v0 + lc] = acc[rt][jj];
        }
      }
    }
    __syncthreads();
  }
}

__global__ void seg_map_kernel(const int64_t* __restrict__ cu, int N, int L, int32_t* __restrict__ chunk_off,
                               int32_t* __restrict__ seg_off) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  int32_t ca = 0, sa = 0;
  chunk_off[0] = 0;
  seg_off[0] = 0;
  for (int n = 0; n < N; ++n) {
    const int64_t len = cu[n + 1] - cu[n];
    const int32_t nc = (int32_t)((len + C - 1) / C);
    ca += nc;
    sa += (nc + L - 1) / L;
    chunk_off[n + 1] = ca;
    seg_off[n + 1] = sa;
  }
}

template <typename Kern>
int set_lds(Kern kern, size_t bytes) {
  if (bytes > 64 * 1024) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)bytes) != hipSuccess)
      return -1;
  }
  return 0;
}

template <typename TC, typename TQ, int K, int V>
int launch_seg_t(const SegFwdArgs& p, hipStream_t s) {
  SegGeom G{p.cu, p.chunk_off, p.seg_off, p.N, p.T, p.H, p.L, p.nseg_fixed};
  const dim3 grid((unsigned)p.ns_grid, (unsigned)p.H);
  auto mark = [&](int i) { return p.events == nullptr || hipEventRecord(p.events[i], s) == hipSuccess; };
  if (!mark(0)) return -1;
  if (p.run_trans) {
    using LT = SegLds<TC, K, V, false>;
    constexpr size_t lds = LT::raw_off + ChunkRegs<TC, TQ, K, V, false, TransCfg<K, V>::NT>::RAW;
    static_assert(lds <= 160 * 1024, "seg_trans tile does not fit in LDS");
    auto kt = seg_trans_kernel<TC, TQ, K, V>;
    if (set_lds(kt, lds)) return -1;
    SegTransArgs ta{p.k, p.v, p.g, p.beta, p.k_scale, p.g_dtype, p.beta_dtype, p.M, p.R};
    hipLaunchKernelGGL(kt, grid, dim3(TransCfg<K, V>::NT), lds, s, ta, G);
    if (hipGetLastError() != hipSuccess) return -1;
  }
  if (!mark(1)) return -1;
  if (p.run_combine) {
    const int total = p.N * p.H * (V / 16);
    const int cgrid = (total + 7) / 8 * 8;
    SegCombineArgs ca{p.M, p.R, p.h0, p.h0_dtype, p.s_init, p.ht, V};
    hipLaunchKernelGGL(seg_combine_kernel<K>, dim3(cgrid), dim3(NT_COMB), 0, s, ca, G, total);
    if (hipGetLastError() != hipSuccess) return -1;
  }
  if (!mark(2)) return -1;
  if (p.ns_grid > 0) {
    using LO = SegLds<TC, K, V, true>;
    constexpr size_t lds = LO::raw_off + ChunkRegs<TC, TQ, K, V, true, OutCfg<K, V>::NT>::RAW;
    static_assert(lds <= 160 * 1024, "seg_out tile does not fit in LDS");
    auto ko = seg_out_kernel<TC, TQ, K, V>;
    if (set_lds(ko, lds)) return -1;
    SegOutArgs oa{p.q, p.k, p.v, p.g, p.beta, p.q_scale, p.k_scale, p.g_dtype, p.beta_dtype,
                  p.h0, p.h0_dtype, p.s_init, p.scale, p.o, p.ht};
    hipLaunchKernelGGL(ko, grid, dim3(OutCfg<K, V>::NT), lds, s, oa, G);
    if (hipGetLastError() != hipSuccess) return -1;
  }
  if (!mark(3)) return -1;
  return 0;
}

}  // namespace

bool seg_fwd_supported(int compute_dtype, int K, int V) {
  if (!(K == 64 || K == 128) || !(V == 64 || V == 128)) return false;
  return compute_dtype == DT_BF16 || K == 64;
}

int launch_seg_map(const int64_t* cu, int N, int L, int32_t* chunk_off, int32_t* seg_off, hipStream_t s) {
  hipLaunchKernelGGL(seg_map_kernel, dim3(1), dim3(64), 0, s, cu, N, L, chunk_off, seg_off);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_seg_fwd(const SegFwdArgs& p, int compute_dtype, int qk_dtype, int K, int V, hipStream_t s) {
#define KGDN_SEG_CASE(TC, TQ, KK, VV) \
  if (K == KK && V == VV) return launch_seg_t<TC, TQ, KK, VV>(p, s);
#define KGDN_SEG_SHAPES(TC, TQ) \
  KGDN_SEG_CASE(TC, TQ, 64, 64) KGDN_SEG_CASE(TC, TQ, 64, 128) \
  KGDN_SEG_CASE(TC, TQ, 128, 64) KGDN_SEG_CASE(TC, TQ, 128, 128)
  // fp32 tiles of K = 128 exceed the LDS of one CU: those shapes run the staged kernels
  if (compute_dtype == DT_F32 && qk_dtype == DT_F32) { KGDN_SEG_CASE(float, float, 64, 64) KGDN_SEG_CASE(float, float, 64, 128) }
  if (compute_dtype == DT_BF16 && qk_dtype == DT_BF16) { KGDN_SEG_SHAPES(bf16, bf16) }
  if (compute_dtype == DT_BF16 && qk_dtype == DT_F8E4M3) { KGDN_SEG_SHAPES(bf16, uint8_t) }
#undef KGDN_SEG_SHAPES
#undef KGDN_SEG_CASE
  return -2;
}

}  // namespace kgdn
