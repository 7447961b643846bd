// Segment-parallel fused forward of the chunked GatedDeltaNet (the path behind
// kairos_gdn_chunk_fwd for bf16 compute: bf16 v with bf16 or fp8 e4m3 q/k).
// It computes what the reference's six stages compute (fla
// ops/gated_delta_rule/chunk.py:16-67: cumsum, K.K^T, solve_tril, w/u,
// chunk_fwd_h, chunk_fwd_o); of their intermediates only the chunk-local
// inverse Ai = (I + A)^-1 (bf16, as solve_tril stores it) goes through HBM.
//
// Every sequence is cut into segments of L consecutive 64-token chunks, so
// that (segment, head) work items fill the GPU even for one long sequence.
// Per chunk c the state recurrence is affine in the incoming state S:
//     S' = M_c S + R_c,   M_c = g I - k^T diag(gate) w,   R_c = k^T diag(gate) u,
// with g = exp(gc_last) and gate_t = exp(gc_last - gc_t) (chunk_delta_h.py:163-211).
//
//   seg_prep_kernel     (chunk, head), fully parallel: chunk-local cumsum, A =
//                       beta exp(gc_i - gc_j) k_i.k_j and its inverse (I + A)^-1
//                       in fp32, stored as bf16 (chunk_scaled_dot_kkt.py,
//                       solve_tril.py).  Keeping the triangular solve out of the
//                       two serial kernels below takes it off their critical path.
//   seg_trans_kernel    (segment, head): forms w and u from Ai and accumulates the
//                       segment's affine map [M | R] (K x (K+V), fp32) from [I | 0].
//   seg_combine_kernel  (sequence, head, 16 V columns): serial over segments,
//                       S_{j+1} = M_j S_j + R_j in fp32, from initial_state.
//   seg_out_kernel      (segment, head): forms w, u and Aqk, runs the exact
//                       recurrence of chunk_delta_h.py from the segment's initial
//                       state and emits o (chunk_o.py:84-128) and, for the last
//                       segment, final_state.
//
// Workgroup: seg_out runs one wave per 16 V columns, seg_trans one wave per 32
// columns of [M | R]; each wave keeps its fp32 state tile (K rows) in VGPRs in
// the MFMA accumulator layout for the whole segment.
//
// Chunk inputs.  q, k, v and Ai of a chunk live in LDS as row-major tiles (row
// = token) whose 16-byte chunks are XOR-swizzled by row.  They arrive by direct
// global->LDS loads (global_load_lds_dwordx4) into one of two buffers while the
// previous chunk computes from the other, so no register holds them and no
// wait stalls on them until the chunk is used.  Every MFMA operand is read
// straight from these tiles:
//   * K.K^T, Q.K^T and Ai as an operand: one 16-byte row fragment per lane;
//   * q as the partner of the state (o = q h): two 8-byte pieces per lane, in
//     the K order in which an accumulator tile pair becomes an operand
//     ({4*lg..+3} and {16+4*lg..+3} of a 32-wide step, lg = lane/16);
//   * k^T, (k beta e^g)^T and (v beta)^T, whose contraction index is the token:
//     ds_read_b64_tr_b16 transposes a 4-token x 16-column block across the 16
//     lanes of a lane group (lane j receives column j of the 4 rows).
// fp8 q/k are converted once per chunk into bf16 tiles of the same layout.
#include <type_traits>

#include "gdn_common.hpp"
#include "gdn_kernels.h"

namespace kgdn {

namespace {

template <int K, int V> struct OutCfg { static constexpr int NW = V / 16, NT = 64 * NW; };
template <int K, int V> struct TransCfg { static constexpr int NW = (K + V) / 32, NT = 64 * NW; };

// Workgroup barrier that orders LDS only: this wave's LDS reads and writes are
// complete (lgkmcnt(0)), then s_barrier.  __syncthreads(), and even a
// workgroup fence on LDS alone, also waits for vmcnt(0), because the direct
// global->LDS loads count as LDS writes: every barrier would then wait for the
// next chunk's prefetch and the output stores.  The waves of a workgroup share
// nothing but LDS, and the direct loads are waited for explicitly
// (wait_loads) before the barrier that publishes them.  The empty asm
// statements keep the compiler from moving memory accesses across the barrier.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);          // lgkmcnt(0); vmcnt, expcnt at their maxima
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Column permutation of the LDS tiles the kernel writes itself (w, Ai, Aqk):
// logical column 16*hh + 4*lg + j of a 32-column block sits at 8*lg + 4*hh + j,
// so the pair-of-accumulator-tiles K order is one 16-byte read.
__device__ __forceinline__ int pcol(int c) {
  return (c & ~31) | (((c >> 2) & 3) << 3) | (((c >> 4) & 1) << 2) | (c & 3);
}

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(1))) void gmem_void;
typedef __attribute__((address_space(3))) void lmem_void;

// LDS byte address of a pointer into this workgroup's LDS
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const lmem_void*)p;
}

template <typename TC>
__device__ __forceinline__ Frag<TC> frag_at(const TC* p) {
  Frag<TC> f;
  f.v = *reinterpret_cast<const bf16x8*>(p);
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

// operand fragment from 8 floats, rounded to bf16
__device__ __forceinline__ Frag<bf16> frag_pack(const float (&x)[8]) {
  Frag<bf16> f;
  bf16x8 v = {(bf16)x[0], (bf16)x[1], (bf16)x[2], (bf16)x[3], (bf16)x[4], (bf16)x[5], (bf16)x[6], (bf16)x[7]};
  f.v = v;
  return f;
}
__device__ __forceinline__ void frag_unpack(const Frag<bf16>& f, float (&x)[8]) {
  const uint4 r = __builtin_bit_cast(uint4, f.v);
  x[0] = bf16_lo(r.x); x[1] = bf16_hi(r.x); x[2] = bf16_lo(r.y); x[3] = bf16_hi(r.y);
  x[4] = bf16_lo(r.z); x[5] = bf16_hi(r.z); x[6] = bf16_lo(r.w); x[7] = bf16_hi(r.w);
}
// Operand fragment from two accumulator tiles (rows 4*lg+j of tile a, then of tile b), rounded to bf16.
__device__ __forceinline__ Frag<bf16> acc_frag(const f32x4& a, const f32x4& b) {
  Frag<bf16> f;
  bf16x8 v = {(bf16)a[0], (bf16)a[1], (bf16)a[2], (bf16)a[3], (bf16)b[0], (bf16)b[1], (bf16)b[2], (bf16)b[3]};
  f.v = v;
  return f;
}

// ---------------------------------------------------------------------------
// swizzled row-major bf16 tiles [64 rows][NC columns]: 16-byte chunk c of row r
// sits at chunk position c ^ swz(r).  Rows of 256 bytes (NC = 128) take
// swz(r) = r mod 16; rows of 128 bytes (NC = 64, two rows per 256-byte bank
// row) take a permutation of r/2 that keeps 16 consecutive rows on distinct
// banks for 16-byte row reads.
// ---------------------------------------------------------------------------
template <int NC>
struct Tile {
  static_assert(NC == 64 || NC == 128, "tiles are 64 or 128 columns wide");
  static constexpr int CPR = NC / 8;                  // 16-byte chunks per row
  __device__ static __forceinline__ int swz(int r) {
    if constexpr (NC == 64) return (((r >> 1) & 3) << 1) | ((r >> 3) & 1);
    else return r & (CPR - 1);
  }
  // element offset of chunk c8 (columns 8*c8 .. +7) of row r
  __device__ static __forceinline__ int off(int r, int c8) { return r * NC + ((c8 ^ swz(r)) << 3); }
  // 8 consecutive columns 8*c8 .. +7 of row r
  __device__ static __forceinline__ Frag<bf16> row8(const bf16* t, int r, int c8) { return frag_at<bf16>(t + off(r, c8)); }
  // columns {32ks + 4lg .. +3} and {32ks + 16 + 4lg .. +3} of row r (the accumulator K order)
  __device__ static __forceinline__ Frag<bf16> row_acc_order(const bf16* t, int r, int ks, int lg) {
    const int c8a = 4 * ks + (lg >> 1), c8b = c8a + 2, h = (lg & 1) * 4;
    const uint2 a = *reinterpret_cast<const uint2*>(t + off(r, c8a) + h);
    const uint2 b = *reinterpret_cast<const uint2*>(t + off(r, c8b) + h);
    Frag<bf16> f;
    f.v = __builtin_bit_cast(bf16x8, make_uint4(a.x, a.y, b.x, b.y));
    return f;
  }
  // Transposed fragment: lane (l%16 = j, l/16 = lg) gets t[32ks + 4lg + e][c0 + j] (e = 0..3) and
  // t[32ks + 16 + 4lg + e][c0 + j].  ds_read_b64_tr_b16 within a 16-lane group: lane i reads 4
  // columns of one row, lane j receives element j%4 of lane 4e + j/4's read as its element e.
  // col_tr_addr gives the LDS byte addresses of the two reads (rows r0 and r0 + 16).
  __device__ static __forceinline__ void col_tr_addr(const bf16* t, int ks, int c0, uint32_t& a0, uint32_t& a1) {
    const int l = lane_id();
    const int lg = l >> 4, i = l & 15;
    const int col = c0 + 4 * (i & 3);
    const int r0 = 32 * ks + 4 * lg + (i >> 2);
    const int r1 = r0 + 16;
    a0 = lds_addr(t + off(r0, col >> 3) + (col & 7));
    a1 = lds_addr(t + off(r1, col >> 3) + (col & 7));
  }
};

// Transposed fragments through inline asm.  The compiler's wait tracking treats
// ds_read_b64_tr_b16 (the builtin) as a possible reader of whatever an
// in-flight direct global->LDS load writes, and puts a vmcnt(0) before it --
// a wait for the next chunk's prefetch in the middle of the current chunk.
// The asm form is outside that tracking; it waits for its own reads
// (lgkmcnt(0)) before returning, so its results are ready when used.
__device__ __forceinline__ Frag<bf16> tr_pair(u32x2 a, u32x2 b) {
  Frag<bf16> f;
  f.v = __builtin_bit_cast(bf16x8, make_uint4(a.x, a.y, b.x, b.y));
  return f;
}
// N = 2 fragments from 4 addresses (fragment f from reads 2f, 2f + 1)
__device__ __forceinline__ void tr_read2(const uint32_t (&a)[4], Frag<bf16> (&f)[2]) {
  u32x2 r0, r1, r2, r3;
  asm volatile(
      "ds_read_b64_tr_b16 %0, %4\n\t"
      "ds_read_b64_tr_b16 %1, %5\n\t"
      "ds_read_b64_tr_b16 %2, %6\n\t"
      "ds_read_b64_tr_b16 %3, %7\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(r0), "=&v"(r1), "=&v"(r2), "=&v"(r3)
      : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]));
  f[0] = tr_pair(r0, r1);
  f[1] = tr_pair(r2, r3);
}
// N = 4 fragments from 8 addresses
__device__ __forceinline__ void tr_read4(const uint32_t (&a)[8], Frag<bf16> (&f)[4]) {
  u32x2 r0, r1, r2, r3, r4, r5, r6, r7;
  asm volatile(
      "ds_read_b64_tr_b16 %0, %8\n\t"
      "ds_read_b64_tr_b16 %1, %9\n\t"
      "ds_read_b64_tr_b16 %2, %10\n\t"
      "ds_read_b64_tr_b16 %3, %11\n\t"
      "ds_read_b64_tr_b16 %4, %12\n\t"
      "ds_read_b64_tr_b16 %5, %13\n\t"
      "ds_read_b64_tr_b16 %6, %14\n\t"
      "ds_read_b64_tr_b16 %7, %15\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(r0), "=&v"(r1), "=&v"(r2), "=&v"(r3), "=&v"(r4), "=&v"(r5), "=&v"(r6), "=&v"(r7)
      : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]), "v"(a[6]), "v"(a[7]));
  f[0] = tr_pair(r0, r1);
  f[1] = tr_pair(r2, r3);
  f[2] = tr_pair(r4, r5);
  f[3] = tr_pair(r6, r7);
}
// both K steps (ks = 0, 1) of the transposed fragment of columns c0 .. c0 + 15
template <int NC>
__device__ __forceinline__ void col_tr2(const bf16* t, int c0, Frag<bf16> (&f)[2]) {
  uint32_t a[4];
  Tile<NC>::col_tr_addr(t, 0, c0, a[0], a[1]);
  Tile<NC>::col_tr_addr(t, 1, c0, a[2], a[3]);
  tr_read2(a, f);
}

// ---------------------------------------------------------------------------
// problem geometry shared by the kernels
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
  int64_t cbase;              // global index of the sequence's first chunk (rows of Ai)
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
    r.cbase = (int64_t)r.n * ((G.T + C - 1) / C);
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
    r.cbase = G.chunk_off[lo];
  }
  const int64_t nc = (r.eos - r.bos + C - 1) / C;
  r.c0 = (int64_t)r.j * G.L;
  r.nch = (int)min((int64_t)G.L, nc - r.c0);
  r.ok = r.nch > 0;
  return r;
}

// ---------------------------------------------------------------------------
// LDS layouts
// ---------------------------------------------------------------------------
// seg_trans / seg_out
template <typename TQ, int K, int V, bool WITH_Q>
struct SegLds {
  static constexpr bool FP8 = sizeof(TQ) == 1;
  static constexpr int LDK = K + 8;        // row stride of s_w [64][K] (pcol order)
  static constexpr int LDT = C + 8;        // row stride of s_Aqk [64][64] (pcol order)
  static constexpr size_t a16(size_t x) { return (x + 15) / 16 * 16; }
  // one input buffer: q (if WITH_Q), k as loaded (TQ), v (bf16), Ai (bf16)
  static constexpr size_t qk_in = (size_t)C * K * sizeof(TQ);
  static constexpr size_t buf_q = 0;
  static constexpr size_t buf_k = WITH_Q ? qk_in : 0;
  static constexpr size_t buf_v = buf_k + qk_in;
  static constexpr size_t buf_ai = buf_v + (size_t)C * V * 2;
  static constexpr size_t buf_bytes = a16(buf_ai + (size_t)C * C * 2);
  static constexpr size_t off_buf = 0;                                   // two input buffers
  static constexpr size_t off_cq = off_buf + 2 * buf_bytes;              // fp8: bf16 q / k tiles
  static constexpr size_t off_ck = off_cq + (FP8 && WITH_Q ? (size_t)C * K * 2 : 0);
  static constexpr size_t off_w = off_ck + (FP8 ? (size_t)C * K * 2 : 0);
  static constexpr size_t off_Aqk = a16(off_w + 2 * (size_t)C * LDK);
  static constexpr size_t off_g = a16(off_Aqk + (WITH_Q ? 2 * (size_t)C * LDT : 0));
  static constexpr size_t total = off_g + sizeof(float) * 4 * C;         // gc, exp(gc), beta, gate
};

// seg_prep
template <typename TQ, int K>
struct PrepLds {
  static constexpr bool FP8 = sizeof(TQ) == 1;
  static constexpr int LDA = C + 4;        // row stride of the fp32 A / solve workspace
  static constexpr int LDT = C + 8;        // row stride of the bf16 Ai staging tile (pcol order)
  static constexpr size_t a16(size_t x) { return (x + 15) / 16 * 16; }
  static constexpr size_t off_in = 0;                                          // k as loaded
  static constexpr size_t off_ck = a16(off_in + (size_t)C * K * sizeof(TQ));   // fp8: bf16 k tile
  static constexpr size_t off_A = a16(off_ck + (FP8 ? (size_t)C * K * 2 : 0));
  static constexpr size_t off_Ai = a16(off_A + 4 * (size_t)C * LDA);
  static constexpr size_t off_g = a16(off_Ai + 2 * (size_t)C * LDT);
  static constexpr size_t total = off_g + sizeof(float) * 2 * C;               // gc, beta
};

// Pointers of the tiles the current chunk computes from.
struct ChunkTiles {
  const bf16* q;
  const bf16* k;
  const bf16* v;
  const bf16* ai;
};

// ---------------------------------------------------------------------------
// chunk input: direct global -> LDS loads
// ---------------------------------------------------------------------------
// 8 input elements per lane: bf16 -> one dwordx4 direct load; fp8 -> two dword loads.
// (the builtin takes the size as a literal)
template <typename T>
__device__ __forceinline__ void direct8(const T* src, unsigned char* wave_blk) {
  if constexpr (sizeof(T) == 2) {
    __builtin_amdgcn_global_load_lds((gmem_void*)src, (lmem_void*)wave_blk, 16, 0, 0);
  } else {
    const unsigned char* p = reinterpret_cast<const unsigned char*>(src);
    __builtin_amdgcn_global_load_lds((gmem_void*)p, (lmem_void*)wave_blk, 4, 0, 0);
    __builtin_amdgcn_global_load_lds((gmem_void*)(p + 4), (lmem_void*)(wave_blk + WAVE * 4), 4, 0, 0);
  }
}

// Issue the loads of one [64][NC] input tile whose row r starts r * row_bytes
// bytes after base.  bf16: unit u = (row, chunk position); the lane loads logical
// chunk pos ^ swz(row) so the LDS image is the swizzled tile.  fp8: plain order,
// 8 bytes per unit as two dwords per lane (converted later).  Rows >= nv read
// row 0 (in bounds).  Addresses are a wave-uniform base (SGPRs) plus a 32-bit
// lane byte offset, the form the saddr encoding takes, so no 64-bit per-lane
// address stays live.
template <typename T, int NC, int NT>
__device__ __forceinline__ void load_tile(const T* base_t, uint32_t row_bytes, int nv, unsigned char* dst) {
  constexpr int CPR = NC / 8;
  constexpr int UNITS = 64 * CPR;
  const int tid = threadIdx.x;
  const int wid = __builtin_amdgcn_readfirstlane(tid / WAVE);
  const unsigned char* base = reinterpret_cast<const unsigned char*>(base_t);
#pragma unroll
  for (int i = 0; i < (UNITS + NT - 1) / NT; ++i) {
    const int u = tid + NT * i;
    if (UNITS % NT != 0 && u - (tid & (WAVE - 1)) >= UNITS) break;      // uniform per wave
    const int r = u / CPR, pos = u % CPR;
    const int c8 = sizeof(T) == 2 ? (pos ^ Tile<NC>::swz(r)) : pos;
    const uint32_t rs = r < nv ? r : 0;
    unsigned char* blk = dst + (NT * i + WAVE * wid) * 8 * sizeof(T);
    direct8<T>(reinterpret_cast<const T*>(base + (rs * row_bytes + (uint32_t)(8 * c8 * sizeof(T)))), blk);
  }
}

// raw per-token scalar (fp32 or bf16 bits) -> float when staged
__device__ __forceinline__ uint32_t ld_raw(const void* p, int64_t i, int dt) {
  return dt == DT_F32 ? reinterpret_cast<const uint32_t*>(p)[i] : (uint32_t)reinterpret_cast<const uint16_t*>(p)[i];
}
__device__ __forceinline__ float raw_to_f32(uint32_t r, int dt) {
  return dt == DT_F32 ? __uint_as_float(r) : __uint_as_float(r << 16);
}

struct GateRaw {
  uint32_t g, b;              // raw bits of g and beta of token tid (fp32, or bf16 in the low half)
};

__device__ __forceinline__ void load_gates(GateRaw& gr, const void* gp, const void* bp, int g_dt, int b_dt, int64_t t0,
                                           int nv, int h, int H) {
  const int tid = threadIdx.x;
  gr.g = 0u;
  gr.b = 0u;
  if (tid < C && tid < nv) {
    gr.g = ld_raw(gp, (t0 + tid) * H + h, g_dt);
    gr.b = ld_raw(bp, (t0 + tid) * H + h, b_dt);
  }
}

// q (if WITH_Q), k, v of tokens t0.. and the chunk's Ai tile (ai: its first row)
template <typename TQ, int K, int V, bool WITH_Q, int NT>
__device__ __forceinline__ void load_chunk(unsigned char* buf, GateRaw& gr, const void* qp, const void* kp,
                                           const void* vp, const void* gp, const void* bp, int g_dt, int b_dt,
                                           int64_t t0, int nv, int h, int H, const bf16* ai) {
  using L = SegLds<TQ, K, V, WITH_Q>;
  load_gates(gr, gp, bp, g_dt, b_dt, t0, nv, h, H);
  const int64_t e0 = t0 * H + h;
  if constexpr (WITH_Q)
    load_tile<TQ, K, NT>(reinterpret_cast<const TQ*>(qp) + e0 * K, (uint32_t)(H * K * sizeof(TQ)), nv, buf + L::buf_q);
  load_tile<TQ, K, NT>(reinterpret_cast<const TQ*>(kp) + e0 * K, (uint32_t)(H * K * sizeof(TQ)), nv, buf + L::buf_k);
  load_tile<bf16, V, NT>(reinterpret_cast<const bf16*>(vp) + e0 * V, (uint32_t)(H * V * 2), nv, buf + L::buf_v);
  load_tile<bf16, C, NT>(ai, (uint32_t)(C * 2), C, buf + L::buf_ai);
}

// fp8 tile (plain order, two dwords per unit) -> dequantised bf16 swizzled tile
template <int NC, int NT>
__device__ __forceinline__ void convert_fp8(const unsigned char* raw, bf16* t, float scale, int nv) {
  constexpr int CPR = NC / 8;
  constexpr int UNITS = 64 * CPR;
  const int tid = threadIdx.x;
  const int l = tid & (WAVE - 1), wid = tid / WAVE;
#pragma unroll
  for (int i = 0; i < (UNITS + NT - 1) / NT; ++i) {
    const int u = tid + NT * i;
    if (UNITS % NT != 0 && u - l >= UNITS) break;
    const int r = u / CPR, c8 = u % CPR;
    const unsigned char* blk = raw + (size_t)(NT * i + WAVE * wid) * 8;
    const uint32_t lo = *reinterpret_cast<const uint32_t*>(blk + 4 * l);
    const uint32_t hi = *reinterpret_cast<const uint32_t*>(blk + WAVE * 4 + 4 * l);
    float x[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[e] = r < nv ? fp8e4m3_to_f32((lo >> (8 * e)) & 0xFF) * scale : 0.f;
      x[4 + e] = r < nv ? fp8e4m3_to_f32((hi >> (8 * e)) & 0xFF) * scale : 0.f;
    }
    *reinterpret_cast<Frag<bf16>*>(t + Tile<NC>::off(r, c8)) = frag_pack(x);
  }
}

// This wave's direct loads have landed.  vmcnt(0) (expcnt and lgkmcnt left at
// their maxima) goes through the builtin so that the compiler's own wait
// tracking knows every load has completed (the compiler does not track direct
// loads as a dependency of LDS reads); the barrier that follows covers the other
// waves' loads.
__device__ __forceinline__ void wait_loads() {
  __builtin_amdgcn_s_waitcnt(0x0F70);
  asm volatile("" ::: "memory");
}

// Chunk-local cumsum gc of g (fla ops/utils/cumsum.py:58-65) over wave 0, from
// the raw g bits of token tid; returns gc of token tid and sets gl = gc of the
// last valid token.
__device__ __forceinline__ float chunk_cumsum(const GateRaw& gr, int g_dt, int nv, float& gl) {
  const int tid = threadIdx.x;
  float gv = raw_to_f32(gr.g, g_dt);
#pragma unroll
  for (int off = 1; off < WAVE; off <<= 1) {
    const float o = __shfl_up(gv, off, WAVE);
    if (tid >= off) gv += o;
  }
  gl = __shfl(gv, nv - 1, WAVE);
  return gv;
}

// Top of a chunk: its loads have landed, fp8 inputs are converted (each lane
// converts the units it loaded itself), and wave 0 forms the chunk vectors: gc,
// exp(gc), beta and the update gate exp(gc_last - gc) (chunk_delta_h.py:163-169).
// Rows nv..63 of a partial chunk hold a copy of row 0 and need no clearing:
// beta and the gate are 0 there, so their rows of A, w and u are zero, they
// add nothing to the state, and their rows of o are not stored.
template <typename TQ, int K, int V, bool WITH_Q, int NT>
__device__ __forceinline__ ChunkTiles stage_chunk(unsigned char* smem, unsigned char* buf, const GateRaw& gr, float qs,
                                                  float ks, int nv, int g_dt, int b_dt) {
  using L = SegLds<TQ, K, V, WITH_Q>;
  wait_loads();
  ChunkTiles T;
  if constexpr (L::FP8) {
    T.q = reinterpret_cast<const bf16*>(smem + L::off_cq);
    T.k = reinterpret_cast<const bf16*>(smem + L::off_ck);
    if constexpr (WITH_Q) convert_fp8<K, NT>(buf + L::buf_q, reinterpret_cast<bf16*>(smem + L::off_cq), qs, nv);
    convert_fp8<K, NT>(buf + L::buf_k, reinterpret_cast<bf16*>(smem + L::off_ck), ks, nv);
  } else {
    T.q = reinterpret_cast<const bf16*>(buf + L::buf_q);
    T.k = reinterpret_cast<const bf16*>(buf + L::buf_k);
  }
  T.v = reinterpret_cast<const bf16*>(buf + L::buf_v);
  T.ai = reinterpret_cast<const bf16*>(buf + L::buf_ai);
  const int tid = threadIdx.x;
  if (tid < WAVE) {
    float* s_g = reinterpret_cast<float*>(smem + L::off_g);
    float gl;
    const float gv = chunk_cumsum(gr, g_dt, nv, gl);
    s_g[tid] = gv;                                         // gc
    s_g[C + tid] = gexp(gv);                               // exp(gc)
    s_g[2 * C + tid] = raw_to_f32(gr.b, b_dt);             // beta
    s_g[3 * C + tid] = tid < nv ? gexp(gl - gv) : 0.f;     // gate
  }
  return T;
}

// Tile (tm, tn), tn <= tm, of the 64 x 64 chunk products (16 x 16 tiles t = 0..9
// in row order: tm = 0, 1, 1, 2, 2, 2, 3, ...):
//   IS_Q false: A = beta_i exp(gc_i - gc_j) k_i.k_j for i > j, fp32 into out[i][j]
//               (chunk_scaled_dot_kkt.py:57-73);
//   IS_Q true:  Aqk = exp(gc_i - gc_j) q_i.k_j for i >= j, bf16 into out[i][pcol(j)]
//               (chunk_o.py:109-118).
__device__ __forceinline__ void tri_tile(int t, int& tm, int& tn) {
  tm = (t >= 1) + (t >= 3) + (t >= 6);
  tn = t - tm * (tm + 1) / 2;
}
template <int K, bool IS_Q, int LDO>
__device__ __forceinline__ void kkt_tile(const bf16* asrc, const bf16* k, const float* s_gc, const float* s_beta,
                                         void* out, int t) {
  using TK = Tile<K>;
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;
  int tm, tn;
  tri_tile(t, tm, tn);
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < K / 32; ++ks)
    mma(acc, TK::row8(asrc, 16 * tm + lc, 4 * ks + lg), TK::row8(k, 16 * tn + lc, 4 * ks + lg));
  const int i0 = 16 * tm + 4 * lg;
  const int j = 16 * tn + lc;
  const f32x4 gi = *reinterpret_cast<const f32x4*>(s_gc + i0);
  f32x4 bi = {1.f, 1.f, 1.f, 1.f};
  if constexpr (!IS_Q) bi = *reinterpret_cast<const f32x4*>(s_beta + i0);
  const float gj = s_gc[j];
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    const int i = i0 + jj;
    const bool keep = IS_Q ? i >= j : i > j;
    const float val = keep ? acc[jj] * gexp(gi[jj] - gj) * bi[jj] : 0.f;
    if constexpr (IS_Q) reinterpret_cast<bf16*>(out)[i * LDO + pcol(j)] = (bf16)val;
    else reinterpret_cast<float*>(out)[i * LDO + j] = val;
  }
}

// ---------------------------------------------------------------------------
// seg_prep: Ai = (I + A)^-1 of one chunk (solve_tril.py:184-331, fp32
// throughout, rounded to bf16 once)
// ---------------------------------------------------------------------------
//   diag_solve:  the four 16x16 diagonal blocks D_i = (I + A_ii)^-1 by forward
//                substitution on one wave (lane = one column of one block), in
//                place in s_A, and rounded into s_Ai;
//   chain_solve: column block j of the inverse, X_ij = -D_i sum_{k=j}^{i-1} A_ik X_kj
//                for i = j+1..3, on one wave per j (j = 0, 1, 2); the X_kj stay in
//                registers as the B operand of the next product, so the three
//                chains need no barrier between their steps.
// s_Ai is [t][pcol(t')].
template <int LDA, int LDT>
__device__ __forceinline__ void diag_solve(float* s_A, bf16* s_Ai) {
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;
  float x[16];
  float* Xb = s_A + (16 * lg) * LDA + 16 * lg;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    float s = 0.f;
#pragma unroll
    for (int r = 0; r < i; ++r) s = fmaf(Xb[i * LDA + r], x[r], s);
    x[i] = (i == lc) ? 1.f : (i < lc ? 0.f : -s);
  }
  // same wave: the reads above are complete before these writes
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    Xb[i * LDA + lc] = x[i];
    s_Ai[(16 * lg + i) * LDT + pcol(16 * lg + lc)] = (bf16)x[i];
  }
}

template <int LDA, int LDT>
__device__ __forceinline__ void chain_solve(const float* s_A, bf16* s_Ai, int j) {
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;
  auto blk = [&](int r, int c) { return s_A + (16 * r) * LDA + 16 * c; };
  f32x4 X[3];                                   // X_{j+1,j}, X_{j+2,j}, X_{j+3,j}
  for (int i = j + 1; i < 4; ++i) {
    f32x4 t = {0.f, 0.f, 0.f, 0.f}, r = {0.f, 0.f, 0.f, 0.f};
    mma16_f32_lds(t, blk(i, j), LDA, blk(j, j), LDA);           // A_ij D_j
#pragma unroll
    for (int k = 1; k < 3; ++k)
      if (j + k < i) mma16_f32_lds_reg(t, blk(i, j + k), LDA, X[k - 1]);   // A_ik X_kj
    mma16_f32_lds_reg(r, blk(i, i), LDA, t);                       // D_i (...)
    r = -r;
#pragma unroll
    for (int k = 0; k < 3; ++k)
      if (k == i - j - 1) X[k] = r;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
      s_Ai[(16 * i + 4 * lg + jj) * LDT + pcol(16 * j + lc)] = (bf16)r[jj];
  }
}

struct SegPrepArgs {
  const void* k;
  const void* g;
  const void* beta;
  const float* k_scale;
  int g_dtype, beta_dtype;
  bf16* Ai;                   // out [chunks, H, 64, 64], row t holds columns pcol(t')
};

constexpr int NT_PREP = 256;

template <typename TQ, int K>
__global__ __launch_bounds__(NT_PREP) void seg_prep_kernel(SegPrepArgs a, SegGeom G) {
  using P = PrepLds<TQ, K>;
  constexpr int NT = NT_PREP, NW = NT / WAVE;
  extern __shared__ __align__(16) unsigned char smem[];
  float* s_A = reinterpret_cast<float*>(smem + P::off_A);
  bf16* s_Ai = reinterpret_cast<bf16*>(smem + P::off_Ai);
  float* s_g = reinterpret_cast<float*>(smem + P::off_g);
  const int h = blockIdx.y;
  const int H = G.H;
  const int64_t ci = blockIdx.x;              // global chunk index
  int64_t bos, eos, c;
  if (G.cu == nullptr) {
    const int64_t nc = (G.T + C - 1) / C;
    if (ci >= (int64_t)G.N * nc) return;
    const int64_t n = ci / nc;
    c = ci - n * nc;
    bos = n * G.T;
    eos = bos + G.T;
  } else {
    if (ci >= G.chunk_off[G.N]) return;
    int lo = 0, hi = G.N - 1;                 // last n with chunk_off[n] <= ci
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (G.chunk_off[mid] <= ci) lo = mid; else hi = mid - 1;
    }
    c = ci - G.chunk_off[lo];
    bos = G.cu[lo];
    eos = G.cu[lo + 1];
  }
  const int64_t t0 = bos + c * C;
  const int nv = (int)min((int64_t)C, eos - t0);
  const int tid = threadIdx.x;
  const int wid = tid / WAVE;

  GateRaw gr;
  load_gates(gr, a.g, a.beta, a.g_dtype, a.beta_dtype, t0, nv, h, H);
  load_tile<TQ, K, NT>(reinterpret_cast<const TQ*>(a.k) + (t0 * H + h) * K, (uint32_t)(H * K * sizeof(TQ)), nv,
                       smem + P::off_in);
  // the upper 16x16 blocks of Ai are zero
  for (int idx = tid; idx < 6 * 256; idx += NT) {
    const int b = idx >> 8, r = (idx >> 4) & 15, cc = idx & 15;
    const int bi = b < 3 ? 0 : (b < 5 ? 1 : 2);
    const int bj = b < 3 ? b + 1 : (b < 5 ? b - 1 : 3);
    s_Ai[(16 * bi + r) * P::LDT + pcol(16 * bj + cc)] = (bf16)0.f;
  }
  wait_loads();
  const bf16* kt;
  if constexpr (P::FP8) {
    convert_fp8<K, NT>(smem + P::off_in, reinterpret_cast<bf16*>(smem + P::off_ck), a.k_scale ? a.k_scale[h] : 1.f,
                       nv);
    kt = reinterpret_cast<const bf16*>(smem + P::off_ck);
  } else {
    kt = reinterpret_cast<const bf16*>(smem + P::off_in);
  }
  if (tid < WAVE) {
    float gl;
    s_g[tid] = chunk_cumsum(gr, a.g_dtype, nv, gl);
    s_g[C + tid] = raw_to_f32(gr.b, a.beta_dtype);
  }
  lds_barrier();
  for (int t = wid; t < 10; t += NW) kkt_tile<K, false, P::LDA>(kt, kt, s_g, s_g + C, s_A, t);
  lds_barrier();
  if (wid == 0) diag_solve<P::LDA, P::LDT>(s_A, s_Ai);
  lds_barrier();
  if (wid >= 1 && wid <= 3) chain_solve<P::LDA, P::LDT>(s_A, s_Ai, wid - 1);
  lds_barrier();
  bf16* dst = a.Ai + (ci * H + h) * C * C;
  for (int u = tid; u < C * C / 8; u += NT) {
    const int r = u >> 3, c8 = u & 7;
    *reinterpret_cast<uint4*>(dst + r * C + 8 * c8) = *reinterpret_cast<const uint4*>(s_Ai + r * P::LDT + 8 * c8);
  }
}

// ---------------------------------------------------------------------------
// w, u and the recurrence
// ---------------------------------------------------------------------------
// kb^T fragments (kb = k beta exp(gc) with the reference's roundings,
// wy_fast.py:67-81) of the d tiles dt = wid + NW * n.
template <int K, int NW>
struct WFrags {
  static constexpr int ND = (K / 16 + NW - 1) / NW;
  Frag<bf16> kb[ND][2];
};
template <typename TQ, int K, int V, bool WITH_Q, int NW>
__device__ __forceinline__ void w_frags(const unsigned char* smem, const ChunkTiles& T, bool beta_lowp,
                                        WFrags<K, NW>& F) {
  using L = SegLds<TQ, K, V, WITH_Q>;
  const float* s_g = reinterpret_cast<const float*>(smem + L::off_g);
  const int wid = threadIdx.x / WAVE;
  const int lg = lane_id() >> 4;
#pragma unroll
  for (int n = 0; n < WFrags<K, NW>::ND; ++n) {
    const int dt = wid + NW * n;
    if (dt >= K / 16) break;
    Frag<bf16> kt[2];
    col_tr2<K>(T.k, 16 * dt, kt);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      float x[8];
      frag_unpack(kt[ks], x);
      const f32x4 b0 = *reinterpret_cast<const f32x4*>(s_g + 2 * C + 32 * ks + 4 * lg);
      const f32x4 b1 = *reinterpret_cast<const f32x4*>(s_g + 2 * C + 32 * ks + 16 + 4 * lg);
      const f32x4 e0 = *reinterpret_cast<const f32x4*>(s_g + C + 32 * ks + 4 * lg);
      const f32x4 e1 = *reinterpret_cast<const f32x4*>(s_g + C + 32 * ks + 16 + 4 * lg);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float v = x[e] * (e < 4 ? b0[e] : b1[e - 4]);
        if (beta_lowp) v = round_to<bf16>(v);
        x[e] = v * (e < 4 ? e0[e] : e1[e - 4]);
      }
      F.kb[n][ks] = frag_pack(x);
    }
  }
}
// w^T = kb^T Ai^T for this wave's d tiles -> s_w[t][pcol(d)]
template <typename TQ, int K, int V, bool WITH_Q, int NW>
__device__ __forceinline__ void w_products(unsigned char* smem, const ChunkTiles& T, const WFrags<K, NW>& F) {
  using L = SegLds<TQ, K, V, WITH_Q>;
  bf16* s_w = reinterpret_cast<bf16*>(smem + L::off_w);
  const int wid = threadIdx.x / WAVE;
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;
#pragma unroll
  for (int n = 0; n < WFrags<K, NW>::ND; ++n) {
    const int dt = wid + NW * n;
    if (dt >= K / 16) break;
#pragma unroll
    for (int tn = 0; tn < 4; ++tn) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks <= tn / 2; ++ks) mma(acc, F.kb[n][ks], Tile<C>::row8(T.ai, 16 * tn + lc, 4 * ks + lg));
      st4<bf16>(s_w + (16 * tn + lc) * L::LDK + pcol(16 * dt + 4 * lg), acc[0], acc[1], acc[2], acc[3]);
    }
  }
}

// (v beta)^T fragments (wy_fast.py:61-65) of V columns v0..v0+15
template <typename TQ, int K, int V, bool WITH_Q>
__device__ __forceinline__ void u_frags(const unsigned char* smem, const ChunkTiles& T, int v0, Frag<bf16> (&vb)[2]) {
  using L = SegLds<TQ, K, V, WITH_Q>;
  const float* s_b = reinterpret_cast<const float*>(smem + L::off_g) + 2 * C;
  const int lg = lane_id() >> 4;
  Frag<bf16> vt[2];
  col_tr2<V>(T.v, v0, vt);
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    float x[8];
    frag_unpack(vt[ks], x);
    const f32x4 b0 = *reinterpret_cast<const f32x4*>(s_b + 32 * ks + 4 * lg);
    const f32x4 b1 = *reinterpret_cast<const f32x4*>(s_b + 32 * ks + 16 + 4 * lg);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] *= (e < 4 ? b0[e] : b1[e - 4]);
    vb[ks] = frag_pack(x);
  }
}
// u (64 rows x 16 columns) = Ai vb, rounded to bf16, in accumulator tiles
__device__ __forceinline__ void u_products(const ChunkTiles& T, const Frag<bf16> (&vb)[2], f32x4 (&u)[4]) {
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;
#pragma unroll
  for (int tm = 0; tm < 4; ++tm) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks <= tm / 2; ++ks) mma(acc, Tile<C>::row8(T.ai, 16 * tm + lc, 4 * ks + lg), vb[ks]);
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = round_to<bf16>(acc[j]);
    u[tm] = acc;
  }
}

// S (K x 16*CT, accumulator tiles) <- gamma S + k^T vg, vg given as operand fragments
template <int K, int CT>
__device__ __forceinline__ void state_update(f32x4 (&S)[K / 16][CT], const Frag<bf16> (&vg)[2][CT],
                                             const ChunkTiles& T, float gamma) {
#pragma unroll
  for (int tp = 0; tp < K / 16; tp += 2) {      // two row tiles per read batch
    uint32_t ad[8];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      Tile<K>::col_tr_addr(T.k, 0, 16 * (tp + e), ad[4 * e], ad[4 * e + 1]);
      Tile<K>::col_tr_addr(T.k, 1, 16 * (tp + e), ad[4 * e + 2], ad[4 * e + 3]);
    }
    Frag<bf16> a[4];
    tr_read4(ad, a);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        S[tp + e][ct] *= gamma;
        mma(S[tp + e][ct], a[2 * e], vg[0][ct]);
        mma(S[tp + e][ct], a[2 * e + 1], vg[1][ct]);
      }
    }
  }
}

// Y (64 x 16*CT) -= w X, X given as operand fragments of its K rows
template <typename TQ, int K, int V, bool WITH_Q, int CT>
__device__ __forceinline__ void sub_wx(f32x4 (&Y)[4][CT], const Frag<bf16> (&xb)[K / 32][CT],
                                       const unsigned char* smem) {
  using L = SegLds<TQ, K, V, WITH_Q>;
  const bf16* s_w = reinterpret_cast<const bf16*>(smem + L::off_w);
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;
#pragma unroll
  for (int tm = 0; tm < 4; ++tm) {
    f32x4 p[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) p[ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < K / 32; ++ks) {
      const Frag<bf16> a = frag_at<bf16>(s_w + (16 * tm + lc) * L::LDK + 32 * ks + 8 * lg);
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) mma(p[ct], a, xb[ks][ct]);
    }
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) Y[tm][ct] -= p[ct];
  }
}

// operand fragments of the gated update input vg = Y * gate (rows t), rounded to bf16
template <int CT>
__device__ __forceinline__ void gate_frags(const f32x4 (&Y)[4][CT], const float* s_gate, Frag<bf16> (&vg)[2][CT]) {
  const int lg = lane_id() >> 4;
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const f32x4 ga = *reinterpret_cast<const f32x4*>(s_gate + 32 * ks + 4 * lg);
    const f32x4 gb = *reinterpret_cast<const f32x4*>(s_gate + 32 * ks + 16 + 4 * lg);
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) vg[ks][ct] = acc_frag(Y[2 * ks][ct] * ga, Y[2 * ks + 1][ct] * gb);
  }
}

// The output tile of a wave (64 tokens x 16 columns, o^T accumulator layout:
// lane holds 4 consecutive columns of token 16*tn + lane%16) as packed bf16,
// held until it is stored.
struct OutPending {
  uint2 v[4];
  int64_t t0;
  int nv;                     // valid tokens; 0 = nothing pending
  __device__ __forceinline__ void set(int tn, const f32x4& r) {
    v[tn].x = pack_bf16x2(r[0], r[1]);
    v[tn].y = pack_bf16x2(r[2], r[3]);
  }
  __device__ __forceinline__ void store(bf16* o, int H, int h, int V, int vw) {
    const int l = lane_id();
    const int lg = l >> 4, lc = l & 15;
    unsigned char* base = reinterpret_cast<unsigned char*>(o + (t0 * H + h) * V + vw);
    const uint32_t row_bytes = (uint32_t)H * V * 2;
#pragma unroll
    for (int tn = 0; tn < 4; ++tn) {
      const uint32_t t = 16 * tn + lc;
      if ((int)t < nv) *reinterpret_cast<uint2*>(base + (t * row_bytes + 8 * lg)) = v[tn];
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
  const bf16* Ai;             // [chunks, H, 64, 64] from seg_prep
  float scale;
  void* o;                    // [B*T, H, V]
  float* ht;                  // [N, H, K, V] or nullptr
};

template <typename TQ, int K, int V>
__global__ __launch_bounds__((OutCfg<K, V>::NT)) void seg_out_kernel(SegOutArgs a, SegGeom G) {
  using L = SegLds<TQ, K, V, true>;
  constexpr int NW = OutCfg<K, V>::NW, NT = OutCfg<K, V>::NT;
  constexpr int KT = K / 16;
  extern __shared__ __align__(16) unsigned char smem[];
  bf16* s_Aqk = reinterpret_cast<bf16*>(smem + L::off_Aqk);
  const float* s_g = reinterpret_cast<const float*>(smem + L::off_g);

  const int h = blockIdx.y;
  const int H = G.H;
  const SegLoc sl = locate_seg(blockIdx.x, G);
  if (!sl.ok) return;
  const int wid = threadIdx.x / WAVE;
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;
  const int vw = wid * 16;              // first V column of this wave
  const float qs = a.q_scale ? a.q_scale[h] : 1.f;
  const float ks_ = a.k_scale ? a.k_scale[h] : 1.f;
  const bool beta_lowp = a.beta_dtype == DT_BF16;

  // ---- initial state of the segment (lane element (tt, j): row 16*tt + 4*lg + j, column vw + lc)
  f32x4 S[KT][1];
  {
    const int lane_off = 4 * lg * V + vw + lc;
    if (sl.j == 0 && a.h0 && a.h0_dtype == DT_F32) {
      const float* p = reinterpret_cast<const float*>(a.h0) + ((int64_t)sl.n * H + h) * K * V + lane_off;
#pragma unroll
      for (int tt = 0; tt < KT; ++tt)
#pragma unroll
        for (int j = 0; j < 4; ++j) S[tt][0][j] = p[(16 * tt + j) * V];
    } else if (sl.j == 0 && a.h0) {
      const bf16* p = reinterpret_cast<const bf16*>(a.h0) + ((int64_t)sl.n * H + h) * K * V + lane_off;
#pragma unroll
      for (int tt = 0; tt < KT; ++tt)
#pragma unroll
        for (int j = 0; j < 4; ++j) S[tt][0][j] = (float)p[(16 * tt + j) * V];
    } else if (sl.j > 0) {
      const float* p = a.s_init + ((int64_t)blockIdx.x * H + h) * K * V + lane_off;
#pragma unroll
      for (int tt = 0; tt < KT; ++tt)
#pragma unroll
        for (int j = 0; j < 4; ++j) S[tt][0][j] = p[(16 * tt + j) * V];
    } else {
#pragma unroll
      for (int tt = 0; tt < KT; ++tt) S[tt][0] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  // upper 16x16 tiles of Aqk that operand fragments read (col tile 2ks+1 of row
  // tile 2ks) are zero; no chunk writes them
  for (int idx = threadIdx.x; idx < 2 * 16 * 16; idx += NT) {
    const int tile = idx >> 8, r = (idx >> 4) & 15, c = idx & 15;
    s_Aqk[(32 * tile + r) * L::LDT + pcol(32 * tile + 16 + c)] = (bf16)0.f;
  }

  GateRaw gr;
  int64_t t0 = sl.bos + sl.c0 * C;
  int nv = (int)min((int64_t)C, sl.eos - t0);
  const bf16* ai = a.Ai + ((sl.cbase + sl.c0) * H + h) * C * C;
  const int64_t ai_step = (int64_t)H * C * C;
  load_chunk<TQ, K, V, true, NT>(smem + L::off_buf, gr, a.q, a.k, a.v, a.g, a.beta, a.g_dtype, a.beta_dtype, t0, nv, h,
                                 H, ai);
  bf16* o = reinterpret_cast<bf16*>(a.o);
  OutPending op;
  op.nv = 0;

  for (int ci = 0; ci < sl.nch; ++ci) {
    unsigned char* buf = smem + L::off_buf + (ci & 1) * L::buf_bytes;
    const ChunkTiles T = stage_chunk<TQ, K, V, true, NT>(smem, buf, gr, qs, ks_, nv, a.g_dtype, a.beta_dtype);
    op.store(o, H, h, V, vw);            // the previous chunk's output, after this chunk's wait
    const int64_t t0c = t0;
    const int nvc = nv;
    if (ci + 1 < sl.nch) {                // the next chunk streams into the other buffer
      t0 += C;
      nv = (int)min((int64_t)C, sl.eos - t0);
      ai += ai_step;
      load_chunk<TQ, K, V, true, NT>(smem + L::off_buf + ((ci + 1) & 1) * L::buf_bytes, gr, a.q, a.k, a.v, a.g,
                                     a.beta, a.g_dtype, a.beta_dtype, t0, nv, h, H, ai);
    }
    lds_barrier();   // chunk tiles and vectors ready

    // ---- Aqk tiles, w = Ai kb -> LDS, u = Ai vb (this wave's columns) -> registers
    for (int t = wid; t < 10; t += NW) kkt_tile<K, true, L::LDT>(T.q, T.k, s_g, nullptr, s_Aqk, t);
    {
      WFrags<K, NW> wf;
      w_frags<TQ, K, V, true, NW>(smem, T, beta_lowp, wf);
      w_products<TQ, K, V, true, NW>(smem, T, wf);
    }
    f32x4 Y[4][1];
    {
      Frag<bf16> vb[2];
      u_frags<TQ, K, V, true>(smem, T, vw, vb);
      f32x4 u[4];
      u_products(T, vb, u);
#pragma unroll
      for (int tm = 0; tm < 4; ++tm) Y[tm][0] = u[tm];
    }
    lds_barrier();   // w and Aqk complete

    // ---- h = S rounded (the snapshot of chunk_delta_h.py:129-139) as operand fragments
    Frag<bf16> hb[K / 32][1];
#pragma unroll
    for (int ks = 0; ks < K / 32; ++ks) hb[ks][0] = acc_frag(S[2 * ks][0], S[2 * ks + 1][0]);
    // ---- v' = u - w h                                   (chunk_delta_h.py:141-157)
    sub_wx<TQ, K, V, true, 1>(Y, hb, smem);

    // ---- o^T = scale (h^T q^T exp(gc) + v_new^T Aqk^T)  (chunk_o.py:84-128)
    op.t0 = t0c;
    op.nv = nvc;
    Frag<bf16> vn[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) vn[ks] = acc_frag(Y[2 * ks][0], Y[2 * ks + 1][0]);
#pragma unroll
    for (int tn = 0; tn < 4; ++tn) {
      const int t = 16 * tn + lc;
      f32x4 o1 = {0.f, 0.f, 0.f, 0.f}, o2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < K / 32; ++ks) mma(o1, hb[ks][0], Tile<K>::row_acc_order(T.q, t, ks, lg));
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        if (ks <= tn / 2) mma(o2, vn[ks], frag_at<bf16>(s_Aqk + t * L::LDT + 32 * ks + 8 * lg));
      const float eg = s_g[C + t] * a.scale;
      op.set(tn, o1 * eg + o2 * a.scale);
    }

    // ---- S = exp(g_last) S + k^T (v' exp(g_last - gc))   (chunk_delta_h.py:163-211)
    Frag<bf16> vg[2][1];
    gate_frags<1>(Y, s_g + 3 * C, vg);
    state_update<K, 1>(S, vg, T, gexp(s_g[nvc - 1]));
    lds_barrier();   // the tiles of this chunk are free for the chunk after next
  }
  op.store(o, H, h, V, vw);

  if (a.ht && sl.j == sl.nseg - 1) {
    float* p = a.ht + ((int64_t)sl.n * H + h) * K * V + 4 * lg * V + vw + lc;
#pragma unroll
    for (int tt = 0; tt < KT; ++tt)
#pragma unroll
      for (int j = 0; j < 4; ++j) p[(16 * tt + j) * V] = S[tt][0][j];
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
  const bf16* Ai;             // [chunks, H, 64, 64] from seg_prep
  float* M;                   // [NS, H, K, K]
  float* R;                   // [NS, H, K, V]
};

template <typename TQ, int K, int V>
__global__ __launch_bounds__((TransCfg<K, V>::NT)) void seg_trans_kernel(SegTransArgs a, SegGeom G) {
  using L = SegLds<TQ, K, V, false>;
  constexpr int NW = TransCfg<K, V>::NW, NT = TransCfg<K, V>::NT;
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
  const bool beta_lowp = a.beta_dtype == DT_BF16;

  f32x4 X[KT][CT];
#pragma unroll
  for (int tt = 0; tt < KT; ++tt) {
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
#pragma unroll
      for (int j = 0; j < 4; ++j) X[tt][ct][j] = (16 * tt + 4 * lg + j == xw + 16 * ct + lc) ? 1.f : 0.f;
    }
  }

  GateRaw gr;
  int64_t t0 = sl.bos + sl.c0 * C;
  int nv = (int)min((int64_t)C, sl.eos - t0);
  const bf16* ai = a.Ai + ((sl.cbase + sl.c0) * H + h) * C * C;
  const int64_t ai_step = (int64_t)H * C * C;
  load_chunk<TQ, K, V, false, NT>(smem + L::off_buf, gr, nullptr, a.k, a.v, a.g, a.beta, a.g_dtype, a.beta_dtype, t0,
                                  nv, h, H, ai);
  for (int ci = 0; ci < sl.nch; ++ci) {
    unsigned char* buf = smem + L::off_buf + (ci & 1) * L::buf_bytes;
    const ChunkTiles T = stage_chunk<TQ, K, V, false, NT>(smem, buf, gr, 1.f, ks_, nv, a.g_dtype, a.beta_dtype);
    const int nvc = nv;
    if (ci + 1 < sl.nch) {
      t0 += C;
      nv = (int)min((int64_t)C, sl.eos - t0);
      ai += ai_step;
      load_chunk<TQ, K, V, false, NT>(smem + L::off_buf + ((ci + 1) & 1) * L::buf_bytes, gr, nullptr, a.k, a.v, a.g,
                                      a.beta, a.g_dtype, a.beta_dtype, t0, nv, h, H, ai);
    }
    lds_barrier();   // chunk tiles and vectors ready
    {
      WFrags<K, NW> wf;
      w_frags<TQ, K, V, false, NW>(smem, T, beta_lowp, wf);
      w_products<TQ, K, V, false, NW>(smem, T, wf);
    }
    f32x4 Y[4][CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      const int c0 = xw + 16 * ct;
      if (c0 >= K) {
        Frag<bf16> vb[2];
        u_frags<TQ, K, V, false>(smem, T, c0 - K, vb);
        f32x4 u[4];
        u_products(T, vb, u);
#pragma unroll
        for (int tm = 0; tm < 4; ++tm) Y[tm][ct] = u[tm];
      } else {
#pragma unroll
        for (int tm = 0; tm < 4; ++tm) Y[tm][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
    lds_barrier();   // w complete
    Frag<bf16> xb[K / 32][CT];
#pragma unroll
    for (int ks = 0; ks < K / 32; ++ks) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) xb[ks][ct] = acc_frag(X[2 * ks][ct], X[2 * ks + 1][ct]);
    }
    sub_wx<TQ, K, V, false, CT>(Y, xb, smem);
    Frag<bf16> yg[2][CT];
    gate_frags<CT>(Y, s_g + 3 * C, yg);
    state_update<K, CT>(X, yg, T, gexp(s_g[nvc - 1]));
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
//
// The chain is serial, so each step must cost only its arithmetic: wave w owns
// output rows 16w .. 16w + 15 and holds its rows of M_j (A operand) and its
// tile of R_j in registers, loaded one step ahead, while the state columns
// (B operand, shared by all waves) sit transposed in LDS so that the four K
// values a lane needs per 16-deep step are one 16-byte read.
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
struct CombineMaps {
  f32x4 m[K / 16];            // M_j[r0 + lane%16][16 kk + 4 (lane/16) .. +3]
  f32x4 r;                    // R_j[r0 + 4 (lane/16) + jj][v0 + lane%16]
};

template <int K>
__device__ __forceinline__ void load_maps(CombineMaps<K>& c, const float* M, const float* R, int V, int r0, int v0) {
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;
  const float* pm = M + (int64_t)(r0 + lc) * K + 4 * lg;
#pragma unroll
  for (int kk = 0; kk < K / 16; ++kk) c.m[kk] = *reinterpret_cast<const f32x4*>(pm + 16 * kk);
  const float* pr = R + (int64_t)(r0 + 4 * lg) * V + v0 + lc;
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) c.r[jj] = pr[(int64_t)jj * V];
}

template <int K> struct CombCfg { static constexpr int NT = K / 16 * WAVE; };   // one 16-row tile per wave

template <int K>
__global__ __launch_bounds__(CombCfg<K>::NT) void seg_combine_kernel(SegCombineArgs a, SegGeom G, int total) {
  constexpr int NT = CombCfg<K>::NT;
  constexpr int LDS_T = K + 4;                              // row stride of the transposed state
  __shared__ __align__(16) float s_St[16][LDS_T];           // s_St[c][r] = S[r][v0 + c]
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
  const int r0 = 16 * wid;

  int nseg, s_first;
  if (G.cu == nullptr) {
    nseg = G.T > 0 ? G.nseg_fixed : 0;
    s_first = n * G.nseg_fixed;
  } else {
    nseg = G.seg_off[n + 1] - G.seg_off[n];
    s_first = G.seg_off[n];
  }
  // Maps of steps j, j + 1, j + 2 in flight (stage j % 3).  Every stage is
  // loaded unconditionally (past the last step: the last step's maps again) so
  // that the number of loads issued after each stage is fixed and the wait for
  // a stage counts only the loads before it.
  constexpr int NST = 3;
  const int nsteps = nseg - 1;
  CombineMaps<K> st[NST];
  auto issue = [&](CombineMaps<K>& c, int j) {
    const int64_t s = s_first + max(0, min(j, nsteps - 1));
    load_maps<K>(c, a.M + (s * H + h) * K * K, a.R + (s * H + h) * K * V, V, r0, v0);
  };
  if (nsteps > 0) {
#pragma unroll
    for (int u = 0; u < NST; ++u) issue(st[u], u);
  }
  for (int idx = threadIdx.x; idx < K * 16; idx += NT) {
    const int r = idx / 16, c = idx % 16;
    float x = 0.f;
    if (a.h0) {
      const int64_t off = (((int64_t)n * H + h) * K + r) * V + v0 + c;
      x = a.h0_dtype == DT_F32 ? reinterpret_cast<const float*>(a.h0)[off]
                               : (float)reinterpret_cast<const bf16*>(a.h0)[off];
    }
    s_St[c][r] = x;
  }
  if (nseg == 0) {
    if (a.ht) {
      __syncthreads();
      for (int idx = threadIdx.x; idx < K * 16; idx += NT) {
        const int r = idx / 16, c = idx % 16;
        a.ht[(((int64_t)n * H + h) * K + r) * V + v0 + c] = s_St[c][r];
      }
    }
    return;
  }
  __syncthreads();
  for (int j0 = 0; j0 < nsteps; j0 += NST) {
#pragma unroll
    for (int u = 0; u < NST; ++u) {
      const int j = j0 + u;
      if (j >= nsteps) break;                               // uniform
      f32x4 acc = st[u].r;
#pragma unroll
      for (int kk = 0; kk < K / 16; ++kk) {
        const f32x4 b = *reinterpret_cast<const f32x4*>(&s_St[lc][16 * kk + 4 * lg]);
#pragma unroll
        for (int qq = 0; qq < 4; ++qq)
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(st[u].m[kk][qq], b[qq], acc, 0, 0, 0);
      }
      issue(st[u], j + NST);                                // this stage's registers are free again
      __syncthreads();
      *reinterpret_cast<f32x4*>(&s_St[lc][r0 + 4 * lg]) = acc;
      float* out = a.s_init + ((s_first + j + 1) * (int64_t)H + h) * K * V + (int64_t)(r0 + 4 * lg) * V + v0 + lc;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) out[(int64_t)jj * V] = acc[jj];
      __syncthreads();
    }
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

template <typename TQ, int K, int V>
int launch_seg_t(const SegFwdArgs& p, hipStream_t s) {
  SegGeom G{p.cu, p.chunk_off, p.seg_off, p.N, p.T, p.H, p.L, p.nseg_fixed};
  const dim3 grid((unsigned)p.ns_grid, (unsigned)p.H);
  bf16* Ai = static_cast<bf16*>(p.Ai);
  auto mark = [&](int i) { return p.events == nullptr || hipEventRecord(p.events[i], s) == hipSuccess; };
  if (!mark(0)) return -1;
  if (p.ns_grid > 0 && p.nc_grid > 0) {
    constexpr size_t lds = PrepLds<TQ, K>::total;
    static_assert(lds <= 64 * 1024, "seg_prep tiles exceed the default LDS limit");
    SegPrepArgs pa{p.k, p.g, p.beta, p.k_scale, p.g_dtype, p.beta_dtype, Ai};
    hipLaunchKernelGGL((seg_prep_kernel<TQ, K>), dim3((unsigned)p.nc_grid, (unsigned)p.H), dim3(NT_PREP), lds, s, pa,
                       G);
    if (hipGetLastError() != hipSuccess) return -1;
  }
  if (!mark(1)) return -1;
  if (p.run_trans) {
    constexpr size_t lds = SegLds<TQ, K, V, false>::total;
    static_assert(lds <= 160 * 1024, "seg_trans tiles do not fit in LDS");
    auto kt = seg_trans_kernel<TQ, K, V>;
    if (set_lds(kt, lds)) return -1;
    SegTransArgs ta{p.k, p.v, p.g, p.beta, p.k_scale, p.g_dtype, p.beta_dtype, Ai, p.M, p.R};
    hipLaunchKernelGGL(kt, grid, dim3(TransCfg<K, V>::NT), lds, s, ta, G);
    if (hipGetLastError() != hipSuccess) return -1;
  }
  if (!mark(2)) return -1;
  if (p.run_combine) {
    const int total = p.N * p.H * (V / 16);
    const int cgrid = (total + 7) / 8 * 8;
    SegCombineArgs ca{p.M, p.R, p.h0, p.h0_dtype, p.s_init, p.ht, V};
    hipLaunchKernelGGL(seg_combine_kernel<K>, dim3(cgrid), dim3(CombCfg<K>::NT), 0, s, ca, G, total);
    if (hipGetLastError() != hipSuccess) return -1;
  }
  if (!mark(3)) return -1;
  if (p.ns_grid > 0) {
    constexpr size_t lds = SegLds<TQ, K, V, true>::total;
    static_assert(lds <= 160 * 1024, "seg_out tiles do not fit in LDS");
    auto ko = seg_out_kernel<TQ, K, V>;
    if (set_lds(ko, lds)) return -1;
    SegOutArgs oa{p.q, p.k, p.v, p.g, p.beta, p.q_scale, p.k_scale, p.g_dtype, p.beta_dtype,
                  p.h0, p.h0_dtype, p.s_init, Ai, p.scale, p.o, p.ht};
    hipLaunchKernelGGL(ko, grid, dim3(OutCfg<K, V>::NT), lds, s, oa, G);
    if (hipGetLastError() != hipSuccess) return -1;
  }
  if (!mark(4)) return -1;
  return 0;
}

}  // namespace

bool seg_fwd_supported(int compute_dtype, int K, int V) {
  // bf16 compute only: the transposed operand reads (ds_read_b64_tr_b16) are 16-bit;
  // fp32 problems run the stage kernels
  return compute_dtype == DT_BF16 && (K == 64 || K == 128) && (V == 64 || V == 128);
}

int launch_seg_map(const int64_t* cu, int N, int L, int32_t* chunk_off, int32_t* seg_off, hipStream_t s) {
  hipLaunchKernelGGL(seg_map_kernel, dim3(1), dim3(64), 0, s, cu, N, L, chunk_off, seg_off);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_seg_fwd(const SegFwdArgs& p, int compute_dtype, int qk_dtype, int K, int V, hipStream_t s) {
  if (compute_dtype != DT_BF16) return -2;
#define KGDN_SEG_CASE(TQ, KK, VV) \
  if (K == KK && V == VV) return launch_seg_t<TQ, KK, VV>(p, s);
#define KGDN_SEG_SHAPES(TQ) \
  KGDN_SEG_CASE(TQ, 64, 64) KGDN_SEG_CASE(TQ, 64, 128) KGDN_SEG_CASE(TQ, 128, 64) KGDN_SEG_CASE(TQ, 128, 128)
  if (qk_dtype == DT_BF16) { KGDN_SEG_SHAPES(bf16) }
  if (qk_dtype == DT_F8E4M3) { KGDN_SEG_SHAPES(uint8_t) }
#undef KGDN_SEG_SHAPES
#undef KGDN_SEG_CASE
  return -2;
}

}  // namespace kgdn
