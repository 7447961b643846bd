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
//   * k^T and v^T, whose contraction index is the token: ds_read_b64_tr_b16
//     transposes a 4-token x 16-column block across the 16 lanes of a lane
//     group (lane j receives column j of the 4 rows).
// fp8 q/k are converted once per chunk into bf16 tiles of the same layout.
// The chunk step itself is described at the chunk engine below.
#include <type_traits>

#include "gdn_common.hpp"
#include "gdn_kernels.h"
#include "gdn_tiles.hpp"

namespace kgdn {

namespace {

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
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
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
// the same conversion, kept as one packed value: the empty asm hides the
// packing from the optimizer, which otherwise splits it into one conversion per
// value when only the rounded values are used, as floats (the conversion
// itself stays a compiler-generated instruction, under its hazard tracking)
__device__ __forceinline__ uint32_t cvt_pk_bf16(float a, float b) {
  uint32_t r = pack_bf16x2(a, b);
  asm("" : "+v"(r));
  return r;
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
// sits at chunk position c ^ swz(r).  LDS serves 256 bytes per clock (64 banks
// of 4 bytes); a read is conflict-free when the lanes served together touch
// distinct banks.  Rows of 256 bytes (NC = 128) take swz(r) = 2 (r mod 8) +
// (r / 8 mod 2): 16 consecutive rows get 16 distinct chunk positions (16-byte
// row reads), and the 8 rows x 2 chunks of a transposed read
// (ds_read_b64_tr_b16, 32 lanes of 8 bytes) get 16 distinct positions too,
// where swz(r) = r mod 16 leaves them two-way conflicted.  Rows of 128 bytes
// (NC = 64, two rows per 256-byte bank row) take a permutation of r/2 with the
// same two properties.
// ---------------------------------------------------------------------------
template <int NC>
struct Tile {
  static_assert(NC == 64 || NC == 128, "tiles are 64 or 128 columns wide");
  static constexpr int CPR = NC / 8;                  // 16-byte chunks per row
  __device__ static __forceinline__ int swz(int r) {
    if constexpr (NC == 64) return (((r >> 1) & 3) << 1) | ((r >> 3) & 1);
    else return ((r & 7) << 1) | ((r >> 3) & 1);
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

// Transposed fragments: the two 8-byte halves read by ds_read_b64_tr_b16.
__device__ __forceinline__ Frag<bf16> tr_pair(u32x2 a, u32x2 b) {
  Frag<bf16> f;
  f.v = __builtin_bit_cast(bf16x8, make_uint4(a.x, a.y, b.x, b.y));
  return f;
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

// seg_prep
// seg_prep LDS of one wave (one (chunk, head) item per wave): the ten lower
// 16x16 blocks of A in fp32 (block (r, c), c <= r, at index r(r+1)/2 + c, row
// stride LDB), then gc and beta of the chunk.  After the solve the block area
// stages the bf16 Ai (64 rows of 64, pcol order) for the record store.
struct PrepLds {
  static constexpr int LDB = 20;
  static constexpr int BLK = 16 * LDB;                   // floats per block
  static constexpr size_t off_A = 0;
  static constexpr size_t off_g = 10 * BLK * sizeof(float);
  static constexpr size_t per_wave = off_g + 2 * C * sizeof(float);
  static constexpr int WAVES = 4;                        // waves (items) per workgroup
  static constexpr size_t total = WAVES * per_wave;
  static_assert(C * C * 2 <= off_g, "Ai staging must fit in the block area");
};
__device__ __forceinline__ int tri_blk(int r, int c) { return r * (r + 1) / 2 + c; }


// ---------------------------------------------------------------------------
// chunk input: direct global -> LDS loads
// ---------------------------------------------------------------------------
// Direct global->LDS loads, issued through inline asm: lane l's 16 (4) bytes
// at base + off land at LDS address lds_dst + 16 l (4 l); base is wave-uniform
// (SGPRs), off a 32-bit lane offset.  The compiler's wait tracking treats every
// LDS read that follows a direct load (the builtin) as a possible reader of it
// and waits for vmcnt first -- for the next chunk's prefetch, in the middle of
// the current chunk.  Hidden in asm, the loads are waited for explicitly
// (wait_loads) before the barrier that publishes their data.  M0 carries the
// LDS address.  The hazard rules are the asm's own: a VALU write of an SGPR
// (v_readfirstlane of the base) needs 5 wait states before a VMEM instruction
// reads that SGPR, and an SALU write of M0 one before the load reads it, hence
// s_nop 4 ahead of each load.
__device__ __forceinline__ const void* uniform_ptr(const void* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<const void*>(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ void dma16(const void* base, uint32_t off, uint32_t lds_dst) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(off), "s"(uniform_ptr(base)), "{m0}"(lds_dst)
               : "memory");
}
__device__ __forceinline__ void dma4(const void* base, uint32_t off, uint32_t lds_dst) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dword %0, %1" : : "v"(off), "s"(uniform_ptr(base)), "{m0}"(lds_dst)
               : "memory");
}

// 8 input elements per lane: bf16 -> one dwordx4 direct load; fp8 -> two dword loads.
// (wave_blk: the LDS byte address of the wave's destination block, wave-uniform)
template <typename T>
__device__ __forceinline__ void direct8(const void* base, uint32_t off, uint32_t wave_blk) {
  const uint32_t d = __builtin_amdgcn_readfirstlane(wave_blk);
  if constexpr (sizeof(T) == 2) {
    dma16(base, off, d);
  } else {
    dma4(base, off, d);
    dma4(base, off + 4, d + WAVE * 4);
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
__device__ __forceinline__ void load_tile(const T* base_t, uint32_t row_bytes, int nv, uint32_t dst) {
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
    direct8<T>(base, rs * row_bytes + (uint32_t)(8 * c8 * sizeof(T)), dst + (NT * i + WAVE * wid) * 8 * sizeof(T));
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
    fp8x4_to_f32(lo, x);
    fp8x4_to_f32(hi, x + 4);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = r < nv ? x[e] * scale : 0.f;
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

// v + (v of the lane selected by DPP control CTRL), 0 where the source lane is
// outside the pattern or its row is masked off (ROWS).
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_plus(float v) {
  const int s = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWS, 0xf, false);
  return v + __int_as_float(s);
}
// 1 / sqrt(sum x^2 + 1e-6) of the in-op L2 norm (l2norm.py:115, eps 1e-6), by the hardware
// reciprocal square root (within 1 ulp); seg_prep and seg_out use this one form, so both
// normalise k to the same values.
__device__ __forceinline__ float l2_rstd(float ss) { return __builtin_amdgcn_rsqf(ss + 1e-6f); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
// acc + a.lo * b.lo + a.hi * b.hi for two packed bf16 pairs (v_dot2_f32_bf16, fp32 accumulate)
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), acc,
                                         false);
}

// Sum over each group of G consecutive lanes (G = 8 or 16, groups aligned), every lane of a group
// receiving it, with DPP moves (no LDS): quad swaps, then the half-row and row mirrors.
template <int G>
__device__ __forceinline__ float row_sum_dpp(float v) {
  static_assert(G == 8 || G == 16, "row_sum_dpp sums groups of 8 or 16 lanes");
  v = dpp_plus<0xB1, 0xf>(v);       // quad_perm [1, 0, 3, 2]
  v = dpp_plus<0x4E, 0xf>(v);       // quad_perm [2, 3, 0, 1]
  v = dpp_plus<0x141, 0xf>(v);      // row_half_mirror: the other quad of the 8
  if constexpr (G == 16) v = dpp_plus<0x140, 0xf>(v);   // row_mirror: the other 8 of the row
  return v;
}

// Inclusive prefix sum over the 64 lanes of a wave with DPP moves (no LDS):
// shifts by 1, 2, 4, 8 within each row of 16 lanes, then row_bcast:15 and
// row_bcast:31 carry the row totals into the rows above.
__device__ __forceinline__ float wave_prefix_sum(float v) {
  v = dpp_plus<0x111, 0xf>(v);      // row_shr:1
  v = dpp_plus<0x112, 0xf>(v);      // row_shr:2
  v = dpp_plus<0x114, 0xf>(v);      // row_shr:4
  v = dpp_plus<0x118, 0xf>(v);      // row_shr:8
  v = dpp_plus<0x142, 0xa>(v);      // row_bcast:15 into rows 1 and 3
  v = dpp_plus<0x143, 0xc>(v);      // row_bcast:31 into rows 2 and 3
  return v;
}

// Chunk-local cumsum gc of g (fla ops/utils/cumsum.py:58-65), lane = token:
// returns gc of token lane and sets gl = gc of the last valid token (nv - 1).
__device__ __forceinline__ float chunk_cumsum(const GateRaw& gr, int g_dt, int nv, float& gl) {
  const float gv = wave_prefix_sum(raw_to_f32(gr.g, g_dt));
  gl = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gv), nv - 1));
  return gv;
}

// Tile (tm, tn), tn <= tm, of the 64 x 64 chunk products (16 x 16 tiles t = 0..9
// in row order: tm = 0, 1, 1, 2, 2, 2, 3, ...).
__device__ __forceinline__ void tri_tile(int t, int& tm, int& tn) {
  tm = (t >= 1) + (t >= 3) + (t >= 6);
  tn = t - tm * (tm + 1) / 2;
}
// ---------------------------------------------------------------------------
// seg_prep: one chunk record per (chunk, head), one wave per item, no barriers
// ---------------------------------------------------------------------------
//   k rows as MFMA operand fragments in registers: lane (lc, lg) of row tile rt
//   holds k[16 rt + lc][32 ks + 8 lg .. + 7] (rows >= nv read row 0);
//   A = beta_i exp(gc_i - gc_j) k_i.k_j, i > j (chunk_scaled_dot_kkt.py:57-73),
//   as ten fp32 16x16 blocks in LDS;
//   Ai = (I + A)^-1 (solve_tril.py:184-331, fp32 throughout, rounded to bf16
//   once): the four diagonal blocks by forward substitution (lane = one column
//   of one block), then X_ij = -D_i sum_{k=j}^{i-1} A_ik X_kj by fp32 MFMA with
//   the X in registers; Ai staged in LDS and written to the record.
struct SegPrepArgs {
  const void* k;
  const void* g;
  const void* beta;
  const float* k_scale;
  int g_dtype, beta_dtype;
  float scale;                // output scale (the record's exp(gc) * scale vector)
  unsigned char* rec;         // out [chunks, H] records of kSegRecordBytes (see gdn_kernels.h)
  int l2;                     // in-op L2 norm of k (bf16 k): normalise the rows and record rstd
};

// One (chunk, head) item of seg_prep: item = chunk * H + head.
struct PrepItem {
  int64_t ci;                 // global chunk index
  int64_t t0;                 // first token
  int nv;                     // valid tokens
  int h;
};

template <bool VARLEN>
__device__ __forceinline__ PrepItem prep_item(int64_t item, const SegGeom& G) {
  PrepItem it;
  it.ci = item / G.H;
  it.h = (int)(item - it.ci * G.H);
  int64_t bos, eos, c;
  if constexpr (!VARLEN) {
    const int64_t nc = (G.T + C - 1) / C;
    const int64_t n = it.ci / nc;
    c = it.ci - n * nc;
    bos = n * G.T;
    eos = bos + G.T;
  } else {
    int lo = 0, hi = G.N - 1;                 // last n with chunk_off[n] <= ci
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (G.chunk_off[mid] <= it.ci) lo = mid; else hi = mid - 1;
    }
    c = it.ci - G.chunk_off[lo];
    bos = G.cu[lo];
    eos = G.cu[lo + 1];
  }
  it.t0 = bos + c * C;
  it.nv = (int)min((int64_t)C, eos - it.t0);
  return it;
}

// k fragment of row r (already clamped), columns 32 ks + 8 lg .. + 7, as bf16.
template <typename TQ, int K>
__device__ __forceinline__ Frag<bf16> k_frag(const TQ* row, int ks, float kscale) {
  const int lg = lane_id() >> 4;
  Frag<bf16> f;
  if constexpr (sizeof(TQ) == 1) {
    float x[8];
    load8_in<TQ>(row + 32 * ks + 8 * lg, kscale, x);
    f = frag_pack(x);
  } else {
    f.v = *reinterpret_cast<const bf16x8*>(row + 32 * ks + 8 * lg);
  }
  return f;
}

// Forward substitution of the four diagonal blocks (lane group lg = block,
// lane column lc): D = (I + A_bb)^-1 replaces A_bb in LDS; x returns column lc
// of D (rows 0..15) for the bf16 output.
__device__ __forceinline__ void diag_blocks(float* s_A, float (&x)[16]) {
  constexpr int LDB = PrepLds::LDB;
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;
  float* Xb = s_A + tri_blk(lg, lg) * PrepLds::BLK;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    float sum = 0.f;
#pragma unroll
    for (int r = 0; r < i; ++r) sum = fmaf(Xb[i * LDB + r], x[r], sum);
    x[i] = (i == lc) ? 1.f : (i < lc ? 0.f : -sum);
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) Xb[i * LDB + lc] = x[i];
}

template <typename TQ, int K, bool VARLEN>
__global__ __launch_bounds__(PrepLds::WAVES * WAVE) void seg_prep_kernel(SegPrepArgs a, SegGeom G) {
  using P = PrepLds;
  constexpr int LDB = P::LDB;
  extern __shared__ __align__(16) unsigned char smem[];
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;
  const int H = G.H;
  const int64_t n_items = (VARLEN ? (int64_t)G.chunk_off[G.N] : (int64_t)G.N * ((G.T + C - 1) / C)) * H;
  const int64_t item = (int64_t)blockIdx.x * P::WAVES + wid;
  if (item >= n_items) return;
  const PrepItem it = prep_item<VARLEN>(item, G);
  float* s_A = reinterpret_cast<float*>(smem + wid * P::per_wave + P::off_A);
  float* s_g = reinterpret_cast<float*>(smem + wid * P::per_wave + P::off_g);

  // gates (lane = token) and the k fragments
  uint32_t graw = 0u, braw = 0u;
  if (l < it.nv) {
    graw = ld_raw(a.g, (it.t0 + l) * H + it.h, a.g_dtype);
    braw = ld_raw(a.beta, (it.t0 + l) * H + it.h, a.beta_dtype);
  }
  const float kscale = (sizeof(TQ) == 1 && a.k_scale) ? a.k_scale[it.h] : 1.f;
  const TQ* kb = reinterpret_cast<const TQ*>(a.k) + (it.t0 * H + it.h) * K;
  Frag<bf16> kf[4][K / 32];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt) {
    const int r = 16 * rt + lc;
    const TQ* row = kb + (int64_t)(r < it.nv ? r : 0) * H * K;
#pragma unroll
    for (int ks = 0; ks < K / 32; ++ks) kf[rt][ks] = k_frag<TQ, K>(row, ks, kscale);
  }
  // in-op L2 norm of k (chunk.py:168-170, l2norm.py:98-119): y = bf16(k / sqrt(sum k^2 + 1e-6)) per
  // row; a row is spread over the four lane groups, so two shuffles complete its sum.  K.K^T uses
  // the normalised rows; the record carries rstd for the two serial kernels, which read raw k.
  float rs_own = 1.f;                                    // rstd of token lane (row 16 lg + lc)
  if constexpr (sizeof(TQ) == 2) {
    if (a.l2) {
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        float ss = 0.f;
#pragma unroll
        for (int ks = 0; ks < K / 32; ++ks)
#pragma unroll
          for (int e = 0; e < 8; ++e) ss = fmaf((float)kf[rt][ks].v[e], (float)kf[rt][ks].v[e], ss);
        ss += __shfl_xor(ss, 16, WAVE);
        ss += __shfl_xor(ss, 32, WAVE);
        const float rs = l2_rstd(ss);
        if (rt == lg) rs_own = rs;
#pragma unroll
        for (int ks = 0; ks < K / 32; ++ks)
#pragma unroll
          for (int e = 0; e < 8; ++e) kf[rt][ks].v[e] = (bf16)((float)kf[rt][ks].v[e] * rs);
      }
    }
  }

  // chunk vectors of the record (lane = token)
  unsigned char* rec = a.rec + (it.ci * H + it.h) * (int64_t)kSegRecordBytes;
  {
    GateRaw gr;
    gr.g = graw;
    gr.b = braw;
    float gl;
    const float gc = chunk_cumsum(gr, a.g_dtype, it.nv, gl);
    const float b = raw_to_f32(braw, a.beta_dtype);
    const float eg = gexp(gc);
    s_g[l] = gc;
    s_g[C + l] = b;
    float* vec = reinterpret_cast<float*>(rec + C * C * 2);
    vec[l] = gc;
    vec[C + l] = eg * a.scale;
    vec[2 * C + l] = eg;
    vec[3 * C + l] = l < it.nv ? gexp(gl - gc) : 0.f;
    vec[4 * C + l] = b;
    vec[5 * C + l] = gexp(gl);
    // with the in-op L2 norm: rstd of k, and the update gate times it (seg_trans folds the
    // normalisation of k into its w operand and its gated v')
    vec[6 * C + l] = a.l2 ? rs_own : 0.f;
    vec[7 * C + l] = a.l2 && l < it.nv ? gexp(gl - gc) * rs_own : 0.f;
  }

  // A: ten 16x16 tiles; lane element (jj): i = 16 tm + 4 lg + jj, j = 16 tn + lc
#pragma unroll
  for (int t = 0; t < 10; ++t) {
    int tm, tn;
    tri_tile(t, tm, tn);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < K / 32; ++ks) mma(acc, kf[tm][ks], kf[tn][ks]);
    const int i0 = 16 * tm + 4 * lg;
    const int j = 16 * tn + lc;
    const f32x4 gi = *reinterpret_cast<const f32x4*>(s_g + i0);
    const f32x4 bi = *reinterpret_cast<const f32x4*>(s_g + C + i0);
    const float gj = s_g[j];
    float* blk = s_A + tri_blk(tm, tn) * P::BLK + (4 * lg) * LDB + lc;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) blk[jj * LDB] = i0 + jj > j ? acc[jj] * gexp(gi[jj] - gj) * bi[jj] : 0.f;
  }

  // diagonal blocks, then the off-diagonal blocks row block by row block
  float x[16];
  diag_blocks(s_A, x);
  auto blk = [&](int r, int c) { return s_A + tri_blk(r, c) * P::BLK; };
  f32x4 X[6];                                            // X_ij at index tri_blk(i - 1, j)
#pragma unroll
  for (int i = 1; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < i; ++j) {
      f32x4 t = {0.f, 0.f, 0.f, 0.f}, r = {0.f, 0.f, 0.f, 0.f};
      mma16_f32_lds(t, blk(i, j), LDB, blk(j, j), LDB);                     // A_ij D_j
#pragma unroll
      for (int k = j + 1; k < i; ++k) mma16_f32_lds_reg(t, blk(i, k), LDB, X[tri_blk(k - 1, j)]);   // A_ik X_kj
      mma16_f32_lds_reg(r, blk(i, i), LDB, t);                               // D_i (...)
      X[tri_blk(i - 1, j)] = -r;
    }
  }

  // Ai rounded to bf16 once (solve_tril.py:331 stores it in k's dtype), rows
  // in pcol order, staged over the dead block area, then stored
  bf16* s_Ai = reinterpret_cast<bf16*>(s_A);
#pragma unroll
  for (int q = 0; q < 8; ++q)
    *reinterpret_cast<uint4*>(s_Ai + 8 * (64 * q + l)) = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
  for (int i = 0; i < 16; ++i) s_Ai[(16 * lg + i) * C + pcol(16 * lg + lc)] = (bf16)x[i];
#pragma unroll
  for (int i = 1; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < i; ++j)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
        s_Ai[(16 * i + 4 * lg + jj) * C + pcol(16 * j + lc)] = (bf16)X[tri_blk(i - 1, j)][jj];
  bf16* dst = reinterpret_cast<bf16*>(rec);
#pragma unroll
  for (int q = 0; q < 8; ++q)
    *reinterpret_cast<uint4*>(dst + 8 * (64 * q + l)) = *reinterpret_cast<const uint4*>(s_Ai + 8 * (64 * q + l));
}

// ---------------------------------------------------------------------------
// the chunk engine: seg_trans on fp8 k (two barriers per chunk)
// ---------------------------------------------------------------------------
// Workgroup: one wave per two 16-column tiles of [M | R] (tiles wid and wid +
// NW).  Each wave keeps its fp32 state tiles (K rows) in VGPRs in the MFMA
// accumulator layout.  (bf16 inputs run the pipelined seg_trans_kernel and the
// producer/consumer seg_out_kernel, which reuse the tiles, lane offsets and
// products defined here.)
//
// Per chunk (two workgroup barriers):
//   top      this wave's direct loads of the chunk have landed (k, v and the
//            chunk record: Ai = (I + A)^-1 and the chunk vectors gc, exp(gc)
//            scale, exp(gc), the update gate exp(gc_last - gc), beta and
//            exp(gc_last), formed once by seg_prep); fp8 k is dequantised to
//            bf16 after a barrier.
//   barrier 1; the next chunk's loads go into the other buffer (every wave is
//            done with the chunk that used it), one direct-load instruction at
//            a time between the steps of phase A, so that no wave stalls on a
//            full memory queue.
//   phase A  [own]    X as bf16 operand fragments; u = Ai bf16(v beta) for
//                     the wave's R columns;
//            [shared] w tiles into LDS.  w = Ai bf16(bf16(k beta) exp(gc)),
//                     stored negated, so that v' = u - w X is one MFMA
//                     accumulation onto u.
//   barrier 2
//   phase B  v' = u + (-w) X; X = exp(gc_last) X + k^T bf16(v' gate).
// LDS lane offsets are computed once per segment and tile bases are
// compile-time constants (the chunk loop is unrolled over the two buffers), so
// a fragment read is a fixed VGPR plus an immediate offset.
template <typename TQ, int K, int V>
struct Eng {
  static constexpr bool FP8 = sizeof(TQ) == 1;
  static constexpr int NW = (K + V) / 32;
  static constexpr int NT = NW * WAVE;
  static constexpr int CT = 2;                            // 16-column state tiles per wave
  static constexpr int KT = K / 16;
  static constexpr int NDG = K / 64;                      // w units per token tile (4 d tiles each)
  static constexpr int LDW = K + 8;                       // s_w row stride (elements), pcol order
  static constexpr uint32_t KB = C * K * 2, VB = C * V * 2, AB = C * C * 2, RAW = C * K;
  // Tiles read transposed (k, v) lie in the first 64 KB, so that one lane VGPR
  // plus a 16-bit immediate reaches them: bf16 k of both buffers (or the one
  // dequantised fp8 k tile), then v of both buffers.
  static constexpr uint32_t k_tile(int p) { return FP8 ? 0u : (uint32_t)p * KB; }
  static constexpr uint32_t v_tile(int p) { return (FP8 ? KB : 2 * KB) + (uint32_t)p * VB; }
  static constexpr uint32_t tr_end = (FP8 ? KB : 2 * KB) + 2 * VB;
  static constexpr uint32_t kraw(int p) { return tr_end + (uint32_t)p * RAW; }       // fp8 inputs as loaded
  static constexpr uint32_t raw_end = FP8 ? tr_end + 2 * RAW : tr_end;
  // the chunk record as loaded: Ai, then the chunk vectors (vec_tile)
  static constexpr uint32_t RB = kSegRecordBytes;
  static constexpr uint32_t ai_tile(int p) { return raw_end + (uint32_t)p * RB; }
  static constexpr uint32_t vec_tile(int p) { return ai_tile(p) + AB; }
  static constexpr uint32_t off_w = raw_end + 2 * RB;
  static constexpr uint32_t total = off_w + C * LDW * 2;
  static_assert(tr_end + 0 <= 65536, "transposed tiles must lie in the first 64 KB of LDS");
  static_assert(total <= 160 * 1024, "chunk tiles do not fit in LDS");
};

// Per-lane LDS byte offsets, fixed for the whole segment (lane l: lc = l % 16, lg = l / 16).
template <int K>
struct LaneOffs {
  uint32_t krow[K / 32];        // Tile<K> row lc, chunk 4ks + lg (q, k rows; rows 16t + lc add 32 t K)
  uint32_t qacc[K / 32][2];     // Tile<K> row lc, the two 8-byte pieces of the accumulator K order
  uint32_t ktr[K / 16];         // absolute LDS address of the transposed read of column tile dt
  uint32_t airow[2];            // Tile<64> row lc, chunk 4ks + lg
  uint32_t w;                   // s_w: row lc, position 8 lg
  uint32_t aqk;                 // s_Aqk: row lc, position 8 lg
};

// LDS address of the transposed read (see Tile::col_tr_addr, rows r0 of K step 0)
// of column tile ct of a Tile<NC>
template <int NC>
__device__ __forceinline__ uint32_t tr_lane_addr(uint32_t lds0, int ct) {
  const int l = lane_id();
  const int lg = l >> 4, i = l & 15;
  const int col = 16 * ct + 4 * (i & 3);
  return lds0 + 2 * (Tile<NC>::off(4 * lg + (i >> 2), col >> 3) + (col & 7));
}

template <int K, int LDW, int LDQ>
__device__ __forceinline__ void lane_offsets(LaneOffs<K>& o, uint32_t lds0) {
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;
#pragma unroll
  for (int ks = 0; ks < K / 32; ++ks) {
    o.krow[ks] = 2 * Tile<K>::off(lc, 4 * ks + lg);
    o.qacc[ks][0] = 2 * (Tile<K>::off(lc, 4 * ks + (lg >> 1)) + 4 * (lg & 1));
    o.qacc[ks][1] = 2 * (Tile<K>::off(lc, 4 * ks + (lg >> 1) + 2) + 4 * (lg & 1));
  }
#pragma unroll
  for (int dt = 0; dt < K / 16; ++dt) o.ktr[dt] = tr_lane_addr<K>(lds0, dt);
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) o.airow[ks] = 2 * Tile<C>::off(lc, 4 * ks + lg);
  o.w = 2 * (lc * LDW + 8 * lg);
  o.aqk = 2 * (lc * LDQ + 8 * lg);
}

// ds_read_b64_tr_b16 at LDS byte address a + O: the constant O folds into the
// instruction's offset field, so the lane address stays one fixed VGPR.  (The
// compiler schedules these reads and their waits; the direct loads it cannot
// see -- they are asm -- so it adds no vmcnt wait for the prefetch in flight.)
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef __attribute__((address_space(3))) unsigned char lds_u8;
template <uint32_t O>
__device__ __forceinline__ u32x2 tr_rd(uint32_t a) {
  lds_u8* p = reinterpret_cast<lds_u8*>(a) + O;
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(reinterpret_cast<lds_s16x4*>(p)));
}
template <int O0, int O1>
__device__ __forceinline__ Frag<bf16> tr2(uint32_t a) {
  return tr_pair(tr_rd<O0>(a), tr_rd<O1>(a));
}
template <int O0, int O1, int O2, int O3>
__device__ __forceinline__ void tr4(uint32_t a, Frag<bf16>& f0, Frag<bf16>& f1) {
  f0 = tr_pair(tr_rd<O0>(a), tr_rd<O1>(a));
  f1 = tr_pair(tr_rd<O2>(a), tr_rd<O3>(a));
}
template <int O0, int O1, int O2, int O3>
__device__ __forceinline__ void tr4x2(uint32_t a, uint32_t b, Frag<bf16>& fa0, Frag<bf16>& fa1, Frag<bf16>& fb0,
                                      Frag<bf16>& fb1) {
  tr4<O0, O1, O2, O3>(a, fa0, fa1);
  tr4<O0, O1, O2, O3>(b, fb0, fb1);
}
// K step 0 (tokens 0-31) or both K steps of a transposed fragment of the
// [64][NC] tile at LDS byte offset TB: rows r0 and r0 + 16 of each step.
template <int NC, uint32_t TB>
__device__ __forceinline__ Frag<bf16> trT1(uint32_t a) {
  return tr2<TB, TB + 32 * NC>(a);
}
template <int NC, uint32_t TB>
__device__ __forceinline__ void trT(uint32_t a, Frag<bf16>& f0, Frag<bf16>& f1) {
  tr4<TB, TB + 32 * NC, TB + 64 * NC, TB + 96 * NC>(a, f0, f1);
}
template <int NC, uint32_t TB>
__device__ __forceinline__ void trT2(uint32_t a, uint32_t b, Frag<bf16>& fa0, Frag<bf16>& fa1, Frag<bf16>& fb0,
                                     Frag<bf16>& fb1) {
  tr4x2<TB, TB + 32 * NC, TB + 64 * NC, TB + 96 * NC>(a, b, fa0, fa1, fb0, fb1);
}

// Four column tiles at once (lane addresses a[0..3]): K step 0 only or both K steps.
template <int O0, int O1>
__device__ __forceinline__ void tr8x(const uint32_t (&a)[4], Frag<bf16> (&f)[4][2]) {
#pragma unroll
  for (int e = 0; e < 4; ++e) f[e][0] = tr_pair(tr_rd<O0>(a[e]), tr_rd<O1>(a[e]));
}
template <int O0, int O1, int O2, int O3>
__device__ __forceinline__ void tr16x(const uint32_t (&a)[4], Frag<bf16> (&f)[4][2]) {
#pragma unroll
  for (int e = 0; e < 4; ++e) tr4<O0, O1, O2, O3>(a[e], f[e][0], f[e][1]);
}
// Four column tiles of a [64][NC] tile at LDS byte offset TB, K step 0 or both K steps.
template <int NC, uint32_t TB>
__device__ __forceinline__ void trT4x1(const uint32_t (&a)[4], Frag<bf16> (&f)[4][2]) {
  tr8x<TB, TB + 32 * NC>(a, f);
}
template <int NC, uint32_t TB>
__device__ __forceinline__ void trT4x2(const uint32_t (&a)[4], Frag<bf16> (&f)[4][2]) {
  tr16x<TB, TB + 32 * NC, TB + 64 * NC, TB + 96 * NC>(a, f);
}

// Direct loads of one [64][NC] input tile with the lane source offsets
// computed once (full chunks; a partial chunk takes load_tile).
template <typename T, int NC, int NT>
struct LoadOffs {
  static constexpr int CPR = NC / 8;
  static constexpr int UNITS = 64 * CPR;
  static constexpr int N = (UNITS + NT - 1) / NT;
  uint32_t o[N];
  __device__ __forceinline__ void init(uint32_t row_bytes) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int u = min(tid + NT * i, UNITS - 1);
      const int r = u / CPR, pos = u % CPR;
      const int c8 = sizeof(T) == 2 ? (pos ^ Tile<NC>::swz(r)) : pos;
      o[i] = (uint32_t)r * row_bytes + (uint32_t)(8 * c8 * sizeof(T));
    }
  }
  __device__ __forceinline__ void issue1(int i, const T* base_t, uint32_t dst) const {
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
    if (UNITS % NT != 0 && NT * i + WAVE * wid >= UNITS) return;      // uniform per wave
    direct8<T>(base_t, o[i], dst + (NT * i + WAVE * wid) * 8 * sizeof(T));
  }
  __device__ __forceinline__ void issue(const T* base_t, uint32_t dst) const {
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
    const unsigned char* base = reinterpret_cast<const unsigned char*>(base_t);
#pragma unroll
    for (int i = 0; i < N; ++i) {
      if (UNITS % NT != 0 && NT * i + WAVE * wid >= UNITS) break;      // uniform per wave
      direct8<T>(base, o[i], dst + (NT * i + WAVE * wid) * 8 * sizeof(T));
    }
  }
};

// Lane source offsets of the chunk record (kSegRecordBytes): the Ai tile in
// 16-byte units with the Tile<64> swizzle, then the vectors in plain order.
template <int NT>
struct RecOffs {
  static constexpr int AU = C * C * 2 / 16;              // Ai units
  static constexpr int UNITS = kSegRecordBytes / 16;
  static constexpr int N = (UNITS + NT - 1) / NT;
  uint32_t o[N];
  __device__ __forceinline__ void init() {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int u = min(tid + NT * i, UNITS - 1);
      if (u < AU) {
        const int r = u / 8, pos = u % 8;
        o[i] = (uint32_t)(r * C * 2 + 16 * (pos ^ Tile<C>::swz(r)));
      } else {
        o[i] = (uint32_t)(16 * u);
      }
    }
  }
  __device__ __forceinline__ void issue1(int i, const unsigned char* base, uint32_t dst) const {
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
    if (UNITS % NT != 0 && NT * i + WAVE * wid >= UNITS) return;      // uniform per wave
    direct8<bf16>(base, o[i], dst + (NT * i + WAVE * wid) * 16);
  }
};

// The direct loads of one chunk, as a fixed sequence of per-wave load
// instructions ("slots"): k, v, then the chunk record.  Slot S of the next
// chunk is issued at a fixed point of the current chunk's step.
template <typename TQ, int K, int V>
struct ChunkLoads {
  using E = Eng<TQ, K, V>;
  static constexpr int NTL = E::NT;                      // loader threads: every wave
  static constexpr int NQ = LoadOffs<TQ, K, NTL>::N;
  static constexpr int NV = LoadOffs<bf16, V, NTL>::N;
  static constexpr int NR = RecOffs<NTL>::N;
  static constexpr int NS = NQ + NV + NR;                 // slots per chunk
  LoadOffs<TQ, K, NTL> qk;
  LoadOffs<bf16, V, NTL> v;
  RecOffs<NTL> rec;
  __device__ __forceinline__ void init(int H) {
    qk.init((uint32_t)(H * K * sizeof(TQ)));
    v.init((uint32_t)(H * V * 2));
    rec.init();
  }
  // Slot S of the chunk at tokens t0 .. t0 + nv - 1 (record rec_src) into
  // buffer P.  A partial chunk (nv < 64) loads a whole k/v tile at the
  // tile's first slot, rows past the end reading row 0.
  template <int P, int S>
  __device__ __forceinline__ void slot(uint32_t lds0, const void* kp, const void* vp, int64_t t0, int nv, int h,
                                       int H, const unsigned char* rec_src) const {
    constexpr int S1 = NQ;                                 // first v slot
    constexpr int S2 = S1 + NV;                            // first record slot
    const int64_t e0 = t0 * H + h;
    if constexpr (S < S1) {
      constexpr int i = S;
      const TQ* src = reinterpret_cast<const TQ*>(kp) + e0 * K;
      const uint32_t dst = lds0 + (E::FP8 ? E::kraw(P) : E::k_tile(P));
      if (nv == C) qk.issue1(i, src, dst);
      else if (i == 0) load_tile<TQ, K, NTL>(src, (uint32_t)(H * K * sizeof(TQ)), nv, dst);
    } else if constexpr (S < S2) {
      constexpr int i = S - S1;
      const bf16* src = reinterpret_cast<const bf16*>(vp) + e0 * V;
      if (nv == C) v.issue1(i, src, lds0 + E::v_tile(P));
      else if (i == 0) load_tile<bf16, V, NTL>(src, (uint32_t)(H * V * 2), nv, lds0 + E::v_tile(P));
    } else if constexpr (S < NS) {
      rec.issue1(S - S2, rec_src, lds0 + E::ai_tile(P));
    }
  }
  // slots S .. NS - 1
  template <int P, int S>
  __device__ __forceinline__ void slots_from(uint32_t lds0, const void* kp, const void* vp, int64_t t0, int nv, int h,
                                             int H, const unsigned char* rec_src) const {
    if constexpr (S < NS) {
      slot<P, S>(lds0, kp, vp, t0, nv, h, H, rec_src);
      slots_from<P, S + 1>(lds0, kp, vp, t0, nv, h, H, rec_src);
    }
  }
};

// Scale the 8 bf16 values of fragment f (K order of an accumulator tile pair:
// indices 32 ks + 4 lg + e, 32 ks + 16 + 4 lg + e) by the vector x, rounded to bf16.
__device__ __forceinline__ Frag<bf16> scale_frag(const Frag<bf16>& f, const float* x, int ks) {
  const int lg = lane_id() >> 4;
  const f32x4 s0 = *reinterpret_cast<const f32x4*>(x + 32 * ks + 4 * lg);
  const f32x4 s1 = *reinterpret_cast<const f32x4*>(x + 32 * ks + 16 + 4 * lg);
  float y[8];
  frag_unpack(f, y);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    y[e] *= s0[e];
    y[4 + e] *= s1[e];
  }
  return frag_pack(y);
}

// The w operand of wy_fast.py:74-78 for the 8 tokens of fragment f (K order as
// in scale_frag): bf16(bf16(k beta) exp(gc)).  k beta is a bf16 product (exact
// in fp32, rounded once), then scaled by exp(gc) in fp32 and rounded again.
__device__ __forceinline__ Frag<bf16> kb_frag(const Frag<bf16>& f, const float* beta, const float* eg, int ks,
                                              const float* rk = nullptr) {
  const int lg = lane_id() >> 4;
  const f32x4 b0 = *reinterpret_cast<const f32x4*>(beta + 32 * ks + 4 * lg);
  const f32x4 b1 = *reinterpret_cast<const f32x4*>(beta + 32 * ks + 16 + 4 * lg);
  const f32x4 e0 = *reinterpret_cast<const f32x4*>(eg + 32 * ks + 4 * lg);
  const f32x4 e1 = *reinterpret_cast<const f32x4*>(eg + 32 * ks + 16 + 4 * lg);
  float y[8];
  frag_unpack(f, y);
  if (rk != nullptr) {                                   // the in-op L2 norm: y = bf16(k rstd) first
    const f32x4 r0 = *reinterpret_cast<const f32x4*>(rk + 32 * ks + 4 * lg);
    const f32x4 r1 = *reinterpret_cast<const f32x4*>(rk + 32 * ks + 16 + 4 * lg);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      y[e] *= r0[e];
      y[4 + e] *= r1[e];
    }
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      const uint32_t r = cvt_pk_bf16(y[e], y[e + 1]);
      y[e] = bf16_lo(r);
      y[e + 1] = bf16_hi(r);
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    y[e] *= b0[e];
    y[4 + e] *= b1[e];
  }
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    const uint32_t r = cvt_pk_bf16(y[e], y[e + 1]);
    y[e] = bf16_lo(r);
    y[e + 1] = bf16_hi(r);
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    y[e] *= e0[e];
    y[4 + e] *= e1[e];
  }
  return frag_pack(y);
}

// Round the 4 floats of an accumulator tile to bf16 and back (two packed conversions).
__device__ __forceinline__ f32x4 round4(const f32x4& a) {
  const uint32_t p0 = cvt_pk_bf16(a[0], a[1]), p1 = cvt_pk_bf16(a[2], a[3]);
  return f32x4{bf16_lo(p0), bf16_hi(p0), bf16_lo(p1), bf16_hi(p1)};
}

// One w unit: token tile tn, d tiles 4 DG .. 4 DG + 3.  B = rows 16 tn + lc of
// Ai, A = kb^T with kb = bf16(bf16(k beta) exp(gc)) (wy_fast.py:67-81); the
// tile -w^T[d][i] goes to s_w[i][pcol(d)].
template <typename E, int K, int DG, int P>
__device__ __forceinline__ void w_unit(unsigned char* smem, const LaneOffs<K>& lo, const float* vec, int tn) {
  const unsigned char* ai = smem + E::ai_tile(P) + 32 * tn * C;
  const int nks = tn / 2 + 1;                                   // Ai is lower triangular
  Frag<bf16> b0 = frag_at<bf16>(reinterpret_cast<const bf16*>(ai + lo.airow[0]));
  Frag<bf16> b1 = b0;
  if (nks == 2) b1 = frag_at<bf16>(reinterpret_cast<const bf16*>(ai + lo.airow[1]));
  unsigned char* wt = smem + E::off_w + lo.w + 32 * tn * E::LDW;
  const uint32_t ka[4] = {lo.ktr[4 * DG], lo.ktr[4 * DG + 1], lo.ktr[4 * DG + 2], lo.ktr[4 * DG + 3]};
  Frag<bf16> kf[4][2];
  if (nks == 2) trT4x2<K, E::k_tile(P)>(ka, kf);
  else trT4x1<K, E::k_tile(P)>(ka, kf);
#pragma unroll
  for (int dd = 0; dd < 4; ++dd) {
    const int dt = 4 * DG + dd;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    mma(acc, kb_frag(kf[dd][0], vec + 4 * C, vec + 2 * C, 0), b0);
    if (nks == 2) mma(acc, kb_frag(kf[dd][1], vec + 4 * C, vec + 2 * C, 1), b1);
    uint2 pk;
    pk.x = pack_bf16x2(-acc[0], -acc[1]);
    pk.y = pack_bf16x2(-acc[2], -acc[3]);
    *reinterpret_cast<uint2*>(wt + 2 * (32 * (dt >> 1) + 4 * (dt & 1))) = pk;
  }
}

// u (64 tokens x 16 columns) = Ai bf16(v beta) of the V column tile whose
// transposed read starts at vtr, rounded to bf16 (wy_fast.py:55-65).
template <typename E, int V, int P>
__device__ __forceinline__ void u_tile(const unsigned char* smem, const uint32_t (&airow)[2], uint32_t vtr,
                                       const float* vec, f32x4 (&Y)[4]) {
  Frag<bf16> vb0, vb1;
  trT<V, E::v_tile(P)>(vtr, vb0, vb1);
  vb0 = scale_frag(vb0, vec + 4 * C, 0);
  vb1 = scale_frag(vb1, vec + 4 * C, 1);
  const unsigned char* ai = smem + E::ai_tile(P);
#pragma unroll
  for (int tm = 0; tm < 4; ++tm) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    mma(acc, frag_at<bf16>(reinterpret_cast<const bf16*>(ai + 32 * tm * C + airow[0])), vb0);
    if (tm >= 2) mma(acc, frag_at<bf16>(reinterpret_cast<const bf16*>(ai + 32 * tm * C + airow[1])), vb1);
    Y[tm] = round4(acc);
  }
}

// Y (64 tokens x 16 CT columns) += (-w) X, X given as operand fragments of its K rows
template <typename E, int K, int CT>
__device__ __forceinline__ void add_wx(const unsigned char* smem, uint32_t w_lane, const Frag<bf16> (&xb)[K / 32][CT],
                                       f32x4 (&Y)[4][CT]) {
  const unsigned char* wt = smem + E::off_w + w_lane;
#pragma unroll
  for (int tm = 0; tm < 4; ++tm) {
#pragma unroll
    for (int ks = 0; ks < K / 32; ++ks) {
      const Frag<bf16> a = frag_at<bf16>(reinterpret_cast<const bf16*>(wt + 32 * tm * E::LDW + 64 * ks));
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) mma(Y[tm][ct], a, xb[ks][ct]);
    }
  }
}

// S (K x 16 CT, accumulator tiles) <- gamma S + k^T vg
template <typename E, int K, int CT, int P>
__device__ __forceinline__ void update_state(const LaneOffs<K>& lo, const Frag<bf16> (&vg)[2][CT], float gamma,
                                             f32x4 (&S)[K / 16][CT]) {
#pragma unroll
  for (int tq = 0; tq < K / 16; tq += 4) {
    const uint32_t ka[4] = {lo.ktr[tq], lo.ktr[tq + 1], lo.ktr[tq + 2], lo.ktr[tq + 3]};
    Frag<bf16> kf[4][2];
    trT4x2<K, E::k_tile(P)>(ka, kf);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        S[tq + e][ct] *= gamma;
        mma(S[tq + e][ct], kf[e][0], vg[0][ct]);
        mma(S[tq + e][ct], kf[e][1], vg[1][ct]);
      }
    }
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

// One Aqk tile t (tm >= tn, tri_tile order) of a chunk whose k and q tiles
// start at kt0 and qt0: lane i = 16 tm + lc (q side) and j = 16 tn + 4 lg + jj
// (k side): Aqk[i][j] = exp(gc_i - gc_j) q_i.k_j for i >= j
// (chunk_o.py:99-118), stored bf16 at s_Aqk[i][pcol(j)] -- four consecutive
// positions, one 8-byte write.
template <int K, int LDQ>
__device__ __forceinline__ void aqk_tile_at(const unsigned char* kt0, const unsigned char* qt0, unsigned char* s_aqk,
                                            const LaneOffs<K>& lo, const float* vec, int t) {
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;
  int tm, tn;
  tri_tile(t, tm, tn);
  const unsigned char* kt = kt0 + 32 * tn * K;
  const unsigned char* qt = qt0 + 32 * tm * K;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < K / 32; ++ks)
    mma(acc, frag_at<bf16>(reinterpret_cast<const bf16*>(kt + lo.krow[ks])),
        frag_at<bf16>(reinterpret_cast<const bf16*>(qt + lo.krow[ks])));
  const float gi = vec[16 * tm + lc];
  const f32x4 gj = *reinterpret_cast<const f32x4*>(vec + 16 * tn + 4 * lg);
  float x[4];
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    x[jj] = acc[jj] * __builtin_amdgcn_exp2f((gi - gj[jj]) * 1.4426950408889634f);
    if (tm == tn && lc < 4 * lg + jj) x[jj] = 0.f;
  }
  *reinterpret_cast<uint2*>(s_aqk + lo.aqk + 2 * (16 * tm * LDQ + 32 * (tn >> 1) + 4 * (tn & 1))) =
      make_uint2(pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3]));
}

// ---------------------------------------------------------------------------
// seg_out: exact recurrence + output over one segment, on two kinds of wave
// ---------------------------------------------------------------------------
// Only part of a chunk step needs the state S: o_inter = q h, v' = u - w h,
// o = (o_inter exp(gc) + Aqk v') scale, and the update S = exp(gc_last) S +
// k^T (v' gate).  w, u and Aqk depend on the chunk's inputs alone.  The
// consumer waves (one per 16 state columns, NCW = V/16) run the
// state-dependent part of chunk c and, after it, Aqk of chunk c + 1; four
// producer waves meanwhile form w and u of chunk c + 1 in registers (the Ai
// rows they share read once) and write them to LDS after the mid-step
// barrier.  The inputs of chunk c + 2 reach LDS through registers, into
// buffers no wave reads then, each part followed by the loads of the same part
// of chunk c + 3; the parts are spread over both halves of the step, since a
// CU issues global loads at a limited rate.
//
// Iteration c (c = -1 .. nch - 1), two workgroup barriers:
//   B1; consumers: h = bf16(S), v' = u + (-w) h, o_inter and o (stored);
//       producers: k of chunk c + 2 to LDS (+ loads of chunk c + 3), w and u
//                  of chunk c + 1 into registers;
//   B2; consumers: S update with k of chunk c, Aqk of chunk c + 1; v, Ai and
//                  the vectors of chunk c + 2 to LDS (+ loads of chunk c + 3);
//       producers: w, u of chunk c + 1 to LDS; q of chunk c + 2 to LDS
//                  (+ loads of chunk c + 3).
// Buffers: q of chunk x in q_tile(x % 2), k in k_tile(x % 3), the chunk
// vectors in vec_tile(x % 3); v and Ai of chunk c + 1 only (the
// producers' inputs); w, Aqk and u of chunk c only.
struct SegOutArgs {
  const void* q;
  const void* k;
  const void* v;
  const float* q_scale;
  const float* k_scale;
  const void* h0;             // [N, H, K, V] or nullptr
  int h0_dtype;
  const float* s_init;        // [NS, H, K, V] fp32 state at each segment start (j >= 1)
  const void* Ai;             // [chunks, H] chunk records from seg_prep
  float scale;
  void* o;                    // [B*T, H, V]
  float* ht;                  // [N, H, K, V] or nullptr
  int l2;                     // normalise q and k rows on their way to LDS (the in-op L2 norm)
  // the layer's gated RMSNorm epilogue fused into the output (seg_out_kernel<..., true>): o is
  // replaced by y = bf16(o) rstd w [+ b], times g sigmoid(g) (or sigmoid(g)), rstd over the V columns
  const bf16* gate;           // [B*T, H, V] bf16
  const void* nw;             // [V] in nw_dtype, or nullptr (ones)
  const void* nb;             // [V] in nw_dtype, or nullptr (zeros)
  int nw_dtype;
  float eps;
  int sigmoid_only;
};

template <typename TQ, int K, int V>
struct OutPlan {
  static constexpr bool FP8 = sizeof(TQ) == 1;
  static constexpr int NCW = V / 16;                     // consumer waves 0 .. NCW-1, one per 16 state columns
  static constexpr int NPW = 4;                          // producer waves NCW .. NCW+3
  static constexpr int NW = NCW + NPW, NT = NW * WAVE;
  static constexpr int CTN = 1;                          // 16-column state tiles per consumer
  static constexpr int KT = K / 16, KS = K / 32, NDG = K / 64;
  static constexpr int LDW = K + 8;                      // -w rows (pcol order)
  static constexpr int LDQ = C + 8;                      // Aqk rows (pcol order)
  static constexpr int LDU = C + 8;                      // u^T rows (token order)
  static constexpr uint32_t KB = C * K * 2, VB = C * V * 2, AB = C * C * 2, VECB = 8 * C * 4;
  // tiles read transposed first (16-bit offset field): k (three buffers), v
  static constexpr uint32_t k_tile(int b) { return (uint32_t)b * KB; }
  static constexpr uint32_t v_tile = 3 * KB;
  static constexpr uint32_t tr_end = v_tile + VB;
  static_assert(tr_end <= 65536, "transposed-read tiles must lie in the first 64 KB");
  static constexpr uint32_t q_tile(int b) { return tr_end + (uint32_t)b * KB; }
  static constexpr uint32_t ai_tile = tr_end + 2 * KB;
  static constexpr uint32_t vec_tile(int b) { return ai_tile + AB + (uint32_t)b * VECB; }
  static constexpr uint32_t off_w = vec_tile(3);
  static constexpr uint32_t off_aqk = off_w + C * LDW * 2;
  static constexpr uint32_t off_u = off_aqk + C * LDQ * 2;
  static constexpr uint32_t total = off_u + V * LDU * 2;
  // with the fused norm epilogue: each consumer wave's sum of squares of its columns per token
  static constexpr uint32_t off_ss = total;
  static constexpr uint32_t off_nw = off_ss + C * NCW * 4;   // its weight and bias, fp32 [2][V]
  static constexpr uint32_t total_norm = off_nw + 2 * V * 4;
  // staging: units of 8 elements (16 bytes bf16, 8 bytes fp8)
  static constexpr int PT = NPW * WAVE;                  // producer threads
  static constexpr int QU = C * K / 8, VU = C * V / 8, RU = kSegRecordBytes / 16, AU = AB / 16;
};

// The inputs of a chunk on their way to LDS.  Producer threads (NPW waves)
// hold q and k, consumer threads (NCW waves) hold v and the record, as units of
// 8 elements (16 bytes bf16, 8 bytes fp8): unit u = thread + threads * i, row
// u / (cols / 8), 8-column group u % (cols / 8); rows past the chunk end read
// row 0.  Record units below AU are Ai (swizzled rows), the rest
// the chunk vectors.
template <typename TQ, int K, int V>
struct ChunkSrc {
  const unsigned char *q, *k, *v, *rec;
  int nv;
  __device__ __forceinline__ ChunkSrc(const SegOutArgs& a, int64_t t0, int nv_, int h, int H, const unsigned char* r)
      : q(reinterpret_cast<const unsigned char*>(a.q) + (t0 * H + h) * K * sizeof(TQ)),
        k(reinterpret_cast<const unsigned char*>(a.k) + (t0 * H + h) * K * sizeof(TQ)),
        v(reinterpret_cast<const unsigned char*>(a.v) + (t0 * H + h) * V * 2),
        rec(r),
        nv(nv_) {}
};

template <typename TQ, int K, int V>
struct ProdStage {
  using P = OutPlan<TQ, K, V>;
  using QT = typename std::conditional<P::FP8, u32x2, u32x4>::type;
  static constexpr int N = P::QU / P::PT;
  static_assert(P::QU % P::PT == 0, "q/k units split evenly over the producer threads");
  QT q[N], k[N];
  __device__ __forceinline__ static uint32_t src_off(int i, int nv, int H) {
    const int u = (int)threadIdx.x - P::NCW * WAVE + P::PT * i;
    const int r = u / (K / 8), c8 = u % (K / 8);
    return (uint32_t)(r < nv ? r : 0) * (uint32_t)(H * K * sizeof(TQ)) + (uint32_t)(c8 * 8 * sizeof(TQ));
  }
  __device__ __forceinline__ static uint32_t dst_off(int i) {
    const int u = (int)threadIdx.x - P::NCW * WAVE + P::PT * i;
    return 2 * Tile<K>::off(u / (K / 8), u % (K / 8));
  }
  __device__ __forceinline__ static u32x4 to_bf16(const QT& x, float scale) {
    if constexpr (P::FP8) {
      float f[8];
      fp8x4_to_f32(x[0], f);
      fp8x4_to_f32(x[1], f + 4);
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] *= scale;
      return __builtin_bit_cast(u32x4, frag_pack(f).v);
    } else {
      return x;
    }
  }
  __device__ __forceinline__ void load_k(const ChunkSrc<TQ, K, V>& s, int H) {
#pragma unroll
    for (int i = 0; i < N; ++i) k[i] = *reinterpret_cast<const QT*>(s.k + src_off(i, s.nv, H));
  }
  __device__ __forceinline__ void load_q(const ChunkSrc<TQ, K, V>& s, int H) {
#pragma unroll
    for (int i = 0; i < N; ++i) q[i] = *reinterpret_cast<const QT*>(s.q + src_off(i, s.nv, H));
  }
  __device__ __forceinline__ void store_k(unsigned char* smem, int kb, float ks, bool l2) const {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      u32x4 x = to_bf16(k[i], ks);
      if (l2) x = l2_row(x);
      *reinterpret_cast<u32x4*>(smem + P::k_tile(kb) + dst_off(i)) = x;
    }
  }
  // the L2 norm of the k rows in registers, ahead of their store (bf16 k only)
  __device__ __forceinline__ void norm_k() {
    if constexpr (!P::FP8) {
#pragma unroll
      for (int i = 0; i < N; ++i) k[i] = l2_row(k[i]);
    }
  }
  // y = bf16(x / sqrt(sum x^2 + 1e-6)) over the row a unit belongs to: the K / 8 units of a row are
  // held by K / 8 consecutive lanes (l2norm.py:98-119, the in-op L2 norm of q and k).  The squares
  // are summed by packed bf16 dot products on the raw words, the row by DPP moves.
  __device__ __forceinline__ static u32x4 l2_row(const u32x4& x) {
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) ss = dot2_bf16(x[e], x[e], ss);
    const float rs = l2_rstd(row_sum_dpp<K / 8>(ss));
    u32x4 y;
#pragma unroll
    for (int e = 0; e < 4; ++e) y[e] = cvt_pk_bf16(__uint_as_float(x[e] << 16) * rs, __uint_as_float(x[e] & 0xffff0000u) * rs);
    return y;
  }
  __device__ __forceinline__ void store_q(unsigned char* smem, int qb, float qs, bool l2) const {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      u32x4 x = to_bf16(q[i], qs);
      if (l2) x = l2_row(x);
      *reinterpret_cast<u32x4*>(smem + P::q_tile(qb) + dst_off(i)) = x;
    }
  }
};

// The in-op L2 norm of a q tile in LDS, in place, by the consumer threads (bf16 q): unit u = thread +
// threads * i as in the producers' staging, so the K / 8 units of a row sit in consecutive lanes
template <typename TQ, int K, int V>
__device__ __forceinline__ void norm_q_tile(unsigned char* tile) {
  using P = OutPlan<TQ, K, V>;
  constexpr int CT = P::NCW * WAVE, NU = P::QU / CT;
  static_assert(P::QU % CT == 0, "q units split evenly over the consumer threads");
#pragma unroll
  for (int i = 0; i < NU; ++i) {
    const int u = (int)threadIdx.x + CT * i;
    u32x4* p = reinterpret_cast<u32x4*>(tile + 2 * Tile<K>::off(u / (K / 8), u % (K / 8)));
    *p = ProdStage<TQ, K, V>::l2_row(*p);
  }
}

template <typename TQ, int K, int V>
struct ConsStage {
  using P = OutPlan<TQ, K, V>;
  static constexpr int CTH = P::NCW * WAVE;              // consumer threads
  static constexpr int NV = P::VU / CTH, NR = (P::RU + CTH - 1) / CTH;
  static_assert(P::VU % CTH == 0 && P::AU % WAVE == 0 && P::RU % WAVE == 0, "units split per wave");
  u32x4 v[NV], r[NR];
  __device__ __forceinline__ void load(const ChunkSrc<TQ, K, V>& s, int H) {
    const int ct = threadIdx.x;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int u = ct + CTH * i;
      const int row = u / (V / 8), c8 = u % (V / 8);
      v[i] = *reinterpret_cast<const u32x4*>(s.v + (uint32_t)(row < s.nv ? row : 0) * (uint32_t)(H * V * 2) +
                                             (uint32_t)(c8 * 16));
    }
#pragma unroll
    for (int i = 0; i < NR; ++i) r[i] = *reinterpret_cast<const u32x4*>(s.rec + 16 * min(ct + CTH * i, P::RU - 1));
  }
  __device__ __forceinline__ void store(unsigned char* smem, int cb) const {
    const int ct = threadIdx.x;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int u = ct + CTH * i;
      *reinterpret_cast<u32x4*>(smem + P::v_tile + 2 * Tile<V>::off(u / (V / 8), u % (V / 8))) = v[i];
    }
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      const int u = ct + CTH * i;                        // uniform per wave against AU and RU
      if (u < P::AU) {
        const int row = u / 8, pos = u % 8;
        *reinterpret_cast<u32x4*>(smem + P::ai_tile + (uint32_t)(row * C * 2 + 16 * (pos ^ Tile<C>::swz(row)))) = r[i];
      } else if (u < P::RU) {
        *reinterpret_cast<u32x4*>(smem + P::vec_tile(cb) + 16 * (uint32_t)(u - P::AU)) = r[i];
      }
    }
  }
};

// The state-independent products of one chunk that the producer waves form,
// held from their computation until the mid-step barrier: the -w tiles of d
// tile pw + 4 i (all four token tiles) and the u column tiles ct = pw + 4 i,
// each as packed bf16.
template <int K, int V>
struct OutProducts {
  static constexpr int NWU = K / 64, NU = (V / 16 + 3) / 4;
  uint2 w[NWU][4];
  uint2 u[NU][4];
};

// sigmoid(z) = 1 / (1 + 2^(-z log2 e)) (v_exp_f32, v_rcp_f32), as the standalone epilogue kernel
__device__ __forceinline__ float norm_sigmoid(float z) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-z * 1.4426950408889634f));
}

template <typename TQ, int K, int V, bool kNorm>
__global__ __launch_bounds__((OutPlan<TQ, K, V>::NT)) void seg_out_kernel(SegOutArgs a, SegGeom G) {
  using P = OutPlan<TQ, K, V>;
  constexpr int KT = P::KT, KS = P::KS, CTN = P::CTN;
  constexpr int LDW = P::LDW, LDQ = P::LDQ, LDU = P::LDU;
  extern __shared__ __align__(16) unsigned char smem[];

  const int h = blockIdx.y;
  const int H = G.H;
  const SegLoc sl = locate_seg(blockIdx.x, G);
  if (!sl.ok) return;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const bool consumer = wid < P::NCW;
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;
  const uint32_t lds0 = lds_addr(smem);
  const float qs = a.q_scale ? a.q_scale[h] : 1.f;
  const float ks_ = a.k_scale ? a.k_scale[h] : 1.f;
  const int64_t t_seg = sl.bos + sl.c0 * C;                 // first token of the segment
  const unsigned char* rec0 = reinterpret_cast<const unsigned char*>(a.Ai) +
                              ((sl.cbase + sl.c0) * H + h) * (int64_t)kSegRecordBytes;
  const int64_t rec_step = (int64_t)H * kSegRecordBytes;
  auto chunk_nv = [&](int c) { return (int)min((int64_t)C, sl.eos - (t_seg + (int64_t)c * C)); };

  LaneOffs<K> lo;
  lane_offsets<K, LDW, LDQ>(lo, lds0);
  // Upper 16x16 tiles of Aqk that operand fragments read (column tile 2 ks + 1
  // of row tile 2 ks) are zero; no chunk writes them.
  {
    bf16* s_aqk = reinterpret_cast<bf16*>(smem + P::off_aqk);
    for (int idx = threadIdx.x; idx < 2 * 16 * 16; idx += P::NT) {
      const int tile = idx >> 8, r = (idx >> 4) & 15, c = idx & 15;
      s_aqk[(32 * tile + r) * LDQ + pcol(32 * tile + 16 + c)] = (bf16)0.f;
    }
  }

  // the in-op L2 norm of bf16 q runs on the consumers (norm_q_tile), that of k on the producers
  const bool q_cons = a.l2 != 0 && !P::FP8;
  // consumer state: lane element (tt, ct, j) = S[16 tt + 4 lg + j][vw + 16 ct + lc]
  const int vw = wid * 16;
  f32x4 S[KT][CTN];
  using SRC = ChunkSrc<TQ, K, V>;
  bf16* o = reinterpret_cast<bf16*>(a.o);
  if (consumer) {
    ConsStage<TQ, K, V> cs;
    const int lane_off = 4 * lg * V + vw + lc;
#pragma unroll
    for (int tt = 0; tt < KT; ++tt)
#pragma unroll
      for (int ct = 0; ct < CTN; ++ct) S[tt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (sl.j == 0 && a.h0 && a.h0_dtype == DT_F32) {
      const float* p = reinterpret_cast<const float*>(a.h0) + ((int64_t)sl.n * H + h) * K * V + lane_off;
#pragma unroll
      for (int tt = 0; tt < KT; ++tt)
#pragma unroll
        for (int ct = 0; ct < CTN; ++ct)
#pragma unroll
          for (int j = 0; j < 4; ++j) S[tt][ct][j] = p[(16 * tt + j) * V + 16 * ct];
    } else if (sl.j == 0 && a.h0) {
      const bf16* p = reinterpret_cast<const bf16*>(a.h0) + ((int64_t)sl.n * H + h) * K * V + lane_off;
#pragma unroll
      for (int tt = 0; tt < KT; ++tt)
#pragma unroll
        for (int ct = 0; ct < CTN; ++ct)
#pragma unroll
          for (int j = 0; j < 4; ++j) S[tt][ct][j] = (float)p[(16 * tt + j) * V + 16 * ct];
    } else if (sl.j > 0) {
      const float* p = a.s_init + ((int64_t)blockIdx.x * H + h) * K * V + lane_off;
#pragma unroll
      for (int tt = 0; tt < KT; ++tt)
#pragma unroll
        for (int ct = 0; ct < CTN; ++ct)
#pragma unroll
          for (int j = 0; j < 4; ++j) S[tt][ct][j] = p[(16 * tt + j) * V + 16 * ct];
    }
    cs.load(SRC(a, t_seg, chunk_nv(0), h, H, rec0), H);
    cs.store(smem, 0);
    if (sl.nch > 1) cs.load(SRC(a, t_seg + C, chunk_nv(1), h, H, rec0 + rec_step), H);
    // the fused epilogue's weight and bias, fp32 in LDS (the consumer threads cover the V columns)
    if constexpr (kNorm) {
      float* s_nw = reinterpret_cast<float*>(smem + P::off_nw);
      for (int col = threadIdx.x; col < V; col += P::NCW * WAVE) {
        s_nw[col] = a.nw ? (a.nw_dtype == DT_F32 ? reinterpret_cast<const float*>(a.nw)[col]
                                                 : (float)reinterpret_cast<const bf16*>(a.nw)[col]) : 1.f;
        s_nw[V + col] = a.nb ? (a.nw_dtype == DT_F32 ? reinterpret_cast<const float*>(a.nb)[col]
                                                     : (float)reinterpret_cast<const bf16*>(a.nb)[col]) : 0.f;
      }
    }
    lds_barrier();
    for (int c = -1; c < sl.nch; ++c) {
      // with the in-op L2 norm of bf16 q: the q rows of chunk c + 1, stored raw by the producers in
      // the previous step, are normalised in place in this half step, where the consumers would wait
      // at B2 for the producers' w and u products; their first reader is Aqk of chunk c + 1 after B2
      if (q_cons && c + 1 < sl.nch) norm_q_tile<TQ, K, V>(smem + P::q_tile((c + 1) & 1));
      // ---------------- B1 .. B2: h, o_inter, v', o of chunk c
      f32x4 Y[4][CTN];
      if (c >= 0) {
        const int qb = c & 1;
        const float* vec = reinterpret_cast<const float*>(smem + P::vec_tile(c % 3));
        const int nvc = chunk_nv(c);
        Frag<bf16> hb[KS][CTN];                          // h = S rounded (chunk_delta_h.py:129-139)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
          for (int ct = 0; ct < CTN; ++ct) hb[ks][ct] = acc_frag(S[2 * ks][ct], S[2 * ks + 1][ct]);
        // v' = u + (-w) h                               (chunk_delta_h.py:141-157)
#pragma unroll
        for (int tm = 0; tm < 4; ++tm)
#pragma unroll
          for (int ct = 0; ct < CTN; ++ct) {
            const uint2 uu = *reinterpret_cast<const uint2*>(
                smem + P::off_u + 2 * ((vw + 16 * ct + lc) * LDU + 16 * tm + 4 * lg));
            Y[tm][ct] = f32x4{bf16_lo(uu.x), bf16_hi(uu.x), bf16_lo(uu.y), bf16_hi(uu.y)};
          }
        {
          const unsigned char* wt = smem + P::off_w + lo.w;
#pragma unroll
          for (int tm = 0; tm < 4; ++tm)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
              const Frag<bf16> wa = frag_at<bf16>(reinterpret_cast<const bf16*>(wt + 32 * tm * LDW + 64 * ks));
#pragma unroll
              for (int ct = 0; ct < CTN; ++ct) mma(Y[tm][ct], wa, hb[ks][ct]);
            }
        }
        if constexpr (kNorm) {
          // the gate of this wave's 16 columns for the epilogue, 64 tokens x 32 bytes, loaded straight
          // into LDS over this wave's 16 rows of u^T: they were read above and the producers rewrite
          // them only after B2.  Lane slot s = 64 j + lane holds token s / 2, 8 columns (s & 1);
          // rows past the chunk end read row 0.
          __builtin_amdgcn_s_waitcnt(0xC07F);          // this wave's u reads have completed
          const unsigned char* gbase = reinterpret_cast<const unsigned char*>(a.gate) +
                                       (((t_seg + (int64_t)c * C) * H + h) * V + vw) * 2;
          const uint32_t slice = lds0 + P::off_u + 2u * vw * LDU;
          // the epilogue's lane-derived addresses are formed where they are used: an opaque copy of
          // the lane index keeps the compiler from holding them in registers across the loop
          int lk = l;
          asm volatile("" : "+v"(lk));
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const int sl_ = 64 * j + lk, t = sl_ >> 1;
            dma16(gbase, (uint32_t)((t < nvc ? t : 0) * H * V * 2 + 16 * (sl_ & 1)),
                  __builtin_amdgcn_readfirstlane(slice + 1024u * j));
          }
        }
        // o^T = (o_inter^T exp(gc) + v'^T bf16(Aqk)^T) scale  (chunk_o.py:84-128), with
        // o_inter^T = h^T q^T (chunk_o.py:84-107)
        Frag<bf16> vn[2][CTN];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
          for (int ct = 0; ct < CTN; ++ct) vn[ks][ct] = acc_frag(Y[2 * ks][ct], Y[2 * ks + 1][ct]);
        const unsigned char* qt = smem + P::q_tile(qb);
        const unsigned char* aq = smem + P::off_aqk + lo.aqk;
        // o_inter^T of the four token tiles (independent accumulation chains)
        f32x4 oi[4][CTN];
#pragma unroll
        for (int tn = 0; tn < 4; ++tn)
#pragma unroll
          for (int ct = 0; ct < CTN; ++ct) oi[tn][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
          for (int tn = 0; tn < 4; ++tn) {
            const uint2 pa = *reinterpret_cast<const uint2*>(qt + 32 * tn * K + lo.qacc[ks][0]);
            const uint2 pb = *reinterpret_cast<const uint2*>(qt + 32 * tn * K + lo.qacc[ks][1]);
            Frag<bf16> b;
            b.v = __builtin_bit_cast(bf16x8, make_uint4(pa.x, pa.y, pb.x, pb.y));
#pragma unroll
            for (int ct = 0; ct < CTN; ++ct) mma(oi[tn][ct], hb[ks][ct], b);
          }
        uint2 ov[4][CTN];
#pragma unroll
        for (int tn = 0; tn < 4; ++tn) {
          const float eg = vec[2 * C + 16 * tn + lc];
#pragma unroll
          for (int ct = 0; ct < CTN; ++ct) {
            f32x4 r = oi[tn][ct] * eg;
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
              if (ks <= tn / 2)
                mma(r, vn[ks][ct], frag_at<bf16>(reinterpret_cast<const bf16*>(aq + 32 * tn * LDQ + 64 * ks)));
            r *= a.scale;
            ov[tn][ct] = make_uint2(pack_bf16x2(r[0], r[1]), pack_bf16x2(r[2], r[3]));
          }
        }
        // store o (token 16 tn + lc, columns vw + 16 ct + 4 lg .. +3).  These compile to FLAT stores
        // (the pointer comes from the argument struct), whose completion the LDS wait of the barrier
        // below includes; as global stores (st_global) the streaming rollout ran 0.1294 ms per frame
        // against 0.1238, config 2 alike.
        unsigned char* ob = reinterpret_cast<unsigned char*>(o + ((t_seg + (int64_t)c * C) * H + h) * V + vw) +
                            8 * lg;
        const uint32_t row_bytes = (uint32_t)H * V * 2;
        if constexpr (kNorm) {
          // the epilogue (fused_norm_gate.py:42-127 on the bf16 o): each wave's share of every token's
          // sum of squares goes to LDS; after a barrier that the producer waves take at the end of
          // their half (the consumers wait there for them in any case) the shares are summed, and y
          // replaces o, with the gate that this wave loaded into LDS above.
          static_assert(CTN == 1, "the epilogue's gate slice holds 16 columns per consumer wave");
          float* s_ss = reinterpret_cast<float*>(smem + P::off_ss);
          int lk = l;
          asm volatile("" : "+v"(lk));
          const int lg = lk >> 4, lc = lk & 15;
#pragma unroll
          for (int tn = 0; tn < 4; ++tn) {
            float ss = 0.f;
            const uint32_t wds[2] = {ov[tn][0].x, ov[tn][0].y};
#pragma unroll
            for (int e = 0; e < 2; ++e) {
              const float x0 = __uint_as_float(wds[e] << 16), x1 = __uint_as_float(wds[e] & 0xffff0000u);
              ss = fmaf(x0, x0, ss);
              ss = fmaf(x1, x1, ss);
            }
            ss += __shfl_xor(ss, 16, WAVE);
            ss += __shfl_xor(ss, 32, WAVE);
            if (lg == 0) s_ss[(16 * tn + lc) * P::NCW + wid] = ss;
          }
          wait_loads();                                  // this wave's gate slice has landed
          lds_barrier();                                 // the row sums (the producers' matching barrier ends their half)
          const float* s_nw = reinterpret_cast<const float*>(smem + P::off_nw);
          const unsigned char* gsl = smem + P::off_u + 2u * vw * LDU + 8 * lg;
          const f32x4 wv4 = *reinterpret_cast<const f32x4*>(s_nw + vw + 4 * lg);
          const f32x4 bv4 = *reinterpret_cast<const f32x4*>(s_nw + V + vw + 4 * lg);
          static_assert(P::NCW % 4 == 0, "row sums are read four shares at a time");
          // lane i sums the shares of token i; each lane then takes rstd of its four tokens
          float tot = 0.f;
#pragma unroll
          for (int w = 0; w < P::NCW; w += 4) {
            const f32x4 sh = *reinterpret_cast<const f32x4*>(s_ss + lk * P::NCW + w);
            tot += (sh[0] + sh[1]) + (sh[2] + sh[3]);
          }
          const float r_own = __builtin_amdgcn_rsqf(tot / (float)V + a.eps);
#pragma unroll
          for (int tn = 0; tn < 4; ++tn) {
            const int t = 16 * tn + lc;
            const float r = __shfl(r_own, t, WAVE);
            const uint2 gq = *reinterpret_cast<const uint2*>(gsl + 32 * t);
            const uint32_t xw[2] = {ov[tn][0].x, ov[tn][0].y}, gw[2] = {gq.x, gq.y};
            float yv[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const uint32_t xb = xw[e >> 1], gbits = gw[e >> 1];
              const float x = (e & 1) ? __uint_as_float(xb & 0xffff0000u) : __uint_as_float(xb << 16);
              const float g = (e & 1) ? __uint_as_float(gbits & 0xffff0000u) : __uint_as_float(gbits << 16);
              const float v = fmaf(x * r, wv4[e], bv4[e]);
              const float sg = norm_sigmoid(g);
              yv[e] = a.sigmoid_only ? v * sg : v * g * sg;
            }
            if (t < nvc)
              *reinterpret_cast<uint2*>(ob + t * row_bytes) = make_uint2(pack_bf16x2(yv[0], yv[1]), pack_bf16x2(yv[2], yv[3]));
          }
        } else if (nvc == C) {
#pragma unroll
          for (int tn = 0; tn < 4; ++tn)
#pragma unroll
            for (int ct = 0; ct < CTN; ++ct)
              *reinterpret_cast<uint2*>(ob + ((16 * tn + lc) * row_bytes + 32 * ct)) = ov[tn][ct];
        } else {
#pragma unroll
          for (int tn = 0; tn < 4; ++tn)
#pragma unroll
            for (int ct = 0; ct < CTN; ++ct)
              if (16 * tn + lc < nvc) *reinterpret_cast<uint2*>(ob + ((16 * tn + lc) * row_bytes + 32 * ct)) = ov[tn][ct];
        }
      }
      lds_barrier();                                     // B2
      // ---------------- B2 .. B1: state update with chunk c
      if (c >= 0) {
        // S = exp(gc_last) S + k^T (v' exp(gc_last - gc))   (chunk_delta_h.py:163-211)
        const float* vec = reinterpret_cast<const float*>(smem + P::vec_tile(c % 3));
        const float gamma = vec[5 * C];
        Frag<bf16> vg[2][CTN];
        gate_frags<CTN>(Y, vec + 3 * C, vg);
        const uint32_t kbo = P::k_tile(c % 3);
#pragma unroll
        for (int tq = 0; tq < KT; tq += 4) {
          Frag<bf16> kf[4][2];
#pragma unroll
          for (int e = 0; e < 4; ++e) tr4<0, 32 * K, 64 * K, 96 * K>(lo.ktr[tq + e] + kbo, kf[e][0], kf[e][1]);
#pragma unroll
          for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int ct = 0; ct < CTN; ++ct) {
              S[tq + e][ct] *= gamma;
              mma(S[tq + e][ct], kf[e][0], vg[0][ct]);
              mma(S[tq + e][ct], kf[e][1], vg[1][ct]);
            }
        }
      }
      // Aqk of chunk c + 1 (its q and k arrived in the previous step; chunk c's
      // Aqk was last read before B2): tiles wid, wid + NCW, ... (< 10)
      if (c + 1 < sl.nch) {
        const int cn = c + 1;
        const float* vec = reinterpret_cast<const float*>(smem + P::vec_tile(cn % 3));
#pragma unroll
        for (int i = 0; i < (10 + P::NCW - 1) / P::NCW; ++i) {
          const int t = wid + P::NCW * i;
          if (t < 10) aqk_tile_at<K, LDQ>(smem + P::k_tile(cn % 3), smem + P::q_tile(cn & 1), smem + P::off_aqk, lo, vec, t);
        }
      }
      // v, Ai and the vectors of chunk c + 2 (the producers are done
      // with those of chunk c + 1), then the loads of chunk c + 3
      if (c + 2 < sl.nch) {
        cs.store(smem, (c + 2) % 3);
        if (c + 3 < sl.nch) cs.load(SRC(a, t_seg + (int64_t)(c + 3) * C, chunk_nv(c + 3), h, H, rec0 + (c + 3) * rec_step), H);
      }
      lds_barrier();                                     // B1
    }
  } else {
    ProdStage<TQ, K, V> ps;
    const SRC s0(a, t_seg, chunk_nv(0), h, H, rec0);
    ps.load_q(s0, H);
    ps.load_k(s0, H);
    ps.store_q(smem, 0, qs, a.l2 != 0 && !q_cons);
    ps.store_k(smem, 0, ks_, a.l2 != 0);
    if (sl.nch > 1) {
      const SRC s1(a, t_seg + C, chunk_nv(1), h, H, rec0 + rec_step);
      ps.load_q(s1, H);
      ps.load_k(s1, H);
    }
    lds_barrier();
    const int pw = wid - P::NCW;
    OutProducts<K, V> pr;
    // transposed-read lane addresses of this producer's d tiles pw + 4 i
    uint32_t ktr_w[OutProducts<K, V>::NWU];
#pragma unroll
    for (int i = 0; i < OutProducts<K, V>::NWU; ++i) ktr_w[i] = tr_lane_addr<K>(lds0, pw + 4 * i);
    // with the in-op L2 norm of bf16 k, the k rows loaded in one step are normalised in registers in
    // that step's second half (where the producers wait for the consumers' state update), so the
    // first half, which bounds the step, only stores them
    const bool k_pre = a.l2 != 0 && !P::FP8;
    for (int c = -1; c < sl.nch; ++c) {
      // ---------------- B1 .. B2
      // producers: w and u of chunk c + 1; k of chunk c + 2 goes to a buffer
      // free in this half, then the loads of k of chunk c + 3
      if (c + 2 < sl.nch) {
        ps.store_k(smem, (c + 2) % 3, ks_, a.l2 != 0 && !(k_pre && c >= 0));
        if (c + 3 < sl.nch) ps.load_k(SRC(a, t_seg + (int64_t)(c + 3) * C, chunk_nv(c + 3), h, H, rec0), H);
      }
      if (c + 1 < sl.nch) {
      const int cn = c + 1;
      const int kb = cn % 3;
      const float* vec = reinterpret_cast<const float*>(smem + P::vec_tile(cn % 3));
      auto issue = [&](auto) {
        __builtin_amdgcn_sched_barrier(0);               // one product at a time: bounded live registers
      };
      // rows 16 t + lc of Ai (K steps 0, 1; the upper blocks are zero): the
      // operand of both w and u, read once
      Frag<bf16> af[4][2];
      {
        const unsigned char* ai = smem + P::ai_tile;
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int ks = 0; ks < 2; ++ks)
            if (ks <= t / 2) af[t][ks] = frag_at<bf16>(reinterpret_cast<const bf16*>(ai + 32 * t * C + lo.airow[ks]));
      }
      // -w (all token tiles tn, d tile pw + 4 i) = -Ai bf16(bf16(k beta) exp(gc))  (wy_fast.py:67-81)
      auto w_item = [&](auto I) {
        constexpr int i = decltype(I)::value;
        if constexpr (i >= OutProducts<K, V>::NWU) return;
        Frag<bf16> k0, k1;
        tr4<0, 32 * K, 64 * K, 96 * K>(ktr_w[i] + P::k_tile(kb), k0, k1);
        const Frag<bf16> kb0 = kb_frag(k0, vec + 4 * C, vec + 2 * C, 0);
        const Frag<bf16> kb1 = kb_frag(k1, vec + 4 * C, vec + 2 * C, 1);
#pragma unroll
        for (int tn = 0; tn < 4; ++tn) {
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
          mma(acc, kb0, af[tn][0]);
          if (tn >= 2) mma(acc, kb1, af[tn][1]);
          pr.w[i][tn] = make_uint2(pack_bf16x2(-acc[0], -acc[1]), pack_bf16x2(-acc[2], -acc[3]));
        }
      };
      // u (column tile ctu) = Ai bf16(v beta)     (wy_fast.py:55-65)
      auto u_item = [&](auto I) {
        constexpr int i = decltype(I)::value;
        if constexpr (i >= OutProducts<K, V>::NU) return;
        const int ctu = pw + 4 * i;
        if (ctu < V / 16) {
          Frag<bf16> vb0, vb1;
          tr4<0, 32 * V, 64 * V, 96 * V>(tr_lane_addr<V>(lds0, ctu) + P::v_tile, vb0, vb1);
          vb0 = scale_frag(vb0, vec + 4 * C, 0);
          vb1 = scale_frag(vb1, vec + 4 * C, 1);
#pragma unroll
          for (int tm = 0; tm < 4; ++tm) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            mma(acc, af[tm][0], vb0);
            if (tm >= 2) mma(acc, af[tm][1], vb1);
            pr.u[i][tm] = make_uint2(pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3]));
          }
        }
      };
      w_item(std::integral_constant<int, 0>{});
      issue(0);
      w_item(std::integral_constant<int, 1>{});
      issue(0);
      u_item(std::integral_constant<int, 0>{});
      issue(0);
      u_item(std::integral_constant<int, 1>{});
      issue(0);
      }
      if constexpr (kNorm) {
        if (c >= 0) lds_barrier();                       // the consumers' epilogue barrier (row sums in LDS)
      }
      lds_barrier();                                     // B2
      // ---------------- B2 .. B1: w, u of chunk c + 1 and q of chunk c + 2 to LDS
      if (c + 1 < sl.nch) {
#pragma unroll
        for (int i = 0; i < OutProducts<K, V>::NWU; ++i) {
          const int dt = pw + 4 * i;
          unsigned char* wt = smem + P::off_w + lo.w + 2 * (32 * (dt >> 1) + 4 * (dt & 1));
#pragma unroll
          for (int tn = 0; tn < 4; ++tn) *reinterpret_cast<uint2*>(wt + 32 * tn * LDW) = pr.w[i][tn];
        }
#pragma unroll
        for (int i = 0; i < OutProducts<K, V>::NU; ++i) {
          const int ctu = pw + 4 * i;
          if (ctu < V / 16) {
#pragma unroll
            for (int tm = 0; tm < 4; ++tm)
              *reinterpret_cast<uint2*>(smem + P::off_u + 2 * ((16 * ctu + lc) * LDU + 16 * tm + 4 * lg)) = pr.u[i][tm];
          }
        }
      }
      if (c + 2 < sl.nch) {
        ps.store_q(smem, (c + 2) & 1, qs, a.l2 != 0 && !q_cons);
        if (c + 3 < sl.nch) {
          ps.load_q(SRC(a, t_seg + (int64_t)(c + 3) * C, chunk_nv(c + 3), h, H, rec0), H);
          if (k_pre) ps.norm_k();                        // k of chunk c + 3, stored in the next step
        }
      }
      lds_barrier();                                     // B1
    }
  }
  if (consumer && a.ht && sl.j == sl.nseg - 1) {
    float* p = a.ht + ((int64_t)sl.n * H + h) * K * V + 4 * lg * V + vw + lc;
#pragma unroll
    for (int tt = 0; tt < KT; ++tt)
#pragma unroll
      for (int ct = 0; ct < CTN; ++ct)
#pragma unroll
        for (int j = 0; j < 4; ++j) p[(16 * tt + j) * V + 16 * ct] = S[tt][ct][j];
  }
}

// ---------------------------------------------------------------------------
// seg_trans: affine map [M | R] of one segment (all but the last segment of a
// sequence).  seg_trans_fp8_kernel below serves fp8 k on the chunk engine;
// bf16 q/k take the pipelined seg_trans_kernel that follows it.
// ---------------------------------------------------------------------------
struct SegTransArgs {
  const void* k;
  const void* v;
  const float* k_scale;
  const void* Ai;             // [chunks, H] chunk records from seg_prep
  uint16_t* M;                // [NS, H] blocks of K x K bf16 M_hi then M_lo
  float* R;                   // [NS, H] blocks of K x V in accumulator-tile order (see seg_combine)
  int l2;                     // k is raw and the record carries its rstd (the in-op L2 norm)
};

template <typename TQ, int K, int V>
__global__ __launch_bounds__((Eng<TQ, K, V>::NT)) void seg_trans_fp8_kernel(SegTransArgs a, SegGeom G) {
  using E = Eng<TQ, K, V>;
  constexpr int NW = E::NW, NT = E::NT, KT = K / 16, KS = K / 32, CT = 2;
  extern __shared__ __align__(16) unsigned char smem[];

  const int h = blockIdx.y;
  const int H = G.H;
  const SegLoc sl = locate_seg(blockIdx.x, G);
  if (!sl.ok || sl.j == sl.nseg - 1) return;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;
  const float ks_ = a.k_scale ? a.k_scale[h] : 1.f;
  const uint32_t lds0 = lds_addr(smem);
  // column tiles of [M | R] owned by this wave: c = wid + NW ct; c < K/16 are M tiles
  int ctile[CT];
  uint32_t vtr[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    ctile[ct] = wid + NW * ct;
    vtr[ct] = tr_lane_addr<V>(lds0, max(ctile[ct] - KT, 0));
  }

  f32x4 X[KT][CT];
#pragma unroll
  for (int tt = 0; tt < KT; ++tt) {
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
#pragma unroll
      for (int j = 0; j < 4; ++j) X[tt][ct][j] = (16 * tt + 4 * lg + j == 16 * ctile[ct] + lc) ? 1.f : 0.f;
    }
  }
  LaneOffs<K> lo;
  lane_offsets<K, E::LDW, C + 8>(lo, lds0);
  ChunkLoads<TQ, K, V> LD;
  LD.init(H);

  int64_t t0 = sl.bos + sl.c0 * C;
  int nv = (int)min((int64_t)C, sl.eos - t0);
  const unsigned char* rec = reinterpret_cast<const unsigned char*>(a.Ai) +
                             ((sl.cbase + sl.c0) * H + h) * (int64_t)kSegRecordBytes;
  const int64_t rec_step = (int64_t)H * kSegRecordBytes;
  LD.template slots_from<0, 0>(lds0, a.k, a.v, t0, nv, h, H, rec);

  auto step = [&](auto PP, int ci) {
    constexpr int P = decltype(PP)::value;
    wait_loads();
    const int nvc = nv;
    const float* vec = reinterpret_cast<const float*>(smem + E::vec_tile(P));
    if constexpr (E::FP8) {
      lds_barrier();
      convert_fp8<K, NT>(smem + E::kraw(P), reinterpret_cast<bf16*>(smem + E::k_tile(P)), ks_, nvc);
    }
    lds_barrier();                       // barrier 1
    const float gamma = vec[5 * C];      // exp(gc_last)
    const bool more = ci + 1 < sl.nch;
    if (more) {
      t0 += C;
      nv = (int)min((int64_t)C, sl.eos - t0);
      rec += rec_step;
    }
    auto slot = [&](auto SS) {
      if (more) LD.template slot<1 - P, decltype(SS)::value>(lds0, a.k, a.v, t0, nv, h, H, rec);
    };
    auto slots_from = [&](auto SS) {
      if (more) LD.template slots_from<1 - P, decltype(SS)::value>(lds0, a.k, a.v, t0, nv, h, H, rec);
    };
    slot(std::integral_constant<int, 0>{});
    // ---- phase A
    Frag<bf16> xb[KS][CT];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) xb[ks][ct] = acc_frag(X[2 * ks][ct], X[2 * ks + 1][ct]);
    }
    slot(std::integral_constant<int, 1>{});
    for (int u = wid; u < 4 * E::NDG; u += NW) {
      if constexpr (E::NDG == 2) {
        if (u & 1) w_unit<E, K, 1, P>(smem, lo, vec, u >> 1);
        else w_unit<E, K, 0, P>(smem, lo, vec, u >> 1);
      } else {
        w_unit<E, K, 0, P>(smem, lo, vec, u);
      }
    }
    slot(std::integral_constant<int, 2>{});
    slot(std::integral_constant<int, 3>{});
    f32x4 Y[4][CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      f32x4 u4[4] = {};
      if (ctile[ct] >= KT) u_tile<E, V, P>(smem, lo.airow, vtr[ct], vec, u4);
#pragma unroll
      for (int tm = 0; tm < 4; ++tm) Y[tm][ct] = u4[tm];
      if (ct == 0) slot(std::integral_constant<int, 4>{});
    }
    slots_from(std::integral_constant<int, 5>{});
    lds_barrier();                       // barrier 2: w complete
    // ---- phase B
    add_wx<E, K, CT>(smem, lo.w, xb, Y);
    Frag<bf16> yg[2][CT];
    gate_frags<CT>(Y, vec + 3 * C, yg);
    update_state<E, K, CT, P>(lo, yg, gamma, X);
  };
  for (int ci = 0; ci < sl.nch; ci += 2) {
    step(std::integral_constant<int, 0>{}, ci);
    if (ci + 1 < sl.nch) step(std::integral_constant<int, 1>{}, ci + 1);
  }

  const int64_t s = blockIdx.x;
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const int c0 = 16 * ctile[ct];
    if (c0 < K) {
      // M as the bf16 pair (hi, lo = bf16(M - hi)) that seg_combine multiplies in three bf16 products
      bf16* ph = reinterpret_cast<bf16*>(a.M) + (s * H + h) * 2 * K * K + 4 * lg * K + c0 + lc;
      bf16* pl = ph + K * K;
#pragma unroll
      for (int tt = 0; tt < KT; ++tt)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float x = X[tt][ct][j];
          const bf16 hi = (bf16)x;
          ph[(16 * tt + j) * K] = hi;
          pl[(16 * tt + j) * K] = (bf16)(x - (float)hi);
        }
    } else {
      // R in accumulator-tile order: tile (row tile tt, column tile cv) is 64 lanes x 4 floats
      const int cv = (c0 - K) / 16;
      float* pr = a.R + (s * H + h) * K * V + 4 * l;
#pragma unroll
      for (int tt = 0; tt < KT; ++tt) *reinterpret_cast<f32x4*>(pr + (tt * (V / 16) + cv) * 256) = X[tt][ct];
    }
  }
}

// ---------------------------------------------------------------------------
// seg_trans for bf16 q/k: software-pipelined chunk steps, one barrier per chunk
// ---------------------------------------------------------------------------
// Each wave owns two 16-column tiles of [M | R] as in the chunk engine, but the
// state-independent half of a step runs one chunk ahead: in the step of chunk
// c every wave forms its w d tile (all 64 tokens) and its u tiles of chunk
// c + 1 (w into the other of two w tiles, u in registers) between the MFMA of
// chunk c's update,
// so one barrier per chunk publishes w and the inputs of the next chunk, and
// the state chain's MFMA and the w/u work fill each other's latency.  The
// chunk inputs are triple buffered (chunk c: update; c + 1: w, u; c + 2:
// direct loads in flight), and the loads of chunk c + 2 go out in three parts
// (record after the barrier, k after the w.X products, v after the next
// chunk's w and u): a CU accepts direct loads at a limited rate, and one burst
// of all three stalled the issuing waves for over a thousand cycles while
// their SIMD partners idled at the barrier.  The w tile has no padding: its 16-byte chunks are
// swizzled like the input tiles (Tile<K>), so the lane offsets of a K row
// fragment (krow) address it.
template <int K, int V>
struct TransPlan {
  static constexpr int NW = (K + V) / 32, NT = NW * WAVE, CT = 2;
  static constexpr int KT = K / 16, KS = K / 32, NDG = K / 64;
  static constexpr uint32_t KB = C * K * 2, VB = C * V * 2, RB = kSegRecordBytes, AB = C * C * 2;
  static constexpr uint32_t k_tile(int b) { return (uint32_t)b * KB; }
  static constexpr uint32_t v_tile(int b) { return 3 * KB + (uint32_t)b * VB; }
  static constexpr uint32_t ai_tile(int b) { return 3 * KB + 3 * VB + (uint32_t)b * RB; }
  static constexpr uint32_t vec_tile(int b) { return ai_tile(b) + AB; }
  static constexpr uint32_t w_tile(int b) { return 3 * KB + 3 * VB + 3 * RB + (uint32_t)b * KB; }
  static constexpr uint32_t total = w_tile(2);
  static_assert(3 * KB <= 65536, "the k tiles are read transposed with 16-bit offsets from one lane address");
};

// The direct loads of one chunk (k, v, record) into buffer b of a TransPlan.
template <int K, int V>
struct TransLoads {
  using P = TransPlan<K, V>;
  LoadOffs<bf16, K, P::NT> ko;
  LoadOffs<bf16, V, P::NT> vo;
  RecOffs<P::NT> ro;
  __device__ __forceinline__ void init(int H) {
    ko.init((uint32_t)(H * K * 2));
    vo.init((uint32_t)(H * V * 2));
    ro.init();
  }
  // the three parts of a chunk's inputs, issued at separate points of a chunk
  // step so that no wave stalls long on a full load queue
  __device__ __forceinline__ void issue_k(uint32_t lds0, int b, const bf16* kp, int64_t e0, int nv, int H) const {
    if (nv == C)
      ko.issue(kp + e0 * K, lds0 + P::k_tile(b));
    else
      load_tile<bf16, K, P::NT>(kp + e0 * K, (uint32_t)(H * K * 2), nv, lds0 + P::k_tile(b));
  }
  __device__ __forceinline__ void issue_v(uint32_t lds0, int b, const bf16* vp, int64_t e0, int nv, int H) const {
    if (nv == C)
      vo.issue(vp + e0 * V, lds0 + P::v_tile(b));
    else
      load_tile<bf16, V, P::NT>(vp + e0 * V, (uint32_t)(H * V * 2), nv, lds0 + P::v_tile(b));
  }
  __device__ __forceinline__ void issue_rec(uint32_t lds0, int b, const unsigned char* rec) const {
#pragma unroll
    for (int i = 0; i < RecOffs<P::NT>::N; ++i) ro.issue1(i, rec, lds0 + P::ai_tile(b));
  }
};

template <int K, int V>
__global__ __launch_bounds__((TransPlan<K, V>::NT)) void seg_trans_kernel(SegTransArgs a, SegGeom G) {
  using P = TransPlan<K, V>;
  constexpr int KT = P::KT, KS = P::KS, CT = P::CT, NW = P::NW;
  extern __shared__ __align__(16) unsigned char smem[];

  const int h = blockIdx.y;
  const int H = G.H;
  const SegLoc sl = locate_seg(blockIdx.x, G);
  if (!sl.ok || sl.j == sl.nseg - 1) return;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;
  const uint32_t lds0 = lds_addr(smem);
  // column tiles of [M | R] owned by this wave: c = wid + NW ct; c < K/16 are M tiles
  int ctile[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) ctile[ct] = wid + NW * ct;
  // whether tile ct is an R tile (known at compile time when K = V: tile 0 is M, tile 1 is R)
  auto is_r = [&](int ct) { return K == V ? ct == 1 : ctile[ct] >= KT; };

  f32x4 X[KT][CT];
#pragma unroll
  for (int tt = 0; tt < KT; ++tt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int j = 0; j < 4; ++j) X[tt][ct][j] = (16 * tt + 4 * lg + j == 16 * ctile[ct] + lc) ? 1.f : 0.f;
  LaneOffs<K> lo;
  lane_offsets<K, K + 8, C + 8>(lo, lds0);
  TransLoads<K, V> LD;
  LD.init(H);
  const bf16* kp = reinterpret_cast<const bf16*>(a.k);
  const bf16* vp = reinterpret_cast<const bf16*>(a.v);
  const int64_t t_seg = sl.bos + sl.c0 * C;
  const unsigned char* rec0 = reinterpret_cast<const unsigned char*>(a.Ai) +
                              ((sl.cbase + sl.c0) * H + h) * (int64_t)kSegRecordBytes;
  const int64_t rec_step = (int64_t)H * kSegRecordBytes;
  auto chunk_nv = [&](int c) { return (int)min((int64_t)C, sl.eos - (t_seg + (int64_t)c * C)); };
  auto load_k = [&](int c) { LD.issue_k(lds0, c % 3, kp, (t_seg + (int64_t)c * C) * H + h, chunk_nv(c), H); };
  auto load_v = [&](int c) { LD.issue_v(lds0, c % 3, vp, (t_seg + (int64_t)c * C) * H + h, chunk_nv(c), H); };
  auto load_rec = [&](int c) { LD.issue_rec(lds0, c % 3, rec0 + c * rec_step); };
  auto load_chunk = [&](int c) {
    load_k(c);
    load_v(c);
    load_rec(c);
  };

  // d tiles of w formed by this wave: dt = wid + NW r (< KT); the lane
  // addresses of their transposed k reads and of their -w stores
  constexpr int DTW = (KT + NW - 1) / NW;
  uint32_t ktr_w[DTW], wst[DTW];
#pragma unroll
  for (int r = 0; r < DTW; ++r) {
    const int dt = min(wid + NW * r, KT - 1);
    ktr_w[r] = tr_lane_addr<K>(lds0, dt);
    wst[r] = 2 * Tile<K>::off(lc, 4 * (dt >> 1) + lg) + 8 * (dt & 1);
  }

  // -w (d tile dt, all token tiles) and the u tiles of chunk cn (wy_fast.py:55-81):
  // w = Ai bf16(bf16(k beta) exp(gc)) to w_tile(cn % 2), u = Ai bf16(v beta) packed into up
  uint2 up[CT][4];
  auto products = [&](int cn) {
    const int b = cn % 3;
    const float* vec = reinterpret_cast<const float*>(smem + P::vec_tile(b));
    const unsigned char* ai = smem + P::ai_tile(b);
#pragma unroll
    for (int r = 0; r < DTW; ++r) {
      if (KT % NW != 0 && wid + NW * r >= KT) break;   // uniform per wave
      Frag<bf16> k0, k1;
      tr4<0, 32 * K, 64 * K, 96 * K>(ktr_w[r] + P::k_tile(b), k0, k1);
      const float* rk = a.l2 ? vec + 6 * C : nullptr;
      const Frag<bf16> kb0 = kb_frag(k0, vec + 4 * C, vec + 2 * C, 0, rk);
      const Frag<bf16> kb1 = kb_frag(k1, vec + 4 * C, vec + 2 * C, 1, rk);
      unsigned char* wt = smem + P::w_tile(cn & 1) + wst[r];
#pragma unroll
      for (int tn = 0; tn < 4; ++tn) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        mma(acc, kb0, frag_at<bf16>(reinterpret_cast<const bf16*>(ai + 32 * tn * C + lo.airow[0])));
        if (tn >= 2)                                      // Ai is lower triangular
          mma(acc, kb1, frag_at<bf16>(reinterpret_cast<const bf16*>(ai + 32 * tn * C + lo.airow[1])));
        *reinterpret_cast<uint2*>(wt + 32 * tn * K) =
            make_uint2(pack_bf16x2(-acc[0], -acc[1]), pack_bf16x2(-acc[2], -acc[3]));
      }
    }
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      if (is_r(ct)) {
        Frag<bf16> vb0, vb1;
        tr4<0, 32 * V, 64 * V, 96 * V>(tr_lane_addr<V>(lds0, ctile[ct] - KT) + P::v_tile(b), vb0, vb1);
        vb0 = scale_frag(vb0, vec + 4 * C, 0);
        vb1 = scale_frag(vb1, vec + 4 * C, 1);
#pragma unroll
        for (int tm = 0; tm < 4; ++tm) {
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
          mma(acc, frag_at<bf16>(reinterpret_cast<const bf16*>(ai + 32 * tm * C + lo.airow[0])), vb0);
          if (tm >= 2) mma(acc, frag_at<bf16>(reinterpret_cast<const bf16*>(ai + 32 * tm * C + lo.airow[1])), vb1);
          up[ct][tm] = make_uint2(pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3]));
        }
      }
    }
  };

  load_chunk(0);
  if (sl.nch > 1) load_chunk(1);
  wait_loads();
  lds_barrier();
  products(0);
  for (int c = 0; c < sl.nch; ++c) {
    wait_loads();                        // this wave's loads of chunk c + 1
    lds_barrier();                       // w of chunk c and the inputs of chunk c + 1 are complete
    // chunk c + 2 goes to the buffers of chunk c - 1, which every wave has left
    const bool more = c + 2 < sl.nch;
    if (more) load_rec(c + 2);
    const int b = c % 3;
    const float* vec = reinterpret_cast<const float*>(smem + P::vec_tile(b));
    // v' = u + (-w) X
    Frag<bf16> xb[KS][CT];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) xb[ks][ct] = acc_frag(X[2 * ks][ct], X[2 * ks + 1][ct]);
    f32x4 Y[4][CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int tm = 0; tm < 4; ++tm)
        Y[tm][ct] = is_r(ct) ? f32x4{bf16_lo(up[ct][tm].x), bf16_hi(up[ct][tm].x), bf16_lo(up[ct][tm].y),
                                            bf16_hi(up[ct][tm].y)}
                                    : f32x4{0.f, 0.f, 0.f, 0.f};
    {
      const unsigned char* wt = smem + P::w_tile(c & 1);
#pragma unroll
      for (int tm = 0; tm < 4; ++tm)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const Frag<bf16> wa = frag_at<bf16>(reinterpret_cast<const bf16*>(wt + 32 * tm * K + lo.krow[ks]));
#pragma unroll
          for (int ct = 0; ct < CT; ++ct) mma(Y[tm][ct], wa, xb[ks][ct]);
        }
    }
    if (more) load_k(c + 2);
    // the next chunk's w and u, independent of the state chain (in the same
    // basic block, so that the two interleave; after the last chunk they are
    // formed from stale buffers and never used)
    products(c + 1);
    if (more) load_v(c + 2);
    // X = exp(gc_last) X + k^T (v' gate)
    const float gamma = vec[5 * C];
    Frag<bf16> vg[2][CT];
    // with the in-op L2 norm the update reads raw k: its rstd rides on the gated v' (gate * rstd,
    // one rounding per element, as the gated v' itself has)
    gate_frags<CT>(Y, vec + (a.l2 ? 7 : 3) * C, vg);
    const uint32_t kbo = P::k_tile(b);
#pragma unroll
    for (int tq = 0; tq < KT; tq += 4) {
      Frag<bf16> kf[4][2];
#pragma unroll
      for (int e = 0; e < 4; ++e) tr4<0, 32 * K, 64 * K, 96 * K>(lo.ktr[tq + e] + kbo, kf[e][0], kf[e][1]);
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          X[tq + e][ct] *= gamma;
          mma(X[tq + e][ct], kf[e][0], vg[0][ct]);
          mma(X[tq + e][ct], kf[e][1], vg[1][ct]);
        }
    }
  }

  const int64_t s = blockIdx.x;
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const int c0 = 16 * ctile[ct];
    if (c0 < K) {
      // M as the bf16 pair (hi, lo = bf16(M - hi)) that seg_combine multiplies in three bf16 products
      bf16* ph = reinterpret_cast<bf16*>(a.M) + (s * H + h) * 2 * K * K + 4 * lg * K + c0 + lc;
      bf16* pl = ph + K * K;
#pragma unroll
      for (int tt = 0; tt < KT; ++tt)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float x = X[tt][ct][j];
          const bf16 hi = (bf16)x;
          ph[(16 * tt + j) * K] = hi;
          pl[(16 * tt + j) * K] = (bf16)(x - (float)hi);
        }
    } else {
      // R in accumulator-tile order: tile (row tile tt, column tile cv) is 64 lanes x 4 floats
      const int cv = (c0 - K) / 16;
      float* pr = a.R + (s * H + h) * K * V + 4 * l;
#pragma unroll
      for (int tt = 0; tt < KT; ++tt) *reinterpret_cast<f32x4*>(pr + (tt * (V / 16) + cv) * 256) = X[tt][ct];
    }
  }
}

// ---------------------------------------------------------------------------
// seg_combine: S_{j+1} = M_j S_j + R_j over the segments of a sequence, 16 V
// columns per workgroup.  Also writes final_state of sequences without tokens.
//
// The chain is serial, so each step must cost only its arithmetic.  M_j and
// S_j enter as bf16 pairs (x = hi + lo, lo = bf16(x - hi), 16 significant bits)
// and M_j S_j as hi.hi + hi.lo + lo.hi on v_mfma_f32_16x16x32_bf16 with fp32
// accumulation onto R_j: the dropped lo.lo term and the split leave a relative
// error near 2^-17, far below the bf16 rounding of the state snapshot that
// seg_out applies.  Wave w owns output rows 16w .. 16w + 15 and holds its rows
// of M_j (A operand) and its tile of R_j in registers, loaded three steps
// ahead; the state columns (B operand, shared by all waves) sit transposed in
// LDS, double buffered so that one barrier per step suffices.
// ---------------------------------------------------------------------------
struct SegCombineArgs {
  const uint16_t* M;          // [NS, H] blocks of K x K bf16 M_hi then M_lo
  const float* R;             // [NS, H] blocks of K x V: 16x16 tile (rt, ct) at 256 (rt V/16 + ct), lane l's
                              // elements (rows 16 rt + 4 (l/16) + jj, column 16 ct + l%16) at 4 l + jj
  const void* h0;
  int h0_dtype;
  float* s_init;              // out [NS, H, K, V]
  float* ht;                  // final_state, written here only for empty sequences
  int V;
};

template <int K>
struct CombineMaps {
  Frag<bf16> mh[K / 32];      // M_hi[r0 + lane%16][32 kb + 8 (lane/16) .. +7]
  Frag<bf16> ml[K / 32];      // M_lo, same positions
  f32x4 r;                    // R_j[r0 + 4 (lane/16) + jj][v0 + lane%16]
};

template <int K>
__device__ __forceinline__ void load_maps(CombineMaps<K>& c, const bf16* M, const float* R, int V, int r0, int v0) {
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;
  const bf16* pm = M + (int64_t)(r0 + lc) * K + 8 * lg;
#pragma unroll
  for (int kb = 0; kb < K / 32; ++kb) {
    c.mh[kb].v = *reinterpret_cast<const bf16x8*>(pm + 32 * kb);
    c.ml[kb].v = *reinterpret_cast<const bf16x8*>(pm + K * K + 32 * kb);
  }
  c.r = *reinterpret_cast<const f32x4*>(R + ((r0 / 16) * (V / 16) + v0 / 16) * 256 + 4 * l);
}

template <int K> struct CombCfg {
  static constexpr int NT = K / 16 * WAVE;                  // one 16-row tile per wave
  static constexpr int LDS_T = K + 8;                       // row stride (bf16) of a transposed state half
};

// f(integral_constant<int, I>, j0 + I) for I = I0 .. N - 1, unrolled
template <int I, int N, typename F>
__device__ __forceinline__ void unroll_steps(F& f, int j0) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{}, j0 + I);
    unroll_steps<I + 1, N>(f, j0);
  }
}
// the same for the first `rem` of them, each nested in the branch of the one before
template <int I, int N, typename F>
__device__ __forceinline__ void unroll_steps_upto(F& f, int j0, int rem) {
  if constexpr (I < N) {
    if (rem > I) {
      f(std::integral_constant<int, I>{}, j0 + I);
      unroll_steps_upto<I + 1, N>(f, j0, rem);
    }
  }
}

template <int K>
__global__ __launch_bounds__(CombCfg<K>::NT) void seg_combine_kernel(SegCombineArgs a, SegGeom G, int total) {
  constexpr int NT = CombCfg<K>::NT;
  constexpr int LDS_T = CombCfg<K>::LDS_T;
  // s_S[buf][half][c][r]: half 0 = bf16 hi, 1 = bf16 lo of S[r][v0 + c]
  __shared__ __align__(16) bf16 s_S[2][2][16][LDS_T];
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
  // Maps of steps j .. j + NST - 1 in flight (stage j % NST).  Every stage is
  // loaded unconditionally (past the last step: the last step's maps again) so
  // that the number of loads issued after each stage is fixed and the wait for
  // a stage counts only the loads before it.  Three stages measured best (28 us
  // at config 2 against 30 with four and 36 with five): the step is bound by the
  // rate at which a CU takes in its 72 KB of maps, not by their latency.
  constexpr int NST = 3;
  const int nsteps = nseg - 1;
  const bf16* Mb = reinterpret_cast<const bf16*>(a.M);
  CombineMaps<K> st[NST];
  auto issue = [&](CombineMaps<K>& c, int j) {
    const int64_t s = s_first + max(0, min(j, nsteps - 1));
    load_maps<K>(c, Mb + (s * H + h) * 2 * K * K, a.R + (s * H + h) * K * V, V, r0, v0);
  };
  if (nseg == 0) {
    if (a.ht) {
      for (int idx = threadIdx.x; idx < K * 16; idx += NT) {
        const int r = idx / 16, c = idx % 16;
        const int64_t off = (((int64_t)n * H + h) * K + r) * V + v0 + c;
        float x = 0.f;
        if (a.h0)
          x = a.h0_dtype == DT_F32 ? reinterpret_cast<const float*>(a.h0)[off]
                                   : (float)reinterpret_cast<const bf16*>(a.h0)[off];
        a.ht[off] = x;
      }
    }
    return;
  }
  // one segment: its initial state is h0, which seg_out reads itself
  if (nsteps <= 0) return;
  // S_0 = h0: its loads go out before the maps', so that waiting for them does
  // not wait for the maps
  float x0[K * 16 / NT];
#pragma unroll
  for (int e = 0; e < K * 16 / NT; ++e) {
    const int idx = threadIdx.x + NT * e;
    const int r = idx / 16, c = idx % 16;
    x0[e] = 0.f;
    if (a.h0) {
      const int64_t off = (((int64_t)n * H + h) * K + r) * V + v0 + c;
      x0[e] = a.h0_dtype == DT_F32 ? reinterpret_cast<const float*>(a.h0)[off]
                                   : (float)reinterpret_cast<const bf16*>(a.h0)[off];
    }
  }
#pragma unroll
  for (int u = 0; u < NST; ++u) issue(st[u], u);
#pragma unroll
  for (int e = 0; e < K * 16 / NT; ++e) {
    const int idx = threadIdx.x + NT * e;
    const int r = idx / 16, c = idx % 16;
    const bf16 hi = (bf16)x0[e];
    s_S[0][0][c][r] = hi;
    s_S[0][1][c][r] = (bf16)(x0[e] - (float)hi);
  }
  __syncthreads();
  // One step of the chain: U2 (a compile-time count) picks the map stage (U2 % NST) and the state
  // buffer (j % 2 = U2 % 2)
  auto step = [&](auto U2, int j) {
    constexpr int u = decltype(U2)::value % NST, b = decltype(U2)::value & 1;
    Frag<bf16> sh[K / 32], sl[K / 32];
#pragma unroll
    for (int kb = 0; kb < K / 32; ++kb) {
      sh[kb].v = *reinterpret_cast<const bf16x8*>(&s_S[b][0][lc][32 * kb + 8 * lg]);
      sl[kb].v = *reinterpret_cast<const bf16x8*>(&s_S[b][1][lc][32 * kb + 8 * lg]);
    }
    f32x4 acc = st[u].r, acc2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < K / 32; ++kb) {
      mma(acc2, st[u].ml[kb], sh[kb]);
      mma(acc2, st[u].mh[kb], sl[kb]);
      mma(acc, st[u].mh[kb], sh[kb]);
    }
    acc += acc2;
    issue(st[u], j + NST);                                  // this stage's registers are free again
    // S_{j+1}: rows r0 + 4 lg + jj, column lc -> the other buffer, and s_init
    uint32_t ph[2], pl[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const bf16 h0_ = (bf16)acc[2 * q], h1_ = (bf16)acc[2 * q + 1];
      ph[q] = (uint32_t)__builtin_bit_cast(uint16_t, h0_) | ((uint32_t)__builtin_bit_cast(uint16_t, h1_) << 16);
      const bf16 l0_ = (bf16)(acc[2 * q] - (float)h0_), l1_ = (bf16)(acc[2 * q + 1] - (float)h1_);
      pl[q] = (uint32_t)__builtin_bit_cast(uint16_t, l0_) | ((uint32_t)__builtin_bit_cast(uint16_t, l1_) << 16);
    }
    *reinterpret_cast<uint2*>(&s_S[b ^ 1][0][lc][r0 + 4 * lg]) = make_uint2(ph[0], ph[1]);
    *reinterpret_cast<uint2*>(&s_S[b ^ 1][1][lc][r0 + 4 * lg]) = make_uint2(pl[0], pl[1]);
    float* out = a.s_init + ((s_first + j + 1) * (int64_t)H + h) * K * V + (int64_t)(r0 + 4 * lg) * V + v0 + lc;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) out[(int64_t)jj * V] = acc[jj];
    lds_barrier();                                          // LDS only: the maps' prefetch stays in flight
  };
  // Whole rounds of RL steps (RL a multiple of NST and of 2: the stage and the state buffer repeat),
  // then the rest in nested branches.  Nothing leaves a round from inside: the compiler counts the
  // loads in flight at each wait over every path that reaches it, and an exit inside an unrolled
  // round also reached the loop header, so every step waited for the maps issued one step before
  // instead of NST steps before.
  constexpr int RL = NST % 2 ? 2 * NST : NST;
  int j0 = 0;
  for (; j0 + RL <= nsteps; j0 += RL) unroll_steps<0, RL>(step, j0);
  unroll_steps_upto<0, RL - 1>(step, j0, nsteps - j0);       // uniform remainder, 0 .. RL - 1 steps
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

// ---------------------------------------------------------------------------
// Segments as sequences (the backward's recomputation and its dh recurrence run
// the stage kernels over segments, each from the state the scan gives it)
// ---------------------------------------------------------------------------
// seg_cu[s] / seg_coff[s]: first token / first global chunk of segment s (slots past
// the last segment: empty), seg_cu[ns] / seg_coff[ns]: the totals.
__global__ void seg_seq_map_kernel(SegGeom G, int ns_grid, int64_t* __restrict__ seg_cu,
                                   int32_t* __restrict__ seg_coff) {
  const int64_t end_tok = G.cu ? G.cu[G.N] : (int64_t)G.N * G.T;
  const int64_t end_ch = G.cu ? (int64_t)G.chunk_off[G.N] : (int64_t)G.N * ((G.T + C - 1) / C);
  for (int s = blockIdx.x * blockDim.x + threadIdx.x; s <= ns_grid; s += gridDim.x * blockDim.x) {
    const SegLoc sl = s < ns_grid ? locate_seg(s, G) : SegLoc{};
    if (s < ns_grid && sl.ok) {
      seg_cu[s] = sl.bos + sl.c0 * C;
      seg_coff[s] = (int32_t)(sl.cbase + sl.c0);
    } else {
      seg_cu[s] = end_tok;
      seg_coff[s] = (int32_t)end_ch;
    }
  }
}

// dst[s] = src[n] for the first (first_seg) or the last segment of each sequence n, zeros for the
// other segments: [ns, H, K * V] fp32 from [N, H, K * V] (src: h0_dtype, or nullptr = zeros).
// With first_seg the other segments are left alone (seg_combine writes them).  blockIdx.z splits
// each K * V state into gridDim.z slices (a (segment, head) grid alone is too few workgroups).
__global__ __launch_bounds__(256) void seg_place_kernel(SegGeom G, const void* src, int src_dtype, float* dst,
                                                        int KV, int first_seg) {
  const int s = blockIdx.x, h = blockIdx.y, H = G.H;
  const SegLoc sl = locate_seg(s, G);
  if (!sl.ok) return;
  const bool pick = first_seg ? sl.j == 0 : sl.j == sl.nseg - 1;
  if (first_seg && !pick) return;
  float* d = dst + ((int64_t)s * H + h) * KV;
  const int64_t so = ((int64_t)sl.n * H + h) * KV;
  const int span = (KV / 4 + gridDim.z - 1) / gridDim.z * 4, i0 = span * blockIdx.z, i1 = min(KV, i0 + span);
  for (int i = i0 + 4 * threadIdx.x; i < i1; i += 4 * blockDim.x) {   // KV and span are multiples of 4
    f32x4 x = {0.f, 0.f, 0.f, 0.f};
    if (pick && src) {
      if (src_dtype == DT_F32) {
        x = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(src) + so + i);
      } else {
        const uint2 r = *reinterpret_cast<const uint2*>(reinterpret_cast<const bf16*>(src) + so + i);
        x = f32x4{bf16_lo(r.x), bf16_hi(r.x), bf16_lo(r.y), bf16_hi(r.y)};
      }
    }
    *reinterpret_cast<f32x4*>(d + i) = x;
  }
}

// Reverse scan of the dh recurrence over the segments of a sequence, one workgroup per
// (sequence, head), V / 16 waves each owning 16 value columns over all K rows (fp32
// accumulator tiles in VGPRs).  Across segment j the state gradient maps as
// dh_start(j) = M_j^T dh_start(j + 1) + B_j, with M_j the forward's segment map (seg_trans, a
// bf16 pair hi + lo) and B_j the dh recurrence of segment j run from zero.  The last segment
// has no map (seg_trans skips it): its Bseg entry is its recurrence from dht, which is
// dh_start(last) itself.  Writes F_j = dh_start(j + 1) (F_last = dht), the state each segment's
// final pass starts from, and dh0 = dh_start(0) (when dh0 is not null).  M_j^T X runs on the
// bf16 MFMA as hi hi + hi lo + lo hi (x = hi + lo on both sides, fp32 accumulation): M_j is
// staged in LDS as K / 64 tiles of [64 rows][K] and read transposed; X's accumulator tiles are
// the B operand.  The next step's map is loaded into registers while the current one computes.
// S: workgroups per (sequence, head), each on V / S of the value columns (each stages the whole map)
template <int K, int V, int S>
struct RCfg {
  static constexpr int NW = V / 16 / S, NT = NW * WAVE;
  static constexpr int KT = K / 16, KS = K / 32;
  static constexpr int EM = K * K;                       // elements of one bf16 half of a map
  static constexpr int UM = 2 * EM / 8 / NT;             // 16-byte units of (hi, lo) per thread
  static_assert(2 * EM % (8 * NT) == 0, "units split evenly over the threads");
  static constexpr size_t lds = (size_t)2 * EM * 2;
};

// offset of element (r, c) of a [K][K] map staged as K / 64 tiles of 64 rows (toff layout)
template <int K>
__device__ __forceinline__ int moff(int r, int c) { return (r >> 6) * 64 * K + toff<bf16>(r & 63, c, K); }

template <int K, int V, int S>
__global__ __launch_bounds__((RCfg<K, V, S>::NT)) void seg_bwd_combine_kernel(SegGeom G, const bf16* __restrict__ M,
                                                                          const float* __restrict__ Bseg,
                                                                          const float* __restrict__ dht,
                                                                          float* __restrict__ F,
                                                                          float* __restrict__ dh0, int total) {
  using RC = RCfg<K, V, S>;
  constexpr int KT = RC::KT, KS = RC::KS;
  extern __shared__ __align__(16) unsigned char smem[];
  bf16* s_mh = reinterpret_cast<bf16*>(smem);
  bf16* s_ml = s_mh + RC::EM;
  const int per_xcd = gridDim.x / 8;
  const int o_idx = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (o_idx >= total) return;
  const int unit = o_idx / S, slice = o_idx % S;       // the slices of a head are neighbours on one XCD
  const int H = G.H, n = unit / H, h = unit % H;
  const int tid = threadIdx.x, wid = tid / WAVE, l = lane_id(), lg = l >> 4, lc = l & 15;
  const int col = 16 * (wid + RC::NW * slice) + lc;
  int nseg, s_first;
  if (G.cu == nullptr) {
    nseg = G.T > 0 ? G.nseg_fixed : 0;
    s_first = n * G.nseg_fixed;
  } else {
    nseg = G.seg_off[n + 1] - G.seg_off[n];
    s_first = G.seg_off[n];
  }
  const int64_t KV = (int64_t)K * V;
  // lane element (tt, j): row 16 tt + 4 lg + j, column col
  auto blk = [&](int64_t b) { return b * KV + (int64_t)(4 * lg) * V + col; };
  f32x4 X[KT];
  const int64_t dn = ((int64_t)n * H + h);
#pragma unroll
  for (int tt = 0; tt < KT; ++tt)
#pragma unroll
    for (int j = 0; j < 4; ++j) X[tt][j] = dht ? dht[blk(dn) + (16 * tt + j) * V] : 0.f;
  if (nseg > 0) {
    const int64_t last = (int64_t)(s_first + nseg - 1) * H + h;
#pragma unroll
    for (int tt = 0; tt < KT; ++tt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        F[blk(last) + (16 * tt + j) * V] = X[tt][j];
        X[tt][j] = Bseg[blk(last) + (16 * tt + j) * V];
      }
  }
  // maps of step j (hi then lo, row-major) as 16-byte units tid + NT i
  u32x4 mcur[RC::UM], mnxt[RC::UM];
  f32x4 bcur[KT], bnxt[KT];
  auto load = [&](int j, u32x4 (&m)[RC::UM], f32x4 (&b)[KT]) {
    const int64_t sj = (int64_t)(s_first + j) * H + h;
    const u32x4* src = reinterpret_cast<const u32x4*>(M + sj * 2 * K * K);
#pragma unroll
    for (int i = 0; i < RC::UM; ++i) m[i] = src[tid + RC::NT * i];
#pragma unroll
    for (int tt = 0; tt < KT; ++tt)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) b[tt][jj] = Bseg[blk(sj) + (16 * tt + jj) * V];
  };
  if (nseg >= 2) load(nseg - 2, mcur, bcur);
  for (int j = nseg - 2; j >= 0; --j) {
    const int64_t sj = (int64_t)(s_first + j) * H + h;
#pragma unroll
    for (int tt = 0; tt < KT; ++tt)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) F[blk(sj) + (16 * tt + jj) * V] = X[tt][jj];
#pragma unroll
    for (int i = 0; i < RC::UM; ++i) {
      const int e = 8 * (tid + RC::NT * i);              // element of [hi | lo]
      const int half = e / RC::EM, r = (e % RC::EM) / K, c = e % K;
      *reinterpret_cast<u32x4*>((half ? s_ml : s_mh) + moff<K>(r, c)) = mcur[i];
    }
    lds_barrier();
    if (j > 0) load(j - 1, mnxt, bnxt);
    // X = M_j^T X + B_j: A[a][b] = M[b][a] read transposed (rows b in the accumulator order)
    Frag<bf16> xh[KS], xl[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      float v8[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v8[e] = X[2 * ks][e];
        v8[4 + e] = X[2 * ks + 1][e];
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const bf16 hi = (bf16)v8[e];
        xh[ks].v[e] = hi;
        xl[ks].v[e] = (bf16)(v8[e] - (float)hi);
      }
    }
#pragma unroll
    for (int rt = 0; rt < KT; ++rt) {
      f32x4 acc = bcur[rt], acc2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int tb = (32 * ks) >> 6, k0 = (32 * ks) & 63;
        const Frag<bf16> ah = tr_frag<64>(s_mh + tb * 64 * K + (16 * rt >> 6) * 4096, k0 >> 5, (16 * rt) & 63);
        const Frag<bf16> al = tr_frag<64>(s_ml + tb * 64 * K + (16 * rt >> 6) * 4096, k0 >> 5, (16 * rt) & 63);
        mma(acc, ah, xh[ks]);
        mma(acc2, ah, xl[ks]);
        mma(acc2, al, xh[ks]);
      }
      X[rt] = acc + acc2;
    }
    lds_barrier();                                      // the map is restaged next step
#pragma unroll
    for (int i = 0; i < RC::UM; ++i) mcur[i] = mnxt[i];
#pragma unroll
    for (int tt = 0; tt < KT; ++tt) bcur[tt] = bnxt[tt];
  }
  if (dh0) {
#pragma unroll
    for (int tt = 0; tt < KT; ++tt)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) dh0[blk(dn) + (16 * tt + jj) * V] = X[tt][jj];
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
  const void* Ai = p.Ai;
  auto mark = [&](int i) { return p.events == nullptr || hipEventRecord(p.events[i], s) == hipSuccess; };
  if (!mark(0)) return -1;
  if (p.ns_grid > 0 && p.nc_grid > 0) {
    constexpr size_t lds = PrepLds::total;
    static_assert(lds <= 64 * 1024, "seg_prep tiles exceed the default LDS limit");
    SegPrepArgs pa{p.k, p.g, p.beta, p.k_scale, p.g_dtype, p.beta_dtype, p.scale, static_cast<unsigned char*>(p.Ai),
                   p.l2 ? 1 : 0};
    const dim3 pgrid((unsigned)((p.nc_grid * p.H + PrepLds::WAVES - 1) / PrepLds::WAVES));
    const dim3 pblock(PrepLds::WAVES * WAVE);
    if (p.cu != nullptr)
      hipLaunchKernelGGL((seg_prep_kernel<TQ, K, true>), pgrid, pblock, lds, s, pa, G);
    else
      hipLaunchKernelGGL((seg_prep_kernel<TQ, K, false>), pgrid, pblock, lds, s, pa, G);
    if (hipGetLastError() != hipSuccess) return -1;
  }
  if (!mark(1)) return -1;
  if (p.run_trans) {
    constexpr size_t lds = Eng<TQ, K, V>::total;
    SegTransArgs ta{p.k, p.v, p.k_scale, Ai, p.M, p.R, p.l2 ? 1 : 0};
    if constexpr (sizeof(TQ) == 2) {
      constexpr size_t lds_p = TransPlan<K, V>::total;
      auto kt = seg_trans_kernel<K, V>;
      if (set_lds(kt, lds_p)) return -1;
      hipLaunchKernelGGL(kt, grid, dim3(TransPlan<K, V>::NT), lds_p, s, ta, G);
    } else {
      auto kt = seg_trans_fp8_kernel<TQ, K, V>;
      if (set_lds(kt, lds)) return -1;
      hipLaunchKernelGGL(kt, grid, dim3(Eng<TQ, K, V>::NT), lds, s, ta, G);
    }
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
  if (p.ns_grid > 0 && !p.skip_out) {
    SegOutArgs oa{p.q, p.k, p.v, p.q_scale, p.k_scale,
                  p.h0, p.h0_dtype, p.s_init, Ai, p.scale, p.o, p.ht, p.l2 ? 1 : 0,
                  reinterpret_cast<const bf16*>(p.gate), p.nw, p.nb, p.nw_dtype, p.eps, p.sigmoid_only};
    if (p.gate) {
      constexpr size_t lds = OutPlan<TQ, K, V>::total_norm;
      static_assert(lds <= 160 * 1024, "the epilogue's sums must fit beside the output tiles");
      auto ko = seg_out_kernel<TQ, K, V, true>;
      if (set_lds(ko, lds)) return -1;
      hipLaunchKernelGGL(ko, grid, dim3(OutPlan<TQ, K, V>::NT), lds, s, oa, G);
    } else {
      constexpr size_t lds = OutPlan<TQ, K, V>::total;
      auto ko = seg_out_kernel<TQ, K, V, false>;
      if (set_lds(ko, lds)) return -1;
      hipLaunchKernelGGL(ko, grid, dim3(OutPlan<TQ, K, V>::NT), lds, s, oa, G);
    }
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

int launch_seg_seq_map(const SegFwdArgs& p, int64_t* seg_cu, int32_t* seg_coff, hipStream_t s) {
  const SegGeom G{p.cu, p.chunk_off, p.seg_off, p.N, p.T, p.H, p.L, p.nseg_fixed};
  const int ns = (int)p.ns_grid;
  hipLaunchKernelGGL(seg_seq_map_kernel, dim3((unsigned)((ns + 1 + 255) / 256)), dim3(256), 0, s, G, ns, seg_cu,
                     seg_coff);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_seg_place(const SegFwdArgs& p, const void* src, int src_dtype, float* dst, int K, int V, bool first_seg,
                     hipStream_t s) {
  const SegGeom G{p.cu, p.chunk_off, p.seg_off, p.N, p.T, p.H, p.L, p.nseg_fixed};
  if (p.ns_grid <= 0) return 0;
  hipLaunchKernelGGL(seg_place_kernel, dim3((unsigned)p.ns_grid, (unsigned)p.H, 8u), dim3(256), 0, s, G, src,
                     src_dtype, dst, K * V, first_seg ? 1 : 0);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_seg_bwd_combine(const SegFwdArgs& p, const float* Bseg, const float* dht, float* F, float* dh0, int K,
                           int V, hipStream_t s) {
  const SegGeom G{p.cu, p.chunk_off, p.seg_off, p.N, p.T, p.H, p.L, p.nseg_fixed};
  if (p.N * p.H <= 0) return 0;
  const bf16* M = reinterpret_cast<const bf16*>(p.M);
  // V = 128: two workgroups per (sequence, head) of four waves (each reads the transposed map once
  // per step instead of eight waves on one CU); fewer threads would hold more of the map each
#define KGDN_RC(KK, VV, SS)                                                                                 \
  if (K == KK && V == VV) {                                                                                 \
    using RC = RCfg<KK, VV, SS>;                                                                            \
    constexpr int nt = RC::NT;                                                                              \
    constexpr size_t lds = RC::lds;                                                                         \
    const int total = p.N * p.H * SS;                                                                       \
    const int grid = (total + 7) / 8 * 8;                                                                   \
    if (set_lds(seg_bwd_combine_kernel<KK, VV, SS>, lds)) return -1;                                        \
    hipLaunchKernelGGL((seg_bwd_combine_kernel<KK, VV, SS>), dim3(grid), dim3(nt), lds, s, G, M, Bseg, dht, F, \
                       dh0, total);                                                                         \
    return hipGetLastError() == hipSuccess ? 0 : -1;                                                        \
  }
  KGDN_RC(64, 64, 1) KGDN_RC(64, 128, 2) KGDN_RC(128, 64, 1) KGDN_RC(128, 128, 2)
#undef KGDN_RC
  return -2;
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
