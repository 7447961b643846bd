// Fused state recurrence + output for K = 256 (the Kairos model's head dim), bf16 compute
// (fla ops/common/chunk_delta_h.py:52-224 followed by ops/common/chunk_o.py:41-128, with
// the state never leaving the workgroup).  The stage path stores a bf16 state snapshot per
// chunk (256 x V) for the output kernel to read back; at V = 512 that is 2.7 GB written and
// read per call.  Here one workgroup per (sequence, head, 64 value columns) walks the
// chunks, each of its four waves owning 16 state columns over all 256 rows (fp32, MFMA
// accumulator layout, in VGPRs), and per chunk computes
//
//   u      = bf16(Ai bf16(beta v))                                wy_fast.py:55-81
//   h      = bf16(S)                                              chunk_delta_h.py:129-139
//   v'     = u - w h                                              :141-157
//   o^T    = (h^T q^T exp(gc) + bf16(v')^T Aqk^T) scale           chunk_o.py:84-128
//   S      = exp(g_last) S + k^T (v' exp(g_last - gc))            chunk_delta_h.py:163-211
//
// with the same cast points as the stage kernels (u, h and v' rounded to bf16 where the reference
// stores them, Aqk rounded before its product).  Ai, Aqk = mask_{i>=j}(q k^T exp(gc_i - gc_j)) and
// k^T per chunk are state-independent and shared by the V tiles of a head: the prepare kernel forms
// them per (chunk, head) beforehand, so the serial loop only reads them.
//
// Operand order.  Every MFMA operand here is read as one 16-byte row piece (ds_read_b128): for a
// 32-deep K step ks, lane group lg = lane / 16 holds K indices 32 ks + 8 lg .. + 7 ("contiguous K
// order").  Operands made from accumulator tiles (bf16(S) for w h and h^T q^T, v' for the output and
// the update) come from a pair of tiles, so those tiles keep their rows in the paired order: tile
// 2 p + x holds, in lane group lg, element j, row 32 p + 8 lg + 4 x + j.  The A operand that produces
// such a tile reads row rowA(x, lc) = 32 p + 4 x + 8 (lc / 4) + lc % 4 in lane lc.  One wave's LDS
// reads run at about 100 B / clock per CU as b128 against about 65 as b64, and with one wave per
// SIMD the serial loop is bound by them.
//
// LDS tiles, each with a swizzle of 16-byte chunks that keeps the reads conflict-free:
//   w, q    [64 t][256]  chunk c of row r at c ^ (r % 4 + 4 ((r / 8) % 4))
//   k^T     [256 d][64]  chunk c of row r at c ^ (2 ((r / 8) % 4) + (r / 2) % 2)
//   Ai, Aqk [64][64]     as k^T
//   v       [64 t][64]   chunk c of row r at c ^ (2 ((r / 8) % 2) + 4 ((r / 2) % 2)), read transposed
//   o       [64 t][64]   chunk c of row r at c ^ ((r / 2) % 2 + 2 ((r / 8) % 4))
// A b128 LDS read serves 16 lanes per pass on gfx950, grouped by lane bit 5 and the parity of lane
// bits 2-4 (measured with the bank-conflict counter on probe patterns); for the rows rowA the swizzles
// above give each such group 16 distinct 16-byte bank positions (w, q: position lg ^ lc; the 128-byte
// rows: 8 (lc % 2) + (lg ^ lc / 2)), and they do not change under the tiles' row offsets 4 x + 32 p.
// o is computed transposed, so each lane stores 4 consecutive columns of one token.
#include <type_traits>

#include <cstdlib>

#include "gdn_common.hpp"
#include "gdn_conv.hpp"
#include "gdn_kernels.h"

namespace kgdn {

namespace {

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int FK = 256;           // K
constexpr int FW = 4;             // waves per workgroup, 16 state columns each
constexpr int FVT = 16 * FW;      // value columns per workgroup
constexpr int NT_F = FW * WAVE;
constexpr int FL = 4;             // loader waves (direct loads only)

// Workgroup barrier on LDS only (lgkmcnt(0), s_barrier): the next chunk's global loads and this
// chunk's o stores stay in flight across it.
__device__ __forceinline__ void f_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);          // lgkmcnt(0); vmcnt, expcnt at their maxima
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ Frag<bf16> pack_acc(const f32x4& a, const f32x4& b) {
  bf16x8 v = {(bf16)a[0], (bf16)a[1], (bf16)a[2], (bf16)a[3], (bf16)b[0], (bf16)b[1], (bf16)b[2], (bf16)b[3]};
  Frag<bf16> f;
  f.v = v;
  return f;
}

// ---------------------------------------------------------------------------
// direct global -> LDS loads and LDS reads
// ---------------------------------------------------------------------------
// Direct loads (inline asm: the compiler does not track them, so the kernel waits for them
// explicitly before the barrier that publishes their data).  Lane l's 16 (4) bytes at base + off
// land at LDS address m0 + 16 l (4 l); base is wave-uniform.  s_nop 4: the hazard between the
// SGPR / M0 writes and the load that reads them.
__device__ __forceinline__ const void* wave_ptr(const void* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<const void*>(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ void dma16_(const void* base, uint32_t off, uint32_t lds_dst) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(off), "s"(wave_ptr(base)),
               "{m0}"(__builtin_amdgcn_readfirstlane(lds_dst)) : "memory");
}
__device__ __forceinline__ void dma4_(const void* base, uint32_t off, uint32_t lds_dst) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dword %0, %1" : : "v"(off), "s"(wave_ptr(base)),
               "{m0}"(__builtin_amdgcn_readfirstlane(lds_dst)) : "memory");
}
// vmcnt(0) through the builtin, so the compiler's own wait tracking sees every load complete
__device__ __forceinline__ void wait_all_loads() {
  __builtin_amdgcn_s_waitcnt(0x0F70);
  asm volatile("" ::: "memory");
}
// vmcnt(N): all but the wave's last N vector memory operations complete (they complete in issue
// order); expcnt and lgkmcnt at their maxima
template <int N>
__device__ __forceinline__ void wait_loads_but() {
  static_assert(N >= 0 && N < 64, "vmcnt holds 6 bits");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
  asm volatile("" ::: "memory");
}
// the same for a count known only at run time (wave-uniform, 4 .. 24; larger counts wait for 24)
__device__ __forceinline__ void wait_loads_but_n(int n) {
  switch (n) {
#define KGDN_WAIT_CASE(N) \
    case N: wait_loads_but<N>(); break;
    KGDN_WAIT_CASE(4) KGDN_WAIT_CASE(5) KGDN_WAIT_CASE(6) KGDN_WAIT_CASE(7) KGDN_WAIT_CASE(8) KGDN_WAIT_CASE(9)
    KGDN_WAIT_CASE(10) KGDN_WAIT_CASE(11) KGDN_WAIT_CASE(12) KGDN_WAIT_CASE(13) KGDN_WAIT_CASE(14)
    KGDN_WAIT_CASE(15) KGDN_WAIT_CASE(16) KGDN_WAIT_CASE(17) KGDN_WAIT_CASE(18) KGDN_WAIT_CASE(19)
    KGDN_WAIT_CASE(20) KGDN_WAIT_CASE(21) KGDN_WAIT_CASE(22) KGDN_WAIT_CASE(23)
#undef KGDN_WAIT_CASE
    default: wait_loads_but<24>(); break;
  }
}
__device__ __forceinline__ uint32_t lds_u32(const void* p) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}

// chunk swizzles (see the file comment)
__device__ __forceinline__ int swz_wq(int r) { return (r & 3) | (((r >> 3) & 3) << 2); }
__device__ __forceinline__ int swz_a(int r) { return (((r >> 3) & 3) << 1) | ((r >> 1) & 1); }
__device__ __forceinline__ int swz_v(int r) { return (((r >> 3) & 1) << 1) | (((r >> 1) & 1) << 2); }
__device__ __forceinline__ int swz_o(int t) { return ((t >> 1) & 1) | (((t >> 3) & 3) << 1); }
// tiles written by a compute wave's 2-byte stores from accumulator tiles (rows 8 apart per lane group)
__device__ __forceinline__ int swz_s(int r) { return ((r >> 3) & 3) << 1; }

typedef __attribute__((address_space(3))) unsigned char lds_b;
typedef short s16x4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4v lds_s16x4v;
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) u32x2 lds_u32x2;

// LDS reads at a lane byte address plus an offset that is a constant after unrolling (it lands
// in the instruction's offset field); volatile keeps them in program order, where the pipelining
// puts them
__device__ __forceinline__ Frag<bf16> ld128(uint32_t a, uint32_t off) {
  Frag<bf16> f;
  f.v = __builtin_bit_cast(bf16x8, *reinterpret_cast<volatile const lds_u32x4*>(reinterpret_cast<lds_b*>(a) + off));
  return f;
}
__device__ __forceinline__ u32x2 ldtr(uint32_t a, uint32_t off) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                       reinterpret_cast<lds_s16x4v*>(reinterpret_cast<lds_b*>(a) + off)));
}
__device__ __forceinline__ void lds_st16(uint32_t a, uint32_t off, bf16 x) {
  *reinterpret_cast<__attribute__((address_space(3))) uint16_t*>(reinterpret_cast<lds_b*>(a) + off) =
      __builtin_bit_cast(uint16_t, x);
}

__device__ __forceinline__ Frag<bf16> frag2(u32x2 a, u32x2 b) {
  Frag<bf16> f;
  f.v = __builtin_bit_cast(bf16x8, u32x4{a[0], a[1], b[0], b[1]});
  return f;
}

// byte offset of the rowA row of accumulator tile x within a tile of row_bytes-long rows
__host__ __device__ constexpr uint32_t rowa_off(int x, uint32_t row_bytes) {
  return (uint32_t)(32 * (x >> 1) + 4 * (x & 1)) * row_bytes;
}

// Lane addresses of the per-step LDS reads, fixed for the whole sequence.
//  wq[k]: w row rowA(0, lc), chunk 4 ks + lg, for ks % 4 = k (q at + 32 KB); ks + 4 adds 256
//    bytes, tile x adds rowa_off(x, 512).
//  kr[ks]: k^T row rowA(0, lc), chunk 4 ks + lg; tile x adds rowa_off(x, 128).  The same lane
//    offsets serve Ai and Aqk (ar[ks]: Aqk buffer 0; Ai at a constant distance).
//  vt: the first of the two transposed reads of the v tile (rows 8 lg + lc / 4 and + 4, columns
//    16 w + 4 (lc % 4)) for ks = 0; ks = 1 adds 4096 bytes.
struct FAddr {
  uint32_t wq[4];
  uint32_t kr[2];
  uint32_t ar[2];
  uint32_t vt;
};

__device__ __forceinline__ void f_addr(FAddr& A, uint32_t w_lds, uint32_t k_lds, uint32_t a_lds, uint32_t v_lds) {
  const int l = lane_id(), lg = l >> 4, lc = l & 15, wid = threadIdx.x / WAVE;
  const int r0 = 8 * (lc >> 2) + (lc & 3);               // rowA(0, lc)
  {
    const int sw = swz_wq(r0);
#pragma unroll
    for (int k = 0; k < 4; ++k) A.wq[k] = w_lds + 512 * r0 + 16 * ((4 * k + lg) ^ sw);
  }
  {
    const int sa = swz_a(r0);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      A.kr[ks] = k_lds + 128 * r0 + 16 * ((4 * ks + lg) ^ sa);
      A.ar[ks] = a_lds + 128 * r0 + 16 * ((4 * ks + lg) ^ sa);
    }
  }
  {
    const int rv = 8 * lg + (lc >> 2), cv = 16 * wid + 4 * (lc & 3);
    A.vt = v_lds + 128 * rv + 16 * ((cv >> 3) ^ swz_v(rv)) + 2 * (cv & 7);
  }
}

// ---------------------------------------------------------------------------
// the loader wave's direct loads: one instruction moves 1 KB (64 lanes x 16 bytes) into consecutive
// LDS, so each instruction's lanes cover whole tile rows; rows past the chunk's end read row 0 (in
// w and q they only reach outputs of rows that are not stored and products with zero Aqk columns,
// in Ai and v rows of u that the gates zero)
// ---------------------------------------------------------------------------
// instruction i of a [64][256] tile (rows 2 i, 2 i + 1) of a token-major tensor
__device__ __forceinline__ void ld_tile256(const unsigned char* base, uint32_t row_bytes, int nv, int i, uint32_t dst) {
  const int l = lane_id(), r = 2 * i + (l >> 5), pos = l & 31;
  const uint32_t rr = r < nv ? (uint32_t)r : 0u;
  dma16_(base, rr * row_bytes + 16u * (pos ^ swz_wq(r)), dst + 1024u * i);
}
// instruction i of a [rows][64] tile (rows 8 i .. 8 i + 7) whose rows are row_bytes apart; swz is
// swz_a or swz_v of the row
template <bool kSwzA>
__device__ __forceinline__ void ld_tile64(const unsigned char* base, uint32_t row_bytes, int nv, int i, uint32_t dst) {
  const int l = lane_id(), r = 8 * i + (l >> 3), pos = l & 7;
  const uint32_t rr = r < nv ? (uint32_t)r : 0u;
  dma16_(base, rr * row_bytes + 16u * (pos ^ (kSwzA ? swz_a(r) : swz_v(r))), dst + 1024u * i);
}

// kRc: the backward's recompute of the forward (chunk_delta_h.py:52-224 alone): the state before each
// chunk (bf16, through the q half of the w / q tile, which q does not use here) and v_new (through the o
// tile) leave as whole rows stored by the loader waves; q, Aqk and the output products are skipped.
// the gated norm's exchange: how many times a workgroup loads a share again while the other workgroups of
// its head have not yet published it (each try a sleep of ~128 clocks and a load, ~1-2 us: ~25 ms in all);
// a share still missing then makes its token's rows NaN rather than holding the GPU
constexpr int kNormSpinMax = 1 << 14;

template <bool kRc, bool kNorm>
__global__ __launch_bounds__(NT_F + FL * WAVE) void wide_fused_kernel(WideFusedArgs a, int V, int total_units) {
  // LDS: w and q of the chunk (adjacent: q reads are w reads + 32 KB), k^T of the chunk, and two
  // buffer sets of the chunk's small tiles: Aqk, Ai, the v tile of the workgroup's 64 columns, gc, beta
  __shared__ __align__(16) bf16 s_wq[2 * C * FK];
  __shared__ __align__(16) bf16 s_k[C * FK];
  __shared__ __align__(16) bf16 s_a[2 * C * C];
  __shared__ __align__(16) bf16 s_ai[2 * C * C];
  __shared__ __align__(16) bf16 s_v[2 * C * C];
  __shared__ __align__(16) float s_g[2 * C];
  __shared__ __align__(16) float s_b[2 * C];
  __shared__ __align__(16) float s_qs[2 * C];             // rstd of the q rows (the in-op L2 norm)
  __shared__ __align__(16) bf16 s_o[C * C];               // the chunk's o tile [64 t][64 columns]
  __shared__ __align__(16) float s_pf[WAVE];              // landing words of the L2 prefetch
  constexpr uint32_t QOFF = C * FK * 2, ABUF = C * C * 2, GBUF = C * 4;

  // XCD-aware order: the V tiles of one head run on one XCD and share its q, w, k^T, Aqk, Ai in L2
  const int per_xcd = gridDim.x / 8;
  const int o_idx = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (o_idx >= total_units) return;
  const int nvt = V / FVT;
  const int unit = o_idx / nvt;
  const int H = a.H;
  const int n = unit / H, h = unit % H;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE), l = lane_id(), lg = l >> 4, lc = l & 15;
  const int vt0 = __builtin_amdgcn_readfirstlane((o_idx % nvt) * FVT);    // the workgroup's first column

  int64_t bos, eos, c_first;
  if (a.cu == nullptr) {
    bos = (int64_t)n * a.T;
    eos = bos + a.T;
    c_first = (int64_t)n * ((a.T + C - 1) / C);
  } else {
    bos = a.cu[n];
    eos = a.cu[n + 1];
    c_first = a.chunk_off[n];
  }
  const int64_t nchunks = (eos - bos + C - 1) / C;
  // the chunks walked: ib .. ie - 1 (h0 is the state before chunk ib)
  const int64_t ib = min(a.it_begin, nchunks), ie = a.it_end > 0 ? min(a.it_end, nchunks) : nchunks;
  auto chunk_nv = [&](int64_t it) { return (int)min((int64_t)C, eos - (bos + it * C)); };
  const uint32_t w_lds = lds_u32(s_wq), k_lds = lds_u32(s_k), a_lds = lds_u32(s_a), ai_lds = lds_u32(s_ai),
                 v_lds = lds_u32(s_v), g_lds = lds_u32(s_g), b_lds = lds_u32(s_b), o_lds = lds_u32(s_o),
                 qs_lds = lds_u32(s_qs);
  // the in-op L2 norm: q arrives raw and o_inter's column t (token t) is scaled by rstd of q row t,
  // which prepare recorded beside the normalised k^T, w and Aqk
  const bool qn = !kRc && a.qs != nullptr;
  // the layer's prologue folded in: the loader waves form the workgroup's v tile from the projection
  // (short convolution + SiLU) instead of loading v
  const bool cvm = !kRc && !kNorm && a.cv.x != nullptr;
  const bf16* aqb = reinterpret_cast<const bf16*>(a.aqk);
  const bf16* ktb = reinterpret_cast<const bf16*>(a.kT);

  if (wid >= FW) {
    // ---- the loader waves: every direct load of the workgroup, so that the four compute waves never
    //      stall on the address unit; four of them, because one wave keeps at most 63 loads in
    //      flight.  Loader lw issues load i of each tile for i % FL = lw.  Per chunk step it, between
    //      the compute waves' two barriers: after B1, k^T of chunk it (8 loads each), the small tiles
    //      of chunk it + 1 into the other buffer set (6 each, and gc / beta from loaders 0 / 1) and its
    //      part of the L2 prefetch of chunk it + 2 (1); with the in-op L2 norm loader 2 also brings the
    //      rstd of the q rows (a word per token, beside gc); before B2 each waits for its k^T loads; after
    //      B2 (the compute waves are done with w and q), w and q of chunk it + 1 (16 each).  The o tile
    //      the compute waves left in LDS in step it - 1 goes out right after B1, as whole 128-byte
    //      rows (two 1 KB stores per loader); from the compute waves, whose lanes hold 4 columns of a
    //      token, the same stores would touch 16 lines each and stall them behind the loads.
    const int lw = wid - FW;
    const int kSmall = (cvm ? 4 : 6) + (lw < 2 || (qn && lw == 2) ? 1 : 0);
    const uint32_t RB = (uint32_t)H * FK * 2;
    auto small = [&](int64_t c, int64_t t0, int nv, uint32_t B) {
      const unsigned char* ab = reinterpret_cast<const unsigned char*>(aqb + (c * H + h) * (int64_t)(C * C));
      const unsigned char* aib = reinterpret_cast<const unsigned char*>(a.Ai) + (size_t)((t0 * H + h) * C) * 2;
      const unsigned char* vb = reinterpret_cast<const unsigned char*>(a.v) + (size_t)((t0 * H + h) * V + vt0) * 2;
#pragma unroll
      for (int j = 0; j < 8 / FL; ++j)
        if constexpr (!kRc) ld_tile64<true>(ab, 128u, C, FL * j + lw, a_lds + B * ABUF);
#pragma unroll
      for (int j = 0; j < 8 / FL; ++j) ld_tile64<true>(aib, (uint32_t)H * C * 2, nv, FL * j + lw, ai_lds + B * ABUF);
      if (!cvm) {
#pragma unroll
        for (int j = 0; j < 8 / FL; ++j) ld_tile64<false>(vb, (uint32_t)H * V * 2, nv, FL * j + lw, v_lds + B * ABUF);
      }
      const uint32_t gl_off = (uint32_t)(l < nv ? l : 0) * (uint32_t)H * 4u;
      if (lw == 0) dma4_(a.gc + t0 * H + h, gl_off, g_lds + B * GBUF);
      if (lw == 1) dma4_(a.beta + t0 * H + h, gl_off, b_lds + B * GBUF);
      if (qn && lw == 2) dma4_(a.qs + t0 * H + h, gl_off, qs_lds + B * GBUF);
    };
    auto wq = [&](int64_t t0, int nv) {
      const unsigned char* wb = reinterpret_cast<const unsigned char*>(a.w) + (size_t)((t0 * H + h) * FK) * 2;
      const unsigned char* qb = reinterpret_cast<const unsigned char*>(a.q) + (size_t)((t0 * H + h) * FK) * 2;
#pragma unroll
      for (int j = 0; j < 32 / FL; ++j) ld_tile256(wb, RB, nv, FL * j + lw, w_lds);
#pragma unroll
      for (int j = 0; j < 32 / FL; ++j)
        if constexpr (!kRc) ld_tile256(qb, RB, nv, FL * j + lw, w_lds + QOFF);
    };
    // L2 prefetch of chunk (c, t0)'s w and q rows and its k^T and Aqk tiles: one 4-byte direct load
    // per 128-byte line into a scratch LDS word (never read), so that the tile loads a step later
    // hit L2 instead of waiting for HBM.  The V tiles of a head share the XCD's L2, so each workgroup
    // touches a quarter of the lines: rows 16 (vt % 4) .. + 15 of w and q, lines 64 (vt % 4) .. + 63
    // of k^T, 16 lines of Aqk.  The address unit works per line, so a full prefetch per workgroup
    // would cost as much of it as the tile loads themselves.
    const uint32_t pf_lds = lds_u32(s_pf);
    const int pf_q = (vt0 / FVT) & 3;
    auto prefetch = [&](int64_t c, int64_t t0, int nv) {     // one load per loader wave (kRc: loaders 0, 2)
      if (kRc && (lw & 1)) return;
      if (lw < 2) {
        const int r = 16 * pf_q + (l >> 2);
        const uint32_t off = (uint32_t)(r < nv ? r : 0) * RB + 128u * (l & 3);
        dma4_(reinterpret_cast<const unsigned char*>(lw == 0 ? a.w : a.q) + (size_t)((t0 * H + h) * FK) * 2, off, pf_lds);
      } else if (lw == 2) {
        dma4_(ktb + (c * H + h) * (int64_t)(FK * C), 128u * (64 * pf_q + l), pf_lds);
      } else {
        dma4_(aqb + (c * H + h) * (int64_t)(C * C), 128u * (16 * pf_q + (l & 15)), pf_lds);
      }
    };
    // the o tile of chunk (t0, nv) from LDS to HBM: rows 8 i .. 8 i + 7 for i % FL = lw
    auto store_o = [&](int64_t t0, int nv) {
      const int c8 = l & 7;
      u32x4 x[8 / FL];                                   // both rows read before either store: one LDS wait
#pragma unroll
      for (int j = 0; j < 8 / FL; ++j) {
        const int t = 8 * (FL * j + lw) + (l >> 3);
        x[j] = *reinterpret_cast<const lds_u32x4*>(reinterpret_cast<lds_b*>(o_lds) + 128 * t + 16 * (c8 ^ swz_o(t)));
      }
#pragma unroll
      for (int j = 0; j < 8 / FL; ++j) {
        const int t = 8 * (FL * j + lw) + (l >> 3);
        if (t < nv)
          st_global(reinterpret_cast<unsigned char*>(kRc ? a.vn_out : a.o) + (((t0 + t) * H + h) * V + vt0 + 8 * c8) * 2,
                    x[j]);
      }
    };
    // kRc: the state snapshot of chunk c (rows d of the q half of the w / q tile) to h_out [NC, H, 256, V]
    auto store_h = [&](int64_t c) {
#pragma unroll
      for (int j = 0; j < 32 / FL; ++j) {
        const int d = 8 * (FL * j + lw) + (l >> 3), c8 = l & 7;
        const u32x4 x = *reinterpret_cast<const lds_u32x4*>(reinterpret_cast<lds_b*>(w_lds + QOFF) + 128 * d + 16 * (c8 ^ swz_s(d)));
        *reinterpret_cast<u32x4*>(reinterpret_cast<unsigned char*>(a.h_out) + (((c * H + h) * FK + d) * V + vt0 + 8 * c8) * 2) = x;
      }
    };
    // ---- kNorm: the layer's gated RMSNorm (fused_norm_gate.py:42-127) over the o the loaders store.
    //      Lane (lw, l) owns the rows store_o moves, tokens t_j = 8 (FL j + lw) + l / 8, columns
    //      vt0 + 8 (l % 8) .. + 7.  Chunk c: in step c + 1 o goes out as before and the workgroup's
    //      share of each token's sum of squares (its 64 columns, from the o tile in LDS) is published
    //      to nss, tagged with the call's epoch; in step c + 3 the head's V / 64 shares of each token,
    //      its gate row and its o row (back from L2) are loaded; in step c + 4, any share without the
    //      call's tag is loaded again until it has it, and y replaces o.  The shares travel as single
    //      8-byte agent-scope atomics, so a matching tag vouches for its value; the head's workgroups run
    //      in step, so a share is normally in place two steps before it is loaded.  The loaders bound
    //      the step: everything here runs after the k^T loads are issued, while the loaders would wait
    //      for them anyway, and every memory instruction from the publication on executes on all lanes
    //      (masked rows go to a dummy line past the shares), so the counted wait before B2 stays exact.
    const int nvt_h = V / FVT, vtile = vt0 / FVT, nc8 = l & 7;
    u32x4 no[2], ng[2];
    unsigned long long nps[2];
    float nsh[2];
    float nwv[8], nbv[8];
    if constexpr (kNorm) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int col = vt0 + 8 * nc8 + e;
        nwv[e] = a.nw == nullptr ? 1.f
                 : a.nw_dtype == DT_F32 ? reinterpret_cast<const float*>(a.nw)[col]
                                        : (float)reinterpret_cast<const bf16*>(a.nw)[col];
        nbv[e] = a.nb == nullptr ? 0.f
                 : a.nw_dtype == DT_F32 ? reinterpret_cast<const float*>(a.nb)[col]
                                        : (float)reinterpret_cast<const bf16*>(a.nb)[col];
      }
    }
    const unsigned long long ntag = (unsigned long long)a.nepoch << 32;
    auto ntok = [&](int j) { return 8 * (FL * j + lw) + (l >> 3); };
    auto nslot = [&](int64_t c, int t) { return a.nss + (((c_first + c) * H + h) * C + t) * 8; };
    // the dummy line: one 16-byte slot per lane past the last share (written, never read)
    u32x4* const ndummy = reinterpret_cast<u32x4*>(a.nss + (size_t)a.nss_chunks * H * C * 8) + l;
    // o of chunk c from LDS to HBM (store_o's rows) and the workgroup's shares of its tokens into nsh
    auto n_store_share = [&](int64_t c) {
      const int64_t t0 = bos + c * C;
      const int nv = chunk_nv(c);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int t = ntok(j);
        const u32x4 x = *reinterpret_cast<const lds_u32x4*>(reinterpret_cast<lds_b*>(o_lds) + 128 * t + 16 * (nc8 ^ swz_o(t)));
        if (t < nv) st_global(reinterpret_cast<bf16*>(a.o) + ((t0 + t) * H + h) * V + vt0 + 8 * nc8, x);
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float x0 = __uint_as_float(x[e] << 16), x1 = __uint_as_float(x[e] & 0xffff0000u);
          ss = fmaf(x0, x0, ss);
          ss = fmaf(x1, x1, ss);
        }
        ss += __shfl_xor(ss, 4, WAVE);
        ss += __shfl_xor(ss, 2, WAVE);
        ss += __shfl_xor(ss, 1, WAVE);
        nsh[j] = ss;
      }
    };
    // two store instructions (the 8 lanes of a token store the same word)
    auto n_publish = [&](int64_t c) {
#pragma unroll
      for (int j = 0; j < 2; ++j)
        __hip_atomic_store(nslot(c, ntok(j)) + vtile, ntag | __float_as_uint(nsh[j]), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    };
    // six load instructions: the shares, the gate row, the o row
    auto n_fetch = [&](int64_t c) {
      const int64_t t0 = bos + c * C;
      const int nv = chunk_nv(c);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int t = ntok(j);
        const unsigned long long sh =
            __hip_atomic_load(nslot(c, t) + min(nc8, nvt_h - 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        nps[j] = nc8 < nvt_h ? sh : ntag;
        const int tr = t < nv ? t : 0;
        const int64_t off = ((t0 + tr) * H + h) * V + vt0 + 8 * nc8;
        ng[j] = ld_global<u32x4>(reinterpret_cast<const bf16*>(a.ngate) + off);
        no[j] = ld_global<u32x4>(reinterpret_cast<const bf16*>(a.o) + off);
      }
    };
    // y of chunk c from the fetched rows; two store instructions
    auto n_finish = [&](int64_t c) {
      const int64_t t0 = bos + c * C;
      const int nv = chunk_nv(c);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int t = ntok(j);
#pragma unroll 1
        for (int spins = 0;; ++spins) {                 // wave-uniform exit
          const bool bad = (nps[j] & 0xffffffff00000000ull) != ntag;
          if (__ballot(bad) == 0) break;
          if (spins == kNormSpinMax) {
            if (bad) nps[j] = ntag | 0x7fc00000u;        // NaN: the share never arrived
            break;
          }
          __builtin_amdgcn_s_sleep(2);
          if (bad) nps[j] = __hip_atomic_load(nslot(c, t) + nc8, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        float tot = __uint_as_float((uint32_t)nps[j]);
        tot += __shfl_xor(tot, 4, WAVE);
        tot += __shfl_xor(tot, 2, WAVE);
        tot += __shfl_xor(tot, 1, WAVE);
        const float r = __builtin_amdgcn_rsqf(tot / (float)V + a.neps);
        const u32x4 x = no[j], gq = ng[j];
        u32x4 y;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float yv[2];
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            const float xf = hh ? __uint_as_float(x[e] & 0xffff0000u) : __uint_as_float(x[e] << 16);
            const float gf = hh ? __uint_as_float(gq[e] & 0xffff0000u) : __uint_as_float(gq[e] << 16);
            const float v = fmaf(xf * r, nwv[2 * e + hh], nbv[2 * e + hh]);
            const float sg = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-gf * 1.4426950408889634f));
            yv[hh] = a.nsigmoid_only ? v * sg : v * gf * sg;
          }
          y[e] = (uint32_t)__builtin_bit_cast(uint16_t, (bf16)yv[0]) |
                 ((uint32_t)__builtin_bit_cast(uint16_t, (bf16)yv[1]) << 16);
        }
        u32x4* dst = t < nv ? reinterpret_cast<u32x4*>(reinterpret_cast<bf16*>(a.o) + ((t0 + t) * H + h) * V + vt0 + 8 * nc8)
                            : ndummy;
        st_global(dst, y);
      }
    };
    // the folded convolution of v: loader lane L = 64 lw + l forms rows 2 (L / 8), + 1 of 16-byte
    // column chunk L % 8 of the workgroup's 64 columns, with that chunk's taps in registers for the
    // whole walk.  The window of chunk c (window buffer (c - ib) % 2) is loaded after B1 of step c - 2
    // (compiler-visible loads, counted in the wait for k^T and complete at the next step's wait for
    // all loads) and convolved into its v buffer after B2 of step c - 1, where the loader waves are
    // otherwise idle and the compute waves are done with the chunk that buffer held.
    const int cL = 64 * lw + l, cch = cL & 7, crp = cL >> 3;
    const int64_t cc0 = (int64_t)h * V + vt0 + 8 * cch;
    ConvTaps ctp;
    ConvWin<2> cwa, cwb;                              // windows of chunks ib, ib + 2, ... / ib + 1, ...
    if (cvm) load_taps(ctp, a.cv, cc0);
    auto conv_issue = [&](ConvWin<2>& w, int64_t it) {
      const int64_t t0 = bos + it * C;
      w.issue(a.cv, t0 + 2 * crp, bos, t0 + chunk_nv(it), cc0);
    };
    auto conv_store = [&](ConvWin<2>& w, int64_t it, uint32_t Bv) {
      const int64_t t0 = bos + it * C;
      cvx4 y[2];
      w.finish(a.cv, ctp, t0 + 2 * crp, bos, n, cc0, y);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int r = 2 * crp + j;
        *reinterpret_cast<lds_u32x4*>(reinterpret_cast<lds_b*>(v_lds + Bv * ABUF) + 128 * r + 16 * (cch ^ swz_v(r))) =
            y[j];
      }
    };
    if (ie - ib > 1) prefetch(c_first + ib + 1, bos + (ib + 1) * C, chunk_nv(ib + 1));
    if (ie > ib) {
      small(c_first + ib, bos + ib * C, chunk_nv(ib), 0u);
      wq(bos + ib * C, chunk_nv(ib));
      if (cvm) {
        conv_issue(cwa, ib);
        conv_store(cwa, ib, 0u);
        if (ie - ib > 1) conv_issue(cwb, ib + 1);
      }
    }
    // one step; PB = (it - ib) % 2 at compile time, so that the window buffers are named registers
    auto loader_step = [&](auto PB, int64_t it) {
      constexpr int PAR = decltype(PB)::value;
      ConvWin<2>& w_next = PAR ? cwb : cwa;              // chunk it + 2
      ConvWin<2>& w_now = PAR ? cwa : cwb;               // chunk it + 1
      // the buffer set of chunk it (with kNorm the step is instantiated once, for code size)
      const uint32_t B = kNorm ? (uint32_t)((it - ib) & 1) : (uint32_t)PAR;
      const int64_t in = it + 1 < ie ? it + 1 : it;       // the last step reloads its own chunk (unused)
      wait_all_loads();
      f_barrier();                                        // B1
      if constexpr (!kNorm) {
        if (it > ib) store_o(bos + (it - 1) * C, chunk_nv(it - 1));
      }
      const unsigned char* kb = reinterpret_cast<const unsigned char*>(ktb + ((c_first + it) * H + h) * (int64_t)(FK * C));
#pragma unroll
      for (int j = 0; j < 32 / FL; ++j) ld_tile64<true>(kb, 128u, FK, FL * j + lw, k_lds);
      if constexpr (kNorm) {
        if (it > ib) n_store_share(it - 1);
      }
      small(c_first + in, bos + in * C, chunk_nv(in), B ^ 1u);
      // the window of chunk it + 2 (convolved after B2 of step it + 1)
      const int nwin = (cvm && it + 2 < ie) ? kConvW + 1 : 0;
      if (nwin) conv_issue(w_next, it + 2);

      // this wave's k^T loads landed; the later ones (6 + gc / beta + the prefetch) stay in flight
      if constexpr (kRc) {                                // small: 4, and gc / beta from loaders 0 / 1
        if (it + 2 < ie) {
          prefetch(c_first + it + 2, bos + (it + 2) * C, chunk_nv(it + 2));
          if (lw == 0) wait_loads_but<6>();
          else if (lw == 3) wait_loads_but<4>();
          else wait_loads_but<5>();
        } else {
          if (lw < 2) wait_loads_but<5>();
          else wait_loads_but<4>();
        }
      } else {
        const int npf = it + 2 < ie ? 1 : 0;
        if (npf) prefetch(c_first + it + 2, bos + (it + 2) * C, chunk_nv(it + 2));
        // kNorm: the shares of chunk it - 1, y of chunk it - 4, the rows of chunk it - 3; all left in
        // flight across B2 (two, two and six instructions)
        int nnorm = 0;
        if constexpr (kNorm) {
          if (it > ib) {
            n_publish(it - 1);
            nnorm += 2;
          }
          if (it - 4 >= ib) {
            n_finish(it - 4);
            nnorm += 2;
          }
          if (it - 3 >= ib) {
            n_fetch(it - 3);
            nnorm += 6;
          }
        }
        wait_loads_but_n(kSmall + nwin + npf + nnorm);
      }
      f_barrier();                                        // B2
      if constexpr (kRc) store_h(c_first + it);           // written by the compute waves before B2
      if (it + 1 < ie) wq(bos + (it + 1) * C, chunk_nv(it + 1));
      if (cvm && it + 1 < ie) conv_store(w_now, it + 1, B ^ 1u);  // its window arrived before B1
    };
    if constexpr (kNorm) {
      for (int64_t it = ib; it < ie; ++it) loader_step(std::integral_constant<int, 0>{}, it);
    } else {
      for (int64_t it = ib; it < ie; it += 2) {
        loader_step(std::integral_constant<int, 0>{}, it);
        if (it + 1 < ie) loader_step(std::integral_constant<int, 1>{}, it + 1);
      }
    }
    f_barrier();                                          // the last o tile is in LDS
    if (ie > ib) {
      if constexpr (kNorm) {
        // y of chunk L - 3 (loaded in step L), then of chunks L - 2, L - 1 (published) and L (in LDS)
        const int64_t L = ie - 1;
        n_store_share(L);
        n_publish(L);
        wait_all_loads();                                 // this workgroup's o rows and shares are in place
        if (L - 3 >= ib) n_finish(L - 3);
        for (int64_t c = L - 2 >= ib ? L - 2 : ib; c <= L; ++c) {
          n_fetch(c);
          n_finish(c);
        }
      } else {
        store_o(bos + (ie - 1) * C, chunk_nv(ie - 1));
      }
    }
    wait_all_loads();                                     // no direct load outlives the workgroup's LDS
    return;
  }

  // ---- the compute waves: wave wid owns value columns v0 .. v0 + 15
  const int v0 = vt0 + 16 * wid;
  const int vcol = v0 + lc;
  const int ra0 = 8 * (lc >> 2) + (lc & 3);               // rowA(0, lc)
  // state: S[kt][j] = S[32 (kt / 2) + 8 lg + 4 (kt % 2) + j][vcol] (the paired row order)
  // (the dtype branch outside the loops, so that the 64 loads go out together)
  f32x4 S[16];
  auto load_state = [&](auto ld) {
#pragma unroll
    for (int kt = 0; kt < 16; ++kt)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        S[kt][j] = ld((((int64_t)n * H + h) * FK + 32 * (kt >> 1) + 8 * lg + 4 * (kt & 1) + j) * V + vcol);
  };
  if (a.h0 == nullptr) {
    load_state([](int64_t) { return 0.f; });
  } else if (a.h0_dtype == DT_F32) {
    const float* h0 = reinterpret_cast<const float*>(a.h0);
    load_state([h0](int64_t off) { return h0[off]; });
  } else {
    const bf16* h0 = reinterpret_cast<const bf16*>(a.h0);
    load_state([h0](int64_t off) { return (float)h0[off]; });
  }
  FAddr A;
  f_addr(A, w_lds, k_lds, a_lds, v_lds);
  const uint32_t AI_OFF = ai_lds - a_lds;                 // Ai tiles share the Aqk lane addresses
  // kRc: 2-byte writes of row 8 lg (+ the accumulator row offsets), column 16 wid + lc: the snapshot into
  // the q half of the w / q tile (swizzle swz_s) and v_new into the o tile (swizzle swz_o, whose row bit
  // 1 is j / 2 of the accumulator element)
  const int cs = 16 * wid + lc;
  const uint32_t snap_w = w_lds + QOFF + 128 * (8 * lg) + 16 * ((cs >> 3) ^ swz_s(8 * lg)) + 2 * (cs & 7);
  const uint32_t vn_w[2] = {o_lds + 128 * (8 * lg) + 16 * ((cs >> 3) ^ swz_o(8 * lg)) + 2 * (cs & 7),
                            o_lds + 128 * (8 * lg) + 16 * ((cs >> 3) ^ swz_o(8 * lg + 2)) + 2 * (cs & 7)};

  // One chunk step between the loader's barriers: after B1 (w, q and the small tiles of chunk it in
  // LDS, buffer set B = it % 2), w h and h^T q^T; after B2 (k^T in LDS), u, v', o and the update.
  auto step = [&](auto BB, int64_t it) {
    constexpr uint32_t B = decltype(BB)::value;
    const int nv = chunk_nv(it);
    f_barrier();                                          // B1
    const float* sg = s_g + B * C;
    const float* sb = s_b + B * C;

    // u = Ai bf16(beta v) (wy_fast.py:55-81), rounded to bf16 as the reference stores it, from tiles
    // already in LDS at B1: the v tile is read transposed (rows s = 32 ks + 8 lg + e) and scaled by
    // beta per row.  -bf16(u) starts the w h accumulators, so they end as w h - u = -v'.
    f32x4 acc[4], oi[4];
    {
      Frag<bf16> vb[2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const uint32_t vo = B * ABUF + 4096u * ks;
        const Frag<bf16> vr = frag2(ldtr(A.vt, vo), ldtr(A.vt, vo + 512u));
        const f32x4 b0 = *reinterpret_cast<const f32x4*>(sb + 32 * ks + 8 * lg);
        const f32x4 b1 = *reinterpret_cast<const f32x4*>(sb + 32 * ks + 8 * lg + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          vb[ks].v[e] = (bf16)((float)vr.v[e] * b0[e]);
          vb[ks].v[4 + e] = (bf16)((float)vr.v[4 + e] * b1[e]);
        }
      }
#pragma unroll
      for (int tm = 0; tm < 4; ++tm) {
        acc[tm] = f32x4{0.f, 0.f, 0.f, 0.f};
        oi[tm] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
          if (ks <= tm / 2) mma(acc[tm], ld128(A.ar[ks], AI_OFF + B * ABUF + rowa_off(tm, 128)), vb[ks]);
      }
#pragma unroll
      for (int tm = 0; tm < 4; ++tm)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[tm][j] = -(float)(bf16)acc[tm][j];
    }

    // w h - u (rows t in the paired order, this wave's columns) and o_inter^T = h^T q^T (rows =
    // columns, cols = t = rowA(tn, lc)), with h = bf16(S) packed per 32-deep step as the B (w h)
    // and A (h^T q^T) operand; operand reads one step ahead of the products
    Frag<bf16> wa[2][4], qa[2][4];
    auto read_wq = [&](int ks, Frag<bf16>(&w4)[4], Frag<bf16>(&q4)[4]) {
      const uint32_t ra = A.wq[ks & 3];
      const uint32_t o8 = 256u * (ks >> 2);
#pragma unroll
      for (int tm = 0; tm < 4; ++tm) {
        w4[tm] = ld128(ra, o8 + rowa_off(tm, 512));
        if constexpr (!kRc) q4[tm] = ld128(ra, QOFF + o8 + rowa_off(tm, 512));
      }
    };
    read_wq(0, wa[0], qa[0]);
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      if (ks + 1 < 8) read_wq(ks + 1, wa[(ks + 1) & 1], qa[(ks + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
      const Frag<bf16> hb = pack_acc(S[2 * ks], S[2 * ks + 1]);
#pragma unroll
      for (int tm = 0; tm < 4; ++tm) {
        if constexpr (!kRc) mma(oi[tm], hb, qa[ks & 1][tm]);
        mma(acc[tm], wa[ks & 1][tm], hb);
      }
      if constexpr (kRc) {                                // the snapshot: rows 32 ks + 8 lg + 4 x + j
#pragma unroll
        for (int x = 0; x < 2; ++x)
#pragma unroll
          for (int j = 0; j < 4; ++j) lds_st16(snap_w, 128u * (32 * ks + 4 * x + j), hb.v[4 * x + j]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    f_barrier();                                          // B2: k^T in LDS; w and q tiles free

    // the output's LDS operands first (one latency for all): Aqk row pieces, exp(gc_t) per tile and
    // with the in-op L2 norm rstd of q row t
    Frag<bf16> aq[6];
    float egt[4], qst[4];
    if constexpr (!kRc) {
#pragma unroll
      for (int tn = 0, f = 0; tn < 4; ++tn) {
        egt[tn] = sg[32 * (tn >> 1) + 4 * (tn & 1) + ra0];
        qst[tn] = qn ? s_qs[B * C + 32 * (tn >> 1) + 4 * (tn & 1) + ra0] : 1.f;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
          if (ks <= tn / 2) aq[f++] = ld128(A.ar[ks], B * ABUF + rowa_off(tn, 128));
      }
    }
    // v' = u - w h (rows t = 32 (tm / 2) + 8 lg + 4 (tm % 2) + j), its bf16 value and the gated form
    const float gl = sg[nv - 1];
    f32x4 Y[4], Yg[4];
#pragma unroll
    for (int tm = 0; tm < 4; ++tm) {
      Y[tm] = -acc[tm];
      const int tr = 32 * (tm >> 1) + 8 * lg + 4 * (tm & 1);
      const f32x4 g4 = *reinterpret_cast<const f32x4*>(sg + tr);
#pragma unroll
      for (int j = 0; j < 4; ++j) Yg[tm][j] = tr + j < nv ? Y[tm][j] * gexp(gl - g4[j]) : 0.f;
    }
    Frag<bf16> vf[2], vg[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      vf[ks] = pack_acc(Y[2 * ks], Y[2 * ks + 1]);
      vg[ks] = pack_acc(Yg[2 * ks], Yg[2 * ks + 1]);
    }
    if constexpr (kRc) {                                  // v_new = bf16(v') into the o tile
#pragma unroll
      for (int tm = 0; tm < 4; ++tm)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          lds_st16(vn_w[j >> 1], 128u * (32 * (tm >> 1) + 4 * (tm & 1) + j), (bf16)Y[tm][j]);
    } else {
    // o^T = (o_inter^T exp(gc_t) + v'^T Aqk^T) scale; lane: columns 16 w + 4 lg .. + 3 of token
    // rowA(tn, lc), into the LDS o tile (the loader waves store it after the next B1)
    f32x4 r[4];
#pragma unroll
    for (int tn = 0, f = 0; tn < 4; ++tn) {
      r[tn] = oi[tn] * (gexp(egt[tn]) * qst[tn]);
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        if (ks <= tn / 2) mma(r[tn], vf[ks], aq[f++]);
    }
#pragma unroll
    for (int tn = 0; tn < 4; ++tn) {
      const int t = 32 * (tn >> 1) + 4 * (tn & 1) + ra0;
      const f32x4 x = r[tn] * a.scale;
      const u32x2 ov = {
          (uint32_t)__builtin_bit_cast(uint16_t, (bf16)x[0]) | ((uint32_t)__builtin_bit_cast(uint16_t, (bf16)x[1]) << 16),
          (uint32_t)__builtin_bit_cast(uint16_t, (bf16)x[2]) | ((uint32_t)__builtin_bit_cast(uint16_t, (bf16)x[3]) << 16)};
      *reinterpret_cast<lds_u32x2*>(reinterpret_cast<lds_b*>(o_lds) + 128 * t + 16 * ((2 * wid + (lg >> 1)) ^ swz_o(t)) +
                                    8 * (lg & 1)) = ov;
    }
    }
    // S = exp(g_last) S + k^T (v' exp(g_last - gc)), pipelined like the products above
    const float eg = gexp(gl);
    Frag<bf16> ka[2][4][2];
    auto read_k = [&](int k4, Frag<bf16>(&k8)[4][2]) {
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        k8[qq][0] = ld128(A.kr[0], rowa_off(k4 + qq, 128));
        k8[qq][1] = ld128(A.kr[1], rowa_off(k4 + qq, 128));
      }
    };
    read_k(0, ka[0]);
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      if (g4 + 1 < 4) read_k(4 * (g4 + 1), ka[(g4 + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        S[4 * g4 + qq] *= eg;
        mma(S[4 * g4 + qq], ka[g4 & 1][qq][0], vg[0]);
        mma(S[4 * g4 + qq], ka[g4 & 1][qq][1], vg[1]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  for (int64_t it = ib; it < ie; it += 2) {
    step(std::integral_constant<uint32_t, 0>{}, it);
    if (it + 1 < ie) step(std::integral_constant<uint32_t, 1>{}, it + 1);
  }
  f_barrier();                                            // the last o tile is in LDS for the loaders

  if (a.ht) {
#pragma unroll
    for (int kt = 0; kt < 16; ++kt) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t off = (((int64_t)n * H + h) * FK + 32 * (kt >> 1) + 8 * lg + 4 * (kt & 1) + j) * V + vcol;
        a.ht[off] = S[kt][j];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Backward dh recurrence for K = 256, bf16 (fla ops/common/chunk_delta_h.py:250-438): one workgroup
// per (sequence, head, 64 value columns), four compute waves of 16 columns each holding dh over all
// 256 rows (fp32, accumulator layout, the paired row order above) and four loader waves.  Per
// chunk, last to first:
//
//   dh[c] = bf16(dh)                                          stored for the gradient kernels
//   dv2   = (k bf16(dh)) exp(g_last - gc) + dv_local          0 past the chunk's end; stored
//   dh    = exp(g_last) dh + q^T (do exp(gc) scale) - w^T bf16(dv2)
//
// The reference forms q exp(gc) in fp32 and takes its product with do in fp32; here q stays bf16
// (exact) and x = do exp(gc) scale enters as hi + lo = bf16(x) + bf16(x - bf16(x)): two bf16
// products, 16 significant bits in that operand.
//
// Operands, all in the contiguous K order: k [64 t][256] as the A operand of k dh (rows rowA, the
// forward's w tile); q^T and w^T [256 d][64 t] per chunk (written by the dv_local stage and the
// prepare kernel) as the A operands of the update (rows rowA, the forward's k^T tile); do and
// dv_local [64 t][64] read transposed (the forward's v tile); dv2 from its accumulator tiles.  After
// B1 (k, q^T, do, gc in LDS): the snapshot, k dh and the q^T x update; after B2 (w^T, dv_local in
// LDS): dv2 and the w^T dv2 update.  The snapshot and dv2 leave through LDS tiles that the loader
// waves store as whole 128-byte rows; chunk c of row r sits at c ^ 2 ((r / 8) % 4), so the four lane
// groups of a compute wave's 2-byte writes (rows 8 apart) land on distinct banks.
// ---------------------------------------------------------------------------
namespace dhu_lds {
constexpr uint32_t K_OFF = 0;                        // k [64][256]
constexpr uint32_t QW_OFF = K_OFF + C * FK * 2;      // q^T [256][64], then w^T
constexpr uint32_t W_REL = FK * C * 2;               // w^T - q^T
constexpr uint32_t SNAP_OFF = QW_OFF + 2 * W_REL;    // bf16(dh) [256][64]
constexpr uint32_t DO_OFF = SNAP_OFF + FK * C * 2;   // do [64][64]
constexpr uint32_t DL_OFF = DO_OFF + C * C * 2;      // dv_local [64][64]
constexpr uint32_t DV_OFF = DL_OFF + C * C * 2;      // bf16(dv2) [64][64]
constexpr uint32_t G_OFF = DV_OFF + C * C * 2;       // gc, two buffers
constexpr uint32_t PF_OFF = G_OFF + 2 * C * 4;       // landing words of the L2 prefetch
constexpr uint32_t TOTAL = PF_OFF + WAVE * 4;
}  // namespace dhu_lds

__global__ __launch_bounds__(NT_F + FL * WAVE) void wide_dhu_kernel(BwdArgs a, int V, int total_units) {
  using namespace dhu_lds;
  __shared__ __align__(16) unsigned char smem[TOTAL];
  const uint32_t base = lds_u32(smem);

  const int per_xcd = gridDim.x / 8;                      // XCD-aware order, as the forward
  const int o_idx = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (o_idx >= total_units) return;
  const int nvt = V / FVT;
  const int unit = o_idx / nvt;
  const int H = a.H;
  const int n = unit / H, h = unit % H;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE), l = lane_id(), lg = l >> 4, lc = l & 15;
  const int vt0 = __builtin_amdgcn_readfirstlane((o_idx % nvt) * FVT);

  int64_t bos, eos, c_first;
  if (a.cu == nullptr) {
    bos = (int64_t)n * a.T;
    eos = bos + a.T;
    c_first = (int64_t)n * ((a.T + C - 1) / C);
  } else {
    bos = a.cu[n];
    eos = a.cu[n + 1];
    c_first = a.chunk_off[n];
  }
  const int64_t nchunks = (eos - bos + C - 1) / C;
  const int64_t top = nchunks - 1;
  auto chunk_nv = [&](int64_t it) { return (int)min((int64_t)C, eos - (bos + it * C)); };
  const bf16* qtb = reinterpret_cast<const bf16*>(a.qT);
  const bf16* wtb = reinterpret_cast<const bf16*>(a.wT);

  if (wid >= FW) {
    // ---- the loader waves.  Loader lw issues load i of each tile for i % FL = lw.  After B1: w^T and
    //      dv_local of chunk it (8 + 2 loads each), then the dv2 tile of chunk it + 1 out (2 stores);
    //      each waits for its loads before B2.  After B2: k, q^T, do of chunk it - 1 (8 + 8 + 2, and gc
    //      from loader 0 into the other buffer), its part of the L2 prefetch of chunk it - 2, then the
    //      snapshot of chunk it out (8 stores); each waits for its loads before the next B1.
    const int lw = wid - FW;
    const uint32_t RB = (uint32_t)H * FK * 2, VB = (uint32_t)H * V * 2;
    // the first half's tiles of chunk it: k and gc (needed at B1), then q^T and do (needed at B1h)
    auto load_a = [&](int64_t it, uint32_t gb) {
      const int64_t c = c_first + it, t0 = bos + it * C;
      const int nv = chunk_nv(it);
      const unsigned char* kb = reinterpret_cast<const unsigned char*>(a.k) + (size_t)((t0 * H + h) * FK) * 2;
      const unsigned char* qb = reinterpret_cast<const unsigned char*>(qtb + (c * H + h) * (int64_t)(FK * C));
      const unsigned char* db = reinterpret_cast<const unsigned char*>(a.do_) + (size_t)((t0 * H + h) * V + vt0) * 2;
#pragma unroll
      for (int j = 0; j < 32 / FL; ++j) ld_tile256(kb, RB, nv, FL * j + lw, base + K_OFF);
      if (lw == 0) dma4_(a.gc + t0 * H + h, (uint32_t)(l < nv ? l : 0) * (uint32_t)H * 4u, base + G_OFF + gb * C * 4);
#pragma unroll
      for (int j = 0; j < 32 / FL; ++j) ld_tile64<true>(qb, 128u, FK, FL * j + lw, base + QW_OFF);
#pragma unroll
      for (int j = 0; j < 8 / FL; ++j) ld_tile64<false>(db, VB, nv, FL * j + lw, base + DO_OFF);
    };
    auto load_b = [&](int64_t it) {
      const int64_t c = c_first + it, t0 = bos + it * C;
      const int nv = chunk_nv(it);
      const unsigned char* wb = reinterpret_cast<const unsigned char*>(wtb + (c * H + h) * (int64_t)(FK * C));
      const unsigned char* lb = reinterpret_cast<const unsigned char*>(a.dvl) + (size_t)((t0 * H + h) * V + vt0) * 2;
#pragma unroll
      for (int j = 0; j < 32 / FL; ++j) ld_tile64<true>(wb, 128u, FK, FL * j + lw, base + QW_OFF + W_REL);
#pragma unroll
      for (int j = 0; j < 8 / FL; ++j) ld_tile64<false>(lb, VB, nv, FL * j + lw, base + DL_OFF);
    };
    // L2 prefetch of chunk it: one 4-byte load per 128-byte line; the shared k, q^T, w^T lines split
    // over the head's V tiles by quarter (loaders 0-2), this tile's do and dv_local rows (loader 3)
    const int pf_q = (vt0 / FVT) & 3;
    auto prefetch = [&](int64_t it) {
      const int64_t c = c_first + it, t0 = bos + it * C;
      const int nv = chunk_nv(it);
      const uint32_t pf = base + PF_OFF;
      if (lw == 0) {
        const int r = 16 * pf_q + (l >> 2);
        dma4_(reinterpret_cast<const unsigned char*>(a.k) + (size_t)((t0 * H + h) * FK) * 2,
              (uint32_t)(r < nv ? r : 0) * RB + 128u * (l & 3), pf);
      } else if (lw == 1) {
        dma4_(qtb + (c * H + h) * (int64_t)(FK * C), 128u * (64 * pf_q + l), pf);
      } else if (lw == 2) {
        dma4_(wtb + (c * H + h) * (int64_t)(FK * C), 128u * (64 * pf_q + l), pf);
      } else {
        const uint32_t off = (uint32_t)(l < nv ? l : 0) * VB;
        dma4_(reinterpret_cast<const unsigned char*>(a.do_) + (size_t)((t0 * H + h) * V + vt0) * 2, off, pf);
        dma4_(reinterpret_cast<const unsigned char*>(a.dvl) + (size_t)((t0 * H + h) * V + vt0) * 2, off, pf);
      }
    };
    // LDS tile rows (128 bytes, swizzle swz_s) out to HBM: rows 8 i .. 8 i + 7 for i % FL = lw
    auto tile_row = [&](uint32_t off, int r) {
      return *reinterpret_cast<const lds_u32x4*>(reinterpret_cast<lds_b*>(base + off) + 128 * r +
                                                 16 * ((l & 7) ^ swz_s(r)));
    };
    auto store_dv = [&](int64_t it) {
      const int64_t t0 = bos + it * C;
      const int nv = chunk_nv(it);
#pragma unroll
      for (int j = 0; j < 8 / FL; ++j) {
        const int t = 8 * (FL * j + lw) + (l >> 3);
        const u32x4 x = tile_row(DV_OFF, t);
        if (t < nv)
          *reinterpret_cast<u32x4*>(reinterpret_cast<unsigned char*>(a.dv2) + (((t0 + t) * H + h) * V + vt0 + 8 * (l & 7)) * 2) = x;
      }
    };
    auto store_snap = [&](int64_t it) {
      const int64_t c = c_first + it;
#pragma unroll
      for (int j = 0; j < 32 / FL; ++j) {
        const int d = 8 * (FL * j + lw) + (l >> 3);
        const u32x4 x = tile_row(SNAP_OFF, d);
        *reinterpret_cast<u32x4*>(reinterpret_cast<unsigned char*>(a.dh) + (((c * H + h) * FK + d) * V + vt0 + 8 * (l & 7)) * 2) = x;
      }
    };
    if (nchunks > 0) {
      load_a(top, 0u);
      if (top >= 1) prefetch(top - 1);
    }
    wait_all_loads();
    // vmcnt counts in issue order; the waits below name how many of this wave's operations issued after
    // the ones waited for may still be in flight: the q^T / do loads (10), the prefetch (1, loader 3: 2),
    // the dv2 stores (2), the w^T / dv_local loads (10), the snapshot stores (8).  The snapshot leaves
    // after B1h, a half step before the next chunk's k loads: issued beside them (after B2) its stores
    // held those loads back by about the length of the second half (measured).
    static_assert(32 / FL == 8 && 8 / FL == 2, "the wait counts below assume four loader waves");
    for (int64_t it = top; it >= 0; --it) {
      const uint32_t gb = (uint32_t)((top - it) & 1);
      f_barrier();                                        // B1
      if (it < top) {
        store_dv(it + 1);                                 // the stores first, then this half's loads
        load_b(it);
        if (it >= 1) {                                    // the previous step prefetched chunk it - 1
          if (lw == 3) wait_loads_but<2 + 2 + 10>();
          else wait_loads_but<1 + 2 + 10>();
        } else {
          wait_loads_but<2 + 10>();
        }
      } else {
        load_b(it);
        wait_loads_but<10>();                             // the prologue's loads are complete
      }
      f_barrier();                                        // B1h: the snapshot of chunk it is in LDS
      store_snap(it);
      wait_loads_but<8>();
      f_barrier();                                        // B2
      if (it > 0) {
        load_a(it - 1, gb ^ 1u);
        if (it > 1) {
          prefetch(it - 2);
          if (lw == 3) wait_loads_but<10 + 2>();
          else wait_loads_but<10 + 1>();
        } else {
          wait_loads_but<10>();
        }
      }
    }
    f_barrier();                                          // dv2 of the first chunk is in LDS
    if (nchunks > 0) store_dv(0);
    wait_all_loads();                                     // no direct load outlives the workgroup's LDS
    return;
  }

  // ---- the compute waves: wave wid owns value columns vt0 + 16 wid .. + 15
  const int vcol = vt0 + 16 * wid + lc;
  // dh[kt][j] = dh[32 (kt / 2) + 8 lg + 4 (kt % 2) + j][vcol] (the paired row order)
  f32x4 dh[16];
#pragma unroll
  for (int kt = 0; kt < 16; ++kt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t off = (((int64_t)n * H + h) * FK + 32 * (kt >> 1) + 8 * lg + 4 * (kt & 1) + j) * V + vcol;
      dh[kt][j] = a.dht ? a.dht[off] : 0.f;
    }
  // lane addresses: kq[k] the k tile (row rowA(0, lc), chunk 4 ks + lg for ks % 4 = k; ks + 4 adds 256
  // bytes, tile tm adds rowa_off(tm, 512)); tq[ks] the q^T tile (row rowA(0, lc), chunk 4 ks + lg; tile
  // kt adds rowa_off(kt, 128), w^T at + W_REL); vt the transposed reads of the do tile (rows 8 lg +
  // lc / 4, columns 16 wid + 4 (lc % 4); dv_local at + DL_OFF - DO_OFF); sw the 2-byte writes of row
  // 8 lg, column 16 wid + lc of the snapshot tile (dv2 tile at + DV_OFF - SNAP_OFF)
  const int r0 = 8 * (lc >> 2) + (lc & 3);
  uint32_t kq[4], tq[2];
#pragma unroll
  for (int k = 0; k < 4; ++k) kq[k] = base + K_OFF + 512 * r0 + 16 * ((4 * k + lg) ^ swz_wq(r0));
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) tq[ks] = base + QW_OFF + 128 * r0 + 16 * ((4 * ks + lg) ^ swz_a(r0));
  uint32_t vt, sw;
  {
    const int rv = 8 * lg + (lc >> 2), cv = 16 * wid + 4 * (lc & 3);
    vt = base + DO_OFF + 128 * rv + 16 * ((cv >> 3) ^ swz_v(rv)) + 2 * (cv & 7);
    const int cs = 16 * wid + lc;
    sw = base + SNAP_OFF + 128 * (8 * lg) + 16 * ((cs >> 3) ^ swz_s(8 * lg)) + 2 * (cs & 7);
  }
  constexpr uint32_t DL_REL = DL_OFF - DO_OFF, DV_REL = DV_OFF - SNAP_OFF;
  const float* s_g = reinterpret_cast<const float*>(smem + G_OFF);

  for (int64_t it = top; it >= 0; --it) {
    const uint32_t gb = (uint32_t)((top - it) & 1);
    const int nv = chunk_nv(it);
    f_barrier();                                          // B1: k, gc of chunk it
    const float* G = s_g + gb * C;
    Frag<bf16> ka[2][4];
    auto read_k = [&](int g, Frag<bf16>(&k4)[4]) {
#pragma unroll
      for (int tm = 0; tm < 4; ++tm) k4[tm] = ld128(kq[g & 3], 256u * (g >> 2) + rowa_off(tm, 512));
    };
    read_k(0, ka[0]);
    const float gl = G[nv - 1];
    f32x4 gv[4];                                          // gc of tokens 32 (i / 2) + 8 lg + 4 (i % 2) + j
#pragma unroll
    for (int i = 0; i < 4; ++i) gv[i] = *reinterpret_cast<const f32x4*>(G + 32 * (i >> 1) + 8 * lg + 4 * (i & 1));
    f32x4 kd[4];
#pragma unroll
    for (int tm = 0; tm < 4; ++tm) kd[tm] = f32x4{0.f, 0.f, 0.f, 0.f};
    // k bf16(dh), 32 rows of dh per group (their bf16 values: the B operand and the snapshot); operand
    // reads one group ahead
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      if (g + 1 < 8) read_k(g + 1, ka[(g + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
      const Frag<bf16> hb = pack_acc(dh[2 * g], dh[2 * g + 1]);
#pragma unroll
      for (int tm = 0; tm < 4; ++tm) mma(kd[tm], ka[g & 1][tm], hb);
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int j = 0; j < 4; ++j) lds_st16(sw, rowa_off(2 * g + x, 128) + 128u * j, hb.v[4 * x + j]);
      __builtin_amdgcn_sched_barrier(0);
    }
    f_barrier();                                          // B1h: q^T, do of chunk it
    Frag<bf16> xr[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) xr[ks] = frag2(ldtr(vt, 4096u * ks), ldtr(vt, 4096u * ks + 512u));
    Frag<bf16> qa[2][4];
    auto read_q = [&](int g, Frag<bf16>(&q4)[4]) {
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) q4[2 * x + ks] = ld128(tq[ks], rowa_off(2 * g + x, 128));
    };
    read_q(0, qa[0]);
    // x = do exp(gc) scale (tokens 32 ks + 8 lg + e, 0 past the chunk's end) as hi + lo
    Frag<bf16> xh[2], xl[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int t = 32 * ks + 8 * lg + e;
        const float x = t < nv ? (float)xr[ks].v[e] * (gexp(gv[2 * ks + (e >> 2)][e & 3]) * a.scale) : 0.f;
        const bf16 hi = (bf16)x;
        xh[ks].v[e] = hi;
        xl[ks].v[e] = (bf16)(x - (float)hi);
      }
    const float eg = gexp(gl);
    // dh = exp(g_last) dh + q^T x, 32 rows per group, operand reads one group ahead
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      if (g + 1 < 8) read_q(g + 1, qa[(g + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        dh[2 * g + x] *= eg;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          mma(dh[2 * g + x], qa[g & 1][2 * x + ks], xh[ks]);
          mma(dh[2 * g + x], qa[g & 1][2 * x + ks], xl[ks]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    f_barrier();                                          // B2: w^T, dv_local of chunk it

    // dv2 = k bf16(dh) exp(g_last - gc) + dv_local (rows 32 (tm / 2) + 8 lg + 4 (tm % 2) + j)
    u32x2 dl[4];
#pragma unroll
    for (int tm = 0; tm < 4; ++tm) dl[tm] = ldtr(vt, DL_REL + rowa_off(tm, 128));
    Frag<bf16> wa[2][8];
    auto read_w = [&](int g4, Frag<bf16>(&w8)[8]) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) w8[2 * q + ks] = ld128(tq[ks], W_REL + rowa_off(4 * g4 + q, 128));
    };
    read_w(0, wa[0]);
    f32x4 dv[4];
#pragma unroll
    for (int tm = 0; tm < 4; ++tm) {
      const float d4[4] = {__uint_as_float(dl[tm][0] << 16), __uint_as_float(dl[tm][0] & 0xffff0000u),
                           __uint_as_float(dl[tm][1] << 16), __uint_as_float(dl[tm][1] & 0xffff0000u)};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = 32 * (tm >> 1) + 8 * lg + 4 * (tm & 1) + j;
        dv[tm][j] = t < nv ? kd[tm][j] * gexp(gl - gv[tm][j]) + d4[j] : 0.f;
      }
    }
    Frag<bf16> nd[2];                                     // -bf16(dv2) as the update's B operand
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) nd[ks] = pack_acc(-dv[2 * ks], -dv[2 * ks + 1]);
#pragma unroll
    for (int tm = 0; tm < 4; ++tm)
#pragma unroll
      for (int j = 0; j < 4; ++j) lds_st16(sw, DV_REL + rowa_off(tm, 128) + 128u * j, (bf16)dv[tm][j]);
    // dh -= w^T bf16(dv2)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      if (g4 + 1 < 4) read_w(g4 + 1, wa[(g4 + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) mma(dh[4 * g4 + q], wa[g4 & 1][2 * q + ks], nd[ks]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  f_barrier();                                            // dv2 of the first chunk is in LDS for the loaders

  if (a.dh0) {
#pragma unroll
    for (int kt = 0; kt < 16; ++kt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t off = (((int64_t)n * H + h) * FK + 32 * (kt >> 1) + 8 * lg + 4 * (kt & 1) + j) * V + vcol;
        a.dh0[off] = dh[kt][j];
      }
  }
}

// ---------------------------------------------------------------------------
// dq, dk, dw, dg for K = 256, bf16 (fla ops/common/chunk_o.py:147-326 with USE_G and USE_DW): one
// workgroup of eight waves per (chunk, head).  Wave w owns K rows 32 w .. 32 w + 31: it reads those
// rows of h and dh once, straight from global memory as A operands, while do, dv2 and v_new pass
// through LDS in 64-column blocks (two buffers, direct loads) shared by the eight waves.  The
// products are formed transposed ([d][t] tiles), so a lane stores 4 consecutive d of one token.
//
//   ds  = mask_{i>=j, i<nv}(do v_new^T exp(g_i - g_j)) scale      rounded to bf16 for its products
//   dq  = (h do)^T exp(gc) scale + ds k
//   dk  = (dh v_new)^T exp(g_last - gc) + ds^T q                  (dk1 + dk2, the WY stage adds more)
//   dw  = -(h dv2)^T
//   dg  = rowsum(ds2) - colsum(ds2) + sum_d (dq1 q - dk1 k), ds2 = ds (q k^T); the last row adds
//         sum dk1 k + exp(g_last) sum h dh
//
// Tiles with natural rows read as b128 row pieces: q, k [64][256] with chunk c of row r at
// c ^ swz_n(r), the 64-column blocks [64][64] at c ^ swz_v(r); both give the 16 lanes of a pass
// distinct bank positions for rows 16 x + lc and chunks 4 ks + lg.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int swz_n(int r) { return ((r & 1) << 1) | (((r >> 1) & 1) << 2) | (((r >> 3) & 1) << 3); }

constexpr int DQ_NW = 8;
constexpr int DQ_NT = DQ_NW * WAVE;

template <int K, int NB>
struct DqLds {
  static constexpr uint32_t RB = K * 2;                   // q / k row bytes
  static constexpr uint32_t Q_OFF = 0;                    // q [64][K]
  static constexpr uint32_t K_OFF = C * RB;               // k [64][K]
  static constexpr uint32_t BLK_OFF = 2 * C * RB;         // NB buffers of do, dv2, v_new [64][64]
  static constexpr uint32_t TILE = C * C * 2;
  static constexpr uint32_t BLK = 3 * TILE;
  static constexpr uint32_t DS_OFF = BLK_OFF + NB * BLK;  // bf16(ds) [64][64]
  static constexpr uint32_t G_OFF = DS_OFF + TILE;        // gc [64]
  static constexpr uint32_t ROW_OFF = G_OFF + C * 4;      // ds2 row sums per lower tile [10][16]
  static constexpr uint32_t COL_OFF = ROW_OFF + 10 * 16 * 4;   // ds2 column sums per lower tile [10][16]
  static constexpr uint32_t DGT_OFF = COL_OFF + 10 * 16 * 4;   // sum_d (dq1 q - dk1 k) per wave [8][64]
  static constexpr uint32_t SC_OFF = DGT_OFF + DQ_NW * C * 4;  // per wave: sum dk1 k [8], sum h dh [8]
  static constexpr uint32_t L2_OFF = SC_OFF + 2 * DQ_NW * 4;   // the L2 backward's sum_d dq q per wave [8][64]
  static constexpr uint32_t TOTAL = L2_OFF + DQ_NW * C * 4;
};

// instruction i of a [64][K] tile with natural rows (1 KB: rows (1024 / 2K) i ..; chunk c of row r at
// c ^ swz_n(r), which for 256- and 512-byte rows gives the 16 lanes of a b128 pass distinct banks)
template <int K>
__device__ __forceinline__ void ld_rows(const unsigned char* base, uint32_t row_bytes, int nv, int i, uint32_t dst) {
  constexpr int CPR = K / 8;                              // 16-byte chunks per row
  const int l = lane_id(), r = (64 / CPR) * i + l / CPR, pos = l % CPR;
  const uint32_t rr = r < nv ? (uint32_t)r : 0u;
  dma16_(base, rr * row_bytes + 16u * (pos ^ swz_n(r)), dst + 1024u * i);
}

__device__ __forceinline__ float wsum_lg(float x) {
  x += __shfl_xor(x, 16, WAVE);
  x += __shfl_xor(x, 32, WAVE);
  return x;
}
__device__ __forceinline__ float wsum16(float x) {
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) x += __shfl_xor(x, o, WAVE);
  return x;
}
__device__ __forceinline__ float wsum64(float x) {
#pragma unroll
  for (int o = 1; o < WAVE; o <<= 1) x += __shfl_xor(x, o, WAVE);
  return x;
}

// NB = 2: the next value block's tiles (and h / dh fragments) load into the other buffer during this
// block's products; NB = 1 (dk = 128: 68 KB, two workgroups per CU, each hiding the other's loads):
// after them.
template <int K, int NB>
__global__ __launch_bounds__(DQ_NT) __attribute__((amdgpu_waves_per_eu(NB == 1 ? 4 : 1))) void wide_dqkwg_kernel(
    BwdArgs a, int V) {
  using L = DqLds<K, NB>;
  constexpr uint32_t RB = L::RB, Q_OFF = L::Q_OFF, K_OFF = L::K_OFF, BLK_OFF = L::BLK_OFF, TILE = L::TILE,
                     BLK = L::BLK, DS_OFF = L::DS_OFF, G_OFF = L::G_OFF, ROW_OFF = L::ROW_OFF,
                     COL_OFF = L::COL_OFF, DGT_OFF = L::DGT_OFF, SC_OFF = L::SC_OFF;
  constexpr int RW = K / DQ_NW, DT = RW / 16;              // K rows per wave, their 16-row tiles
  __shared__ __align__(16) unsigned char smem[L::TOTAL];
  const uint32_t base = lds_u32(smem);
  const int h = blockIdx.y, H = a.H;
  const int64_t c = blockIdx.x;
  const ChunkLoc loc = locate_chunk(c, a.cu, a.chunk_off, a.N, a.T);
  if (!loc.ok) return;
  const int64_t t0 = loc.t0;
  const int nv = loc.nv;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE), l = lane_id(), lg = l >> 4, lc = l & 15;
  const int nvb = V / C;                                   // 64-column blocks
  const uint32_t RBg = (uint32_t)H * K * 2, VB = (uint32_t)H * V * 2;   // global row strides
  const unsigned char* dob = reinterpret_cast<const unsigned char*>(a.do_) + (size_t)((t0 * H + h) * V) * 2;
  const unsigned char* dvb = reinterpret_cast<const unsigned char*>(a.dv2) + (size_t)((t0 * H + h) * V) * 2;
  const unsigned char* vnb = reinterpret_cast<const unsigned char*>(a.vn) + (size_t)((t0 * H + h) * V) * 2;
  // block vb of do, dv2, v_new into buffer P: 24 loads, 3 per wave
  auto load_blk = [&](int vb, uint32_t P) {
    const uint32_t dst = base + BLK_OFF + P * BLK;
    ld_tile64<false>(dob + (size_t)vb * C * 2, VB, nv, wid, dst);               // rows 8 wid .. + 7 of each
    ld_tile64<false>(dvb + (size_t)vb * C * 2, VB, nv, wid, dst + TILE);
    ld_tile64<false>(vnb + (size_t)vb * C * 2, VB, nv, wid, dst + 2 * TILE);
  };
  {
    const unsigned char* qb = reinterpret_cast<const unsigned char*>(a.q) + (size_t)((t0 * H + h) * K) * 2;
    const unsigned char* kb = reinterpret_cast<const unsigned char*>(a.k) + (size_t)((t0 * H + h) * K) * 2;
#pragma unroll
    for (int j = 0; j < K / 8 / DQ_NW; ++j) ld_rows<K>(qb, RBg, nv, DQ_NW * j + wid, base + Q_OFF);
#pragma unroll
    for (int j = 0; j < K / 8 / DQ_NW; ++j) ld_rows<K>(kb, RBg, nv, DQ_NW * j + wid, base + K_OFF);
    load_blk(0, 0u);
    if (wid == 0) dma4_(a.gc + t0 * H + h, (uint32_t)(l < nv ? l : 0) * (uint32_t)H * 4u, base + G_OFF);
  }
  // this wave's rows of h and dh: A operands of rows d = 32 wid + 16 dt + lc, columns 64 vb + 32 ks + 8 lg ..
  const bf16* hrow = reinterpret_cast<const bf16*>(a.h) + ((c * H + h) * K + RW * wid + lc) * (int64_t)V + 8 * lg;
  const bf16* dhrow = reinterpret_cast<const bf16*>(a.dh) + ((c * H + h) * K + RW * wid + lc) * (int64_t)V + 8 * lg;
  auto load_hd = [&](int vb, Frag<bf16>(&hf)[2 * DT], Frag<bf16>(&df)[2 * DT]) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int64_t off = 16 * dt * (int64_t)V + C * vb + 32 * ks;
        hf[2 * dt + ks].v = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(hrow + off));
        df[2 * dt + ks].v = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(dhrow + off));
      }
  };
  Frag<bf16> hf[2][2 * DT], df[2][2 * DT];
  load_hd(0, hf[0], df[0]);
  wait_all_loads();
  f_barrier();

  // the lower 16 x 16 tiles (tm >= tn) of ds this wave accumulates: tile wid, and tile wid + 8 for waves 0, 1
  const int ntile = wid < 2 ? 2 : 1;
  auto tile_mn = [](int idx, int& tm, int& tn) {
    tm = idx < 1 ? 0 : idx < 3 ? 1 : idx < 6 ? 2 : 3;
    tn = idx - tm * (tm + 1) / 2;
  };
  const int r0 = lc;                                       // natural rows 16 x + lc
  const uint32_t qrd = base + Q_OFF + RB * r0, krd = base + K_OFF + RB * r0;
  // q k^T of the ds tiles (B1 data: q, k)
  f32x4 aqk[2], dsa[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    aqk[s] = f32x4{0.f, 0.f, 0.f, 0.f};
    dsa[s] = aqk[s];
    if (s < ntile) {
      int tm, tn;
      tile_mn(wid + 8 * s, tm, tn);
#pragma unroll
      for (int ks = 0; ks < K / 32; ++ks) {
        const uint32_t co = 16u * ((4 * ks + lg) ^ swz_n(r0));
        mma(aqk[s], ld128(qrd, RB * 16 * tm + co), ld128(krd, RB * 16 * tn + co));
      }
    }
  }

  // the main products over the value columns
  f32x4 aq[DT][4], aw[DT][4], ak[DT][4];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) aq[dt][tt] = aw[dt][tt] = ak[dt][tt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float hdh = 0.f;
  const uint32_t brd = base + BLK_OFF + 128 * r0;          // block tiles, row r0
  auto block = [&](auto PP, int vb) {
    constexpr uint32_t P = decltype(PP)::value;            // register set of the h / dh fragments
    constexpr uint32_t PB = NB == 2 ? P : 0u;              // LDS buffer of the block's tiles
    if constexpr (NB == 2) {
      if (vb + 1 < nvb) {
        load_blk(vb + 1, P ^ 1u);
        load_hd(vb + 1, hf[P ^ 1u], df[P ^ 1u]);
      }
    }
    const uint32_t bb = brd + PB * BLK;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      Frag<bf16> fdo[2], fdv[2], fvn[2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const uint32_t o = 128u * 16 * tt + 16u * ((4 * ks + lg) ^ swz_v(r0));
        fdo[ks] = ld128(bb, o);
        fdv[ks] = ld128(bb, TILE + o);
        fvn[ks] = ld128(bb, 2 * TILE + o);
      }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          mma(aq[dt][tt], hf[P][2 * dt + ks], fdo[ks]);    // sum_v h[d][v] do[t][v]
          mma(aw[dt][tt], hf[P][2 * dt + ks], fdv[ks]);    // sum_v h[d][v] dv2[t][v]
          mma(ak[dt][tt], df[P][2 * dt + ks], fvn[ks]);    // sum_v dh[d][v] v_new[t][v]
        }
    }
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      if (s < ntile) {
        int tm, tn;
        tile_mn(wid + 8 * s, tm, tn);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const uint32_t o = 16u * ((4 * ks + lg) ^ swz_v(r0));
          mma(dsa[s], ld128(bb, 128u * 16 * tm + o), ld128(bb, 2 * TILE + 128u * 16 * tn + o));   // do v_new^T
        }
      }
    }
#pragma unroll
    for (int f = 0; f < 2 * DT; ++f)
#pragma unroll
      for (int e = 0; e < 8; ++e) hdh += (float)hf[P][f].v[e] * (float)df[P][f].v[e];
    if constexpr (NB == 1) {                               // (the h / dh fragments too: fewer registers)
      if (vb + 1 < nvb) {
        load_hd(vb + 1, hf[P ^ 1u], df[P ^ 1u]);
        f_barrier();                                       // every wave is done with this block's tiles
        load_blk(vb + 1, 0u);
      }
    }
    wait_all_loads();
    f_barrier();
  };
  for (int vb = 0; vb < nvb; vb += 2) {
    block(std::integral_constant<uint32_t, 0>{}, vb);
    if (vb + 1 < nvb) block(std::integral_constant<uint32_t, 1>{}, vb + 1);
  }

  // ds (rounded into LDS) and the row / column sums of ds2 = ds (q k^T), per tile
  const float* s_g = reinterpret_cast<const float*>(smem + G_OFF);
  float* s_row = reinterpret_cast<float*>(smem + ROW_OFF);
  float* s_col = reinterpret_cast<float*>(smem + COL_OFF);
  float* s_dgt = reinterpret_cast<float*>(smem + DGT_OFF);
  float* s_sc = reinterpret_cast<float*>(smem + SC_OFF);
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    if (s < ntile) {
      const int idx = wid + 8 * s;
      int tm, tn;
      tile_mn(idx, tm, tn);
      const int j = 16 * tn + lc;
      float colp = 0.f;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int i = 16 * tm + 4 * lg + jj;
        const float ds = (i >= j && i < nv) ? dsa[s][jj] * gexp(s_g[i] - s_g[j]) * a.scale : 0.f;
        const float ds2 = ds * aqk[s][jj];
        colp += ds2;
        const float rs = wsum16(ds2);
        if (lc == 0) s_row[idx * 16 + 4 * lg + jj] = rs;
        *reinterpret_cast<__attribute__((address_space(3))) uint16_t*>(
            reinterpret_cast<lds_b*>(base + DS_OFF) + 128 * i + 16 * ((j >> 3) ^ swz_v(i)) + 2 * (j & 7)) =
            __builtin_bit_cast(uint16_t, (bf16)ds);
      }
      colp = wsum_lg(colp);
      if (lg == 0) s_col[idx * 16 + lc] = colp;
    }
  }
  if (wid >= 2) {                                          // the six upper tiles of ds are zero
    const int u = wid - 2, tm = u < 3 ? 0 : u < 5 ? 1 : 2, tn = u < 3 ? u + 1 : u < 5 ? u - 1 : 3;
    const int j = 16 * tn + lc;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int i = 16 * tm + 4 * lg + jj;
      *reinterpret_cast<__attribute__((address_space(3))) uint16_t*>(
          reinterpret_cast<lds_b*>(base + DS_OFF) + 128 * i + 16 * ((j >> 3) ^ swz_v(i)) + 2 * (j & 7)) = 0;
    }
  }
  f_barrier();

  // dq = dq1 + ds k, dk = dk1 + ds^T q, dw; the state terms of dg
  const float gl = s_g[nv - 1];
  float dglp = 0.f;
  bf16* dq_out = reinterpret_cast<bf16*>(a.dq);
  bf16* dk_out = reinterpret_cast<bf16*>(a.dk1);
  bf16* dw_out = reinterpret_cast<bf16*>(a.dw);
  // with the in-op L2 norm (a.rq): dq of the normalised row y_q = q, rounded as the two-step form
  // stores it, is kept here until the row sums sum_d dq y_q are complete across the waves
  const bool l2q = a.rq != nullptr;
  float* s_l2 = reinterpret_cast<float*>(smem + L::L2_OFF);
  u32x2 dqy[4][DT];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    const int t = 16 * tt + lc;
    const float egs = gexp(s_g[t]) * a.scale;
    const float gate = t < nv ? gexp(gl - s_g[t]) : 0.f;
    float dgt = 0.f, dqq = 0.f;
    // B operands: row t of ds (dq's ds k, K = t'), column t of ds read transposed (dk's ds^T q, K = i)
    Frag<bf16> bq[2], bk[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      bq[ks] = ld128(base + DS_OFF + 128 * t, 16u * ((4 * ks + lg) ^ swz_v(t)));
      const int ri = 32 * ks + 8 * lg + (lc >> 2), ci = 16 * tt + 4 * (lc & 3);
      const uint32_t ta = base + DS_OFF + 128 * ri + 16 * ((ci >> 3) ^ swz_v(ri)) + 2 * (ci & 7);
      bk[ks] = frag2(ldtr(ta, 0), ldtr(ta, 512u));       // rows ri + 4: the same swizzle (bits 1, 3)
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const int d0 = RW * wid + 16 * dt, k0 = d0 + 4 * lg;
      const u32x2 qw = *reinterpret_cast<const lds_u32x2*>(reinterpret_cast<lds_b*>(base + Q_OFF) + RB * t +
                                                             16 * ((k0 >> 3) ^ swz_n(t)) + 2 * (k0 & 7));
      const u32x2 kw = *reinterpret_cast<const lds_u32x2*>(reinterpret_cast<lds_b*>(base + K_OFF) + RB * t +
                                                             16 * ((k0 >> 3) ^ swz_n(t)) + 2 * (k0 & 7));
      const float qv[4] = {__uint_as_float(qw[0] << 16), __uint_as_float(qw[0] & 0xffff0000u),
                           __uint_as_float(qw[1] << 16), __uint_as_float(qw[1] & 0xffff0000u)};
      const float kv[4] = {__uint_as_float(kw[0] << 16), __uint_as_float(kw[0] & 0xffff0000u),
                           __uint_as_float(kw[1] << 16), __uint_as_float(kw[1] & 0xffff0000u)};
      f32x4 dq = aq[dt][tt] * egs, dk = ak[dt][tt] * gate;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        dgt += dq[j] * qv[j] - kv[j] * dk[j];
        dglp += dk[j] * kv[j];
      }
      // A operands k^T, q^T: rows d0 + lc, K = t' = 32 ks + 8 lg .. + 7 (transposed reads of the row tiles)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int rt = 32 * ks + 8 * lg + (lc >> 2), ct = d0 + 4 * (lc & 3);
        const uint32_t oa = RB * rt + 16 * ((ct >> 3) ^ swz_n(rt)) + 2 * (ct & 7);
        const uint32_t ob = RB * (rt + 4) + 16 * ((ct >> 3) ^ swz_n(rt + 4)) + 2 * (ct & 7);
        mma(dq, frag2(ldtr(base + K_OFF + oa, 0), ldtr(base + K_OFF + ob, 0)), bq[ks]);
        mma(dk, frag2(ldtr(base + Q_OFF + oa, 0), ldtr(base + Q_OFF + ob, 0)), bk[ks]);
      }
      if (l2q) {
        dqy[tt][dt] = u32x2{cv_pack(dq[0], dq[1]), cv_pack(dq[2], dq[3])};
#pragma unroll
        for (int j = 0; j < 4; ++j) dqq = fmaf(j & 1 ? cv_hi(dqy[tt][dt][j >> 1]) : cv_lo(dqy[tt][dt][j >> 1]), qv[j], dqq);
      }
      if (t < nv) {
        const int64_t o = ((t0 + t) * H + h) * (int64_t)K + k0;
        if (!l2q) st4<bf16>(dq_out + o, dq[0], dq[1], dq[2], dq[3]);
        st4<bf16>(dk_out + o, dk[0], dk[1], dk[2], dk[3]);
        st4<bf16>(dw_out + o, -aw[dt][tt][0], -aw[dt][tt][1], -aw[dt][tt][2], -aw[dt][tt][3]);
      }
    }
    dgt = wsum_lg(dgt);
    if (lg == 0) s_dgt[wid * C + t] = dgt;
    if (l2q) {
      dqq = wsum_lg(dqq);
      if (lg == 0) s_l2[wid * C + t] = dqq;
    }
  }
  dglp = wsum64(dglp);
  hdh = wsum64(hdh);
  if (l == 0) {
    s_sc[wid] = dglp;
    s_sc[DQ_NW + wid] = hdh;
  }
  f_barrier();
  // the L2 norm's backward of q (l2norm.py:132-154): dq_raw = dq rstd - (sum_d dq y_q) y_q rstd, the
  // row sum added over the eight waves in a fixed order
  if (l2q) {
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const int t = 16 * tt + lc;
      if (t < nv) {
        float dot = s_l2[t];
#pragma unroll
        for (int w = 1; w < DQ_NW; ++w) dot += s_l2[w * C + t];
        const float rs = a.rq[(t0 + t) * H + h];
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const int k0 = RW * wid + 16 * dt + 4 * lg;
          const u32x2 qw = *reinterpret_cast<const lds_u32x2*>(reinterpret_cast<lds_b*>(base + Q_OFF) + RB * t +
                                                                 16 * ((k0 >> 3) ^ swz_n(t)) + 2 * (k0 & 7));
          float x[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint32_t yw = dqy[tt][dt][j >> 1], qq = qw[j >> 1];
            const float y = j & 1 ? cv_hi(yw) : cv_lo(yw), qn = j & 1 ? cv_hi(qq) : cv_lo(qq);
            x[j] = y * rs - dot * qn * rs;
          }
          st4<bf16>(dq_out + ((t0 + t) * H + h) * (int64_t)K + k0, x[0], x[1], x[2], x[3]);
        }
      }
    }
  }
  if (threadIdx.x < C) {
    const int t = threadIdx.x;
    if (t < nv) {
      const int tm = t >> 4, r = t & 15;
      float row = 0.f, col = 0.f, dgt = 0.f;
      for (int tn = 0; tn <= tm; ++tn) row += s_row[(tm * (tm + 1) / 2 + tn) * 16 + r];
      for (int m = tm; m < 4; ++m) col += s_col[(m * (m + 1) / 2 + tm) * 16 + r];
#pragma unroll
      for (int w = 0; w < DQ_NW; ++w) dgt += s_dgt[w * C + t];
      float dg = row - col + dgt;
      if (t == nv - 1) {
        float sl = 0.f, sh = 0.f;
#pragma unroll
        for (int w = 0; w < DQ_NW; ++w) {
          sl += s_sc[w];
          sh += s_sc[DQ_NW + w];
        }
        dg += sl + sh * gexp(gl);
      }
      a.dg1[(t0 + t) * H + h] = dg;
    }
  }
}

}  // namespace

__global__ void marker_kernel() {}

bool wide_fused_supported(int compute_dtype, int qk_dtype, int K, int V) {
  return compute_dtype == DT_BF16 && qk_dtype == DT_BF16 && K == FK && V > 0 && V % FVT == 0;
}

int launch_marker(hipStream_t s) {
  hipLaunchKernelGGL(marker_kernel, dim3(1), dim3(WAVE), 0, s);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

bool wide_dhu_supported(int compute_dtype, int K, int V) {
  return compute_dtype == DT_BF16 && K == FK && V > 0 && V % FVT == 0;
}

int launch_wide_dhu(const BwdArgs& a, int V, hipStream_t s) {
  if (V % FVT != 0 || !a.qT || !a.wT || !a.dh || !a.dv2) return -2;
  const int total = a.N * a.H * (V / FVT);
  if (total == 0) return 0;
  const int grid = (total + 7) / 8 * 8;
  hipLaunchKernelGGL(wide_dhu_kernel, dim3(grid), dim3(NT_F + FL * WAVE), 0, s, a, V, total);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_wide_dqkwg(const BwdArgs& a, int K, int V, int64_t nc_grid, hipStream_t s) {
  if (V % C != 0 || a.H <= 0 || !(K == 128 || K == 256)) return -2;
  if (nc_grid <= 0) return 0;
  // dk = 128: one block buffer, two workgroups per CU (backward 2.633 -> 2.544 ms at config 2's shape,
  // 8 VGPRs spilled at four waves per SIMD), unless KAIROS_GDN_BWD_DQK_BUFS=2
  const char* e = std::getenv("KAIROS_GDN_BWD_DQK_BUFS");
  const bool two = e && e[0] == '2' && e[1] == 0;
  const dim3 grid((unsigned)nc_grid, (unsigned)a.H);
  if (K == 256) hipLaunchKernelGGL((wide_dqkwg_kernel<256, 2>), grid, dim3(DQ_NT), 0, s, a, V);
  else if (two) hipLaunchKernelGGL((wide_dqkwg_kernel<128, 2>), grid, dim3(DQ_NT), 0, s, a, V);
  else hipLaunchKernelGGL((wide_dqkwg_kernel<128, 1>), grid, dim3(DQ_NT), 0, s, a, V);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_wide_fused(const WideFusedArgs& a, int V, hipStream_t s) {
  if (V % FVT != 0 || a.N * a.H == 0) return -2;
  const int total = a.N * a.H * (V / FVT);
  const int grid = (total + 7) / 8 * 8;
  if (a.h_out) {
    if (!a.vn_out || a.ht || a.ngate) return -2;
    hipLaunchKernelGGL((wide_fused_kernel<true, false>), dim3(grid), dim3(NT_F + FL * WAVE), 0, s, a, V, total);
  } else if (a.ngate) {
    if (V > 8 * FVT || a.nss == nullptr) return -2;
    hipLaunchKernelGGL((wide_fused_kernel<false, true>), dim3(grid), dim3(NT_F + FL * WAVE), 0, s, a, V, total);
  } else {
    hipLaunchKernelGGL((wide_fused_kernel<false, false>), dim3(grid), dim3(NT_F + FL * WAVE), 0, s, a, V, total);
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace kgdn
