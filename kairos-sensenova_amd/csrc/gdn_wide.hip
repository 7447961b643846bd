// Fused state recurrence + output for K = 256 (the Kairos model's head dim), bf16 compute
// (fla ops/common/chunk_delta_h.py:52-224 followed by ops/common/chunk_o.py:41-128, with
// the state never leaving the workgroup).  The stage path stores a bf16 state snapshot per
// chunk (256 x V) for the output kernel to read back; at V = 512 that is 2.7 GB written and
// read per call.  Here one workgroup per (sequence, head, 64 value columns) walks the
// chunks, each of its four waves owning 16 state columns over all 256 rows (fp32, MFMA
// accumulator layout, in VGPRs), and per chunk computes
//
//   h      = bf16(S)                                          chunk_delta_h.py:129-139
//   v'     = u - w h                                          :141-157
//   o^T    = (h^T q^T exp(gc) + bf16(v')^T Aqk^T) scale       chunk_o.py:84-128
//   S      = exp(g_last) S + k^T (v' exp(g_last - gc))        chunk_delta_h.py:163-211
//
// with the same cast points as the stage kernels (h and v' rounded to bf16 where the reference
// stores them, Aqk rounded before its product).  Aqk = mask_{i>=j}(q k^T exp(gc_i - gc_j)) is
// state-independent and shared by the V tiles of a head; the prepare kernel forms it per (chunk,
// head) beforehand (beside w and u, while k is in its LDS), so the serial loop only reads it.
//
// Operand layouts: w, q and k of a chunk are staged in LDS as swizzled [64][256] bf16 tiles
// (swz_off<256>): w and q are read as row pieces in the accumulator K order (the order in which
// bf16(S) is packed from its accumulator tiles), k transposed (ds_read_b64_tr_b16) for the update.
// v' and the gated v' go from their accumulator tiles straight into MFMA operands.  o is computed
// transposed, so each lane stores 4 consecutive columns of one token.
#include <type_traits>

#include "gdn_common.hpp"
#include "gdn_kernels.h"

namespace kgdn {

namespace {

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int FK = 256;           // K
constexpr int FW = 4;             // waves per workgroup, 16 state columns each
constexpr int FVT = 16 * FW;      // value columns per workgroup
constexpr int NT_F = FW * WAVE;
constexpr int kSmallLoads = 6;    // direct loads per wave of a chunk's Aqk, Ai and v tiles (2 each)
constexpr int kPrefetchLoads = 1; // direct loads per wave of the L2 prefetch (w, q, k rows or Aqk lines)

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

__device__ __forceinline__ float lo16(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi16(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// ---------------------------------------------------------------------------
// the fused recurrence + output
// ---------------------------------------------------------------------------
// Direct global -> LDS loads (inline asm: the compiler does not track them, so the kernel waits
// for them explicitly with wait_all_loads before the barrier that publishes their data).  Lane l's
// 16 (4) bytes at base + off land at LDS address m0 + 16 l (4 l); base is wave-uniform.  s_nop 4:
// the hazard between the SGPR / M0 writes and the load that reads them.
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
__device__ __forceinline__ uint32_t lds_u32(const void* p) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}

// swizzle of the [64][64] Aqk tile (16-byte chunk c8 of row r sits at c8 ^ swz64(r)): the row
// pieces read for the product are conflict-free
__device__ __forceinline__ int swz64(int r) { return (((r >> 1) & 3) << 1) | ((r >> 3) & 1); }
// swizzle of the [64][256] tiles (swz_off<256>)
__device__ __forceinline__ int swz256(int r) { return ((r & 7) << 1) | ((r >> 3) & 1); }

typedef __attribute__((address_space(3))) unsigned char lds_b;
typedef short s16x4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4v lds_s16x4v;
typedef __attribute__((address_space(3))) u32x2 lds_u32x2;
typedef __attribute__((address_space(3))) f32x4 lds_f32x4;
typedef __attribute__((address_space(3))) float lds_f32;

// LDS reads at a lane byte address plus an offset that is a constant after unrolling (it lands
// in the instruction's offset field)
// (volatile: the compiler would otherwise pair reads that share a base into ds_read2st64_b64, whose
// register layout does not match the operand fragments, and then copy every fragment)
__device__ __forceinline__ u32x2 ld64(uint32_t a, uint32_t off) {
  return *reinterpret_cast<volatile const lds_u32x2*>(reinterpret_cast<lds_b*>(a) + off);
}
__device__ __forceinline__ u32x2 ldtr(uint32_t a, uint32_t off) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                       reinterpret_cast<lds_s16x4v*>(reinterpret_cast<lds_b*>(a) + off)));
}
__device__ __forceinline__ Frag<bf16> frag2(u32x2 a, u32x2 b) {
  Frag<bf16> f;
  f.v = __builtin_bit_cast(bf16x8, u32x4{a[0], a[1], b[0], b[1]});
  return f;
}

// Lane addresses of the per-step LDS reads, fixed for the whole sequence (the tiles sit at fixed
// places; the double-buffered ones differ by a constant).
//  row[h][k]: w row lc (and q at + (s_q - s_w)), the accumulator-order piece h (elements 4 lg ..
//    and 16 + 4 lg .. of a 32-deep step) of step ks with ks % 4 = k; step ks + 4 adds 256 bytes,
//    row tile tm adds tm * 8192.  Chunk position of piece h of step ks is 4 (ks ^ s2) + (y_h ^ s3)
//    with s = swz256(lc), y_a = lg / 2, y_b = 2 + lg / 2.
//  tra[k], trb[k]: the two ds_read_b64_tr_b16 of tr_frag<256>(k, ks, 16 tt) (rows r0 and r0 + 16 of
//    the 32-deep step) for tt % 8 = k; tt + 8 adds 256 bytes, ks adds 16384.
//  aq[ks][h]: Aqk row 16 tn + lc, piece h of step ks; tn adds 2048 bytes.
struct FAddr {
  uint32_t row[2][4];
  uint32_t tra[8], trb[8];
  uint32_t aq[2][2];
};

__device__ __forceinline__ void f_addr(FAddr& A, uint32_t w_lds, uint32_t k_lds, uint32_t a_lds) {
  const int l = lane_id(), lg = l >> 4, lc = l & 15, i = l & 15;
  {
    const int sw = swz256(lc), s2 = sw >> 2, s3 = sw & 3;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int y = 2 * h + (lg >> 1);
#pragma unroll
      for (int k = 0; k < 4; ++k)
        A.row[h][k] = w_lds + lc * 512 + 16 * (4 * (k ^ s2) + (y ^ s3)) + 8 * (lg & 1);
    }
  }
  {
    const int r0 = 4 * lg + (i >> 2);                    // row of the first read within a 32-row step
    const int sa = swz256(r0), sa1 = sa >> 1, za = ((i >> 1) & 1) ^ (sa & 1);
    const uint32_t base = k_lds + 512 * r0 + 8 * (i & 1);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      A.tra[k] = base + 16 * za + 32 * (k ^ sa1);
      A.trb[k] = A.tra[k] + 8192;                          // row r0 + 16 (the same swizzle)
    }
  }
  {
    const int s = swz64(lc);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int c8 = 4 * ks + 2 * h + (lg >> 1);
        A.aq[ks][h] = a_lds + lc * 128 + 16 * (c8 ^ s) + 8 * (lg & 1);
      }
  }
}

// Lane parts of the global offsets, fixed for the whole sequence.
struct FOff {
  uint32_t tile[2];           // [64][256] tile direct loads: row tid / 32 (+ 8 i), swizzled chunk, i even / odd
  uint32_t aqk[2];            // Aqk tile direct loads ([NC, H, 64, 64]), i = 0, 1
  uint32_t row64[2];          // [64][64] tiles of token-major rows (Ai, v): row p / 8, swizzled chunk, i = 0, 1
  int r64[2];                 // their rows
  uint32_t o;                 // o of lane: token lc, columns 4 lg .. (bytes from the wave's row-0 base)
};

__device__ __forceinline__ void f_off(FOff& F, int H, int V) {
  const int tid = threadIdx.x, l = lane_id(), lg = l >> 4, lc = l & 15;
  const uint32_t row_bytes = (uint32_t)H * FK * 2;
  const int r0 = tid >> 5, pos = tid & 31;
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const int c8 = pos ^ ((r0 << 1) | par);             // swz256(r0 + 8 i), r0 < 8
    F.tile[par] = (uint32_t)r0 * row_bytes + 16u * c8;
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int p = tid + 256 * i, r = p >> 3, ps = p & 7;
    F.aqk[i] = (uint32_t)(r * C + 8 * (ps ^ swz64(r))) * 2u;
    F.row64[i] = 16u * (uint32_t)(ps ^ swz64(r));
    F.r64[i] = r;
  }
  F.o = ((uint32_t)lc * (uint32_t)(H * V) + 4u * lg) * 2u;
}

// Direct loads of a swizzled [64][256] tile of the token-major tensor x (rows t0 .. t0 + 63 of
// head h).  Rows past the chunk's end read row 0: in w and q they only reach outputs of rows
// that are not stored and products with zero Aqk columns, in k only zero gated v' rows.
__device__ __forceinline__ void dma_tile256(const void* x, const FOff& F, int64_t t0, int nv, int h, int H,
                                            uint32_t dst) {
  const int tid = threadIdx.x, wid = tid / WAVE;
  const unsigned char* base = reinterpret_cast<const unsigned char*>(x) + ((t0 * H + h) * FK) * 2;
  const uint32_t row_bytes = (uint32_t)H * FK * 2;
  if (nv == C) {
#pragma unroll
    for (int i = 0; i < 8; ++i) dma16_(base + (size_t)(8 * i) * row_bytes, F.tile[i & 1], dst + 16u * (256 * i + 64 * wid));
  } else {
    const int r0 = tid >> 5;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = r0 + 8 * i;
      const uint32_t off = r < nv ? F.tile[i & 1] + (uint32_t)(8 * i) * row_bytes : F.tile[i & 1] - (uint32_t)r0 * row_bytes;
      dma16_(base, off, dst + 16u * (256 * i + 64 * wid));
    }
  }
}

// Direct loads of a swizzled [64][64] bf16 tile (swz64) whose token rows are row_bytes apart
// (rows past the chunk's end read row 0).
__device__ __forceinline__ void dma_tile64(const unsigned char* base, uint32_t row_bytes, const FOff& F, int nv,
                                           uint32_t dst) {
  const int wid = threadIdx.x / WAVE;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint32_t rr = F.r64[i] < nv ? (uint32_t)F.r64[i] : 0u;
    dma16_(base, rr * row_bytes + F.row64[i], dst + 16u * (256 * i + 64 * wid));
  }
}

__global__ __launch_bounds__(NT_F) void wide_fused_kernel(WideFusedArgs a, int V, int total_units) {
  // LDS: w and q of the chunk (adjacent: q reads are w reads + 32 KB), k of the chunk, and two
  // buffer sets of the chunk's small tiles: Aqk, Ai, the v tile of the workgroup's 64 columns, gc, beta
  __shared__ __align__(16) bf16 s_wq[2 * C * FK];
  __shared__ __align__(16) bf16 s_k[C * FK];
  __shared__ __align__(16) bf16 s_a[2 * C * C];
  __shared__ __align__(16) bf16 s_ai[2 * C * C];
  __shared__ __align__(16) bf16 s_v[2 * C * C];
  __shared__ __align__(16) float s_g[2 * C];
  __shared__ __align__(16) float s_b[2 * C];
  __shared__ __align__(16) float s_pf[WAVE];              // landing words of the L2 prefetch
  constexpr uint32_t QOFF = C * FK * 2, ABUF = C * C * 2, GBUF = C * 4;

  // XCD-aware order: the V tiles of one head run on one XCD and share its q, k, w, Aqk in L2
  const int per_xcd = gridDim.x / 8;
  const int o_idx = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (o_idx >= total_units) return;
  const int nvt = V / FVT;
  const int unit = o_idx / nvt;
  const int H = a.H;
  const int n = unit / H, h = unit % H;
  const int tid = threadIdx.x, wid = tid / WAVE, l = lane_id(), lg = l >> 4, lc = l & 15;
  const int vt0 = __builtin_amdgcn_readfirstlane((o_idx % nvt) * FVT);    // the workgroup's first column
  const int v0 = vt0 + 16 * wid;                          // this wave's first column
  const int vcol = v0 + lc;

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
  auto chunk_nv = [&](int64_t it) { return (int)min((int64_t)C, eos - (bos + it * C)); };

  // state: S[kt][j] = S[16 kt + 4 lg + j][vcol]
  f32x4 S[16];
#pragma unroll
  for (int kt = 0; kt < 16; ++kt) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float x = 0.f;
      if (a.h0) {
        const int64_t off = (((int64_t)n * H + h) * FK + 16 * kt + 4 * lg + j) * V + vcol;
        x = a.h0_dtype == DT_F32 ? reinterpret_cast<const float*>(a.h0)[off]
                                 : (float)reinterpret_cast<const bf16*>(a.h0)[off];
      }
      S[kt][j] = x;
    }
  }
  const uint32_t w_lds = lds_u32(s_wq), k_lds = lds_u32(s_k), a_lds = lds_u32(s_a), ai_lds = lds_u32(s_ai),
                 v_lds = lds_u32(s_v), g_lds = lds_u32(s_g), b_lds = lds_u32(s_b);
  FAddr A;
  f_addr(A, w_lds, k_lds, a_lds);
  FOff F;
  f_off(F, H, V);
  const bf16* aqb = reinterpret_cast<const bf16*>(a.aqk);
  unsigned char* ob = reinterpret_cast<unsigned char*>(a.o) + (size_t)v0 * 2;
  const uint32_t AI_OFF = ai_lds - a_lds;                 // Ai tiles share the Aqk lane addresses

  // the chunk's small tiles into buffer set B: Aqk, Ai, the v tile, gc (wave 0), beta (wave 1)
  auto dma_small = [&](int64_t c, int64_t t0, int nv, uint32_t B) {
    const unsigned char* ab = reinterpret_cast<const unsigned char*>(aqb + (c * H + h) * (int64_t)(C * C));
#pragma unroll
    for (int i = 0; i < 2; ++i) dma16_(ab, F.aqk[i], a_lds + B * ABUF + 16u * (256 * i + 64 * wid));
    dma_tile64(reinterpret_cast<const unsigned char*>(a.Ai) + (size_t)((t0 * H + h) * C) * 2, (uint32_t)H * C * 2, F,
               nv, ai_lds + B * ABUF);
    dma_tile64(reinterpret_cast<const unsigned char*>(a.v) + (size_t)((t0 * H + h) * V + vt0) * 2, (uint32_t)H * V * 2,
               F, nv, v_lds + B * ABUF);
    if (wid == 0) dma4_(a.gc + t0 * H + h, (uint32_t)(l < nv ? l : 0) * (uint32_t)H * 4u, g_lds + B * GBUF);
    if (wid == 1) dma4_(a.beta + t0 * H + h, (uint32_t)(l < nv ? l : 0) * (uint32_t)H * 4u, b_lds + B * GBUF);
  };
  // L2 prefetch of chunk (c, t0)'s w, q, k rows and Aqk tile: one 4-byte direct load per 128-byte
  // line into a scratch LDS word (shared by the waves: never read), so that the tile loads a step
  // later hit L2 instead of waiting for HBM.  The V tiles of a head share the XCD's L2, so each
  // workgroup touches a quarter of the lines (rows 16 (vt % 4) .. + 15): waves 0-2 one line per lane
  // of w, q, k, wave 3 16 lines of Aqk.  The address unit works per line, so a full prefetch per
  // workgroup would cost as much of it as the tile loads themselves.
  const uint32_t pf_lds = lds_u32(s_pf);
  const int pf_r = 16 * ((vt0 / FVT) & 3);
  auto prefetch = [&](int64_t c, int64_t t0, int nv) {
    if (__builtin_amdgcn_readfirstlane(wid) < 3) {
      const int r = pf_r + (l >> 2);
      const uint32_t off = (uint32_t)(r < nv ? r : 0) * (uint32_t)H * FK * 2 + 128u * (l & 3);
      const void* x = wid == 0 ? a.w : wid == 1 ? a.q : a.k;
      dma4_(reinterpret_cast<const unsigned char*>(x) + (size_t)((t0 * H + h) * FK) * 2, off, pf_lds);
    } else {
      dma4_(aqb + (c * H + h) * (int64_t)(C * C), 128u * (pf_r + (l & 15)), pf_lds);
    }
  };

  // One chunk step, two barriers.  On entry w and q of chunk it (their tiles) and its small tiles
  // (buffer set B = it % 2) are in flight.  After B1: k of chunk it, then the small tiles of chunk
  // it + 1 (other set) and the L2 prefetch of chunk it + 2; then w h and h^T q^T.  B2 waits for k
  // alone (the later loads stay in flight for a step); after it (every wave is done with w and q):
  // w and q of chunk it + 1; then u, v', o and the state update.
  auto step = [&](auto BB, int64_t it) {
    constexpr uint32_t B = decltype(BB)::value;
    const int64_t t0 = bos + it * C;
    const int nv = chunk_nv(it);
    const int64_t in = it + 1 < nchunks ? it + 1 : it;    // the last step reloads its own chunk (unused)
    const int nv1 = chunk_nv(in);
    wait_all_loads();
    f_barrier();                                          // B1
    dma_tile256(a.k, F, t0, nv, h, H, k_lds);
    dma_small(c_first + in, bos + in * C, nv1, B ^ 1u);
    const bool pf = it + 2 < nchunks;
    if (pf) prefetch(c_first + it + 2, bos + (it + 2) * C, chunk_nv(it + 2));
    const float* sg = s_g + B * C;
    const float* sb = s_b + B * C;

    // w h (rows t, this wave's columns) and o_inter^T = h^T q^T (rows = columns, cols = t), with
    // h = bf16(S) packed per 32-deep step as the B (w h) and A (h^T q^T) operand: K = state rows
    // in the accumulator order; operand reads one step ahead of the products
    f32x4 acc[4], oi[4];
#pragma unroll
    for (int tm = 0; tm < 4; ++tm) {
      acc[tm] = f32x4{0.f, 0.f, 0.f, 0.f};
      oi[tm] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    Frag<bf16> wa[2][4], qa[2][4];
    auto read_wq = [&](int ks, Frag<bf16>(&w4)[4], Frag<bf16>(&q4)[4]) {
      const uint32_t ra = A.row[0][ks & 3], rb = A.row[1][ks & 3];
      const uint32_t o8 = 256u * (ks >> 2);
#pragma unroll
      for (int tm = 0; tm < 4; ++tm) {
        w4[tm] = frag2(ld64(ra, o8 + 8192u * tm), ld64(rb, o8 + 8192u * tm));
        q4[tm] = frag2(ld64(ra, QOFF + o8 + 8192u * tm), ld64(rb, QOFF + o8 + 8192u * tm));
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
        mma(acc[tm], wa[ks & 1][tm], hb);
        mma(oi[tm], hb, qa[ks & 1][tm]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // k of this chunk: the loads issued after it (6 + one gc / beta row in waves 0 and 1, one of
    // the prefetch) may stay in flight
    if (__builtin_amdgcn_readfirstlane(wid) < 2) {
      if (pf) wait_loads_but<kSmallLoads + 1 + kPrefetchLoads>();
      else wait_loads_but<kSmallLoads + 1>();
    } else {
      if (pf) wait_loads_but<kSmallLoads + kPrefetchLoads>();
      else wait_loads_but<kSmallLoads>();
    }
    f_barrier();                                          // B2: k in LDS; w and q tiles free
    dma_tile256(a.w, F, bos + in * C, nv1, h, H, w_lds);
    dma_tile256(a.q, F, bos + in * C, nv1, h, H, w_lds + QOFF);

    // u = Ai bf16(beta v) (wy_fast.py:55-81), rounded to bf16 as the reference stores it; the v tile
    // is read transposed (rows t in the accumulator order) and scaled by beta per row
    Frag<bf16> vb[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const Frag<bf16> vr = tr_frag<64>(s_v + B * C * C, ks, 16 * wid);
      const f32x4 b0 = *reinterpret_cast<const f32x4*>(sb + 32 * ks + 4 * lg);
      const f32x4 b1 = *reinterpret_cast<const f32x4*>(sb + 32 * ks + 16 + 4 * lg);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        vb[ks].v[e] = (bf16)((float)vr.v[e] * b0[e]);
        vb[ks].v[4 + e] = (bf16)((float)vr.v[4 + e] * b1[e]);
      }
    }
    // v' = u - w h (rows t = 16 tm + 4 lg + j), its bf16 value and the gated form
    const float gl = sg[nv - 1];
    f32x4 Y[4], Yg[4];
#pragma unroll
    for (int tm = 0; tm < 4; ++tm) {
      f32x4 u = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        if (ks <= tm / 2)
          mma(u, frag2(ld64(A.aq[ks][0], AI_OFF + B * ABUF + 2048u * tm), ld64(A.aq[ks][1], AI_OFF + B * ABUF + 2048u * tm)),
              vb[ks]);
#pragma unroll
      for (int j = 0; j < 4; ++j) u[j] = (float)(bf16)u[j];
      Y[tm] = u - acc[tm];
      const f32x4 g4 = *reinterpret_cast<const f32x4*>(sg + 16 * tm + 4 * lg);
#pragma unroll
      for (int j = 0; j < 4; ++j) Yg[tm][j] = 16 * tm + 4 * lg + j < nv ? Y[tm][j] * gexp(gl - g4[j]) : 0.f;
    }
    Frag<bf16> vf[2], vg[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      vf[ks] = pack_acc(Y[2 * ks], Y[2 * ks + 1]);
      vg[ks] = pack_acc(Yg[2 * ks], Yg[2 * ks + 1]);
    }
    // o^T = (o_inter^T exp(gc_t) + v'^T Aqk^T) scale; lane: columns v0 + 4 lg .. + 3 of token 16 tn + lc
    unsigned char* orow = ob + (size_t)((t0 * H + h) * V) * 2;
#pragma unroll
    for (int tn = 0; tn < 4; ++tn) {
      const int t = 16 * tn + lc;
      f32x4 r = oi[tn] * gexp(sg[t]);
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        if (ks <= tn / 2)
          mma(r, vf[ks], frag2(ld64(A.aq[ks][0], B * ABUF + 2048u * tn), ld64(A.aq[ks][1], B * ABUF + 2048u * tn)));
      r *= a.scale;
      if (t < nv) {
        const uint2 ov = make_uint2(
            (uint32_t)__builtin_bit_cast(uint16_t, (bf16)r[0]) | ((uint32_t)__builtin_bit_cast(uint16_t, (bf16)r[1]) << 16),
            (uint32_t)__builtin_bit_cast(uint16_t, (bf16)r[2]) | ((uint32_t)__builtin_bit_cast(uint16_t, (bf16)r[3]) << 16));
        *reinterpret_cast<uint2*>(orow + (size_t)(16 * tn) * (size_t)(H * V) * 2 + F.o) = ov;
      }
    }
    // S = exp(g_last) S + k^T (v' exp(g_last - gc)), pipelined like the products above
    const float eg = gexp(gl);
    Frag<bf16> ka[2][4][2];
    auto read_k = [&](int k4, Frag<bf16>(&k8)[4][2]) {
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const int tt = k4 + qq;
        const uint32_t off = 256u * (tt >> 3);
        k8[qq][0] = frag2(ldtr(A.tra[tt & 7], off), ldtr(A.trb[tt & 7], off));
        k8[qq][1] = frag2(ldtr(A.tra[tt & 7], off + 16384u), ldtr(A.trb[tt & 7], off + 16384u));
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

  if (nchunks > 1) prefetch(c_first + 1, bos + C, chunk_nv(1));
  if (nchunks > 0) {
    const int nv0 = chunk_nv(0);
    dma_small(c_first, bos, nv0, 0u);
    dma_tile256(a.w, F, bos, nv0, h, H, w_lds);
    dma_tile256(a.q, F, bos, nv0, h, H, w_lds + QOFF);
  }
  for (int64_t it = 0; it < nchunks; it += 2) {
    step(std::integral_constant<uint32_t, 0>{}, it);
    if (it + 1 < nchunks) step(std::integral_constant<uint32_t, 1>{}, it + 1);
  }
  wait_all_loads();                                       // no direct load outlives the workgroup's LDS

  if (a.ht) {
#pragma unroll
    for (int kt = 0; kt < 16; ++kt) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t off = (((int64_t)n * H + h) * FK + 16 * kt + 4 * lg + j) * V + vcol;
        a.ht[off] = S[kt][j];
      }
    }
  }
}

}  // namespace

bool wide_fused_supported(int compute_dtype, int qk_dtype, int K, int V) {
  return compute_dtype == DT_BF16 && qk_dtype == DT_BF16 && K == FK && V > 0 && V % FVT == 0;
}

int launch_wide_fused(const WideFusedArgs& a, int V, hipStream_t s) {
  if (V % FVT != 0 || a.N * a.H == 0) return -2;
  const int total = a.N * a.H * (V / FVT);
  const int grid = (total + 7) / 8 * 8;
  hipLaunchKernelGGL(wide_fused_kernel, dim3(grid), dim3(NT_F), 0, s, a, V, total);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace kgdn
