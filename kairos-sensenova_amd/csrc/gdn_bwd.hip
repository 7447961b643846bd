// Backward pass of the chunked GatedDeltaNet (fla ops/gated_delta_rule/chunk.py:70-146),
// after the forward has been recomputed by the stage kernels (prepare: gc, w, u, Ai;
// fwd_h with row-major outputs: h [NC, H, K, V] and v_new [B*T, H, V]):
//
//   bwd_dvl_kernel    dv_local = mask_{j<=i}(scale k_j.q_i e^{g_i-g_j}) @ do   chunk_o.py:413-468
//                     (bwd_dvl_split_kernel: the same with its tiles staged in parts)
//   bwd_dhu_kernel    reverse state recurrence of dh, dv2 = gate (k @ dh) + dv_local, dh0
//                                                                          chunk_delta_h.py:250-438
//   bwd_dqkwg_kernel  dq, dk (state and intra-chunk terms), -dw, dg        chunk_o.py:147-326
//   bwd_wy_kernel     WY backward (dk2, dv, dbeta, dg2), dk = dk + dk2 and
//                     the reverse chunk cumsum of dg                        wy_fast.py:98-210,
//                                                                          chunk.py:140-145
//   l2norm_bwd_kernel dx = dy rstd - sum(dy y) y rstd                      l2norm.py:132-154
//                     (l2norm_bwd_rows_kernel: D / 8 lanes per row for power-of-two D)
//
// MFMA operands follow one convention in every kernel: the K index of a 32-deep
// step is taken in "accumulator order" (rows 4 lg .. 4 lg + 3 and 16 + 4 lg ..
// of the step for lane group lg) whenever one operand is a transposed read or an
// accumulator tile; row-major tiles read in that order use two 8-byte reads.
// Tiles in LDS have 64 rows (the chunk's tokens); bf16 tiles are stored as
// [64][64] column blocks swizzled by swz_off<64>, so 16-byte row reads, 8-byte
// accumulator-order reads and ds_read_b64_tr_b16 transposed reads (contractions
// over the token axis) are bank-conflict free; fp32 tiles are padded rows read
// transposed element by element.
#include <cstdlib>

#include "gdn_common.hpp"
#include "gdn_kernels.h"
#include "gdn_tiles.hpp"

namespace kgdn {

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// the row of K index e of an accumulator-order fragment (relative to k0), for per-row operand scaling
__device__ __forceinline__ int acc_row(int e) { return 4 * (lane_id() >> 4) + (e & 3) + (e >> 2) * 16; }

// 4 consecutive elements (c % 4 == 0) of a tile row as floats
template <typename TC>
__device__ __forceinline__ f32x4 t_row4(const TC* t, int ncol, int r, int c) {
  const TC* p = t + toff<TC>(r, c, ncol);
  if constexpr (sizeof(TC) == 2) {
    const bf16x4 v = *reinterpret_cast<const bf16x4*>(p);
    return f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
  } else {
    return *reinterpret_cast<const f32x4*>(p);
  }
}

// fragment element access and scaling with rounding to the operand type
template <typename TC> __device__ __forceinline__ float fget(const Frag<TC>& f, int e);
template <> __device__ __forceinline__ float fget<bf16>(const Frag<bf16>& f, int e) { return (float)f.v[e]; }
template <> __device__ __forceinline__ float fget<float>(const Frag<float>& f, int e) { return e < 4 ? f.lo[e] : f.hi[e - 4]; }
template <typename TC> __device__ __forceinline__ void fset(Frag<TC>& f, int e, float x);
template <> __device__ __forceinline__ void fset<bf16>(Frag<bf16>& f, int e, float x) { f.v[e] = (bf16)x; }
template <> __device__ __forceinline__ void fset<float>(Frag<float>& f, int e, float x) {
  if (e < 4) f.lo[e] = x; else f.hi[e - 4] = x;
}
template <typename TC>
__device__ __forceinline__ Frag<TC> fscale(Frag<TC> f, float s) {
#pragma unroll
  for (int e = 0; e < 8; ++e) fset<TC>(f, e, fget<TC>(f, e) * s);
  return f;
}
template <typename TC>
__device__ __forceinline__ Frag<TC> fzero() {
  Frag<TC> f;
#pragma unroll
  for (int e = 0; e < 8; ++e) fset<TC>(f, e, 0.f);
  return f;
}

// natural fragment of a row-major tensor in global memory (row = the lane's row start), or zeros
// where !valid.  The load is issued unconditionally and masked after, so that the loads of
// consecutive fragments go out together (a load in a branch of its own is waited for before the
// next is issued): row must be readable, so callers clamp rows past the chunk's end to its first.
template <typename TC>
__device__ __forceinline__ Frag<TC> g_nat(const TC* row, int k0, bool valid) {
  const TC* p = row + k0 + 8 * (lane_id() >> 4);
  Frag<TC> f;
  if constexpr (sizeof(TC) == 2) {
    uint4 x = *reinterpret_cast<const uint4*>(p);
    x.x = valid ? x.x : 0u;
    x.y = valid ? x.y : 0u;
    x.z = valid ? x.z : 0u;
    x.w = valid ? x.w : 0u;
    f.v = __builtin_bit_cast(bf16x8, x);
  } else {
    const f32x4 lo = *reinterpret_cast<const f32x4*>(p), hi = *reinterpret_cast<const f32x4*>(p + 4);
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
    f.lo = valid ? lo : z;
    f.hi = valid ? hi : z;
  }
  return f;
}

// fragment built from two accumulator tiles (rows 0-15 and 16-31 of a 32-deep K step)
template <typename TC>
__device__ __forceinline__ Frag<TC> acc_frag(const f32x4& a, const f32x4& b) {
  Frag<TC> f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    fset<TC>(f, e, a[e]);
    fset<TC>(f, e + 4, b[e]);
  }
  return f;
}

// stage 64 token rows [t0, t0 + nv) of a row-major [*, H, ncol] tensor into a tile (zeros past nv),
// four units per thread in flight at a time (every load of a batch is issued before its stores)
template <typename TC>
__device__ __forceinline__ void stage_rows(TC* tile, const TC* src, int64_t t0, int nv, int H, int h, int ncol) {
  const int per_row = ncol / 8, total = 64 * per_row, nt = blockDim.x;
  for (int base = threadIdx.x; base < total; base += 4 * nt) {
    Vec8<TC> x[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = base + i * nt, r = idx / per_row, c8 = (idx % per_row) * 8;
      x[i] = (idx < total && r < nv) ? ld8<TC>(src + ((t0 + r) * H + h) * (int64_t)ncol + c8) : vzero<TC>();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = base + i * nt, r = idx / per_row, c8 = (idx % per_row) * 8;
      if (idx < total) st8<TC>(tile + toff<TC>(r, c8, ncol), x[i]);
    }
  }
}

// The same staging by direct global -> LDS loads (bf16): every load of the tile is in flight at once
// (one instruction moves 8 rows of a 64-column block, 1 KB); lanes of rows past nv are masked off the
// loads and write zeros with plain stores instead.  The caller waits for its loads (stage_wait) and
// barriers before reading.
__device__ __forceinline__ void stage_dma16(const void* base, uint32_t off, uint32_t lds_dst) {
  const uint64_t v = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(off),
               "s"(reinterpret_cast<const void*>(((uint64_t)hi << 32) | lo)),
               "{m0}"(__builtin_amdgcn_readfirstlane(lds_dst)) : "memory");
}
__device__ __forceinline__ void stage_rows_dma(bf16* tile, const bf16* src, int64_t t0, int nv, int H, int h, int ncol) {
  const int nw = blockDim.x / WAVE, wid = threadIdx.x / WAVE, l = lane_id();
  const unsigned char* base = reinterpret_cast<const unsigned char*>(src + (t0 * H + h) * (int64_t)ncol);
  const uint32_t row_bytes = (uint32_t)(H * ncol * 2);
  const uint32_t tile_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) bf16*)tile;
  for (int i = wid; i < ncol / 8; i += nw) {
    const int cb = i >> 3, r = 8 * (i & 7) + (l >> 3);
    const int c8 = (l & 7) ^ ((((r >> 1) & 3) << 1) | ((r >> 3) & 1));   // swz_off<64>'s chunk order
    const uint32_t dst = tile_lds + 8192u * cb + 1024u * (i & 7);
    if (r < nv) {
      stage_dma16(base, (uint32_t)r * row_bytes + (uint32_t)(64 * cb + 8 * c8) * 2u, dst);
    } else {
      *reinterpret_cast<__attribute__((address_space(3))) u32x4*>((uintptr_t)(dst + 16u * l)) = u32x4{0u, 0u, 0u, 0u};
    }
  }
}
__device__ __forceinline__ void stage_wait() {
  __builtin_amdgcn_s_waitcnt(0x0F70);          // vmcnt(0): the direct loads have landed
  asm volatile("" ::: "memory");
}

// sum over the 16 lanes of a row group (l % 16) or over the 4 lane groups (l / 16)
__device__ __forceinline__ float sum16(float x) {
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) x += __shfl_xor(x, o, WAVE);
  return x;
}
__device__ __forceinline__ float sum_lg(float x) {
  x += __shfl_xor(x, 16, WAVE);
  x += __shfl_xor(x, 32, WAVE);
  return x;
}
__device__ __forceinline__ float sum64(float x) {
#pragma unroll
  for (int o = 1; o < WAVE; o <<= 1) x += __shfl_xor(x, o, WAVE);
  return x;
}

template <typename TC>
__device__ __forceinline__ void st4v(TC* p, const f32x4& v) { st4<TC>(p, v[0], v[1], v[2], v[3]); }

template <typename TC>
__device__ __forceinline__ f32x4 g_row4(const TC* p) { return ld4<TC>(p); }

constexpr int NT_B = 256;   // threads of the chunk-parallel backward kernels (4 waves, one per 16 tokens)

// ---------------------------------------------------------------------------
// dv_local (chunk_o.py:413-468): dv_local[j] = sum_{i >= j} scale (q_i.k_j) e^{g_i - g_j} do_i
// ---------------------------------------------------------------------------
template <typename TC>
__host__ __device__ constexpr size_t dvl_lds(int K, int V) {
  return sizeof(TC) * (2 * (size_t)tile_elems<TC>(K) + tile_elems<TC>(V) + tile_elems<TC>(64)) + 64 * sizeof(float);
}

template <typename TC, int K, int NW = 4>
__global__ __launch_bounds__(64 * NW) void bwd_dvl_kernel(BwdArgs a, int V) {
  extern __shared__ __align__(16) unsigned char smem[];
  TC* s_q = reinterpret_cast<TC*>(smem);
  TC* s_k = s_q + tile_elems<TC>(K);
  TC* s_do = s_k + tile_elems<TC>(K);
  TC* s_M = s_do + tile_elems<TC>(V);
  float* s_g = reinterpret_cast<float*>(s_M + tile_elems<TC>(64));
  const int h = blockIdx.y, H = a.H;
  const ChunkLoc loc = locate_chunk(blockIdx.x, a.cu, a.chunk_off, a.N, a.T);
  if (!loc.ok) return;
  const int64_t t0 = loc.t0;
  const int nv = loc.nv;
  const int wid = threadIdx.x / WAVE, l = lane_id(), lg = l >> 4, lc = l & 15;
  if constexpr (sizeof(TC) == 2) {
    stage_rows_dma(s_q, reinterpret_cast<const TC*>(a.q), t0, nv, H, h, K);
    stage_rows_dma(s_k, reinterpret_cast<const TC*>(a.k), t0, nv, H, h, K);
    stage_rows_dma(s_do, reinterpret_cast<const TC*>(a.do_), t0, nv, H, h, V);
  } else {
    stage_rows<TC>(s_q, reinterpret_cast<const TC*>(a.q), t0, nv, H, h, K);
    stage_rows<TC>(s_k, reinterpret_cast<const TC*>(a.k), t0, nv, H, h, K);
    stage_rows<TC>(s_do, reinterpret_cast<const TC*>(a.do_), t0, nv, H, h, V);
  }
  if (threadIdx.x < 64) s_g[threadIdx.x] = threadIdx.x < nv ? a.gc[(t0 + threadIdx.x) * H + h] : 0.f;
  stage_wait();
  __syncthreads();

  // optional q^T per chunk, [NC, H, K, 64] (zero past the chunk's end), the K = 256 dh recurrence's
  // operand: transposed reads of the staged q tile (lane: 4 tokens of one d, one 8-byte store)
  if constexpr (sizeof(TC) == 2 && K == 256) {
    if (a.qT) {
      TC* qt = reinterpret_cast<TC*>(a.qT) + (blockIdx.x * (int64_t)H + h) * (K * C);
      for (int i = wid; i < (K / 16) * 4; i += NW) {
        const int d0 = 16 * (i >> 2), tr0 = 16 * (i & 3) + 4 * lg;
        const s16x4_t x = lds_read_tr16(s_q + toff<TC>(tr0 + (lc >> 2), d0 + 4 * (lc & 3), K));
        *reinterpret_cast<s16x4_t*>(qt + (d0 + lc) * C + tr0) = x;
      }
    }
  }

  // M^T[j][i], j <= i, rounded to the storage type (the reference's b_A.to(do.dtype))
  for (int tile = wid; tile < 16; tile += NW) {
    const int tj = tile >> 2, ti = tile & 3;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    if (tj <= ti) {
#pragma unroll
      for (int ks = 0; ks < K / 32; ++ks) mma(acc, t_nat<TC>(s_k, K, 16 * tj, 32 * ks), t_nat<TC>(s_q, K, 16 * ti, 32 * ks));
    }
    const int i = 16 * ti + lc;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int j = 16 * tj + 4 * lg + jj;
      const float val = (j <= i && i < nv) ? acc[jj] * a.scale * gexp(s_g[i] - s_g[j]) : 0.f;
      s_M[toff<TC>(j, i, 64)] = from_f32<TC>(val);
    }
  }
  __syncthreads();

  // dv_local^T[v][j] = sum_i do[i][v] M^T[j][i]
  TC* out = reinterpret_cast<TC*>(a.dvl);
  for (int tile = wid; tile < (V / 16) * 4; tile += NW) {
    const int tv = tile >> 2, tj = tile & 3;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) mma(acc, t_tr<TC>(s_do, V, 32 * ks, 16 * tv), t_acc<TC>(s_M, 64, 16 * tj, 32 * ks));
    const int j = 16 * tj + lc;
    if (j < nv) st4v<TC>(out + ((t0 + j) * H + h) * (int64_t)V + 16 * tv + 4 * lg, acc);
  }
}

// The same stage for bf16 with its tiles staged in parts through one buffer: q and k in two halves
// of K / 2 columns (M accumulated across them in registers), then do in blocks of VB columns.  At
// dk = 256 (VB = 256) 40 KB of LDS, three workgroups per CU instead of one (136 KB); at dk = 128
// (VB = 128) 24 KB.
__device__ __forceinline__ void stage_rows_dma_cols(bf16* tile, const bf16* src, int64_t t0, int nv, int H, int h,
                                                    int row_len, int c0, int ncol) {
  const int nw = blockDim.x / WAVE, wid = threadIdx.x / WAVE, l = lane_id();
  const unsigned char* base = reinterpret_cast<const unsigned char*>(src + (t0 * H + h) * (int64_t)row_len + c0);
  const uint32_t row_bytes = (uint32_t)(H * row_len * 2);
  const uint32_t tile_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) bf16*)tile;
  for (int i = wid; i < ncol / 8; i += nw) {
    const int cb = i >> 3, r = 8 * (i & 7) + (l >> 3);
    const int c8 = (l & 7) ^ ((((r >> 1) & 3) << 1) | ((r >> 3) & 1));   // swz_off<64>'s chunk order
    const uint32_t dst = tile_lds + 8192u * cb + 1024u * (i & 7);
    if (r < nv) {
      stage_dma16(base, (uint32_t)r * row_bytes + (uint32_t)(64 * cb + 8 * c8) * 2u, dst);
    } else {
      *reinterpret_cast<__attribute__((address_space(3))) u32x4*>((uintptr_t)(dst + 16u * l)) = u32x4{0u, 0u, 0u, 0u};
    }
  }
}

constexpr int DVL_SPLIT_NW = 8;
template <int K, int VB>
constexpr size_t dvl_split_lds() {
  return (size_t)2 * 64 * (K > VB ? K : VB) + (size_t)2 * 64 * 64 + 64 * sizeof(float);
}

template <int K, int VB>
__global__ __launch_bounds__(64 * DVL_SPLIT_NW) void bwd_dvl_split_kernel(BwdArgs a, int V) {
  constexpr int KH = K / 2, NW = DVL_SPLIT_NW, BUF = K > VB ? K : VB;
  static_assert(KH % 32 == 0 && VB % 64 == 0, "halves of whole MMA steps, blocks of whole column tiles");
  extern __shared__ __align__(16) unsigned char smem[];
  bf16* s_buf = reinterpret_cast<bf16*>(smem);          // q, k halves [64][128] each, or a do block [64][256]
  bf16* s_qh = s_buf;
  bf16* s_kh = s_buf + 64 * KH;
  bf16* s_M = s_buf + 64 * BUF;
  float* s_g = reinterpret_cast<float*>(s_M + 64 * 64);
  const int h = blockIdx.y, H = a.H;
  const ChunkLoc loc = locate_chunk(blockIdx.x, a.cu, a.chunk_off, a.N, a.T);
  if (!loc.ok) return;
  const int64_t t0 = loc.t0;
  const int nv = loc.nv;
  const int wid = threadIdx.x / WAVE, l = lane_id(), lg = l >> 4, lc = l & 15;
  const bf16* q = reinterpret_cast<const bf16*>(a.q);
  const bf16* k = reinterpret_cast<const bf16*>(a.k);
  if (threadIdx.x < 64) s_g[threadIdx.x] = threadIdx.x < nv ? a.gc[(t0 + threadIdx.x) * H + h] : 0.f;
  // M^T[j][i] = k_j . q_i over the two halves of the head dim, tiles wid and wid + 8 of this wave
  f32x4 acc[16 / NW];
#pragma unroll
  for (int u = 0; u < 16 / NW; ++u) acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
  bf16* qt = a.qT ? reinterpret_cast<bf16*>(a.qT) + (blockIdx.x * (int64_t)H + h) * (K * C) : nullptr;
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    if (half) __syncthreads();                          // every wave is done with the first half
    stage_rows_dma_cols(s_qh, q, t0, nv, H, h, K, KH * half, KH);
    stage_rows_dma_cols(s_kh, k, t0, nv, H, h, K, KH * half, KH);
    stage_wait();
    __syncthreads();
    // q^T per chunk, [NC, H, K, 64] (zero past the chunk's end): rows d of this half
    if (qt) {
      for (int i = wid; i < (KH / 16) * 4; i += NW) {
        const int d0 = 16 * (i >> 2), tr0 = 16 * (i & 3) + 4 * lg;
        const s16x4_t x = lds_read_tr16(s_qh + toff<bf16>(tr0 + (lc >> 2), d0 + 4 * (lc & 3), KH));
        *reinterpret_cast<s16x4_t*>(qt + (KH * half + d0 + lc) * C + tr0) = x;
      }
    }
#pragma unroll
    for (int u = 0; u < 16 / NW; ++u) {
      const int tile = wid + NW * u, tj = tile >> 2, ti = tile & 3;
      if (tj <= ti) {
#pragma unroll
        for (int ks = 0; ks < KH / 32; ++ks)
          mma(acc[u], t_nat<bf16>(s_kh, KH, 16 * tj, 32 * ks), t_nat<bf16>(s_qh, KH, 16 * ti, 32 * ks));
      }
    }
  }
  // M^T rounded to bf16 (the reference's b_A.to(do.dtype))
#pragma unroll
  for (int u = 0; u < 16 / NW; ++u) {
    const int tile = wid + NW * u, tj = tile >> 2, ti = tile & 3;
    const int i = 16 * ti + lc;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int j = 16 * tj + 4 * lg + jj;
      const float val = (j <= i && i < nv) ? acc[u][jj] * a.scale * gexp(s_g[i] - s_g[j]) : 0.f;
      s_M[toff<bf16>(j, i, 64)] = (bf16)val;
    }
  }
  // dv_local^T[v][j] = sum_i do[i][v] M^T[j][i], do in blocks of 256 columns
  bf16* out = reinterpret_cast<bf16*>(a.dvl);
  const bf16* dO = reinterpret_cast<const bf16*>(a.do_);
  for (int vb = 0; vb < V; vb += VB) {
    __syncthreads();                                    // s_M written / the previous block read
    stage_rows_dma_cols(s_buf, dO, t0, nv, H, h, V, vb, VB);
    stage_wait();
    __syncthreads();
    for (int tile = wid; tile < (VB / 16) * 4; tile += NW) {
      const int tv = tile >> 2, tj = tile & 3;
      f32x4 r = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) mma(r, t_tr<bf16>(s_buf, VB, 32 * ks, 16 * tv), t_acc<bf16>(s_M, 64, 16 * tj, 32 * ks));
      const int j = 16 * tj + lc;
      if (j < nv) st4v<bf16>(out + ((t0 + j) * H + h) * (int64_t)V + vb + 16 * tv + 4 * lg, r);
    }
  }
}

// ---------------------------------------------------------------------------
// dh recurrence (chunk_delta_h.py:250-438).  One workgroup per (sequence, head,
// 16 value columns), NW waves splitting the K rows of the state gradient dh
// [K x 16] (fp32, accumulator layout, in VGPRs).  Per chunk, last to first:
//   dh[c] = dh (stored, rounded)
//   dv2   = (k @ bf16(dh)) e^{g_last - gc} + dv_local            (stored)
//   dh    = e^{g_last} dh + scale (q e^{gc})^T do - w^T bf16(dv2)
// The q e^{gc} operand is fp32 in the reference; the bf16 path feeds it to the
// bf16 MFMA as hi + lo = bf16(x) + bf16(x - bf16(x)) (16 significant bits).
// ---------------------------------------------------------------------------
constexpr int DBV = 16;
constexpr int LDT = C + 8;

// Workgroup barrier that waits for LDS operations only (lgkmcnt(0), s_barrier): within a chunk step
// the waves share only LDS, and __syncthreads() would also wait for the next chunk's loads (vmcnt(0))
// and this chunk's stores.  The empty asm statements keep memory accesses from moving across it.
__device__ __forceinline__ void step_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);          // lgkmcnt(0); vmcnt, expcnt at their maxima
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <int K> struct DCfg {
  static constexpr int NW = K == 64 ? 2 : 4;
  static constexpr int KW = K / NW;
  static constexpr int KT = KW / 16;
  static constexpr int KS = KW / 32;
  static constexpr int OWN = 4 / NW;
  static constexpr int DO_COLS = DBV / NW;    // do columns each wave stages
};

template <typename TC, int K>
struct DhuChunk {
  using Cfg = DCfg<K>;
  Frag<TC> kf[4][Cfg::KS];      // k rows 16 tm + lc, the wave's K slice, accumulator order
  Vec8<TC> qrow[Cfg::KW / 8];   // q[t = lane][wave's K slice]
  Vec8<TC> wrow[Cfg::KW / 8];   // w[t = lane][wave's K slice]
  float dov[Cfg::DO_COLS];      // do[t = lane][this wave's columns]
  f32x4 dvl[Cfg::OWN];          // dv_local of the owned row tiles (C layout)
  f32x4 gv[Cfg::OWN];           // gc of the owned rows
  float gt;                     // gc of token lane
  float gl;
  int64_t t0;
  int nv;
};

template <typename TC, int K>
__device__ __forceinline__ void dhu_load(DhuChunk<TC, K>& P, const BwdArgs& a, int64_t t0, int nv, int h, int v0,
                                         int wid, int V) {
  using Cfg = DCfg<K>;
  const int l = lane_id(), lg = l >> 4, lc = l & 15;
  const int H = a.H;
  P.t0 = t0;
  P.nv = nv;
  const TC* k = reinterpret_cast<const TC*>(a.k);
  const TC* q = reinterpret_cast<const TC*>(a.q);
  const TC* w = reinterpret_cast<const TC*>(a.w);
#pragma unroll
  for (int tm = 0; tm < 4; ++tm) {
    const int t = 16 * tm + lc;
#pragma unroll
    for (int ks = 0; ks < Cfg::KS; ++ks) {
      Frag<TC> f = fzero<TC>();
      if (t < nv) {
        const TC* p = k + ((t0 + t) * H + h) * (int64_t)K + Cfg::KW * wid + 32 * ks + 4 * lg;
        const f32x4 x0 = ld4<TC>(p), x1 = ld4<TC>(p + 16);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          fset<TC>(f, e, x0[e]);
          fset<TC>(f, e + 4, x1[e]);
        }
      }
      P.kf[tm][ks] = f;
    }
  }
#pragma unroll
  for (int d8 = 0; d8 < Cfg::KW / 8; ++d8) {
    P.qrow[d8] = l < nv ? ld8<TC>(q + ((t0 + l) * H + h) * (int64_t)K + Cfg::KW * wid + 8 * d8) : vzero<TC>();
    P.wrow[d8] = l < nv ? ld8<TC>(w + ((t0 + l) * H + h) * (int64_t)K + Cfg::KW * wid + 8 * d8) : vzero<TC>();
  }
  const TC* dov = reinterpret_cast<const TC*>(a.do_);
#pragma unroll
  for (int cc = 0; cc < Cfg::DO_COLS; ++cc)
    P.dov[cc] = l < nv ? to_f32(dov[((t0 + l) * H + h) * (int64_t)V + v0 + Cfg::DO_COLS * wid + cc]) : 0.f;
  const TC* dvl = reinterpret_cast<const TC*>(a.dvl);
#pragma unroll
  for (int o = 0; o < Cfg::OWN; ++o) {
    const int tm = wid + Cfg::NW * o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = 16 * tm + 4 * lg + j;
      P.dvl[o][j] = t < nv ? to_f32(dvl[((t0 + t) * H + h) * (int64_t)V + v0 + lc]) : 0.f;
      P.gv[o][j] = t < nv ? a.gc[(t0 + t) * H + h] : 0.f;
    }
  }
  P.gt = l < nv ? a.gc[(t0 + l) * H + h] : 0.f;
  P.gl = a.gc[(t0 + nv - 1) * H + h];
}

template <typename TC, int K>
__global__ __launch_bounds__(64 * DCfg<K>::NW) void bwd_dhu_kernel(BwdArgs a, int V, int total_units) {
  using Cfg = DCfg<K>;
  constexpr int NW = Cfg::NW, KW = Cfg::KW, KT = Cfg::KT, KS = Cfg::KS, OWN = Cfg::OWN;
  constexpr int NP = sizeof(TC) == 2 ? 2 : 1;          // q e^{gc} parts (hi, lo) for bf16
  __shared__ __align__(16) f32x4 s_red[NW][4][WAVE];
  __shared__ __align__(16) TC s_qT[NP][K * LDT];       // rows k (wave slices), cols t
  __shared__ __align__(16) TC s_wT[K * LDT];           // -w^T
  __shared__ __align__(16) TC s_doT[DBV * LDT];        // do^T of the 16 columns
  __shared__ __align__(16) TC s_dvT[DBV * LDT];        // bf16(dv2)^T

  const int per_xcd = gridDim.x / 8;                   // XCD-aware unit order
  const int o_idx = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (o_idx >= total_units) return;
  const int nvt = V / DBV;
  const int unit = o_idx / nvt;
  const int v0 = (o_idx % nvt) * DBV;
  const int H = a.H;
  const int n = unit / H, h = unit % H;
  const int wid = threadIdx.x / WAVE, l = lane_id(), lg = l >> 4, lc = l & 15;

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

  // dh slice: rows KW wid + 16 tt + 4 lg + j, column v0 + lc; starts at dht
  f32x4 dh[KT];
#pragma unroll
  for (int tt = 0; tt < KT; ++tt) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t off = (((int64_t)n * H + h) * K + KW * wid + 16 * tt + 4 * lg + j) * V + v0 + lc;
      dh[tt][j] = a.dht ? a.dht[off] : 0.f;
    }
  }

  DhuChunk<TC, K> cur, nxt;
  auto chunk_start = [&](int64_t it) { return bos + it * C; };
  auto chunk_len = [&](int64_t it) { return (int)min((int64_t)C, eos - chunk_start(it)); };
  if (nchunks > 0) dhu_load<TC, K>(cur, a, chunk_start(nchunks - 1), chunk_len(nchunks - 1), h, v0, wid, V);

  TC* dh_out = reinterpret_cast<TC*>(a.dh);
  TC* dv2_out = reinterpret_cast<TC*>(a.dv2);
  for (int64_t it = nchunks - 1; it >= 0; --it) {
    const int64_t c = c_first + it;
    if (it > 0) dhu_load<TC, K>(nxt, a, chunk_start(it - 1), chunk_len(it - 1), h, v0, wid, V);
    const int nv = cur.nv;
    const int64_t t0 = cur.t0;

    // dh snapshot, row-major [NC, H, K, V] (no outputs: a segment's first pass, which only needs dh0)
    if (dh_out) {
      TC* p = dh_out + ((c * H + h) * K + KW * wid + 4 * lg) * (int64_t)V + v0 + lc;
#pragma unroll
      for (int tt = 0; tt < KT; ++tt)
#pragma unroll
        for (int j = 0; j < 4; ++j) p[(16 * tt + j) * (int64_t)V] = from_f32<TC>(dh[tt][j]);
    }
    // partial k @ bf16(dh) over this wave's K slice
    Frag<TC> hb[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) hb[ks] = acc_frag<TC>(dh[2 * ks], dh[2 * ks + 1]);
#pragma unroll
    for (int tm = 0; tm < 4; ++tm) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) mma(acc, cur.kf[tm][ks], hb[ks]);
      s_red[wid][tm][l] = acc;
    }
    // transposed update operands of this wave's K slice (t = lane) and its do columns
    {
      const float qs = l < nv ? gexp(cur.gt) * a.scale : 0.f;
#pragma unroll
      for (int d8 = 0; d8 < KW / 8; ++d8) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int r = KW * wid + 8 * d8 + e;
          const float qg = vget<TC>(cur.qrow[d8], e) * qs;
          const TC hi = from_f32<TC>(qg);
          s_qT[0][r * LDT + l] = hi;
          if constexpr (NP == 2) s_qT[NP - 1][r * LDT + l] = from_f32<TC>(qg - to_f32(hi));
          s_wT[r * LDT + l] = from_f32<TC>(-vget<TC>(cur.wrow[d8], e));
        }
      }
    }
    step_barrier();

    // do^T columns of this wave (after the barrier: every wave has finished the previous
    // chunk's update, which reads s_doT and s_dvT); dv2 of the owned row tiles
#pragma unroll
    for (int cc = 0; cc < Cfg::DO_COLS; ++cc) s_doT[(Cfg::DO_COLS * wid + cc) * LDT + l] = from_f32<TC>(cur.dov[cc]);
#pragma unroll
    for (int o = 0; o < OWN; ++o) {
      const int tm = wid + NW * o;
      f32x4 kd = s_red[0][tm][l];
#pragma unroll
      for (int w2 = 1; w2 < NW; ++w2) kd += s_red[w2][tm][l];
      float dv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = 16 * tm + 4 * lg + j;
        dv[j] = t < nv ? kd[j] * gexp(cur.gl - cur.gv[o][j]) + cur.dvl[o][j] : 0.f;
        if (dv2_out && t < nv) dv2_out[((t0 + t) * H + h) * (int64_t)V + v0 + lc] = from_f32<TC>(dv[j]);
      }
      st4<TC>(s_dvT + lc * LDT + 16 * tm + 4 * lg, dv[0], dv[1], dv[2], dv[3]);
    }
    step_barrier();

    // dh = e^{g_last} dh + (scale q e^{gc})^T do - w^T bf16(dv2)
    const float eg = gexp(cur.gl);
#pragma unroll
    for (int tt = 0; tt < KT; ++tt) {
      dh[tt] *= eg;
      const int r0 = KW * wid + 16 * tt;
#pragma unroll
      for (int ks2 = 0; ks2 < 2; ++ks2) {
        const Frag<TC> bdo = lds_frag<TC>(s_doT, LDT, 0, 32 * ks2);
#pragma unroll
        for (int p = 0; p < NP; ++p) mma(dh[tt], lds_frag<TC>(s_qT[p], LDT, r0, 32 * ks2), bdo);
        mma(dh[tt], lds_frag<TC>(s_wT, LDT, r0, 32 * ks2), lds_frag<TC>(s_dvT, LDT, 0, 32 * ks2));
      }
    }
    cur = nxt;
  }

  if (a.dh0) {
#pragma unroll
    for (int tt = 0; tt < KT; ++tt) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t off = (((int64_t)n * H + h) * K + KW * wid + 16 * tt + 4 * lg + j) * V + v0 + lc;
        a.dh0[off] = dh[tt][j];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// dh recurrence, bf16, one workgroup per (sequence, head) with all value columns
// (chunk_delta_h.py:250-438, the same step as bwd_dhu_kernel).  V / 16 waves, wave w owning
// columns 16 w .. 16 w + 15 of dh over all K rows (fp32, accumulator layout, in VGPRs); the
// chunk's k, q e^{gc} scale (as a bf16 pair hi + lo), -w, do and dv_local are staged once in LDS
// for every wave (the per-16-column form re-stages them for each column slice).  Inputs of the
// next chunk (in reverse order) are loaded into registers while the current chunk computes.
//   dv2 = e^{g_last - gc} (k bf16(dh)) + dv_local        A = k rows, K = dh rows (accumulator order)
//   dh  = e^{g_last} dh + (q e^{gc} scale)^T do - w^T bf16(dv2)   A = transposed tiles, B = do
//                                                        (transposed) and dv2's accumulator tiles
// ---------------------------------------------------------------------------
template <int K, int V>
struct DW {
  static constexpr int NW = V / 16, NT = NW * WAVE;
  static constexpr int KT = K / 16, KS = K / 32;
  static constexpr int EK = C * K, EV = C * V;            // elements of a [64][K] / [64][V] tile
  static constexpr int off_k = 0, off_qh = EK, off_ql = 2 * EK, off_w = 3 * EK, off_do = 4 * EK;
  static constexpr int off_dvl = 4 * EK + EV;              // dv_local [64][V] (same tile layout)
  static constexpr int n_el = 4 * EK + 2 * EV;
  // the outputs of a chunk step, bf16 row-major with 16-byte chunks swizzled by row (swz_out): the dh
  // snapshot [K][V] and dv2 [64][V], written out as whole rows by every thread after the step
  static constexpr size_t off_hs = (size_t)n_el * 2 + C * sizeof(float);
  static constexpr size_t off_dv2 = off_hs + (size_t)K * V * 2;
  static constexpr size_t lds = off_dv2 + (size_t)C * V * 2;
  static constexpr int UK = EK / 8 / NT, UV = EV / 8 / NT;  // 16-byte units per thread
  static_assert(EK % (8 * NT) == 0 && EV % (8 * NT) == 0, "units split evenly over the threads");
};

template <int K, int V>
struct DWChunk {
  using D = DW<K, V>;
  u32x4 q[D::UK], k[D::UK], w[D::UK], dO[D::UV], dvl[D::UV];
  float qs[D::UK];            // e^{gc} scale of the row of each q unit (0 past the chunk's end)
  float gt;                   // gc of token = lane (0 past the end)
  int64_t t0;
  int nv;
};

template <int K, int V>
__device__ __forceinline__ void dw_load(DWChunk<K, V>& P, const BwdArgs& a, int64_t t0, int nv, int h) {
  using D = DW<K, V>;
  const int tid = threadIdx.x, l = lane_id();
  const int H = a.H;
  P.t0 = t0;
  P.nv = nv;
  const u32x4 z = {0u, 0u, 0u, 0u};
  const bf16* q = reinterpret_cast<const bf16*>(a.q);
  const bf16* k = reinterpret_cast<const bf16*>(a.k);
  const bf16* w = reinterpret_cast<const bf16*>(a.w);
#pragma unroll
  for (int i = 0; i < D::UK; ++i) {
    const int u = tid + D::NT * i, r = u / (K / 8), c8 = u % (K / 8);
    const int64_t off = ((t0 + r) * H + h) * (int64_t)K + 8 * c8;
    P.q[i] = r < nv ? *reinterpret_cast<const u32x4*>(q + off) : z;
    P.k[i] = r < nv ? *reinterpret_cast<const u32x4*>(k + off) : z;
    P.w[i] = r < nv ? *reinterpret_cast<const u32x4*>(w + off) : z;
    P.qs[i] = r < nv ? a.gc[(t0 + r) * H + h] : 0.f;     // exponentiated at staging
  }
  const bf16* dO = reinterpret_cast<const bf16*>(a.do_);
  const bf16* dvl = reinterpret_cast<const bf16*>(a.dvl);
#pragma unroll
  for (int i = 0; i < D::UV; ++i) {
    const int u = tid + D::NT * i, r = u / (V / 8), c8 = u % (V / 8);
    const int64_t off = ((t0 + r) * H + h) * (int64_t)V + 8 * c8;
    P.dO[i] = r < nv ? *reinterpret_cast<const u32x4*>(dO + off) : z;
    P.dvl[i] = r < nv ? *reinterpret_cast<const u32x4*>(dvl + off) : z;
  }
  P.gt = l < nv ? a.gc[(t0 + l) * H + h] : 0.f;
}

// 16-byte chunk ch of row r of an output tile with V / 8 chunks per row: rows 4 apart (the rows of one
// lane group's 2-byte writes) land on distinct pairs of chunks
template <int V>
__device__ __forceinline__ int swz_out(int r, int ch) { return ch ^ ((2 * (r >> 2)) & (V / 8 - 1)); }

// kOut: the pass that writes the dh snapshots and dv2 (a.dh or a.dv2 set); without, only dh0
template <int K, int V, bool kOut>
__global__ __launch_bounds__((DW<K, V>::NT)) void bwd_dhu_wide_kernel(BwdArgs a, int total_units) {
  using D = DW<K, V>;
  constexpr int KT = D::KT, KS = D::KS;
  extern __shared__ __align__(16) unsigned char smem[];
  bf16* sm = reinterpret_cast<bf16*>(smem);
  bf16* s_k = sm + D::off_k;
  bf16* s_qh = sm + D::off_qh;
  bf16* s_ql = sm + D::off_ql;
  bf16* s_w = sm + D::off_w;
  bf16* s_do = sm + D::off_do;
  bf16* s_dvl = sm + D::off_dvl;
  float* s_g = reinterpret_cast<float*>(smem + (size_t)D::n_el * 2);
  bf16* s_hs = reinterpret_cast<bf16*>(smem + D::off_hs);
  bf16* s_dv2 = reinterpret_cast<bf16*>(smem + D::off_dv2);

  const int per_xcd = gridDim.x / 8;                   // XCD-aware unit order
  const int unit = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (unit >= total_units) return;
  const int H = a.H;
  const int n = unit / H, h = unit % H;
  const int tid = threadIdx.x, wid = tid / WAVE, l = lane_id(), lg = l >> 4, lc = l & 15;
  const int c0 = 16 * wid;                             // this wave's columns

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

  // dh: rows 16 tt + 4 lg + j, column c0 + lc; starts at dht
  f32x4 dh[KT];
#pragma unroll
  for (int tt = 0; tt < KT; ++tt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t off = (((int64_t)n * H + h) * K + 16 * tt + 4 * lg + j) * V + c0 + lc;
      dh[tt][j] = a.dht ? a.dht[off] : 0.f;
    }

  auto chunk_start = [&](int64_t it) { return bos + it * C; };
  auto chunk_len = [&](int64_t it) { return (int)min((int64_t)C, eos - chunk_start(it)); };
  DWChunk<K, V> cur, nxt;
  if (nchunks > 0) dw_load<K, V>(cur, a, chunk_start(nchunks - 1), chunk_len(nchunks - 1), h);
  bf16* dh_out = reinterpret_cast<bf16*>(a.dh);
  bf16* dv2_out = reinterpret_cast<bf16*>(a.dv2);
  // a step's dh snapshot and dv2, from their LDS tiles to HBM as 16-byte row pieces (every thread)
  auto flush = [&](int64_t c, int64_t t0, int nv) {
    if (dh_out) {
      bf16* base = dh_out + (c * H + h) * (int64_t)K * V;            // [K][V], contiguous
#pragma unroll
      for (int i = 0; i < K * V / 8 / D::NT; ++i) {
        const int u = tid + D::NT * i, r = u / (V / 8), ch = u % (V / 8);
        const u32x4 x = *reinterpret_cast<const u32x4*>(s_hs + r * V + 8 * swz_out<V>(r, ch));
        st_global(base + (int64_t)r * V + 8 * ch, x);
      }
    }
    if (dv2_out) {
#pragma unroll
      for (int i = 0; i < C * V / 8 / D::NT; ++i) {
        const int u = tid + D::NT * i, t = u / (V / 8), ch = u % (V / 8);
        const u32x4 x = *reinterpret_cast<const u32x4*>(s_dv2 + t * V + 8 * swz_out<V>(t, ch));
        if (t < nv) st_global(dv2_out + ((t0 + t) * H + h) * (int64_t)V + 8 * ch, x);
      }
    }
  };
  int64_t prev_c = 0, prev_t0 = 0;
  int prev_nv = 0;

  for (int64_t it = nchunks - 1; it >= 0; --it) {
    const int64_t c = c_first + it;
    const int nv = cur.nv;
    const int64_t t0 = cur.t0;
    if (kOut && it < nchunks - 1) flush(prev_c, prev_t0, prev_nv);   // the previous step's outputs (published
                                                              // by its closing barrier)
    prev_c = c;
    prev_t0 = t0;
    prev_nv = nv;
    // ---- stage the chunk: k, q e^{gc} scale as hi + lo, -w, do, dv_local, gc
#pragma unroll
    for (int i = 0; i < D::UK; ++i) {
      const int u = tid + D::NT * i, r = u / (K / 8), cc = 8 * (u % (K / 8));
      const int o = toff<bf16>(r, cc, K);
      *reinterpret_cast<u32x4*>(s_k + o) = cur.k[i];
      u32x4 nw = cur.w[i];
#pragma unroll
      for (int e = 0; e < 4; ++e) nw[e] ^= 0x80008000u;  // -w
      *reinterpret_cast<u32x4*>(s_w + o) = nw;
      const float sc = r < nv ? gexp(cur.qs[i]) * a.scale : 0.f;
      const bf16x8 qv = __builtin_bit_cast(bf16x8, cur.q[i]);
      bf16x8 hi, lo;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = (float)qv[e] * sc;
        hi[e] = (bf16)x;
        lo[e] = (bf16)(x - (float)hi[e]);
      }
      *reinterpret_cast<bf16x8*>(s_qh + o) = hi;
      *reinterpret_cast<bf16x8*>(s_ql + o) = lo;
    }
#pragma unroll
    for (int i = 0; i < D::UV; ++i) {
      const int u = tid + D::NT * i, r = u / (V / 8), cc = 8 * (u % (V / 8));
      const int o = toff<bf16>(r, cc, V);
      *reinterpret_cast<u32x4*>(s_do + o) = cur.dO[i];
      *reinterpret_cast<u32x4*>(s_dvl + o) = cur.dvl[i];
    }
    if (wid == 0) s_g[l] = cur.gt;
    step_barrier();
    if (it > 0) dw_load<K, V>(nxt, a, chunk_start(it - 1), chunk_len(it - 1), h);

    // dh snapshot (before this chunk), row-major [NC, H, K, V], into its LDS tile
    if constexpr (kOut) {
#pragma unroll
      for (int tt = 0; tt < KT; ++tt)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 16 * tt + 4 * lg + j, col = c0 + lc;
          s_hs[r * V + 8 * swz_out<V>(r, col >> 3) + (col & 7)] = (bf16)dh[tt][j];
        }
    }
    // dv2 = e^{g_last - gc} (k bf16(dh)) + dv_local, rows t = 16 tm + 4 lg + j
    Frag<bf16> hb[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) hb[ks] = acc_frag<bf16>(dh[2 * ks], dh[2 * ks + 1]);
    const float gl = s_g[nv - 1];
    f32x4 dv[4];
#pragma unroll
    for (int tm = 0; tm < 4; ++tm) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) mma(acc, t_acc<bf16>(s_k, K, 16 * tm, 32 * ks), hb[ks]);
      const f32x4 g4 = *reinterpret_cast<const f32x4*>(s_g + 16 * tm + 4 * lg);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = 16 * tm + 4 * lg + j;
        const float dl = (float)s_dvl[toff<bf16>(t, c0 + lc, V)];
        dv[tm][j] = t < nv ? acc[j] * gexp(gl - g4[j]) + dl : 0.f;
        if constexpr (kOut) {
          const int col = c0 + lc;
          s_dv2[t * V + 8 * swz_out<V>(t, col >> 3) + (col & 7)] = (bf16)dv[tm][j];
        }
      }
    }
    // dh = e^{g_last} dh + (q e^{gc} scale)^T do - w^T bf16(dv2)
    Frag<bf16> bdo[2], bdv[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      bdo[ks] = t_tr<bf16>(s_do, V, 32 * ks, c0);
      bdv[ks] = acc_frag<bf16>(dv[2 * ks], dv[2 * ks + 1]);
    }
    const float eg = gexp(gl);
#pragma unroll
    for (int tt = 0; tt < KT; ++tt) {
      dh[tt] *= eg;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        mma(dh[tt], t_tr<bf16>(s_qh, K, 32 * ks, 16 * tt), bdo[ks]);
        mma(dh[tt], t_tr<bf16>(s_ql, K, 32 * ks, 16 * tt), bdo[ks]);
        mma(dh[tt], t_tr<bf16>(s_w, K, 32 * ks, 16 * tt), bdv[ks]);
      }
    }
    step_barrier();                                    // the tiles are restaged next chunk
    cur = nxt;
  }
  if (kOut && nchunks > 0) flush(prev_c, prev_t0, prev_nv);

  if (a.dh0) {
#pragma unroll
    for (int tt = 0; tt < KT; ++tt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t off = (((int64_t)n * H + h) * K + 16 * tt + 4 * lg + j) * V + c0 + lc;
        a.dh0[off] = dh[tt][j];
      }
  }
}

// ---------------------------------------------------------------------------
// dq, dk, dw, dg (chunk_o.py:147-326, USE_G and USE_DW).  Wave w owns tokens
// 16 w .. 16 w + 15 of the chunk.  Outputs are computed transposed ([d][t]
// tiles) so that each lane stores 4 consecutive d of one token.
// ---------------------------------------------------------------------------
template <typename TC>
__host__ __device__ constexpr size_t dqkwg_lds(int K) {
  return sizeof(TC) * (2 * (size_t)tile_elems<TC>(K) + tile_elems<TC>(64)) + (6 * 64 + 4) * sizeof(float);
}

template <typename TC, int K>
__global__ __launch_bounds__(NT_B) void bwd_dqkwg_kernel(BwdArgs a, int V) {
  extern __shared__ __align__(16) unsigned char smem[];
  TC* s_q = reinterpret_cast<TC*>(smem);
  TC* s_k = s_q + tile_elems<TC>(K);
  TC* s_ds = s_k + tile_elems<TC>(K);
  float* s_g = reinterpret_cast<float*>(s_ds + tile_elems<TC>(64));
  float* s_dgrow = s_g + 64;
  float* s_dgcol = s_dgrow + 64;                      // [4][64]: one row of column sums per wave
  float* s_dgl = s_dgcol + 4 * 64;                    // [4]: per-wave parts of the last row's extra term
  const int h = blockIdx.y, H = a.H;
  const int64_t c = blockIdx.x;
  const ChunkLoc loc = locate_chunk(c, a.cu, a.chunk_off, a.N, a.T);
  if (!loc.ok) return;
  const int64_t t0 = loc.t0;
  const int nv = loc.nv;
  const int wid = threadIdx.x / WAVE, l = lane_id(), lg = l >> 4, lc = l & 15;
  stage_rows<TC>(s_q, reinterpret_cast<const TC*>(a.q), t0, nv, H, h, K);
  stage_rows<TC>(s_k, reinterpret_cast<const TC*>(a.k), t0, nv, H, h, K);
  if (threadIdx.x < 64) s_g[threadIdx.x] = threadIdx.x < nv ? a.gc[(t0 + threadIdx.x) * H + h] : 0.f;
  __syncthreads();
  const float gl = s_g[nv - 1];

  const TC* do_ = reinterpret_cast<const TC*>(a.do_);
  const TC* vn = reinterpret_cast<const TC*>(a.vn);
  const TC* dv2 = reinterpret_cast<const TC*>(a.dv2);
  const int tr = 16 * wid + lc;                       // token of this lane's operand rows
  const bool tr_ok = tr < nv;
  const TC* do_row = do_ + ((t0 + (tr_ok ? tr : 0)) * H + h) * (int64_t)V;

  // ---- ds = mask_{i>=j}(do v_new^T e^{g_i - g_j}) scale; ds2 = ds * q k^T -> dg row and column sums
  float rowp[4] = {0.f, 0.f, 0.f, 0.f};
  for (int tj = 0; tj < 4; ++tj) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f}, aqk = {0.f, 0.f, 0.f, 0.f};
    if (tj <= wid) {
      const int tv = 16 * tj + lc;
      const TC* vn_row = vn + ((t0 + (tv < nv ? tv : 0)) * H + h) * (int64_t)V;
      for (int vs = 0; vs < V / 32; ++vs) mma(acc, g_nat<TC>(do_row, 32 * vs, tr_ok), g_nat<TC>(vn_row, 32 * vs, tv < nv));
#pragma unroll
      for (int ks = 0; ks < K / 32; ++ks) mma(aqk, t_nat<TC>(s_q, K, 16 * wid, 32 * ks), t_nat<TC>(s_k, K, 16 * tj, 32 * ks));
    }
    const int j = 16 * tj + lc;
    float colp = 0.f;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int i = 16 * wid + 4 * lg + jj;
      const bool m = i >= j && i < nv;
      const float ds = m ? acc[jj] * gexp(s_g[i] - s_g[j]) * a.scale : 0.f;
      const float ds2 = ds * aqk[jj];
      rowp[jj] += ds2;
      colp += ds2;
      s_ds[toff<TC>(i, j, 64)] = from_f32<TC>(ds);
    }
    colp = sum_lg(colp);                              // (plain stores and a fixed-order sum below:
    if (lg == 0) s_dgcol[wid * 64 + j] = colp;        //  dg is bitwise reproducible)
  }
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    const float r = sum16(rowp[jj]);
    if (lc == 0) s_dgrow[16 * wid + 4 * lg + jj] = r;
  }
  __syncthreads();

  // ---- per 16-row tile of K: dq, dk, -dw for this wave's 16 tokens
  const TC* hp = reinterpret_cast<const TC*>(a.h) + (c * H + h) * (int64_t)K * V;
  const TC* dhp = reinterpret_cast<const TC*>(a.dh) + (c * H + h) * (int64_t)K * V;
  const TC* vn_row = vn + ((t0 + (tr_ok ? tr : 0)) * H + h) * (int64_t)V;
  const TC* dv2_row = dv2 + ((t0 + (tr_ok ? tr : 0)) * H + h) * (int64_t)V;
  const int t = tr;                                   // output token of this lane (column lc of the tiles)
  const float eg = gexp(s_g[t]) * a.scale;
  const float gate = t < nv ? gexp(gl - s_g[t]) : 0.f;
  float dgt = 0.f, dglp = 0.f, hdh = 0.f;
  TC* dq_out = reinterpret_cast<TC*>(a.dq);
  TC* dk_out = reinterpret_cast<TC*>(a.dk1);
  TC* dw_out = reinterpret_cast<TC*>(a.dw);
  // bf16 with V <= 128: this wave's do, dv2 and v_new rows (the B operands of every K tile) are
  // loaded once into registers, and each K tile's h and dh fragments are all in flight before its
  // products
  constexpr bool kHoist = sizeof(TC) == 2;
  constexpr int VF = 4;                               // V / 32 fragments held (V <= 128)
  Frag<TC> fdo[VF], fdv2[VF], fvn[VF];
  const bool hoist = kHoist && V <= 32 * VF;
  if (hoist) {
#pragma unroll
    for (int vs = 0; vs < VF; ++vs) {
      if (vs < V / 32) {
        fdo[vs] = g_nat<TC>(do_row, 32 * vs, tr_ok);
        fdv2[vs] = g_nat<TC>(dv2_row, 32 * vs, tr_ok);
        fvn[vs] = g_nat<TC>(vn_row, 32 * vs, tr_ok);
      }
    }
  }
  for (int kt = 0; kt < K / 16; ++kt) {
    f32x4 aq = {0.f, 0.f, 0.f, 0.f}, ak = aq, aw = aq, aq2 = aq, ak2 = aq;
    const TC* hrow = hp + (16 * kt + lc) * (int64_t)V;
    const TC* dhrow = dhp + (16 * kt + lc) * (int64_t)V;
    if (hoist) {
      Frag<TC> hf[VF], dhf[VF];
#pragma unroll
      for (int vs = 0; vs < VF; ++vs) {
        if (vs < V / 32) {
          hf[vs] = g_nat<TC>(hrow, 32 * vs, true);
          dhf[vs] = g_nat<TC>(dhrow, 32 * vs, true);
        }
      }
#pragma unroll
      for (int vs = 0; vs < VF; ++vs) {
        if (vs < V / 32) {
          mma(aq, hf[vs], fdo[vs]);                   // sum_v h[k][v] do[t][v]
          mma(aw, hf[vs], fdv2[vs]);                  // sum_v h[k][v] dv2[t][v]
          mma(ak, dhf[vs], fvn[vs]);                  // sum_v dh[k][v] v_new[t][v]
          if (wid == 0) {
#pragma unroll
            for (int e = 0; e < 8; ++e) hdh += fget<TC>(hf[vs], e) * fget<TC>(dhf[vs], e);
          }
        }
      }
    } else {
      for (int vs = 0; vs < V / 32; ++vs) {
        const Frag<TC> hf = g_nat<TC>(hrow, 32 * vs, true);
        const Frag<TC> dhf = g_nat<TC>(dhrow, 32 * vs, true);
        mma(aq, hf, g_nat<TC>(do_row, 32 * vs, tr_ok));     // sum_v h[k][v] do[t][v]
        mma(aw, hf, g_nat<TC>(dv2_row, 32 * vs, tr_ok));    // sum_v h[k][v] dv2[t][v]
        mma(ak, dhf, g_nat<TC>(vn_row, 32 * vs, tr_ok));    // sum_v dh[k][v] v_new[t][v]
        if (wid == 0) {
#pragma unroll
          for (int e = 0; e < 8; ++e) hdh += fget<TC>(hf, e) * fget<TC>(dhf, e);
        }
      }
    }
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      mma(aq2, t_tr<TC>(s_k, K, 32 * s, 16 * kt), t_acc<TC>(s_ds, 64, 16 * wid, 32 * s));   // sum_t' k[t'][k] ds[t][t']
      mma(ak2, t_tr<TC>(s_q, K, 32 * s, 16 * kt), t_tr<TC>(s_ds, 64, 32 * s, 16 * wid));   // sum_i q[i][k] ds[i][t]
    }
    const int k0 = 16 * kt + 4 * lg;
    const f32x4 qv = t_row4<TC>(s_q, K, t, k0);
    const f32x4 kv = t_row4<TC>(s_k, K, t, k0);
    f32x4 dq, dk, dw;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const float dq1 = aq[jj] * eg;
      dgt += dq1 * qv[jj];
      dq[jj] = dq1 + aq2[jj];
      const float dk1 = ak[jj] * gate;
      dgt -= kv[jj] * dk1;
      dglp += dk1 * kv[jj];
      dk[jj] = dk1 + ak2[jj];
      dw[jj] = -aw[jj];
    }
    if (t < nv) {
      const int64_t o = ((t0 + t) * H + h) * (int64_t)K + k0;
      st4v<TC>(dq_out + o, dq);
      st4v<TC>(dk_out + o, dk);
      st4v<TC>(dw_out + o, dw);
    }
  }
  dgt = sum_lg(dgt);
  dglp = sum64(dglp);
  if (wid == 0) dglp += sum64(hdh) * gexp(gl);
  if (l == 0) s_dgl[wid] = dglp;
  __syncthreads();
  if (lg == 0 && t < nv) {
    float dg = s_dgrow[t] - (s_dgcol[t] + s_dgcol[64 + t] + s_dgcol[128 + t] + s_dgcol[192 + t]) + dgt;
    if (t == nv - 1) dg += s_dgl[0] + s_dgl[1] + s_dgl[2] + s_dgl[3];
    a.dg1[(t0 + t) * H + h] = dg;
  }
}

// ---------------------------------------------------------------------------
// WY backward (wy_fast.py:98-210, USE_G) with the final sums of chunk.py:140-145:
// dk = dk1 + dk2 (in the storage type), dg = reverse chunk cumsum of dg1 + dg2.
//
// G groups of four waves per chunk: wave w works on token tile ti = w % 4 and, within each phase, on
// the column tiles of group gq = w / 4: every G-th dA, dA1 and dA tile from gq, and the gq-th of G
// equal runs of consecutive K tiles of dk and V tiles of dv (so that each token's dk and dv row pieces
// of one wave fill whole 128-byte lines).  Sums over a token's columns (dg, dbeta) leave each group as one LDS row
// per group and are added in group order by the last phase, so the gradients are reproducible.
// ---------------------------------------------------------------------------
template <typename TC, int G = 1>
__host__ __device__ constexpr size_t wy_lds(int K, int V) {
  return sizeof(TC) * (2 * (size_t)tile_elems<TC>(K) + tile_elems<TC>(V) + 3 * (size_t)tile_elems<TC>(64)) +
         (6 + 2 * G) * 64 * sizeof(float);
}

template <typename TC, int K, int G>
__global__ __launch_bounds__(NT_B * G) void bwd_wy_kernel(BwdArgs a, int V) {
  static_assert(G == 1 || G == 2 || G == 4, "four, eight or sixteen waves");
  extern __shared__ __align__(16) unsigned char smem[];
  TC* s_k = reinterpret_cast<TC*>(smem);
  TC* s_dw = s_k + tile_elems<TC>(K);
  TC* s_du = s_dw + tile_elems<TC>(K);
  TC* s_Ai = s_du + tile_elems<TC>(V);
  TC* s_dA = s_Ai + tile_elems<TC>(64);
  TC* s_dA1 = s_dA + tile_elems<TC>(64);
  float* s_g = reinterpret_cast<float*>(s_dA1 + tile_elems<TC>(64));
  float* s_b = s_g + 64;
  float* s_dgc = s_b + 64;                            // [4][64]: column parts of dg2, one row per token tile
  float* s_dgp = s_dgc + 4 * 64;                      // [G][64]: row parts of dg2 (+ dkbg.kbg), one row per group
  float* s_dbp = s_dgp + G * 64;                      // [G][64]: dbeta, one row per group
  const int h = blockIdx.y, H = a.H;
  const ChunkLoc loc = locate_chunk(blockIdx.x, a.cu, a.chunk_off, a.N, a.T);
  if (!loc.ok) return;
  const int64_t t0 = loc.t0;
  const int nv = loc.nv;
  const int wid = threadIdx.x / WAVE, l = lane_id(), lg = l >> 4, lc = l & 15;
  const int ti = wid & 3, gq = wid >> 2;              // token tile, group
  if constexpr (sizeof(TC) == 2) {
    stage_rows_dma(s_k, reinterpret_cast<const TC*>(a.k), t0, nv, H, h, K);
    stage_rows_dma(s_dw, reinterpret_cast<const TC*>(a.dw), t0, nv, H, h, K);
    stage_rows_dma(s_du, reinterpret_cast<const TC*>(a.dv2), t0, nv, H, h, V);
    stage_rows_dma(s_Ai, reinterpret_cast<const TC*>(a.Ai), t0, nv, H, h, 64);
  } else {
    stage_rows<TC>(s_k, reinterpret_cast<const TC*>(a.k), t0, nv, H, h, K);
    stage_rows<TC>(s_dw, reinterpret_cast<const TC*>(a.dw), t0, nv, H, h, K);
    stage_rows<TC>(s_du, reinterpret_cast<const TC*>(a.dv2), t0, nv, H, h, V);
    stage_rows<TC>(s_Ai, reinterpret_cast<const TC*>(a.Ai), t0, nv, H, h, 64);
  }
  if (threadIdx.x < 64) {
    const int r = threadIdx.x;
    s_g[r] = r < nv ? a.gc[(t0 + r) * H + h] : 0.f;
    s_b[r] = r < nv ? ld_scalar(a.beta, (t0 + r) * H + h, a.beta_dtype) : 0.f;
  }
  // this lane's token of the last phase: its dk1 row pieces (the group's K tiles) and the first batch
  // of its v row pieces.  With four waves they go out now, so that their latency passes under the
  // staging and the dA phases; with more waves (a quarter of the registers each) before the last phase.
  const int t = 16 * ti + lc;
  constexpr int NKT = K / 16 / G;                     // K tiles of this group: kt = NKT gq + i
  const TC* dk1 = reinterpret_cast<const TC*>(a.dk1);
  f32x4 d1s[NKT];                                     // (rows past the end read row 0: dk is not stored there)
  const TC* vtok = reinterpret_cast<const TC*>(a.v) + ((t0 + (t < nv ? t : 0)) * H + h) * (int64_t)V + 4 * lg;
  const int nvt = V / 16, vt0 = nvt / G * gq, vt1 = vt0 + nvt / G;   // V tiles; this group's: vt0 .. vt1 - 1
  f32x4 vnext[4];                                     // v of this group's V tiles m .. m + 3
  auto load_dk1 = [&]() {
#pragma unroll
    for (int i = 0; i < NKT; ++i)
      d1s[i] = g_row4<TC>(dk1 + ((t0 + (t < nv ? t : 0)) * H + h) * (int64_t)K + 16 * (NKT * gq + i) + 4 * lg);
  };
  auto load_v = [&](int m) {                          // (rows past the end read row 0: their dbeta is not stored)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int vt = vt0 + m + e;
      vnext[e] = vt < vt1 ? g_row4<TC>(vtok + 16 * vt) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  if constexpr (G == 1) {
    load_dk1();
    load_v(0);
  }
  stage_wait();
  __syncthreads();

  // ---- dA = dw bf16(k beta e^g)^T + du bf16(v beta)^T, strictly lower (tile ti x tj; zeros above)
  const TC* v = reinterpret_cast<const TC*>(a.v);
  for (int tj = gq; tj < 4; tj += G) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    if (tj <= ti) {
      const int j = 16 * tj + lc;                     // operand row of the B fragments
      const float fk = s_b[j] * gexp(s_g[j]);
#pragma unroll
      for (int ks = 0; ks < K / 32; ++ks)
        mma(acc, t_nat<TC>(s_dw, K, 16 * ti, 32 * ks), fscale<TC>(t_nat<TC>(s_k, K, 16 * tj, 32 * ks), fk));
      // this tile's v rows: every fragment's load of a batch in flight before its products (all of
      // them with four waves, eight at a time with more: the layer-shape backward 7.74 -> 7.69 ms
      // against four, 7.73 with all sixteen)
      const TC* vrow = v + ((t0 + (j < nv ? j : 0)) * H + h) * (int64_t)V;
      constexpr int NVF = sizeof(TC) == 2 ? 16 : 4;     // V / 32 at most (bf16 V <= 512, fp32 V <= 128)
      constexpr int NVB = G == 1 ? NVF : 8;
      // (raw loads in the V-guarded blocks, the mask of rows past the end applied at the products:
      // a use of the value inside its block would wait for each load before the next is issued)
      const bool jv = j < nv;
#pragma unroll
      for (int vb = 0; vb < NVF; vb += NVB) {
        if (32 * vb < V) {
          Frag<TC> vf[NVB];
#pragma unroll
          for (int vs = 0; vs < NVB; ++vs)
            if (vb + vs < V / 32) vf[vs] = g_nat<TC>(vrow, 32 * (vb + vs), true);
#pragma unroll
          for (int vs = 0; vs < NVB; ++vs)
            if (vb + vs < V / 32)
              mma(acc, t_nat<TC>(s_du, V, 16 * ti, 32 * (vb + vs)), fscale<TC>(jv ? vf[vs] : fzero<TC>(), s_b[j]));
        }
      }
    }
    const int j = 16 * tj + lc;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int i = 16 * ti + 4 * lg + jj;
      s_dA[toff<TC>(i, j, 64)] = from_f32<TC>(i > j && i < nv ? acc[jj] : 0.f);
    }
  }
  __syncthreads();
  // ---- dA1 = bf16(dA) Ai^T
  for (int tc = gq; tc < 4; tc += G) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 2; ++s) mma(acc, t_nat<TC>(s_dA, 64, 16 * ti, 32 * s), t_nat<TC>(s_Ai, 64, 16 * tc, 32 * s));
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) s_dA1[toff<TC>(16 * ti + 4 * lg + jj, 16 * tc + lc, 64)] = from_f32<TC>(acc[jj]);
  }
  __syncthreads();
  // ---- dA = -(Ai^T bf16(dA1)) e^{g_t - g_c}, strictly lower; AdA = dA * (bf16(k beta) k^T) -> dg
  float rowp[4] = {0.f, 0.f, 0.f, 0.f};
  {
    const float fb = s_b[16 * ti + lc];               // beta of the A fragment's row
    for (int tc = gq; tc < 4; tc += G) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f}, a2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 2; ++s) mma(acc, t_tr<TC>(s_Ai, 64, 32 * s, 16 * ti), t_tr<TC>(s_dA1, 64, 32 * s, 16 * tc));
#pragma unroll
      for (int ks = 0; ks < K / 32; ++ks)
        mma(a2, fscale<TC>(t_nat<TC>(s_k, K, 16 * ti, 32 * ks), fb), t_nat<TC>(s_k, K, 16 * tc, 32 * ks));
      const int cc = 16 * tc + lc;
      float colp = 0.f;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int tt = 16 * ti + 4 * lg + jj;
        const bool m = tt > cc && tt < nv;
        const float dA = round_to<TC>(m ? -acc[jj] * gexp(s_g[tt] - s_g[cc]) : 0.f);
        s_dA[toff<TC>(tt, cc, 64)] = from_f32<TC>(dA);
        const float ada = dA * a2[jj];
        rowp[jj] += ada;
        colp += ada;
      }
      colp = sum_lg(colp);
      if (lg == 0) s_dgc[ti * 64 + cc] = -colp;
    }
  }
  float rowsum[4];
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) rowsum[jj] = sum16(rowp[jj]);
  if (lc == 0) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) s_dgp[gq * 64 + 16 * ti + 4 * lg + jj] = rowsum[jj];
  }
  __syncthreads();

  // ---- per token tile ti, this group's K and V tiles: dk2, dk, dv, dbeta and the dkbg.kbg part of dg
  if constexpr (G > 1) {
    load_dk1();
    load_v(0);
  }
  const float bt = s_b[t], egt = gexp(s_g[t]);
  Frag<TC> bAi[2], bdA[2], bdAt[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    bAi[s] = t_tr<TC>(s_Ai, 64, 32 * s, 16 * ti);      // B[n = t][j] = Ai[j][t]
    bdA[s] = t_acc<TC>(s_dA, 64, 16 * ti, 32 * s);     // B[n = t][j] = dA[t][j]
    bdAt[s] = t_tr<TC>(s_dA, 64, 32 * s, 16 * ti);     // B[n = t][j] = dA[j][t]
  }
  float dbt = 0.f, dgt = 0.f;
  TC* dk_out = reinterpret_cast<TC*>(a.dk);
#pragma unroll
  for (int i = 0; i < NKT; ++i) {
    const int kt = NKT * gq + i;
    f32x4 a1 = {0.f, 0.f, 0.f, 0.f}, a2 = a1, a3 = a1;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      mma(a1, t_tr<TC>(s_dw, K, 32 * s, 16 * kt), bAi[s]);     // dkbg^T[k][t] = sum_j dw[j][k] Ai[j][t]
      const Frag<TC> kT = t_tr<TC>(s_k, K, 32 * s, 16 * kt);
      mma(a2, kT, bdA[s]);                                    // dkb^T[k][t] = sum_j k[j][k] dA[t][j]
      Frag<TC> kbT;                                           // bf16(k beta)^T: K index = row j
#pragma unroll
      for (int e = 0; e < 8; ++e) fset<TC>(kbT, e, fget<TC>(kT, e) * s_b[32 * s + acc_row(e)]);
      mma(a3, kbT, bdAt[s]);                                  // (dA^T kb)^T[k][t]
    }
    const int k0 = 16 * kt + 4 * lg;
    const f32x4 kv = t_row4<TC>(s_k, K, t, k0);
    const f32x4 d1 = d1s[i];
    f32x4 dk;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const float dkr = round_to<TC>(a1[jj] * egt * bt);
      dbt += a1[jj] * kv[jj] * egt + a2[jj] * kv[jj];
      dgt += a1[jj] * (kv[jj] * bt * egt);
      const float dk2 = round_to<TC>(dkr + a3[jj] + a2[jj] * bt);
      dk[jj] = d1[jj] + dk2;
    }
    if (t < nv) st4v<TC>(dk_out + ((t0 + t) * H + h) * (int64_t)K + k0, dk);
  }
  TC* dv_out = reinterpret_cast<TC*>(a.dv);
  // batches of 4 of this group's V tiles, the next batch's v loads issued before this batch's products
  for (int m0 = 0; vt0 + m0 < vt1; m0 += 4) {
    f32x4 vv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) vv[e] = vnext[e];
    load_v(m0 + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int vt = vt0 + m0 + e;
      if (vt < vt1) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 2; ++s) mma(acc, t_tr<TC>(s_du, V, 32 * s, 16 * vt), bAi[s]);   // dvb^T[v][t]
        const int v0 = 16 * vt + 4 * lg;
        if (t < nv) {
          f32x4 dv;
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            dv[jj] = acc[jj] * bt;
            dbt += acc[jj] * vv[e][jj];
          }
          st4v<TC>(dv_out + ((t0 + t) * H + h) * (int64_t)V + v0, dv);
        }
      }
    }
  }
  dbt = sum_lg(dbt);
  dgt = sum_lg(dgt);
  if (lg == 0) {
    s_dgp[gq * 64 + t] += dgt;                        // token t's entry of this group's row is this wave's
    s_dbp[gq * 64 + t] = dbt;
  }
  __syncthreads();
  // ---- dbeta = the groups' parts in group order; dg = reverse cumsum within the chunk of dg1 + dg2
  if (wid == 0) {
    float x = 0.f, db = 0.f;
    if (l < nv) {
      float rp = s_dgp[l];
#pragma unroll
      for (int q = 1; q < G; ++q) rp += s_dgp[q * 64 + l];
      x = a.dg1[(t0 + l) * H + h] + rp + (s_dgc[l] + s_dgc[64 + l] + s_dgc[128 + l] + s_dgc[192 + l]);
      db = s_dbp[l];
#pragma unroll
      for (int q = 1; q < G; ++q) db += s_dbp[q * 64 + l];
      const int64_t o = (t0 + l) * H + h;
      if (a.beta_dtype == DT_F32) reinterpret_cast<float*>(a.db)[o] = db;
      else reinterpret_cast<bf16*>(a.db)[o] = (bf16)db;
    }
#pragma unroll
    for (int o = 1; o < WAVE; o <<= 1) {
      const float y = __shfl_down(x, o, WAVE);
      if (l + o < WAVE) x += y;
    }
    if (l < nv) a.dg[(t0 + l) * H + h] = x;
  }
}

// ---------------------------------------------------------------------------
// l2norm backward (l2norm.py:132-154) with rstd and y recomputed from the input x:
// rstd = 1 / sqrt(sum x^2 + 1e-6), y = x rstd (rounded), dx = dy rstd - sum(dy y) y rstd.
// One wave per row, D <= 512.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void l2norm_bwd_kernel(const T* __restrict__ x, const T* __restrict__ dy,
                                                         T* __restrict__ dx, int64_t rows, int D) {
  const int64_t row = (int64_t)blockIdx.x * 4 + threadIdx.x / WAVE;
  if (row >= rows) return;
  const int l = lane_id();
  const bool act = 8 * l < D;
  Vec8<T> xv = vzero<T>(), gv = vzero<T>();
  if (act) {
    xv = ld8<T>(x + row * D + 8 * l);
    gv = ld8<T>(dy + row * D + 8 * l);
  }
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss = fmaf(vget<T>(xv, e), vget<T>(xv, e), ss);
  ss = sum64(ss);
  const float rstd = 1.0f / sqrtf(ss + 1e-6f);
  float y[8], dot = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    y[e] = round_to<T>(vget<T>(xv, e) * rstd);
    dot = fmaf(vget<T>(gv, e), y[e], dot);
  }
  dot = sum64(dot);
  if (act) {
    Vec8<T> o;
#pragma unroll
    for (int e = 0; e < 8; ++e) vset<T>(o, e, vget<T>(gv, e) * rstd - dot * y[e] * rstd);
    st8<T>(dx + row * D + 8 * l, o);
  }
}

// The same for D a power of two (8 .. 512): a row takes LPR = D / 8 lanes, a wave holds 64 / LPR rows,
// and each thread handles RPT row groups with all their loads issued before the first reduction (the
// one-wave-per-row form leaves lanes idle below D = 512 and keeps one row's loads in flight).
template <typename T, int D>
__global__ __launch_bounds__(256) void l2norm_bwd_rows_kernel(const T* __restrict__ x, const T* __restrict__ dy,
                                                              T* __restrict__ dx, int64_t rows) {
  constexpr int LPR = D / 8, RPW = WAVE / LPR, RPT = 4;
  const int l = lane_id();
  const int64_t wave = ((int64_t)blockIdx.x * 4 + threadIdx.x / WAVE) * RPT;
  const int sub = l / LPR, col = 8 * (l % LPR);
  Vec8<T> xv[RPT], gv[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int64_t row = (wave + i) * RPW + sub;
    xv[i] = row < rows ? ld8<T>(x + row * D + col) : vzero<T>();
    gv[i] = row < rows ? ld8<T>(dy + row * D + col) : vzero<T>();
  }
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int64_t row = (wave + i) * RPW + sub;
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = fmaf(vget<T>(xv[i], e), vget<T>(xv[i], e), ss);
#pragma unroll
    for (int off = LPR / 2; off > 0; off >>= 1) ss += __shfl_xor(ss, off, WAVE);
    const float rstd = 1.0f / sqrtf(ss + 1e-6f);
    float y[8], dot = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      y[e] = round_to<T>(vget<T>(xv[i], e) * rstd);
      dot = fmaf(vget<T>(gv[i], e), y[e], dot);
    }
#pragma unroll
    for (int off = LPR / 2; off > 0; off >>= 1) dot += __shfl_xor(dot, off, WAVE);
    if (row < rows) {
      Vec8<T> o;
#pragma unroll
      for (int e = 0; e < 8; ++e) vset<T>(o, e, vget<T>(gv[i], e) * rstd - dot * y[e] * rstd);
      st8<T>(dx + row * D + col, o);
    }
  }
}

template <typename K_>
int set_lds(K_ kern, size_t bytes) {
  if (bytes > 64 * 1024 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)bytes) != hipSuccess)
    return -1;
  return 0;
}

template <typename TC, int K>
int launch_bwd_t(const BwdArgs& a, int V, int64_t nc_grid, int stages, hipStream_t s) {
  const dim3 grid((unsigned)nc_grid, (unsigned)a.H);
  if (nc_grid > 0 && (stages & BWD_DVL)) {
    // eight waves where the tiles leave room for one workgroup per CU, sixteen where two fit
    // (KAIROS_GDN_BWD_DVL_WAVES=4, 8 or 16 forces one).  Backward measured with 16 / 8 / 4 waves:
    // 7.79 / 7.74 / 7.75 ms at dk = 256, dv = 512, T = 32760, H = 20; 2.633 / 2.637 / 2.652 ms at
    // dk = dv = 128.
    const size_t l1 = dvl_lds<TC>(K, V);
    if (l1 > 160 * 1024) return -1;
    const char* e = std::getenv("KAIROS_GDN_BWD_DVL_WAVES");
    const int want = e ? std::atoi(e) : 0;
    bool split = false;
    if constexpr (sizeof(TC) == 2 && K >= 128) {       // the halves form (KAIROS_GDN_BWD_DVL_SPLIT=0: whole tiles)
      const char* es = std::getenv("KAIROS_GDN_BWD_DVL_SPLIT");
      constexpr int VB = K;
      if (V % VB == 0 && want == 0 && !(es && es[0] == '0' && es[1] == 0)) {
        constexpr size_t lds_s = dvl_split_lds<K, VB>();
        hipLaunchKernelGGL((bwd_dvl_split_kernel<K, VB>), grid, dim3(64 * DVL_SPLIT_NW), lds_s, s, a, V);
        split = true;
      }
    }
    const int nw = want == 4 || want == 8 || want == 16 ? want : l1 > 80 * 1024 ? 8 : 16;
    if (split) {
    } else if (nw == 16) {
      if (set_lds(bwd_dvl_kernel<TC, K, 16>, l1)) return -1;
      hipLaunchKernelGGL((bwd_dvl_kernel<TC, K, 16>), grid, dim3(64 * 16), l1, s, a, V);
    } else if (nw == 8) {
      if (set_lds(bwd_dvl_kernel<TC, K, 8>, l1)) return -1;
      hipLaunchKernelGGL((bwd_dvl_kernel<TC, K, 8>), grid, dim3(64 * 8), l1, s, a, V);
    } else {
      if (set_lds(bwd_dvl_kernel<TC, K, 4>, l1)) return -1;
      hipLaunchKernelGGL((bwd_dvl_kernel<TC, K, 4>), grid, dim3(64 * 4), l1, s, a, V);
    }
  }
  if (stages & BWD_DHU) {
    bool wide = false;
    if constexpr (sizeof(TC) == 2 && K == 256) {
      if (a.qT && a.wT && a.dh && a.dv2) {
        if (int rc = launch_wide_dhu(a, V, s)) return rc;
        wide = true;
      }
    }
    if constexpr (sizeof(TC) == 2 && K <= 128) {
      if (V == 64 || V == 128) {
        const char* e = std::getenv("KAIROS_GDN_BWD_DHU_WIDE");
        wide = !(e && e[0] == '0' && e[1] == 0);
      }
      if (wide) {
        const int total = a.N * a.H;
        const int g8 = (total + 7) / 8 * 8;
        if (total > 0) {
          if (V == 64) {
            using D = DW<K, 64>;
            constexpr int nt = D::NT;
            constexpr size_t lds = D::lds;
            if (a.dh || a.dv2) {
              if (set_lds(bwd_dhu_wide_kernel<K, 64, true>, lds)) return -1;
              hipLaunchKernelGGL((bwd_dhu_wide_kernel<K, 64, true>), dim3(g8), dim3(nt), lds, s, a, total);
            } else {
              if (set_lds(bwd_dhu_wide_kernel<K, 64, false>, lds)) return -1;
              hipLaunchKernelGGL((bwd_dhu_wide_kernel<K, 64, false>), dim3(g8), dim3(nt), lds, s, a, total);
            }
          } else {
            using D = DW<K, 128>;
            constexpr int nt = D::NT;
            constexpr size_t lds = D::lds;
            if (a.dh || a.dv2) {
              if (set_lds(bwd_dhu_wide_kernel<K, 128, true>, lds)) return -1;
              hipLaunchKernelGGL((bwd_dhu_wide_kernel<K, 128, true>), dim3(g8), dim3(nt), lds, s, a, total);
            } else {
              if (set_lds(bwd_dhu_wide_kernel<K, 128, false>, lds)) return -1;
              hipLaunchKernelGGL((bwd_dhu_wide_kernel<K, 128, false>), dim3(g8), dim3(nt), lds, s, a, total);
            }
          }
        }
      }
    }
    if (!wide) {
      const int total = a.N * a.H * (V / DBV);
      const int g8 = (total + 7) / 8 * 8;
      if (total > 0) hipLaunchKernelGGL((bwd_dhu_kernel<TC, K>), dim3(g8), dim3(64 * DCfg<K>::NW), 0, s, a, V, total);
    }
  }
  if (nc_grid > 0 && (stages & BWD_GRADS)) {
    bool wide = false;
    if constexpr (sizeof(TC) == 2 && K >= 128) {      // eight waves per chunk (KAIROS_GDN_BWD_DQK_WIDE=0: four)
      wide = bwd_dqk_wide(DT_BF16, K);
      if (wide) {
        if (int rc = launch_wide_dqkwg(a, K, V, nc_grid, s)) return rc;
      }
    }
    if (!wide && a.rq) return -2;                     // the q side of the L2 backward lives in the wide kernel
    if (!wide) {
      const size_t l3 = dqkwg_lds<TC>(K);
      if (set_lds(bwd_dqkwg_kernel<TC, K>, l3)) return -1;
      hipLaunchKernelGGL((bwd_dqkwg_kernel<TC, K>), grid, dim3(NT_B), l3, s, a, V);
    }
    // WY: groups of four waves per chunk (bf16).  Sixteen waves where a workgroup's LDS leaves room
    // for no second one on a CU (dk = 256: with four waves, 4 per CU), eight where two fit (16 per
    // CU, the two overlapping each other's staging).  Measured, sixteen / eight / four waves: 7.89 /
    // 8.02 / 8.24 ms for the backward at dk = 256, dv = 512, T = 32760, H = 20; 2.79 / 2.67 / 2.72 ms
    // at dk = dv = 128.  KAIROS_GDN_BWD_WY_WAVES=4, 8 or 16 forces one.
    int wg = 1;
    if constexpr (sizeof(TC) == 2) {
      const char* e = std::getenv("KAIROS_GDN_BWD_WY_WAVES");
      const int want = e ? std::atoi(e) : 0;
      wg = want == 4 ? 1 : want == 8 ? 2 : want == 16 ? 4 : (wy_lds<TC, 2>(K, V) > 80 * 1024 ? 4 : 2);
      if (wy_lds<TC, 4>(K, V) > 160 * 1024) wg = 1;
      if (wg == 4) {
        const size_t l4 = wy_lds<TC, 4>(K, V);
        if (set_lds(bwd_wy_kernel<TC, K, 4>, l4)) return -1;
        hipLaunchKernelGGL((bwd_wy_kernel<TC, K, 4>), grid, dim3(NT_B * 4), l4, s, a, V);
      } else if (wg == 2) {
        const size_t l4 = wy_lds<TC, 2>(K, V);
        if (set_lds(bwd_wy_kernel<TC, K, 2>, l4)) return -1;
        hipLaunchKernelGGL((bwd_wy_kernel<TC, K, 2>), grid, dim3(NT_B * 2), l4, s, a, V);
      }
    }
    if (wg == 1) {
      const size_t l4 = wy_lds<TC, 1>(K, V);
      if (l4 > 160 * 1024 || set_lds(bwd_wy_kernel<TC, K, 1>, l4)) return -1;
      hipLaunchKernelGGL((bwd_wy_kernel<TC, K, 1>), grid, dim3(NT_B), l4, s, a, V);
    }
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace

bool bwd_dqk_wide(int compute_dtype, int K) {
  if (compute_dtype != DT_BF16 || K < 128) return false;
  const char* e = std::getenv("KAIROS_GDN_BWD_DQK_WIDE");
  return !(e && e[0] == '0' && e[1] == 0);
}

bool bwd_supported(int compute_dtype, int K, int V) {
  if (V <= 0 || V % 64 != 0 || !(K == 64 || K == 128 || K == 256)) return false;
  if (compute_dtype == DT_BF16) return V <= 512 && wy_lds<bf16>(K, V) <= 160 * 1024 && dvl_lds<bf16>(K, V) <= 160 * 1024;
  if (compute_dtype == DT_F32) return K <= 128 && V <= 128;
  return false;
}

int launch_bwd(const BwdArgs& a, int compute_dtype, int K, int V, int64_t nc_grid, int stages, hipStream_t s) {
  if (!bwd_supported(compute_dtype, K, V)) return -2;
#define KGDN_B_CASE(TC, KK) \
  if (K == KK) return launch_bwd_t<TC, KK>(a, V, nc_grid, stages, s);
  if (compute_dtype == DT_BF16) { KGDN_B_CASE(bf16, 64) KGDN_B_CASE(bf16, 128) KGDN_B_CASE(bf16, 256) }
  if (compute_dtype == DT_F32) { KGDN_B_CASE(float, 64) KGDN_B_CASE(float, 128) }
#undef KGDN_B_CASE
  return -2;
}

template <typename T>
bool launch_l2norm_bwd_rows(const void* x, const void* dy, void* dx, int64_t rows, int D, hipStream_t s) {
  auto go = [&](auto kern, int lpr) {
    const int64_t per_block = 4 * 4 * (WAVE / lpr);        // waves x row groups x rows per group
    hipLaunchKernelGGL(kern, dim3((unsigned)((rows + per_block - 1) / per_block)), dim3(256), 0, s,
                       static_cast<const T*>(x), static_cast<const T*>(dy), static_cast<T*>(dx), rows);
    return true;
  };
  switch (D) {
    case 64: return go(l2norm_bwd_rows_kernel<T, 64>, 8);
    case 128: return go(l2norm_bwd_rows_kernel<T, 128>, 16);
    case 256: return go(l2norm_bwd_rows_kernel<T, 256>, 32);
    case 512: return go(l2norm_bwd_rows_kernel<T, 512>, 64);
    default: return false;
  }
}

int launch_l2norm_bwd(const void* x, const void* dy, void* dx, int dtype, int64_t rows, int D, hipStream_t s) {
  if (D % 8 != 0 || D > 512 || rows <= 0) return -2;
  if (dtype == DT_F32 && launch_l2norm_bwd_rows<float>(x, dy, dx, rows, D, s))
    return hipGetLastError() == hipSuccess ? 0 : -1;
  if (dtype == DT_BF16 && launch_l2norm_bwd_rows<bf16>(x, dy, dx, rows, D, s))
    return hipGetLastError() == hipSuccess ? 0 : -1;
  const dim3 grid((unsigned)((rows + 3) / 4));
  if (dtype == DT_F32) {
    hipLaunchKernelGGL(l2norm_bwd_kernel<float>, grid, dim3(256), 0, s, static_cast<const float*>(x),
                       static_cast<const float*>(dy), static_cast<float*>(dx), rows, D);
  } else if (dtype == DT_BF16) {
    hipLaunchKernelGGL(l2norm_bwd_kernel<bf16>, grid, dim3(256), 0, s, static_cast<const bf16*>(x),
                       static_cast<const bf16*>(dy), static_cast<bf16*>(dx), rows, D);
  } else {
    return -2;
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace kgdn
