// Serial inter-chunk state recurrence of the chunked GatedDeltaNet forward
// (fla ops/common/chunk_delta_h.py:52-224).  For each (sequence, head,
// 16-column slice of V) one workgroup walks the chunks in order:
//
//   hT[c]  = S (stored, before the update)               chunk_delta_h.py:129-139
//   v'     = u_c - w_c @ S_stored                        :141-157
//   vnT[c] = v' (stored, ungated)                         :159-161
//   S      = exp(g_last) S + k_c^T (v' exp(g_last - gc)) :163-211
//   ht     = S after the last chunk (fp32)               :213-224
//
// The fp32 state slice S[K x 16] stays in VGPRs for the whole sequence, in the
// MFMA accumulator layout, split over the waves along K (each wave owns KW
// rows).  The accumulator tile is fed back as the B operand of w @ S without
// a shuffle: the K index of a 32-deep step is permuted the same way in the w
// fragment (two 4-element pieces per lane).  Partial w @ S products of the
// waves are summed through LDS; the gated v' goes through LDS once more as the
// B operand of the rank-64 update.  Everything the next chunk needs (w, k, u,
// gc) is prefetched into registers while the current chunk computes.
#include <cstdlib>

#include "gdn_common.hpp"
#include "gdn_kernels.h"
#include "gdn_tiles.hpp"

namespace kgdn {

namespace {

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int BV = 16;     // V columns per workgroup
constexpr int LDT = C + 8; // row stride of the [*][64] LDS tiles

template <int K> struct HCfg {
  static constexpr int NW = K == 64 ? 2 : 4;   // waves
  static constexpr int KW = K / NW;            // state rows per wave
  static constexpr int KT = KW / 16;           // 16-row accumulator tiles per wave
  static constexpr int KS = KW / 32;           // 32-deep K steps per wave
  static constexpr int OWN = 4 / NW;           // 16-row tiles of v' reduced by each wave
};

// Workgroup barrier that waits for LDS operations only (lgkmcnt(0), s_barrier): the waves share
// only LDS within a chunk step, and __syncthreads() would also wait for the next chunk's prefetch
// (vmcnt(0)) and this chunk's stores.  The empty asm statements keep memory accesses from moving
// across the barrier.
__device__ __forceinline__ void step_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);          // lgkmcnt(0); vmcnt, expcnt at their maxima
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <typename TC> struct Half;             // 4 storage elements (8 B bf16 / 16 B fp32)
template <> struct Half<bf16> { bf16x4 v; };
template <> struct Half<float> { f32x4 v; };

template <typename TC>
__device__ __forceinline__ Half<TC> ld_half(const TC* p) {
  Half<TC> r;
  if constexpr (sizeof(TC) == 2) r.v = *reinterpret_cast<const bf16x4*>(p);
  else r.v = *reinterpret_cast<const f32x4*>(p);
  return r;
}
template <typename TC>
__device__ __forceinline__ Half<TC> zero_half() {
  Half<TC> r;
#pragma unroll
  for (int e = 0; e < 4; ++e) r.v[e] = (TC)0.f;
  return r;
}
template <typename TC>
__device__ __forceinline__ Frag<TC> join(const Half<TC>& a, const Half<TC>& b) {
  Frag<TC> f;
  if constexpr (sizeof(TC) == 2) {
    f.v = __builtin_shufflevector(a.v, b.v, 0, 1, 2, 3, 4, 5, 6, 7);
  } else {
    f.lo = a.v;
    f.hi = b.v;
  }
  return f;
}
template <typename TC>
__device__ __forceinline__ Frag<TC> frag_from_acc(const f32x4& a, const f32x4& b) {
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

template <typename TC, typename TK, int K>
struct ChunkPrefetch {
  using Cfg = HCfg<K>;
  Frag<TC> wf[4][Cfg::KS];      // A fragments of w for the 4 row tiles
  Vec8<TC> krow[Cfg::KW / 8];   // k[t = lane][wave's K slice]
  f32x4 uv[Cfg::OWN];           // u (C layout) of the owned row tiles
  f32x4 gv[Cfg::OWN];           // gc of the owned rows
  float gl;                     // gc of the last valid row
  int64_t t0;
  int nv;
};

template <typename TC, typename TK, int K>
__device__ __forceinline__ void prefetch_chunk(ChunkPrefetch<TC, TK, K>& P, const FwdHArgs& a, int64_t c,
                                               int64_t t0, int nv, int h, int v0, int wid, int V) {
  using Cfg = HCfg<K>;
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;
  const int H = a.H;
  P.t0 = t0;
  P.nv = nv;
  const TC* w = reinterpret_cast<const TC*>(a.w);
#pragma unroll
  for (int tm = 0; tm < 4; ++tm) {
    const int t = 16 * tm + lc;
#pragma unroll
    for (int ks = 0; ks < Cfg::KS; ++ks) {
      if (t < nv) {
        const TC* p = w + ((t0 + t) * H + h) * K + Cfg::KW * wid + 32 * ks + 4 * lg;
        P.wf[tm][ks] = join<TC>(ld_half<TC>(p), ld_half<TC>(p + 16));
      } else {
        P.wf[tm][ks] = join<TC>(zero_half<TC>(), zero_half<TC>());
      }
    }
  }
  const TK* k = reinterpret_cast<const TK*>(a.k);
  const float ks_ = a.k_scale ? a.k_scale[h] : 1.f;
#pragma unroll
  for (int d8 = 0; d8 < Cfg::KW / 8; ++d8) {
    float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (l < nv) load8_in<TK>(k + ((t0 + l) * H + h) * K + Cfg::KW * wid + 8 * d8, ks_, x);
#pragma unroll
    for (int e = 0; e < 8; ++e) vset<TC>(P.krow[d8], e, x[e]);
  }
  const TC* uT = reinterpret_cast<const TC*>(a.uT) + ((c * H + h) * V + v0 + lc) * C;
#pragma unroll
  for (int o = 0; o < Cfg::OWN; ++o) {
    const int tm = wid + Cfg::NW * o;
    P.uv[o] = ld4<TC>(uT + 16 * tm + 4 * lg);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = 16 * tm + 4 * lg + j;
      P.gv[o][j] = t < nv ? a.gc[(t0 + t) * H + h] : 0.f;
    }
  }
  P.gl = a.gc[(t0 + nv - 1) * H + h];
}

template <typename TC, typename TK, int K>
__global__ __launch_bounds__(64 * HCfg<K>::NW) void fwd_h_kernel(FwdHArgs a, int V, int total_units) {
  using Cfg = HCfg<K>;
  constexpr int NW = Cfg::NW, KW = Cfg::KW, KT = Cfg::KT, KS = Cfg::KS, OWN = Cfg::OWN;
  __shared__ __align__(16) f32x4 s_red[NW][4][WAVE];
  __shared__ __align__(16) TC s_vgT[BV * LDT];
  __shared__ __align__(16) TC s_kT[NW][KW * LDT];

  // XCD-aware unit order: consecutive work items share an XCD (and its L2),
  // so the V slices of one head read w and k through the same cache.
  const int per_xcd = gridDim.x / 8;
  const int o_idx = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (o_idx >= total_units) return;
  const int nvt = V / BV;
  const int unit = o_idx / nvt;
  const int v0 = (o_idx % nvt) * BV;
  const int H = a.H;
  const int n = unit / H, h = unit % H;

  const int wid = threadIdx.x / WAVE;
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;

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

  // state slice: rows KW*wid + 16*tt + 4*lg + j, column v0 + lc
  f32x4 S[KT];
  with_state_loader(a.h0, a.h0_dtype == DT_F32 ? 0 : 1, [&](auto ld) {
#pragma unroll
    for (int tt = 0; tt < KT; ++tt)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        S[tt][j] = ld((((int64_t)n * H + h) * K + KW * wid + 16 * tt + 4 * lg + j) * V + v0 + lc);
  });

  ChunkPrefetch<TC, TK, K> cur, nxt;
  if (nchunks > 0) prefetch_chunk<TC, TK, K>(cur, a, c_first, bos, (int)min((int64_t)C, eos - bos), h, v0, wid, V);

  TC* hT = reinterpret_cast<TC*>(a.hT);
  TC* vnT = reinterpret_cast<TC*>(a.vnT);
  TC* kT = s_kT[wid];

  for (int64_t it = 0; it < nchunks; ++it) {
    const int64_t c = c_first + it;
    if (it + 1 < nchunks) {
      const int64_t t1 = bos + (it + 1) * C;
      prefetch_chunk<TC, TK, K>(nxt, a, c + 1, t1, (int)min((int64_t)C, eos - t1), h, v0, wid, V);
    }
    const int nv = cur.nv;

    // snapshot of the state before this chunk
    if (a.row_major) {            // h [NC, H, K, V]: 16 lanes write 16 consecutive columns of a row
      TC* hcol = hT + ((c * H + h) * K + KW * wid + 4 * lg) * (int64_t)V + v0 + lc;
#pragma unroll
      for (int tt = 0; tt < KT; ++tt)
#pragma unroll
        for (int j = 0; j < 4; ++j) hcol[(16 * tt + j) * (int64_t)V] = from_f32<TC>(S[tt][j]);
    } else {
      TC* hrow = hT + ((c * H + h) * V + v0 + lc) * K + KW * wid + 4 * lg;
#pragma unroll
      for (int tt = 0; tt < KT; ++tt) st4<TC>(hrow + 16 * tt, S[tt][0], S[tt][1], S[tt][2], S[tt][3]);
    }

    // partial w @ S over this wave's K slice
    Frag<TC> hb[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) hb[ks] = frag_from_acc<TC>(S[2 * ks], S[2 * ks + 1]);
#pragma unroll
    for (int tm = 0; tm < 4; ++tm) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) mma(acc, cur.wf[tm][ks], hb[ks]);
      s_red[wid][tm][l] = acc;
    }
    step_barrier();

    // k^T slice of this wave (read only by this wave, in the update below: t = lane)
#pragma unroll
    for (int d8 = 0; d8 < KW / 8; ++d8) {
#pragma unroll
      for (int e = 0; e < 8; ++e) kT[(8 * d8 + e) * LDT + l] = from_f32<TC>(vget<TC>(cur.krow[d8], e));
    }

    // v' = u - w @ S for the owned row tiles; store v_new; gate into LDS
    TC* vrow = vnT + ((c * H + h) * V + v0 + lc) * C;
#pragma unroll
    for (int o = 0; o < OWN; ++o) {
      const int tm = wid + NW * o;
      f32x4 vp = cur.uv[o];
#pragma unroll
      for (int w2 = 0; w2 < NW; ++w2) vp -= s_red[w2][tm][l];
      if (a.row_major) {          // v_new [B*T, H, V]
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int t = 16 * tm + 4 * lg + j;
          if (t < nv) vnT[((cur.t0 + t) * H + h) * (int64_t)V + v0 + lc] = from_f32<TC>(vp[j]);
        }
      } else {
        st4<TC>(vrow + 16 * tm + 4 * lg, vp[0], vp[1], vp[2], vp[3]);
      }
      float vg[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = 16 * tm + 4 * lg + j;
        vg[j] = t < nv ? vp[j] * gexp(cur.gl - cur.gv[o][j]) : 0.f;
      }
      st4<TC>(s_vgT + lc * LDT + 16 * tm + 4 * lg, vg[0], vg[1], vg[2], vg[3]);
    }
    step_barrier();

    // S = exp(g_last) S + k^T (v' gated)
    const float eg = gexp(cur.gl);
#pragma unroll
    for (int tt = 0; tt < KT; ++tt) {
      S[tt] *= eg;
#pragma unroll
      for (int ks2 = 0; ks2 < 2; ++ks2)
        mma(S[tt], lds_frag<TC>(kT, LDT, 16 * tt, 32 * ks2), lds_frag<TC>(s_vgT, LDT, 0, 32 * ks2));
    }
    cur = nxt;
  }

  if (a.ht) {
#pragma unroll
    for (int tt = 0; tt < KT; ++tt) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t off = (((int64_t)n * H + h) * K + KW * wid + 16 * tt + 4 * lg + j) * V + v0 + lc;
        a.ht[off] = S[tt][j];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Wide form for K = 256 (the Kairos model's head dim), bf16 compute.  Here the
// split-K form above re-reads the whole w and k chunk (64 KB) for every 16
// state columns; instead one workgroup of WW waves stages the chunk's w
// (row-major) and k^T in LDS once, and each wave owns 16 state columns over all
// 256 rows (16 accumulator tiles in VGPRs), so w @ S needs no cross-wave
// reduction and the gated v' stays in wave-private LDS.  Same outputs as the
// split-K form (hT, vnT, ht) and the same cast points.
// ---------------------------------------------------------------------------
constexpr int WW = 4;                     // waves (x 16 columns) per workgroup
constexpr int WK = 256;
constexpr int LDW = WK + 8;               // w row stride (elements)

// k tile [64 tokens][256] in LDS, 16-byte chunks swizzled (swz_off, gdn_common.hpp), read as k^T
// with the transposed read (tr_frag).
__device__ __forceinline__ int kswz_off(int r, int c8) { return swz_off<WK>(r, c8); }
__device__ __forceinline__ Frag<bf16> k_tr_frag(const bf16* s_k, int ks, int d0) { return tr_frag<WK>(s_k, ks, d0); }

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

template <typename TK>
struct WideChunk {
  u32x4 w[8];            // this thread's 8 x 8 elements of w (row-major items tid + 256 i)
  u32x4 k[8];            // the same items of k, as bf16 (fp8 k dequantised at load)
  u32x2 u[4];            // u of the wave's 16 columns, C layout, 4 row tiles, 4 bf16 each
  float gcl;             // gc of token t0 + lane (0 past the chunk's end); rows get theirs by shuffle
  int nv;
};

template <typename TK>
__device__ __forceinline__ void wide_prefetch(WideChunk<TK>& P, const FwdHArgs& a, int64_t c, int64_t t0, int nv,
                                              int h, int vcol, bool active, int V) {
  const int tid = threadIdx.x;
  const int l = lane_id();
  const int lg = l >> 4;
  const int H = a.H;
  P.nv = nv;
  const bf16* w = reinterpret_cast<const bf16*>(a.w);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int item = tid + 256 * i;                 // 64 rows x 32 blocks of 8
    const int r = item >> 5, cb = item & 31;
    P.w[i] = r < nv ? *reinterpret_cast<const u32x4*>(w + ((t0 + r) * H + h) * WK + 8 * cb) : u32x4{0u, 0u, 0u, 0u};
  }
  const TK* k = reinterpret_cast<const TK*>(a.k);
  const float ks_ = a.k_scale ? a.k_scale[h] : 1.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int item = tid + 256 * i;
    const int r = item >> 5, cb = item & 31;
    if constexpr (sizeof(TK) == 2) {
      P.k[i] = r < nv ? *reinterpret_cast<const u32x4*>(k + ((t0 + r) * H + h) * WK + 8 * cb) : u32x4{0u, 0u, 0u, 0u};
    } else {                                          // fp8: dequantise to bf16 (scalar locals for the bit casts)
      float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      if (r < nv) load8_in<TK>(k + ((t0 + r) * H + h) * WK + 8 * cb, ks_, x);
      uint32_t wd[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const bf16 lo = (bf16)x[2 * q], hi = (bf16)x[2 * q + 1];
        wd[q] = (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
      }
      P.k[i] = u32x4{wd[0], wd[1], wd[2], wd[3]};
    }
  }
  if (active) {
    const bf16* uT = reinterpret_cast<const bf16*>(a.uT) + ((c * H + h) * V + vcol) * C;
#pragma unroll
    for (int tm = 0; tm < 4; ++tm) P.u[tm] = *reinterpret_cast<const u32x2*>(uT + 16 * tm + 4 * lg);
  }
  P.gcl = l < nv ? a.gc[(t0 + l) * H + h] : 0.f;
}

// Workgroup barrier that waits for LDS operations only, so the next chunk's
// global loads (registers) and this chunk's hT / vnT stores stay in flight
// across it; the compiler waits for those loads where their registers are used.
// The empty asm statements keep memory accesses from moving across the barrier.
__device__ __forceinline__ void wide_lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);          // lgkmcnt(0); vmcnt, expcnt at their maxima
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <typename TK>
__global__ __launch_bounds__(64 * WW) void fwd_h_wide_kernel(FwdHArgs a, int V, int total_units) {
  __shared__ __align__(16) bf16 s_w[C * LDW];            // w rows [t][k]
  __shared__ __align__(16) bf16 s_k[C * WK];              // k rows [t][k], 16-byte chunks swizzled (kswz)
  __shared__ __align__(16) bf16 s_vg[WW][16 * LDT];      // per wave: gated v'^T [col][t]
  __shared__ __align__(16) bf16 s_hs[WW][16 * LDW];      // per wave: h snapshot [col][k] on its way to HBM
  __shared__ __align__(16) bf16 s_vn[WW][16 * LDT];      // per wave: v_new [col][t] on its way to HBM

  const int per_xcd = gridDim.x / 8;                      // XCD-aware order (see fwd_h_kernel)
  const int o_idx = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (o_idx >= total_units) return;
  const int nvt = (V + 16 * WW - 1) / (16 * WW);
  const int unit = o_idx / nvt;
  const int H = a.H;
  const int n = unit / H, h = unit % H;
  const int wid = threadIdx.x / WAVE;
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;
  const int v0 = (o_idx % nvt) * 16 * WW + 16 * wid;      // this wave's first column
  const bool active = v0 < V;
  const int vcol = active ? v0 + lc : 0;

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

  // state: rows 16 kt + 4 lg + j, column vcol
  f32x4 S[16];
  with_state_loader(active ? a.h0 : nullptr, a.h0_dtype == DT_F32 ? 0 : 1, [&](auto ld) {
#pragma unroll
    for (int kt = 0; kt < 16; ++kt)
#pragma unroll
      for (int j = 0; j < 4; ++j) S[kt][j] = ld((((int64_t)n * H + h) * WK + 16 * kt + 4 * lg + j) * V + vcol);
  });

  // two chunks of loads in flight: a chunk's loads are issued two steps before it is staged
  // (measured: with one step of distance the step waits on its global loads for most of its time)
  WideChunk<TK> cur, nx1, nx2;
  if (nchunks > 0) wide_prefetch<TK>(cur, a, c_first, bos, (int)min((int64_t)C, eos - bos), h, vcol, active, V);
  if (nchunks > 1) {
    const int64_t t1 = bos + C;
    wide_prefetch<TK>(nx1, a, c_first + 1, t1, (int)min((int64_t)C, eos - t1), h, vcol, active, V);
  }
  bf16* hT = reinterpret_cast<bf16*>(a.hT);
  bf16* vnT = reinterpret_cast<bf16*>(a.vnT);
  bf16* vg = s_vg[wid];
  const int tid = threadIdx.x;

  for (int64_t it = 0; it < nchunks; ++it) {
    const int64_t c = c_first + it;
    // ---- stage this chunk's w and k^T
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int item = tid + 256 * i;
      *reinterpret_cast<u32x4*>(s_w + (item >> 5) * LDW + 8 * (item & 31)) = cur.w[i];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int item = tid + 256 * i;
      *reinterpret_cast<u32x4*>(s_k + kswz_off(item >> 5, item & 31)) = cur.k[i];
    }
    wide_lds_barrier();
    if (it + 2 < nchunks) {
      const int64_t t2 = bos + (it + 2) * C;
      wide_prefetch<TK>(nx2, a, c + 2, t2, (int)min((int64_t)C, eos - t2), h, vcol, active, V);
    }
    const int nv = cur.nv;
    if (active) {
      // snapshot of the state before this chunk, rounded (chunk_delta_h.py:129-139): through the
      // wave's LDS tile [col][k], so that each store instruction writes whole rows
      bf16* hs = s_hs[wid];
#pragma unroll
      for (int kt = 0; kt < 16; ++kt) st4<bf16>(hs + lc * LDW + 16 * kt + 4 * lg, S[kt][0], S[kt][1], S[kt][2], S[kt][3]);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (a.row_major) {
        // h [NC, H, K, V]: four transposed reads of the tile give lane (lg, i) the wave's 16 columns
        // of row 16 lg + 64 p + i (read m: lane i fetches rows 16 lg + 64 p + 4 (i % 4) .. + 3 of
        // column 4 m + i / 4 and receives columns 4 m .. + 3 of row 16 lg + 64 p + i); two 16-byte
        // stores per row
        bf16* hrow = hT + ((c * H + h) * WK) * (int64_t)V + v0;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const int r0 = 16 * lg + 64 * p;
          s16x4_t x[4];
#pragma unroll
          for (int m = 0; m < 4; ++m) x[m] = lds_read_tr16(hs + (4 * m + (lc >> 2)) * LDW + r0 + 4 * (lc & 3));
          uint4* dst = reinterpret_cast<uint4*>(hrow + (int64_t)(r0 + lc) * V);
          dst[0] = __builtin_bit_cast(uint4, __builtin_shufflevector(x[0], x[1], 0, 1, 2, 3, 4, 5, 6, 7));
          dst[1] = __builtin_bit_cast(uint4, __builtin_shufflevector(x[2], x[3], 0, 1, 2, 3, 4, 5, 6, 7));
        }
      } else {
        bf16* hcol = hT + ((c * H + h) * V + v0) * WK;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int pc = l + 64 * i, r = pc >> 5, ch = pc & 31;   // row (column of S), 16-byte chunk
          *reinterpret_cast<uint4*>(hcol + r * WK + 8 * ch) = *reinterpret_cast<const uint4*>(hs + r * LDW + 8 * ch);
        }
      }
      // w @ bf16(S): the B fragment of a 32-deep step is two accumulator tiles; the A
      // fragment takes the same K order (rows 4 lg .. and 16 + 4 lg .. of the step).
      // K steps outermost: one B fragment live, the 4 row tiles' A reads batched.
      f32x4 acc[4];
#pragma unroll
      for (int tm = 0; tm < 4; ++tm) acc[tm] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        const Frag<bf16> hb = frag_from_acc<bf16>(S[2 * ks], S[2 * ks + 1]);
        Frag<bf16> wa[4];
#pragma unroll
        for (int tm = 0; tm < 4; ++tm) {
          const bf16* wr = s_w + (16 * tm + lc) * LDW + 4 * lg + 32 * ks;
          wa[tm] = join<bf16>(ld_half<bf16>(wr), ld_half<bf16>(wr + 16));
        }
#pragma unroll
        for (int tm = 0; tm < 4; ++tm) mma(acc[tm], wa[tm], hb);
      }
      float vgv[4][4];
      const float gl = __shfl(cur.gcl, nv - 1);     // gc of the chunk's last token
#pragma unroll
      for (int tm = 0; tm < 4; ++tm) {
        const f32x4 uv = {bf16_lo(cur.u[tm][0]), bf16_hi(cur.u[tm][0]), bf16_lo(cur.u[tm][1]), bf16_hi(cur.u[tm][1])};
        const f32x4 vp = uv - acc[tm];              // v' = u - w h (chunk_delta_h.py:141-157)
        st4<bf16>(s_vn[wid] + lc * LDT + 16 * tm + 4 * lg, vp[0], vp[1], vp[2], vp[3]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int t = 16 * tm + 4 * lg + j;
          const float gt = __shfl(cur.gcl, t);
          vgv[tm][j] = t < nv ? vp[j] * gexp(gl - gt) : 0.f;
        }
      }
#pragma unroll
      for (int tm = 0; tm < 4; ++tm)
        st4<bf16>(vg + lc * LDT + 16 * tm + 4 * lg, vgv[tm][0], vgv[tm][1], vgv[tm][2], vgv[tm][3]);
      // the gated v' tile is read back by other lanes of this wave only, in the accumulator K
      // order of the transposed k fragments (tokens 32 ks + 4 lg .. and 32 ks + 16 + 4 lg ..);
      // v_new (ungated) leaves through the wave's LDS tile as whole 128-byte rows of vnT
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (a.row_major) {          // v_new [B*T, H, V] from the wave's [col][t] tile, as the h rows above
        s16x4_t x[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) x[m] = lds_read_tr16(s_vn[wid] + (4 * m + (lc >> 2)) * LDT + 16 * lg + 4 * (lc & 3));
        const int tok = 16 * lg + lc;
        if (tok < nv) {
          const int64_t t0 = bos + it * C;
          uint4* dst = reinterpret_cast<uint4*>(vnT + ((t0 + tok) * H + h) * (int64_t)V + v0);
          dst[0] = __builtin_bit_cast(uint4, __builtin_shufflevector(x[0], x[1], 0, 1, 2, 3, 4, 5, 6, 7));
          dst[1] = __builtin_bit_cast(uint4, __builtin_shufflevector(x[2], x[3], 0, 1, 2, 3, 4, 5, 6, 7));
        }
      } else {
        bf16* vcolp = vnT + ((c * H + h) * V + v0) * C;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int pc = l + 64 * i, r = pc >> 3, ch = pc & 7;
          *reinterpret_cast<uint4*>(vcolp + r * C + 8 * ch) = *reinterpret_cast<const uint4*>(s_vn[wid] + r * LDT + 8 * ch);
        }
      }
      const bf16* vgr = vg + lc * LDT + 4 * lg;
      const Frag<bf16> b0 = join<bf16>(ld_half<bf16>(vgr), ld_half<bf16>(vgr + 16));
      const Frag<bf16> b1 = join<bf16>(ld_half<bf16>(vgr + 32), ld_half<bf16>(vgr + 48));
      // S = exp(g_last) S + k^T (v' gated) (chunk_delta_h.py:163-211)
      const float eg = gexp(gl);
#pragma unroll
      for (int k4 = 0; k4 < 16; k4 += 4) {           // 8 A fragments read per batch of 4 row tiles
        Frag<bf16> ka[4][2];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          ka[q][0] = k_tr_frag(s_k, 0, 16 * (k4 + q));
          ka[q][1] = k_tr_frag(s_k, 1, 16 * (k4 + q));
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          S[k4 + q] *= eg;
          mma(S[k4 + q], ka[q][0], b0);
          mma(S[k4 + q], ka[q][1], b1);
        }
      }
    }
    wide_lds_barrier();                               // w / k^T are overwritten next step
    cur = nx1;
    nx1 = nx2;
  }

  if (a.ht && active) {
#pragma unroll
    for (int kt = 0; kt < 16; ++kt) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t off = (((int64_t)n * H + h) * WK + 16 * kt + 4 * lg + j) * V + vcol;
        a.ht[off] = S[kt][j];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// All-columns form for bf16 K, V in {64, 128}: one workgroup per (sequence, head), V / 16 waves,
// wave w owning state columns 16 w .. + 15 over all K rows (fp32 accumulator tiles in VGPRs).  The
// chunk's w and k are staged in LDS once for every wave (the split-K form stages them once per 16
// columns); u comes from uT in the accumulator layout, the next chunk's inputs are loaded into
// registers while the current one computes.  Same outputs and cast points as the other forms.
// ---------------------------------------------------------------------------
template <int K, int V>
struct HCols {
  static constexpr int NW = V / 16, NT = NW * WAVE;
  static constexpr int KT = K / 16, KS = K / 32;
  static constexpr int EK = C * K;
  static constexpr int UK = EK / 8 / NT;                 // 16-byte units of a [64][K] tile per thread
  static_assert(EK % (8 * NT) == 0, "units split evenly over the threads");
  // row-major outputs of a step (bf16, 16-byte chunks swizzled by row, hcols_swz): the snapshot
  // [K][V] and v_new [64][V], written out as whole rows by every thread after the step
  static constexpr size_t off_hs = (size_t)2 * EK * 2 + C * sizeof(float);
  static constexpr size_t off_vn = off_hs + (size_t)K * V * 2;
  static constexpr size_t lds_rm = off_vn + (size_t)C * V * 2;
  static constexpr size_t lds = (size_t)2 * EK * 2 + C * sizeof(float);
};

// 16-byte chunk ch of row r of an output tile with V / 8 chunks per row: rows 4 apart (one lane
// group's 2-byte writes) land on distinct pairs of chunks
template <int V>
__device__ __forceinline__ int hcols_swz(int r, int ch) { return ch ^ ((2 * (r >> 2)) & (V / 8 - 1)); }

template <int K, int V>
struct HColsChunk {
  using P = HCols<K, V>;
  u32x4 w[P::UK], k[P::UK];
  u32x2 u[4];                 // u of the wave's column lc, rows 16 tm + 4 lg .. + 3
  float gt;                   // gc of token = lane (0 past the end)
  int64_t t0;
  int nv;
};

template <int K, int V>
__device__ __forceinline__ void hcols_load(HColsChunk<K, V>& P, const FwdHArgs& a, int64_t c, int64_t t0, int nv,
                                           int h, int vcol) {
  using HP = HCols<K, V>;
  const int tid = threadIdx.x, l = lane_id(), lg = l >> 4;
  const int H = a.H;
  P.t0 = t0;
  P.nv = nv;
  const u32x4 z = {0u, 0u, 0u, 0u};
  const bf16* w = reinterpret_cast<const bf16*>(a.w);
  const bf16* k = reinterpret_cast<const bf16*>(a.k);
#pragma unroll
  for (int i = 0; i < HP::UK; ++i) {
    const int u = tid + HP::NT * i, r = u / (K / 8), c8 = u % (K / 8);
    const int64_t off = ((t0 + r) * H + h) * (int64_t)K + 8 * c8;
    P.w[i] = r < nv ? *reinterpret_cast<const u32x4*>(w + off) : z;
    P.k[i] = r < nv ? *reinterpret_cast<const u32x4*>(k + off) : z;
  }
  const bf16* uT = reinterpret_cast<const bf16*>(a.uT) + ((c * H + h) * V + vcol) * C;
#pragma unroll
  for (int tm = 0; tm < 4; ++tm) P.u[tm] = *reinterpret_cast<const u32x2*>(uT + 16 * tm + 4 * lg);
  P.gt = l < nv ? a.gc[(t0 + l) * H + h] : 0.f;
}

// kRM: row-major outputs (h [NC, H, K, V], v_new [B*T, H, V], through LDS tiles), else hT and vnT
template <int K, int V, bool kRM>
__global__ __launch_bounds__((HCols<K, V>::NT)) void fwd_h_cols_kernel(FwdHArgs a, int total_units) {
  using HP = HCols<K, V>;
  constexpr int KT = HP::KT, KS = HP::KS;
  extern __shared__ __align__(16) unsigned char smem[];
  bf16* s_w = reinterpret_cast<bf16*>(smem);
  bf16* s_k = s_w + HP::EK;
  float* s_g = reinterpret_cast<float*>(smem + (size_t)2 * HP::EK * 2);
  bf16* s_hs = reinterpret_cast<bf16*>(smem + HP::off_hs);   // (kRM only)
  bf16* s_vn = reinterpret_cast<bf16*>(smem + HP::off_vn);

  const int per_xcd = gridDim.x / 8;                      // XCD-aware unit order
  const int unit = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (unit >= total_units) return;
  const int H = a.H;
  const int n = unit / H, h = unit % H;
  const int tid = threadIdx.x, wid = tid / WAVE, l = lane_id(), lg = l >> 4, lc = l & 15;
  const int c0 = 16 * wid, vcol = c0 + lc;

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

  // state: rows 16 tt + 4 lg + j, column vcol
  f32x4 S[KT];
  with_state_loader(a.h0, a.h0_dtype == DT_F32 ? 0 : 1, [&](auto ld) {
#pragma unroll
    for (int tt = 0; tt < KT; ++tt)
#pragma unroll
      for (int j = 0; j < 4; ++j) S[tt][j] = ld((((int64_t)n * H + h) * K + 16 * tt + 4 * lg + j) * V + vcol);
  });

  auto chunk_start = [&](int64_t it) { return bos + it * C; };
  auto chunk_len = [&](int64_t it) { return (int)min((int64_t)C, eos - chunk_start(it)); };
  HColsChunk<K, V> cur, nxt;
  if (nchunks > 0) hcols_load<K, V>(cur, a, c_first, bos, chunk_len(0), h, vcol);
  bf16* hT = reinterpret_cast<bf16*>(a.hT);
  bf16* vnT = reinterpret_cast<bf16*>(a.vnT);
  // a step's row-major snapshot and v_new, from their LDS tiles to HBM as 16-byte row pieces
  auto flush = [&](int64_t c, int64_t t0, int nv) {
    bf16* base = hT + (c * H + h) * (int64_t)K * V;       // [K][V], contiguous
#pragma unroll
    for (int i = 0; i < K * V / 8 / HP::NT; ++i) {
      const int u = tid + HP::NT * i, r = u / (V / 8), ch = u % (V / 8);
      const u32x4 x = *reinterpret_cast<const u32x4*>(s_hs + r * V + 8 * hcols_swz<V>(r, ch));
      st_global(base + (int64_t)r * V + 8 * ch, x);
    }
#pragma unroll
    for (int i = 0; i < C * V / 8 / HP::NT; ++i) {
      const int u = tid + HP::NT * i, t = u / (V / 8), ch = u % (V / 8);
      const u32x4 x = *reinterpret_cast<const u32x4*>(s_vn + t * V + 8 * hcols_swz<V>(t, ch));
      if (t < nv) st_global(vnT + ((t0 + t) * H + h) * (int64_t)V + 8 * ch, x);
    }
  };
  int64_t prev_c = 0, prev_t0 = 0;
  int prev_nv = 0;

  for (int64_t it = 0; it < nchunks; ++it) {
    const int64_t c = c_first + it;
    const int nv = cur.nv;
    const int64_t t0 = cur.t0;
    if (kRM && it > 0) flush(prev_c, prev_t0, prev_nv);   // the previous step's outputs (published by
                                                          // its closing barrier)
    prev_c = c;
    prev_t0 = t0;
    prev_nv = nv;
#pragma unroll
    for (int i = 0; i < HP::UK; ++i) {
      const int u = tid + HP::NT * i, r = u / (K / 8), cc = 8 * (u % (K / 8));
      const int o = toff<bf16>(r, cc, K);
      *reinterpret_cast<u32x4*>(s_w + o) = cur.w[i];
      *reinterpret_cast<u32x4*>(s_k + o) = cur.k[i];
    }
    if (wid == 0) s_g[l] = cur.gt;
    step_barrier();
    if (it + 1 < nchunks) hcols_load<K, V>(nxt, a, c + 1, chunk_start(it + 1), chunk_len(it + 1), h, vcol);

    // snapshot of the state before this chunk, rounded (chunk_delta_h.py:129-139)
    if constexpr (kRM) {          // h [NC, H, K, V], into its LDS tile
#pragma unroll
      for (int tt = 0; tt < KT; ++tt)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 16 * tt + 4 * lg + j;
          s_hs[r * V + 8 * hcols_swz<V>(r, vcol >> 3) + (vcol & 7)] = (bf16)S[tt][j];
        }
    } else {                      // hT [NC, H, V, K]
      bf16* p = hT + ((c * H + h) * V + vcol) * (int64_t)K + 4 * lg;
#pragma unroll
      for (int tt = 0; tt < KT; ++tt) st4<bf16>(p + 16 * tt, S[tt][0], S[tt][1], S[tt][2], S[tt][3]);
    }
    // v' = u - w bf16(S) (chunk_delta_h.py:141-157), rows t = 16 tm + 4 lg + j
    Frag<bf16> hb[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) hb[ks] = frag_from_acc<bf16>(S[2 * ks], S[2 * ks + 1]);
    const float gl = s_g[nv - 1];
    f32x4 Y[4], Yg[4];
#pragma unroll
    for (int tm = 0; tm < 4; ++tm) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) mma(acc, t_acc<bf16>(s_w, K, 16 * tm, 32 * ks), hb[ks]);
      const f32x4 uv = {bf16_lo(cur.u[tm][0]), bf16_hi(cur.u[tm][0]), bf16_lo(cur.u[tm][1]), bf16_hi(cur.u[tm][1])};
      Y[tm] = uv - acc;
      const f32x4 g4 = *reinterpret_cast<const f32x4*>(s_g + 16 * tm + 4 * lg);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = 16 * tm + 4 * lg + j;
        Yg[tm][j] = t < nv ? Y[tm][j] * gexp(gl - g4[j]) : 0.f;
      }
      if constexpr (kRM) {        // v_new [B*T, H, V], into its LDS tile
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int t = 16 * tm + 4 * lg + j;
          s_vn[t * V + 8 * hcols_swz<V>(t, vcol >> 3) + (vcol & 7)] = (bf16)Y[tm][j];
        }
      } else {                    // vnT [NC, H, V, 64]
        st4<bf16>(vnT + ((c * H + h) * V + vcol) * C + 16 * tm + 4 * lg, Y[tm][0], Y[tm][1], Y[tm][2], Y[tm][3]);
      }
    }
    // S = exp(g_last) S + k^T (v' exp(g_last - gc)) (chunk_delta_h.py:163-211)
    Frag<bf16> vg[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) vg[ks] = frag_from_acc<bf16>(Yg[2 * ks], Yg[2 * ks + 1]);
    const float eg = gexp(gl);
#pragma unroll
    for (int tt = 0; tt < KT; ++tt) {
      S[tt] *= eg;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) mma(S[tt], t_tr<bf16>(s_k, K, 32 * ks, 16 * tt), vg[ks]);
    }
    step_barrier();                                       // the tiles are restaged next chunk
    cur = nxt;
  }
  if (kRM && nchunks > 0) flush(prev_c, prev_t0, prev_nv);

  if (a.ht) {
#pragma unroll
    for (int tt = 0; tt < KT; ++tt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t off = (((int64_t)n * H + h) * K + 16 * tt + 4 * lg + j) * V + vcol;
        a.ht[off] = S[tt][j];
      }
  }
}

template <int K, int V>
int launch_fwd_h_cols(const FwdHArgs& a, hipStream_t s) {
  using HP = HCols<K, V>;
  constexpr int nt = HP::NT;
  const int total = a.N * a.H;
  const int grid = (total + 7) / 8 * 8;
  auto go = [&](auto kern, size_t lds) -> int {
    if (lds > 64 * 1024 &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess)
      return -1;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(nt), lds, s, a, total);
    return 0;
  };
  if (int rc = a.row_major ? go(fwd_h_cols_kernel<K, V, true>, HP::lds_rm) : go(fwd_h_cols_kernel<K, V, false>, HP::lds))
    return rc;
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <typename TK>
int launch_fwd_h_wide(const FwdHArgs& a, int V, hipStream_t s) {
  const int total = a.N * a.H * ((V + 16 * WW - 1) / (16 * WW));
  const int grid = (total + 7) / 8 * 8;
  hipLaunchKernelGGL((fwd_h_wide_kernel<TK>), dim3(grid), dim3(64 * WW), 0, s, a, V, total);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <typename TC, typename TK, int K>
int launch_fwd_h_t(const FwdHArgs& a, int V, hipStream_t s) {
  const int total = a.N * a.H * (V / BV);
  const int grid = (total + 7) / 8 * 8;
  hipLaunchKernelGGL((fwd_h_kernel<TC, TK, K>), dim3(grid), dim3(64 * HCfg<K>::NW), 0, s, a, V, total);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace

int launch_fwd_h(const FwdHArgs& a, int compute_dtype, int k_dtype, int K, int V, hipStream_t s) {
  if (V % BV != 0 || a.N * a.H == 0) return -2;
#define KGDN_H_CASE(TC, TK, KK) \
  if (K == KK) return launch_fwd_h_t<TC, TK, KK>(a, V, s);
#define KGDN_H_SHAPES(TC, TK) KGDN_H_CASE(TC, TK, 64) KGDN_H_CASE(TC, TK, 128) KGDN_H_CASE(TC, TK, 256)
  // bf16 K = 256 runs the wide form; bf16 K, V in {64, 128} the all-columns form
  // (KAIROS_GDN_FWD_H_COLS=0: the split-K form, which stays for fp32 and fp8 k)
  if (K == 256 && compute_dtype == DT_BF16 && k_dtype == DT_BF16) return launch_fwd_h_wide<bf16>(a, V, s);
  if (compute_dtype == DT_BF16 && k_dtype == DT_BF16 && (K == 64 || K == 128) && (V == 64 || V == 128)) {
    const char* e = std::getenv("KAIROS_GDN_FWD_H_COLS");
    if (!(e && e[0] == '0' && e[1] == 0)) {
      if (K == 64) return V == 64 ? launch_fwd_h_cols<64, 64>(a, s) : launch_fwd_h_cols<64, 128>(a, s);
      return V == 64 ? launch_fwd_h_cols<128, 64>(a, s) : launch_fwd_h_cols<128, 128>(a, s);
    }
  }
  if (K == 256 && compute_dtype == DT_BF16 && k_dtype == DT_F8E4M3) return launch_fwd_h_wide<uint8_t>(a, V, s);
  if (compute_dtype == DT_F32 && k_dtype == DT_F32) { KGDN_H_SHAPES(float, float) }
  if (compute_dtype == DT_BF16 && k_dtype == DT_BF16) { KGDN_H_SHAPES(bf16, bf16) }
  if (compute_dtype == DT_BF16 && k_dtype == DT_F8E4M3) { KGDN_H_SHAPES(bf16, uint8_t) }
#undef KGDN_H_SHAPES
#undef KGDN_H_CASE
  return -2;
}

}  // namespace kgdn
