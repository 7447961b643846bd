// Chunk-parallel "prepare" stage of the chunked GatedDeltaNet forward, one
// workgroup (4 waves) per (chunk, head):
//   gc  = per-chunk prefix sum of g                 (fla ops/utils/cumsum.py:27-65)
//   A   = beta_i exp(gc_i - gc_j) k_i.k_j, i > j    (ops/common/chunk_scaled_dot_kkt.py:57-73)
//   Ai  = (I + A)^-1, fp32 in LDS, stored rounded   (ops/utils/solve_tril.py:184-331)
//   w   = Ai (k beta exp(gc)),  u = Ai (v beta)     (ops/gated_delta_rule/wy_fast.py:55-81)
// The reference runs these as four kernels with fp32 A and the Ai round trip
// through HBM; here they are one pass that reads k, v, g, beta once and
// writes gc, w and u (A / Ai only when a test asks for them).
//
// Output layouts: gc [B*T, H] fp32; w [B*T, H, K] (token-major, as the
// reference); u per chunk transposed, uT [NC, H, V, 64], which is the
// K-contiguous operand layout the state kernel reads.
#include <type_traits>

#include "gdn_common.hpp"
#include "gdn_kernels.h"

namespace kgdn {

namespace {

constexpr int NT_PREP = 256;   // 4 waves

// Two values of consecutive tokens into a transposed tile [d][t] at t even: one
// packed 4-byte store for bf16 (rounded), one 8-byte store for fp32.
template <typename TC>
__device__ __forceinline__ void st_pair(TC* p, float a, float b) {
  if constexpr (sizeof(TC) == 2) {
    const bf16 lo = (bf16)a, hi = (bf16)b;     // scalar locals for the bit casts
    *reinterpret_cast<uint32_t*>(p) =
        (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
  } else {
    *reinterpret_cast<f32x2*>(p) = f32x2{a, b};
  }
}

// LDS plan.  Region 0 holds k row-major for K.K^T.  The A tiles wait in
// registers until every wave is done with k, then region 0 holds A (fp32), which
// the rounded inverse Ai later overwrites, and after that the v pass buffer: v is staged VP
// columns at a time (u is separable over V).  VP is the widest pass that keeps
// the tile within 80 KB (two workgroups per CU, so one's serial phases overlap
// the other's), else within 160 KB.
template <typename TC, int K>
struct PrepLds {
  static constexpr int LDK = K + 8;      // s_k row stride (elements)
  static constexpr int LDT = C + 8;      // transposed tiles / Ai row stride
  static constexpr int LDA = C + 4;      // fp32 A / inverse row stride
  static constexpr size_t al16(size_t x) { return (x + 15) / 16 * 16; }
  static constexpr size_t k_bytes = sizeof(TC) * C * LDK;
  static constexpr size_t a_bytes = al16(sizeof(float) * C * LDA);
  static constexpr size_t ai_bytes = al16(sizeof(TC) * C * LDT);
  static constexpr size_t fixed = al16(sizeof(TC) * K * LDT) + sizeof(float) * 3 * C;
  static constexpr size_t aai_bytes = a_bytes > ai_bytes ? a_bytes : ai_bytes;   // A, then Ai over it
  static constexpr size_t region0_for(int vp) {
    return k_bytes > aai_bytes + sizeof(TC) * vp * LDT ? al16(k_bytes) : aai_bytes + al16(sizeof(TC) * vp * LDT);
  }
  static constexpr size_t fits(int vp, size_t cap) { return region0_for(vp) + fixed <= cap; }
  static constexpr int VP = fits(256, 80 * 1024) ? 256 : fits(128, 80 * 1024) ? 128 : fits(64, 80 * 1024) ? 64
                          : fits(256, 160 * 1024) ? 256 : fits(128, 160 * 1024) ? 128 : 64;   // v columns per pass
  static constexpr size_t region0 = region0_for(VP);
  static constexpr size_t off_A = 0;                            // region 0 after K.K^T
  static constexpr size_t off_Ai = 0;                           // over A once the inverse is read
  static constexpr size_t off_vbT = aai_bytes;                  // after A / Ai
  static constexpr size_t off_kbT = region0;
  static constexpr size_t off_g = off_kbT + al16(sizeof(TC) * K * LDT);
  static constexpr size_t total = off_g + sizeof(float) * 3 * C;
};

template <typename TC, typename TK, int K>
__global__ __launch_bounds__(NT_PREP) void prepare_kernel(PrepareArgs a, int V) {
  using L = PrepLds<TC, K>;
  extern __shared__ __align__(16) unsigned char smem[];
  TC* s_k = reinterpret_cast<TC*>(smem);
  float* s_A = reinterpret_cast<float*>(smem + L::off_A);  // aliases s_k once K.K^T is done
  TC* s_Ai = reinterpret_cast<TC*>(smem + L::off_Ai);     // over A
  TC* s_vbT = reinterpret_cast<TC*>(smem + L::off_vbT);   // after Ai
  TC* s_kbT = reinterpret_cast<TC*>(smem + L::off_kbT);
  float* s_g = reinterpret_cast<float*>(smem + L::off_g);
  float* s_eg = s_g + C;
  float* s_b = s_g + 2 * C;

  const int h = blockIdx.y;
  const int H = a.H;
  // the chunk: blockIdx.x, or with it_span > 0 (fixed-length sequences only) local chunk
  // it0 + x % it_span of sequence x / it_span
  int64_t cidx = blockIdx.x;
  if (a.it_span > 0) {
    const int64_t nt = (a.T + C - 1) / C, it = a.it0 + blockIdx.x % a.it_span;
    if (it >= nt) return;
    cidx = (int64_t)(blockIdx.x / a.it_span) * nt + it;
  }
  const ChunkLoc loc = locate_chunk(cidx, a.cu, a.chunk_off, a.N, a.T);
  if (!loc.ok) return;
  const int64_t t0 = loc.t0;
  const int nv = loc.nv;
  const int tid = threadIdx.x;
  const int wid = tid / WAVE;
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;

  // ---- gates: chunk-local cumsum of g (one wave, inclusive scan over 64 lanes)
  if (wid == 0) {
    float gv = 0.f, bv = 0.f;
    if (l < nv) {
      gv = ld_scalar(a.g, (t0 + l) * H + h, a.g_dtype);
      bv = ld_scalar(a.beta, (t0 + l) * H + h, a.beta_dtype);
    }
#pragma unroll
    for (int off = 1; off < WAVE; off <<= 1) {
      const float o = __shfl_up(gv, off, WAVE);
      if (l >= off) gv += o;
    }
    s_g[l] = gv;
    s_eg[l] = gexp(gv);
    s_b[l] = bv;
    if (l < nv) a.gc[(t0 + l) * H + h] = gv;
    if (a.beta_out && l < nv) a.beta_out[(t0 + l) * H + h] = bv;
  }
  __syncthreads();

  // ---- with aqk_out: q row tile wid as MFMA fragments (rows 16 wid + lc, zero past the chunk's
  //      end), loaded now so that they arrive during the k staging and K.K^T
  Frag<TC> qf[K / 32];
  if (a.aqk_out) {
    const TK* qin = reinterpret_cast<const TK*>(a.q);
    const int qr = 16 * wid + lc;
#pragma unroll
    for (int ks = 0; ks < K / 32; ++ks) {
      float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      if (qr < nv) load8_in<TK>(qin + ((t0 + qr) * H + h) * K + 32 * ks + 8 * lg, 1.f, x);
      if constexpr (sizeof(TC) == 2) {
#pragma unroll
        for (int e = 0; e < 8; ++e) qf[ks].v[e] = (bf16)x[e];
      } else {
        qf[ks].lo = f32x4{x[0], x[1], x[2], x[3]};
        qf[ks].hi = f32x4{x[4], x[5], x[6], x[7]};
      }
    }
  }

  // ---- v of the first pass (below) into registers now, so its loads overlap K.K^T and the solve
  const TC* vin = reinterpret_cast<const TC*>(a.v);
  const int pr = tid & 31, cg = tid >> 5;                // token pair (2 pr, 2 pr + 1), column group of 8
  const bool v_vec = V % 64 == 0;                         // every pass width a multiple of 64 (VP is)
  Vec8<TC> vr[2][L::VP / 64];
  auto load_v = [&](int p0) {
    const int cpg = min(L::VP, V - p0) / 8;               // columns per group, a multiple of 8
#pragma unroll
    for (int ch = 0; ch < L::VP / 64; ++ch) {
      if (8 * ch >= cpg) break;
      const int c = p0 + cg * cpg + 8 * ch;
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        const int r = 2 * pr + rr;
        vr[rr][ch] = r < nv ? ld8<TC>(vin + ((t0 + r) * H + h) * V + c) : vzero<TC>();
      }
    }
  };
  const bool want_u = a.uT != nullptr;                   // without uT: no u pass (the fused K = 256 form forms u)
  if (v_vec && want_u) load_v(0);

  // ---- stage k (row-major, for K.K^T) and the transposed, scaled operand
  //      kb^T[d][t] = k*beta*exp(gc).  Lane = token pair, so each transposed store packs the pair
  //      (one 4-byte store in bf16) and the 32 lanes of a group hit 32 consecutive banks.
  const float kscale = a.k_scale ? a.k_scale[h] : 1.f;
  const TK* kin = reinterpret_cast<const TK*>(a.k);
  {
    const float b0 = s_b[2 * pr], b1 = s_b[2 * pr + 1], e0 = s_eg[2 * pr], e1 = s_eg[2 * pr + 1];
#pragma unroll
    for (int ch = 0; ch < K / 64; ++ch) {
      const int c8 = cg * (K / 8) + 8 * ch;
      float x0[8], x1[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) x0[e] = x1[e] = 0.f;
      if (2 * pr < nv) load8_in<TK>(kin + ((t0 + 2 * pr) * H + h) * K + c8, kscale, x0);
      if (2 * pr + 1 < nv) load8_in<TK>(kin + ((t0 + 2 * pr + 1) * H + h) * K + c8, kscale, x1);
      Vec8<TC> r0, r1;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float kv0 = round_to<TC>(x0[e]), kv1 = round_to<TC>(x1[e]);   // stored k (fp8: dequantised)
        vset<TC>(r0, e, kv0);
        vset<TC>(r1, e, kv1);
        float kb0 = kv0 * b0, kb1 = kv1 * b1;
        if (a.beta_dtype == 1) {                           // bf16*bf16 -> bf16 (wy_fast.py:77)
          kb0 = round_to<TC>(kb0);
          kb1 = round_to<TC>(kb1);
        }
        st_pair<TC>(s_kbT + (c8 + e) * L::LDT + 2 * pr, kb0 * e0, kb1 * e1);
      }
      st8<TC>(s_k + (2 * pr) * L::LDK + c8, r0);
      st8<TC>(s_k + (2 * pr + 1) * L::LDK + c8, r1);
    }
  }
  __syncthreads();

  // ---- A = beta exp(dg) K K^T, strictly lower (10 lower 16x16 tiles over 4 waves); the tiles
  //      stay in registers until every wave has read k, then go to region 0
  f32x4 av[3];
#pragma unroll
  for (int q = 0; q < 3; ++q) {
    const int tile = wid + 4 * q;
    if (tile >= 10) break;                         // uniform per wave
    const int tm = tile < 1 ? 0 : tile < 3 ? 1 : tile < 6 ? 2 : 3;
    const int tn = tile - tm * (tm + 1) / 2;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < K / 32; ++ks)
      mma(acc, lds_frag<TC>(s_k, L::LDK, 16 * tm, 32 * ks), lds_frag<TC>(s_k, L::LDK, 16 * tn, 32 * ks));
    const int j = 16 * tn + lc;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int i = 16 * tm + 4 * lg + jj;
      av[q][jj] = (i > j && i < nv) ? acc[jj] * gexp(s_g[i] - s_g[j]) * s_b[i] : 0.f;
    }
  }
  // ---- optional Aqk = mask_{i>=j, i<nv}(q_i.k_j exp(gc_i - gc_j)) rounded to the storage type,
  //      [NC, H, 64, 64] with the upper triangle zero (chunk_o.py:84-118), for the fused K = 256
  //      recurrence + output: wave w forms row tile w from its q fragments (loaded above) and k
  //      from s_k
  if (a.aqk_out) {
    TC* aq = reinterpret_cast<TC*>(a.aqk_out) + (cidx * H + h) * (C * C);
    const int tm = wid;
#pragma unroll
    for (int tn = 0; tn < 4; ++tn) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      if (tn <= tm) {
#pragma unroll
        for (int ks = 0; ks < K / 32; ++ks) mma(acc, qf[ks], lds_frag<TC>(s_k, L::LDK, 16 * tn, 32 * ks));
      }
      const int j = 16 * tn + lc;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int i = 16 * tm + 4 * lg + jj;
        aq[i * C + j] = from_f32<TC>((i >= j && i < nv) ? acc[jj] * gexp(s_g[i] - s_g[j]) : 0.f);
      }
    }
  }
  // ---- optional k^T per chunk, [NC, H, K, 64] (zero past the chunk's end), for the fused K = 256
  //      recurrence's update operand: wave w writes rows d = 16 (w + 4 i) .. + 15 from transposed
  //      reads of s_k (lane: 4 tokens of one d, one 8-byte store)
  if constexpr (std::is_same<TC, bf16>::value) {
    if (a.kT_out) {
      TC* kt = reinterpret_cast<TC*>(a.kT_out) + (cidx * H + h) * (K * C);
#pragma unroll
      for (int i = 0; i < K / 64; ++i) {
        const int d0 = 16 * (wid + 4 * i);
#pragma unroll
        for (int t4 = 0; t4 < 4; ++t4) {
          const int tr = 16 * t4 + 4 * lg + (lc >> 2);
          const s16x4_t x = lds_read_tr16(s_k + tr * L::LDK + d0 + 4 * (lc & 3));
          *reinterpret_cast<s16x4_t*>(kt + (d0 + lc) * C + 16 * t4 + 4 * lg) = x;
        }
      }
    }
  }
  __syncthreads();                                 // k is dead: region 0 becomes A
#pragma unroll
  for (int q = 0; q < 3; ++q) {
    const int tile = wid + 4 * q;
    if (tile >= 10) break;
    const int tm = tile < 1 ? 0 : tile < 3 ? 1 : tile < 6 ? 2 : 3;
    const int tn = tile - tm * (tm + 1) / 2;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) s_A[(16 * tm + 4 * lg + jj) * L::LDA + 16 * tn + lc] = av[q][jj];
  }
  __syncthreads();

  if (a.A_out) {   // optional fp32 A, [B*T, H, 64] (test hook)
    for (int idx = tid; idx < nv * C; idx += NT_PREP) {
      const int i = idx / C, j = idx % C;
      a.A_out[((t0 + i) * H + h) * C + j] = j < i ? s_A[i * L::LDA + j] : 0.f;
    }
    __syncthreads();
  }

  // ---- (I + A)^-1: invert the four 16x16 diagonal blocks by forward substitution
  //      (wave 0; lane = one column of one block), overwriting the diagonal blocks.
  {
    float x[16];
    float* Xb = s_A + (16 * lg) * L::LDA + 16 * lg;
    if (wid == 0) {
      const int c = lc;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float s = 0.f;
#pragma unroll
        for (int r = 0; r < i; ++r) s = fmaf(Xb[i * L::LDA + r], x[r], s);
        x[i] = (i == c) ? 1.f : (i < c ? 0.f : -s);
      }
    }
    __syncthreads();   // all reads of the diagonal blocks are done before they are overwritten
    if (wid == 0) {
#pragma unroll
      for (int i = 0; i < 16; ++i) Xb[i * L::LDA + lc] = x[i];
    }
  }
  __syncthreads();

  // ---- block merges (fp32 MFMA), X_ij = -X_ii sum_k L_ik X_kj; X_ij (i > j) is
  //      kept in the unused upper block (j, i) so L stays intact for later levels.
  auto blk = [&](int i, int j) { return s_A + (16 * i) * L::LDA + 16 * j; };
  auto put_neg = [&](float* dst, const f32x4& r) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) dst[(4 * lg + jj) * L::LDA + lc] = -r[jj];
  };
  if (wid < 3) {                                  // X_{w+1,w}
    const int i = wid + 1, j = wid;
    f32x4 t = {0.f, 0.f, 0.f, 0.f}, r = {0.f, 0.f, 0.f, 0.f};
    mma16_f32_lds(t, blk(i, j), L::LDA, blk(j, j), L::LDA);
    mma16_f32_lds_reg(r, blk(i, i), L::LDA, t);
    put_neg(blk(j, i), r);
  }
  __syncthreads();
  if (wid < 2) {                                  // X_{w+2,w}
    const int i = wid + 2, j = wid;
    f32x4 t = {0.f, 0.f, 0.f, 0.f}, r = {0.f, 0.f, 0.f, 0.f};
    mma16_f32_lds(t, blk(i, j), L::LDA, blk(j, j), L::LDA);
    mma16_f32_lds(t, blk(i, j + 1), L::LDA, blk(j, j + 1), L::LDA);      // L_{i,j+1} X_{j+1,j}
    mma16_f32_lds_reg(r, blk(i, i), L::LDA, t);
    put_neg(blk(j, i), r);
  }
  __syncthreads();
  if (wid == 0) {                                 // X_{3,0}
    f32x4 t = {0.f, 0.f, 0.f, 0.f}, r = {0.f, 0.f, 0.f, 0.f};
    mma16_f32_lds(t, blk(3, 0), L::LDA, blk(0, 0), L::LDA);
    mma16_f32_lds(t, blk(3, 1), L::LDA, blk(0, 1), L::LDA);               // L_31 X_10
    mma16_f32_lds(t, blk(3, 2), L::LDA, blk(0, 2), L::LDA);               // L_32 X_20
    mma16_f32_lds_reg(r, blk(3, 3), L::LDA, t);
    put_neg(blk(0, 3), r);
  }
  __syncthreads();

  // ---- Ai (rounded to the storage type) into LDS as the K-contiguous [t][s] operand, over A:
  //      every thread reads its entries into registers before any is written
  constexpr int kAiPer = C * C / NT_PREP;
  static_assert(C * C % NT_PREP == 0, "Ai entries must split evenly over the threads");
  TC xr[kAiPer];
#pragma unroll
  for (int q = 0; q < kAiPer; ++q) {
    const int idx = tid + q * NT_PREP;
    const int i = idx / C, j = idx % C;
    const int bi = i >> 4, bj = j >> 4;
    float x = 0.f;
    if (bi == bj) x = s_A[i * L::LDA + j];
    else if (bi > bj) x = s_A[(16 * bj + (i & 15)) * L::LDA + 16 * bi + (j & 15)];
    xr[q] = from_f32<TC>(x);
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < kAiPer; ++q) {
    const int idx = tid + q * NT_PREP;
    const int i = idx / C, j = idx % C;
    s_Ai[i * L::LDT + j] = xr[q];
    if (a.Ai_out && i < nv) reinterpret_cast<TC*>(a.Ai_out)[((t0 + i) * H + h) * C + j] = xr[q];
  }
  __syncthreads();

  // ---- w^T = kb^T Ai^T  (rows d, cols t) -> token-major w, 4 consecutive d per lane
  TC* w_out = reinterpret_cast<TC*>(a.w);
  for (int tm = wid; tm < K / 16; tm += 4) {
#pragma unroll
    for (int tn = 0; tn < 4; ++tn) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks <= tn / 2; ++ks)
        mma(acc, lds_frag<TC>(s_kbT, L::LDT, 16 * tm, 32 * ks), lds_frag<TC>(s_Ai, L::LDT, 16 * tn, 32 * ks));
      const int t = 16 * tn + lc;
      if (t < nv) st4<TC>(w_out + ((t0 + t) * H + h) * K + 16 * tm + 4 * lg, acc[0], acc[1], acc[2], acc[3]);
    }
  }
  // ---- optional w^T per chunk, [NC, H, K, 64]: the same product with the operands swapped (rows t,
  //      cols d), so that a lane holds 4 consecutive t of one d (one 8-byte store); rows t past the
  //      chunk's end are zero (k is zero there and Ai is the identity)
  if constexpr (std::is_same<TC, bf16>::value) {
    if (a.wT_out) {
      TC* wt = reinterpret_cast<TC*>(a.wT_out) + (cidx * H + h) * (K * C);
      for (int tn = wid; tn < K / 16; tn += 4) {
#pragma unroll
        for (int tm = 0; tm < 4; ++tm) {
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks <= tm / 2; ++ks)
            mma(acc, lds_frag<TC>(s_Ai, L::LDT, 16 * tm, 32 * ks), lds_frag<TC>(s_kbT, L::LDT, 16 * tn, 32 * ks));
          st4<TC>(wt + (16 * tn + lc) * C + 16 * tm + 4 * lg, acc[0], acc[1], acc[2], acc[3]);
        }
      }
    }
  }
  // ---- u = Ai vb  (rows t, cols v) -> uT[c][h][v][t], 4 consecutive t per lane;
  //      vb^T[v][t] = v*beta staged VP columns at a time into region 0 after Ai,
  //      so staging overlaps the w products above
  TC* uT = reinterpret_cast<TC*>(a.uT) + (cidx * H + h) * V * C;
  for (int p0 = 0; want_u && p0 < V; p0 += L::VP) {
    const int vw = min(L::VP, V - p0);             // a multiple of 16
    if (v_vec) {                                   // from registers, token pairs packed per store
      const float b0 = s_b[2 * pr], b1 = s_b[2 * pr + 1];
      const int cpg = vw / 8;
#pragma unroll
      for (int ch = 0; ch < L::VP / 64; ++ch) {
        if (8 * ch >= cpg) break;
        const int c8 = cg * cpg + 8 * ch;
#pragma unroll
        for (int e = 0; e < 8; ++e)
          st_pair<TC>(s_vbT + (c8 + e) * L::LDT + 2 * pr, vget<TC>(vr[0][ch], e) * b0, vget<TC>(vr[1][ch], e) * b1);
      }
      if (p0 + L::VP < V) load_v(p0 + L::VP);      // the next pass's loads overlap this pass's products
    } else {
      for (int idx = tid; idx < C * (vw / 8); idx += NT_PREP) {
        const int r = idx / (vw / 8), c8 = (idx % (vw / 8)) * 8;
        Vec8<TC> x = r < nv ? ld8<TC>(vin + ((t0 + r) * H + h) * V + p0 + c8) : vzero<TC>();
        const float b = s_b[r];
#pragma unroll
        for (int e = 0; e < 8; ++e) s_vbT[(c8 + e) * L::LDT + r] = from_f32<TC>(vget<TC>(x, e) * b);
      }
    }
    __syncthreads();
    for (int tn = wid; tn < vw / 16; tn += 4) {
#pragma unroll
      for (int tm = 0; tm < 4; ++tm) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks <= tm / 2; ++ks)
          mma(acc, lds_frag<TC>(s_Ai, L::LDT, 16 * tm, 32 * ks), lds_frag<TC>(s_vbT, L::LDT, 16 * tn, 32 * ks));
        st4<TC>(uT + (p0 + 16 * tn + lc) * C + 16 * tm + 4 * lg, acc[0], acc[1], acc[2], acc[3]);
      }
    }
    if (p0 + L::VP < V) __syncthreads();           // the next pass overwrites vb^T
  }
}

template <typename TC, typename TK, int K>
int launch_prepare_t(const PrepareArgs& a, int V, int64_t nc_grid, hipStream_t s) {
  using L = PrepLds<TC, K>;
  static_assert(L::total <= 160 * 1024, "prepare tile does not fit in LDS");
  auto kern = prepare_kernel<TC, TK, K>;
  if (L::total > 64 * 1024) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)L::total) != hipSuccess)
      return -1;
  }
  dim3 grid((unsigned)nc_grid, (unsigned)a.H);
  hipLaunchKernelGGL(kern, grid, dim3(NT_PREP), L::total, s, a, V);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace

int launch_prepare(const PrepareArgs& a, int compute_dtype, int k_dtype, int K, int V, int64_t nc_grid,
                   hipStream_t s) {
  if (V <= 0 || V % 16 != 0) return -2;
#define KGDN_PREP_CASE(TC, TK, KK) \
  if (K == KK) return launch_prepare_t<TC, TK, KK>(a, V, nc_grid, s);
#define KGDN_PREP_SHAPES(TC, TK) KGDN_PREP_CASE(TC, TK, 64) KGDN_PREP_CASE(TC, TK, 128) KGDN_PREP_CASE(TC, TK, 256)
  if (compute_dtype == DT_F32 && k_dtype == DT_F32) { KGDN_PREP_SHAPES(float, float) }
  if (compute_dtype == DT_BF16 && k_dtype == DT_BF16) { KGDN_PREP_SHAPES(bf16, bf16) }
  if (compute_dtype == DT_BF16 && k_dtype == DT_F8E4M3) { KGDN_PREP_SHAPES(bf16, uint8_t) }
#undef KGDN_PREP_SHAPES
#undef KGDN_PREP_CASE
  return -2;
}

}  // namespace kgdn
