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
#include <cstdlib>
#include <type_traits>

#include "gdn_common.hpp"
#include "gdn_conv.hpp"
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
// the tile within a third of the LDS (three workgroups per CU, so one's serial
// phases overlap the others'; at K = 128 two passes of 64 columns: the backward
// at config 2's shape 2.548 -> 2.504 ms), else within 80 KB (two), else 160 KB.
//
// Compact plan (bf16, no u pass): k stays row-major for the whole kernel and the w operand
// (k beta e^gc)^T is formed from transposed reads of it (ds_read_b64_tr_b16) instead of a
// tile of its own; A / Ai sit beside k.  At K = 256 that is 52 KB, three workgroups per CU
// (the full plan's 72 KB allows two).
template <typename TC, int K>
struct PrepLdsCompact {
  static constexpr int LDK = K + 8;
  static constexpr int LDT = C + 8;
  static constexpr int LDA = C + 4;
  static constexpr size_t al16(size_t x) { return (x + 15) / 16 * 16; }
  static constexpr size_t k_bytes = al16(sizeof(TC) * C * LDK);
  static constexpr size_t a_bytes = al16(sizeof(float) * C * LDA);
  static constexpr size_t ai_bytes = al16(sizeof(TC) * C * LDT);
  static constexpr int VP = 64;                                 // unused: no u pass
  static constexpr size_t off_A = k_bytes;
  static constexpr size_t off_Ai = k_bytes;                     // over A once the inverse is read
  static constexpr size_t off_vbT = 0;                          // unused
  static constexpr size_t off_kbT = 0;                          // unused: read from k
  static constexpr size_t off_g = off_A + (a_bytes > ai_bytes ? a_bytes : ai_bytes);
  static constexpr size_t total = off_g + sizeof(float) * 3 * C;
};

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
  static constexpr size_t kThird = 160 * 1024 / 3 / 16 * 16;
  static constexpr int VP = fits(256, kThird) ? 256 : fits(128, kThird) ? 128 : fits(64, kThird) ? 64
                          : fits(256, 80 * 1024) ? 256 : fits(128, 80 * 1024) ? 128 : fits(64, 80 * 1024) ? 64
                          : fits(256, 160 * 1024) ? 256 : fits(128, 160 * 1024) ? 128 : 64;   // v columns per pass
  static constexpr size_t region0 = region0_for(VP);
  static constexpr size_t off_A = 0;                            // region 0 after K.K^T
  static constexpr size_t off_Ai = 0;                           // over A once the inverse is read
  static constexpr size_t off_vbT = aai_bytes;                  // after A / Ai
  static constexpr size_t off_kbT = region0;
  static constexpr size_t off_g = off_kbT + al16(sizeof(TC) * K * LDT);
  static constexpr size_t total = off_g + sizeof(float) * 3 * C;
};

// (k beta e^gc)^T as an MMA operand from the row-major k tile: rows d = d0 + l % 16, tokens
// t0 + 8 (l / 16) .. + 7, by two transposed reads (tokens + 0..3 and + 4..7); k beta is rounded
// when beta is bf16 (wy_fast.py:77) and the product once more, as the staged tile stores it.
template <int LDK>
__device__ __forceinline__ Frag<bf16> kbT_frag(const bf16* s_k, int d0, int t0, const float* s_b, const float* s_eg,
                                               bool beta_bf16) {
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;
  const int tb = t0 + 8 * lg;
  const s16x4_t x0 = lds_read_tr16(s_k + (tb + (lc >> 2)) * LDK + d0 + 4 * (lc & 3));
  const s16x4_t x1 = lds_read_tr16(s_k + (tb + 4 + (lc >> 2)) * LDK + d0 + 4 * (lc & 3));
  const f32x4 b0 = *reinterpret_cast<const f32x4*>(s_b + tb), b1 = *reinterpret_cast<const f32x4*>(s_b + tb + 4);
  const f32x4 e0 = *reinterpret_cast<const f32x4*>(s_eg + tb), e1 = *reinterpret_cast<const f32x4*>(s_eg + tb + 4);
  Frag<bf16> f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const short bits = e < 4 ? x0[e] : x1[e - 4];
    const float kv = __uint_as_float((uint32_t)(uint16_t)bits << 16);
    float kb = kv * (e < 4 ? b0[e] : b1[e - 4]);
    if (beta_bf16) kb = (float)(bf16)kb;
    f.v[e] = (bf16)(kb * (e < 4 ? e0[e] : e1[e - 4]));
  }
  return f;
}

// g and beta of one token row, fp32 or bf16 each (0 / 1), both loads issued before either value
// is used (one memory latency for the pair, not two)
__device__ __forceinline__ void ld_gate_pair(const void* g, int g_dt, const void* b, int b_dt, int64_t i, float& gv,
                                             float& bv) {
  if (g_dt == 0 && b_dt == 0) {
    const float x = reinterpret_cast<const float*>(g)[i], y = reinterpret_cast<const float*>(b)[i];
    gv = x;
    bv = y;
  } else if (g_dt == 0) {
    const float x = reinterpret_cast<const float*>(g)[i];
    const bf16 y = reinterpret_cast<const bf16*>(b)[i];
    gv = x;
    bv = (float)y;
  } else if (b_dt == 0) {
    const bf16 x = reinterpret_cast<const bf16*>(g)[i];
    const float y = reinterpret_cast<const float*>(b)[i];
    gv = (float)x;
    bv = y;
  } else {
    const bf16 x = reinterpret_cast<const bf16*>(g)[i], y = reinterpret_cast<const bf16*>(b)[i];
    gv = (float)x;
    bv = (float)y;
  }
}

template <typename TC, typename TK, int K, bool kCompact, bool kConv>
__device__ __forceinline__ void prepare_body(const PrepareArgs& a, int V) {
  using L = std::conditional_t<kCompact, PrepLdsCompact<TC, K>, PrepLds<TC, K>>;
  static_assert(!kCompact || std::is_same<TC, bf16>::value, "the compact plan reads k with 16-bit transposed reads");
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

  // ---- the chunk's k rows (token pair pr, column group cg) and, with aqk_out, q row tile wid are
  //      loaded first, raw, so that their latency overlaps the gates and each other.  Every load is
  //      issued unconditionally, rows past the chunk's end reading row 0: k is zeroed there when it
  //      is staged, and q rows past the end only feed Aqk rows that are stored as zero.  (Loads in
  //      a branch of their own would each be waited for before the next is issued.)
  const int pr = tid & 31, cg = tid >> 5;                // token pair (2 pr, 2 pr + 1), column group of 8
  using Raw = std::conditional_t<sizeof(TK) == 1, uint2, Vec8<TK>>;
  auto ld_raw = [](const TK* p) -> Raw {
    if constexpr (sizeof(TK) == 1) return *reinterpret_cast<const uint2*>(p);
    else return ld8<TK>(p);
  };
  auto cvt_raw = [](const Raw& r, float scale, float (&out)[8]) {
    if constexpr (sizeof(TK) == 1) {
      fp8x4_to_f32(r.x, out);
      fp8x4_to_f32(r.y, out + 4);
#pragma unroll
      for (int e = 0; e < 8; ++e) out[e] *= scale;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) out[e] = vget<TK>(r, e);
    }
  };
  const TK* kin = reinterpret_cast<const TK*>(a.k);
  const bool ok0 = 2 * pr < nv, ok1 = 2 * pr + 1 < nv;
  Raw kraw[K / 64][2];
  // with the layer's prologue folded in (compact bf16 plan): k and q are formed here from their
  // projections, each staged row piece convolved from its own window of raw rows (gdn_conv.hpp)
  constexpr bool kConvOk = kConv && kCompact && std::is_same<TK, bf16>::value;
  const bool conv_k = kConvOk && a.ck.x != nullptr, conv_q = kConvOk && a.cq.x != nullptr;
  // the taps of both projections in the A region (free until K.K^T; the L2 norm's row sums use its
  // first 2 KB): k at +2 KB, q after them, 5 K floats each
  float* s_tk = s_A + 512;
  float* s_tq = s_tk + 5 * K;
  if constexpr (kConvOk) {
    static_assert(512 + 10 * K <= C * L::LDA, "the taps fit in the A region");
    if (conv_k) stage_taps<K, NT_PREP>(s_tk, a.ck, h);
    if (conv_q) stage_taps<K, NT_PREP>(s_tq, a.cq, h);
    __syncthreads();
  }
  if (conv_k) {
    if constexpr (kConvOk) {
      // two windows in flight: the next one's loads go out before the current one is convolved
      ConvWin<2> wa, wb;
      auto k_issue = [&](ConvWin<2>& w, int ch) {
        w.issue(a.ck, t0 + 2 * pr, loc.bos, t0 + nv, (int64_t)h * K + cg * (K / 8) + 8 * ch);
      };
      k_issue(wa, 0);
#pragma unroll
      for (int ch = 0; ch < K / 64; ++ch) {
        ConvWin<2>& cur = (ch & 1) ? wb : wa;
        ConvWin<2>& nxt = (ch & 1) ? wa : wb;
        if (ch + 1 < K / 64) k_issue(nxt, ch + 1);
        const int cl = cg * (K / 8) + 8 * ch;            // channel within the head
        const ConvTapsLds tp{s_tk + 4 * cl, a.ck.b ? s_tk + 4 * K + cl : nullptr};
        cvx4 y[2];
        cur.finish(a.ck, tp, t0 + 2 * pr, loc.bos, loc.n, (int64_t)h * K + cl, y);
        kraw[ch][0].v = __builtin_bit_cast(bf16x8, y[0]);
        kraw[ch][1].v = __builtin_bit_cast(bf16x8, y[1]);
      }
    }
  } else {
    const TK* krow0 = kin + ((t0 + (ok0 ? 2 * pr : 0)) * H + h) * K + cg * (K / 8);
    const TK* krow1 = kin + ((t0 + (ok1 ? 2 * pr + 1 : 0)) * H + h) * K + cg * (K / 8);
#pragma unroll
    for (int ch = 0; ch < K / 64; ++ch) {
      kraw[ch][0] = ld_raw(krow0 + 8 * ch);
      kraw[ch][1] = ld_raw(krow1 + 8 * ch);
    }
  }
  Raw qraw[K / 32];
  if (a.aqk_out) {
    const int qr = 16 * wid + lc;
    if (conv_q) {
      if constexpr (kConvOk) {
        const int64_t t = t0 + (qr < nv ? qr : 0);
        ConvWin<1> wa, wb;
        auto q_issue = [&](ConvWin<1>& w, int ks) {
          w.issue(a.cq, t, loc.bos, t0 + nv, (int64_t)h * K + 32 * ks + 8 * lg);
        };
        q_issue(wa, 0);
#pragma unroll
        for (int ks = 0; ks < K / 32; ++ks) {
          ConvWin<1>& cur = (ks & 1) ? wb : wa;
          ConvWin<1>& nxt = (ks & 1) ? wa : wb;
          if (ks + 1 < K / 32) q_issue(nxt, ks + 1);
          const int cl = 32 * ks + 8 * lg;
          const ConvTapsLds tp{s_tq + 4 * cl, a.cq.b ? s_tq + 4 * K + cl : nullptr};
          cvx4 y[1];
          cur.finish(a.cq, tp, t, loc.bos, loc.n, (int64_t)h * K + cl, y);
          qraw[ks].v = __builtin_bit_cast(bf16x8, y[0]);
        }
      }
    } else {
      const TK* qrow = reinterpret_cast<const TK*>(a.q) + ((t0 + (qr < nv ? qr : 0)) * H + h) * K + 8 * lg;
#pragma unroll
      for (int ks = 0; ks < K / 32; ++ks) qraw[ks] = ld_raw(qrow + 32 * ks);
    }
  }
  // in-op L2 norm of k (chunk.py:168-170, l2norm.py:98-119; compact plan): each thread's share of the
  // sum of squares of its two rows goes to the A region, free until K.K^T, and is summed after the
  // gates' barrier
  const bool l2 = kCompact && a.l2 != 0;
  if constexpr (kCompact) {
    if (l2) {
      float ss0 = 0.f, ss1 = 0.f;
#pragma unroll
      for (int ch = 0; ch < K / 64; ++ch) {
        float x0[8], x1[8];
        cvt_raw(kraw[ch][0], 1.f, x0);
        cvt_raw(kraw[ch][1], 1.f, x1);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          ss0 = fmaf(x0[e], x0[e], ss0);
          ss1 = fmaf(x1[e], x1[e], ss1);
        }
      }
      s_A[(2 * pr) * 8 + cg] = ss0;
      s_A[(2 * pr + 1) * 8 + cg] = ss1;
    }
  }

  // ---- gates: chunk-local cumsum of g (one wave, inclusive scan over 64 lanes)
  if (wid == 0) {
    float gv = 0.f, bv = 0.f;
    ld_gate_pair(a.g, a.g_dtype, a.beta, a.beta_dtype, (t0 + (l < nv ? l : 0)) * H + h, gv, bv);
    if (l >= nv) gv = bv = 0.f;
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

  // ---- with aqk_out: q row tile wid as MFMA fragments (rows 16 wid + lc), from the raw loads; with
  //      the in-op L2 norm the row (spread over the four lane groups) is normalised and rounded, and
  //      its rstd recorded for the output's q h product, which reads raw q
  Frag<TC> qf[K / 32];
  if (a.aqk_out) {
#pragma unroll
    for (int ks = 0; ks < K / 32; ++ks) {
      if constexpr (sizeof(TC) == 2 && sizeof(TK) == 2) {
        qf[ks].v = __builtin_bit_cast(bf16x8, qraw[ks]);
        if constexpr (kCompact) {
          if (ks == K / 32 - 1 && l2) {
            float ss = 0.f;
#pragma unroll
            for (int k2 = 0; k2 < K / 32; ++k2)
#pragma unroll
              for (int e = 0; e < 8; ++e) ss = fmaf((float)qf[k2].v[e], (float)qf[k2].v[e], ss);
            ss += __shfl_xor(ss, 16, WAVE);
            ss += __shfl_xor(ss, 32, WAVE);
            const float rs = 1.0f / sqrtf(ss + 1e-6f);
#pragma unroll
            for (int k2 = 0; k2 < K / 32; ++k2)
#pragma unroll
              for (int e = 0; e < 8; ++e) qf[k2].v[e] = (bf16)((float)qf[k2].v[e] * rs);
            const int qr = 16 * wid + lc;
            if (lg == 0 && qr < nv && a.qs_out && !conv_q) a.qs_out[(t0 + qr) * H + h] = rs;
          }
        }
      } else {
        float x[8];
        cvt_raw(qraw[ks], 1.f, x);
        if constexpr (sizeof(TC) == 2) {
#pragma unroll
          for (int e = 0; e < 8; ++e) qf[ks].v[e] = (bf16)x[e];
        } else {
          qf[ks].lo = f32x4{x[0], x[1], x[2], x[3]};
          qf[ks].hi = f32x4{x[4], x[5], x[6], x[7]};
        }
      }
    }
    // q formed here (the folded prologue): the recurrence reads it as prepare leaves it (convolved and,
    // with the in-op L2 norm, normalised), one 16-byte row piece per fragment
    if constexpr (kConvOk) {
      const int qr = 16 * wid + lc;
      if (conv_q && a.q_out && qr < nv) {
        bf16* qo = reinterpret_cast<bf16*>(a.q_out) + ((t0 + qr) * H + h) * K + 8 * lg;
#pragma unroll
        for (int ks = 0; ks < K / 32; ++ks) *reinterpret_cast<bf16x8*>(qo + 32 * ks) = qf[ks].v;
      }
    }
  }

  // ---- v of the first pass (below) into registers now, so its loads overlap K.K^T and the solve
  const TC* vin = reinterpret_cast<const TC*>(a.v);
  const bool v_vec = V % 64 == 0;                         // every pass width a multiple of 64 (VP is)
  Vec8<TC> vr[2][L::VP / 64];
  auto load_v = [&](int p0) {
    const int cpg = min(L::VP, V - p0) / 8;               // columns per group, a multiple of 8
#pragma unroll
    for (int ch = 0; ch < L::VP / 64; ++ch) {
      if (8 * ch >= cpg) break;
      const int c = p0 + cg * cpg + 8 * ch;
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {                    // rows past the end read row 0, masked at use
        const int r = 2 * pr + rr;
        vr[rr][ch] = ld8<TC>(vin + ((t0 + (r < nv ? r : 0)) * H + h) * V + c);
      }
    }
  };
  const bool want_u = a.uT != nullptr;                   // without uT: no u pass (the fused K = 256 form forms u)
  if (v_vec && want_u) load_v(0);

  // ---- stage k (row-major, for K.K^T) and the transposed, scaled operand
  //      kb^T[d][t] = k*beta*exp(gc).  Lane = token pair, so each transposed store packs the pair
  //      (one 4-byte store in bf16) and the 32 lanes of a group hit 32 consecutive banks.
  const float kscale = a.k_scale ? a.k_scale[h] : 1.f;
  float rk0 = 1.f, rk1 = 1.f;                            // rstd of k rows 2 pr, 2 pr + 1 (in-op L2 norm)
  if (l2) {
    float ss0 = 0.f, ss1 = 0.f;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      ss0 += s_A[(2 * pr) * 8 + c];
      ss1 += s_A[(2 * pr + 1) * 8 + c];
    }
    rk0 = 1.0f / sqrtf(ss0 + 1e-6f);
    rk1 = 1.0f / sqrtf(ss1 + 1e-6f);
  }
  {
    const float b0 = s_b[2 * pr], b1 = s_b[2 * pr + 1], e0 = s_eg[2 * pr], e1 = s_eg[2 * pr + 1];
#pragma unroll
    for (int ch = 0; ch < K / 64; ++ch) {
      const int c8 = cg * (K / 8) + 8 * ch;
      float x0[8], x1[8];
      cvt_raw(kraw[ch][0], kscale, x0);
      cvt_raw(kraw[ch][1], kscale, x1);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        x0[e] = ok0 ? x0[e] : 0.f;
        x1[e] = ok1 ? x1[e] : 0.f;
      }
      Vec8<TC> r0, r1;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float kv0 = round_to<TC>(x0[e]), kv1 = round_to<TC>(x1[e]);         // stored k (fp8: dequantised)
        if (l2) {                                          // y = bf16(x rstd), as l2norm_fwd stores it
          kv0 = round_to<TC>(kv0 * rk0);
          kv1 = round_to<TC>(kv1 * rk1);
        }
        vset<TC>(r0, e, kv0);
        vset<TC>(r1, e, kv1);
        if constexpr (!kCompact) {
          float kb0 = kv0 * b0, kb1 = kv1 * b1;
          if (a.beta_dtype == 1) {                         // bf16*bf16 -> bf16 (wy_fast.py:77)
            kb0 = round_to<TC>(kb0);
            kb1 = round_to<TC>(kb1);
          }
          st_pair<TC>(s_kbT + (c8 + e) * L::LDT + 2 * pr, kb0 * e0, kb1 * e1);
        }
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
  auto kb_op = [&](int d0, int tk) {                    // rows d0 + lc, tokens tk + 8 lg .. + 7
    if constexpr (kCompact) return kbT_frag<L::LDK>(s_k, d0, tk, s_b, s_eg, a.beta_dtype == 1);
    else return lds_frag<TC>(s_kbT, L::LDT, d0, tk);
  };
  for (int tm = wid; tm < K / 16; tm += 4) {
    const Frag<TC> kf0 = kb_op(16 * tm, 0), kf1 = kb_op(16 * tm, 32);
#pragma unroll
    for (int tn = 0; tn < 4; ++tn) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      mma(acc, kf0, lds_frag<TC>(s_Ai, L::LDT, 16 * tn, 0));
      if (tn >= 2) mma(acc, kf1, lds_frag<TC>(s_Ai, L::LDT, 16 * tn, 32));
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
        const Frag<TC> kf0 = kb_op(16 * tn, 0), kf1 = kb_op(16 * tn, 32);
#pragma unroll
        for (int tm = 0; tm < 4; ++tm) {
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
          mma(acc, lds_frag<TC>(s_Ai, L::LDT, 16 * tm, 0), kf0);
          if (tm >= 2) mma(acc, lds_frag<TC>(s_Ai, L::LDT, 16 * tm, 32), kf1);
          st4<TC>(wt + (16 * tn + lc) * C + 16 * tm + 4 * lg, acc[0], acc[1], acc[2], acc[3]);
        }
      }
    }
  }
  // ---- u = Ai vb  (rows t, cols v) -> uT[c][h][v][t], 4 consecutive t per lane;
  //      vb^T[v][t] = v*beta staged VP columns at a time into region 0 after Ai,
  //      so staging overlaps the w products above
  if constexpr (kCompact) return;
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
          st_pair<TC>(s_vbT + (c8 + e) * L::LDT + 2 * pr, 2 * pr < nv ? vget<TC>(vr[0][ch], e) * b0 : 0.f,
                      2 * pr + 1 < nv ? vget<TC>(vr[1][ch], e) * b1 : 0.f);
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

template <typename TC, typename TK, int K, bool kCompact>
__global__ __launch_bounds__(NT_PREP) void prepare_kernel(PrepareArgs a, int V) {
  prepare_body<TC, TK, K, kCompact, false>(a, V);
}

// The compact plan with the layer's prologue folded in (k and q convolved from their projections as
// they are staged): the windows need more registers than the plain form's 127, so two workgroups per CU
// instead of three.
template <typename TC, typename TK, int K>
__global__ __launch_bounds__(NT_PREP) __attribute__((amdgpu_waves_per_eu(2, 2))) void prepare_conv_kernel(
    PrepareArgs a, int V) {
  prepare_body<TC, TK, K, true, true>(a, V);
}

template <typename TC, typename TK, int K, bool kCompact>
int launch_prepare_t(const PrepareArgs& a, int V, int64_t nc_grid, hipStream_t s) {
  using L = std::conditional_t<kCompact, PrepLdsCompact<TC, K>, PrepLds<TC, K>>;
  static_assert(L::total <= 160 * 1024, "prepare tile does not fit in LDS");
  auto kern = prepare_kernel<TC, TK, K, kCompact>;
  if constexpr (kCompact && std::is_same<TK, bf16>::value && K == 256) {
    if (a.ck.x || a.cq.x) kern = prepare_conv_kernel<TC, TK, K>;
  }
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
  // the compact LDS plan for bf16 without the u pass (KAIROS_GDN_PREP_COMPACT=0 selects the full one)
  const char* e = std::getenv("KAIROS_GDN_PREP_COMPACT");
  const bool compact = a.uT == nullptr && compute_dtype == DT_BF16 && !(e && e[0] == '0' && e[1] == 0);
  // the folded L2 norm and the folded convolution live in the compact plan
  if ((a.l2 || a.ck.x || a.cq.x) && !(compact && k_dtype == DT_BF16)) return -2;
  if ((a.ck.x || a.cq.x) && K != 256) return -2;        // the folded convolution is built for K = 256
  if ((a.ck.x || a.cq.x) && ((a.aqk_out == nullptr) != (a.cq.x == nullptr) || (a.ck.x == nullptr) != (a.cq.x == nullptr)))
    return -2;                                            // k and q are convolved together, q for Aqk
#define KGDN_PREP_CASE(TC, TK, KK)                                                                  \
  if (K == KK) {                                                                                    \
    if constexpr (std::is_same<TC, bf16>::value)                                                    \
      if (compact) return launch_prepare_t<TC, TK, KK, true>(a, V, nc_grid, s);                     \
    return launch_prepare_t<TC, TK, KK, false>(a, V, nc_grid, s);                                   \
  }
#define KGDN_PREP_SHAPES(TC, TK) KGDN_PREP_CASE(TC, TK, 64) KGDN_PREP_CASE(TC, TK, 128) KGDN_PREP_CASE(TC, TK, 256)
  if (compute_dtype == DT_F32 && k_dtype == DT_F32) { KGDN_PREP_SHAPES(float, float) }
  if (compute_dtype == DT_BF16 && k_dtype == DT_BF16) { KGDN_PREP_SHAPES(bf16, bf16) }
  if (compute_dtype == DT_BF16 && k_dtype == DT_F8E4M3) { KGDN_PREP_SHAPES(bf16, uint8_t) }
#undef KGDN_PREP_SHAPES
#undef KGDN_PREP_CASE
  return -2;
}

}  // namespace kgdn
