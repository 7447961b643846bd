// Token-by-token gated delta rule, the short-sequence mode of the GatedDeltaNet
// layer (fused_recurrent_gated_delta_rule, fla ops/gated_delta_rule/fused_recurrent.py:21-135,
// used by layers/gated_deltanet.py:220 for q_len <= 64 and decoding).  Per token,
// all in fp32 (fused_recurrent.py:88-125):
//
//   q, k   <- [q / sqrt(sum q^2 + 1e-6)], [k / ...]   (use_qk_l2norm_in_kernel)
//   q      <- q * scale
//   S      <- S * exp(g)          (scalar gate per token and value head, optional)
//   S      <- S * exp(gk)[:, None] (per key row, optional)
//   S      <- S * exp(gv)[None, :] (per value column, optional)
//   v'     <- beta * (v - S^T k)   (beta per head, or per value column)
//   S      <- S + k v'^T
//   o      <- S^T q                (stored in v's dtype)
//
// with S the fp32 [K, V] state of one (sequence, value head); q and k heads are
// shared by HV / H consecutive value heads (grouped value attention).
//
// Layout: one wave per (sequence, value head, 16 value columns).  Lane l holds
// column c = l / 4 of the tile and the K / 4 consecutive state rows
// kq * K/4 .. of quarter kq = l % 4, so every per-column reduction over K is a
// register sum plus two DPP quad exchanges, and a lane's q / k rows are one or
// more 16-byte loads.  The next token's inputs are loaded while the current
// token computes.  The state is read once from h0 and written once to ht:
// for decoding (T = 1) the kernel is bound by those two state passes in HBM.
// For K in {64, 128, 256} and V a multiple of 16 a vector form (below) moves the
// state in 16-byte accesses; the scalar form serves every other shape.
#include "gdn_common.hpp"
#include "gdn_kernels.h"

namespace kgdn {

namespace {

constexpr int kRecWaves = 4;   // waves per workgroup (independent work items)

// Sum over the 4 lanes of a quad (lanes l ^ 1, l ^ 2) through DPP quad_perm.
__device__ __forceinline__ float quad_sum(float x) {
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xf, 0xf, false));  // [1,0,3,2]
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xf, 0xf, false));  // [2,3,0,1]
  return x;
}

// RK consecutive elements of a q / k row as raw storage, loaded 16 bytes at a time
// where RK elements span at least 16 bytes.
template <typename T, int RK>
struct Row {
  static constexpr int kBytes = RK * (int)sizeof(T);
  static constexpr int kWords = kBytes / 4;
  uint32_t w[kWords];
};

template <typename T, int RK>
__device__ __forceinline__ void ld_row(Row<T, RK>& r, const T* p) {
  constexpr int W = Row<T, RK>::kWords;
  if constexpr (W % 4 == 0) {
#pragma unroll
    for (int i = 0; i < W / 4; ++i) {
      const uint4 x = reinterpret_cast<const uint4*>(p)[i];
      r.w[4 * i] = x.x; r.w[4 * i + 1] = x.y; r.w[4 * i + 2] = x.z; r.w[4 * i + 3] = x.w;
    }
  } else {   // W == 2 (8 bytes)
    const uint2 x = *reinterpret_cast<const uint2*>(p);
    r.w[0] = x.x; r.w[1] = x.y;
  }
}

template <typename T, int RK>
__device__ __forceinline__ float row_get(const Row<T, RK>& r, int j) {
  if constexpr (sizeof(T) == 4) {
    return __uint_as_float(r.w[j]);
  } else {
    const uint32_t x = r.w[j >> 1];
    return __uint_as_float((j & 1) ? (x & 0xffff0000u) : (x << 16));   // bf16 -> fp32 is exact
  }
}

template <typename TQ, typename TV, int RK>
struct TokIn {
  Row<TQ, RK> q, k;
  float v, g, beta, gv;
};

template <typename TQ, typename TV, int RK>
__device__ __forceinline__ void load_token(TokIn<TQ, TV, RK>& in, const RecArgs& a, int64_t tok, int i_h, int hv,
                                           int col, bool col_ok, int kq) {
  const int64_t qk_row = (tok * a.H + i_h) * (int64_t)(4 * RK) + kq * RK;
  ld_row<TQ, RK>(in.q, static_cast<const TQ*>(a.q) + qk_row);
  ld_row<TQ, RK>(in.k, static_cast<const TQ*>(a.k) + qk_row);
  const int64_t th = tok * a.HV + hv;
  in.v = col_ok ? to_f32(static_cast<const TV*>(a.v)[th * a.V + col]) : 0.f;
  in.g = a.g ? ld_scalar(a.g, th, a.g_dtype) : 0.f;
  in.gv = (a.gv && col_ok) ? ld_scalar(a.gv, th * a.V + col, a.gv_dtype) : 0.f;
  if (a.beta == nullptr) in.beta = 1.f;
  else if (a.beta_headwise) in.beta = ld_scalar(a.beta, th, a.beta_dtype);
  else in.beta = col_ok ? ld_scalar(a.beta, th * a.V + col, a.beta_dtype) : 0.f;
}

template <typename TQ, typename TV, int RK>
__global__ __launch_bounds__(WAVE * kRecWaves) void fused_recurrent_kernel(RecArgs a, int64_t total_waves) {
  const int64_t wv = (int64_t)blockIdx.x * kRecWaves + threadIdx.x / WAVE;
  if (wv >= total_waves) return;
  const int nvt = (a.V + 15) / 16;
  const int64_t nh = wv / nvt;
  const int col = (int)(wv % nvt) * 16 + lane_id() / 4;
  const int kq = lane_id() & 3;
  const int n = (int)(nh / a.HV), hv = (int)(nh % a.HV);
  const int i_h = hv / (a.HV / a.H);
  const bool col_ok = col < a.V;
  constexpr int K = 4 * RK;

  int64_t bos, T;
  if (a.cu) {
    bos = a.cu[n];
    T = a.cu[n + 1] - bos;
  } else {
    bos = (int64_t)n * a.T;
    T = a.T;
  }

  // state rows kq*RK + j of column col
  float S[RK];
  const int64_t st0 = ((int64_t)n * a.HV + hv) * K * a.V + (int64_t)(kq * RK) * a.V + col;
  with_state_loader(col_ok ? a.h0 : nullptr, a.h0_dtype == DT_F32 ? 0 : 1, [&](auto ld) {
#pragma unroll
    for (int j = 0; j < RK; ++j) S[j] = ld(st0 + (int64_t)j * a.V);
  });

  TokIn<TQ, TV, RK> cur, nxt;
  if (T > 0) load_token<TQ, TV, RK>(cur, a, bos, i_h, hv, col, col_ok, kq);
  TV* o = static_cast<TV*>(a.o);
  for (int64_t t = 0; t < T; ++t) {
    if (t + 1 < T) load_token<TQ, TV, RK>(nxt, a, bos + t + 1, i_h, hv, col, col_ok, kq);
    float q[RK], k[RK];
#pragma unroll
    for (int j = 0; j < RK; ++j) {
      q[j] = row_get<TQ, RK>(cur.q, j);
      k[j] = row_get<TQ, RK>(cur.k, j);
    }
    if (a.l2) {
      float sq = 0.f, sk = 0.f;
#pragma unroll
      for (int j = 0; j < RK; ++j) {
        sq = fmaf(q[j], q[j], sq);
        sk = fmaf(k[j], k[j], sk);
      }
      const float iq = 1.f / __builtin_sqrtf(quad_sum(sq) + 1e-6f);
      const float ik = 1.f / __builtin_sqrtf(quad_sum(sk) + 1e-6f);
#pragma unroll
      for (int j = 0; j < RK; ++j) {
        q[j] *= iq;
        k[j] *= ik;
      }
    }
#pragma unroll
    for (int j = 0; j < RK; ++j) q[j] *= a.scale;
    if (a.g) {
      const float e = gexp(cur.g);
#pragma unroll
      for (int j = 0; j < RK; ++j) S[j] *= e;
    }
    if (a.gk) {
      const int64_t gk0 = ((bos + t) * a.HV + hv) * (int64_t)K + kq * RK;
#pragma unroll
      for (int j = 0; j < RK; ++j) S[j] *= gexp(ld_scalar(a.gk, gk0 + j, a.gk_dtype));
    }
    if (a.gv) {
      const float e = gexp(cur.gv);
#pragma unroll
      for (int j = 0; j < RK; ++j) S[j] *= e;
    }
    float kS = 0.f;
#pragma unroll
    for (int j = 0; j < RK; ++j) kS = fmaf(S[j], k[j], kS);
    const float vp = cur.beta * (cur.v - quad_sum(kS));
    float oS = 0.f;
#pragma unroll
    for (int j = 0; j < RK; ++j) {
      S[j] = fmaf(k[j], vp, S[j]);
      oS = fmaf(S[j], q[j], oS);
    }
    oS = quad_sum(oS);
    if (kq == 0 && col_ok) o[((bos + t) * a.HV + hv) * a.V + col] = from_f32<TV>(oS);
    cur = nxt;
  }

  if (a.ht && col_ok) {
#pragma unroll
    for (int j = 0; j < RK; ++j) a.ht[st0 + (int64_t)j * a.V] = S[j];
  }
}

// ---------------------------------------------------------------------------
// Vector form (K in {64, 128, 256}, V a multiple of 16, 16-byte aligned state and
// 8-byte aligned v / o): lane l holds the 4 adjacent columns 4 (l / 16) .. of the
// wave's 16 and the K / 16 state rows of group kq = l % 16, so the state moves in
// 16-byte loads and stores (a quarter of the instructions of the scalar form) and
// every per-column reduction over K is a register sum plus 4 DPP steps inside a
// row of 16 lanes.
// ---------------------------------------------------------------------------

// Sum over the 16 lanes of a DPP row: quad exchanges, then half-row and row mirrors.
__device__ __forceinline__ float row16_sum(float x) {
  x = quad_sum(x);
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xf, 0xf, false));  // half mirror
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xf, 0xf, false));  // row mirror
  return x;
}

template <typename TV>
__device__ __forceinline__ f32x4 ld4_cols(const TV* p) { return ld4<TV>(p); }

template <typename TQ, int R>
struct VecTok {
  Row<TQ, R> q, k;
  f32x4 v, b;
  float g;
};

template <typename TQ, typename TV, int R>
__device__ __forceinline__ void load_vec_token(VecTok<TQ, R>& in, const RecArgs& a, int64_t tok, int i_h, int hv,
                                               int col, int kq) {
  const int64_t qk_row = (tok * a.H + i_h) * (int64_t)(16 * R) + kq * R;
  ld_row<TQ, R>(in.q, static_cast<const TQ*>(a.q) + qk_row);
  ld_row<TQ, R>(in.k, static_cast<const TQ*>(a.k) + qk_row);
  const int64_t th = tok * a.HV + hv;
  in.v = ld4_cols<TV>(static_cast<const TV*>(a.v) + th * a.V + col);
  if (a.beta == nullptr) {
    in.b = f32x4{1.f, 1.f, 1.f, 1.f};
  } else if (a.beta_headwise) {
    const float b = ld_scalar(a.beta, th, a.beta_dtype);
    in.b = f32x4{b, b, b, b};
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c) in.b[c] = ld_scalar(a.beta, th * a.V + col + c, a.beta_dtype);
  }
  in.g = a.g ? ld_scalar(a.g, th, a.g_dtype) : 0.f;
}

template <typename TQ, typename TV, int R>
__global__ __launch_bounds__(WAVE * kRecWaves) void fused_recurrent_vec_kernel(RecArgs a, int64_t total_waves) {
  const int64_t wv = (int64_t)blockIdx.x * kRecWaves + threadIdx.x / WAVE;
  if (wv >= total_waves) return;
  const int nvt = a.V / 16;
  const int64_t nh = wv / nvt;
  const int l = lane_id();
  const int kq = l & 15;
  const int col = (int)(wv % nvt) * 16 + 4 * (l >> 4);     // first of the lane's 4 columns
  const int n = (int)(nh / a.HV), hv = (int)(nh % a.HV);
  const int i_h = hv / (a.HV / a.H);
  constexpr int K = 16 * R;

  int64_t bos, T;
  if (a.cu) {
    bos = a.cu[n];
    T = a.cu[n + 1] - bos;
  } else {
    bos = (int64_t)n * a.T;
    T = a.T;
  }

  // state rows kq*R + j, columns col .. col+3
  f32x4 S[R];
  const int64_t st0 = ((int64_t)n * a.HV + hv) * K * a.V + (int64_t)(kq * R) * a.V + col;
#pragma unroll
  for (int j = 0; j < R; ++j) {
    if (a.h0 == nullptr) S[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    else if (a.h0_dtype == DT_F32) S[j] = *reinterpret_cast<const f32x4*>(static_cast<const float*>(a.h0) + st0 + (int64_t)j * a.V);
    else S[j] = ld4<bf16>(static_cast<const bf16*>(a.h0) + st0 + (int64_t)j * a.V);
  }

  TV* o = static_cast<TV*>(a.o);
  VecTok<TQ, R> cur, nxt;                              // the next token loads while this one computes
  if (T > 0) load_vec_token<TQ, TV, R>(cur, a, bos, i_h, hv, col, kq);
  for (int64_t t = 0; t < T; ++t) {
    const int64_t tok = bos + t;
    if (t + 1 < T) load_vec_token<TQ, TV, R>(nxt, a, tok + 1, i_h, hv, col, kq);
    const int64_t th = tok * a.HV + hv;
    const f32x4 vv = cur.v, bt = cur.b;
    float q[R], k[R];
#pragma unroll
    for (int j = 0; j < R; ++j) {
      q[j] = row_get<TQ, R>(cur.q, j);
      k[j] = row_get<TQ, R>(cur.k, j);
    }
    if (a.l2) {
      float sq = 0.f, sk = 0.f;
#pragma unroll
      for (int j = 0; j < R; ++j) {
        sq = fmaf(q[j], q[j], sq);
        sk = fmaf(k[j], k[j], sk);
      }
      const float iq = 1.f / __builtin_sqrtf(row16_sum(sq) + 1e-6f);
      const float ik = 1.f / __builtin_sqrtf(row16_sum(sk) + 1e-6f);
#pragma unroll
      for (int j = 0; j < R; ++j) {
        q[j] *= iq;
        k[j] *= ik;
      }
    }
#pragma unroll
    for (int j = 0; j < R; ++j) q[j] *= a.scale;
    if (a.g) {
      const float e = gexp(cur.g);
#pragma unroll
      for (int j = 0; j < R; ++j) S[j] *= e;
    }
    if (a.gk) {
      const int64_t gk0 = th * (int64_t)K + kq * R;
#pragma unroll
      for (int j = 0; j < R; ++j) S[j] *= gexp(ld_scalar(a.gk, gk0 + j, a.gk_dtype));
    }
    if (a.gv) {
      f32x4 e;
#pragma unroll
      for (int c = 0; c < 4; ++c) e[c] = gexp(ld_scalar(a.gv, th * a.V + col + c, a.gv_dtype));
#pragma unroll
      for (int j = 0; j < R; ++j) S[j] *= e;
    }
    f32x4 kS = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < R; ++j) {
#pragma unroll
      for (int c = 0; c < 4; ++c) kS[c] = fmaf(S[j][c], k[j], kS[c]);
    }
    f32x4 vp;
#pragma unroll
    for (int c = 0; c < 4; ++c) vp[c] = bt[c] * (vv[c] - row16_sum(kS[c]));
    f32x4 oS = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < R; ++j) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        S[j][c] = fmaf(k[j], vp[c], S[j][c]);
        oS[c] = fmaf(S[j][c], q[j], oS[c]);
      }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) oS[c] = row16_sum(oS[c]);
    if (kq == 0) st4<TV>(o + th * a.V + col, oS[0], oS[1], oS[2], oS[3]);
    cur = nxt;
  }

  if (a.ht) {
#pragma unroll
    for (int j = 0; j < R; ++j) *reinterpret_cast<f32x4*>(a.ht + st0 + (int64_t)j * a.V) = S[j];
  }
}

template <typename TQ, typename TV>
int launch_rec_t(const RecArgs& a, hipStream_t s) {
  const auto al = [](const void* p, uintptr_t m) { return (reinterpret_cast<uintptr_t>(p) & (m - 1)) == 0; };
  if ((a.K == 64 || a.K == 128 || a.K == 256) && a.V % 16 == 0 && al(a.h0, 16) && al(a.ht, 16) && al(a.v, 16) &&
      al(a.o, 16)) {
    const int64_t total = (int64_t)a.N * a.HV * (a.V / 16);
    if (total == 0) return 0;
    const dim3 grid((unsigned)((total + kRecWaves - 1) / kRecWaves));
#define KGDN_RECV_CASE(KK)                                                                                       \
    if (a.K == KK) {                                                                                             \
      hipLaunchKernelGGL((fused_recurrent_vec_kernel<TQ, TV, KK / 16>), grid, dim3(WAVE * kRecWaves), 0, s, a, total); \
      return hipGetLastError() == hipSuccess ? 0 : -1;                                                           \
    }
    KGDN_RECV_CASE(64) KGDN_RECV_CASE(128) KGDN_RECV_CASE(256)
#undef KGDN_RECV_CASE
  }
  const int64_t total = (int64_t)a.N * a.HV * ((a.V + 15) / 16);
  if (total == 0) return 0;
  const dim3 grid((unsigned)((total + kRecWaves - 1) / kRecWaves));
#define KGDN_REC_CASE(KK)                                                                                   \
  if (a.K == KK) {                                                                                          \
    hipLaunchKernelGGL((fused_recurrent_kernel<TQ, TV, KK / 4>), grid, dim3(WAVE * kRecWaves), 0, s, a, total); \
    return hipGetLastError() == hipSuccess ? 0 : -1;                                                        \
  }
  KGDN_REC_CASE(16) KGDN_REC_CASE(32) KGDN_REC_CASE(64) KGDN_REC_CASE(128) KGDN_REC_CASE(256)
#undef KGDN_REC_CASE
  return -2;
}

}  // namespace

int launch_fused_recurrent(const RecArgs& a, hipStream_t s) {
  if (a.qk_dtype == DT_BF16 && a.v_dtype == DT_BF16) return launch_rec_t<bf16, bf16>(a, s);
  if (a.qk_dtype == DT_F32 && a.v_dtype == DT_F32) return launch_rec_t<float, float>(a, s);
  if (a.qk_dtype == DT_BF16 && a.v_dtype == DT_F32) return launch_rec_t<bf16, float>(a, s);
  if (a.qk_dtype == DT_F32 && a.v_dtype == DT_BF16) return launch_rec_t<float, bf16>(a, s);
  return -2;
}

}  // namespace kgdn
