// Gated RMSNorm, the output epilogue of the GatedDeltaNet layer
// (GatedDeltaNet.o_norm = FusedRMSNormGated, fla layers/gated_deltanet.py:197,311;
// kernel fla modules/fused_norm_gate.py:42-127, RMS path, no residual):
//
//   rstd = 1 / sqrt(sum_d x^2 / D + eps)          (per row, fp32)
//   y    = x rstd w [+ b]                          (w, b optional, per column)
//   y   *= g sigmoid(g)   (activation swish / silu)  or  y *= sigmoid(g)  (sigmoid)
//
// x, g: [rows, D] in fp32 or bf16 (each its own dtype), w and b: [D] fp32 or
// bf16, y: x's dtype, rstd: [rows] fp32 (optional).  All arithmetic in fp32,
// y rounded once.  The op streams 2 reads and 1 write per element: HBM-bound.
//
// Layout: 8 consecutive elements per lane (one 16-byte bf16 load), LP lanes per
// row (LP = the power of two covering D / 8), 64 / LP rows per wave; the row
// sum is a butterfly over the LP lanes of the row.
#include "gdn_common.hpp"
#include "gdn_kernels.h"

namespace kgdn {

namespace {

// 8 consecutive per-column parameters (weight or bias) of dtype dt, as floats
__device__ __forceinline__ void ld_param8(const void* p, int c0, int dt, float (&out)[8]) {
  if (dt == DT_F32) {
    const Vec8<float> v = ld8<float>(static_cast<const float*>(p) + c0);
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = vget<float>(v, e);
  } else {
    const Vec8<bf16> v = ld8<bf16>(static_cast<const bf16*>(p) + c0);
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = vget<bf16>(v, e);
  }
}

// sigmoid(z) = 1 / (1 + e^-z) with e^-z = 2^(-z log2 e) (v_exp_f32) and the
// reciprocal on v_rcp_f32 (both within 1 ulp)
__device__ __forceinline__ float sigmoidf_(float z) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-z * 1.4426950408889634f));
}

template <typename TX, typename TG, int LP>
__global__ __launch_bounds__(256) void rmsnorm_gated_kernel(const TX* __restrict__ x, const TG* __restrict__ g,
                                                            const void* __restrict__ w, const void* __restrict__ b,
                                                            int w_dtype, TX* __restrict__ y, float* __restrict__ rstd,
                                                            int64_t rows, int D, float eps, int sigmoid_only) {
  constexpr int RPW = WAVE / LP;                         // rows per wave
  const int l = lane_id();
  const int sub = l / LP, lane = l % LP;
  const int64_t row = ((int64_t)blockIdx.x * (blockDim.x / WAVE) + threadIdx.x / WAVE) * RPW + sub;
  const int c0 = 8 * lane;
  const bool act = row < rows && c0 < D;
  Vec8<TX> xv = vzero<TX>();
  Vec8<TG> gv = vzero<TG>();
  if (act) {
    xv = ld8<TX>(x + row * D + c0);
    gv = ld8<TG>(g + row * D + c0);
  }
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float f = vget<TX>(xv, e);
    ss = fmaf(f, f, ss);
  }
#pragma unroll
  for (int off = LP / 2; off > 0; off >>= 1) ss += __shfl_xor(ss, off, LP);
  const float r = __builtin_amdgcn_rsqf(ss / (float)D + eps);
  if (!act) return;
  if (rstd != nullptr && lane == 0) rstd[row] = r;
  float wv[8], bv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    wv[e] = 1.f;
    bv[e] = 0.f;
  }
  if (w != nullptr) ld_param8(w, c0, w_dtype, wv);
  if (b != nullptr) ld_param8(b, c0, w_dtype, bv);
  Vec8<TX> yv;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float v = fmaf(vget<TX>(xv, e) * r, wv[e], bv[e]);
    const float gg = vget<TG>(gv, e);
    const float sg = sigmoidf_(gg);
    vset<TX>(yv, e, sigmoid_only ? v * sg : v * gg * sg);
  }
  st8<TX>(y + row * D + c0, yv);
}

template <typename TX, typename TG>
int launch_rmsnorm_gated_t(const NormArgs& a, hipStream_t s) {
  const int lanes = (a.D + 7) / 8;
  int lp = 1;
  while (lp < lanes) lp *= 2;
  const int rows_per_block = 4 * (WAVE / lp);
  const dim3 grid((unsigned)((a.rows + rows_per_block - 1) / rows_per_block));
  const TX* x = static_cast<const TX*>(a.x);
  const TG* g = static_cast<const TG*>(a.g);
  TX* y = static_cast<TX*>(a.y);
#define KGDN_NORM_CASE(LP)                                                                                        \
  if (lp == LP) {                                                                                                 \
    hipLaunchKernelGGL((rmsnorm_gated_kernel<TX, TG, LP>), grid, dim3(256), 0, s, x, g, a.w, a.b, a.w_dtype, y,   \
                       a.rstd, a.rows, a.D, a.eps, a.sigmoid_only);                                               \
    return hipGetLastError() == hipSuccess ? 0 : -1;                                                              \
  }
  KGDN_NORM_CASE(1) KGDN_NORM_CASE(2) KGDN_NORM_CASE(4) KGDN_NORM_CASE(8) KGDN_NORM_CASE(16) KGDN_NORM_CASE(32)
  KGDN_NORM_CASE(64)
#undef KGDN_NORM_CASE
  return -2;
}

}  // namespace

int launch_rmsnorm_gated(const NormArgs& a, hipStream_t s) {
  if (a.D <= 0 || a.D % 8 != 0 || a.D > 512 || a.rows <= 0) return -2;
  if (a.x_dtype == DT_BF16 && a.g_dtype == DT_BF16) return launch_rmsnorm_gated_t<bf16, bf16>(a, s);
  if (a.x_dtype == DT_BF16 && a.g_dtype == DT_F32) return launch_rmsnorm_gated_t<bf16, float>(a, s);
  if (a.x_dtype == DT_F32 && a.g_dtype == DT_BF16) return launch_rmsnorm_gated_t<float, bf16>(a, s);
  if (a.x_dtype == DT_F32 && a.g_dtype == DT_F32) return launch_rmsnorm_gated_t<float, float>(a, s);
  return -2;
}

}  // namespace kgdn
