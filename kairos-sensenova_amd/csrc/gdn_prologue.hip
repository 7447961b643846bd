// Prologue of the GatedDeltaNet layer: the inputs of the chunked op.
//
// 1. Short causal convolution over time, per channel (ShortConvolution /
//    causal_conv1d, fla modules/convolution.py:410-458, kernel :54-141), with
//    the layer's SiLU (layers/gated_deltanet.py:176-189,235-253):
//      y[t, d] = act( sum_{i<W} w[d, i] x~[t - W + 1 + i, d] + bias[d] )
//    where x~ is x inside the sequence and, before its first token, the cache
//    [N, D, W] of the previous call (slot W-1 = most recent input) or zeros.
//    fp32 accumulation, y rounded once to x's dtype.  Optionally the rounded y
//    is then L2-normalised per head of hd channels (y / sqrt(sum y^2 + 1e-6),
//    fla modules/l2norm.py:115-118), the q/k normalisation the layer asks the
//    chunked op for (use_qk_l2norm_in_kernel=True, gated_deltanet.py:283):
//    fusing it here saves the op a read and a write of q and k.
// 2. The final cache: the last W entries of [cache, x] per sequence
//    (causal_conv1d_update_states, convolution.py:539-602).
// 3. The gates (gated_deltanet.py:265-271): g = -exp(A_log) softplus(a + dt_bias)
//    in fp32 (softplus threshold 20), beta = sigmoid(b) in b's dtype (times 2
//    with allow_neg_eigval).
//
// Layout of the convolution: lane = 8 consecutive channels (one 16-byte bf16
// load), wave = 512 channels, and a wave walks a run of kConvRun consecutive
// tokens keeping the W - 1 previous inputs in registers, so each input row is
// read once (plus W - 1 halo rows per run).  Every kernel here is HBM-bound.
#include "gdn_common.hpp"
#include "gdn_kernels.h"

namespace kgdn {

namespace {

constexpr int kConvRun = 64;     // tokens per wave (a sweep of 8..256 at the model shape: 64 fastest)
constexpr int kConvWaves = 4;

__device__ __forceinline__ float sigmoid_f(float z) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-z * 1.4426950408889634f));
}

// 8 channels of a runtime-typed per-channel parameter array (fp32 or bf16)
__device__ __forceinline__ void ld_chan8(const void* p, int64_t i, int dt, float (&out)[8]) {
#pragma unroll
  for (int e = 0; e < 8; ++e) out[e] = ld_scalar(p, i + e, dt);
}

template <typename TX>
__device__ __forceinline__ void ld_row8(const TX* p, float (&out)[8]) {
  const Vec8<TX> v = ld8<TX>(p);
#pragma unroll
  for (int e = 0; e < 8; ++e) out[e] = vget<TX>(v, e);
}

// Sequence containing flattened token t: [bos, eos) and its index.
__device__ __forceinline__ void seq_of(int64_t t, const ConvArgs& a, int& n, int64_t& bos, int64_t& eos) {
  if (a.cu == nullptr) {
    n = (int)(t / a.T);
    bos = (int64_t)n * a.T;
    eos = bos + a.T;
    return;
  }
  int lo = 0, hi = a.N - 1;                        // last n with cu[n] <= t
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (a.cu[mid] <= t) lo = mid; else hi = mid - 1;
  }
  while (lo + 1 < a.N && a.cu[lo + 1] <= t) ++lo;  // skip empty sequences ending at t
  n = lo;
  bos = a.cu[lo];
  eos = a.cu[lo + 1];
}

template <typename TX, int W, int HL>
__global__ __launch_bounds__(WAVE * kConvWaves) void conv1d_kernel(ConvArgs a, int64_t n_runs) {
  const int64_t wv = (int64_t)blockIdx.x * kConvWaves + threadIdx.x / WAVE;
  const int ncg = (a.D + 511) / 512;
  const int64_t run = wv / ncg;
  if (run >= n_runs) return;
  const int l = lane_id();
  const int c0 = (int)(wv % ncg) * 512 + 8 * l;
  const bool ok = c0 < a.D;
  const int64_t t_begin = run * kConvRun;
  const int64_t t_stop = min(t_begin + (int64_t)kConvRun, a.total_tokens);
  const TX* x = static_cast<const TX*>(a.x);
  TX* y = static_cast<TX*>(a.y);

  // taps of the lane's 8 channels: 8 W consecutive elements of weight [D, W], read 8 at a time
  float wt[W][8], bias[8];
#pragma unroll
  for (int q = 0; q < W; ++q) {
    float w8[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (ok) {
      if (a.w_dtype == DT_F32) ld_row8<float>(static_cast<const float*>(a.w) + (int64_t)c0 * W + 8 * q, w8);
      else ld_row8<bf16>(static_cast<const bf16*>(a.w) + (int64_t)c0 * W + 8 * q, w8);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int f = 8 * q + e;                       // flat index (channel c0 + f / W, tap f % W)
      wt[f % W][f / W] = w8[e];
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) bias[e] = 0.f;
  if (a.bias && ok) ld_chan8(a.bias, c0, a.w_dtype, bias);

  int n;
  int64_t bos, eos;
  seq_of(t_begin, a, n, bos, eos);
  // window: win[i] = x~[t - (W - 1) + i], i < W - 1
  float win[W > 1 ? W - 1 : 1][8];
  auto fill_window = [&](int64_t t) {
#pragma unroll
    for (int i = 0; i < W - 1; ++i) {
      const int64_t s = t - (W - 1) + i;
#pragma unroll
      for (int e = 0; e < 8; ++e) win[i][e] = 0.f;
      if (!ok) continue;
      if (s >= bos) {
        ld_row8<TX>(x + s * a.D + c0, win[i]);
      } else if (a.h0 && s - bos + W >= 0) {       // cache slot of x~[s]
#pragma unroll
        for (int e = 0; e < 8; ++e)
          win[i][e] = ld_scalar(a.h0, ((int64_t)n * a.D + c0 + e) * W + (s - bos + W), a.x_dtype);
      }
    }
  };
  fill_window(t_begin);

  for (int64_t t = t_begin; t < t_stop; ++t) {
    if (t >= eos) {                                 // next sequence (varlen): restart the window
      seq_of(t, a, n, bos, eos);
      fill_window(t);
    }
    float cur[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) cur[e] = 0.f;
    if (ok) ld_row8<TX>(x + t * a.D + c0, cur);
    float out[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float acc = bias[e];
#pragma unroll
      for (int i = 0; i < W - 1; ++i) acc = fmaf(wt[i][e], win[i][e], acc);
      acc = fmaf(wt[W - 1][e], cur[e], acc);
      if (a.silu) acc = acc * sigmoid_f(acc);
      out[e] = round_to<TX>(acc);
    }
    if constexpr (HL > 0) {                         // per-head L2 norm over HL lanes of 8 channels
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(out[e], out[e], ss);
#pragma unroll
      for (int off = HL / 2; off > 0; off >>= 1) ss += __shfl_xor(ss, off, HL);
      const float r = 1.0f / __builtin_sqrtf(ss + 1e-6f);
#pragma unroll
      for (int e = 0; e < 8; ++e) out[e] *= r;
    }
    if (ok) {
      Vec8<TX> o;
#pragma unroll
      for (int e = 0; e < 8; ++e) vset<TX>(o, e, out[e]);
      st8<TX>(y + t * a.D + c0, o);
    }
#pragma unroll
    for (int i = 0; i + 1 < W - 1; ++i) {
#pragma unroll
      for (int e = 0; e < 8; ++e) win[i][e] = win[i + 1][e];
    }
    if constexpr (W > 1) {
#pragma unroll
      for (int e = 0; e < 8; ++e) win[W - 2][e] = cur[e];
    }
  }
}

// final cache [N, D, W]: entry w = x~[eos - W + w] (x inside the sequence, else the old cache
// slot w + T, else zero), one thread per (sequence, channel)
template <typename TX>
__global__ __launch_bounds__(256) void conv_state_kernel(ConvArgs a) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)a.N * a.D) return;
  const int n = (int)(i / a.D), d = (int)(i % a.D);
  const int64_t bos = a.cu ? a.cu[n] : (int64_t)n * a.T;
  const int64_t eos = a.cu ? a.cu[n + 1] : bos + a.T;
  const int64_t T = eos - bos;
  const TX* x = static_cast<const TX*>(a.x);
  TX* ht = static_cast<TX*>(a.ht);
  for (int w = 0; w < a.W; ++w) {
    const int64_t s = eos - a.W + w;
    TX v = from_f32<TX>(0.f);
    if (s >= bos) v = x[s * a.D + d];
    else if (a.h0 && w + T < a.W) v = from_f32<TX>(ld_scalar(a.h0, i * a.W + w + T, a.x_dtype));
    ht[i * a.W + w] = v;
  }
}

__device__ __forceinline__ float softplus_f(float x) {   // torch softplus, beta 1, threshold 20
  return x > 20.f ? x : log1pf(expf(x));
}

template <typename TB>
__global__ __launch_bounds__(256) void gates_kernel(GateArgs a) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= a.rows * a.HV) return;
  const int h = (int)(i % a.HV);
  const float av = ld_scalar(a.a, i, a.a_dtype) + ld_scalar(a.dt_bias, h, a.p_dtype);
  a.g[i] = -expf(ld_scalar(a.A_log, h, a.p_dtype)) * softplus_f(av);
  const float bv = ld_scalar(a.b, i, a.b_dtype);
  float beta = round_to<TB>(1.0f / (1.0f + expf(-bv)));
  if (a.neg_eigval) beta *= 2.f;                    // exact in either dtype
  static_cast<TB*>(a.beta)[i] = from_f32<TB>(beta);
}

// fp32 copy of n values of a runtime-typed array (the folded convolution reads fp32 taps)
__global__ __launch_bounds__(256) void to_f32_kernel(const void* src, int dt, float* dst, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) dst[i] = ld_scalar(src, i, dt);
}

template <typename TX, int W>
int launch_conv_w(const ConvArgs& a, int64_t n_runs, hipStream_t s) {
  const int64_t waves = n_runs * ((a.D + 511) / 512);
  const dim3 grid((unsigned)((waves + kConvWaves - 1) / kConvWaves));
  switch (a.head_lanes) {
#define KGDN_CONV_CASE(HL) \
    case HL: hipLaunchKernelGGL((conv1d_kernel<TX, W, HL>), grid, dim3(WAVE * kConvWaves), 0, s, a, n_runs); break;
    KGDN_CONV_CASE(0) KGDN_CONV_CASE(8) KGDN_CONV_CASE(16) KGDN_CONV_CASE(32) KGDN_CONV_CASE(64)
#undef KGDN_CONV_CASE
    default: return -2;
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <typename TX>
int launch_conv_t(const ConvArgs& a, hipStream_t s) {
  const int64_t n_runs = (a.total_tokens + kConvRun - 1) / kConvRun;
  if (n_runs > 0) {
    int rc = -2;
    switch (a.W) {
      case 1: rc = launch_conv_w<TX, 1>(a, n_runs, s); break;
      case 2: rc = launch_conv_w<TX, 2>(a, n_runs, s); break;
      case 3: rc = launch_conv_w<TX, 3>(a, n_runs, s); break;
      case 4: rc = launch_conv_w<TX, 4>(a, n_runs, s); break;
      default: return -2;
    }
    if (rc) return rc;
  }
  if (a.ht && a.N > 0) {
    const int64_t total = (int64_t)a.N * a.D;
    hipLaunchKernelGGL(conv_state_kernel<TX>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, a);
    if (hipGetLastError() != hipSuccess) return -1;
  }
  return 0;
}

}  // namespace

int launch_conv1d(const ConvArgs& a, hipStream_t s) {
  if (a.x_dtype == DT_BF16) return launch_conv_t<bf16>(a, s);
  if (a.x_dtype == DT_F32) return launch_conv_t<float>(a, s);
  return -2;
}

int launch_conv_state(const ConvArgs& a, hipStream_t s) {
  if (!a.ht || a.N <= 0) return 0;
  const int64_t total = (int64_t)a.N * a.D;
  if (a.x_dtype == DT_BF16)
    hipLaunchKernelGGL(conv_state_kernel<bf16>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, a);
  else if (a.x_dtype == DT_F32)
    hipLaunchKernelGGL(conv_state_kernel<float>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, a);
  else
    return -2;
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_to_f32(const void* src, int dtype, float* dst, int64_t n, hipStream_t s) {
  if (n <= 0) return 0;
  hipLaunchKernelGGL(to_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, src, dtype, dst, n);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_gates(const GateArgs& a, hipStream_t s) {
  const int64_t total = a.rows * a.HV;
  if (total == 0) return 0;
  const dim3 grid((unsigned)((total + 255) / 256));
  if (a.b_dtype == DT_BF16) hipLaunchKernelGGL(gates_kernel<bf16>, grid, dim3(256), 0, s, a);
  else hipLaunchKernelGGL(gates_kernel<float>, grid, dim3(256), 0, s, a);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace kgdn
