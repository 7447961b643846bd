// The GatedDeltaNet layer's short causal convolution + SiLU, applied where the chunked op stages the
// rows of q, k and v (the layer's prologue folded into the op's loads, gated_deltanet.py:234-271).
//
//   y[t, c] = bf16( silu( sum_{i<4} w[c][i] x~[t - 3 + i][c] + b[c] ) )
//
// (modules/convolution.py:54-141, the layer's ShortConvolution with activation 'silu'), x~ being the
// projection inside the sequence and, before its first token, the cache of the previous call
// ([N, D, 4], slot 3 the most recent input) or zero.  The arithmetic is the standalone convolution
// kernel's (gdn_prologue.hip): bias first, the taps in order by fma, SiLU as z / (1 + 2^(-z log2 e)),
// one rounding to bf16, so a staged row equals that kernel's output bit for bit.
#pragma once

#include "gdn_common.hpp"
#include "gdn_kernels.h"

namespace kgdn {

typedef unsigned int cvx4 __attribute__((ext_vector_type(4)));   // 8 bf16 channels (16 bytes)

// ConvIn (gdn_kernels.h): x [rows, D] bf16 with D = H * Dh (the channels of head h are h * Dh .. + Dh - 1,
// the layout of q / k / v), taps [D, 4] and bias [D] (may be null) in fp32 here, cache [N, D, 4] bf16 or
// null.

__device__ __forceinline__ float conv_silu(float z) {
  return z * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-z * 1.4426950408889634f));
}

// The taps and bias of 8 consecutive channels, fp32 (the launcher converts bf16 taps once), in
// registers: w[e] holds the 4 taps of channel c0 + e (one 16-byte row of the [D, 4] taps).
struct ConvTaps {
  cvx4 w[8];
  cvx4 b[2];
  __device__ __forceinline__ f32x4 taps(int e) const {
    return f32x4{__uint_as_float(w[e][0]), __uint_as_float(w[e][1]), __uint_as_float(w[e][2]),
                 __uint_as_float(w[e][3])};
  }
  __device__ __forceinline__ float bias(int e) const { return __uint_as_float(b[e >> 2][e & 3]); }
};

// taps [D, 4] and bias [D] fp32 (bias may be null: zeros)
__device__ __forceinline__ void load_taps(ConvTaps& t, const ConvIn& c, int64_t c0) {
  const cvx4* p = reinterpret_cast<const cvx4*>(reinterpret_cast<const float*>(c.w) + c0 * kConvW);
#pragma unroll
  for (int e = 0; e < 8; ++e) t.w[e] = p[e];
  if (c.b) {
    t.b[0] = *reinterpret_cast<const cvx4*>(reinterpret_cast<const float*>(c.b) + c0);
    t.b[1] = *reinterpret_cast<const cvx4*>(reinterpret_cast<const float*>(c.b) + c0 + 4);
  } else {
    t.b[0] = cvx4{0u, 0u, 0u, 0u};
    t.b[1] = cvx4{0u, 0u, 0u, 0u};
  }
}

// The same read from a copy in LDS (a head's taps [Dh][4] and bias [Dh], staged once per workgroup by
// stage_taps), one channel at a time: no tap is held in registers across the window.
struct ConvTapsLds {
  const float* w;                      // taps of channel c0: w[4 e + i]
  const float* b;                      // bias of channel c0 (or nullptr)
  __device__ __forceinline__ f32x4 taps(int e) const { return *reinterpret_cast<const f32x4*>(w + 4 * e); }
  __device__ __forceinline__ float bias(int e) const { return b ? b[e] : 0.f; }
};

// The taps [Dh][4] and bias [Dh] (zeros without a bias) of head h into LDS (fp32, 5 Dh floats), by the
// workgroup's NT threads; the caller publishes them with a barrier
template <int Dh, int NT>
__device__ __forceinline__ void stage_taps(float* dst, const ConvIn& c, int h) {
  const float* w = reinterpret_cast<const float*>(c.w) + (int64_t)h * Dh * kConvW;
  for (int i = threadIdx.x; i < Dh; i += NT) {
    *reinterpret_cast<f32x4*>(dst + 4 * i) = *reinterpret_cast<const f32x4*>(w + 4 * i);
    dst[kConvW * Dh + i] = c.b ? reinterpret_cast<const float*>(c.b)[(int64_t)h * Dh + i] : 0.f;
  }
}

// bf16 pair helpers on a packed word
__device__ __forceinline__ float cv_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float cv_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ uint32_t cv_pack(float a, float b) {
  const bf16 lo = (bf16)a, hi = (bf16)b;
  return (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
}

// Row s of the sequence [bos, eos) of sequence n, 8 channels from c0, as raw bf16: rows inside the
// sequence are loaded (rows past its end read its first row; their outputs are not used), rows before
// it come from the cache (slot s - bos + 4) or are zero.
struct ConvRow {
  __device__ __forceinline__ static int64_t clamp_row(int64_t s, int64_t bos, int64_t eos) {
    return s < bos || s >= eos ? bos : s;
  }
};

// R output rows t .. t + R - 1 (8 channels from c0) from the raw rows t - 3 .. t + R - 1 in
// registers.  issue() sends the loads; finish() forms the outputs.
template <int R>
struct ConvWin {
  cvx4 x[R + kConvW - 1];
  __device__ __forceinline__ void issue(const ConvIn& c, int64_t t, int64_t bos, int64_t eos, int64_t c0) {
#pragma unroll
    for (int i = 0; i < R + kConvW - 1; ++i) {
      const int64_t s = ConvRow::clamp_row(t - (kConvW - 1) + i, bos, eos);
      x[i] = *reinterpret_cast<const cvx4*>(reinterpret_cast<const bf16*>(c.x) + s * c.D + c0);
    }
  }
  // y rows as packed bf16 (out[r] = row t + r); rows before bos are taken from the cache or zero.
  // TP: ConvTaps or ConvTapsLds.
  template <typename TP>
  __device__ __forceinline__ void finish(const ConvIn& c, const TP& tp, int64_t t, int64_t bos, int n,
                                         int64_t c0, cvx4 (&out)[R]) {
    if (t - (kConvW - 1) < bos) {                        // the window starts before the sequence
#pragma unroll
      for (int i = 0; i < kConvW - 1; ++i) {
        const int64_t s = t - (kConvW - 1) + i;
        if (s < bos) {
          cvx4 v = {0u, 0u, 0u, 0u};
          const int slot = (int)(s - bos + kConvW);
          if (c.cache && slot >= 0) {
            const bf16* cp = reinterpret_cast<const bf16*>(c.cache) + ((int64_t)n * c.D + c0) * kConvW + slot;
#pragma unroll
            for (int e = 0; e < 4; ++e)
              v[e] = (uint32_t)__builtin_bit_cast(uint16_t, cp[(2 * e) * kConvW]) |
                     ((uint32_t)__builtin_bit_cast(uint16_t, cp[(2 * e + 1) * kConvW]) << 16);
          }
          x[i] = v;
        }
      }
    }
    float y[R][8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const f32x4 w4 = tp.taps(e);
      const float b0 = tp.bias(e);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float acc = b0;
#pragma unroll
        for (int i = 0; i < kConvW; ++i) {
          const uint32_t wd = x[r + i][e >> 1];
          acc = fmaf(w4[i], (e & 1) ? cv_hi(wd) : cv_lo(wd), acc);
        }
        y[r][e] = conv_silu(acc);
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int e = 0; e < 4; ++e) out[r][e] = cv_pack(y[r][2 * e], y[r][2 * e + 1]);
  }
};

// Sum of squares of 8 bf16 values (a packed row piece)
__device__ __forceinline__ float ss8(const cvx4& v) {
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    s = fmaf(cv_lo(v[e]), cv_lo(v[e]), s);
    s = fmaf(cv_hi(v[e]), cv_hi(v[e]), s);
  }
  return s;
}

// y = bf16(x r) on a packed row piece
__device__ __forceinline__ cvx4 scale8(const cvx4& v, float r) {
  cvx4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = cv_pack(cv_lo(v[e]) * r, cv_hi(v[e]) * r);
  return o;
}

}  // namespace kgdn
