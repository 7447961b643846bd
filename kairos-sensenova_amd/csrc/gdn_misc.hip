// Small kernels around the chunked GatedDeltaNet forward:
//  * l2norm_kernel     y = x / sqrt(sum x^2 + 1e-6) per row (fla modules/l2norm.py:98-119),
//                      q and k in one launch,
//                      the optional q/k prologue of chunk.py:168-170;
//  * chunk_off_kernel  per-sequence chunk offsets from cu_seqlens
//                      (fla ops/utils/index.py:122-127), computed on the device so
//                      varlen calls need no host synchronisation;
//  * cumsum_kernel     chunk-local prefix sum of g (fla ops/utils/cumsum.py:27-65),
//                      the standalone form of the stage the prepare kernel fuses.
#include "gdn_common.hpp"
#include "gdn_kernels.h"

namespace kgdn {

namespace {

// Rows of D elements (a power of two, 8 <= D <= 512): a row takes LPR = D / 8 lanes
// (8 elements, one 16-byte load each in bf16), so a wave normalises 64 / LPR rows
// at once and every lane is busy; each thread handles RPT row groups, their loads
// all issued before the first reduction.  Up to two tensors per launch
// (blockIdx.y), each with its own rows.  rstd (fp32 per row) is written where
// its pointer is not null (l2norm.py:115-119 returns it beside y).
template <typename T, int D>
__global__ __launch_bounds__(256) void l2norm_kernel(const T* __restrict__ x0, T* __restrict__ y0,
                                                     const T* __restrict__ x1, T* __restrict__ y1,
                                                     float* __restrict__ r0, float* __restrict__ r1, int64_t rows) {
  constexpr int LPR = D / 8, RPW = WAVE / LPR, RPT = 4;
  const T* x = blockIdx.y ? x1 : x0;
  T* y = blockIdx.y ? y1 : y0;
  float* r = blockIdx.y ? r1 : r0;
  const int l = lane_id();
  const int64_t wave = ((int64_t)blockIdx.x * 4 + threadIdx.x / WAVE) * RPT;
  const int sub = l / LPR, col = 8 * (l % LPR);
  Vec8<T> v[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int64_t row = (wave + i) * RPW + sub;
    v[i] = row < rows ? ld8<T>(x + row * D + col) : vzero<T>();
  }
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int64_t row = (wave + i) * RPW + sub;
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float f = vget<T>(v[i], e);
      ss = fmaf(f, f, ss);
    }
#pragma unroll
    for (int off = LPR / 2; off > 0; off >>= 1) ss += __shfl_xor(ss, off, WAVE);
    const float rstd = 1.0f / sqrtf(ss + 1e-6f);
    if (row < rows) {
      Vec8<T> o;
#pragma unroll
      for (int e = 0; e < 8; ++e) vset<T>(o, e, vget<T>(v[i], e) * rstd);
      st8<T>(y + row * D + col, o);
      if (r != nullptr && col == 0) r[row] = rstd;
    }
  }
}

// Rows of any D (a multiple of 8, at most 512): one wave per row.
template <typename T>
__global__ __launch_bounds__(256) void l2norm_wave_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                          float* __restrict__ r, int64_t rows, int D) {
  const int64_t row = (int64_t)blockIdx.x * 4 + threadIdx.x / WAVE;
  if (row >= rows) return;
  const int l = lane_id();
  Vec8<T> v = vzero<T>();
  const bool act = 8 * l < D;
  if (act) v = ld8<T>(x + row * D + 8 * l);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float f = vget<T>(v, e);
    ss = fmaf(f, f, ss);
  }
#pragma unroll
  for (int off = WAVE / 2; off > 0; off >>= 1) ss += __shfl_xor(ss, off, WAVE);
  const float rstd = 1.0f / sqrtf(ss + 1e-6f);
  if (act) {
    Vec8<T> o;
#pragma unroll
    for (int e = 0; e < 8; ++e) vset<T>(o, e, vget<T>(v, e) * rstd);
    st8<T>(y + row * D + 8 * l, o);
  }
  if (r != nullptr && l == 0) r[row] = rstd;
}

__global__ void chunk_off_kernel(const int64_t* __restrict__ cu, int N, int32_t* __restrict__ off) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  int32_t acc = 0;
  off[0] = 0;
  for (int n = 0; n < N; ++n) {
    const int64_t len = cu[n + 1] - cu[n];
    acc += (int32_t)((len + C - 1) / C);
    off[n + 1] = acc;
  }
}

__global__ __launch_bounds__(64) void cumsum_kernel(const void* g, int g_dtype, float* gc, const int64_t* cu,
                                                    const int32_t* chunk_off, int N, int64_t T, int H) {
  const int h = blockIdx.y;
  const ChunkLoc loc = locate_chunk(blockIdx.x, cu, chunk_off, N, T);
  if (!loc.ok) return;
  const int l = lane_id();
  float gv = l < loc.nv ? ld_scalar(g, (loc.t0 + l) * H + h, g_dtype) : 0.f;
#pragma unroll
  for (int off = 1; off < WAVE; off <<= 1) {
    const float o = __shfl_up(gv, off, WAVE);
    if (l >= off) gv += o;
  }
  if (l < loc.nv) gc[(loc.t0 + l) * H + h] = gv;
}

}  // namespace

template <typename T, int D>
void launch_l2norm_t(const void* x0, void* y0, const void* x1, void* y1, float* r0, float* r1, int64_t rows,
                     hipStream_t s) {
  constexpr int64_t per_block = 4 * 4 * (WAVE / (D / 8));     // waves x row groups x rows per group
  const dim3 grid((unsigned)((rows + per_block - 1) / per_block), x1 ? 2u : 1u);
  hipLaunchKernelGGL((l2norm_kernel<T, D>), grid, dim3(256), 0, s, static_cast<const T*>(x0), static_cast<T*>(y0),
                     static_cast<const T*>(x1), static_cast<T*>(y1), r0, r1, rows);
}

template <typename T>
int launch_l2norm_dt(const void* x0, void* y0, const void* x1, void* y1, float* r0, float* r1, int64_t rows, int D,
                     hipStream_t s) {
  switch (D) {
    case 64: launch_l2norm_t<T, 64>(x0, y0, x1, y1, r0, r1, rows, s); break;
    case 128: launch_l2norm_t<T, 128>(x0, y0, x1, y1, r0, r1, rows, s); break;
    case 256: launch_l2norm_t<T, 256>(x0, y0, x1, y1, r0, r1, rows, s); break;
    case 512: launch_l2norm_t<T, 512>(x0, y0, x1, y1, r0, r1, rows, s); break;
    default: {
      const dim3 grid((unsigned)((rows + 3) / 4));
      hipLaunchKernelGGL(l2norm_wave_kernel<T>, grid, dim3(256), 0, s, static_cast<const T*>(x0), static_cast<T*>(y0),
                         r0, rows, D);
      if (x1)
        hipLaunchKernelGGL(l2norm_wave_kernel<T>, grid, dim3(256), 0, s, static_cast<const T*>(x1),
                           static_cast<T*>(y1), r1, rows, D);
    }
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_l2norm2(const void* x0, void* y0, const void* x1, void* y1, int dtype, int64_t rows, int D,
                   hipStream_t s, float* r0, float* r1) {
  if (D % 8 != 0 || D > 512 || rows <= 0) return -2;
  if (dtype == DT_F32) return launch_l2norm_dt<float>(x0, y0, x1, y1, r0, r1, rows, D, s);
  if (dtype == DT_BF16) return launch_l2norm_dt<bf16>(x0, y0, x1, y1, r0, r1, rows, D, s);
  return -2;
}

int launch_l2norm(const void* x, void* y, float* rstd, int dtype, int64_t rows, int D, hipStream_t s) {
  if (D % 8 != 0 || D > 512 || rows <= 0) return -2;
  if (dtype == DT_F32) return launch_l2norm_dt<float>(x, y, nullptr, nullptr, rstd, nullptr, rows, D, s);
  if (dtype == DT_BF16) return launch_l2norm_dt<bf16>(x, y, nullptr, nullptr, rstd, nullptr, rows, D, s);
  return -2;
}

int launch_chunk_offsets(const int64_t* cu, int N, int32_t* chunk_off, hipStream_t s) {
  hipLaunchKernelGGL(chunk_off_kernel, dim3(1), dim3(64), 0, s, cu, N, chunk_off);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_cumsum(const void* g, int g_dtype, float* gc, const int64_t* cu, const int32_t* chunk_off, int N,
                  int64_t T, int H, int64_t nc_grid, hipStream_t s) {
  hipLaunchKernelGGL(cumsum_kernel, dim3((unsigned)nc_grid, (unsigned)H), dim3(64), 0, s, g, g_dtype, gc, cu,
                     chunk_off, N, T, H);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace kgdn
