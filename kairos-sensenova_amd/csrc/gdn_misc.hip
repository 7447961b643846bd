// Small kernels around the chunked GatedDeltaNet forward:
//  * l2norm_kernel     y = x / sqrt(sum x^2 + 1e-6) per row (fla modules/l2norm.py:98-119),
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

// One wave per row; D <= 512, a multiple of 8.
template <typename T>
__global__ __launch_bounds__(256) void l2norm_kernel(const T* __restrict__ x, T* __restrict__ y, int64_t rows,
                                                     int D) {
  const int64_t row = (int64_t)blockIdx.x * 4 + threadIdx.x / WAVE;
  if (row >= rows) return;
  const int l = lane_id();
  const T* xr = x + row * D;
  T* yr = y + row * D;
  Vec8<T> v = vzero<T>();
  const bool act = 8 * l < D;
  if (act) v = ld8<T>(xr + 8 * l);
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
    st8<T>(yr + 8 * l, o);
  }
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

int launch_l2norm(const void* x, void* y, int dtype, int64_t rows, int D, hipStream_t s) {
  if (D % 8 != 0 || D > 512 || rows <= 0) return -2;
  const dim3 grid((unsigned)((rows + 3) / 4));
  if (dtype == DT_F32) {
    hipLaunchKernelGGL(l2norm_kernel<float>, grid, dim3(256), 0, s, static_cast<const float*>(x),
                       static_cast<float*>(y), rows, D);
  } else if (dtype == DT_BF16) {
    hipLaunchKernelGGL(l2norm_kernel<bf16>, grid, dim3(256), 0, s, static_cast<const bf16*>(x),
                       static_cast<bf16*>(y), rows, D);
  } else {
    return -2;
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
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
