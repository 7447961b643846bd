// Layout moves behind the stage entry points that take and return the
// reference's own tensor layouts (fla ops/common/chunk_delta_h.py:454-500 gives
// h [B, NT, H, K, V] and v_new [B, T, H, V]; fla ops/common/chunk_o.py:498-535
// takes them back; wy_fast.py:213-248 gives u [B, T, H, V]):
//  * chunk_tiles_kernel  token rows [B*T, H, D] <-> per-chunk transposed tiles
//                        [NCb, H, D, 64], the layout the stage kernels stream;
//                        token columns past a chunk's end, and chunks past the
//                        last real one, are written as zeros;
//  * state_tiles_kernel  per-chunk states [NCb, H, R, S] -> [NCb, H, S, R].
// Both are pure moves, HBM-bound (2 x the tensor's bytes): one 64 x 64 tile per
// workgroup, staged through LDS so that the read and the write both walk
// contiguous 64-element rows of a wave.
#include "gdn_common.hpp"
#include "gdn_kernels.h"

namespace kgdn {

namespace {

constexpr int TILE = 64;
constexpr int LAYOUT_THREADS = 256;
constexpr int ROW_GROUPS = LAYOUT_THREADS / TILE;   // rows a pass of the workgroup covers

// E is the element's storage word (2 bytes for bf16, 4 for fp32): nothing is converted.
// to_tiles = 1: tokens -> tiles; 0: tiles -> tokens.  grid (NCb, H, D / 64).
template <typename E>
__global__ __launch_bounds__(LAYOUT_THREADS) void chunk_tiles_kernel(const E* __restrict__ src, E* __restrict__ dst,
                                                                      int to_tiles, const int64_t* cu,
                                                                      const int32_t* chunk_off, int N, int64_t T,
                                                                      int H, int D) {
  __shared__ E tile[TILE][TILE + 1];            // [token][d]
  const int64_t c = blockIdx.x;
  const int h = blockIdx.y;
  const int d0 = blockIdx.z * TILE;
  const int lane = threadIdx.x % TILE, grp = threadIdx.x / TILE;
  const ChunkLoc loc = locate_chunk(c, cu, chunk_off, N, T);
  const int nv = loc.ok ? loc.nv : 0;
  const int64_t tile_base = (((int64_t)c * H + h) * D + d0) * TILE;   // row j = d0 + j, column i = token
  if (to_tiles) {
    for (int i = grp; i < TILE; i += ROW_GROUPS)                      // lane = d
      tile[i][lane] = i < nv ? src[((loc.t0 + i) * H + h) * D + d0 + lane] : E(0);
    __syncthreads();
    for (int j = grp; j < TILE; j += ROW_GROUPS)                      // lane = token
      dst[tile_base + (int64_t)j * TILE + lane] = tile[lane][j];
  } else {
    if (nv == 0) return;
    for (int j = grp; j < TILE; j += ROW_GROUPS)                      // lane = token
      tile[lane][j] = src[tile_base + (int64_t)j * TILE + lane];
    __syncthreads();
    for (int i = grp; i < nv; i += ROW_GROUPS)                        // lane = d
      dst[((loc.t0 + i) * H + h) * D + d0 + lane] = tile[i][lane];
  }
}

// grid (NCb * H, (R / 64) * (S / 64)); chunks past the last real one get zeros.
template <typename E>
__global__ __launch_bounds__(LAYOUT_THREADS) void state_tiles_kernel(const E* __restrict__ src, E* __restrict__ dst,
                                                                      const int64_t* cu, const int32_t* chunk_off,
                                                                      int N, int64_t T, int H, int R, int S) {
  __shared__ E tile[TILE][TILE + 1];            // [r][s]
  const int64_t ch = blockIdx.x;
  const int64_t c = ch / H;
  const int r0 = (blockIdx.y / (S / TILE)) * TILE, s0 = (blockIdx.y % (S / TILE)) * TILE;
  const int lane = threadIdx.x % TILE, grp = threadIdx.x / TILE;
  const bool ok = locate_chunk(c, cu, chunk_off, N, T).ok;
  const int64_t base = ch * R * S;
  for (int r = grp; r < TILE; r += ROW_GROUPS)                        // lane = s
    tile[r][lane] = ok ? src[base + (int64_t)(r0 + r) * S + s0 + lane] : E(0);
  __syncthreads();
  for (int s = grp; s < TILE; s += ROW_GROUPS)                        // lane = r
    dst[base + (int64_t)(s0 + s) * R + r0 + lane] = tile[lane][s];
}

}  // namespace

int launch_chunk_tiles(const void* src, void* dst, int to_tiles, int elem_bytes, const int64_t* cu,
                       const int32_t* chunk_off, int N, int64_t T, int H, int D, int64_t nc_grid, hipStream_t s) {
  if (D <= 0 || D % TILE != 0 || nc_grid <= 0 || nc_grid > 0x7fffffff || H <= 0 || H > 65535) return -2;
  const dim3 grid((unsigned)nc_grid, (unsigned)H, (unsigned)(D / TILE));
  if (elem_bytes == 2)
    hipLaunchKernelGGL(chunk_tiles_kernel<uint16_t>, grid, dim3(LAYOUT_THREADS), 0, s,
                       static_cast<const uint16_t*>(src), static_cast<uint16_t*>(dst), to_tiles, cu, chunk_off, N, T,
                       H, D);
  else if (elem_bytes == 4)
    hipLaunchKernelGGL(chunk_tiles_kernel<uint32_t>, grid, dim3(LAYOUT_THREADS), 0, s,
                       static_cast<const uint32_t*>(src), static_cast<uint32_t*>(dst), to_tiles, cu, chunk_off, N, T,
                       H, D);
  else
    return -2;
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_state_tiles(const void* src, void* dst, int elem_bytes, const int64_t* cu, const int32_t* chunk_off, int N,
                       int64_t T, int H, int R, int S, int64_t nc_grid, hipStream_t s) {
  if (R <= 0 || S <= 0 || R % TILE != 0 || S % TILE != 0 || nc_grid <= 0 || H <= 0) return -2;
  if (nc_grid * H > 0x7fffffff) return -2;
  const dim3 grid((unsigned)(nc_grid * H), (unsigned)((R / TILE) * (S / TILE)));
  if (elem_bytes == 2)
    hipLaunchKernelGGL(state_tiles_kernel<uint16_t>, grid, dim3(LAYOUT_THREADS), 0, s,
                       static_cast<const uint16_t*>(src), static_cast<uint16_t*>(dst), cu, chunk_off, N, T, H, R, S);
  else if (elem_bytes == 4)
    hipLaunchKernelGGL(state_tiles_kernel<uint32_t>, grid, dim3(LAYOUT_THREADS), 0, s,
                       static_cast<const uint32_t*>(src), static_cast<uint32_t*>(dst), cu, chunk_off, N, T, H, R, S);
  else
    return -2;
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace kgdn
