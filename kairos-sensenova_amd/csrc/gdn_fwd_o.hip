// Chunk-parallel output stage of the chunked GatedDeltaNet forward
// (fla ops/common/chunk_o.py:41-128), one workgroup (4 waves) per (chunk, head):
//
//   o = scale * (q @ h_c) * exp(gc)
//     + scale * (mask_{i>=j}(q k^T * exp(gc_i - gc_j))).to(storage) @ v_new
//
// q of the chunk is staged row-major in LDS (K-contiguous for q.k^T and as the
// B operand of the transposed products); k is read as 16-byte fragments from
// global memory when it is stored in the compute type (staged otherwise), so the
// bf16 K=256 tile takes 43 KB and three workgroups share a CU.  The kernel computes o^T
// (rows = V columns, cols = tokens): the A operands are then the stored state
// snapshot hT [NC, H, V, K] and v_new^T [NC, H, V, 64], read as 16-byte
// fragments straight from global memory, and the accumulator layout gives each
// lane 4 consecutive V elements of one token, i.e. 8-byte token-major stores.
#include <type_traits>

#include "gdn_common.hpp"
#include "gdn_kernels.h"

namespace kgdn {

namespace {

// workgroup size: 8 waves at K = 256 (78 VGPRs, 43 KB LDS: 24 waves share a CU), else 4
template <int K> constexpr int nt_o() { return K >= 256 ? 512 : 256; }
constexpr int LDT = C + 8;

template <typename TC, int K, bool StageK>
struct OLds {
  static constexpr int LDK = K + 8;
  static constexpr size_t off_k = sizeof(TC) * C * LDK;
  static constexpr size_t off_A = off_k * (StageK ? 2 : 1);
  static constexpr size_t off_g = off_A + sizeof(TC) * C * LDT;
  static constexpr size_t total = off_g + sizeof(float) * C;
};

template <typename TC>
__device__ __forceinline__ Frag<TC> gfrag(const TC* p) {   // 8 consecutive elements, 16/32-byte aligned
  Frag<TC> f;
  if constexpr (sizeof(TC) == 2) {
    f.v = *reinterpret_cast<const bf16x8*>(p);
  } else {
    f.lo = *reinterpret_cast<const f32x4*>(p);
    f.hi = *reinterpret_cast<const f32x4*>(p + 4);
  }
  return f;
}

template <typename TC, typename TQ, int K>
// bf16: three workgroups share a CU as the LDS allows (at most 168 VGPRs with 4 waves,
// 80 with 8)
__global__ __launch_bounds__(nt_o<K>(), sizeof(TC) == 2 ? 3 * nt_o<K>() / 256 : 1) void fwd_o_kernel(FwdOArgs a, int V) {
  constexpr int NT_O = nt_o<K>(), NW = NT_O / WAVE;
  constexpr bool kStageK = !std::is_same<TC, TQ>::value;   // fp8 k is dequantised into LDS
  using L = OLds<TC, K, kStageK>;
  extern __shared__ __align__(16) unsigned char smem[];
  TC* s_q = reinterpret_cast<TC*>(smem);
  TC* s_k = reinterpret_cast<TC*>(smem + L::off_k);
  TC* s_Aqk = reinterpret_cast<TC*>(smem + L::off_A);
  float* s_g = reinterpret_cast<float*>(smem + L::off_g);

  const int h = blockIdx.y;
  const int H = a.H;
  const int64_t c = blockIdx.x;
  const ChunkLoc loc = locate_chunk(c, a.cu, a.chunk_off, a.N, a.T);
  if (!loc.ok) return;
  const int64_t t0 = loc.t0;
  const int nv = loc.nv;
  const int tid = threadIdx.x;
  const int wid = tid / WAVE;
  const int l = lane_id();
  const int lg = l >> 4, lc = l & 15;

  // ---- stage q, k (stored precision; fp8 inputs dequantised) and gc
  const TQ* qin = reinterpret_cast<const TQ*>(a.q);
  const TQ* kin = reinterpret_cast<const TQ*>(a.k);
  const float qs = a.q_scale ? a.q_scale[h] : 1.f;
  const float ksc = a.k_scale ? a.k_scale[h] : 1.f;
  for (int idx = tid; idx < (kStageK ? 2 : 1) * C * (K / 8); idx += NT_O) {
    const int which = idx / (C * (K / 8));
    const int rem = idx % (C * (K / 8));
    const int r = rem / (K / 8), c8 = (rem % (K / 8)) * 8;
    float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (r < nv) load8_in<TQ>((which ? kin : qin) + ((t0 + r) * H + h) * K + c8, which ? ksc : qs, x);
    Vec8<TC> row;
#pragma unroll
    for (int e = 0; e < 8; ++e) vset<TC>(row, e, x[e]);
    st8<TC>((which ? s_k : s_q) + r * L::LDK + c8, row);
  }
  if (tid < C) s_g[tid] = tid < nv ? a.gc[(t0 + tid) * H + h] : 0.f;
  __syncthreads();

  // ---- Aqk = mask_{i>=j}(q k^T exp(gc_i - gc_j)), rounded to the storage type
  for (int tile = wid; tile < 16; tile += NW) {
    const int tm = tile >> 2, tn = tile & 3;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    if (tn <= tm) {
      if constexpr (kStageK) {
#pragma unroll
        for (int ks = 0; ks < K / 32; ++ks)
          mma(acc, lds_frag<TC>(s_q, L::LDK, 16 * tm, 32 * ks), lds_frag<TC>(s_k, L::LDK, 16 * tn, 32 * ks));
      } else {
        // k row 16 tn + lc; rows past the chunk read as zero (their products are masked anyway,
        // and the last chunk's rows may lie past the end of the tensor)
        const int kr = 16 * tn + lc;
        const TC* krow = reinterpret_cast<const TC*>(a.k) + ((t0 + kr) * H + h) * K + 8 * lg;
        Frag<TC> kf[K / 32];
#pragma unroll
        for (int ks = 0; ks < K / 32; ++ks) kf[ks] = kr < nv ? gfrag<TC>(krow + 32 * ks) : Frag<TC>{};
#pragma unroll
        for (int ks = 0; ks < K / 32; ++ks) mma(acc, lds_frag<TC>(s_q, L::LDK, 16 * tm, 32 * ks), kf[ks]);
      }
    }
    const int j = 16 * tn + lc;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int i = 16 * tm + 4 * lg + jj;
      float val = 0.f;
      if (i >= j && i < nv) val = acc[jj] * gexp(s_g[i] - s_g[j]);
      s_Aqk[i * LDT + j] = from_f32<TC>(val);
    }
  }
  __syncthreads();

  // ---- o^T tiles: rows v (V/16 tiles over the waves), cols t (4 tiles)
  const TC* hT = reinterpret_cast<const TC*>(a.hT) + (c * H + h) * (int64_t)V * K;
  const TC* vnT = reinterpret_cast<const TC*>(a.vnT) + (c * H + h) * (int64_t)V * C;
  TC* o = reinterpret_cast<TC*>(a.o);
  // NP value tiles per wave per step (vt0, vt0 + NW, ..): their loads are all in flight before
  // the first one's products start (one at K = 256: two would not fit in 168 VGPRs)
  constexpr int NP = K >= 256 ? 1 : 2;
  for (int vt0 = wid; vt0 < V / 16; vt0 += NW * NP) {
    // compiler-only fence: q is re-read from LDS each step rather than hoisted into
    // 128 VGPRs, which would leave room for only two workgroups per CU
    if constexpr (K >= 256) asm volatile("" ::: "memory");
    Frag<TC> hf[NP][K / 32], vf[NP][2];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      if (vt0 + NW * p >= V / 16) break;           // uniform per wave
      const int vt = vt0 + NW * p;
#pragma unroll
      for (int ks = 0; ks < K / 32; ++ks) hf[p][ks] = gfrag<TC>(hT + (16 * vt + lc) * K + 32 * ks + 8 * lg);
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) vf[p][ks] = gfrag<TC>(vnT + (16 * vt + lc) * C + 32 * ks + 8 * lg);
    }
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      if (vt0 + NW * p >= V / 16) break;
      const int vt = vt0 + NW * p;
#pragma unroll
      for (int tn = 0; tn < 4; ++tn) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f}, acc2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < K / 32; ++ks) mma(acc, hf[p][ks], lds_frag<TC>(s_q, L::LDK, 16 * tn, 32 * ks));
#pragma unroll
        for (int ks = 0; ks <= tn / 2; ++ks) mma(acc2, vf[p][ks], lds_frag<TC>(s_Aqk, LDT, 16 * tn, 32 * ks));
        const int t = 16 * tn + lc;
        const float eg = gexp(s_g[t]);
        if (t < nv) {
          st4<TC>(o + ((t0 + t) * H + h) * V + 16 * vt + 4 * lg,
                  acc[0] * eg * a.scale + acc2[0] * a.scale, acc[1] * eg * a.scale + acc2[1] * a.scale,
                  acc[2] * eg * a.scale + acc2[2] * a.scale, acc[3] * eg * a.scale + acc2[3] * a.scale);
        }
      }
    }
  }
}

template <typename TC, typename TQ, int K>
int launch_fwd_o_t(const FwdOArgs& a, int V, int64_t nc_grid, hipStream_t s) {
  using L = OLds<TC, K, !std::is_same<TC, TQ>::value>;
  static_assert(L::total <= 160 * 1024, "output tile does not fit in LDS");
  auto kern = fwd_o_kernel<TC, TQ, K>;
  if (L::total > 64 * 1024) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)L::total) != hipSuccess)
      return -1;
  }
  dim3 grid((unsigned)nc_grid, (unsigned)a.H);
  hipLaunchKernelGGL(kern, grid, dim3(nt_o<K>()), L::total, s, a, V);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace

int launch_fwd_o(const FwdOArgs& a, int compute_dtype, int qk_dtype, int K, int V, int64_t nc_grid,
                 hipStream_t s) {
  if (V % 16 != 0) return -2;
#define KGDN_O_CASE(TC, TQ, KK) \
  if (K == KK) return launch_fwd_o_t<TC, TQ, KK>(a, V, nc_grid, s);
#define KGDN_O_SHAPES(TC, TQ) KGDN_O_CASE(TC, TQ, 64) KGDN_O_CASE(TC, TQ, 128) KGDN_O_CASE(TC, TQ, 256)
  if (compute_dtype == DT_F32 && qk_dtype == DT_F32) { KGDN_O_SHAPES(float, float) }
  if (compute_dtype == DT_BF16 && qk_dtype == DT_BF16) { KGDN_O_SHAPES(bf16, bf16) }
  if (compute_dtype == DT_BF16 && qk_dtype == DT_F8E4M3) { KGDN_O_SHAPES(bf16, uint8_t) }
#undef KGDN_O_SHAPES
#undef KGDN_O_CASE
  return -2;
}

}  // namespace kgdn
