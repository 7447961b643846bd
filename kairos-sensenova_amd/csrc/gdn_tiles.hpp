// LDS tiles of 64 token rows x ncol columns shared by the backward kernels and the all-columns
// state recurrence: bf16 tiles as [64][64] column blocks swizzled by swz_off<64> (16-byte row reads,
// 8-byte accumulator-order reads and ds_read_b64_tr_b16 transposed reads are bank-conflict free),
// fp32 tiles as padded rows.
#pragma once

#include "gdn_common.hpp"

namespace kgdn {

template <typename TC>
__host__ __device__ constexpr int tile_elems(int ncol) {
  return sizeof(TC) == 2 ? 64 * ncol : 64 * (ncol + 4);
}

template <typename TC>
__device__ __forceinline__ int toff(int r, int c, int ncol) {
  if constexpr (sizeof(TC) == 2) {
    return (c >> 6) * 4096 + swz_off<64>(r, (c & 63) >> 3) + (c & 7);
  } else {
    return r * (ncol + 4) + c;
  }
}

// natural K order: M/N index = row r0 + l % 16, K index = k0 + 8 (l / 16) + e
template <typename TC>
__device__ __forceinline__ Frag<TC> t_nat(const TC* t, int ncol, int r0, int k0) {
  const int l = lane_id();
  const TC* p = t + toff<TC>(r0 + (l & 15), k0 + 8 * (l >> 4), ncol);
  Frag<TC> f;
  if constexpr (sizeof(TC) == 2) {
    f.v = *reinterpret_cast<const bf16x8*>(p);
  } else {
    f.lo = *reinterpret_cast<const f32x4*>(p);
    f.hi = *reinterpret_cast<const f32x4*>(p + 4);
  }
  return f;
}

// accumulator K order: M/N index = row r0 + l % 16, K index = k0 + 4 lg + e and k0 + 16 + 4 lg + e
template <typename TC>
__device__ __forceinline__ Frag<TC> t_acc(const TC* t, int ncol, int r0, int k0) {
  const int l = lane_id();
  const int r = r0 + (l & 15), lg = l >> 4;
  const TC* p0 = t + toff<TC>(r, k0 + 4 * lg, ncol);
  const TC* p1 = t + toff<TC>(r, k0 + 16 + 4 * lg, ncol);
  Frag<TC> f;
  if constexpr (sizeof(TC) == 2) {
    const bf16x4 a = *reinterpret_cast<const bf16x4*>(p0);
    const bf16x4 b = *reinterpret_cast<const bf16x4*>(p1);
    f.v = __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
  } else {
    f.lo = *reinterpret_cast<const f32x4*>(p0);
    f.hi = *reinterpret_cast<const f32x4*>(p1);
  }
  return f;
}

// transposed: M/N index = column c0 + l % 16, K index = row k0 + (accumulator order), k0 a multiple of 32
template <typename TC>
__device__ __forceinline__ Frag<TC> t_tr(const TC* t, int ncol, int k0, int c0) {
  if constexpr (sizeof(TC) == 2) {
    return tr_frag<64>(t + (c0 >> 6) * 4096, k0 >> 5, c0 & 63);
  } else {
    const int l = lane_id();
    const int c = c0 + (l & 15), lg = l >> 4;
    Frag<float> f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      f.lo[e] = t[toff<float>(k0 + 4 * lg + e, c, ncol)];
      f.hi[e] = t[toff<float>(k0 + 16 + 4 * lg + e, c, ncol)];
    }
    return f;
  }
}

}  // namespace kgdn
