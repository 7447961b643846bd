// Shared device helpers for the gfx950 chunked GatedDeltaNet forward.
//
// Conventions used by every kernel in this directory:
//  * One "chunk" is 64 consecutive tokens of one sequence (C = 64).
//  * Matrix products run on the CDNA4 matrix cores with 16x16 output tiles:
//      bf16: v_mfma_f32_16x16x32_bf16 (one instruction per 32-deep K step)
//      fp32: eight v_mfma_f32_16x16x4f32 per 32-deep K step
//    Lane l of a 64-wide wave holds, for a K step of 32,
//      A fragment: A[row0 + l%16][k0 + 8*(l/16) + e], e = 0..7
//      B fragment: B[k0 + 8*(l/16) + e][col0 + l%16], e = 0..7
//      C/D tile  : D[row0 + 4*(l/16) + j][col0 + l%16], j = 0..3
//    Any permutation of the K index is allowed as long as A and B use the
//    same one; several kernels exploit that to feed accumulator tiles back
//    as operands without a shuffle.
//  * Operands staged in LDS are stored "K-contiguous": A as [m][k] and B as
//    [n][k], padded by 8 elements per row, so one fragment is one 16-byte read.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kgdn {

constexpr int C = 64;        // chunk length (tokens)
constexpr int WAVE = 64;     // CDNA wavefront width

typedef __bf16 bf16;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2;

// ---------------------------------------------------------------------------
// element conversion
// ---------------------------------------------------------------------------
__device__ __forceinline__ float to_f32(bf16 x) { return (float)x; }
__device__ __forceinline__ float to_f32(float x) { return x; }

// Device-memory accesses through address-space-1 pointers.  A plain pointer that the compiler cannot
// place in an address space (here: one computed from a pointer field of a kernel's argument struct)
// is accessed with FLAT instructions, which also count against lgkmcnt: every later wait for an LDS
// access of the wave then waits for those stores to reach memory too.
// (T is moved as a plain vector of 4-byte words of its size: HIP's vector structs have no assignment
// through an address-space-1 pointer.)
template <int N> struct GWords { typedef __attribute__((ext_vector_type(N))) unsigned type; };
template <> struct GWords<1> { typedef unsigned type; };
template <typename T>
__device__ __forceinline__ void st_global(void* p, const T& x) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8 || sizeof(T) == 16, "4, 8 or 16 bytes");
  using W = typename GWords<sizeof(T) / 4>::type;
  *(__attribute__((address_space(1))) W*)p = __builtin_bit_cast(W, x);
}
template <typename T>
__device__ __forceinline__ T ld_global(const void* p) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8 || sizeof(T) == 16, "4, 8 or 16 bytes");
  using W = typename GWords<sizeof(T) / 4>::type;
  return __builtin_bit_cast(T, *(const __attribute__((address_space(1))) W*)p);
}

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
// float -> bf16 with round-to-nearest-even (the hardware conversion on gfx950).
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float x) { return (bf16)x; }

// Round a float to the storage precision T and back (identity for float).
template <typename T> __device__ __forceinline__ float round_to(float x) { return to_f32(from_f32<T>(x)); }

// Four OCP fp8 e4m3 ("fn") codes packed in a dword (byte i = element i) -> four floats, exact.
// gfx950 decodes the OCP format in hardware, two codes per v_cvt_pk_f32_fp8 (sign, 4-bit exponent of
// bias 7, 3-bit mantissa, subnormals at exponent 0, 0x7f / 0xff NaN).  The same instruction decodes
// the FNUZ format (bias 8, one NaN) on earlier targets, so device code for any other target is
// refused here rather than decoding with another meaning.
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "kairos_gdn device code is written for gfx950 (OCP fp8 decode, 16-bit transposed LDS reads)"
#endif
__device__ __forceinline__ void fp8x4_to_f32(uint32_t w, float out[4]) {
  const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);    // bytes 0, 1
  const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);     // bytes 2, 3
  out[0] = lo[0];
  out[1] = lo[1];
  out[2] = hi[0];
  out[3] = hi[1];
}

// exp(x) via the native base-2 exponential (v_exp_f32): exp(x) = 2^(x*log2(e)).
__device__ __forceinline__ float gexp(float x) {
  return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}

// ---------------------------------------------------------------------------
// MFMA fragments
// ---------------------------------------------------------------------------
template <typename T> struct Frag;
template <> struct Frag<bf16> { bf16x8 v; };
template <> struct Frag<float> { f32x4 lo, hi; };

__device__ __forceinline__ int lane_id() { return threadIdx.x & (WAVE - 1); }

// Fragment of a K-contiguous LDS matrix: rows row0 + l%16, k = k0 + 8*(l/16) .. +7.
template <typename T>
__device__ __forceinline__ Frag<T> lds_frag(const T* base, int ld, int row0, int k0) {
  const int l = lane_id();
  const T* p = base + (row0 + (l & 15)) * ld + k0 + 8 * (l >> 4);
  Frag<T> f;
  if constexpr (sizeof(T) == 2) {
    f.v = *reinterpret_cast<const bf16x8*>(p);
  } else {
    f.lo = *reinterpret_cast<const f32x4*>(p);
    f.hi = *reinterpret_cast<const f32x4*>(p + 4);
  }
  return f;
}

// acc (16x16 fp32) += A(16x32) * B(32x16)
__device__ __forceinline__ void mma(f32x4& acc, const Frag<bf16>& a, const Frag<bf16>& b) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.v, b.v, acc, 0, 0, 0);
}
__device__ __forceinline__ void mma(f32x4& acc, const Frag<float>& a, const Frag<float>& b) {
  // step e feeds k = 8*(l/16) + e from every lane group: the 8 steps cover the 32-deep slice.
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.lo[0], b.lo[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.lo[1], b.lo[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.lo[2], b.lo[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.lo[3], b.lo[3], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.hi[0], b.hi[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.hi[1], b.hi[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.hi[2], b.hi[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.hi[3], b.hi[3], acc, 0, 0, 0);
}

// fp32 16x16x16 product from LDS with arbitrary strides (used by the triangular
// solve): acc += A[16x16] * B[16x16], A row-major (lda), B row-major (ldb).
// Step q feeds k = 4*(l/16) + q, so A is read as one 16-byte row piece.
__device__ __forceinline__ void mma16_f32_lds(f32x4& acc, const float* A, int lda, const float* B, int ldb) {
  const int l = lane_id();
  const int g = l >> 4, c = l & 15;
  const f32x4 a = *reinterpret_cast<const f32x4*>(A + c * lda + 4 * g);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[q], B[(4 * g + q) * ldb + c], acc, 0, 0, 0);
  }
}

// Same product with the B operand taken from a C-layout accumulator tile held
// in registers (lane holds B[4*(l/16) + q][l%16] in b[q]).
__device__ __forceinline__ void mma16_f32_lds_reg(f32x4& acc, const float* A, int lda, const f32x4& b) {
  const int l = lane_id();
  const int g = l >> 4, c = l & 15;
  const f32x4 a = *reinterpret_cast<const f32x4*>(A + c * lda + 4 * g);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[q], b[q], acc, 0, 0, 0);
  }
}

// ---------------------------------------------------------------------------
// vector memory helpers
// ---------------------------------------------------------------------------
template <typename T> struct Vec8;   // 8 elements = 16 bytes (bf16) or 32 bytes (fp32)
template <> struct Vec8<bf16> { bf16x8 v; };
template <> struct Vec8<float> { f32x4 lo, hi; };

template <typename T>
__device__ __forceinline__ Vec8<T> ld8(const T* p) {
  Vec8<T> r;
  if constexpr (sizeof(T) == 2) {
    r.v = *reinterpret_cast<const bf16x8*>(p);
  } else {
    r.lo = *reinterpret_cast<const f32x4*>(p);
    r.hi = *reinterpret_cast<const f32x4*>(p + 4);
  }
  return r;
}
template <typename T>
__device__ __forceinline__ void st8(T* p, const Vec8<T>& x) {
  if constexpr (sizeof(T) == 2) {
    *reinterpret_cast<bf16x8*>(p) = x.v;
  } else {
    *reinterpret_cast<f32x4*>(p) = x.lo;
    *reinterpret_cast<f32x4*>(p + 4) = x.hi;
  }
}
template <typename T> __device__ __forceinline__ float vget(const Vec8<T>& x, int e);
template <> __device__ __forceinline__ float vget<bf16>(const Vec8<bf16>& x, int e) { return (float)x.v[e]; }
template <> __device__ __forceinline__ float vget<float>(const Vec8<float>& x, int e) { return e < 4 ? x.lo[e] : x.hi[e - 4]; }
template <typename T> __device__ __forceinline__ void vset(Vec8<T>& x, int e, float val);
template <> __device__ __forceinline__ void vset<bf16>(Vec8<bf16>& x, int e, float val) { x.v[e] = (bf16)val; }
template <> __device__ __forceinline__ void vset<float>(Vec8<float>& x, int e, float val) {
  if (e < 4) x.lo[e] = val; else x.hi[e - 4] = val;
}
template <typename T>
__device__ __forceinline__ Vec8<T> vzero() {
  Vec8<T> r;
#pragma unroll
  for (int e = 0; e < 8; ++e) vset<T>(r, e, 0.0f);
  return r;
}

// 4 consecutive storage elements from 4 floats (one C-layout column piece).
template <typename T>
__device__ __forceinline__ void st4(T* p, float a, float b, float c, float d) {
  if constexpr (sizeof(T) == 2) {
    bf16x4 v = {(bf16)a, (bf16)b, (bf16)c, (bf16)d};
    *reinterpret_cast<bf16x4*>(p) = v;
  } else {
    f32x4 v = {a, b, c, d};
    *reinterpret_cast<f32x4*>(p) = v;
  }
}
template <typename T>
__device__ __forceinline__ f32x4 ld4(const T* p) {
  if constexpr (sizeof(T) == 2) {
    const bf16x4 v = *reinterpret_cast<const bf16x4*>(p);
    f32x4 r = {(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
    return r;
  } else {
    return *reinterpret_cast<const f32x4*>(p);
  }
}

// Load 8 consecutive q/k input elements (fp32, bf16 or fp8 e4m3 times a scale) as floats.
template <typename TK>
__device__ __forceinline__ void load8_in(const TK* p, float scale, float out[8]) {
  if constexpr (sizeof(TK) == 1) {
    const uint2 raw = *reinterpret_cast<const uint2*>(p);
    fp8x4_to_f32(raw.x, out);
    fp8x4_to_f32(raw.y, out + 4);
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] *= scale;
  } else {
    const Vec8<TK> x = ld8<TK>(p);
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = vget<TK>(x, e);
  }
}

// Calls f(ld) with ld(off) reading entry off of an initial state that is fp32 or bf16 (dt 0 / 1),
// or returning 0 without one: the dtype branch sits outside the caller's loops, so that all of
// its loads go out together (a per-element branch waits for each load before the next).
template <typename F>
__device__ __forceinline__ void with_state_loader(const void* h0, int dt, F&& f) {
  if (h0 == nullptr) {
    f([](int64_t) { return 0.f; });
  } else if (dt == 0) {
    const float* p = reinterpret_cast<const float*>(h0);
    f([p](int64_t off) { return p[off]; });
  } else {
    const bf16* p = reinterpret_cast<const bf16*>(h0);
    f([p](int64_t off) { return (float)p[off]; });
  }
}

// Load one scalar of a runtime-typed per-token array (g, beta): 0 = fp32, 1 = bf16.
__device__ __forceinline__ float ld_scalar(const void* p, int64_t i, int dt) {
  return dt == 0 ? reinterpret_cast<const float*>(p)[i] : (float)reinterpret_cast<const bf16*>(p)[i];
}

// ---------------------------------------------------------------------------
// swizzled row-major bf16 tiles [rows][NC] read transposed
// ---------------------------------------------------------------------------
// 16-byte chunk c of row r sits at chunk position c ^ swz(r).  LDS serves 256
// bytes per clock (64 banks of 4 bytes).  For NC >= 128 (rows of 256 bytes or
// more) only the position mod 16 decides a 16-byte piece's bank group, and
// swz(r) = 2 (r mod 8) + (r / 8 mod 2) gives the 8 rows x 2 chunks of a
// transposed read (ds_read_b64_tr_b16, 32 lanes of 8 bytes) 16 distinct
// positions; for NC = 64 (two rows per 256-byte bank row) a permutation of r / 2
// does the same within the row's 8 chunks.
template <int NC>
__device__ __forceinline__ int swz_off(int r, int c8) {
  static_assert(NC == 64 || NC % 128 == 0, "swizzled tiles are 64 or a multiple of 128 columns wide");
  const int s = NC >= 128 ? ((r & 7) << 1) | ((r >> 3) & 1) : (((r >> 1) & 3) << 1) | ((r >> 3) & 1);
  return r * NC + ((c8 ^ s) << 3);
}

typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;
typedef __attribute__((address_space(3))) const void lds_cvoid_t;

// ds_read_b64_tr_b16 of the 8 bytes at p (a pointer into this workgroup's LDS)
__device__ __forceinline__ s16x4_t lds_read_tr16(const void* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_s16x4_t*)(uintptr_t)(uint32_t)(uintptr_t)(lds_cvoid_t*)p);
}

// Transposed MFMA fragment of a swizzled tile t [rows][NC]: lane (l % 16 = j, l / 16 = lg) gets
// t[32 ks + 4 lg + e][c0 + j] and t[32 ks + 16 + 4 lg + e][c0 + j], e = 0..3 -- as an operand its
// M / N index is the column c0 + j and its K index the row, in the accumulator order (rows 4 lg ..
// and 16 + 4 lg .. of the 32-deep step).  Within 16 lanes, lane i reads 4 columns of one row and
// lane j receives element j % 4 of lane 4e + j / 4's read as its element e.
template <int NC>
__device__ __forceinline__ Frag<bf16> tr_frag(const bf16* t, int ks, int c0) {
  const int l = lane_id();
  const int lg = l >> 4, i = l & 15;
  const int col = c0 + 4 * (i & 3);
  const int r0 = 32 * ks + 4 * lg + (i >> 2);
  const s16x4_t a = lds_read_tr16(t + swz_off<NC>(r0, col >> 3) + (col & 7));
  const s16x4_t b = lds_read_tr16(t + swz_off<NC>(r0 + 16, col >> 3) + (col & 7));
  Frag<bf16> f;
  f.v = __builtin_bit_cast(bf16x8, __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7));
  return f;
}

// ---------------------------------------------------------------------------
// sequence / chunk addressing
// ---------------------------------------------------------------------------
// Chunks of all sequences are numbered 0..NC-1 in order (sequence-major).
// Fixed-length batches: sequence n covers tokens [n*T, n*T + T).
// Varlen: sequence n covers [cu[n], cu[n+1]) and chunk_off[n] is the index
// of its first chunk (chunk_off has N+1 entries; chunk_off[N] = NC).
struct ChunkLoc {
  int64_t bos;     // first token of the sequence (flattened B*T axis)
  int64_t t0;      // first token of the chunk
  int n;           // sequence index
  int nv;          // valid rows in this chunk (1..64)
  bool ok;
};

__device__ __forceinline__ ChunkLoc locate_chunk(int64_t c, const int64_t* cu, const int32_t* chunk_off,
                                                 int N, int64_t T) {
  ChunkLoc L;
  L.ok = false;
  if (cu == nullptr) {
    const int64_t nt = (T + C - 1) / C;
    if (c >= nt * N) return L;
    L.n = (int)(c / nt);
    const int64_t it = c % nt;
    L.bos = (int64_t)L.n * T;
    L.t0 = L.bos + it * C;
    L.nv = (int)min((int64_t)C, T - it * C);
    L.ok = true;
    return L;
  }
  if (c >= chunk_off[N]) return L;
  int lo = 0, hi = N - 1;              // last n with chunk_off[n] <= c
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (chunk_off[mid] <= c) lo = mid; else hi = mid - 1;
  }
  L.n = lo;
  L.bos = cu[lo];
  const int64_t it = c - chunk_off[lo];
  L.t0 = L.bos + it * C;
  L.nv = (int)min((int64_t)C, cu[lo + 1] - L.t0);
  L.ok = true;
  return L;
}

}  // namespace kgdn
