// Device helpers shared by the gfx950 attention kernels.
//
// MFMA lane layouts used throughout (checked on gfx950 hardware):
//   v_mfma_f32_32x32x16_{f16,bf16}: A[i][k] sits in lane i + 32*(k/8), element
//   k%8; B[k][j] in lane j + 32*(k/8), element k%8; C[i][j] in lane
//   j + 32*((i/4)%2), element (i/8)*4 + i%4.
// Every kernel computes S^T = K Q^T so that one lane owns one query row: the
// 16 scores of a 32x32 C tile in a lane all belong to query (lane % 32), half
// of the tile's keys sit in the lane, the other half in lane ^ 32. Row max and
// row sum therefore need one cross-half exchange (v_permlane32_swap) per tile
// instead of a butterfly over 32 lanes. The key axis is the contraction axis
// of P.V, so the C registers of S^T convert straight into the B operand of
// O^T += V^T P^T under a fixed permutation of the keys, applied identically
// to the rows of V^T read from LDS.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cie {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;

// Element traits: 0 = fp16, 1 = bf16 (the CIE_DTYPE_* codes).
template <int DTYPE> struct Elt;

template <> struct Elt<0> {
  static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  // Round-to-nearest-even conversion of two floats, packed low|high.
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    _Float16 a = (_Float16)lo, b = (_Float16)hi;
    return (uint32_t)__builtin_bit_cast(uint16_t, a) |
           ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
  }
};

template <> struct Elt<1> {
  static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    __bf16 a = (__bf16)lo, b = (__bf16)hi;
    return (uint32_t)__builtin_bit_cast(uint16_t, a) |
           ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
  }
};

// Reductions over the two lanes (l, l ^ 32) that share a query row.
__device__ __forceinline__ float xhalf_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xhalf_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Online-softmax weight of a partial whose running max is m against the new
// max M: 0 for an empty partial (m = -inf), exp2(m - M) otherwise.
__device__ __forceinline__ float rescale_weight(float m, float M) {
  return m == -INFINITY ? 0.f : exp2_fast(m - M);
}

// Unsigned division by a runtime constant: q = (umulhi(n, mul) + n) >> shift
// with shift = ceil(log2 d) and mul = floor(2^32 (2^shift - d) / d) + 1
// (Granlund & Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, section 4). Exact for 0 <= n < 2^31.
struct FastDiv {
  uint32_t d, mul, shift;
};

__host__ inline FastDiv make_fastdiv(uint32_t d) {
  uint32_t s = 0;
  while ((1ull << s) < d) ++s;
  uint64_t m = ((1ull << 32) * ((1ull << s) - d)) / d + 1;
  return FastDiv{d, (uint32_t)m, s};
}

__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) {
  return (__umulhi(n, f.mul) + n) >> f.shift;
}

// 16-byte global load that yields zeros when !ok (no memory access then).
// Used outside the streaming loops; the loops use load16_clamped.
__device__ __forceinline__ u32x4 load16(const uint16_t* p, bool ok) {
  u32x4 r = {0u, 0u, 0u, 0u};
  if (ok) r = *reinterpret_cast<const u32x4*>(p);
  return r;
}

// Unconditional 16-byte load from an address the caller has already clamped
// into the tensor. No branch, so the compiler keeps the loads of a whole tile
// in flight together and waits only where the data is consumed.
__device__ __forceinline__ u32x4 load16_clamped(const uint16_t* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

// Same, marked non-temporal: for data read exactly once (the paged KV pool).
__device__ __forceinline__ u32x4 load16_stream(const uint16_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

__device__ __forceinline__ u32x4 zero_unless(u32x4 v, bool ok) {
  return u32x4{ok ? v[0] : 0u, ok ? v[1] : 0u, ok ? v[2] : 0u, ok ? v[3] : 0u};
}

// Transpose helpers for 16-bit data held two per dword: from four rows
// r0..r3 (dword w covers columns 2w, 2w+1) build the 4 keys of column 2w
// (even) or 2w+1 (odd) as an 8-byte [r0 r1 r2 r3] pair of dwords.
__device__ __forceinline__ u32x2 col4_even(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  return u32x2{(a & 0xffffu) | (b << 16), (c & 0xffffu) | (d << 16)};
}
__device__ __forceinline__ u32x2 col4_odd(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  return u32x2{(a >> 16) | (b & 0xffff0000u), (c >> 16) | (d & 0xffff0000u)};
}

}  // namespace cie
