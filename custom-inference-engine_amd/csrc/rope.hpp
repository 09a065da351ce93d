// Rotary position embedding on 16-byte chunks, shared by the standalone rope
// kernel and the kernels that fuse it (K in the paged KV append, Q in the
// query loads of prefill and paged attention).
//
// Restates apply_rotary_ref (kernels/ref/rope_apply_ref.py:46-53): with
// x1 = x[:D/2], x2 = x[D/2:] and c = cos[pos], s = sin[pos] read from fp32
// tables of shape (rows, D/2) (kernels/ref/rope_apply_ref.py:6-19),
//   rot1 = x1*c - x2*s,   rot2 = x1*s + x2*c,
// evaluated the way torch evaluates that expression for fp16/bf16 x and
// fp32 tables: x widened exactly, each product rounded to fp32, the
// difference / sum rounded to fp32, then the result rounded to x's type
// (nearest even). A fused multiply-add would skip a product rounding, so
// contraction is off in rope8.
#pragma once

#include "common.hpp"

namespace cie {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));

template <int DTYPE> __device__ __forceinline__ f32x8 widen8(u32x4 v);
template <> __device__ __forceinline__ f32x8 widen8<0>(u32x4 v) {
  return __builtin_convertvector(__builtin_bit_cast(f16x8, v), f32x8);
}
template <> __device__ __forceinline__ f32x8 widen8<1>(u32x4 v) {
  f32x8 r;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    r[2 * e] = __uint_as_float(v[e] << 16);
    r[2 * e + 1] = __uint_as_float(v[e] & 0xffff0000u);
  }
  return r;
}

template <int DTYPE> __device__ __forceinline__ u32x4 narrow8(f32x8 f) {
  return u32x4{Elt<DTYPE>::pack2(f[0], f[1]), Elt<DTYPE>::pack2(f[2], f[3]), Elt<DTYPE>::pack2(f[4], f[5]),
               Elt<DTYPE>::pack2(f[6], f[7])};
}

// Eight consecutive table entries (16-byte aligned: rows of D/2 >= 8 floats,
// chunk offsets multiples of 8).
__device__ __forceinline__ f32x8 tab8(const float* t) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(t);
  const f32x4 b = *reinterpret_cast<const f32x4*>(t + 4);
  return f32x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// lo = x[j .. j+8), hi = x[D/2 + j .. D/2 + j+8); c, s = cos/sin[pos][j .. j+8).
template <int DTYPE>
__device__ __forceinline__ void rope8(u32x4& lo, u32x4& hi, f32x8 c, f32x8 s) {
#pragma clang fp contract(off)
  const f32x8 x1 = widen8<DTYPE>(lo), x2 = widen8<DTYPE>(hi);
  const f32x8 a = x1 * c, b = x2 * s, e = x1 * s, f = x2 * c;
  lo = narrow8<DTYPE>(a - b);
  hi = narrow8<DTYPE>(e + f);
}

// Rotates the query row a lane holds in the MFMA B-operand layout
// (q[16 kk + 8 hl .. +8] in register kk, hl = lane / 32) at position pos.
// For D >= 32 the partner of register kk < D/32 is register kk + D/32 of the
// same lane; for D = 16 it is the same register of lane ^ 32 (every lane of
// the wave must call this then). An out-of-range position makes the row NaN
// when the lane's row is live; the table reads stay in row 0 then.
template <int DTYPE, int D>
__device__ __forceinline__ void rope_q_lane(u32x4 (&qf)[D / 16], const float* cos, const float* sin, int rows,
                                            int pos, bool live, int hl) {
  constexpr int KK = D / 16;
  const bool ok = pos >= 0 && pos < rows;
  const int64_t row = ok ? (int64_t)pos * (D / 2) : 0;
  if constexpr (KK == 1) {
    u32x4 other;
#pragma unroll
    for (int e = 0; e < 4; ++e) other[e] = (uint32_t)__shfl_xor((int)qf[0][e], 32);
    u32x4 lo = hl ? other : qf[0], hi = hl ? qf[0] : other;
    rope8<DTYPE>(lo, hi, tab8(cos + row), tab8(sin + row));
    qf[0] = hl ? hi : lo;
  } else {
#pragma unroll
    for (int kk = 0; kk < KK / 2; ++kk) {
      const int j = 16 * kk + 8 * hl;
      rope8<DTYPE>(qf[kk], qf[kk + KK / 2], tab8(cos + row + j), tab8(sin + row + j));
    }
  }
  if (live && !ok) {
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) qf[kk] = u32x4{0x7fff7fffu, 0x7fff7fffu, 0x7fff7fffu, 0x7fff7fffu};
  }
}

}  // namespace cie
