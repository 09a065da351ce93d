// Rotary position embedding on 16-byte chunks, shared by the standalone rope
// kernel and the kernels that fuse it (K in the paged KV append, Q in the
// query loads of prefill and paged attention).
//
// Restates apply_rotary_ref (kernels/ref/rope_apply_ref.py:46-53): with
// x1 = x[:D/2], x2 = x[D/2:] and c = cos[pos], s = sin[pos] read from tables
// of shape (rows, D/2) (kernels/ref/rope_apply_ref.py:6-19),
//   rot1 = x1*c - x2*s,   rot2 = x1*s + x2*c,
// evaluated the way torch evaluates that expression for fp16/bf16 x:
//   * fp32 tables (as built), or 16-bit tables of the other 16-bit type
//     (torch promotes fp16 x bf16 to fp32): x and the table widened exactly,
//     each product rounded to fp32, the difference / sum rounded to fp32,
//     the result rounded to x's type (nearest even);
//   * tables of x's own type (what the reference engine's
//     cast_non_quantized_params leaves in RotaryEmbedding, engine/runtime.py:
//     22-37): every product and the difference / sum rounded to x's type.
//     Those products are exact in fp32 (11 x 11 or 8 x 8 significand bits),
//     so rounding the fp32 product gives torch's half / bfloat16 product, and
//     the difference of two 16-bit values rounded from fp32 is torch's too.
// A fused multiply-add would skip a product rounding, so contraction is off.
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

// Eight consecutive fp32 table entries (16-byte aligned: rows of D/2 >= 8
// floats, chunk offsets multiples of 8).
__device__ __forceinline__ f32x8 tab8(const float* t) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(t);
  const f32x4 b = *reinterpret_cast<const f32x4*>(t + 4);
  return f32x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// lo = x[j .. j+8), hi = x[D/2 + j .. D/2 + j+8); c, s = cos/sin[pos][j .. j+8)
// widened to fp32. fp32 arithmetic, one rounding to x's type at the end.
template <int DTYPE>
__device__ __forceinline__ void rope8(u32x4& lo, u32x4& hi, f32x8 c, f32x8 s) {
#pragma clang fp contract(off)
  const f32x8 x1 = widen8<DTYPE>(lo), x2 = widen8<DTYPE>(hi);
  const f32x8 a = x1 * c, b = x2 * s, e = x1 * s, f = x2 * c;
  lo = narrow8<DTYPE>(a - b);
  hi = narrow8<DTYPE>(e + f);
}

// The same with every product and the difference / sum rounded to x's type
// (tables of x's own type).
template <int DTYPE>
__device__ __forceinline__ void rope8_narrow(u32x4& lo, u32x4& hi, f32x8 c, f32x8 s) {
#pragma clang fp contract(off)
  const f32x8 x1 = widen8<DTYPE>(lo), x2 = widen8<DTYPE>(hi);
  const f32x8 a = widen8<DTYPE>(narrow8<DTYPE>(x1 * c)), b = widen8<DTYPE>(narrow8<DTYPE>(x2 * s));
  const f32x8 e = widen8<DTYPE>(narrow8<DTYPE>(x1 * s)), f = widen8<DTYPE>(narrow8<DTYPE>(x2 * c));
  lo = narrow8<DTYPE>(a - b);
  hi = narrow8<DTYPE>(e + f);
}

// Raw bits of eight cos and eight sin entries: fp32 tables fill all four
// vectors, 16-bit tables c0 / s0 only. Loaded apart from the rotation so a
// caller can keep several chunks' loads in flight.
struct RopeChunk {
  u32x4 c0, c1, s0, s1;
};

// Entries [e, e + 8) of both tables (e = pos * D/2 + j, j a multiple of 8).
__device__ __forceinline__ RopeChunk rope_load(const RopeTables& t, int64_t e) {
  RopeChunk r;
  if (t.dt == kTabF32) {
    const u32x4* c = reinterpret_cast<const u32x4*>(static_cast<const float*>(t.cos) + e);
    const u32x4* s = reinterpret_cast<const u32x4*>(static_cast<const float*>(t.sin) + e);
    r.c0 = c[0], r.c1 = c[1], r.s0 = s[0], r.s1 = s[1];
  } else {
    r.c0 = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(t.cos) + e);
    r.s0 = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(t.sin) + e);
    r.c1 = r.s1 = u32x4{0u, 0u, 0u, 0u};
  }
  return r;
}

__device__ __forceinline__ f32x8 f32x8_of(u32x4 a, u32x4 b) {
  return f32x8{__uint_as_float(a[0]), __uint_as_float(a[1]), __uint_as_float(a[2]), __uint_as_float(a[3]),
               __uint_as_float(b[0]), __uint_as_float(b[1]), __uint_as_float(b[2]), __uint_as_float(b[3])};
}

// Rotates one chunk pair with table entries r of element type dt, with the
// arithmetic torch uses for x's type against that table type.
template <int DTYPE>
__device__ __forceinline__ void rope_apply8(u32x4& lo, u32x4& hi, const RopeChunk& r, int dt) {
  if (dt == kTabF32) rope8<DTYPE>(lo, hi, f32x8_of(r.c0, r.c1), f32x8_of(r.s0, r.s1));
  else if (dt == DTYPE) rope8_narrow<DTYPE>(lo, hi, widen8<DTYPE>(r.c0), widen8<DTYPE>(r.s0));
  else rope8<DTYPE>(lo, hi, widen8<1 - DTYPE>(r.c0), widen8<1 - DTYPE>(r.s0));
}

// Rotates the query row a lane holds in the MFMA B-operand layout
// (q[16 kk + 8 hl .. +8] in register kk, hl = lane / 32) at position pos.
// For D >= 32 the partner of register kk < D/32 is register kk + D/32 of the
// same lane; for D = 16 it is the same register of lane ^ 32 (every lane of
// the wave must call this then). An out-of-range position makes the row NaN
// when the lane's row is live; the table reads stay in row 0 then.
template <int DTYPE, int D>
__device__ __forceinline__ void rope_q_lane(u32x4 (&qf)[D / 16], const RopeTables& t, int pos, bool live, int hl) {
  constexpr int KK = D / 16;
  const bool ok = pos >= 0 && pos < t.rows;
  const int64_t row = ok ? (int64_t)pos * (D / 2) : 0;
  if constexpr (KK == 1) {
    u32x4 other;
#pragma unroll
    for (int e = 0; e < 4; ++e) other[e] = (uint32_t)__shfl_xor((int)qf[0][e], 32);
    u32x4 lo = hl ? other : qf[0], hi = hl ? qf[0] : other;
    rope_apply8<DTYPE>(lo, hi, rope_load(t, row), t.dt);
    qf[0] = hl ? hi : lo;
  } else {
    RopeChunk r[KK / 2];
#pragma unroll
    for (int kk = 0; kk < KK / 2; ++kk) r[kk] = rope_load(t, row + 16 * kk + 8 * hl);
#pragma unroll
    for (int kk = 0; kk < KK / 2; ++kk) rope_apply8<DTYPE>(qf[kk], qf[kk + KK / 2], r[kk], t.dt);
  }
  if (live && !ok) {
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) qf[kk] = u32x4{0x7fff7fffu, 0x7fff7fffu, 0x7fff7fffu, 0x7fff7fffu};
  }
}

}  // namespace cie
