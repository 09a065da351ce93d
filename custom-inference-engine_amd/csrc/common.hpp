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
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;

// Element traits: 0 = fp16, 1 = bf16 (the CIE_DTYPE_* codes).
template <int DTYPE> struct Elt;

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

template <> struct Elt<0> {
  static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  // Round-to-nearest-even conversion of two floats, packed low|high (v_cvt_pk_f16_f32).
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, f16x2));
  }
  // acc + lo + hi of a packed pair (v_dot2c_f32_f16 against ones).
  static __device__ __forceinline__ float sum2(uint32_t pk, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, pk), f16x2{(_Float16)1.f, (_Float16)1.f}, acc, false);
  }
  // acc + a.lo * b.lo + a.hi * b.hi, fp32 accumulation of exact products.
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), acc, false);
  }
  // 16x16x32 MFMA: A[i][k] in lane i + 16 (k / 8), B[k][j] in lane j + 16 (k / 8),
  // C[i][j] in lane j + 16 (i / 4), element i % 4.
  static __device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  }
  // 4x4x4, 16 blocks: with A all ones, every element of lane l's result is
  // c + the sum of lane l's own four B values (checked on gfx950; a NaN in
  // one lane stays in that lane).
  static __device__ __forceinline__ f32x4 mfma4(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
  }
};

template <> struct Elt<1> {
  static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
  }
  static __device__ __forceinline__ float sum2(uint32_t pk, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pk), bf16x2{(__bf16)1.f, (__bf16)1.f}, acc,
                                           false);
  }
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), acc, false);
  }
  static __device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mfma4(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b), c, 0, 0,
                                                  0);
  }
};

// NaN-propagating maximum (llvm.maximum): selects to v_maximum3_f32 with no
// quieting of the operands, which fmaxf needs in IEEE mode (a v_max_f32 x, x
// per operand). NaN scores (from NaN inputs) propagate like the reference's
// softmax.
__device__ __forceinline__ float maxf(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float max3f(float a, float b, float c) { return maxf(maxf(a, b), c); }

// Reductions over the two lanes (l, l ^ 32) that share a query row.
__device__ __forceinline__ float xhalf_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return max3f(__uint_as_float(r[0]), __uint_as_float(r[1]), x);
}
__device__ __forceinline__ float xhalf_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Balanced reductions over the 16 accumulator values of a lane (the compiler
// does not reassociate a linear fmaxf / fadd chain).
__device__ __forceinline__ float max16(const f32x16& v) {
  const float a0 = max3f(v[0], v[1], v[2]), a1 = max3f(v[3], v[4], v[5]), a2 = max3f(v[6], v[7], v[8]);
  const float a3 = max3f(v[9], v[10], v[11]), a4 = max3f(v[12], v[13], v[14]);
  return max3f(max3f(a0, a1, a2), max3f(a3, a4, v[15]), a0);
}
__device__ __forceinline__ float sum16(const f32x16& v) {
  float a0 = (v[0] + v[1]) + (v[2] + v[3]);
  float a1 = (v[4] + v[5]) + (v[6] + v[7]);
  float a2 = (v[8] + v[9]) + (v[10] + v[11]);
  float a3 = (v[12] + v[13]) + (v[14] + v[15]);
  return (a0 + a1) + (a2 + a3);
}

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

// ---- LDS DMA and LDS transpose reads (gfx950) ------------------------------
//
// global_load_lds (16 bytes): lane l's 16 bytes land at lds_base + 16 * l,
// lds_base wave-uniform (passed in M0). The load is issued from inline
// assembly so that the compiler's wait-count pass does not treat it as an LDS
// store aliasing every later LDS read (it would drain the whole queue with
// vmcnt(0) before each one). Every consumer therefore waits explicitly with
// vm_wait<N>(): N = number of vector-memory instructions issued after the
// ones being waited for (they complete in order). M0 is written right before
// each load; the kernels use no other M0-dependent instruction.
//
// ds_read_b64_tr_b16: within each 16-lane group, lane r supplies the address
// of a row of four 16-bit elements M[r][0..3]; lane i receives
// M[4j + i/4][i%4] for j = 0..3. With lane r pointing at
// X[k0 + r/4][d0 + 4*(r%4)] of a row-major X[key][d], lane i receives
// X[k0 .. k0+3][d0 + i]: four consecutive keys of one column, i.e. the
// key-contiguous MFMA operand of X^T, read from row-major X.

typedef __attribute__((address_space(3))) void lds_void;

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void* gptr, void* lds_wave_base) {
  // lds_wave_base is uniform across the wave by contract; readfirstlane puts it in an SGPR
  const uint32_t lds_addr = __builtin_amdgcn_readfirstlane((uint32_t)(size_t)(lds_void*)lds_wave_base);
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gptr), "s"(lds_addr) : "memory", "m0");
}
// LDS byte address of a pointer into __shared__ memory, as a wave-uniform
// value. Take it in uniform control flow: the generic-to-LDS cast checks for
// null, which only the scalar unit can do.
__device__ __forceinline__ uint32_t lds_addr_of(void* lds_ptr) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(size_t)(lds_void*)lds_ptr);
}
// Same, with the wave-uniform LDS byte address given directly.
__device__ __forceinline__ void dma16_at(const void* gptr, uint32_t lds_addr) {
  lds_addr = __builtin_amdgcn_readfirstlane(lds_addr);
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gptr), "s"(lds_addr) : "memory", "m0");
}
// Scalar-base form: lane l loads sbase + voff (voff a 32-bit byte offset),
// no per-lane 64-bit address arithmetic. sbase must be wave-uniform.
__device__ __forceinline__ const void* uniform_ptr(const void* p) {
  const uint64_t a = (uint64_t)(size_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  return (const void*)(size_t)(((uint64_t)hi << 32) | lo);
}
// Non-temporal forms, for data a kernel streams exactly once (the paged KV
// pool, INT8 weights): the hint keeps those bytes from displacing the small
// tensors every workgroup rereads (block tables, lengths, activations) from
// L2 and the Infinity Cache.
__device__ __forceinline__ void dma16_sv_nt(const void* sbase, uint32_t voff, uint32_t lds_addr) {
  lds_addr = __builtin_amdgcn_readfirstlane(lds_addr);
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(voff), "s"(sbase), "s"(lds_addr)
               : "memory", "m0");
}
__device__ __forceinline__ void dma16_at_nt(const void* gptr, uint32_t lds_addr) {
  lds_addr = __builtin_amdgcn_readfirstlane(lds_addr);
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(gptr), "s"(lds_addr) : "memory", "m0");
}
__device__ __forceinline__ void dma16_sv(const void* sbase, uint32_t voff, uint32_t lds_addr) {
  lds_addr = __builtin_amdgcn_readfirstlane(lds_addr);
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds_addr)
               : "memory", "m0");
}
// 4-byte variant: lane l's dword lands at LDS byte address lds_addr + 4 * l.
__device__ __forceinline__ void dma4(const void* gptr, uint32_t lds_addr) {
  lds_addr = __builtin_amdgcn_readfirstlane(lds_addr);
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(gptr), "s"(lds_addr) : "memory", "m0");
}
#pragma clang diagnostic pop

__device__ __forceinline__ u32x2 lds_read_tr16(const void* lds_ptr) {
  const s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)lds_ptr);
  return __builtin_bit_cast(u32x2, r);
}

// Explicit waits are inline assembly so no compiler pass can relax them.
template <int N>
__device__ __forceinline__ void vm_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ void lgkm_wait0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Bring every 64-byte line of a kernel's argument block (BYTES of it, at
// most 512) into the scalar cache with one batch of scalar loads and one
// wait. The compiler loads the arguments where each branch first needs them:
// the paged kernel made three dependent argument round trips before its
// first memory request, each a scalar-cache miss on a CU's first wave. The
// loaded dwords are discarded; touches at most 64 bytes apart, the last at
// BYTES - 4, reach every line whatever the block's alignment.
template <int BYTES>
__device__ __forceinline__ void warm_kernargs() {
  static_assert(BYTES >= 4 && BYTES <= 512 && BYTES % 4 == 0, "argument block size");
  constexpr int L = BYTES - 4;
  const auto ka = __builtin_amdgcn_kernarg_segment_ptr();
  uint32_t d;  // every load writes it; only the wait below orders them
  asm volatile(
      "s_load_dword %0, %1, %2\n\t"
      "s_load_dword %0, %1, %3\n\t"
      "s_load_dword %0, %1, %4\n\t"
      "s_load_dword %0, %1, %5\n\t"
      "s_load_dword %0, %1, %6\n\t"
      "s_load_dword %0, %1, %7\n\t"
      "s_load_dword %0, %1, %8\n\t"
      "s_load_dword %0, %1, %9\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&s"(d)
      : "s"(ka), "n"(0), "n"(64 < L ? 64 : L), "n"(128 < L ? 128 : L), "n"(192 < L ? 192 : L),
        "n"(256 < L ? 256 : L), "n"(320 < L ? 320 : L), "n"(384 < L ? 384 : L), "n"(448 < L ? 448 : L)
      : "memory");
}

// XOR swizzle of the 16-byte chunks of row r in an LDS tile with S chunks per
// row. LDS is 64 banks x 4 bytes (256-byte bank rows), so a row of S chunks
// covers S/16 of a bank row and rows r, r + 16/S, ... share bank columns. Two
// access patterns must be conflict-free:
//   ds_read_b128 of one chunk from 16 consecutive rows, and
//   ds_read_b64_tr_b16 of 4 consecutive chunks from 4 consecutive rows,
// so rows sharing bank columns get distinct swizzles (bijective within each
// bank-sharing class) and the swizzles of consecutive such rows differ in the
// high bits (bit reversal), which moves a 4-chunk run to another bank quarter.
__device__ __forceinline__ int bitrev3(int x) { return ((x & 1) << 2) | (x & 2) | ((x >> 2) & 1); }
__device__ __forceinline__ int bitrev4(int x) {
  return ((x & 1) << 3) | ((x & 2) << 1) | ((x >> 1) & 2) | ((x >> 3) & 1);
}
template <int S>
__device__ __forceinline__ int chunk_swizzle(int r) {
  if constexpr (S >= 16) return bitrev4(r & 15);
  else if constexpr (S == 8) return bitrev3((r >> 1) & 7);
  else if constexpr (S == 4) return (r >> 2) & 3;
  else return (r >> 3) & 1;
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

// Per-workgroup timeline stamps for benchmarks/timeline.py, which builds the
// library a second time with CIE_TIMELINE defined: thread 0 of each of the
// first kTimelineMaxWg workgroups writes kTimelineSlots values of its own
// (s_memrealtime, 100 MHz ticks, or a plain value) into a per-kernel device
// array that an extern "C" accessor of the timeline build copies out. In
// the product build every stamp compiles to nothing.
#ifdef CIE_TIMELINE
constexpr int kTimelineSlots = 8;
constexpr int kTimelineMaxWg = 16384;
#define CIE_STAMP(buf, slot)                                                                       \
  do {                                                                                             \
    if (threadIdx.x == 0 && blockIdx.x < (unsigned)kTimelineMaxWg)                                 \
      (buf)[(size_t)blockIdx.x * kTimelineSlots + (slot)] = __builtin_amdgcn_s_memrealtime();      \
  } while (0)
#define CIE_STAMP_VALUE(buf, slot, v)                                                              \
  do {                                                                                             \
    if (threadIdx.x == 0 && blockIdx.x < (unsigned)kTimelineMaxWg)                                 \
      (buf)[(size_t)blockIdx.x * kTimelineSlots + (slot)] = (unsigned long long)(v);               \
  } while (0)
// where the workgroup runs: XCC_ID in the high word, HW_ID (wave, SIMD, CU,
// shader array, shader engine) in the low word
#define CIE_STAMP_WHERE(buf, slot)                                                                 \
  CIE_STAMP_VALUE(buf, slot,                                                                       \
                  ((unsigned long long)__builtin_amdgcn_s_getreg((20) | ((4 - 1) << 11)) << 32) |  \
                      __builtin_amdgcn_s_getreg((4) | ((32 - 1) << 11)))
#else
#define CIE_STAMP(buf, slot) \
  do {                       \
  } while (0)
#define CIE_STAMP_VALUE(buf, slot, v) \
  do {                                \
  } while (0)
#define CIE_STAMP_WHERE(buf, slot) \
  do {                             \
  } while (0)
#endif

}  // namespace cie
