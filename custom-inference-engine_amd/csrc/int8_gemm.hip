// INT8-weight GEMM for gfx950: y = (x . w^T) * s[n] (+ bias[n]), x fp16/bf16
// (M, K), w int8 (N, K) with per-output-channel scales s (N,), y (M, N) in x's
// dtype. Replaces the Triton dequant-on-load kernel behind Int8Linear
// (kernels/int8_matmul.py:16-62, wrapper :65-110, caller
// engine/quant/int8_linear.py:37-41).
//
// Arithmetic. int8 values are exact in fp16 and bf16, so the weights are
// converted in registers (fp16: byte | 0x6400 is 1024 + byte, minus 1152;
// bf16: byte -> f32 -> bf16) and multiplied against x on the matrix cores
// (v_mfma_f32_32x32x16_{f16,bf16}) with fp32 accumulation: the products are
// exact, as in the reference, which up-casts both operands to fp32 before
// tl.dot (:47-53). The scale multiplies the fp32 sum once per output
// (:56-57) and the result is rounded to x's dtype; the bias is added after
// that rounding, in x's dtype, as the wrapper does (:107-109).
//
// Tiling. A workgroup of 4 waves owns 128 weight rows (32 per wave, one MFMA
// row tile) and BM = 32 * MT activation rows, and walks its K range in steps
// of 64. Each step's x tile (BM x 64, 128-byte rows) and w tile (128 x 64,
// 64-byte rows) are copied global -> LDS with direct-to-LDS loads into a
// ring of NST stages, 16-byte chunks XOR-swizzled per row so that the
// fragment reads below are bank-conflict free. The MFMA operands use a fixed
// permutation of the contraction axis: for a 32-wide k group, lane (r, h)
// (r = lane % 32, h = lane / 32) takes w[n_r][16h .. 16h+16) -- one 16-byte
// fragment read -- whose first 8 values feed MFMA 0 and last 8 MFMA 1; the
// x operand takes x[m_r][16h .. 16h+16) split the same way, so MFMA 0
// contracts k in {0..7, 16..23} and MFMA 1 k in {8..15, 24..31}.
//
// Kernels by M: up to 2 a row-streaming VALU dot kernel with the activations
// in LDS (a VALU dot kernel reading them from L2 when they do not fit), up to
// 64 a weight-streaming MFMA kernel (all one launch, no workspace; below),
// above that the tiled kernel described here.
//
// Any K. The reference masks the K tail of its last tile
// (kernels/int8_matmul.py:43-50). Here each kernel's main loop covers the
// largest prefix of K its step divides (64 for the tiled kernel, 32 for the
// streaming one, 16 for the dot kernel) and never reads past it; the
// remaining k < 64 terms of every output are added in the epilogue, in fp32
// with exact products and in ascending k, before the scale is applied.
//
// Split K. When the (n, m) tiles alone cannot occupy the GPU, the K steps
// are cut into `splits` contiguous ranges; each
// workgroup writes its fp32 partial tile to the workspace in lane order
// (16 contiguous bytes per lane, 1 KiB per wave instruction) and a second
// kernel sums the partials of every output in split order (deterministic),
// scales, rounds and adds the bias. (Folding that sum into the last
// workgroup to finish a tile needs device-coherent stores, an arrival
// atomic and coherent reloads in series; on MI355X that chain cost more than
// the second launch.)
#include <type_traits>
#include <utility>

#include "kernels.hpp"

namespace cie {

#define CIE_GV_INLINE __attribute__((always_inline))

// f(integral_constant<int, 0>), ..., f(integral_constant<int, N - 1>), in order.
template <typename F, int... I>
__device__ __forceinline__ void gv_static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void gv_static_for(F&& f) {
  gv_static_for_impl(f, std::make_integer_sequence<int, N>{});
}

typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kI8BN = 128;  // weight rows per workgroup
constexpr int kI8BK = 64;   // k per step

constexpr int kI8MaxSplits = 16;

// KW: waves per 32 weight rows. With KW = 2 (eight waves) waves w and w + 4
// take the two 32-k halves of every step for the same weight rows and are
// summed through LDS at the end, so one workgroup per CU still puts two
// waves on every SIMD.
template <int MT, int NST_, int KW = 1>
struct I8Cfg {
  static constexpr int BM = 32 * MT;
  static constexpr int NST = NST_;  // LDS ring stages
  static constexpr int NT = 256 * KW;                    // threads
  static constexpr int X_BYTES = BM * kI8BK * 2;        // x tile per stage
  static constexpr int W_BYTES = kI8BN * kI8BK;         // w tile per stage
  static constexpr int STAGE = X_BYTES + W_BYTES;
  static constexpr int XI = X_BYTES / (NT * 16);        // x copies per lane per stage
  static constexpr int WI = W_BYTES / (NT * 16);        // w copies per lane per stage
  static constexpr int PER = XI + WI;
  static constexpr int G2 = 2 / KW;                     // 32-k halves of a step per wave
  static_assert(KW == 1 || KW == 2, "one or two waves per 32 weight rows");
  static_assert(XI >= 1 && WI * KW == 2, "tile must split over the waves");
  static_assert(NST * STAGE >= 4 * MT * 16 * 64 * 4, "the k-half partials fit the ring");
  static_assert(PER * (NST - 1) < 64, "vmcnt range");
};

// 16 int8 -> two groups of 8 fp16 / bf16 (u32x4 each), exact.
template <int DTYPE> __device__ __forceinline__ void dequant16(u32x4 q, u32x4& a0, u32x4& a1);

template <> __device__ __forceinline__ void dequant16<0>(u32x4 q, u32x4& a0, u32x4& a1) {
  uint32_t o[8];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const uint32_t u = q[d] ^ 0x80808080u;  // byte b -> b + 128
    const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);  // 0x64 u1 0x64 u0
    const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);  // 0x64 u3 0x64 u2
    const f16x2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    o[2 * d] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, lo) - bias);
    o[2 * d + 1] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, hi) - bias);
  }
  a0 = u32x4{o[0], o[1], o[2], o[3]};
  a1 = u32x4{o[4], o[5], o[6], o[7]};
}

template <> __device__ __forceinline__ void dequant16<1>(u32x4 q, u32x4& a0, u32x4& a1) {
  uint32_t o[8];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const uint32_t u = q[d] ^ 0x80808080u;
    const float f0 = (float)(u & 0xffu) - 128.0f, f1 = (float)((u >> 8) & 0xffu) - 128.0f;
    const float f2 = (float)((u >> 16) & 0xffu) - 128.0f, f3 = (float)(u >> 24) - 128.0f;
    o[2 * d] = Elt<1>::pack2(f0, f1);
    o[2 * d + 1] = Elt<1>::pack2(f2, f3);
  }
  a0 = u32x4{o[0], o[1], o[2], o[3]};
  a1 = u32x4{o[4], o[5], o[6], o[7]};
}

template <int DTYPE>
__device__ __forceinline__ float elt_to_f32(uint16_t h) {
  if constexpr (DTYPE == 0) return (float)__builtin_bit_cast(_Float16, h);
  else return __uint_as_float((uint32_t)h << 16);
}

__device__ __forceinline__ float load_scale(const void* s, int n, int sdtype) {
  if (sdtype == 2) return static_cast<const float*>(s)[n];
  const uint16_t h = static_cast<const uint16_t*>(s)[n];
  return sdtype == 0 ? (float)__builtin_bit_cast(_Float16, h) : __uint_as_float((uint32_t)h << 16);
}

// y = round(acc * s) (+ bias, rounded again), for 4 consecutive outputs.
template <int DTYPE>
__device__ __forceinline__ u32x2 finish4(const float (&a)[4], const I8GemmParams& p, int n) {
  float v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int ne = min(n + e, p.N - 1);
    float t = a[e] * load_scale(p.scales, ne, p.scale_dtype);
    if (p.bias) {
      // the reference adds the bias to the rounded product, in the output dtype
      const uint32_t r = Elt<DTYPE>::pack2(t, 0.f);
      t = elt_to_f32<DTYPE>((uint16_t)r) + elt_to_f32<DTYPE>(p.bias[ne]);
    }
    v[e] = t;
  }
  return u32x2{Elt<DTYPE>::pack2(v[0], v[1]), Elt<DTYPE>::pack2(v[2], v[3])};
}

template <int DTYPE>
__device__ __forceinline__ void store4(const I8GemmParams& p, int m, int n, u32x2 pk) {
  if (m >= p.M || n >= p.N) return;
  uint16_t* dst = p.y + (int64_t)m * p.ys + n;
  if (n + 3 < p.N && (p.ys & 3) == 0) {  // 8-byte aligned (n is a multiple of 4)
    *reinterpret_cast<u32x2*>(dst) = pk;
  } else {
    const uint16_t h[4] = {(uint16_t)pk[0], (uint16_t)(pk[0] >> 16), (uint16_t)pk[1], (uint16_t)(pk[1] >> 16)};
    for (int e = 0; e < 4 && n + e < p.N; ++e) dst[e] = h[e];
  }
}

// sum over k in [k0, K) of x[m][k] * w[n][k] (products exact in fp32), k
// ascending, with m, n clamped into the tensors (rows past M / N are never
// stored). The K tail the vector main loops leave.
template <int DTYPE>
__device__ __forceinline__ float tail_dot(const I8GemmParams& p, int m, int n, int k0) {
  const uint16_t* xr = p.x + (int64_t)min(m, p.M - 1) * p.xs;
  const int8_t* wr = p.w + (int64_t)min(n, p.N - 1) * p.wsr;
  float a = 0.f;
  for (int k = k0; k < p.K; ++k) a = fmaf(elt_to_f32<DTYPE>(xr[k]), (float)wr[k], a);
  return a;
}

// vm_wait for the copies of `ahead` k steps issued after the one needed (uniform `ahead`)
template <int PER, int MAXA>
__device__ __forceinline__ void wait_steps_ahead(int ahead) {
  if constexpr (MAXA > 0) {
    if (ahead >= MAXA) {
      vm_wait<MAXA * PER>();
      return;
    }
    wait_steps_ahead<PER, MAXA - 1>(ahead);
  } else {
    vm_wait<0>();
  }
}

template <int DTYPE, int MT, int NST, int KW>
__global__ __launch_bounds__(256 * KW, KW == 1 ? 2 : 1) void int8_gemm_kernel(const I8GemmParams p) {
  using C = I8Cfg<MT, NST, KW>;
  using E = Elt<DTYPE>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  // tile order: the m tiles of one weight tile are consecutive logical ids,
  // and consecutive logical ids land on one XCD (round-robin dispatch), so a
  // weight tile read by several m tiles is shared through that XCD's L2
  const int logical = xcd_logical(blockIdx.x, p.n_tiles * p.m_tiles * p.splits, p.xcd_shift);
  const int split = logical % p.splits;
  const int rest = logical / p.splits;
  const int mt_i = rest % p.m_tiles;
  const int nt_i = rest / p.m_tiles;
  const int n0 = nt_i * kI8BN, m0 = mt_i * C::BM;
  const int ks0 = (int)((int64_t)split * p.ksteps / p.splits);
  const int ks1 = (int)((int64_t)(split + 1) * p.ksteps / p.splits);
  const int T = ks1 - ks0;

  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave 0 .. 4 KW - 1
  const int w = wv & 3, kh = KW == 1 ? 0 : wv >> 2;  // 32 weight rows w, k half kh
  const int r32 = lane & 31, hk = lane >> 5;
  const uint32_t lds0 = lds_addr_of(smem);

  // per-lane copy sources (row clamped into the tensor; rows past M / N are
  // computed but never stored)
  const uint8_t* xsrc[C::XI];
  uint32_t xdst[C::XI];
#pragma unroll
  for (int j = 0; j < C::XI; ++j) {
    const int P = (j * 4 * KW + wv) * 64 + lane;  // x chunk slot in the tile: 8 per row
    const int r = P >> 3, c = (P & 7) ^ chunk_swizzle<8>(r);
    const int m = min(m0 + r, p.M - 1);
    xsrc[j] = reinterpret_cast<const uint8_t*>(p.x + (int64_t)m * p.xs + 8 * c);
    xdst[j] = (uint32_t)((j * 4 * KW + wv) * 64 * 16);
  }
  const uint8_t* wsrc[C::WI];
  uint32_t wdst[C::WI];
#pragma unroll
  for (int j = 0; j < C::WI; ++j) {
    const int P = (j * 4 * KW + wv) * 64 + lane;  // w chunk slot: 4 per row
    const int r = P >> 2, c = (P & 3) ^ chunk_swizzle<4>(r);
    const int n = min(n0 + r, p.N - 1);
    wsrc[j] = reinterpret_cast<const uint8_t*>(p.w) + (int64_t)n * p.wsr + 16 * c;
    wdst[j] = (uint32_t)(C::X_BYTES + (j * 4 * KW + wv) * 64 * 16);
  }
  auto issue = [&](int t) {
    const uint32_t st = lds0 + (uint32_t)((t % C::NST) * C::STAGE);
    const int64_t kx = (int64_t)(ks0 + t) * kI8BK * 2;  // bytes into an x row
    const int64_t kw = (int64_t)(ks0 + t) * kI8BK;      // bytes into a w row
#pragma unroll
    for (int j = 0; j < C::XI; ++j) dma16_at(xsrc[j] + kx, st + xdst[j]);
#pragma unroll
    for (int j = 0; j < C::WI; ++j) dma16_at(wsrc[j] + kw, st + wdst[j]);
  };

  // fragment read offsets within a stage (bytes), for this wave's k halves
  // g2 = kh G2 + i of each step
  uint32_t woff[C::G2], xoff[MT][C::G2][2];
  {
    const int r = w * 32 + r32;
#pragma unroll
    for (int i = 0; i < C::G2; ++i) {
      const int g2 = kh * C::G2 + i;
      woff[i] = C::X_BYTES + r * 64 + 16 * ((2 * g2 + hk) ^ chunk_swizzle<4>(r));
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int rx = mt * 32 + r32;
#pragma unroll
      for (int i = 0; i < C::G2; ++i)
#pragma unroll
        for (int g = 0; g < 2; ++g)
          xoff[mt][i][g] = rx * 128 + 16 * ((4 * (kh * C::G2 + i) + 2 * hk + g) ^ chunk_swizzle<8>(rx));
    }
  }

  f32x16 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x16{};

  // One barrier per step: it publishes step t and, as every wave has left
  // step t-1, frees that step's stage, which is refilled at once with step
  // t + NST - 1 (NST - 1 steps in flight during the compute of step t).
  const int pro = min(C::NST - 1, T);
  for (int t = 0; t < pro; ++t) issue(t);
  for (int t = 0; t < T; ++t) {
    wait_steps_ahead<C::PER, C::NST - 2>(min(C::NST - 2, T - 1 - t));  // steps issued after step t
    __syncthreads();  // step t is in LDS for every wave; the stage of step t-1 is free
    if (t + C::NST - 1 < T) issue(t + C::NST - 1);
    const uint8_t* st = smem + (t % C::NST) * C::STAGE;
    // every fragment of the step is read first, so the LDS latency is paid
    // once per step rather than in front of each MFMA
    // (this wave's k halves g2 = kh G2 .. kh G2 + G2 - 1 of the step)
    u32x4 wq[C::G2], xb[MT][C::G2][2];
#pragma unroll
    for (int i = 0; i < C::G2; ++i) wq[i] = *reinterpret_cast<const u32x4*>(st + woff[i]);
#pragma unroll
    for (int i = 0; i < C::G2; ++i)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int g = 0; g < 2; ++g) xb[mt][i][g] = *reinterpret_cast<const u32x4*>(st + xoff[mt][i][g]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < C::G2; ++i) {
      u32x4 a0, a1;
      dequant16<DTYPE>(wq[i], a0, a1);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        acc[mt] = E::mfma(a0, xb[mt][i][0], acc[mt]);
        acc[mt] = E::mfma(a1, xb[mt][i][1], acc[mt]);
      }
    }
  }
  if constexpr (KW == 2) {
    // the k-half-1 sums join the k-half-0 ones through LDS (fixed order:
    // half 0 + half 1); the ring is free once every wave has left the loop
    __syncthreads();
    float* red = reinterpret_cast<float*>(smem);
    if (kh == 1) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int e = 0; e < 16; ++e) red[((w * MT + mt) * 16 + e) * 64 + lane] = acc[mt][e];
    }
    __syncthreads();
    if (kh == 1) return;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[mt][e] += red[((w * MT + mt) * 16 + e) * 64 + lane];
  }

  // C[i][j] of a 32x32 tile: lane j + 32 * ((i / 4) % 2), element (i / 8) * 4 + i % 4;
  // here i = weight row (n), j = activation row (m)
  const int k_main = p.ksteps * kI8BK;  // k of the MFMA steps; the last split adds the tail
  if (k_main < p.K && split == p.splits - 1) {
    // this lane's MT activation rows and 16 weight rows, clamped into the
    // tensors (rows past M / N are never stored); each tail k loads every
    // row's element once
    const uint16_t* xr[MT];
    const int8_t* wr[16];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) xr[mt] = p.x + (int64_t)min(m0 + mt * 32 + r32, p.M - 1) * p.xs;
#pragma unroll
    for (int el = 0; el < 16; ++el)
      wr[el] = p.w + (int64_t)min(n0 + w * 32 + 8 * (el >> 2) + 4 * hk + (el & 3), p.N - 1) * p.wsr;
    float ta[MT][16];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int el = 0; el < 16; ++el) ta[mt][el] = 0.f;
    for (int k = k_main; k < p.K; ++k) {
      float xv[MT], wv[16];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) xv[mt] = elt_to_f32<DTYPE>(xr[mt][k]);
#pragma unroll
      for (int el = 0; el < 16; ++el) wv[el] = (float)wr[el][k];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int el = 0; el < 16; ++el) ta[mt][el] = fmaf(xv[mt], wv[el], ta[mt][el]);
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int el = 0; el < 16; ++el) acc[mt][el] += ta[mt][el];
  }
  if (p.splits == 1) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = m0 + mt * 32 + r32;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int nl = w * 32 + 8 * q + 4 * hk;  // first of 4 consecutive rows in the tile
        const float a[4] = {acc[mt][4 * q], acc[mt][4 * q + 1], acc[mt][4 * q + 2], acc[mt][4 * q + 3]};
        store4<DTYPE>(p, m, n0 + nl, finish4<DTYPE>(a, p, n0 + nl));
      }
    }
    return;
  }

  // partial tile in lane order: slot (split, tile, wave, mt, q, lane) holds
  // the lane's 4 sums as 16 contiguous bytes (MT * 16 KiB per (split, tile))
  const int tile = nt_i * p.m_tiles + mt_i;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    if (m0 + mt * 32 + r32 >= p.M) continue;  // rows past M are never summed
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t slot = (((((int64_t)split * p.n_tiles * p.m_tiles + tile) * 4 + w) * MT + mt) * 4 + q) * 64 + lane;
      *reinterpret_cast<f32x4_t*>(p.partial + 4 * slot) =
          f32x4_t{acc[mt][4 * q], acc[mt][4 * q + 1], acc[mt][4 * q + 2], acc[mt][4 * q + 3]};
    }
  }
}

// One thread per (tile, wave, mt, q, lane) slot of the partial layout: the
// same 4 outputs that lane held in the main kernel, summed over the splits in
// split order, then scaled, rounded and stored.
template <int DTYPE, int MT>
__global__ __launch_bounds__(256) void int8_gemm_reduce_kernel(const I8GemmParams p) {
  const int64_t per_split = (int64_t)p.n_tiles * p.m_tiles * 4 * MT * 4 * 64;  // tiles x waves x MT x q x lanes
  const int64_t slot = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (slot >= per_split) return;
  const int lane = (int)(slot & 63);
  const int64_t r = slot >> 6;
  const int q = (int)(r & 3);
  const int mt = (int)((r >> 2) % MT);
  const int64_t r3 = (r >> 2) / MT;
  const int w = (int)(r3 & 3), tile = (int)(r3 >> 2);
  const int mt_i = tile % p.m_tiles, nt_i = tile / p.m_tiles;
  const int m = mt_i * 32 * MT + mt * 32 + (lane & 31);
  const int n = nt_i * kI8BN + w * 32 + 8 * q + 4 * (lane >> 5);
  if (m >= p.M) return;
  f32x4_t v[kI8MaxSplits];  // every split's partial in flight at once
#pragma unroll
  for (int sp = 0; sp < kI8MaxSplits; ++sp)
    if (sp < p.splits) v[sp] = *reinterpret_cast<const f32x4_t*>(p.partial + 4 * (sp * per_split + slot));
  float a[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int sp = 0; sp < kI8MaxSplits; ++sp) {
    if (sp < p.splits) {
      a[0] += v[sp][0];
      a[1] += v[sp][1];
      a[2] += v[sp][2];
      a[3] += v[sp][3];
    }
  }
  store4<DTYPE>(p, m, n, finish4<DTYPE>(a, p, n));
}

// Decode-sized layers (2 < M <= 64, and M <= 2 with activation rows too long
// for the row-streaming kernel's LDS): weight streaming in one launch. A
// workgroup owns kGvRows = 16 weight rows and its 4 waves split K into
// quarters. A wave streams its quarter in passes of PG 32-k groups: per pass
// WI direct-to-LDS loads move the 16 weight rows (32 PG contiguous bytes of
// each) and XI more move the staged activation rows (64 PG contiguous bytes
// of each; rows past M repeat row M - 1), into a private ring of NS pass
// buffers, so the copies run up to NS - 1 passes ahead of the dequant +
// MFMA work. Staging the activations through LDS keeps the vector-memory
// instructions per pass at WI + XI (loading the MFMA operand per lane took
// 8 per 128 k, and those loads, not the weight bytes, bounded the kernel).
// Chunks are XOR-swizzled by row so the fragment reads spread over the LDS
// banks. The products run on 16x16x32 MFMAs (see the kernel); the 4 waves'
// partial tiles are summed through LDS in wave order (deterministic), then
// scaled, rounded, stored. Staging 4 rows instead of 8 at M = 3-4 halves the
// activation copies (N = K = 4096: 5.61 / 5.65 us against 5.75 / 5.79);
// eight or sixteen waves per workgroup (K in eighths or sixteenths, two
// to four pass buffers per wave) ran 1-9 % slower at M = 3-16.
constexpr int kGvWaves = 4;
constexpr int kGvRows = 16;

template <int XROWS, int MT>
struct WsCfg {
  static constexpr int PG = MT == 1 ? 4 : 2;            // 32-k groups per pass
  static constexpr int WRB = 32 * PG;                   // bytes of a weight row per pass
  static constexpr int WCH = WRB / 16;                  // its 16-byte chunks
  static constexpr int WRI = 64 / WCH;                  // weight rows per copy instruction
  static constexpr int WI = kGvRows / WRI;              // weight copies per pass
  static constexpr int WPH = 256 / WRB;                 // rows sharing a bank phase
  static constexpr int XRB = 64 * PG;                   // bytes of an activation row per pass
  static constexpr int XCH = XRB / 16;
  static constexpr int XRI = 64 / XCH;                  // activation rows per copy instruction
  static constexpr int XI = XROWS / XRI;                // activation copies per pass
  static constexpr int XPH = 256 / XRB;
  static constexpr int WBYTES = kGvRows * WRB;
  static constexpr int PASS = WBYTES + XROWS * XRB;     // LDS bytes per pass buffer
  static constexpr int NS = XROWS >= 32 ? 3 : 4;        // pass buffers per wave
  static constexpr int PER = WI + XI;                   // copies per pass
  static constexpr int LDS = kGvWaves * NS * PASS;
  static_assert((NS - 1) * PER < 64, "vmcnt range");
  static_assert(WI * WRI == kGvRows && XI * XRI == XROWS, "copies split evenly");
  // chunk swizzles: rows in one bank phase get distinct chunk positions
  static __device__ __forceinline__ int wswz(int row) { return (row / WPH) % WCH; }
  static __device__ __forceinline__ int xswz(int row) { return (row / XPH) % XCH; }
};

// The activations are NT16 16-column tiles on v_mfma_f32_16x16x32 with the
// 16 weight rows as the A operand: no discarded A rows (the 32x32x16 form
// would discard half of them and read twice the weight fragments per k).
template <int DTYPE, int XROWS, int MT, int NT16>
__global__ __launch_bounds__(256) void int8_gemv_kernel(const I8GemmParams p) {
  using E = Elt<DTYPE>;
  using C = WsCfg<XROWS, MT>;
  constexpr int CH = 4 / NT16 > 1 ? 4 / NT16 : 1;  // accumulator chains per tile
  static_assert(NT16 >= 1 && NT16 <= kGvWaves && 16 * (NT16 - 1) < XROWS && C::PG % 2 == 0, "tiles");
  extern __shared__ __attribute__((aligned(16))) uint8_t ws_lds[];
  __shared__ f32x4_t red[kGvWaves][NT16][64];
  const int n0 = blockIdx.x * kGvRows;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int G = p.K / 32;
  const int g0 = w * G / kGvWaves, g1 = (w + 1) * G / kGvWaves;
  const int NP = (g1 - g0 + C::PG - 1) / C::PG;  // passes of this wave (wave-uniform)
  const uint32_t ring = lds_addr_of(ws_lds) + (uint32_t)(w * C::NS * C::PASS);
  const uint8_t* ring_p = ws_lds + w * C::NS * C::PASS;
  // weight copy i: lane -> row WRI i + lane / WCH, stored chunk lane % WCH,
  // which holds chunk (lane % WCH) ^ wswz(row) of the row's pass bytes
  const uint8_t* wsrc[C::WI];
  int wcg[C::WI];  // 32-k group (within the pass) of this lane's chunk
#pragma unroll
  for (int i = 0; i < C::WI; ++i) {
    const int rr = C::WRI * i + lane / C::WCH;
    const int c = (lane % C::WCH) ^ C::wswz(rr);
    wsrc[i] = reinterpret_cast<const uint8_t*>(p.w) + (int64_t)min(n0 + rr, p.N - 1) * p.wsr + 16 * (c & 1);
    wcg[i] = c >> 1;
  }
  // activation copy i: lane -> row XRI i + lane / XCH, stored chunk lane % XCH,
  // which holds chunk (lane % XCH) ^ xswz(row)
  const uint16_t* xsrc[C::XI];
  int xcg[C::XI];
#pragma unroll
  for (int i = 0; i < C::XI; ++i) {
    const int rr = C::XRI * i + lane / C::XCH;
    const int c = (lane % C::XCH) ^ C::xswz(rr);
    xsrc[i] = p.x + (int64_t)min(rr, p.M - 1) * p.xs + 8 * (c & 3);
    xcg[i] = c >> 2;
  }
  // pass q (< NP) into buffer q % NS; groups past the end of K are clamped
  // to the last group (loaded, never used)
  auto issue = [&](int q) CIE_GV_INLINE {
    const int gq = g0 + C::PG * q;
    const uint32_t dst = ring + (uint32_t)((q % C::NS) * C::PASS);
#pragma unroll
    for (int i = 0; i < C::WI; ++i) dma16_at_nt(wsrc[i] + 32 * (int64_t)min(gq + wcg[i], G - 1), dst + 1024u * i);
#pragma unroll
    for (int i = 0; i < C::XI; ++i)
      dma16_at(xsrc[i] + 32 * (int64_t)min(gq + xcg[i], G - 1), dst + (uint32_t)C::WBYTES + 1024u * i);
  };

  f32x4 acc[NT16][CH];
#pragma unroll
  for (int t = 0; t < NT16; ++t)
#pragma unroll
    for (int ch = 0; ch < CH; ++ch) acc[t][ch] = f32x4{};
#pragma unroll
  for (int q = 0; q < C::NS; ++q)
    if (q < NP) issue(q);
  // lane (i = lane % 16, kq = lane / 16) holds 16 k of weight row i at
  // 64 h + 16 kq .. +16 (h: 64-k half of the pass) and the same 16 k of
  // activation row 16 t + i of tile t; the first 8 feed MFMA 0, the last 8 MFMA 1
  const int i16 = lane & 15, kq = lane >> 4;
  for (int q = 0; q < NP; ++q) {
    // copies issued after pass q's: those of passes q+1 .. min(q+NS-1, NP-1)
    const int ahead = min(C::NS - 1, NP - 1 - q);
    if (C::NS > 3 && ahead >= 3) vm_wait<(C::NS > 3 ? 3 : 0) * C::PER>();
    else if (ahead == 2) vm_wait<2 * C::PER>();
    else if (ahead == 1) vm_wait<C::PER>();
    else vm_wait<0>();
    const uint8_t* buf = ring_p + (q % C::NS) * C::PASS;
    const int ng = min(C::PG, g1 - g0 - C::PG * q);  // groups of this pass
    u32x4 wq[C::PG / 2], xq[NT16][C::PG / 2][2];
#pragma unroll
    for (int h = 0; h < C::PG / 2; ++h) {
      const int wc = 4 * h + kq;
      wq[h] = *reinterpret_cast<const u32x4*>(buf + i16 * C::WRB + 16 * (wc ^ C::wswz(i16)));
#pragma unroll
      for (int t = 0; t < NT16; ++t) {
        const int xr = min(16 * t + i16, XROWS - 1);
        const uint8_t* xb = buf + C::WBYTES + xr * C::XRB;
        const int xc = 8 * h + 2 * kq;
        xq[t][h][0] = *reinterpret_cast<const u32x4*>(xb + 16 * (xc ^ C::xswz(xr)));
        xq[t][h][1] = *reinterpret_cast<const u32x4*>(xb + 16 * ((xc + 1) ^ C::xswz(xr)));
      }
    }
#pragma unroll
    for (int h = 0; h < C::PG / 2; ++h) {
      if (2 * h < ng) {
        // the half's second group lies past the range: its lanes (kq >= 2) contribute nothing
        const u32x4 wv = zero_unless(wq[h], 2 * h + 1 < ng || kq < 2);
        u32x4 a0, a1;
        dequant16<DTYPE>(wv, a0, a1);
#pragma unroll
        for (int t = 0; t < NT16; ++t) {
          acc[t][(2 * h) % CH] = E::mfma16(a0, xq[t][h][0], acc[t][(2 * h) % CH]);
          acc[t][(2 * h + 1) % CH] = E::mfma16(a1, xq[t][h][1], acc[t][(2 * h + 1) % CH]);
        }
      }
    }
    lgkm_wait0();  // this buffer's reads are complete before it is refilled
    if (q + C::NS < NP) issue(q + C::NS);
  }
  vm_wait<0>();  // no copy into LDS may be in flight when the workgroup ends
  // lane (j = lane % 16, iq = lane / 16) of tile t holds weight rows 4 iq .. +4
  // for activation row 16 t + j; chains summed in a fixed order
#pragma unroll
  for (int t = 0; t < NT16; ++t) {
    f32x4_t v;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float a = acc[t][0][e];
#pragma unroll
      for (int ch = 1; ch < CH; ++ch) a += acc[t][ch][e];
      v[e] = a;
    }
    red[w][t][lane] = v;
  }
  __syncthreads();
  if (w < NT16) {  // wave t finishes tile t, summing the waves in order
    float a[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int wv = 0; wv < kGvWaves; ++wv) {
      const f32x4_t v = red[wv][w][lane];
      a[0] += v[0];
      a[1] += v[1];
      a[2] += v[2];
      a[3] += v[3];
    }
    const int n = n0 + 4 * (lane >> 4);
    if (32 * G < p.K) {  // the K tail past the last whole 32-k group
#pragma unroll
      for (int e = 0; e < 4; ++e) a[e] += tail_dot<DTYPE>(p, 16 * w + (lane & 15), n + e, 32 * G);
    }
    store4<DTYPE>(p, 16 * w + (lane & 15), n, finish4<DTYPE>(a, p, n));
  }
}

template <int DTYPE, int XROWS, int MT, int NT16>
static hipError_t launch_ws_t(const I8GemmParams& p, hipStream_t stream) {
  using C = WsCfg<XROWS, MT>;
  const hipError_t attr = set_dynamic_lds(reinterpret_cast<const void*>(&int8_gemv_kernel<DTYPE, XROWS, MT, NT16>), C::LDS);
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL((int8_gemv_kernel<DTYPE, XROWS, MT, NT16>), dim3((unsigned)((p.N + kGvRows - 1) / kGvRows)),
                     dim3(64 * kGvWaves), C::LDS, stream, p);
  return hipGetLastError();
}

// Decode at M = 1 when the activation row does not fit the LDS of the
// row-streaming kernel below (K > 32768): VALU dot products. The MFMA
// operand of the kernel above spans 32 activation rows, so at M = 1 it
// computes 32x the products it keeps and still loads each wave's whole K
// share before its first MFMA.
// Here a single-wave workgroup streams kDotRows weight rows in 1 KiB chunks
// (lane l covers k = 1024 c + 16 l .. +16 of chunk c: one 16-byte load per
// row and chunk, the contiguous-run pattern), kDotDepth chunks ahead in a
// register ring, with the activation fragments of the same k (read from L2)
// in the same ring. Each chunk is dequantized exactly as in the MFMA path and
// multiplied into fp32 accumulators with v_dot2 (products exact in fp32); a
// fixed xor butterfly over the 64 lanes then sums every (row, activation row)
// and lane r * MC + m finishes output (m, n0 + r). Two rows per wave and two
// chunks ahead measured fastest at M = 1-4 among 1-16 rows and 2-8 chunks
// (more waves in flight beat deeper per-wave rings); from M = 2 the MFMA
// streaming kernel above is faster. The row-streaming kernel below, which
// stages the activations in LDS instead, runs N = K = 4096 in 5.06 us
// against 5.36.
constexpr int kDotRows = 2;
constexpr int kDotDepth = 2;
constexpr int kDotMaxM = 1;  // from M = 2 the MFMA streaming kernel is faster

template <int DTYPE, int MC>
__global__ __launch_bounds__(64) void int8_gemv_dot_kernel(const I8GemmParams p) {
  using E = Elt<DTYPE>;
  constexpr int PERC = kDotRows + 2 * MC;  // loads per chunk
  const int lane = threadIdx.x;
  const int n0 = blockIdx.x * kDotRows;
  const int K16 = p.K & ~15;  // k of the 16-element lane chunks; the rest is added at the end
  const int nch = (K16 + 1023) >> 10;
  const bool tail = (K16 & 1023) != 0;
  // rows past N / M are clamped to the last one (loaded, never stored)
  const int8_t* wrow[kDotRows];
#pragma unroll
  for (int r = 0; r < kDotRows; ++r) wrow[r] = p.w + (int64_t)min(n0 + r, p.N - 1) * p.wsr;
  const uint16_t* xrow[MC];
#pragma unroll
  for (int m = 0; m < MC; ++m) xrow[m] = p.x + (int64_t)min(m, p.M - 1) * p.xs;

  u32x4 wq[kDotDepth][kDotRows], xq[kDotDepth][MC][2];
  // chunk c into ring slot s; lanes past K16 (last chunk) read its last 16 k, zeroed before use
  auto issue = [&](auto S, int c) CIE_GV_INLINE {
    constexpr int s = decltype(S)::value;
    const int k = min(1024 * c + 16 * lane, K16 - 16);
#pragma unroll
    for (int r = 0; r < kDotRows; ++r) wq[s][r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow[r] + k));
#pragma unroll
    for (int m = 0; m < MC; ++m) {
      xq[s][m][0] = load16_clamped(xrow[m] + k);
      xq[s][m][1] = load16_clamped(xrow[m] + k + 8);
    }
  };
  float acc[kDotRows][MC];
#pragma unroll
  for (int r = 0; r < kDotRows; ++r)
#pragma unroll
    for (int m = 0; m < MC; ++m) acc[r][m] = 0.f;

  gv_static_for<kDotDepth>([&](auto S) CIE_GV_INLINE {
    if (decltype(S)::value < nch) issue(S, decltype(S)::value);
  });
  for (int c0 = 0; c0 < nch; c0 += kDotDepth) {
    gv_static_for<kDotDepth>([&](auto S) CIE_GV_INLINE {
      constexpr int s = decltype(S)::value;
      const int c = c0 + s;
      if (c < nch) {  // wave-uniform
        wait_steps_ahead<PERC, kDotDepth - 1>(min(kDotDepth - 1, nch - 1 - c));
        const bool kin = !(tail && c == nch - 1) || 1024 * c + 16 * lane < K16;
#pragma unroll
        for (int r = 0; r < kDotRows; ++r) {
          u32x4 a0, a1;
          dequant16<DTYPE>(zero_unless(wq[s][r], kin), a0, a1);
#pragma unroll
          for (int m = 0; m < MC; ++m) {
            float t = acc[r][m];
#pragma unroll
            for (int i = 0; i < 4; ++i) t = E::dot2(a0[i], xq[s][m][0][i], t);
#pragma unroll
            for (int i = 0; i < 4; ++i) t = E::dot2(a1[i], xq[s][m][1][i], t);
            acc[r][m] = t;
          }
        }
        if (c + kDotDepth < nch) issue(S, c + kDotDepth);
      }
    });
  }

  float out = 0.f;
#pragma unroll
  for (int r = 0; r < kDotRows; ++r)
#pragma unroll
    for (int m = 0; m < MC; ++m) {
      float v = acc[r][m];
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
      if (lane == r * MC + m) out = v;
    }
  const int r = lane / MC, m = lane - (lane / MC) * MC;
  if (lane < kDotRows * MC && m < p.M && n0 + r < p.N) {
    const int n = n0 + r;
    if (K16 < p.K) out += tail_dot<DTYPE>(p, m, n, K16);
    float t = out * load_scale(p.scales, n, p.scale_dtype);
    if (p.bias) {  // the reference adds the bias to the rounded product, in the output dtype
      const uint32_t rr = Elt<DTYPE>::pack2(t, 0.f);
      t = elt_to_f32<DTYPE>((uint16_t)rr) + elt_to_f32<DTYPE>(p.bias[n]);
    }
    p.y[(int64_t)m * p.ys + n] = (uint16_t)Elt<DTYPE>::pack2(t, 0.f);
  }
}

// Decode at M <= kRvMaxM: every weight byte loaded once, all of a wave's
// loads in flight together, the activations read from LDS. A workgroup of
// NWV waves owns RPW = 64 / SL weight rows; its waves split the K steps
// (KSTEP = 16 SL columns each) into NWV contiguous shares, and within a wave
// lane (r = lane / SL, j = lane % SL) takes 16 contiguous bytes of row r per
// step (k = KSTEP s + 16 j: the SL lanes of a row read one contiguous
// KSTEP-byte run). The activation rows (MC of them, the K prefix the steps
// cover) are copied into LDS once per workgroup by direct-to-LDS loads
// issued before the weight loads, so the only loads per step are the
// weights (the VALU dot kernel above reloads the activation fragments from
// L2 next to every weight chunk). Each wave keeps kRvDepth steps of weight
// loads in flight in a register ring; products are exact in fp32 (v_dot2 on
// the dequantized pairs), a lane's terms are summed in ascending k, the SL
// lanes of a row by a fixed xor butterfly and the waves of the workgroup in
// wave order through LDS (deterministic); the K tail past the steps is added
// last, in ascending k. N = K = 4096, graph replay (us; the dot kernel 5.36
// at M = 1, the MFMA streaming kernel 5.74 at M = 2, 5.77 at M = 4):
// SL x NWV x depth 4x8x8 6.55, 8x8x8 5.29, 8x8x4 5.22, 8x8x2 5.14, 16x8x8 5.36,
// 16x4x8 5.52, 32x4x8 5.43, 8x16x2 5.06-5.10 (M = 2: 5.64), 8x16x4 5.18,
// 16x16x2 6.76; at M = 3-4 (four staged rows) 6.77, slower than the MFMA
// streaming kernel, so it takes M <= 2.
constexpr int kRvWaves = 16;
constexpr int kRvSL = 8;
constexpr int kRvDepth = 2;
constexpr int kRvMaxM = 2;
constexpr int kRvMaxLds = 64 * 1024;  // activation bytes staged per workgroup
constexpr int rv_rows(int M) { return M <= 1 ? 1 : 2; }  // activation rows a launch stages

template <int MC, int SL>
struct RvCfg {
  static constexpr int RPW = 64 / SL;     // weight rows per workgroup
  static constexpr int KSTEP = 16 * SL;   // k per step
  static int kmain(int K) { return K - K % KSTEP; }
  static int kpad(int K) { return (kmain(K) + 511) / 512 * 512; }  // LDS row pitch (elements, 1 KiB units)
  static size_t lds(int K) { return (size_t)MC * kpad(K) * 2; }
};

template <int DTYPE, int MC, int SL, int NWV>
__global__ __launch_bounds__(64 * NWV) void int8_gemv_rows_kernel(const I8GemmParams p) {
  using E = Elt<DTYPE>;
  using C = RvCfg<MC, SL>;
  extern __shared__ __attribute__((aligned(16))) uint8_t rv_lds[];
  __shared__ float part[NWV][MC][C::RPW];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane / SL, j = lane % SL;
  const int n0 = blockIdx.x * C::RPW;
  const int KM = p.K - p.K % C::KSTEP, KP = (KM + 511) / 512 * 512;
  const int S = KM / C::KSTEP;
  const int s0 = w * S / NWV, ns = (w + 1) * S / NWV - s0;  // this wave's steps (uniform)

  // activation rows -> LDS: 1 KiB units (64 chunks of 16 bytes) of row m,
  // unit u at byte 2 (m KP + 512 u); lanes past the row's KM / 8 chunks
  // copy its last chunk into the row's padding
  const uint32_t xl = lds_addr_of(rv_lds);
  const int upr = KP / 512, nu = MC * upr;
  for (int v = w; v < nu; v += NWV) {
    const int m = v / upr, u = v - m * upr;
    const int c = min(64 * u + lane, KM / 8 - 1);
    dma16_at(p.x + (int64_t)min(m, p.M - 1) * p.xs + 8 * c, xl + 2u * (uint32_t)(m * KP + 512 * u));
  }
  // weight loads of the first kRvDepth steps (rows past N clamped: loaded, never stored)
  const int8_t* wrow = p.w + (int64_t)min(n0 + r, p.N - 1) * p.wsr + 16 * j;
  u32x4 wq[kRvDepth];
  gv_static_for<kRvDepth>([&](auto I) CIE_GV_INLINE {
    constexpr int i = decltype(I)::value;
    if (i < ns) wq[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow + C::KSTEP * (s0 + i)));
  });
  // this wave's activation copies landed (the weight loads were issued after them)
  wait_steps_ahead<1, kRvDepth>(min(ns, kRvDepth));
  __syncthreads();  // every wave's copies landed

  float acc[MC];
#pragma unroll
  for (int m = 0; m < MC; ++m) acc[m] = 0.f;
  for (int q0 = 0; q0 < ns; q0 += kRvDepth) {
    gv_static_for<kRvDepth>([&](auto I) CIE_GV_INLINE {
      constexpr int i = decltype(I)::value;
      const int q = q0 + i;
      if (q < ns) {  // wave-uniform
        u32x4 a0, a1;
        dequant16<DTYPE>(wq[i], a0, a1);
        if (q + kRvDepth < ns)
          wq[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow + C::KSTEP * (s0 + q + kRvDepth)));
        const int k = C::KSTEP * (s0 + q) + 16 * j;
#pragma unroll
        for (int m = 0; m < MC; ++m) {
          const uint8_t* xb = rv_lds + 2 * (m * KP + k);
          const u32x4 x0 = *reinterpret_cast<const u32x4*>(xb);
          const u32x4 x1 = *reinterpret_cast<const u32x4*>(xb + 16);
          float t = acc[m];
#pragma unroll
          for (int e = 0; e < 4; ++e) t = E::dot2(a0[e], x0[e], t);
#pragma unroll
          for (int e = 0; e < 4; ++e) t = E::dot2(a1[e], x1[e], t);
          acc[m] = t;
        }
      }
    });
  }
#pragma unroll
  for (int m = 0; m < MC; ++m) {
    float v = acc[m];
#pragma unroll
    for (int off = 1; off < SL; off <<= 1) v += __shfl_xor(v, off);
    if (j == 0) part[w][m][r] = v;
  }
  __syncthreads();
  if (threadIdx.x < MC * C::RPW) {
    const int m = threadIdx.x / C::RPW, rr = threadIdx.x % C::RPW, n = n0 + rr;
    float out = 0.f;
#pragma unroll
    for (int wv = 0; wv < NWV; ++wv) out += part[wv][m][rr];
    if (m < p.M && n < p.N) {
      if (KM < p.K) out += tail_dot<DTYPE>(p, m, n, KM);
      float t = out * load_scale(p.scales, n, p.scale_dtype);
      if (p.bias) {  // the reference adds the bias to the rounded product, in the output dtype
        const uint32_t rb = Elt<DTYPE>::pack2(t, 0.f);
        t = elt_to_f32<DTYPE>((uint16_t)rb) + elt_to_f32<DTYPE>(p.bias[n]);
      }
      p.y[(int64_t)m * p.ys + n] = (uint16_t)Elt<DTYPE>::pack2(t, 0.f);
    }
  }
}

I8Geom int8_gemm_geometry(int M, int N, int K, DeviceShape dev) {
  I8Geom g{};
  g.dev = dev;
  g.n_tiles = (N + kI8BN - 1) / kI8BN;
  g.ksteps = K / kI8BK;
  if (M <= 64) {  // weight streaming, one launch, no workspace (2: VALU dot products)
    g.gemv = M <= kDotMaxM ? 2 : 1;
    if (M <= kRvMaxM && (size_t)rv_rows(M) * RvCfg<1, kRvSL>::lds(K) <= (size_t)kRvMaxLds) g.gemv = 3;
    g.mt = M <= 32 ? 1 : 2;
    g.m_tiles = 1;
    g.splits = 1;
    g.m_pad = 32 * g.mt;
    g.n_pad = g.n_tiles * kI8BN;
    return g;
  }
  // activation tile: the larger of 128 / 64 rows that gives two (n, m) tiles
  // per CU; failing both, 128 rows when that gives one tile per CU, else 64
  // (N = K = 4096: M = 1024 ran 47.3 us at 64 rows against 52.1 at 128; at
  // M = 512, 32-row tiles or a K split for two tiles per CU were slower)
  const int64_t cus = dev.cus;
  const int64_t t128 = (int64_t)g.n_tiles * ((M + 127) / 128), t64 = (int64_t)g.n_tiles * ((M + 63) / 64);
  g.mt = t128 >= 2 * cus ? 4 : (t64 >= 2 * cus ? 2 : (t128 >= cus ? 4 : 2));
  // 3-4 ring stages let two workgroups share a CU
  g.nst = g.mt >= 4 ? 3 : 4;
  const int bm = 32 * g.mt;
  g.m_tiles = (M + bm - 1) / bm;
  const int64_t tiles = (int64_t)g.m_tiles * g.n_tiles;
  // split K only as far as needed for one workgroup per CU, keeping >= 4 k steps per split
  int s = 1;
  if (tiles < cus) s = (int)std::min<int64_t>((cus + tiles - 1) / tiles, std::max(1, g.ksteps / 4));
  g.splits = std::max(1, std::min(s, kI8MaxSplits));
  // one workgroup per CU or fewer: eight waves (two k halves) so every SIMD
  // holds two waves (512 x 4096 x 4096: 31.9 -> 30.1 us); else four waves and
  // two workgroups per CU. Not with K split three ways or more (128 x 4096 x
  // 4096, four splits: 1 % slower).
  g.kw2 = tiles * g.splits <= cus && g.splits <= 2;
  g.m_pad = g.m_tiles * bm;
  g.n_pad = g.n_tiles * kI8BN;
  g.workspace_bytes = g.splits > 1 ? (size_t)g.splits * g.m_pad * g.n_pad * sizeof(float) : 0;
  g.lds_bytes = (size_t)g.nst * (bm * kI8BK * 2 + kI8BN * kI8BK);
  return g;
}

template <int DTYPE, int MT, int NST>
static hipError_t launch_i8_t(const I8GemmParams& p, size_t lds, bool kw2, hipStream_t stream) {
  using C = I8Cfg<MT, NST>;
  if (lds != (size_t)C::NST * C::STAGE) return hipErrorInvalidValue;  // geometry and kernel disagree
  const int nwg = p.n_tiles * p.m_tiles * p.splits;
  const void* fn = kw2 ? reinterpret_cast<const void*>(&int8_gemm_kernel<DTYPE, MT, NST, 2>)
                       : reinterpret_cast<const void*>(&int8_gemm_kernel<DTYPE, MT, NST, 1>);
  const hipError_t attr = set_dynamic_lds(fn, C::NST * C::STAGE);
  if (attr != hipSuccess) return attr;
  if (kw2)
    hipLaunchKernelGGL((int8_gemm_kernel<DTYPE, MT, NST, 2>), dim3(nwg), dim3(512), lds, stream, p);
  else
    hipLaunchKernelGGL((int8_gemm_kernel<DTYPE, MT, NST, 1>), dim3(nwg), dim3(256), lds, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.splits == 1) return e;
  const int64_t slots = (int64_t)p.n_tiles * p.m_tiles * 4 * MT * 4 * 64;
  hipLaunchKernelGGL((int8_gemm_reduce_kernel<DTYPE, MT>), dim3((unsigned)((slots + 255) / 256)), dim3(256), 0,
                     stream, p);
  return hipGetLastError();
}

template <int DTYPE, int MC>
static hipError_t launch_rv_t(const I8GemmParams& p, hipStream_t stream) {
  using C = RvCfg<MC, kRvSL>;
  const size_t lds = C::lds(p.K);
  if (lds > (size_t)kRvMaxLds) return hipErrorInvalidValue;  // geometry and kernel disagree
  const void* fn = reinterpret_cast<const void*>(&int8_gemv_rows_kernel<DTYPE, MC, kRvSL, kRvWaves>);
  const hipError_t attr = set_dynamic_lds(fn, kRvMaxLds);
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL((int8_gemv_rows_kernel<DTYPE, MC, kRvSL, kRvWaves>), dim3((unsigned)((p.N + C::RPW - 1) / C::RPW)),
                     dim3(64 * kRvWaves), lds, stream, p);
  return hipGetLastError();
}

template <int DTYPE>
static hipError_t launch_i8_d(const I8GemmParams& p, const I8Geom& g, hipStream_t stream) {
  if (g.gemv == 3) return p.M == 1 ? launch_rv_t<DTYPE, 1>(p, stream) : launch_rv_t<DTYPE, 2>(p, stream);
  if (g.gemv == 2) {
    const dim3 grid((unsigned)((p.N + kDotRows - 1) / kDotRows));
    hipLaunchKernelGGL((int8_gemv_dot_kernel<DTYPE, 1>), grid, dim3(64), 0, stream, p);
    return hipGetLastError();
  }
  if (g.gemv) {  // staged activation rows: 4, 8, 16, 32 or 64
    if (p.M <= 4) return launch_ws_t<DTYPE, 4, 1, 1>(p, stream);
    if (p.M <= 8) return launch_ws_t<DTYPE, 8, 1, 1>(p, stream);
    if (p.M <= 16) return launch_ws_t<DTYPE, 16, 1, 1>(p, stream);
    if (p.M <= 32) return launch_ws_t<DTYPE, 32, 1, 2>(p, stream);
    return launch_ws_t<DTYPE, 64, 2, 4>(p, stream);
  }
  if (g.mt == 2 && g.nst == 4) return launch_i8_t<DTYPE, 2, 4>(p, g.lds_bytes, g.kw2, stream);
  if (g.mt == 4 && g.nst == 3) return launch_i8_t<DTYPE, 4, 3>(p, g.lds_bytes, g.kw2, stream);
  return hipErrorInvalidValue;
}

hipError_t launch_int8_gemm(const I8GemmParams& p, const I8Geom& g, int dtype, hipStream_t stream) {
  return dtype == 0 ? launch_i8_d<0>(p, g, stream) : launch_i8_d<1>(p, g, stream);
}

}  // namespace cie
