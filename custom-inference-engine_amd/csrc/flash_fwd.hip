// Causal / full GQA prefill attention for gfx950.
//
// Replaces the Triton program kernels/flash_attention.py:21-120 and the GQA
// expansion of its wrapper (:150-155): a workgroup of 4 waves owns 128 query
// rows of one query head (32 rows per wave), streams the K/V tiles of the kv
// head h / (Hq / Hk) through double-buffered LDS, and keeps the online-softmax
// state (running max m, row sum l, output accumulator) in registers.
//
// Per K/V tile of BN keys and per wave:
//   S^T[BN x 32] = K_tile . Q_w^T        MFMA 32x32x16, K from LDS (row-major),
//                                          Q^T resident in registers
//   mask + running max (one v_permlane32_swap), p = exp2(s*c - m), c = scale*log2e
//   O^T[D x 32] += V^T_tile . P^T         MFMA 32x32x16, V^T from LDS, P^T
//                                          straight from the S^T registers
// The bottom-right causal rule (key j visible to row i iff j <= Lk - Lq + i,
// kernels/flash_attention.py:99-102) is applied only on tiles that cross a
// wave's diagonal or the key tail; a workgroup stops at the last key any of
// its rows can see (the n_end bound of kernels/flash_attention.py:75-77).
//
// The running max is refreshed lazily: a row keeps its reference max m until
// a tile raises the row max by more than 2^8 (so p <= 256, exact to fp16 /
// bf16 rounding), and the accumulator rescale is skipped for the whole wave
// when no row needs it. The final acc / l is unchanged by the choice of m.
#include "kernels.hpp"

namespace cie {

constexpr float kLazyRescale = 8.0f;  // log2 of the largest p tolerated before rescaling

template <int D>
struct FlashCfg {
  static constexpr int BM = 128;                                            // query rows per workgroup
  static constexpr int BN = D <= 32 ? 128 : (D <= 128 ? 64 : 32);           // keys per tile
  static constexpr int KSTR = D + 8;                                        // LDS row pitch of K
  static constexpr int VSTR = BN + 4;                                       // LDS row pitch of V^T
  static constexpr int DT = D >= 32 ? D / 32 : 1;                           // 32-row output tiles
  static constexpr int KK = D / 16;                                         // MFMA steps over head_dim
  static constexpr int MT = BN / 32;                                        // 32-key score tiles
  static constexpr int KBUF = BN * KSTR;
  static constexpr int VBUF = D * VSTR;
  static constexpr int BUF = KBUF + VBUF;                                   // elements per LDS stage
  static constexpr int KCH = BN * D / 8 / 256;                              // 16-byte K chunks per thread
  static constexpr int VGR = (BN / 4) * (D / 8);                            // 4-key x 8-dim V groups
  static constexpr int VG = (VGR + 255) / 256;                              // V groups per thread
  static_assert(KCH >= 1 && BN * D / 8 == KCH * 256, "K tile must split evenly over 256 threads");
};

template <int DTYPE, int D>
__global__ __launch_bounds__(256, 2) void flash_fwd_kernel(const FlashParams p) {
  using C = FlashCfg<D>;
  using E = Elt<DTYPE>;
  constexpr int BN = C::BN;
  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * C::BUF];

  // Workgroups are dispatched round-robin over the 8 XCDs; give each XCD a
  // contiguous run of logical tiles so the query heads of a kv head (and its
  // neighbouring query tiles) share one L2. Within a kv head the longest
  // (last) query tiles go first.
  const int N = p.n_wg;
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
  const int logical = xcd * (N >> 3) + min(xcd, N & 7) + slot;
  const int G = p.group;
  const int per_grp = p.n_mt * G;
  const int grp = logical / per_grp;
  const int rem = logical - grp * per_grp;
  const int mt = p.n_mt - 1 - rem / G;
  const int g = rem - (rem / G) * G;
  const int b = grp / p.Hk, kvh = grp - b * p.Hk, hq = kvh * G + g;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hl = lane >> 5;
  const int q0w = mt * C::BM + wave * 32;  // first row of this wave
  const int qi = q0w + l32;                // row owned by this lane

  // Q^T as the B operand: lane holds Q[qi][16kk + 8hl .. +8] (sign-flipped
  // when the caller's scale is negative, so c below is never negative).
  const uint16_t* qrow = p.q + b * p.qs0 + hq * p.qs1 + (int64_t)qi * p.qs2;
  u32x4 qf[C::KK];
#pragma unroll
  for (int kk = 0; kk < C::KK; ++kk) {
    qf[kk] = load16(qrow + 16 * kk + 8 * hl, qi < p.Lq);
    qf[kk] ^= u32x4{p.q_sign, p.q_sign, p.q_sign, p.q_sign};
  }

  // Key range of the workgroup and of this wave; lim = last key this row sees.
  const int wg_last_row = min(p.Lq, mt * C::BM + C::BM) - 1;
  int kend = p.Lk;
  if (p.causal) kend = max(0, min(p.Lk, p.Lk - p.Lq + wg_last_row + 1));
  int wave_kend = 0;
  if (q0w < p.Lq) {
    wave_kend = p.Lk;
    if (p.causal) wave_kend = max(0, min(p.Lk, p.Lk - p.Lq + min(q0w + 31, p.Lq - 1) + 1));
  }
  const int lim = p.causal ? min(p.Lk - 1, p.Lk - p.Lq + qi) : p.Lk - 1;
  const int wave_lim0 = p.causal ? min(p.Lk - 1, p.Lk - p.Lq + q0w) : p.Lk - 1;  // smallest lim in the wave
  const int n_tiles = (kend + BN - 1) / BN;
  const float c = p.scale_log2;

  const uint16_t* kb = p.k + b * p.ks0 + kvh * p.ks1;
  const uint16_t* vb = p.v + b * p.vs0 + kvh * p.vs1;
  const int last_key = max(p.Lk - 1, 0);

  u32x4 kreg[C::KCH];
  u32x4 vreg[C::VG][4];
  uint32_t vok[C::VG];  // bit r: key 4*p4 + r of the group exists
  auto gload = [&](int n0) {
#pragma unroll
    for (int cc = 0; cc < C::KCH; ++cc) {
      const int idx = tid + 256 * cc;
      const int row = idx / (D / 8), c8 = idx % (D / 8);
      const int key = min(n0 + row, last_key);  // rows past the end are masked as scores
      kreg[cc] = load16_clamped(kb + (int64_t)key * p.ks2 + 8 * c8);
    }
#pragma unroll
    for (int gg = 0; gg < C::VG; ++gg) {
      const int gi = min(tid + 256 * gg, C::VGR - 1);
      const int p4 = gi / (D / 8), qd = gi % (D / 8);
      uint32_t okm = 0;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = n0 + 4 * p4 + r;
        okm |= (key < p.Lk ? 1u : 0u) << r;
        vreg[gg][r] = load16_clamped(vb + (int64_t)min(key, last_key) * p.vs2 + 8 * qd);
      }
      vok[gg] = okm;
    }
  };
  auto sstore = [&](uint16_t* buf) {
#pragma unroll
    for (int cc = 0; cc < C::KCH; ++cc) {
      const int idx = tid + 256 * cc;
      const int row = idx / (D / 8), c8 = idx % (D / 8);
      *reinterpret_cast<u32x4*>(buf + row * C::KSTR + 8 * c8) = kreg[cc];
    }
    uint16_t* vt = buf + C::KBUF;
#pragma unroll
    for (int gg = 0; gg < C::VG; ++gg) {
      const int gi = tid + 256 * gg;
      if (C::VGR % 256 == 0 || gi < C::VGR) {
        const int p4 = gi / (D / 8), qd = gi % (D / 8);
        u32x4 r0 = zero_unless(vreg[gg][0], vok[gg] & 1u);
        u32x4 r1 = zero_unless(vreg[gg][1], vok[gg] & 2u);
        u32x4 r2 = zero_unless(vreg[gg][2], vok[gg] & 4u);
        u32x4 r3 = zero_unless(vreg[gg][3], vok[gg] & 8u);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const int d = 8 * qd + 2 * w;
          *reinterpret_cast<u32x2*>(vt + d * C::VSTR + 4 * p4) = col4_even(r0[w], r1[w], r2[w], r3[w]);
          *reinterpret_cast<u32x2*>(vt + (d + 1) * C::VSTR + 4 * p4) = col4_odd(r0[w], r1[w], r2[w], r3[w]);
        }
      }
    }
  };

  f32x16 acc[C::DT];
#pragma unroll
  for (int dt = 0; dt < C::DT; ++dt) acc[dt] = f32x16{};
  float m = -INFINITY, l = 0.f;

  if (n_tiles > 0) {
    gload(0);
    sstore(smem);
  }
  __syncthreads();

  for (int t = 0; t < n_tiles; ++t) {
    const int n0 = t * BN;
    if (t + 1 < n_tiles) gload(n0 + BN);
    const uint16_t* ks = smem + (t & 1) * C::BUF;
    const uint16_t* vt = ks + C::KBUF;

    if (n0 < wave_kend) {
      f32x16 s[C::MT];
#pragma unroll
      for (int mt2 = 0; mt2 < C::MT; ++mt2) s[mt2] = f32x16{};
#pragma unroll
      for (int kk = 0; kk < C::KK; ++kk) {
#pragma unroll
        for (int mt2 = 0; mt2 < C::MT; ++mt2) {
          const u32x4 a = *reinterpret_cast<const u32x4*>(ks + (32 * mt2 + l32) * C::KSTR + 16 * kk + 8 * hl);
          s[mt2] = E::mfma(a, qf[kk], s[mt2]);
        }
      }
      // mask (tiles crossing the diagonal or the key tail only) and row max
      float mx = -INFINITY;
      if (n0 + BN - 1 > wave_lim0) {
#pragma unroll
        for (int mt2 = 0; mt2 < C::MT; ++mt2)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int key = n0 + 32 * mt2 + 8 * (e >> 2) + 4 * hl + (e & 3);
            s[mt2][e] = key <= lim ? s[mt2][e] : -INFINITY;
          }
      }
#pragma unroll
      for (int mt2 = 0; mt2 < C::MT; ++mt2)
#pragma unroll
        for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[mt2][e]);
      const float mxs = xhalf_max(mx) * c;
      const bool grow = mxs > m + kLazyRescale;
      if (__builtin_amdgcn_ballot_w64(grow)) {
        const float m_new = grow ? mxs : m;
        const float alpha = grow ? exp2_fast(m - m_new) : 1.f;  // 0 when m was -inf
        l *= alpha;
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) acc[dt] *= alpha;
        m = m_new;
      }
      const float neg_m = m == -INFINITY ? 0.f : -m;

      u32x4 pb[2 * C::MT];
#pragma unroll
      for (int mt2 = 0; mt2 < C::MT; ++mt2) {
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const int e0 = 8 * cc + 2 * w;
            const float p0 = exp2_fast(fmaf(s[mt2][e0], c, neg_m));
            const float p1 = exp2_fast(fmaf(s[mt2][e0 + 1], c, neg_m));
            l += p0 + p1;
            pb[2 * mt2 + cc][w] = E::pack2(p0, p1);
          }
        }
      }
#pragma unroll
      for (int dt = 0; dt < C::DT; ++dt) {
        const int drow = 32 * dt + l32;
#pragma unroll
        for (int cc = 0; cc < 2 * C::MT; ++cc) {
          u32x4 a = {0u, 0u, 0u, 0u};
          if (D >= 32 || drow < D) {
            const u32x2 lo = *reinterpret_cast<const u32x2*>(vt + drow * C::VSTR + 16 * cc + 4 * hl);
            const u32x2 hi = *reinterpret_cast<const u32x2*>(vt + drow * C::VSTR + 16 * cc + 8 + 4 * hl);
            a = u32x4{lo[0], lo[1], hi[0], hi[1]};
          }
          acc[dt] = E::mfma(a, pb[cc], acc[dt]);
        }
      }
    }

    if (t + 1 < n_tiles) sstore(smem + ((t + 1) & 1) * C::BUF);
    __syncthreads();
  }

  // Epilogue: rows with keys but none visible give 0 * inf = NaN like the
  // reference's softmax over an all -inf row; Lk == 0 gives zeros.
  const float l_tot = xhalf_sum(l);
  const float inv = p.Lk == 0 ? 0.f : 1.f / l_tot;
  if (qi < p.Lq) {
    uint16_t* orow = p.o + b * p.os0 + hq * p.os1 + (int64_t)qi * p.os2;
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) {
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d = 32 * dt + 8 * g4 + 4 * hl;
        if (D >= 32 || d < D) {
          const u32x2 w = {E::pack2(acc[dt][4 * g4] * inv, acc[dt][4 * g4 + 1] * inv),
                           E::pack2(acc[dt][4 * g4 + 2] * inv, acc[dt][4 * g4 + 3] * inv)};
          *reinterpret_cast<u32x2*>(orow + d) = w;
        }
      }
    }
  }
}

template <int DTYPE, int D>
static hipError_t launch_flash_t(const FlashParams& p, hipStream_t stream) {
  hipLaunchKernelGGL((flash_fwd_kernel<DTYPE, D>), dim3(p.n_wg), dim3(256), 0, stream, p);
  return hipGetLastError();
}

template <int DTYPE>
static hipError_t launch_flash_d(const FlashParams& p, int D, hipStream_t stream) {
  switch (D) {
    case 16: return launch_flash_t<DTYPE, 16>(p, stream);
    case 32: return launch_flash_t<DTYPE, 32>(p, stream);
    case 64: return launch_flash_t<DTYPE, 64>(p, stream);
    case 128: return launch_flash_t<DTYPE, 128>(p, stream);
    case 256: return launch_flash_t<DTYPE, 256>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_flash(const FlashParams& p, int dtype, int D, hipStream_t stream) {
  return dtype == 0 ? launch_flash_d<0>(p, D, stream) : launch_flash_d<1>(p, D, stream);
}

}  // namespace cie
