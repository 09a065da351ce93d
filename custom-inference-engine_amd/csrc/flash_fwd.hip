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
//   mask + running max (one v_permlane32_swap), p = exp2(s*scale*log2e - m)
//   O^T[D x 32] += V^T_tile . P^T         MFMA 32x32x16, V^T from LDS, P^T
//                                          straight from the S^T registers
// The bottom-right causal rule (key j visible to row i iff j <= Lk - Lq + i,
// kernels/flash_attention.py:99-102) is applied only on tiles that cross a
// wave's diagonal or the key tail; a workgroup stops at the last key any of
// its rows can see (the n_end bound of kernels/flash_attention.py:75-77).
#include "kernels.hpp"

namespace cie {

template <int D>
struct FlashCfg {
  static constexpr int BM = 128;                                 // query rows per workgroup
  static constexpr int BN = D <= 64 ? 128 : (D == 128 ? 64 : 32);  // keys per tile
  static constexpr int KSTR = D + 8;                             // LDS row pitch of K (elements)
  static constexpr int VSTR = BN + 4;                            // LDS row pitch of V^T (elements)
  static constexpr int DT = D >= 32 ? D / 32 : 1;                // 32-row output tiles
  static constexpr int KK = D / 16;                              // MFMA steps over head_dim
  static constexpr int MT = BN / 32;                             // 32-key score tiles
  static constexpr int KBUF = BN * KSTR;
  static constexpr int VBUF = D * VSTR;
  static constexpr int BUF = KBUF + VBUF;                        // elements per LDS stage
  static constexpr int KCH = BN * D / 8 / 256;                   // 16-byte K chunks per thread
  static constexpr int VGR = (BN / 4) * (D / 8);                 // 4-key x 8-dim V groups
  static constexpr int VG = (VGR + 255) / 256;                   // V groups per thread
  static_assert(KCH >= 1 && BN * D / 8 == KCH * 256, "K tile must split evenly over 256 threads");
};

template <int DTYPE, int D>
__global__ __launch_bounds__(256) void flash_fwd_kernel(const FlashParams p) {
  using C = FlashCfg<D>;
  using E = Elt<DTYPE>;
  constexpr int BN = C::BN;
  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * C::BUF];

  // Workgroups are dispatched round-robin over the 8 XCDs; give each XCD a
  // contiguous run of logical tiles so the 4 query heads of a kv head (and
  // its neighbouring query tiles) share one L2. Within a kv head the longest
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

  // Q^T as the B operand: lane holds Q[qi][16kk + 8hl .. +8].
  const uint16_t* qrow = p.q + b * p.qs0 + hq * p.qs1 + (int64_t)qi * p.qs2;
  u32x4 qf[C::KK];
#pragma unroll
  for (int kk = 0; kk < C::KK; ++kk) qf[kk] = load16(qrow + 16 * kk + 8 * hl, qi < p.Lq);

  // Key range of the workgroup and of this wave.
  const int wg_last_row = min(p.Lq, mt * C::BM + C::BM) - 1;
  int kend = p.Lk;
  if (p.causal) kend = max(0, min(p.Lk, p.Lk - p.Lq + wg_last_row + 1));
  int wave_kend = 0;
  if (q0w < p.Lq) {
    wave_kend = p.Lk;
    if (p.causal) wave_kend = max(0, min(p.Lk, p.Lk - p.Lq + min(q0w + 31, p.Lq - 1) + 1));
  }
  const int wave_diag0 = p.Lk - p.Lq + q0w;  // last visible key of the wave's first row
  const int diag = p.Lk - p.Lq + qi;         // last visible key of this lane's row
  const int n_tiles = (kend + BN - 1) / BN;

  const uint16_t* kb = p.k + b * p.ks0 + kvh * p.ks1;
  const uint16_t* vb = p.v + b * p.vs0 + kvh * p.vs1;

  u32x4 kreg[C::KCH];
  u32x4 vreg[C::VG][4];
  auto gload = [&](int n0) {
#pragma unroll
    for (int c = 0; c < C::KCH; ++c) {
      const int idx = tid + 256 * c;
      const int row = idx / (D / 8), c8 = idx % (D / 8);
      const int key = n0 + row;
      kreg[c] = load16(kb + (int64_t)key * p.ks2 + 8 * c8, key < p.Lk);
    }
#pragma unroll
    for (int gg = 0; gg < C::VG; ++gg) {
      const int gi = tid + 256 * gg;
      const int p4 = gi / (D / 8), qd = gi % (D / 8);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = n0 + 4 * p4 + r;
        vreg[gg][r] = load16(vb + (int64_t)key * p.vs2 + 8 * qd, gi < C::VGR && key < p.Lk);
      }
    }
  };
  auto sstore = [&](uint16_t* buf) {
#pragma unroll
    for (int c = 0; c < C::KCH; ++c) {
      const int idx = tid + 256 * c;
      const int row = idx / (D / 8), c8 = idx % (D / 8);
      *reinterpret_cast<u32x4*>(buf + row * C::KSTR + 8 * c8) = kreg[c];
    }
    uint16_t* vt = buf + C::KBUF;
#pragma unroll
    for (int gg = 0; gg < C::VG; ++gg) {
      const int gi = tid + 256 * gg;
      if (gi < C::VGR) {
        const int p4 = gi / (D / 8), qd = gi % (D / 8);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const int d = 8 * qd + 2 * w;
          *reinterpret_cast<u32x2*>(vt + d * C::VSTR + 4 * p4) =
              col4_even(vreg[gg][0][w], vreg[gg][1][w], vreg[gg][2][w], vreg[gg][3][w]);
          *reinterpret_cast<u32x2*>(vt + (d + 1) * C::VSTR + 4 * p4) =
              col4_odd(vreg[gg][0][w], vreg[gg][1][w], vreg[gg][2][w], vreg[gg][3][w]);
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
      for (int mt2 = 0; mt2 < C::MT; ++mt2) {
        s[mt2] = f32x16{};
#pragma unroll
        for (int kk = 0; kk < C::KK; ++kk) {
          const u32x4 a = *reinterpret_cast<const u32x4*>(ks + (32 * mt2 + l32) * C::KSTR + 16 * kk + 8 * hl);
          s[mt2] = E::mfma(a, qf[kk], s[mt2]);
        }
      }
      const bool need_mask = (n0 + BN > p.Lk) || (p.causal && n0 + BN - 1 > wave_diag0);
      float mx = -INFINITY;
#pragma unroll
      for (int mt2 = 0; mt2 < C::MT; ++mt2) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          float x = s[mt2][e] * p.scale_log2;
          if (need_mask) {
            const int key = n0 + 32 * mt2 + 8 * (e >> 2) + 4 * hl + (e & 3);
            const bool ok = key < p.Lk && (!p.causal || key <= diag);
            x = ok ? x : -INFINITY;
          }
          s[mt2][e] = x;
          mx = fmaxf(mx, x);
        }
      }
      mx = xhalf_max(mx);
      const float m_new = fmaxf(m, mx);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = exp2_fast(m - m_use);
      l *= alpha;
#pragma unroll
      for (int dt = 0; dt < C::DT; ++dt) acc[dt] *= alpha;

      u32x4 pb[2 * C::MT];
#pragma unroll
      for (int mt2 = 0; mt2 < C::MT; ++mt2) {
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const int e0 = 8 * cc + 2 * w;
            const float p0 = exp2_fast(s[mt2][e0] - m_use);
            const float p1 = exp2_fast(s[mt2][e0 + 1] - m_use);
            l += p0 + p1;
            pb[2 * mt2 + cc][w] = E::pack2(p0, p1);
          }
        }
      }
#pragma unroll
      for (int dt = 0; dt < C::DT; ++dt) {
        const int drow = 32 * dt + l32;
#pragma unroll
        for (int c = 0; c < 2 * C::MT; ++c) {
          u32x4 a = {0u, 0u, 0u, 0u};
          if (D >= 32 || drow < D) {
            const u32x2 lo = *reinterpret_cast<const u32x2*>(vt + drow * C::VSTR + 16 * c + 4 * hl);
            const u32x2 hi = *reinterpret_cast<const u32x2*>(vt + drow * C::VSTR + 16 * c + 8 + 4 * hl);
            a = u32x4{lo[0], lo[1], hi[0], hi[1]};
          }
          acc[dt] = E::mfma(a, pb[c], acc[dt]);
        }
      }
      m = m_new;
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
