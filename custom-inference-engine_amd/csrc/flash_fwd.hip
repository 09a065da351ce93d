// Causal / full GQA prefill attention for gfx950.
//
// Replaces the Triton program kernels/flash_attention.py:21-120 and the GQA
// expansion of its wrapper (:150-155): a workgroup of 4 waves owns 128 query
// rows of one query head (32 rows per wave) and streams the K/V tiles of kv
// head h / (Hq / Hk) through an LDS ring; the online-softmax state (running
// max m, row sum l, output accumulator) stays in registers.
//
// Memory path: each K/V tile (BN keys) is copied global -> LDS by 16-byte
// direct-to-LDS loads issued by all four waves (no VGPR staging), row-major
// with the 16-byte chunks of each row XOR-swizzled (chunk_swizzle). One or
// two tiles are in flight while the tiles being read stay resident; one
// workgroup barrier per tile publishes the next tile and frees the stage
// refilled next (three or four stages).
// Per tile and wave:
//   S^T[BN x 32] = K_tile . Q_w^T     MFMA 32x32x16; A = ds_read_b128 of K rows,
//                                      B = Q^T resident in registers (unscaled)
//   p = exp2(s * c - m)                one fma per score on the fp32
//                                      accumulator, c = scale * log2 e
//   O^T[D x 32] += V^T_tile . P^T      MFMA 32x32x16; A = ds_read_b64_tr_b16 of
//                                      the row-major V tile, B = P^T straight
//                                      from the S^T registers
// The bottom-right causal rule (key j visible to row i iff j <= Lk - Lq + i,
// kernels/flash_attention.py:99-102) is applied only on tiles that cross a
// wave's diagonal or the key tail; a workgroup stops at the last key any of
// its rows can see (the n_end bound of kernels/flash_attention.py:75-77).
//
// The softmax scale is applied to the fp32 score accumulator, as the
// reference applies it to the fp32 dot product (kernels/flash_attention.py:
// 98): q enters the MFMA exactly as given (a negative scale flips its sign,
// which is exact), so no rounding of scale * q to 16 bits enters the scores.
// The running max is refreshed lazily and without a per-tile row max: p(t)
// is computed against the reference max m, and only when a row's
// probabilities of the tile sum past 2^10 (so some p may not fit the 16-bit
// P.V operand; always the case for a row that had no visible key before)
// does the wave recompute S(t) from the still-resident K tile, take its row
// max, raise m to it and redo the tile. Otherwise every p <= 2^10, exact to
// fp16 / bf16 rounding. The final acc / l is unchanged by the choice of m. l
// accumulates the probabilities as rounded for the P.V product, summed on
// the matrix pipe (see sum_ones).
//
// The tile loop is unrolled by a multiple of the ring depth so that every
// LDS stage offset is an immediate of the fragment reads.
//
// head_dim 128 runs flash_fwd_il_kernel below instead: same tiles and
// softmax rules, its MFMA and VALU work issued as one interleaved stream.
// head_dim 64 launches with enough work (r64_pays) run flash_fwd_r64_kernel:
// two 32-row groups per wave (the same rows of two query heads, or 64 rows
// of one head) sharing every K/V fragment read.
#include <algorithm>
#include <type_traits>
#include <utility>

#include "kernels.hpp"
#include "rope.hpp"

namespace cie {

#ifdef CIE_TIMELINE
__device__ unsigned long long flash_timeline[kTimelineMaxWg * kTimelineSlots];  // benchmarks/timeline.py
#endif

// Every lambda of the kernel is inlined: the score arrays they take by
// pointer must stay in registers.
#define CIE_INLINE __attribute__((always_inline))

constexpr float kSumTrigger = 1024.0f;  // a lane's tile sum of p above this recomputes the row max

// f(integral_constant<int, 0>), ..., f(integral_constant<int, N - 1>), in order.
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

template <int D>
struct FlashCfg {
  static constexpr int BM = 128;                                   // query rows per workgroup
  static constexpr int BN = D <= 32 ? 128 : (D == 64 ? 64 : 32);   // keys per tile
  static constexpr int S = D / 8;                                  // 16-byte chunks per row
  static constexpr int DT = D >= 32 ? D / 32 : 1;                  // 32-row output tiles
  static constexpr int KK = D / 16;                                // MFMA steps over head_dim
  static constexpr int MT = BN / 32;                               // 32-key score tiles
  static constexpr int TILE = BN * D;                              // elements of one tensor tile
  static constexpr int STAGE = 2 * TILE;                           // K tile, then V tile
  static constexpr int NST = D == 256 ? 3 : 4;                     // ring stages (see the tile loop)
  static constexpr int NW = BN * S / 256;                          // 1 KiB copies per wave per tensor
  static constexpr int PER_TILE = 2 * NW;                          // copies per wave per tile
  static constexpr int OCC = D <= 128 ? 2 : 1;                     // workgroups per CU
  static constexpr int NQK = KK * MT;                              // QK^T MFMAs per tile
  static constexpr int NPV = DT * 2 * MT;                          // P.V MFMAs per tile
  static_assert(NW >= 1 && BN * S == NW * 256, "tile must split evenly over 4 waves");
};

// vm_wait for the copies of `ahead` tiles issued after the one needed.
template <int NST, int PER_TILE>
__device__ __forceinline__ void wait_ahead(int ahead) {
  if (NST > 3 && ahead >= 2) vm_wait<(NST > 3 ? 2 : 0) * PER_TILE>();
  else if (NST > 2 && ahead == 1) vm_wait<PER_TILE>();
  else vm_wait<0>();
}

template <int DTYPE, int D>
__global__ __launch_bounds__(256, FlashCfg<D>::OCC) void flash_fwd_kernel(const FlashParams p) {
  using C = FlashCfg<D>;
  using E = Elt<DTYPE>;
  constexpr int BN = C::BN;
  __shared__ __attribute__((aligned(16))) uint16_t ring[C::NST * C::STAGE];

  // Workgroups are dispatched round-robin over the XCDs; give each XCD a
  // contiguous run of logical tiles so the query heads of a kv head (and its
  // neighbouring query tiles) share one L2. Within a kv head the longest
  // (last) query tiles go first.
  const int logical = xcd_logical(blockIdx.x, p.n_wg, p.xcd_shift);
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

  // Q^T as the B operand: lane holds Q[qi][16kk + 8hl .. +8], its sign
  // flipped when the caller's scale is negative (p.scale_log2 is |scale| *
  // log2 e, never negative).
  const uint16_t* qrow = p.q + b * p.qs0 + hq * p.qs1 + (int64_t)qi * p.qs2;
  u32x4 qf[C::KK];
#pragma unroll
  for (int kk = 0; kk < C::KK; ++kk) qf[kk] = load16(qrow + 16 * kk + 8 * hl, qi < p.Lq);
  if (p.rope.cos)  // RoPE fused into the load: row qi at position q_pos0[b] + qi
    rope_q_lane<DTYPE, D>(qf, p.rope, (p.q_pos0 ? p.q_pos0[b] : 0) + qi, qi < p.Lq, hl);
  const float c = p.scale_log2;
#pragma unroll
  for (int kk = 0; kk < C::KK; ++kk) qf[kk] ^= u32x4{p.q_sign, p.q_sign, p.q_sign, p.q_sign};

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

  const uint16_t* kb = p.k + b * p.ks0 + kvh * p.ks1;
  const uint16_t* vb = p.v + b * p.vs0 + kvh * p.vs1;
  const int last_key = max(p.Lk - 1, 0);

  // Tile copy: copy j of this wave moves 16-byte chunk P = (wave*NW + j)*64 + lane
  // of the tile, i.e. row P / S, chunk (P % S) XOR chunk_swizzle(row). Rows
  // past the last key are clamped to it (masked as scores, zero weight in P.V).
  int lrow[C::NW], lchk[C::NW];
#pragma unroll
  for (int j = 0; j < C::NW; ++j) {
    const int P = (wave * C::NW + j) * 64 + lane;
    lrow[j] = P / C::S;
    lchk[j] = 8 * ((P % C::S) ^ chunk_swizzle<C::S>(lrow[j]));
  }
  // Byte offsets of this lane's chunks from the first key of a tile; full
  // tiles add them to a scalar tile base (no per-lane address math), the
  // key-tail tile clamps rows to the last key.
  const bool off32 = (int64_t)BN * max(p.ks2, p.vs2) * 2 + 2 * D < ((int64_t)1 << 31);
  uint32_t koff[C::NW], voff[C::NW];
#pragma unroll
  for (int j = 0; j < C::NW; ++j) {
    koff[j] = off32 ? (uint32_t)(2 * ((int64_t)lrow[j] * p.ks2 + lchk[j])) : 0u;
    voff[j] = off32 ? (uint32_t)(2 * ((int64_t)lrow[j] * p.vs2 + lchk[j])) : 0u;
  }
  const uint32_t ring_lds = lds_addr_of(ring);
  auto issue = [&](int t) CIE_INLINE {
    const int n0 = t * BN;
    const uint32_t st = ring_lds + 2u * (uint32_t)((t % C::NST) * C::STAGE + wave * C::NW * 512);
    if (off32 && n0 + BN <= p.Lk) {
      const void* kt = uniform_ptr(kb + (int64_t)n0 * p.ks2);
      const void* vt = uniform_ptr(vb + (int64_t)n0 * p.vs2);
#pragma unroll
      for (int j = 0; j < C::NW; ++j) {
        dma16_sv(kt, koff[j], st + 1024u * j);
        dma16_sv(vt, voff[j], st + 2u * C::TILE + 1024u * j);
      }
    } else {
#pragma unroll
      for (int j = 0; j < C::NW; ++j) {
        const int key = min(n0 + lrow[j], last_key);
        dma16_at(kb + (int64_t)key * p.ks2 + lchk[j], st + 1024u * j);
        dma16_at(vb + (int64_t)key * p.vs2 + lchk[j], st + 2u * C::TILE + 1024u * j);
      }
    }
  };

  // S^T of tile t from its ring stage (rows past the tile data are finite
  // copies of the last key or stale LDS; the caller masks or discards them).
  auto qk = [&](int t, f32x16* s) CIE_INLINE {
    const uint16_t* ks = ring + (t % C::NST) * C::STAGE;
#pragma unroll
    for (int mt2 = 0; mt2 < C::MT; ++mt2) s[mt2] = f32x16{};
#pragma unroll
    for (int kk = 0; kk < C::KK; ++kk) {
#pragma unroll
      for (int mt2 = 0; mt2 < C::MT; ++mt2) {
        const int row = 32 * mt2 + l32;
        const int sl = (2 * kk + hl) ^ chunk_swizzle<C::S>(row);
        const u32x4 a = *reinterpret_cast<const u32x4*>(ks + (row * C::S + sl) * 8);
        s[mt2] = E::mfma(a, qf[kk], s[mt2]);
      }
    }
  };
  // Bottom-right causal / key-tail mask of tile t (only tiles that cross the
  // smallest visible limit of the wave need it).
  auto mask = [&](int t, f32x16* s) CIE_INLINE {
    const int n0 = t * BN;
    if (n0 + BN - 1 > wave_lim0) {
#pragma unroll
      for (int mt2 = 0; mt2 < C::MT; ++mt2)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int key = n0 + 32 * mt2 + 8 * (e >> 2) + 4 * hl + (e & 3);
          s[mt2][e] = key <= lim ? s[mt2][e] : -INFINITY;
        }
    }
  };
  auto rowmax = [&](const f32x16* s) CIE_INLINE {
    float mx = max16(s[0]);
#pragma unroll
    for (int mt2 = 1; mt2 < C::MT; ++mt2) mx = maxf(mx, max16(s[mt2]));
    return mx;
  };

  f32x16 acc[C::DT];
#pragma unroll
  for (int dt = 0; dt < C::DT; ++dt) acc[dt] = f32x16{};
  // m: the row's reference max in the exp2 domain (c * s), -inf until the
  // row has a visible key; nm = -m, or 0 while m is -inf.
  float m = -INFINITY, l = 0.f, nm = 0.f;
  auto set_m = [&](float x) CIE_INLINE {
    m = x;
    nm = x == -INFINITY ? 0.f : -x;
  };
  // Row sums of P: 4x4x4 MFMAs (16 blocks) with A all ones add four packed
  // p of a lane into that lane's accumulator and nothing else (a p that is
  // inf or NaN stays in its row); two chains, then one cross-lane add per
  // tile for the row.
  const u32x2 sum_ones = {E::pack2(1.f, 1.f), E::pack2(1.f, 1.f)};

  vm_wait<0>();  // Q is in registers before the copies start (explicit waits from here on)
  const int pro = min(C::NST - 1, n_tiles);
  for (int t = 0; t < pro; ++t) issue(t);

  // Software pipeline: iteration t holds S(t) in registers, computes
  // S(t+1) = K(t+1) Q^T while turning S(t) into P(t), then O += V(t) P(t),
  // so tiles t and t+1 are read. Each step (four stages; three at D=256)
  // waits for tile t+1, the barrier publishes it, and the stage of tile t-1
  // is refilled.
  f32x16 sc[C::MT];
  if (n_tiles > 0) {
    wait_ahead<C::NST, C::PER_TILE>(pro - 1);
    __syncthreads();
    qk(0, sc);
    mask(0, sc);
    set_m(xhalf_max(rowmax(sc)) * c);  // the reference max starts at tile 0's row max
  }
  const int rq = lane & 15, gq = lane >> 4;  // transpose-read lane coordinates
  // One pipeline step: sc holds S(t), S(t+1) is produced in sn; ST is the
  // ring stage of tile t (t % NST). The loop below runs U steps per trip with
  // the two score arrays swapped each step, so the scores are never copied
  // between registers.
  auto step = [&](auto ST, const int t, f32x16* sc, f32x16* sn) CIE_INLINE {
    constexpr int st = decltype(ST)::value, st1 = (st + 1) % C::NST;
    if (t + 1 < n_tiles) {
      wait_ahead<C::NST, C::PER_TILE>(min(C::NST - 3, n_tiles - 2 - t));
      __syncthreads();  // tile t+1 resident for all waves; stage of tile t-1 free
      if (t + C::NST - 1 < n_tiles) issue(t + C::NST - 1);
    }
    if (t * BN >= wave_kend) return;  // wave-uniform: every row of the wave is done

    // (c) S(t+1) on the MFMA pipe, P(t) on the VALU, interleaved by hand:
    // after each QK MFMA the next EPC elements of S(t) become probabilities.
    // sched_barrier(0) keeps the compiler from regrouping the MFMAs. For the
    // last tile the stage read is stale and S(t+1) is discarded. The empty
    // volatile asm consumes each packed pair inside its chunk; without it the
    // softmax would be sunk next to the P.V MFMAs that use it.
    // Raised wave priority for this phase: with two waves per SIMD, the wave
    // turning S(t) into P(t) next to its QK MFMAs issues first and the other
    // wave's P.V phase fills the gaps (measured 4-5 % faster at D=64).
    __builtin_amdgcn_s_setprio(1);
    u32x4 pb[2 * C::MT];
    f32x4 tsm[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};  // this lane's sums of the tile's p
    {
      const uint16_t* ks = ring + st1 * C::STAGE;
      u32x4 ka[C::NQK];
#pragma unroll
      for (int i = 0; i < C::NQK; ++i) {
        const int kk = i / C::MT, mt2 = i % C::MT;
        const int row = 32 * mt2 + l32;
        const int sl = (2 * kk + hl) ^ chunk_swizzle<C::S>(row);
        ka[i] = *reinterpret_cast<const u32x4*>(ks + (row * C::S + sl) * 8);
      }
#pragma unroll
      for (int mt2 = 0; mt2 < C::MT; ++mt2) sn[mt2] = f32x16{};
      constexpr int EPC = 16 * C::MT / C::NQK;  // S(t) elements per MFMA
#pragma unroll
      for (int i = 0; i < C::NQK; ++i) {
        const int kk = i / C::MT, mt2 = i % C::MT;
        sn[mt2] = E::mfma(ka[i], qf[kk], sn[mt2]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int e = i * EPC; e < (i + 1) * EPC; ++e) {
          const int m2 = e / 16, ee = e % 16;
          sc[m2][ee] = exp2_fast(fmaf(sc[m2][ee], c, nm));
          if (ee & 1) {  // a pair is complete: pack it
            const uint32_t pk = E::pack2(sc[m2][ee - 1], sc[m2][ee]);
            asm volatile("" ::"v"(pk));  // pin the work of this chunk next to its MFMA
            pb[2 * m2 + (ee >> 3)][(ee & 7) >> 1] = pk;
          }
          // four p of P(t) are packed: their sum on the matrix pipe (a DOT
          // instruction per pair would wait for the pipe to drain)
          if ((ee & 3) == 3) {
            const int cb = 2 * m2 + (ee >> 3), w = (ee & 7) >> 1;
            tsm[(ee >> 2) & 1] = E::mfma4(sum_ones, u32x2{pb[cb][w - 1], pb[cb][w]}, tsm[(ee >> 2) & 1]);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }

    __builtin_amdgcn_s_setprio(0);

    // Slow path of the lazy max (rare: a row's max rose by ~2^5 or more, or
    // its first visible key): S(t) again from the resident K tile, m raised
    // to the row max, accumulators rescaled, the tile's p recomputed.
    float ts = xhalf_sum(tsm[0][0] + tsm[1][0]);  // the row's sum of the tile's p
    if (__builtin_amdgcn_ballot_w64(!(ts <= kSumTrigger))) {
      qk(t, sc);
      mask(t, sc);
      const float m_old = m;
      set_m(maxf(m, xhalf_max(rowmax(sc)) * c));
      const float alpha = m > m_old ? exp2_fast(m_old - m) : 1.f;  // 0 when m was -inf
      l *= alpha;
#pragma unroll
      for (int dt = 0; dt < C::DT; ++dt) acc[dt] *= alpha;
#pragma unroll
      for (int e = 0; e < 16 * C::MT; e += 2) {
        const int m2 = e / 16, ee = e % 16;
        pb[2 * m2 + (ee >> 3)][(ee & 7) >> 1] =
            E::pack2(exp2_fast(fmaf(sc[m2][ee], c, nm)), exp2_fast(fmaf(sc[m2][ee + 1], c, nm)));
      }
      tsm[0] = tsm[1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int cc = 0; cc < 2 * C::MT; ++cc) {
        tsm[0] = E::mfma4(sum_ones, u32x2{pb[cc][0], pb[cc][1]}, tsm[0]);
        tsm[1] = E::mfma4(sum_ones, u32x2{pb[cc][2], pb[cc][3]}, tsm[1]);
      }
      ts = xhalf_sum(tsm[0][0] + tsm[1][0]);
    }
    l += ts;
    mask(t + 1, sn);

    // (d) O += V(t) P(t) on the MFMA pipe.
    {
      const uint16_t* vs = ring + st * C::STAGE + C::TILE;
      u32x4 va[C::NPV];
#pragma unroll
      for (int dt = 0; dt < C::DT; ++dt) {
        int d = 32 * dt + 16 * (gq & 1) + 4 * (rq & 3);
        if (D < 32) d = min(d, D - 4);  // rows >= D of O^T are discarded
        const int chunk = d >> 3, within = d & 7;
#pragma unroll
        for (int cc = 0; cc < 2 * C::MT; ++cc) {
          const int tlo = 16 * cc + 4 * hl + (rq >> 2);
          const int thi = tlo + 8;
          const u32x2 lo = lds_read_tr16(vs + (tlo * C::S + (chunk ^ chunk_swizzle<C::S>(tlo))) * 8 + within);
          const u32x2 hi = lds_read_tr16(vs + (thi * C::S + (chunk ^ chunk_swizzle<C::S>(thi))) * 8 + within);
          va[dt * 2 * C::MT + cc] = u32x4{lo[0], lo[1], hi[0], hi[1]};
        }
      }
#pragma unroll
      for (int i = 0; i < C::NPV; ++i) {
        const int dt = i % C::DT, cc = i / C::DT;  // alternate accumulators
        acc[dt] = E::mfma(va[dt * 2 * C::MT + cc], pb[cc], acc[dt]);
      }
    }
  };
  f32x16 sb[C::MT];
  // steps per trip: stage and score buffer repeat
  constexpr int U = C::NST % 2 == 0 ? C::NST : 2 * C::NST;
  for (int t = 0; t < n_tiles; t += U) {
    static_for<U>([&](auto I) CIE_INLINE {
      constexpr int i = decltype(I)::value;
      if (t + i < n_tiles) {
        if constexpr (i % 2 == 0) step(std::integral_constant<int, i % C::NST>{}, t + i, sc, sb);
        else step(std::integral_constant<int, i % C::NST>{}, t + i, sb, sc);
      }
    });
  }

  // Epilogue: rows with keys but none visible give 0 * inf = NaN like the
  // reference's softmax over an all -inf row; Lk == 0 gives zeros.
  const float l_tot = l;  // l sums both lanes of the row
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

// ---------------------------------------------------------------------------
// Interleaved kernel (head_dim 128; the configuration also covers 64).
//
// Same copies, lazy running max and causal rule as flash_fwd_kernel, with
// two changes to what a wave issues per tile:
//  * one pipeline step t issues S(t+1) = K(t+1) Q^T (QK MFMAs), O += V(t-1)
//    P(t-1) (P.V MFMAs, one tile behind) and the softmax of S(t) (exp2 and
//    packing on the VALU) as one stream, MFMA and VALU work alternating in a
//    fixed ratio, so the VALU work of one wave overlaps the MFMAs of both
//    waves of its SIMD;
//  * the row sums of the rounded probabilities come from 4x4x4 MFMAs with
//    A all ones (no DOT instruction: those wait for the matrix pipe), each
//    lane's own values only, then one cross-lane add for the row.
// The slow path of the lazy max acts on the rows that triggered it only, so
// a row's arithmetic does not depend on the other rows of its wave.
// P.V one tile behind keeps V(t-1) resident one step longer: the ring holds
// tiles t-1, t, t+1 while step t runs (K(t) for the slow path).
template <int D>
struct IlCfg {
  static constexpr int BM = 128;                 // query rows per workgroup
  static constexpr int BN = D == 64 ? 64 : 32;   // keys per tile
  static constexpr int S = D / 8;                // 16-byte chunks per row
  static constexpr int DT = D / 32;              // 32-row output tiles
  static constexpr int KK = D / 16;              // MFMA steps over head_dim
  static constexpr int MT = BN / 32;             // 32-key score tiles
  static constexpr int NCC = 2 * MT;             // 16-key blocks of P per tile
  static constexpr int TILE = BN * D;
  static constexpr int STAGE = 2 * TILE;         // K tile, then V tile
  static constexpr int NST = 4;                  // ring stages (one tile in flight; S=16384 1760 -> 1744 us against five)
  static constexpr int AHEAD = NST - 3;          // tiles in flight behind the one a barrier publishes
  static constexpr int NW = BN * S / 256;        // 1 KiB copies per wave per tensor
  static constexpr int PER_TILE = 2 * NW;
  static constexpr int NQK = KK * MT;            // QK^T MFMAs per tile
  static constexpr int NPV = DT * NCC;           // P.V MFMAs per tile
  static constexpr int NE = 16 * MT;             // scores per lane per tile
  static constexpr int EPC = NE / (2 * NQK);     // scores per VALU chunk
  static_assert(NQK == NPV, "QK and P.V MFMAs alternate one for one");
  static_assert(EPC >= 1 && EPC * 2 * NQK == NE, "softmax chunks must split evenly");
  static_assert(NW * 256 == BN * S, "tile must split evenly over 4 waves");
};

// vm_wait for the copies of k tiles (0 <= k <= KMAX) issued after the one needed.
template <int PER_TILE, int KMAX>
__device__ __forceinline__ void wait_tiles(int k) {
  if constexpr (KMAX >= 2) {
    if (k >= 2) {
      vm_wait<2 * PER_TILE>();
      return;
    }
  }
  if constexpr (KMAX >= 1) {
    if (k == 1) {
      vm_wait<PER_TILE>();
      return;
    }
  }
  vm_wait<0>();
}

template <int DTYPE, int D>
__global__ __launch_bounds__(256, 2) void flash_fwd_il_kernel(const FlashParams p) {
  using C = IlCfg<D>;
  using E = Elt<DTYPE>;
  constexpr int BN = C::BN;
  __shared__ __attribute__((aligned(16))) uint16_t ring[C::NST * C::STAGE];

  const int logical = xcd_logical(blockIdx.x, p.n_wg, p.xcd_shift);
  const int G = p.group;
  const int per_grp = p.n_mt * G;
  const int grp = logical / per_grp;
  const int rem = logical - grp * per_grp;
  const int mt = p.n_mt - 1 - rem / G;
  const int g = rem - (rem / G) * G;
  const int b = grp / p.Hk, kvh = grp - b * p.Hk, hq = kvh * G + g;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hl = lane >> 5;
  const int q0w = mt * C::BM + wave * 32;
  const int qi = q0w + l32;

  const uint16_t* qrow = p.q + b * p.qs0 + hq * p.qs1 + (int64_t)qi * p.qs2;
  u32x4 qf[C::KK];
#pragma unroll
  for (int kk = 0; kk < C::KK; ++kk) qf[kk] = load16(qrow + 16 * kk + 8 * hl, qi < p.Lq);
  if (p.rope.cos) rope_q_lane<DTYPE, D>(qf, p.rope, (p.q_pos0 ? p.q_pos0[b] : 0) + qi, qi < p.Lq, hl);
#pragma unroll
  for (int kk = 0; kk < C::KK; ++kk) qf[kk] ^= u32x4{p.q_sign, p.q_sign, p.q_sign, p.q_sign};
  const float c = p.scale_log2;

  const int wg_last_row = min(p.Lq, mt * C::BM + C::BM) - 1;
  int kend = p.Lk;
  if (p.causal) kend = max(0, min(p.Lk, p.Lk - p.Lq + wg_last_row + 1));
  int wave_kend = 0;
  if (q0w < p.Lq) {
    wave_kend = p.Lk;
    if (p.causal) wave_kend = max(0, min(p.Lk, p.Lk - p.Lq + min(q0w + 31, p.Lq - 1) + 1));
  }
  const int lim = p.causal ? min(p.Lk - 1, p.Lk - p.Lq + qi) : p.Lk - 1;
  const int wave_lim0 = p.causal ? min(p.Lk - 1, p.Lk - p.Lq + q0w) : p.Lk - 1;
  const int n_tiles = (kend + BN - 1) / BN;
  const int wave_nt = (wave_kend + BN - 1) / BN;  // tiles this wave needs (0: no rows)

  const uint16_t* kb = p.k + b * p.ks0 + kvh * p.ks1;
  const uint16_t* vb = p.v + b * p.vs0 + kvh * p.vs1;
  const int last_key = max(p.Lk - 1, 0);

  int lrow[C::NW], lchk[C::NW];
#pragma unroll
  for (int j = 0; j < C::NW; ++j) {
    const int P = (wave * C::NW + j) * 64 + lane;
    lrow[j] = P / C::S;
    lchk[j] = 8 * ((P % C::S) ^ chunk_swizzle<C::S>(lrow[j]));
  }
  const bool off32 = (int64_t)BN * max(p.ks2, p.vs2) * 2 + 2 * D < ((int64_t)1 << 31);
  uint32_t koff[C::NW], voff[C::NW];
#pragma unroll
  for (int j = 0; j < C::NW; ++j) {
    koff[j] = off32 ? (uint32_t)(2 * ((int64_t)lrow[j] * p.ks2 + lchk[j])) : 0u;
    voff[j] = off32 ? (uint32_t)(2 * ((int64_t)lrow[j] * p.vs2 + lchk[j])) : 0u;
  }
  const uint32_t ring_lds = lds_addr_of(ring);
  auto issue = [&](int t) CIE_INLINE {
    const int n0 = t * BN;
    const uint32_t st = ring_lds + 2u * (uint32_t)((t % C::NST) * C::STAGE + wave * C::NW * 512);
    if (off32 && n0 + BN <= p.Lk) {
      const void* kt = uniform_ptr(kb + (int64_t)n0 * p.ks2);
      const void* vt = uniform_ptr(vb + (int64_t)n0 * p.vs2);
#pragma unroll
      for (int j = 0; j < C::NW; ++j) {
        dma16_sv(kt, koff[j], st + 1024u * j);
        dma16_sv(vt, voff[j], st + 2u * C::TILE + 1024u * j);
      }
    } else {
#pragma unroll
      for (int j = 0; j < C::NW; ++j) {
        const int key = min(n0 + lrow[j], last_key);
        dma16_at(kb + (int64_t)key * p.ks2 + lchk[j], st + 1024u * j);
        dma16_at(vb + (int64_t)key * p.vs2 + lchk[j], st + 2u * C::TILE + 1024u * j);
      }
    }
  };

  // K fragment (head_dim step kk, 32-key score tile mt2) of the tile in stage ks.
  auto kfrag = [&](const uint16_t* ks, int kk, int mt2) CIE_INLINE {
    const int row = 32 * mt2 + l32;
    const int sl = (2 * kk + hl) ^ chunk_swizzle<C::S>(row);
    return *reinterpret_cast<const u32x4*>(ks + (row * C::S + sl) * 8);
  };
  // S^T of the tile in stage ks.
  auto qk = [&](const uint16_t* ks, f32x16* s) CIE_INLINE {
#pragma unroll
    for (int mt2 = 0; mt2 < C::MT; ++mt2) s[mt2] = f32x16{};
#pragma unroll
    for (int kk = 0; kk < C::KK; ++kk)
#pragma unroll
      for (int mt2 = 0; mt2 < C::MT; ++mt2) s[mt2] = E::mfma(kfrag(ks, kk, mt2), qf[kk], s[mt2]);
  };
  // Element e of score tile mt2 in a lane is key n0 + 32 mt2 + 4 hl + 8 (e / 4)
  // + e % 4: the test key <= lim compares one per-lane value with a constant.
  auto mask = [&](int t, f32x16* s) CIE_INLINE {
    const int n0 = t * BN;
    if (n0 + BN - 1 > wave_lim0) {
      const int r = lim - n0 - 4 * hl;
#pragma unroll
      for (int mt2 = 0; mt2 < C::MT; ++mt2)
#pragma unroll
        for (int e = 0; e < 16; ++e) s[mt2][e] = 32 * mt2 + 8 * (e >> 2) + (e & 3) <= r ? s[mt2][e] : -INFINITY;
    }
  };
  auto rowmax = [&](const f32x16* s) CIE_INLINE {
    float mx = max16(s[0]);
#pragma unroll
    for (int mt2 = 1; mt2 < C::MT; ++mt2) mx = maxf(mx, max16(s[mt2]));
    return xhalf_max(mx);
  };
  // V^T fragment (output tile dt, 16-key block cc) of the tile in stage vs.
  const int rq = lane & 15, gq = lane >> 4;
  auto vfrag = [&](const uint16_t* vs, int dt, int cc) CIE_INLINE {
    const int d = 32 * dt + 16 * (gq & 1) + 4 * (rq & 3);
    const int chunk = d >> 3, within = d & 7;
    const int tlo = 16 * cc + 4 * hl + (rq >> 2);
    const int thi = tlo + 8;
    const u32x2 lo = lds_read_tr16(vs + (tlo * C::S + (chunk ^ chunk_swizzle<C::S>(tlo))) * 8 + within);
    const u32x2 hi = lds_read_tr16(vs + (thi * C::S + (chunk ^ chunk_swizzle<C::S>(thi))) * 8 + within);
    return u32x4{lo[0], lo[1], hi[0], hi[1]};
  };

  f32x16 acc[C::DT];
#pragma unroll
  for (int dt = 0; dt < C::DT; ++dt) acc[dt] = f32x16{};
  // m: the row's reference max in the exp2 domain (c * s); nm = -m, or 0
  // while m is -inf. l: the row's sum over both lanes.
  float m = -INFINITY, l = 0.f, nm = 0.f;
  auto set_m = [&](float x) CIE_INLINE {
    m = x;
    nm = x == -INFINITY ? 0.f : -x;
  };
  // Row sums of P: 4x4x4 MFMAs with A all ones (see flash_fwd_kernel).
  const u32x2 sum_ones = {E::pack2(1.f, 1.f), E::pack2(1.f, 1.f)};

  vm_wait<0>();  // q (and RoPE tables) in registers before the copies start
  const int pro = min(C::AHEAD + 1, n_tiles);
  for (int t = 0; t < pro; ++t) issue(t);

  f32x16 sA[C::MT], sB[C::MT];
  u32x4 pA[C::NCC], pB[C::NCC];
  if (n_tiles > 0) {
    wait_tiles<C::PER_TILE, C::AHEAD>(pro - 1);
    __syncthreads();
    qk(ring, sA);
    mask(0, sA);
    set_m(rowmax(sA) * c);  // the reference max starts at tile 0's row max
  }

  // Lazy-max check of tile tc (its P in pq, its row sum of p in ts; K(tc)
  // in stage kst). A row whose sum passed 2^10 (some p may not fit the
  // 16-bit P.V operand; always the case for a row that had no visible key
  // before) recomputes S(tc) from the resident K tile, raises m to its row
  // max, rescales O and l, and redoes its p; the other rows keep theirs.
  auto check = [&](const int tc, const uint16_t* kst, u32x4* pq, float ts) CIE_INLINE {
    const bool trig = !(ts <= kSumTrigger);
    if (__builtin_amdgcn_ballot_w64(trig)) {
      f32x16 s2[C::MT];
      qk(kst, s2);
      mask(tc, s2);
      const float mx = rowmax(s2) * c;
      const float m_old = m;
      if (trig) set_m(maxf(m_old, mx));
      const float alpha = m > m_old ? exp2_fast(m_old - m) : 1.f;  // 0 when m was -inf
      l *= alpha;
#pragma unroll
      for (int dt = 0; dt < C::DT; ++dt) acc[dt] *= alpha;
#pragma unroll
      for (int e = 0; e < C::NE; e += 2) {
        const int m2 = e / 16, ee = e % 16;
        const uint32_t w = pq[2 * m2 + (ee >> 3)][(ee & 7) >> 1];
        pq[2 * m2 + (ee >> 3)][(ee & 7) >> 1] =
            trig ? E::pack2(exp2_fast(fmaf(s2[m2][ee], c, nm)), exp2_fast(fmaf(s2[m2][ee + 1], c, nm))) : w;
      }
      f32x4 t2[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
      for (int cc = 0; cc < C::NCC; ++cc) {
        t2[0] = E::mfma4(sum_ones, u32x2{pq[cc][0], pq[cc][1]}, t2[0]);
        t2[1] = E::mfma4(sum_ones, u32x2{pq[cc][2], pq[cc][3]}, t2[1]);
      }
      const float ts2 = xhalf_sum(t2[0][0] + t2[1][0]);
      if (trig) ts = ts2;
    }
    l += ts;
  };

  // One pipeline step t: ST = t % NST, PV = t > 0. sc = S(t), sn receives
  // S(t+1), pb receives P(t), pp holds P(t-1).
  auto step = [&](auto ST, auto PV, const int t, f32x16* sc, f32x16* sn, u32x4* pb, u32x4* pp) CIE_INLINE {
    constexpr int st = decltype(ST)::value;
    constexpr int st1 = (st + 1) % C::NST, stp = (st + C::NST - 1) % C::NST;
    constexpr bool has_pv = decltype(PV)::value;
    if (t + 1 < n_tiles) {
      // tile t+1 resident for all waves; the stage of tile t-2 is free (its
      // last reads were in step t-1)
      wait_tiles<C::PER_TILE, C::AHEAD - 1>(min(n_tiles - 1, t + C::AHEAD) - (t + 1));
      __syncthreads();
      if (t + C::AHEAD + 1 < n_tiles) issue(t + C::AHEAD + 1);
    }
    // A wave works on tiles [0, wave_nt); step wave_nt only finishes P.V of
    // its last tile (its S(t) is fully masked: p = 0).
    if (wave_nt == 0 || t > wave_nt) return;

    const uint16_t* ks = ring + st1 * C::STAGE;
    const uint16_t* vs = ring + stp * C::STAGE + C::TILE;
    // Fragments are read LA MFMA pairs ahead of their use.
    constexpr int LA = 1;
    u32x4 ka[C::NQK], va[C::NPV];
    auto fetch = [&](int i) CIE_INLINE {
      ka[i] = kfrag(ks, i / C::MT, i % C::MT);
      if constexpr (has_pv) va[i] = vfrag(vs, i % C::DT, i / C::DT);
    };
#pragma unroll
    for (int i = 0; i < LA; ++i) fetch(i);
#pragma unroll
    for (int mt2 = 0; mt2 < C::MT; ++mt2) sn[mt2] = f32x16{};
    f32x4 tsum[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    // VALU chunk c: exp2 of scores [c EPC, (c + 1) EPC) of S(t) (score tile
    // e / 16, element e % 16), pairs packed into P(t); every four packed p
    // are summed by an MFMA.
    auto chunk = [&](auto CI) CIE_INLINE {
      constexpr int c0 = decltype(CI)::value;
#pragma unroll
      for (int e = c0 * C::EPC; e < (c0 + 1) * C::EPC; ++e) {
        const int m2 = e / 16, ee = e % 16;
        sc[m2][ee] = exp2_fast(fmaf(sc[m2][ee], c, nm));
        if (ee & 1) {
          const uint32_t pk = E::pack2(sc[m2][ee - 1], sc[m2][ee]);
          asm volatile("" ::"v"(pk));  // pin the work of this chunk next to its MFMA
          pb[2 * m2 + (ee >> 3)][(ee & 7) >> 1] = pk;
        }
        if ((ee & 3) == 3) {
          const int cb = 2 * m2 + (ee >> 3), w = (ee & 7) >> 1;
          tsum[(ee >> 2) & 1] = E::mfma4(sum_ones, u32x2{pb[cb][w - 1], pb[cb][w]}, tsum[(ee >> 2) & 1]);
        }
      }
    };
    // the interleaved MFMA / exp stream runs at raised wave priority and the
    // lazy-max check and masking after it at the normal one, so the SIMD's
    // other wave yields to a wave in its stream (S=16384: 1825 -> 1770 us)
    __builtin_amdgcn_s_setprio(1);
    static_for<C::NQK>([&](auto I) CIE_INLINE {
      constexpr int i = decltype(I)::value;
      if constexpr (i + LA < C::NQK) fetch(i + LA);
      sn[i % C::MT] = E::mfma(ka[i], qf[i / C::MT], sn[i % C::MT]);
      __builtin_amdgcn_sched_barrier(0);
      chunk(std::integral_constant<int, 2 * i>{});
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (has_pv) acc[i % C::DT] = E::mfma(va[i], pp[i / C::DT], acc[i % C::DT]);
      __builtin_amdgcn_sched_barrier(0);
      chunk(std::integral_constant<int, 2 * i + 1>{});
      __builtin_amdgcn_sched_barrier(0);
    });
    __builtin_amdgcn_s_setprio(0);
    check(t, ring + st * C::STAGE, pb, xhalf_sum(tsum[0][0] + tsum[1][0]));
    mask(t + 1, sn);
  };

  if (n_tiles > 0) step(std::integral_constant<int, 0>{}, std::false_type{}, 0, sA, sB, pA, pB);
  constexpr int U = 2 * C::NST;  // stage and buffer parity repeat
  for (int t = 1; t < n_tiles; t += U) {
    static_for<U>([&](auto I) CIE_INLINE {
      constexpr int i = decltype(I)::value;
      constexpr int st = (1 + i) % C::NST;
      if (t + i < n_tiles) {
        if constexpr ((1 + i) % 2 == 1)
          step(std::integral_constant<int, st>{}, std::true_type{}, t + i, sB, sA, pB, pA);
        else
          step(std::integral_constant<int, st>{}, std::true_type{}, t + i, sA, sB, pA, pB);
      }
    });
  }
  // P.V of the last tile when no further step ran it.
  if (wave_nt > 0 && wave_nt == n_tiles) {
    const int tl = n_tiles - 1;
    const uint16_t* vs = ring + (tl % C::NST) * C::STAGE + C::TILE;
    auto fin = [&](const u32x4* pq) CIE_INLINE {
      u32x4 va[C::NPV];
#pragma unroll
      for (int i = 0; i < C::NPV; ++i) va[i] = vfrag(vs, i % C::DT, i / C::DT);
#pragma unroll
      for (int i = 0; i < C::NPV; ++i) acc[i % C::DT] = E::mfma(va[i], pq[i / C::DT], acc[i % C::DT]);
    };
    if (tl & 1) fin(pB);
    else fin(pA);
  }

  // Epilogue: rows with keys but none visible give 0 * inf = NaN like the
  // reference's softmax over an all -inf row; Lk == 0 gives zeros.
  const float inv = p.Lk == 0 ? 0.f : 1.f / l;
  if (qi < p.Lq) {
    uint16_t* orow = p.o + b * p.os0 + hq * p.os1 + (int64_t)qi * p.os2;
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) {
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d = 32 * dt + 8 * g4 + 4 * hl;
        const u32x2 w = {E::pack2(acc[dt][4 * g4] * inv, acc[dt][4 * g4 + 1] * inv),
                         E::pack2(acc[dt][4 * g4 + 2] * inv, acc[dt][4 * g4 + 3] * inv)};
        *reinterpret_cast<u32x2*>(orow + d) = w;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Two row groups per wave (head_dim 64).
//
// Each wave owns two groups of 32 query rows and streams 32-key tiles: every
// K fragment read from LDS feeds the QK^T MFMAs of both groups and every V^T
// fragment the P.V MFMAs of both, so a tile's LDS reads, copies and barrier
// serve twice the MFMA work of flash_fwd_kernel's 32-row waves. HEADS: the
// groups are the same 32 rows of two query heads that share the kv head
// (128-row workgroups; a wave's causal span stays 32 rows); otherwise they
// are rows q0w + 32 rg + l32 of one head (256-row workgroups). Per tile and
// wave: 8 QK^T MFMAs, 32 fma + exp2 per lane, 8 P.V MFMAs. The
// copies, causal rule and lazy max are those of flash_fwd_kernel; the slow
// path acts on the rows that triggered it only (as in flash_fwd_il_kernel).
template <int D, bool HEADS>
struct R64Cfg {
  static constexpr int RW = HEADS ? 32 : 64;   // query rows per wave
  static constexpr int BM = 4 * RW;            // query rows per workgroup
  static constexpr int NRG = 2;                // 32-row groups per wave
  static constexpr int BN = 32;                // keys per tile
  static constexpr int S = D / 8;              // 16-byte chunks per row
  static constexpr int DT = D / 32;            // 32-row output tiles
  static constexpr int KK = D / 16;            // MFMA steps over head_dim
  static constexpr int TILE = BN * D;
  static constexpr int STAGE = 2 * TILE;       // K tile, then V tile
  static constexpr int NST = 4;                // ring stages (measured against 6 and 8: 2 % faster)
  static constexpr int NW = BN * S / 256;      // 1 KiB copies per wave per tensor
  static constexpr int PER_TILE = 2 * NW;
  static constexpr int NQK = KK * NRG;         // QK^T MFMAs per tile
  static constexpr int EPC = 16 * NRG / NQK;   // S(t) elements per QK MFMA
  static_assert(D == 64, "two row groups per wave fit the registers at head_dim 64");
  static_assert(NW * 256 == BN * S, "tile must split evenly over 4 waves");
  static_assert(EPC * NQK == 16 * NRG, "softmax chunks must split evenly");
};


template <int DTYPE, int D, bool HEADS>
__global__ __launch_bounds__(256, 2) void flash_fwd_r64_kernel(const FlashParams p) {
  CIE_STAMP(flash_timeline, 0);  // entry
  CIE_STAMP_WHERE(flash_timeline, 5);
  warm_kernargs<sizeof(FlashParams)>();
  using C = R64Cfg<D, HEADS>;
  using E = Elt<DTYPE>;
  constexpr int BN = C::BN, NRG = C::NRG;
  __shared__ __attribute__((aligned(16))) uint16_t ring[C::NST * C::STAGE];

  // p.n_mt counts BM-row query tiles here and a work item is one query
  // tile of one head (of a pair of heads with HEADS; see launch_flash_t).
  // Each XCD takes a contiguous run of items (whole kv heads when the run
  // divides evenly) and dispatches it longest first across all of its kv
  // heads: items are few and long here, and kv-head-major order left long
  // items for the end of the run.
  const int N = p.n_wg, xmask = (1 << p.xcd_shift) - 1;
  const int xcd = blockIdx.x & xmask, slot = blockIdx.x >> p.xcd_shift;
  const int x0 = xcd * (N >> p.xcd_shift) + min(xcd, N & xmask);    // first item of the run
  const int cnt = (N >> p.xcd_shift) + (xcd < (N & xmask) ? 1 : 0);  // items of the run (slot < cnt)
  const int G = p.group, GI = HEADS ? G / 2 : G;
  const int per_grp = p.n_mt * GI;                            // items per kv head
  int grp, mt, g;
  if (x0 % per_grp == 0 && cnt % per_grp == 0) {
    const int width = (cnt / per_grp) * GI;                   // items per query tile in the run
    const int rank = slot / width, r2 = slot - rank * width;
    grp = x0 / per_grp + r2 / GI;
    g = r2 - (r2 / GI) * GI;
    mt = p.n_mt - 1 - rank;
  } else {
    const int logical = x0 + slot;
    grp = logical / per_grp;
    const int rem = logical - grp * per_grp;
    mt = p.n_mt - 1 - rem / GI;
    g = rem - (rem / GI) * GI;
  }
  const int b = grp / p.Hk, kvh = grp - b * p.Hk;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hl = lane >> 5;
  const int q0w = mt * C::BM + wave * C::RW;  // first row of this wave
  int qi[NRG], hq[NRG];                        // rows and heads owned by this lane
#pragma unroll
  for (int rg = 0; rg < NRG; ++rg) {
    qi[rg] = q0w + (HEADS ? 0 : 32 * rg) + l32;
    hq[rg] = HEADS ? kvh * G + 2 * g + rg : kvh * G + g;
  }

  // q rows as loaded, sign flipped when the caller's scale is negative
  u32x4 qf[NRG][C::KK];
  const float c = p.scale_log2;
  const u32x4 qsg = {p.q_sign, p.q_sign, p.q_sign, p.q_sign};
  {
    if (!p.rope.cos) {
#pragma unroll
      for (int rg = 0; rg < NRG; ++rg) {
        const uint16_t* qrow = p.q + b * p.qs0 + hq[rg] * p.qs1 + (int64_t)qi[rg] * p.qs2;
#pragma unroll
        for (int kk = 0; kk < C::KK; ++kk) qf[rg][kk] = load16(qrow + 16 * kk + 8 * hl, qi[rg] < p.Lq) ^ qsg;
      }
    } else {
      // With RoPE every q load of the lane is issued first (rows clamped into
      // the tensor, rows past Lq zeroed after the load, no branch), then the
      // rotary table chunks of its rows (read once with HEADS: both row
      // groups are the same positions), so the prologue waits for one round
      // trip instead of one per row group and table read (fused-RoPE
      // prefill_s2048: 83.4 -> 82.1 us; without RoPE the per-row-group loads
      // above measured 1 % faster).
      bool live[NRG];
#pragma unroll
      for (int rg = 0; rg < NRG; ++rg) {
        live[rg] = qi[rg] < p.Lq;
        // (this kernel runs only with Lq > 128, so row Lq - 1 exists)
        const uint16_t* qrow = p.q + b * p.qs0 + hq[rg] * p.qs1 + (int64_t)min(qi[rg], p.Lq - 1) * p.qs2;
#pragma unroll
        for (int kk = 0; kk < C::KK; ++kk) qf[rg][kk] = load16_clamped(qrow + 16 * kk + 8 * hl);
      }
      constexpr int NT = HEADS ? 1 : NRG;  // distinct positions among the row groups
      const int pos0 = p.q_pos0 ? p.q_pos0[b] : 0;
      RopeChunk rc[NT][C::KK / 2];
      bool ok[NT];
#pragma unroll
      for (int r = 0; r < NT; ++r) {
        const int pos = pos0 + qi[r];
        ok[r] = pos >= 0 && pos < p.rope.rows;
        const int64_t row = ok[r] ? (int64_t)pos * (D / 2) : 0;
#pragma unroll
        for (int kk = 0; kk < C::KK / 2; ++kk) rc[r][kk] = rope_load(p.rope, row + 16 * kk + 8 * hl);
      }
#pragma unroll
      for (int rg = 0; rg < NRG; ++rg) {
        const int r = HEADS ? 0 : rg;
#pragma unroll
        for (int kk = 0; kk < C::KK / 2; ++kk)
          rope_apply8<DTYPE>(qf[rg][kk], qf[rg][kk + C::KK / 2], rc[r][kk], p.rope.dt);
#pragma unroll
        for (int kk = 0; kk < C::KK; ++kk) {
          if (!ok[r]) qf[rg][kk] = u32x4{0x7fff7fffu, 0x7fff7fffu, 0x7fff7fffu, 0x7fff7fffu};  // outside the tables: NaN
          if (!live[rg]) qf[rg][kk] = u32x4{0u, 0u, 0u, 0u};
          qf[rg][kk] ^= qsg;
        }
      }
    }
  }

  const int wg_last_row = min(p.Lq, mt * C::BM + C::BM) - 1;
  int kend = p.Lk;
  if (p.causal) kend = max(0, min(p.Lk, p.Lk - p.Lq + wg_last_row + 1));
  int wave_kend = 0;
  if (q0w < p.Lq) {
    wave_kend = p.Lk;
    if (p.causal) wave_kend = max(0, min(p.Lk, p.Lk - p.Lq + min(q0w + C::RW - 1, p.Lq - 1) + 1));
  }
  int lim[NRG];
#pragma unroll
  for (int rg = 0; rg < NRG; ++rg) lim[rg] = p.causal ? min(p.Lk - 1, p.Lk - p.Lq + qi[rg]) : p.Lk - 1;
  const int wave_lim0 = p.causal ? min(p.Lk - 1, p.Lk - p.Lq + q0w) : p.Lk - 1;  // smallest lim in the wave
  const int n_tiles = (kend + BN - 1) / BN;

  const uint16_t* kb = p.k + b * p.ks0 + kvh * p.ks1;
  const uint16_t* vb = p.v + b * p.vs0 + kvh * p.vs1;
  const int last_key = max(p.Lk - 1, 0);

  // Tile copy: as in flash_fwd_kernel (one 16-byte chunk per lane and tensor).
  int lrow[C::NW], lchk[C::NW];
#pragma unroll
  for (int j = 0; j < C::NW; ++j) {
    const int P = (wave * C::NW + j) * 64 + lane;
    lrow[j] = P / C::S;
    lchk[j] = 8 * ((P % C::S) ^ chunk_swizzle<C::S>(lrow[j]));
  }
  const bool off32 = (int64_t)BN * max(p.ks2, p.vs2) * 2 + 2 * D < ((int64_t)1 << 31);
  uint32_t koff[C::NW], voff[C::NW];
#pragma unroll
  for (int j = 0; j < C::NW; ++j) {
    koff[j] = off32 ? (uint32_t)(2 * ((int64_t)lrow[j] * p.ks2 + lchk[j])) : 0u;
    voff[j] = off32 ? (uint32_t)(2 * ((int64_t)lrow[j] * p.vs2 + lchk[j])) : 0u;
  }
  const uint32_t ring_lds = lds_addr_of(ring);
  auto issue = [&](int t) CIE_INLINE {
    const int n0 = t * BN;
    const uint32_t st = ring_lds + 2u * (uint32_t)((t % C::NST) * C::STAGE + wave * C::NW * 512);
    if (off32 && n0 + BN <= p.Lk) {
      const void* kt = uniform_ptr(kb + (int64_t)n0 * p.ks2);
      const void* vt = uniform_ptr(vb + (int64_t)n0 * p.vs2);
#pragma unroll
      for (int j = 0; j < C::NW; ++j) {
        dma16_sv(kt, koff[j], st + 1024u * j);
        dma16_sv(vt, voff[j], st + 2u * C::TILE + 1024u * j);
      }
    } else {
#pragma unroll
      for (int j = 0; j < C::NW; ++j) {
        const int key = min(n0 + lrow[j], last_key);
        dma16_at(kb + (int64_t)key * p.ks2 + lchk[j], st + 1024u * j);
        dma16_at(vb + (int64_t)key * p.vs2 + lchk[j], st + 2u * C::TILE + 1024u * j);
      }
    }
  };

  // K fragment (head_dim step kk) of the tile in stage ks: key l32 of the tile.
  auto kfrag = [&](const uint16_t* ks, int kk) CIE_INLINE {
    const int sl = (2 * kk + hl) ^ chunk_swizzle<C::S>(l32);
    return *reinterpret_cast<const u32x4*>(ks + (l32 * C::S + sl) * 8);
  };
  // S^T of both row groups from the tile in stage ks.
  auto qk = [&](const uint16_t* ks, f32x16* s) CIE_INLINE {
#pragma unroll
    for (int rg = 0; rg < NRG; ++rg) s[rg] = f32x16{};
#pragma unroll
    for (int kk = 0; kk < C::KK; ++kk) {
      const u32x4 a = kfrag(ks, kk);
#pragma unroll
      for (int rg = 0; rg < NRG; ++rg) s[rg] = E::mfma(a, qf[rg][kk], s[rg]);
    }
  };
  // Element e of a row group's scores in a lane is key n0 + 4 hl + 8 (e / 4)
  // + e % 4 of row qi[rg].
  auto mask = [&](int t, f32x16* s) CIE_INLINE {
    const int n0 = t * BN;
    if (n0 + BN - 1 > wave_lim0) {
#pragma unroll
      for (int rg = 0; rg < NRG; ++rg) {
        const int r = lim[rg] - n0 - 4 * hl;
#pragma unroll
        for (int e = 0; e < 16; ++e) s[rg][e] = 8 * (e >> 2) + (e & 3) <= r ? s[rg][e] : -INFINITY;
      }
    }
  };
  // V^T fragment (output tile dt, 16-key block cc) of the tile in stage vs.
  const int rq = lane & 15, gq = lane >> 4;
  auto vfrag = [&](const uint16_t* vs, int dt, int cc) CIE_INLINE {
    const int d = 32 * dt + 16 * (gq & 1) + 4 * (rq & 3);
    const int chunk = d >> 3, within = d & 7;
    const int tlo = 16 * cc + 4 * hl + (rq >> 2);
    const int thi = tlo + 8;
    const u32x2 lo = lds_read_tr16(vs + (tlo * C::S + (chunk ^ chunk_swizzle<C::S>(tlo))) * 8 + within);
    const u32x2 hi = lds_read_tr16(vs + (thi * C::S + (chunk ^ chunk_swizzle<C::S>(thi))) * 8 + within);
    return u32x4{lo[0], lo[1], hi[0], hi[1]};
  };

  f32x16 acc[NRG][C::DT];
#pragma unroll
  for (int rg = 0; rg < NRG; ++rg)
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) acc[rg][dt] = f32x16{};
  // m: a row's reference max in the exp2 domain (c * s); nm = -m, or 0
  // while m is -inf. l: the row's sum over both lanes.
  float m[NRG], l[NRG], nm[NRG];
  auto set_m = [&](int rg, float x) CIE_INLINE {
    m[rg] = x;
    nm[rg] = x == -INFINITY ? 0.f : -x;
  };
#pragma unroll
  for (int rg = 0; rg < NRG; ++rg) {
    set_m(rg, -INFINITY);
    l[rg] = 0.f;
  }
  // Row sums of P: 4x4x4 MFMAs with A all ones (see flash_fwd_kernel).
  const u32x2 sum_ones = {E::pack2(1.f, 1.f), E::pack2(1.f, 1.f)};

  vm_wait<0>();  // q (and RoPE tables) in registers before the copies start
  CIE_STAMP(flash_timeline, 6);  // q in registers
  const int pro = min(C::NST - 1, n_tiles);
  for (int t = 0; t < pro; ++t) issue(t);

  f32x16 sc[NRG];
  if (n_tiles > 0) {
    wait_tiles<C::PER_TILE, 2>(pro - 1);
    __syncthreads();
    CIE_STAMP(flash_timeline, 7);  // first K/V tile in LDS
    qk(ring, sc);
    mask(0, sc);
#pragma unroll
    for (int rg = 0; rg < NRG; ++rg) set_m(rg, xhalf_max(max16(sc[rg])) * c);  // the reference max starts at tile 0's row max
  }

  // One pipeline step: sc holds S(t), S(t+1) is produced in sn; ST is the
  // ring stage of tile t.
  auto step = [&](auto ST, const int t, f32x16* sc, f32x16* sn) CIE_INLINE {
    constexpr int st = decltype(ST)::value, st1 = (st + 1) % C::NST;
    if (t + 1 < n_tiles) {
      wait_tiles<C::PER_TILE, 2>(min(C::NST - 3, n_tiles - 2 - t));
      __syncthreads();  // tile t+1 resident for all waves; stage of tile t-1 free
      if (t + C::NST - 1 < n_tiles) issue(t + C::NST - 1);
    }
    if (t * BN >= wave_kend) return;  // wave-uniform: every row of the wave is done

    // S(t+1) on the MFMA pipe, P(t) on the VALU (as in flash_fwd_kernel).
    __builtin_amdgcn_s_setprio(1);
    u32x4 pb[NRG][2];                 // P(t): row group, 16-key block
    f32x4 tsm[NRG];                   // this lane's sums of the tile's p
    {
      const uint16_t* ks = ring + st1 * C::STAGE;
      u32x4 ka[C::KK];
#pragma unroll
      for (int kk = 0; kk < C::KK; ++kk) ka[kk] = kfrag(ks, kk);
#pragma unroll
      for (int rg = 0; rg < NRG; ++rg) {
        sn[rg] = f32x16{};
        tsm[rg] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int i = 0; i < C::NQK; ++i) {
        const int kk = i / NRG, rgq = i % NRG;
        sn[rgq] = E::mfma(ka[kk], qf[rgq][kk], sn[rgq]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int e = i * C::EPC; e < (i + 1) * C::EPC; ++e) {
          const int rg = e / 16, ee = e % 16;
          sc[rg][ee] = exp2_fast(fmaf(sc[rg][ee], c, nm[rg]));
          if (ee & 1) {
            const uint32_t pk = E::pack2(sc[rg][ee - 1], sc[rg][ee]);
            asm volatile("" ::"v"(pk));  // pin the work of this chunk next to its MFMA
            pb[rg][ee >> 3][(ee & 7) >> 1] = pk;
          }
          if ((ee & 3) == 3) {
            const int cb = ee >> 3, w = (ee & 7) >> 1;
            tsm[rg] = E::mfma4(sum_ones, u32x2{pb[rg][cb][w - 1], pb[rg][cb][w]}, tsm[rg]);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    __builtin_amdgcn_s_setprio(0);

    // Lazy-max check: a row whose tile sum of p passed 2^10 recomputes S(t)
    // from the resident K tile, raises m to its row max, rescales O and l and
    // redoes its p; the other rows keep theirs.
    float ts[NRG];
    bool trig[NRG];
#pragma unroll
    for (int rg = 0; rg < NRG; ++rg) {
      ts[rg] = xhalf_sum(tsm[rg][0]);
      trig[rg] = !(ts[rg] <= kSumTrigger);
    }
    if (__builtin_amdgcn_ballot_w64(trig[0] || trig[1])) {
      qk(ring + st * C::STAGE, sc);
      mask(t, sc);
#pragma unroll
      for (int rg = 0; rg < NRG; ++rg) {
        const float mx = xhalf_max(max16(sc[rg])) * c;
        const float m_old = m[rg];
        if (trig[rg]) set_m(rg, maxf(m_old, mx));
        const float alpha = m[rg] > m_old ? exp2_fast(m_old - m[rg]) : 1.f;  // 0 when m was -inf
        l[rg] *= alpha;
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) acc[rg][dt] *= alpha;
#pragma unroll
        for (int e = 0; e < 16; e += 2) {
          const uint32_t w = pb[rg][e >> 3][(e & 7) >> 1];
          pb[rg][e >> 3][(e & 7) >> 1] =
              trig[rg] ? E::pack2(exp2_fast(fmaf(sc[rg][e], c, nm[rg])), exp2_fast(fmaf(sc[rg][e + 1], c, nm[rg])))
                       : w;
        }
        f32x4 t2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
          t2 = E::mfma4(sum_ones, u32x2{pb[rg][cc][0], pb[rg][cc][1]}, t2);
          t2 = E::mfma4(sum_ones, u32x2{pb[rg][cc][2], pb[rg][cc][3]}, t2);
        }
        const float ts2 = xhalf_sum(t2[0]);
        if (trig[rg]) ts[rg] = ts2;
      }
    }
#pragma unroll
    for (int rg = 0; rg < NRG; ++rg) l[rg] += ts[rg];
    mask(t + 1, sn);

    // O += V(t) P(t): each V^T fragment serves both row groups.
    {
      const uint16_t* vs = ring + st * C::STAGE + C::TILE;
      u32x4 va[C::DT][2];
#pragma unroll
      for (int cc = 0; cc < 2; ++cc)
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) va[dt][cc] = vfrag(vs, dt, cc);
#pragma unroll
      for (int cc = 0; cc < 2; ++cc)
#pragma unroll
        for (int rg = 0; rg < NRG; ++rg)
#pragma unroll
          for (int dt = 0; dt < C::DT; ++dt) acc[rg][dt] = E::mfma(va[dt][cc], pb[rg][cc], acc[rg][dt]);
    }
  };
  CIE_STAMP(flash_timeline, 1);  // loop start
  CIE_STAMP_VALUE(flash_timeline, 4, n_tiles);
  f32x16 sb[NRG];
  static_assert(C::NST % 2 == 0, "stage and score buffer repeat after NST steps");
  for (int t = 0; t < n_tiles; t += C::NST) {
    static_for<C::NST>([&](auto I) CIE_INLINE {
      constexpr int i = decltype(I)::value;
      if (t + i < n_tiles) {
        if constexpr (i % 2 == 0) step(std::integral_constant<int, i>{}, t + i, sc, sb);
        else step(std::integral_constant<int, i>{}, t + i, sb, sc);
      }
    });
  }

  CIE_STAMP(flash_timeline, 2);  // loop end
  // Epilogue: rows with keys but none visible give 0 * inf = NaN like the
  // reference's softmax over an all -inf row; Lk == 0 gives zeros.
  // O goes out through LDS so that every store instruction writes whole
  // 128-byte rows: straight from the accumulators a store instruction would
  // write 16 bytes into each of 32 rows. The ring is free once every wave
  // is past its last tile; each wave stages its 64 (row, head) rows in its
  // own quarter, 16-byte chunks XOR-swizzled by row pair, and reads back
  // only what it wrote.
  static_assert(4 * 2 * 32 * D <= C::NST * C::STAGE, "O staging fits the ring");
  __syncthreads();  // no wave reads the ring any more
  uint16_t* stg = ring + wave * (2 * 32 * D);
#pragma unroll
  for (int rg = 0; rg < NRG; ++rg) {
    const float inv = p.Lk == 0 ? 0.f : 1.f / l[rg];
    const int slot = 32 * rg + l32, sw = (slot >> 1) & 7;
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) {
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int chunk = 4 * dt + g4;  // 16-byte chunk of d = 32 dt + 8 g4 .. +8
        const u32x2 w = {E::pack2(acc[rg][dt][4 * g4] * inv, acc[rg][dt][4 * g4 + 1] * inv),
                         E::pack2(acc[rg][dt][4 * g4 + 2] * inv, acc[rg][dt][4 * g4 + 3] * inv)};
        *reinterpret_cast<u32x2*>(stg + slot * D + 8 * (chunk ^ sw) + 4 * hl) = w;
      }
    }
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's staging writes are done
  {
    const int c = lane & 7;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int slot = 8 * i + (lane >> 3), rg = slot >> 5, r32 = slot & 31;
      const int row = q0w + (HEADS ? 0 : 32 * rg) + r32;
      const int head = HEADS ? kvh * G + 2 * g + rg : kvh * G + g;
      const u32x4 v = *reinterpret_cast<const u32x4*>(stg + slot * D + 8 * (c ^ ((slot >> 1) & 7)));
      if (row < p.Lq) *reinterpret_cast<u32x4*>(p.o + b * p.os0 + head * p.os1 + (int64_t)row * p.os2 + 8 * c) = v;
    }
  }
  CIE_STAMP(flash_timeline, 3);  // stores issued
}

// head_dim 128 runs the interleaved kernel (S=16384 bf16 causal: 1863 ->
// 1774 us); at head_dim 64 it measured 2 % slower than flash_fwd_kernel, whose
// VALU-heavy and MFMA-only phases the other wave of each SIMD pairs up.
// head_dim 64 runs the two-row-group kernel (on pairs of query heads when
// the group size is even, else on 256-row query tiles; both modes give every
// row the same arithmetic) when r64_pays says so, else flash_fwd_kernel.
//
// A two-row-group item is twice the work of a flash_fwd_kernel item and there
// are half as many, so it pays only with enough of them: at least one per
// workgroup slot of the GPU (2 per CU: 512 on an MI355X), and, causal, its longest item
// (the last query tile: every key, 32 per step, plus ~4 steps of start-up)
// within 1.6x the average work per slot; otherwise the critical path or the
// idle slots cost more than the shared fragment reads save (measured on
// B x S x Hq / Hk = 1x4096x32/8 causal 101 against 78 us, 2x1024x32/8 27 against
// 20, 1x512x32/8 16 against 10; gains on 4x2048x32/8 78 against 86, 8x512x32/8
// 21 against 23, 16x256x32/8 16 against 18, 1x4096x32/8 non-causal 134 against
// 143). The estimate uses B * Hq / 2 items of 128 rows whatever the group
// size, so GQA and its expanded MHA take the same kernel and stay equal bit
// for bit.
static bool r64_pays(const FlashParams& p) {
  const int64_t kSlots = 2 * (int64_t)p.cus, kStartup = 4;
  if (p.Lq <= 128) return false;
  const int64_t n_mt = (p.Lq + 127) / 128;
  const int64_t items = (int64_t)(p.n_wg / p.n_mt) / 2;  // B * Hq / 2 per query tile
  if (n_mt * items < kSlots) return false;
  if (!p.causal) return true;
  int64_t work = 0, longest = 0;
  for (int64_t mt = 0; mt < n_mt; ++mt) {
    const int64_t kend = std::max<int64_t>(0, std::min<int64_t>(p.Lk, (int64_t)p.Lk - p.Lq + std::min<int64_t>(p.Lq, 128 * (mt + 1))));
    const int64_t steps = (kend + 31) / 32 + kStartup;
    work += steps;
    longest = std::max(longest, steps);
  }
  return longest * kSlots * 10 <= 16 * work * items;
}

template <int DTYPE, int D, bool HEADS>
static void launch_r64(const FlashParams& p, hipStream_t stream) {
  FlashParams q = p;
  q.n_mt = (p.Lq + R64Cfg<D, HEADS>::BM - 1) / R64Cfg<D, HEADS>::BM;
  q.n_wg = q.n_mt * (p.n_wg / p.n_mt) / (HEADS ? 2 : 1);  // B * Hq (/ 2) items per query tile
  hipLaunchKernelGGL((flash_fwd_r64_kernel<DTYPE, D, HEADS>), dim3(q.n_wg), dim3(256), 0, stream, q);
}

FlashKernel flash_kernel_choice(const FlashParams& p, int D) {
  if (D == 128) return kFlashIl;
  if (D == 64 && r64_pays(p)) return p.group % 2 == 0 ? kFlashR64Heads : kFlashR64Rows;
  return kFlash32;
}

template <int DTYPE, int D>
static hipError_t launch_flash_t(const FlashParams& p, hipStream_t stream) {
  switch (flash_kernel_choice(p, D)) {
    case kFlashIl:
      if constexpr (D == 128) hipLaunchKernelGGL((flash_fwd_il_kernel<DTYPE, D>), dim3(p.n_wg), dim3(256), 0, stream, p);
      break;
    case kFlashR64Heads:
      if constexpr (D == 64) launch_r64<DTYPE, D, true>(p, stream);
      break;
    case kFlashR64Rows:
      if constexpr (D == 64) launch_r64<DTYPE, D, false>(p, stream);
      break;
    default:
      if constexpr (D != 128) hipLaunchKernelGGL((flash_fwd_kernel<DTYPE, D>), dim3(p.n_wg), dim3(256), 0, stream, p);
      break;
  }
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

#ifdef CIE_TIMELINE
// timeline build only: the stamps of the last flash_fwd_r64_kernel launch
extern "C" int cie_timeline_flash(void* host, size_t bytes) {
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(cie::flash_timeline), bytes, 0, hipMemcpyDeviceToHost);
}
#endif
