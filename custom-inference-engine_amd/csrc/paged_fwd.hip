// Paged decode / speculative-verify attention for gfx950.
//
// Replaces the reference's per-layer gather-then-dense sequence
// (engine/model/block.py:56-71: cache.gather -> index_select of the whole
// history, engine/cache/kv_cache.py:141-165, then the dense Triton kernel):
// K and V are read once, straight out of the (num_blocks, block_size, Hk, D)
// pool through the int32 block table, with 16-byte loads.
//
// Grid: (context split, query tile, batch * kv head); 4 waves per workgroup.
// All Hq/Hk query heads x Lq new tokens of a kv head (R = group * Lq rows,
// up to 32 per query tile) share each K/V byte. Each wave walks every 4th
// 32-key tile of its split:
//   S^T[32 x 32] = K_tile . Q^T    K rows go from global memory straight into
//                                   the MFMA A operand (one token row per lane)
//   online softmax in registers (one v_permlane32_swap per reduction)
//   O^T += V^T_tile . P^T          V tile transposed through a per-wave LDS slab
// The 4 waves merge in LDS; a workgroup whose sequence has a single split
// writes the final output, otherwise it writes (m, l, acc) partials that
// paged_reduce_kernel combines.
#include "kernels.hpp"

namespace cie {

template <int D>
struct PagedCfg {
  static constexpr int KK = D / 16;
  static constexpr int DT = D >= 32 ? D / 32 : 1;
  static constexpr int VSTR = kPagedTile + 4;           // LDS pitch of a V^T row (elements)
  static constexpr int VT_WAVE = D * VSTR;              // elements per wave slab
  static constexpr int VGL = (D + 63) / 64;             // 4-token x 8-dim V groups per lane
  static constexpr int MERGE = DT * 16 * 64 + 2 * 64;   // floats per merge slot
  static constexpr int LDS_VT = kPagedWaves * VT_WAVE * 2;
  static constexpr int LDS_MERGE = 2 * MERGE * 4;
  static constexpr int LDS = LDS_VT > LDS_MERGE ? LDS_VT : LDS_MERGE;
};

template <int DTYPE, int D>
__global__ __launch_bounds__(256) void paged_fwd_kernel(const PagedParams p) {
  using C = PagedCfg<D>;
  using E = Elt<DTYPE>;
  __shared__ __attribute__((aligned(16))) unsigned char smem[C::LDS];

  const int s = blockIdx.x, qt = blockIdx.y, bk = blockIdx.z;
  const int b = bk / p.Hk, kvh = bk - b * p.Hk;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hl = lane >> 5;

  int ctx = p.lens[b];
  const bool bad_len = ctx < 0 || ctx > p.max_blocks * p.block_size || ctx > p.n_splits * p.split_len;
  if (bad_len) ctx = 0;  // never dereference; the output is poisoned below
  const int nsb = max(1, (ctx + p.split_len - 1) / p.split_len);
  if (s >= nsb) return;  // uniform over the workgroup
  const int split0 = s * p.split_len;
  const int split1 = min(ctx, split0 + p.split_len);

  // Query row of this lane: r = g * Lq + i (query head kvh*group + g, token i).
  const int r = qt * 32 + l32;
  const bool rv = r < p.R;
  const int g = rv ? r / p.Lq : 0;
  const int i = rv ? r - g * p.Lq : 0;
  const int hq = kvh * p.group + g;
  const uint16_t* qrow = p.q + b * p.qs0 + hq * p.qs1 + (int64_t)i * p.qs2;
  u32x4 qf[C::KK];
#pragma unroll
  for (int kk = 0; kk < C::KK; ++kk) qf[kk] = load16(qrow + 16 * kk + 8 * hl, rv);
  // Last key visible to this row: the Lq new tokens are the newest Lq
  // positions of the context (bottom-right causal alignment).
  const int lim = p.causal ? ctx - p.Lq + i : ctx - 1;

  const int32_t* btr = p.bt + (int64_t)b * p.max_blocks;
  const uint16_t* kbase = p.kc + kvh * p.ks2;
  const uint16_t* vbase = p.vc + kvh * p.vs2;
  bool bad_blk = false;

  // Pool address of token t (t < split1 <= max_blocks * block_size).
  auto tok = [&](int t, int64_t s0, int64_t s1, const uint16_t* base, bool& ok) -> const uint16_t* {
    const uint32_t blk = fdiv((uint32_t)t, p.bsdiv);
    const uint32_t off = (uint32_t)t - blk * (uint32_t)p.block_size;
    const int bid = btr[blk];
    const bool inb = bid >= 0 && bid < p.num_blocks;
    bad_blk |= !inb;
    ok = inb;
    return base + (int64_t)(inb ? bid : 0) * s0 + (int64_t)off * s1;
  };

  u32x4 kn[C::KK];
  u32x4 vn[C::VGL][4];
  auto gload = [&](int t0) {
    {
      const int t = t0 + l32;
      bool ok = false;
      const uint16_t* kp = kbase;
      if (t < split1) kp = tok(t, p.ks0, p.ks1, kbase, ok);
#pragma unroll
      for (int kk = 0; kk < C::KK; ++kk) kn[kk] = load16(kp + 16 * kk + 8 * hl, ok);
    }
#pragma unroll
    for (int gg = 0; gg < C::VGL; ++gg) {
      const int gi = lane + 64 * gg;
      const int p4 = gi / (D / 8), qd = gi % (D / 8);
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int t = t0 + 4 * p4 + rr;
        bool ok = false;
        const uint16_t* vp = vbase;
        if (gi < D && t < split1) vp = tok(t, p.vs0, p.vs1, vbase, ok);
        vn[gg][rr] = load16(vp + 8 * qd, ok);
      }
    }
  };

  f32x16 acc[C::DT];
#pragma unroll
  for (int dt = 0; dt < C::DT; ++dt) acc[dt] = f32x16{};
  float m = -INFINITY, l = 0.f;

  uint16_t* vtw = reinterpret_cast<uint16_t*>(smem) + wave * C::VT_WAVE;
  int t0 = split0 + kPagedTile * wave;
  if (t0 < split1) gload(t0);
  for (; t0 < split1; t0 += kPagedWaves * kPagedTile) {
    u32x4 kc[C::KK];
    u32x4 vc[C::VGL][4];
#pragma unroll
    for (int kk = 0; kk < C::KK; ++kk) kc[kk] = kn[kk];
#pragma unroll
    for (int gg = 0; gg < C::VGL; ++gg)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) vc[gg][rr] = vn[gg][rr];
    if (t0 + kPagedWaves * kPagedTile < split1) gload(t0 + kPagedWaves * kPagedTile);

    f32x16 sc = f32x16{};
#pragma unroll
    for (int kk = 0; kk < C::KK; ++kk) sc = E::mfma(kc[kk], qf[kk], sc);

    float mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int key = t0 + 8 * (e >> 2) + 4 * hl + (e & 3);
      const float x = (key < split1 && key <= lim) ? sc[e] * p.scale_log2 : -INFINITY;
      sc[e] = x;
      mx = fmaxf(mx, x);
    }
    mx = xhalf_max(mx);
    const float m_new = fmaxf(m, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = exp2_fast(m - m_use);
    l *= alpha;
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) acc[dt] *= alpha;
    u32x4 pb[2];
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const int e0 = 8 * cc + 2 * w;
        const float p0 = exp2_fast(sc[e0] - m_use);
        const float p1 = exp2_fast(sc[e0 + 1] - m_use);
        l += p0 + p1;
        pb[cc][w] = E::pack2(p0, p1);
      }
    }
    m = m_new;

    // V tile -> V^T slab of this wave (LDS ops of one wave complete in order).
#pragma unroll
    for (int gg = 0; gg < C::VGL; ++gg) {
      const int gi = lane + 64 * gg;
      if (gi < D) {
        const int p4 = gi / (D / 8), qd = gi % (D / 8);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const int d = 8 * qd + 2 * w;
          *reinterpret_cast<u32x2*>(vtw + d * C::VSTR + 4 * p4) =
              col4_even(vc[gg][0][w], vc[gg][1][w], vc[gg][2][w], vc[gg][3][w]);
          *reinterpret_cast<u32x2*>(vtw + (d + 1) * C::VSTR + 4 * p4) =
              col4_odd(vc[gg][0][w], vc[gg][1][w], vc[gg][2][w], vc[gg][3][w]);
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) {
      const int drow = 32 * dt + l32;
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        u32x4 a = {0u, 0u, 0u, 0u};
        if (D >= 32 || drow < D) {
          const u32x2 lo = *reinterpret_cast<const u32x2*>(vtw + drow * C::VSTR + 16 * c + 4 * hl);
          const u32x2 hi = *reinterpret_cast<const u32x2*>(vtw + drow * C::VSTR + 16 * c + 8 + 4 * hl);
          a = u32x4{lo[0], lo[1], hi[0], hi[1]};
        }
        acc[dt] = E::mfma(a, pb[c], acc[dt]);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  // Merge the 4 waves' partial softmax states: (1,3) into (0,2), then 2 into 0.
  float* mb = reinterpret_cast<float*>(smem);
  auto put = [&](float* slot) {
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) slot[(dt * 16 + e) * 64 + lane] = acc[dt][e];
    slot[C::DT * 16 * 64 + lane] = m;
    slot[C::DT * 16 * 64 + 64 + lane] = l;
  };
  auto take = [&](const float* slot) {
    const float mo = slot[C::DT * 16 * 64 + lane];
    const float lo = slot[C::DT * 16 * 64 + 64 + lane];
    const float M = fmaxf(m, mo);
    const float wa = rescale_weight(m, M), wb = rescale_weight(mo, M);
    l = l * wa + lo * wb;
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[dt][e] = acc[dt][e] * wa + slot[(dt * 16 + e) * 64 + lane] * wb;
    m = M;
  };
  const bool any_bad = __syncthreads_or(bad_blk ? 1 : 0) != 0;
  if (wave & 1) put(mb + (wave >> 1) * C::MERGE);
  __syncthreads();
  if (!(wave & 1)) take(mb + (wave >> 1) * C::MERGE);
  __syncthreads();
  if (wave == 2) put(mb);
  __syncthreads();
  if (wave != 0) return;
  take(mb);

  const float l_tot = xhalf_sum(l);
  if (!rv) return;
  if (nsb == 1 || bad_len || any_bad) {
    const float inv = (bad_len || any_bad) ? __builtin_nanf("") : (ctx == 0 ? 0.f : 1.f / l_tot);
    uint16_t* orow = p.o + b * p.os0 + hq * p.os1 + (int64_t)i * p.os2;
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
    if (nsb == 1) return;
  }
  // Partial state of this split for the reduction pass (a poisoned split
  // stores NaN so the combined row is NaN as well).
  const float poison = any_bad ? __builtin_nanf("") : 1.f;
  const int64_t row = ((int64_t)(b * p.Hq + hq) * p.Lq + i) * p.n_splits + s;
  float* wa = p.ws_acc + row * D;
#pragma unroll
  for (int dt = 0; dt < C::DT; ++dt) {
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int d = 32 * dt + 8 * g4 + 4 * hl;
      if (D >= 32 || d < D) {
        *reinterpret_cast<float4*>(wa + d) =
            float4{acc[dt][4 * g4] * poison, acc[dt][4 * g4 + 1] * poison,
                   acc[dt][4 * g4 + 2] * poison, acc[dt][4 * g4 + 3] * poison};
      }
    }
  }
  if (hl == 0) *reinterpret_cast<float2*>(p.ws_ml + 2 * row) = float2{m * poison, l_tot * poison};
}

// Combines the split partials of every (sequence, query head, token) row
// whose sequence spans more than one split.
template <int DTYPE, int D>
__global__ __launch_bounds__(64) void paged_reduce_kernel(const PagedParams p) {
  using E = Elt<DTYPE>;
  const int row = blockIdx.x;  // (b * Hq + hq) * Lq + i
  const int i = row % p.Lq;
  const int bh = row / p.Lq;
  const int hq = bh % p.Hq, b = bh / p.Hq;
  const int ctx = p.lens[b];
  if (ctx < 0 || ctx > p.max_blocks * p.block_size || ctx > p.n_splits * p.split_len) return;  // NaN already
  const int nsb = max(1, (ctx + p.split_len - 1) / p.split_len);
  if (nsb <= 1) return;
  const int64_t base = (int64_t)row * p.n_splits;
  float M = -INFINITY;
  for (int s = 0; s < nsb; ++s) M = fmaxf(M, p.ws_ml[2 * (base + s)]);
  float L = 0.f;
  for (int s = 0; s < nsb; ++s) L += rescale_weight(p.ws_ml[2 * (base + s)], M) * p.ws_ml[2 * (base + s) + 1];
  const float inv = 1.f / L;
  uint16_t* orow = p.o + b * p.os0 + hq * p.os1 + (int64_t)i * p.os2;
  for (int d = threadIdx.x; d < D; d += 64) {
    float acc = 0.f;
    for (int s = 0; s < nsb; ++s)
      acc += rescale_weight(p.ws_ml[2 * (base + s)], M) * p.ws_acc[(base + s) * D + d];
    const uint32_t w = E::pack2(acc * inv, 0.f);
    orow[d] = (uint16_t)(w & 0xffffu);
  }
}

int paged_split_len(int B, int Hk, int n_qt, int max_ctx) {
  const int64_t pairs = (int64_t)B * Hk * n_qt;
  int split = kPagedWaves * kPagedTile * 2;
  while (split < max_ctx && pairs * ((max_ctx + split - 1) / split) > 2048) split *= 2;
  return split;
}

template <int DTYPE, int D>
static hipError_t launch_paged_t(const PagedParams& p, hipStream_t stream) {
  const int n_qt = (p.R + 31) / 32;
  hipLaunchKernelGGL((paged_fwd_kernel<DTYPE, D>), dim3(p.n_splits, n_qt, p.B * p.Hk), dim3(256), 0, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.n_splits <= 1) return e;
  hipLaunchKernelGGL((paged_reduce_kernel<DTYPE, D>), dim3(p.B * p.Hq * p.Lq), dim3(64), 0, stream, p);
  return hipGetLastError();
}

template <int DTYPE>
static hipError_t launch_paged_d(const PagedParams& p, int D, hipStream_t stream) {
  switch (D) {
    case 16: return launch_paged_t<DTYPE, 16>(p, stream);
    case 32: return launch_paged_t<DTYPE, 32>(p, stream);
    case 64: return launch_paged_t<DTYPE, 64>(p, stream);
    case 128: return launch_paged_t<DTYPE, 128>(p, stream);
    case 256: return launch_paged_t<DTYPE, 256>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_paged(const PagedParams& p, int dtype, int D, hipStream_t stream) {
  return dtype == 0 ? launch_paged_d<0>(p, D, stream) : launch_paged_d<1>(p, D, stream);
}

}  // namespace cie
