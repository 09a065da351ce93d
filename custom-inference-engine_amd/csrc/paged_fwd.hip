// Paged decode / speculative-verify attention for gfx950.
//
// Replaces the reference's per-layer gather-then-dense sequence
// (engine/model/block.py:56-71: cache.gather -> index_select of the whole
// history, engine/cache/kv_cache.py:141-165, then the dense Triton kernel):
// K and V are read once, straight out of the (num_blocks, block_size, Hk, D)
// pool through the int32 block table, with 16-byte loads.
//
// One workgroup (4 waves) per (sequence, context split, query tile, kv head);
// the kv heads of one (sequence, split) are adjacent workgroup ids so the
// pool blocks they share (block_size * Hk * D contiguous elements) are read
// at the same time. All Hq/Hk query heads x Lq new tokens of a kv head
// (R = group * Lq rows, up to 32 per query tile) share each K/V byte. The
// split's block ids are staged in LDS once; each wave then walks every 4th
// 32-key tile of the split:
//   S^T[32 x 32] = K_tile . Q^T    K rows go from global memory straight into
//                                   the MFMA A operand (one token row per lane)
//   online softmax in registers (one v_permlane32_swap per reduction)
//   O^T += V^T_tile . P^T          V tile transposed through a per-wave LDS slab
// Loads are unconditional (addresses clamped to a valid token, data of
// out-of-range tokens zeroed or masked), so a tile's loads stay in flight
// together. The 4 waves merge in LDS; a workgroup whose sequence has a single
// split writes the final output, otherwise it writes (m, l, acc) partials
// that paged_reduce_kernel combines.
#include "kernels.hpp"

namespace cie {

constexpr float kLazyRescalePaged = 8.0f;

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
  static constexpr int LDS_WORK = LDS_VT > LDS_MERGE ? LDS_VT : LDS_MERGE;
  static constexpr int LDS = LDS_WORK + kPagedMaxSplitBlocks * 4;  // + staged block ids
};

template <int DTYPE, int D>
__global__ __launch_bounds__(256) void paged_fwd_kernel(const PagedParams p) {
  using C = PagedCfg<D>;
  using E = Elt<DTYPE>;
  __shared__ __attribute__((aligned(16))) unsigned char smem[C::LDS];
  int32_t* sbt = reinterpret_cast<int32_t*>(smem + C::LDS_WORK);

  // blockIdx.x = ((b * n_splits + s) * n_qt + qt) * Hk + kvh
  int id = blockIdx.x;
  const int kvh = id % p.Hk;
  id /= p.Hk;
  const int qt = id % p.n_qt;
  id /= p.n_qt;
  const int s = id % p.n_splits;
  const int b = id / p.n_splits;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hl = lane >> 5;

  int ctx = p.lens[b];
  const bool bad_len = ctx < 0 || ctx > p.max_blocks * p.block_size || ctx > p.n_splits * p.split_len ||
                       (ctx > 0 && p.num_blocks < 1);
  if (bad_len) ctx = 0;  // never dereference; the output is poisoned below
  const int nsb = max(1, (ctx + p.split_len - 1) / p.split_len);
  if (s >= nsb) return;  // uniform over the workgroup
  const int split0 = s * p.split_len;
  const int split1 = min(ctx, split0 + p.split_len);

  // Stage the split's block ids (validated) in LDS.
  const int blk0 = split1 > split0 ? (int)fdiv((uint32_t)split0, p.bsdiv) : 0;
  const int nblk = split1 > split0 ? (int)fdiv((uint32_t)(split1 - 1), p.bsdiv) - blk0 + 1 : 0;
  bool bad_blk = false;
  const int32_t* btr = p.bt + (int64_t)b * p.max_blocks;
  for (int j = tid; j < nblk; j += 256) {
    const int bid = btr[blk0 + j];
    const bool inb = bid >= 0 && bid < p.num_blocks;
    bad_blk |= !inb;
    sbt[j] = inb ? bid : 0;
  }
  const bool any_bad = __syncthreads_or(bad_blk ? 1 : 0) != 0;

  // Query row of this lane: r = g * Lq + i (query head kvh*group + g, token i).
  const int r = qt * 32 + l32;
  const bool rv = r < p.R;
  const int g = rv ? r / p.Lq : 0;
  const int i = rv ? r - g * p.Lq : 0;
  const int hq = kvh * p.group + g;
  const uint16_t* qrow = p.q + b * p.qs0 + hq * p.qs1 + (int64_t)i * p.qs2;
  u32x4 qf[C::KK];
#pragma unroll
  for (int kk = 0; kk < C::KK; ++kk) {
    qf[kk] = load16(qrow + 16 * kk + 8 * hl, rv);
    qf[kk] ^= u32x4{p.q_sign, p.q_sign, p.q_sign, p.q_sign};
  }
  // Last key visible to this row: the Lq new tokens are the newest Lq
  // positions of the context (bottom-right causal alignment).
  const int lim = min(split1 - 1, p.causal ? ctx - p.Lq + i : ctx - 1);
  const float c = p.scale_log2;

  const uint16_t* kbase = p.kc + kvh * p.ks2;
  const uint16_t* vbase = p.vc + kvh * p.vs2;
  const int last = split1 - 1;
  // Pool row of token t, clamped into this split (valid whenever the split is non-empty).
  auto row_ptr = [&](const uint16_t* base, int64_t s0, int64_t s1, int t) -> const uint16_t* {
    t = min(t, last);
    const uint32_t blk = fdiv((uint32_t)t, p.bsdiv);
    const uint32_t off = (uint32_t)t - blk * (uint32_t)p.block_size;
    return base + (int64_t)sbt[blk - blk0] * s0 + (int64_t)off * s1;
  };

  u32x4 kn[C::KK];
  u32x4 vn[C::VGL][4];
  uint32_t vok[C::VGL];
  auto gload = [&](int t0) {
    const uint16_t* kp = row_ptr(kbase, p.ks0, p.ks1, t0 + l32);
#pragma unroll
    for (int kk = 0; kk < C::KK; ++kk) kn[kk] = load16_stream(kp + 16 * kk + 8 * hl);
#pragma unroll
    for (int gg = 0; gg < C::VGL; ++gg) {
      const int gi = min(lane + 64 * gg, D - 1);
      const int p4 = gi / (D / 8), qd = gi % (D / 8);
      uint32_t okm = 0;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int t = t0 + 4 * p4 + rr;
        okm |= (t < split1 ? 1u : 0u) << rr;
        vn[gg][rr] = load16_stream(row_ptr(vbase, p.vs0, p.vs1, t) + 8 * qd);
      }
      vok[gg] = okm;
    }
  };

  f32x16 acc[C::DT];
#pragma unroll
  for (int dt = 0; dt < C::DT; ++dt) acc[dt] = f32x16{};
  float m = -INFINITY, l = 0.f;

  uint16_t* vtw = reinterpret_cast<uint16_t*>(smem) + wave * C::VT_WAVE;
  constexpr int kStep = kPagedWaves * kPagedTile;
  int t0 = split0 + kPagedTile * wave;
  if (t0 < split1) gload(t0);
  for (; t0 < split1; t0 += kStep) {
    u32x4 kc[C::KK];
    u32x4 vc[C::VGL][4];
    uint32_t vokc[C::VGL];
#pragma unroll
    for (int kk = 0; kk < C::KK; ++kk) kc[kk] = kn[kk];
#pragma unroll
    for (int gg = 0; gg < C::VGL; ++gg) {
      vokc[gg] = vok[gg];
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) vc[gg][rr] = vn[gg][rr];
    }
    if (t0 + kStep < split1) gload(t0 + kStep);

    f32x16 sc = f32x16{};
#pragma unroll
    for (int kk = 0; kk < C::KK; ++kk) sc = E::mfma(kc[kk], qf[kk], sc);

    float mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int key = t0 + 8 * (e >> 2) + 4 * hl + (e & 3);
      sc[e] = key <= lim ? sc[e] : -INFINITY;
      mx = fmaxf(mx, sc[e]);
    }
    const float mxs = xhalf_max(mx) * c;
    const bool grow = mxs > m + kLazyRescalePaged;
    if (__builtin_amdgcn_ballot_w64(grow)) {
      const float m_new = grow ? mxs : m;
      const float alpha = grow ? exp2_fast(m - m_new) : 1.f;
      l *= alpha;
#pragma unroll
      for (int dt = 0; dt < C::DT; ++dt) acc[dt] *= alpha;
      m = m_new;
    }
    const float neg_m = m == -INFINITY ? 0.f : -m;
    u32x4 pb[2];
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const int e0 = 8 * cc + 2 * w;
        const float p0 = exp2_fast(fmaf(sc[e0], c, neg_m));
        const float p1 = exp2_fast(fmaf(sc[e0 + 1], c, neg_m));
        l += p0 + p1;
        pb[cc][w] = E::pack2(p0, p1);
      }
    }

    // V tile -> V^T slab of this wave (LDS ops of one wave complete in order).
#pragma unroll
    for (int gg = 0; gg < C::VGL; ++gg) {
      const int gi = lane + 64 * gg;
      if (D % 64 == 0 || gi < D) {
        const int p4 = gi / (D / 8), qd = gi % (D / 8);
        const u32x4 r0 = zero_unless(vc[gg][0], vokc[gg] & 1u);
        const u32x4 r1 = zero_unless(vc[gg][1], vokc[gg] & 2u);
        const u32x4 r2 = zero_unless(vc[gg][2], vokc[gg] & 4u);
        const u32x4 r3 = zero_unless(vc[gg][3], vokc[gg] & 8u);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const int d = 8 * qd + 2 * w;
          *reinterpret_cast<u32x2*>(vtw + d * C::VSTR + 4 * p4) = col4_even(r0[w], r1[w], r2[w], r3[w]);
          *reinterpret_cast<u32x2*>(vtw + (d + 1) * C::VSTR + 4 * p4) = col4_odd(r0[w], r1[w], r2[w], r3[w]);
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
      for (int cc = 0; cc < 2; ++cc) {
        u32x4 a = {0u, 0u, 0u, 0u};
        if (D >= 32 || drow < D) {
          const u32x2 lo = *reinterpret_cast<const u32x2*>(vtw + drow * C::VSTR + 16 * cc + 4 * hl);
          const u32x2 hi = *reinterpret_cast<const u32x2*>(vtw + drow * C::VSTR + 16 * cc + 8 + 4 * hl);
          a = u32x4{lo[0], lo[1], hi[0], hi[1]};
        }
        acc[dt] = E::mfma(a, pb[cc], acc[dt]);
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
  __syncthreads();
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
  const bool poisoned = bad_len || any_bad;
  if (nsb == 1 || poisoned) {
    const float inv = poisoned ? __builtin_nanf("") : (ctx == 0 ? 0.f : 1.f / l_tot);
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

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x = fmaxf(x, __shfl_xor(x, off));
  return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off);
  return x;
}

// Combines the split partials of every (sequence, query head, token) row
// whose sequence spans more than one split. One wave per row.
template <int DTYPE, int D>
__global__ __launch_bounds__(64) void paged_reduce_kernel(const PagedParams p) {
  using E = Elt<DTYPE>;
  __shared__ float wsh[kPagedReduceChunk];
  const int row = blockIdx.x;  // (b * Hq + hq) * Lq + i
  const int i = row % p.Lq;
  const int bh = row / p.Lq;
  const int hq = bh % p.Hq, b = bh / p.Hq;
  const int ctx = p.lens[b];
  if (ctx < 0 || ctx > p.max_blocks * p.block_size || ctx > p.n_splits * p.split_len ||
      (ctx > 0 && p.num_blocks < 1))
    return;  // written as NaN by the main kernel
  const int nsb = max(1, (ctx + p.split_len - 1) / p.split_len);
  if (nsb <= 1) return;
  const int64_t base = (int64_t)row * p.n_splits;
  const int lane = threadIdx.x;

  float M = -INFINITY;
  for (int s = lane; s < nsb; s += 64) M = fmaxf(M, p.ws_ml[2 * (base + s)]);
  M = wave_max(M);
  float L = 0.f;
  for (int s = lane; s < nsb; s += 64) L += rescale_weight(p.ws_ml[2 * (base + s)], M) * p.ws_ml[2 * (base + s) + 1];
  L = wave_sum(L);
  const float inv = 1.f / L;

  constexpr int PER = (D + 63) / 64;
  float acc[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) acc[j] = 0.f;
  for (int s0 = 0; s0 < nsb; s0 += kPagedReduceChunk) {
    const int cnt = min(kPagedReduceChunk, nsb - s0);
    __syncthreads();
    for (int j = lane; j < cnt; j += 64) wsh[j] = rescale_weight(p.ws_ml[2 * (base + s0 + j)], M);
    __syncthreads();
    const float* src = p.ws_acc + (base + s0) * D;
    for (int j = 0; j < cnt; ++j) {
      const float w = wsh[j];
#pragma unroll
      for (int q = 0; q < PER; ++q) {
        const int d = lane + 64 * q;
        if (D >= 64 || d < D) acc[q] += w * src[(int64_t)j * D + d];
      }
    }
  }
  uint16_t* orow = p.o + b * p.os0 + hq * p.os1 + (int64_t)i * p.os2;
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int d = lane + 64 * q;
    if (D >= 64 || d < D) orow[d] = (uint16_t)(E::pack2(acc[q] * inv, 0.f) & 0xffffu);
  }
}

int paged_split_len(int B, int Hk, int n_qt, int max_ctx, int block_size) {
  constexpr int kStep = kPagedWaves * kPagedTile;
  // The split's block ids must fit the LDS staging area.
  const int64_t cap_tokens = (int64_t)(kPagedMaxSplitBlocks - 2) * block_size;
  const int cap = (int)std::min<int64_t>(1 << 20, std::max<int64_t>(kStep, cap_tokens / kStep * kStep));
  const int64_t pairs = (int64_t)B * Hk * n_qt;
  int split = std::min(2 * kStep, cap);
  while (split < max_ctx && 2 * split <= cap && pairs * ((max_ctx + split - 1) / split) > 2048) split *= 2;
  return split;
}

template <int DTYPE, int D>
static hipError_t launch_paged_t(const PagedParams& p, hipStream_t stream) {
  const int64_t n_wg = (int64_t)p.B * p.n_splits * p.n_qt * p.Hk;
  hipLaunchKernelGGL((paged_fwd_kernel<DTYPE, D>), dim3((unsigned)n_wg), dim3(256), 0, stream, p);
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
