// Paged decode / speculative-verify attention for gfx950.
//
// Replaces the reference's per-layer gather-then-dense sequence
// (engine/model/block.py:56-71: cache.gather -> index_select of the whole
// history, engine/cache/kv_cache.py:141-165, then the dense Triton kernel):
// K and V are read once, straight out of the (num_blocks, block_size, Hk, D)
// pool through the int32 block table.
//
// One wave per (sequence, context split, query tile, kv head). The kv heads
// of one (sequence, split) are adjacent workgroup ids, so the pool blocks they
// share (block_size * Hk * D contiguous elements) are read at the same time.
// All Hq/Hk query heads x Lq new tokens of a kv head (R = group * Lq rows, up
// to 32 per query tile) share each K/V byte.
//
// Memory path: the split's block ids are staged in LDS; K and V tiles of 32
// tokens are copied global -> LDS by 16-byte direct-to-LDS loads into a ring
// of NST stages (NST-1 tiles in flight, no VGPR staging). Rows are stored
// with their 16-byte chunks XOR-swizzled (chunk_swizzle) so the fragment
// reads below are conflict-free.
// Per tile:
//   S^T[32 x 32] = K_tile . Q^T    A operand: ds_read_b128 of one token row
//   online softmax in registers (one v_permlane32_swap per reduction)
//   O^T += V^T_tile . P^T          A operand: ds_read_b64_tr_b16 turns the
//                                   row-major V tile into key-contiguous V^T
// A wave whose sequence has a single split writes the final output; otherwise
// it writes (m, l, acc) partials that paged_reduce_kernel combines.
#include "kernels.hpp"

namespace cie {

constexpr float kLazyRescalePaged = 8.0f;

template <int D>
struct PagedCfg {
  static constexpr int KK = D / 16;
  static constexpr int DT = D >= 32 ? D / 32 : 1;
  static constexpr int S = D / 8;                         // 16-byte chunks per token row
  static constexpr int NDMA = S / 2;                      // 1 KiB loads per tensor per tile
  static constexpr int NST = D <= 64 ? 3 : 2;
  static constexpr int TILE = kPagedTile * D;             // elements of one tensor tile
  static constexpr int STAGE = 2 * TILE;                  // K tile, then V tile
};

template <int N, int NDMA>
__device__ __forceinline__ void wait_tiles_ahead(int ahead) {
  // vmcnt counts the 2 * NDMA loads of every tile issued after the one needed
  if (N > 3 && ahead >= 3) vm_wait<(N > 3 ? 3 : 0) * 2 * NDMA>();
  else if (N > 2 && ahead == 2) vm_wait<(N > 2 ? 2 : 0) * 2 * NDMA>();
  else if (N > 1 && ahead == 1) vm_wait<2 * NDMA>();
  else vm_wait<0>();
}

template <int DTYPE, int D>
__global__ __launch_bounds__(64) void paged_fwd_kernel(const PagedParams p) {
  using C = PagedCfg<D>;
  using E = Elt<DTYPE>;
  __shared__ __attribute__((aligned(16))) uint16_t ring[C::NST * C::STAGE];
  __shared__ int32_t sbt[kPagedMaxSplitBlocks];

  // blockIdx.x = ((b * n_splits + s) * n_qt + qt) * Hk + kvh
  int id = blockIdx.x;
  const int kvh = id % p.Hk;
  id /= p.Hk;
  const int qt = id % p.n_qt;
  id /= p.n_qt;
  const int s = id % p.n_splits;
  const int b = id / p.n_splits;
  const int lane = threadIdx.x, l32 = lane & 31, hl = lane >> 5;

  int ctx = p.lens[b];
  const bool bad_len = ctx < 0 || ctx > p.max_blocks * p.block_size || ctx > p.n_splits * p.split_len ||
                       (ctx > 0 && p.num_blocks < 1);
  if (bad_len) ctx = 0;  // never dereference; the output is poisoned below
  const int nsb = max(1, (ctx + p.split_len - 1) / p.split_len);
  if (s >= nsb) return;
  const int split0 = s * p.split_len;
  const int split1 = min(ctx, split0 + p.split_len);
  const int ntiles = split1 > split0 ? (split1 - split0 + kPagedTile - 1) / kPagedTile : 0;

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

  // Stage the split's block ids (validated) in LDS.
  const int blk0 = ntiles ? (int)fdiv((uint32_t)split0, p.bsdiv) : 0;
  const int nblk = ntiles ? (int)fdiv((uint32_t)(split1 - 1), p.bsdiv) - blk0 + 1 : 0;
  bool bad_blk = false;
  const int32_t* btr = p.bt + (int64_t)b * p.max_blocks;
  for (int j = lane; j < nblk; j += 64) {
    const int bid = btr[blk0 + j];
    const bool inb = bid >= 0 && bid < p.num_blocks;
    bad_blk |= !inb;
    sbt[j] = inb ? bid : 0;
  }
  const bool any_bad = __builtin_amdgcn_ballot_w64(bad_blk) != 0;
  // Q and the block ids are in registers / LDS before the first LDS DMA is
  // issued; an explicit wait here keeps the compiler from draining the DMA
  // queue inside the tile loop on their account.
  vm_wait<0>();

  // Last key visible to this row: the Lq new tokens are the newest Lq
  // positions of the context (bottom-right causal alignment). lim_min is the
  // smallest lim of the wave; tiles entirely at or below it need no mask.
  const int lim = min(split1 - 1, p.causal ? ctx - p.Lq + i : ctx - 1);
  const int lim_min = min(split1 - 1, p.causal ? ctx - p.Lq : ctx - 1);
  const float c = p.scale_log2;

  const uint16_t* kbase = p.kc + kvh * p.ks2;
  const uint16_t* vbase = p.vc + kvh * p.vs2;
  const int last = split1 - 1;

  // Tile copy: load j of a tile moves 16-byte chunk P = 64 j + lane, i.e.
  // chunk (P % S) XOR swizzle of token P / S. Per-lane parts are fixed.
  int ltok[C::NDMA], lchk[C::NDMA];
#pragma unroll
  for (int j = 0; j < C::NDMA; ++j) {
    const int P = 64 * j + lane;
    ltok[j] = P / C::S;
    lchk[j] = 8 * ((P % C::S) ^ chunk_swizzle<C::S>(ltok[j]));
  }
  // Copy tile k (tokens split0 + 32k ...) into ring stage k % NST. Tokens past
  // the split are clamped to its last token (masked as scores, zero weight).
  auto issue = [&](int k) {
    const int t0 = split0 + kPagedTile * k;
    uint16_t* st = ring + (k % C::NST) * C::STAGE;
    int bid[C::NDMA], off[C::NDMA];
#pragma unroll
    for (int j = 0; j < C::NDMA; ++j) {  // all block-id reads in flight together
      const int t = min(t0 + ltok[j], last);
      const uint32_t blk = fdiv((uint32_t)t, p.bsdiv);
      off[j] = t - (int)blk * p.block_size;
      bid[j] = sbt[blk - blk0];
    }
    if (p.narrow) {  // pool offsets < 2^31 elements, ids and strides < 2^24: 24-bit multiplies
#pragma unroll
      for (int j = 0; j < C::NDMA; ++j) {
        const uint32_t ko = __umul24(bid[j], p.ks0_24) + __umul24(off[j], p.ks1_24) + lchk[j];
        const uint32_t vo = __umul24(bid[j], p.vs0_24) + __umul24(off[j], p.vs1_24) + lchk[j];
        dma16(kbase + ko, st + 512 * j);
        dma16(vbase + vo, st + C::TILE + 512 * j);
      }
    } else {
#pragma unroll
      for (int j = 0; j < C::NDMA; ++j) {
        dma16(kbase + (int64_t)bid[j] * p.ks0 + (int64_t)off[j] * p.ks1 + lchk[j], st + 512 * j);
        dma16(vbase + (int64_t)bid[j] * p.vs0 + (int64_t)off[j] * p.vs1 + lchk[j], st + C::TILE + 512 * j);
      }
    }
  };

  f32x16 acc[C::DT];
#pragma unroll
  for (int dt = 0; dt < C::DT; ++dt) acc[dt] = f32x16{};
  float m = -INFINITY, l = 0.f;

  const int pro = min(C::NST - 1, ntiles);
  for (int k = 0; k < pro; ++k) issue(k);
  for (int n = 0; n < ntiles; ++n) {
    if (n + C::NST - 1 < ntiles) {
      lgkm_wait0();  // the previous tile's LDS reads of the recycled stage are done
      issue(n + C::NST - 1);
    }
    wait_tiles_ahead<C::NST, C::NDMA>(min(C::NST - 1, ntiles - 1 - n));
    const uint16_t* kst = ring + (n % C::NST) * C::STAGE;
    const uint16_t* vst = kst + C::TILE;
    const int t0 = split0 + kPagedTile * n;

    f32x16 sc = f32x16{};
#pragma unroll
    for (int kk = 0; kk < C::KK; ++kk) {
      const int slot = (2 * kk + hl) ^ chunk_swizzle<C::S>(l32);
      const u32x4 a = *reinterpret_cast<const u32x4*>(kst + (l32 * C::S + slot) * 8);
      sc = E::mfma(a, qf[kk], sc);
    }

    if (t0 + kPagedTile - 1 > lim_min) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int key = t0 + 8 * (e >> 2) + 4 * hl + (e & 3);
        sc[e] = key <= lim ? sc[e] : -INFINITY;
      }
    }
    const float mx = max16(sc);
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
#pragma unroll
    for (int e = 0; e < 16; ++e) sc[e] = exp2_fast(fmaf(sc[e], c, neg_m));
    l += sum16(sc);
    u32x4 pb[2];
#pragma unroll
    for (int cc = 0; cc < 2; ++cc)
#pragma unroll
      for (int w = 0; w < 4; ++w) pb[cc][w] = E::pack2(sc[8 * cc + 2 * w], sc[8 * cc + 2 * w + 1]);

    // V^T fragments: lane (group gq = lane/16, r = lane%16) points at token
    // k0 + r/4, dims d0 + 4*(r%4); the transpose read hands lane l the four
    // keys k0..k0+3 of dim 32*dt + lane%32.
    const int rq = lane & 15, gq = lane >> 4;
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) {
      int d = 32 * dt + 16 * (gq & 1) + 4 * (rq & 3);
      if (D < 32) d = min(d, D - 4);  // rows >= D of O^T are discarded
      const int chunk = d >> 3, within = d & 7;
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
        const int tlo = 16 * cc + 4 * hl + (rq >> 2);
        const int thi = tlo + 8;
        const u32x2 lo = lds_read_tr16(vst + (tlo * C::S + (chunk ^ chunk_swizzle<C::S>(tlo))) * 8 + within);
        const u32x2 hi = lds_read_tr16(vst + (thi * C::S + (chunk ^ chunk_swizzle<C::S>(thi))) * 8 + within);
        acc[dt] = E::mfma(u32x4{lo[0], lo[1], hi[0], hi[1]}, pb[cc], acc[dt]);
      }
    }
  }

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
  // Longest split (<= 512 tokens) that still yields about 1.5k waves at the
  // longest context; the split's block ids must fit the LDS staging area.
  const int64_t pairs = (int64_t)B * Hk * n_qt;
  const int64_t cap = std::max<int64_t>(kPagedTile, (int64_t)(kPagedMaxSplitBlocks - 2) * block_size);
  int split = 512;
  while (split > kPagedTile && (split > cap || pairs * ((max_ctx + split - 1) / split) < 1536)) split /= 2;
  return split;
}

template <int DTYPE, int D>
static hipError_t launch_paged_t(const PagedParams& p, hipStream_t stream) {
  const int64_t n_wg = (int64_t)p.B * p.n_splits * p.n_qt * p.Hk;
  hipLaunchKernelGGL((paged_fwd_kernel<DTYPE, D>), dim3((unsigned)n_wg), dim3(64), 0, stream, p);
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
