// Paged KV append for gfx950: writes the new tokens of a batch of sequences
// into the (num_blocks, block_size, Hk, D) pool through int32 block tables.
//
// Replaces the reference's per-block slice loop of PagedKVCache.append
// (engine/cache/kv_cache.py:128-136: one k and one v slice assignment per
// block spanned, per layer, per sequence) and the host-to-device copy of the
// block ids each gather makes (kv_cache.py:154): one launch per layer moves
// every new token of every sequence, reading the block table already on the
// device (the same table paged attention reads).
//
// Token i of sequence b (rows cu_new[b] + i of k_new / v_new) lands at
// position start[b] + i, i.e. pool[block_tables[b][pos / bs], pos % bs].
// One thread moves one 16-byte chunk of K and the same chunk of V; the
// chunks of one token row are consecutive threads, so both the source rows
// and the pool rows (Hk * D contiguous elements per token) are read and
// written fully coalesced. A position outside the table or a block id outside
// [0, num_blocks) is never written; the launch then sets *status to 1 when a
// status word is given.
#include "kernels.hpp"

namespace cie {

constexpr int kAppendUnroll = 4;  // chunks per thread per trip, all loads in flight together

__global__ __launch_bounds__(256) void kv_append_kernel(const AppendParams p) {
  const int b = blockIdx.y;
  const int n0 = p.cu_new[b];
  const int L = p.cu_new[b + 1] - n0;
  if (L <= 0) return;
  const int start = p.start[b];
  const uint32_t total = (uint32_t)L * p.cpr;  // chunks of this sequence (< 2^31, checked on the host)
  const int32_t* btr = p.bt + (int64_t)b * p.max_blocks;
  const int limit = p.max_blocks * p.block_size;
  const uint32_t stride = gridDim.x * 256u;
  bool bad = false;
  for (uint32_t c0 = blockIdx.x * 256u + threadIdx.x; c0 < total; c0 += kAppendUnroll * stride) {
    u32x4 kv[kAppendUnroll], vv[kAppendUnroll];
    int64_t dk[kAppendUnroll], dv[kAppendUnroll];
    bool ok[kAppendUnroll];
#pragma unroll
    for (int u = 0; u < kAppendUnroll; ++u) {
      const uint32_t c = c0 + u * stride;
      const bool in = c < total;
      const uint32_t cc = in ? c : c0;  // clamped: every load stays inside the sources
      const uint32_t i = fdiv(cc, p.cprdiv);
      const uint32_t ch = cc - i * p.cpr;
      const uint32_t h = ch >> p.lg_cph, d8 = ch & ((1u << p.lg_cph) - 1u);
      const int pos = start + (int)i;
      const bool pos_ok = pos >= 0 && pos < limit;
      const int blk = pos_ok ? (int)fdiv((uint32_t)pos, p.bsdiv) : 0;
      const int off = pos_ok ? pos - blk * p.block_size : 0;
      const int bid = pos_ok ? btr[blk] : -1;
      const bool bid_ok = (uint32_t)bid < (uint32_t)p.num_blocks;
      ok[u] = in && pos_ok && bid_ok;
      bad |= in && !(pos_ok && bid_ok);
      const int64_t row = (int64_t)(n0 + (int)i);
      kv[u] = *reinterpret_cast<const u32x4*>(p.k_new + row * p.ns0 + h * p.ns1 + 8 * d8);
      vv[u] = *reinterpret_cast<const u32x4*>(p.v_new + row * p.ms0 + h * p.ms1 + 8 * d8);
      dk[u] = (int64_t)bid * p.ks0 + (int64_t)off * p.ks1 + h * p.ks2 + 8 * d8;
      dv[u] = (int64_t)bid * p.vs0 + (int64_t)off * p.vs1 + h * p.vs2 + 8 * d8;
    }
#pragma unroll
    for (int u = 0; u < kAppendUnroll; ++u) {
      if (ok[u]) {
        *reinterpret_cast<u32x4*>(p.kc + dk[u]) = kv[u];
        *reinterpret_cast<u32x4*>(p.vc + dv[u]) = vv[u];
      }
    }
  }
  if (p.status && __builtin_amdgcn_ballot_w64(bad) != 0 && (threadIdx.x & 63) == 0) atomicOr(p.status, 1u);
}

hipError_t launch_kv_append(const AppendParams& p, int B, int max_new, hipStream_t stream) {
  if (B <= 0 || max_new <= 0) return hipSuccess;
  // enough workgroups for one trip over the longest sequence, at most 1024 per sequence
  const int64_t chunks = (int64_t)max_new * p.cpr;
  const int gx = (int)std::min<int64_t>(1024, (chunks + 256 * kAppendUnroll - 1) / (256 * kAppendUnroll));
  hipLaunchKernelGGL(kv_append_kernel, dim3(gx, B), dim3(256), 0, stream, p);
  return hipGetLastError();
}

}  // namespace cie
