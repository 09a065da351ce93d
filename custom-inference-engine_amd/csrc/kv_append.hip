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
#include "rope.hpp"

namespace cie {

constexpr int kAppendUnroll = 4;  // chunks per thread per trip, all loads in flight together

// The pool rows are written once: those stores carry the non-temporal hint
// (a 4 x 2048-token append in 6.9 us instead of 8.9). The new rows are read
// with ordinary loads, which leave them in the caches for the prefill
// attention that reads the same K/V next (non-temporal loads made the
// append-then-attention section 3.5 % slower); the dense rotated copy of K
// (k_out), read by that attention too, is written normally.

__global__ __launch_bounds__(256) void kv_append_kernel(const AppendParams p) {
  warm_kernargs<sizeof(AppendParams)>();
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
        __builtin_nontemporal_store(kv[u], reinterpret_cast<u32x4*>(p.kc + dk[u]));
        __builtin_nontemporal_store(vv[u], reinterpret_cast<u32x4*>(p.vc + dv[u]));
      }
    }
  }
  if (p.status && __builtin_amdgcn_ballot_w64(bad) != 0 && (threadIdx.x & 63) == 0) atomicOr(p.status, 1u);
}

// With RoPE on K (rope/rope.hpp restates kernels/ref/rope_apply_ref.py:46-53):
// one thread moves the chunk pair (j, j + D/16) of one head of one token, K
// rotated at position start[b] + i through the tables, V copied, both
// pairs written to the pool and the rotated K optionally also to the dense
// k_out rows (what prefill attention over the new tokens reads).
constexpr int kRopeUnroll = 2;

template <int DTYPE>
__global__ __launch_bounds__(256) void kv_append_rope_kernel(const AppendParams p) {
  warm_kernargs<sizeof(AppendParams)>();
  const int b = blockIdx.y;
  const int n0 = p.cu_new[b];
  const int L = p.cu_new[b + 1] - n0;
  if (L <= 0) return;
  const int start = p.start[b];
  const uint32_t upr = p.cpr >> 1;            // chunk pairs per token row
  const uint32_t total = (uint32_t)L * upr;
  const uint32_t lg_half = p.lg_cph - 1u;     // log2(D / 16)
  const int half = 4 << p.lg_cph;             // D / 2 elements
  const int32_t* btr = p.bt + (int64_t)b * p.max_blocks;
  const int limit = p.max_blocks * p.block_size;
  const uint32_t stride = gridDim.x * 256u;
  uint32_t bad = 0;
  for (uint32_t c0 = blockIdx.x * 256u + threadIdx.x; c0 < total; c0 += kRopeUnroll * stride) {
    u32x4 klo[kRopeUnroll], khi[kRopeUnroll], vlo[kRopeUnroll], vhi[kRopeUnroll];
    RopeChunk cs[kRopeUnroll];
    int64_t dk[kRopeUnroll], dv[kRopeUnroll], dout[kRopeUnroll];
    bool in[kRopeUnroll], ok[kRopeUnroll];
#pragma unroll
    for (int u = 0; u < kRopeUnroll; ++u) {
      const uint32_t c = c0 + u * stride;
      in[u] = c < total;
      const uint32_t cc = in[u] ? c : c0;  // clamped: every load stays inside the sources
      const uint32_t i = fdiv(cc, p.updiv);
      const uint32_t ch = cc - i * upr;
      const uint32_t h = ch >> lg_half, j = ch & ((1u << lg_half) - 1u);
      const int pos = start + (int)i;
      const bool rope_ok = pos >= 0 && pos < p.rope.rows;
      const bool pos_ok = pos >= 0 && pos < limit;
      const int blk = pos_ok ? (int)fdiv((uint32_t)pos, p.bsdiv) : 0;
      const int off = pos_ok ? pos - blk * p.block_size : 0;
      const int bid = pos_ok ? btr[blk] : -1;
      const bool bid_ok = (uint32_t)bid < (uint32_t)p.num_blocks;
      ok[u] = in[u] && rope_ok && pos_ok && bid_ok;
      bad |= (in[u] && !(pos_ok && bid_ok)) ? 1u : 0u;
      bad |= (in[u] && !rope_ok) ? 2u : 0u;
      in[u] = in[u] && rope_ok;
      const int64_t row = (int64_t)(n0 + (int)i);
      const uint16_t* ks = p.k_new + row * p.ns0 + h * p.ns1 + 8 * j;
      const uint16_t* vs = p.v_new + row * p.ms0 + h * p.ms1 + 8 * j;
      klo[u] = *reinterpret_cast<const u32x4*>(ks);
      khi[u] = *reinterpret_cast<const u32x4*>(ks + half);
      vlo[u] = *reinterpret_cast<const u32x4*>(vs);
      vhi[u] = *reinterpret_cast<const u32x4*>(vs + half);
      const int64_t tr = (rope_ok ? (int64_t)pos : 0) * half + 8 * j;
      cs[u] = rope_load(p.rope, tr);
      dk[u] = (int64_t)bid * p.ks0 + (int64_t)off * p.ks1 + h * p.ks2 + 8 * j;
      dv[u] = (int64_t)bid * p.vs0 + (int64_t)off * p.vs1 + h * p.vs2 + 8 * j;
      dout[u] = row * p.os0 + h * p.os1 + 8 * j;
    }
#pragma unroll
    for (int u = 0; u < kRopeUnroll; ++u) {
      rope_apply8<DTYPE>(klo[u], khi[u], cs[u], p.rope.dt);
      if (ok[u]) {
        __builtin_nontemporal_store(klo[u], reinterpret_cast<u32x4*>(p.kc + dk[u]));
        __builtin_nontemporal_store(khi[u], reinterpret_cast<u32x4*>(p.kc + dk[u] + half));
        __builtin_nontemporal_store(vlo[u], reinterpret_cast<u32x4*>(p.vc + dv[u]));
        __builtin_nontemporal_store(vhi[u], reinterpret_cast<u32x4*>(p.vc + dv[u] + half));
      }
      if (p.k_out && in[u]) {
        *reinterpret_cast<u32x4*>(p.k_out + dout[u]) = klo[u];
        *reinterpret_cast<u32x4*>(p.k_out + dout[u] + half) = khi[u];
      }
    }
  }
  if (p.status) {
    const uint32_t any1 = __builtin_amdgcn_ballot_w64((bad & 1u) != 0) != 0 ? 1u : 0u;
    const uint32_t any2 = __builtin_amdgcn_ballot_w64((bad & 2u) != 0) != 0 ? 2u : 0u;
    if ((any1 | any2) && (threadIdx.x & 63) == 0) atomicOr(p.status, any1 | any2);
  }
}

hipError_t launch_kv_append(const AppendParams& p, int B, int max_new, int dtype, int D, hipStream_t stream) {
  if (B <= 0 || max_new <= 0) return hipSuccess;
  (void)D;
  if (p.rope.cos) {
    const int64_t pairs = (int64_t)max_new * (p.cpr >> 1);
    const int gx = (int)std::min<int64_t>(1024, (pairs + 256 * kRopeUnroll - 1) / (256 * kRopeUnroll));
    if (dtype == 0)
      hipLaunchKernelGGL(kv_append_rope_kernel<0>, dim3(gx, B), dim3(256), 0, stream, p);
    else
      hipLaunchKernelGGL(kv_append_rope_kernel<1>, dim3(gx, B), dim3(256), 0, stream, p);
    return hipGetLastError();
  }
  // enough workgroups for one trip over the longest sequence, at most 1024 per sequence
  const int64_t chunks = (int64_t)max_new * p.cpr;
  const int gx = (int)std::min<int64_t>(1024, (chunks + 256 * kAppendUnroll - 1) / (256 * kAppendUnroll));
  hipLaunchKernelGGL(kv_append_kernel, dim3(gx, B), dim3(256), 0, stream, p);
  return hipGetLastError();
}

}  // namespace cie
