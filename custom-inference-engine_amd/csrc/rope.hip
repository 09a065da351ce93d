// Standalone rotary position embedding for gfx950: out = RoPE(x) for
// x (B, H, L, D), the operation of RotaryEmbedding.apply
// (engine/model/rope.py:18-19 -> kernels/ref/rope_apply_ref.py:22-53),
// with positions (L,), (B, L) or the default 0..L-1.
//
// One thread rotates one chunk pair (x[j*8 .. +8), x[D/2 + j*8 .. +8)) of
// one position l in each of up to HG heads (HG = kRopeHeads for launches
// large enough to keep 512 workgroups, else 1): the cos/sin row chunks of
// the position (read through L2) are loaded once for all of them, and
// the thread's 2 * HG row loads are in flight together.
// Consecutive threads take consecutive chunk pairs of a row, then the next
// position, so for every head the loads and stores of a wave cover
// contiguous row halves. A position outside the table yields NaN for the
// row and ORs 2 into the status word (the reference's table indexing raises
// there).
#include "kernels.hpp"
#include "rope.hpp"

namespace cie {

template <int DTYPE, int D, int HG>
__global__ __launch_bounds__(256) void rope_kernel(const RopeParams p) {
  warm_kernargs<sizeof(RopeParams)>();
  constexpr uint32_t UPR = D / 16;  // chunk pairs per row
  constexpr int HALF = D / 2;
  const uint32_t stride = gridDim.x * 256u;
  bool bad = false;
  for (uint32_t u = blockIdx.x * 256u + threadIdx.x; u < p.total; u += stride) {
    const uint32_t r = u / UPR, j = u % UPR;  // r = (b * NHG + hg) * L + l
    const uint32_t bg = fdiv(r, p.ldiv);
    const int l = (int)(r - bg * (uint32_t)p.L);
    const uint32_t b = fdiv(bg, p.hgdiv);
    const int h0 = (int)(bg - b * (uint32_t)p.NHG) * HG;
    const int nh = min(HG, p.H - h0);
    const int pos = p.pos ? p.pos[(int64_t)b * p.pos_bs + l] : l;
    const bool ok = pos >= 0 && pos < p.tab.rows;
    bad |= !ok;
    const int64_t tr = (ok ? (int64_t)pos : 0) * HALF + 8 * j;
    const RopeChunk cs = rope_load(p.tab, tr);
    const uint16_t* x = p.x + (int64_t)b * p.xs0 + (int64_t)h0 * p.xs1 + (int64_t)l * p.xs2 + 8 * j;
    uint16_t* o = p.out + (int64_t)b * p.os0 + (int64_t)h0 * p.os1 + (int64_t)l * p.os2 + 8 * j;
    u32x4 lo[HG], hi[HG];
#pragma unroll
    for (int e = 0; e < HG; ++e) {
      if (e < nh) {
        lo[e] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(x + e * p.xs1));  // streamed once
        hi[e] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(x + e * p.xs1 + HALF));
      }
    }
#pragma unroll
    for (int e = 0; e < HG; ++e) {
      if (e < nh) {
        rope_apply8<DTYPE>(lo[e], hi[e], cs, p.tab.dt);
        if (!ok) lo[e] = hi[e] = u32x4{0x7fff7fffu, 0x7fff7fffu, 0x7fff7fffu, 0x7fff7fffu};
        *reinterpret_cast<u32x4*>(o + e * p.os1) = lo[e];  // cached: attention reads the rotated rows next
        *reinterpret_cast<u32x4*>(o + e * p.os1 + HALF) = hi[e];
      }
    }
  }
  if (p.status && __builtin_amdgcn_ballot_w64(bad) != 0 && (threadIdx.x & 63) == 0) atomicOr(p.status, 2u);
}

template <int DTYPE, int HG>
static hipError_t launch_rope_g(const RopeParams& p, int D, int grid, hipStream_t stream) {
  switch (D) {
    case 16: hipLaunchKernelGGL((rope_kernel<DTYPE, 16, HG>), dim3(grid), dim3(256), 0, stream, p); break;
    case 32: hipLaunchKernelGGL((rope_kernel<DTYPE, 32, HG>), dim3(grid), dim3(256), 0, stream, p); break;
    case 64: hipLaunchKernelGGL((rope_kernel<DTYPE, 64, HG>), dim3(grid), dim3(256), 0, stream, p); break;
    case 128: hipLaunchKernelGGL((rope_kernel<DTYPE, 128, HG>), dim3(grid), dim3(256), 0, stream, p); break;
    case 256: hipLaunchKernelGGL((rope_kernel<DTYPE, 256, HG>), dim3(grid), dim3(256), 0, stream, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int DTYPE>
static hipError_t launch_rope_d(const RopeParams& p, int D, int grid, hipStream_t stream) {
  if (p.HG == kRopeHeads) return launch_rope_g<DTYPE, kRopeHeads>(p, D, grid, stream);
  if (p.HG == 1) return launch_rope_g<DTYPE, 1>(p, D, grid, stream);
  return hipErrorInvalidValue;
}

hipError_t launch_rope(const RopeParams& p, int dtype, int D, hipStream_t stream) {
  if (p.total == 0) return hipSuccess;
  // one chunk pair of a head group per thread up to 64K workgroups, grid-stride beyond
  const int grid = (int)std::min<uint32_t>(65536u, (p.total + 255u) / 256u);
  return dtype == 0 ? launch_rope_d<0>(p, D, grid, stream) : launch_rope_d<1>(p, D, grid, stream);
}

}  // namespace cie
