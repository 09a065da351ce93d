// Standalone rotary position embedding for gfx950: out = RoPE(x) for
// x (B, H, L, D), the operation of RotaryEmbedding.apply
// (engine/model/rope.py:18-19 -> kernels/ref/rope_apply_ref.py:22-53),
// with positions (L,), (B, L) or the default 0..L-1.
//
// One thread rotates one chunk pair (x[j*8 .. +8), x[D/2 + j*8 .. +8)) of one
// row; consecutive threads take consecutive pairs of a row, then the next
// row, so the loads and stores of a wave cover whole row halves. The fp32
// cos/sin rows (D/2 floats each) are read through L2, where every head of a
// position shares them. A position outside the table yields NaN for the row
// and ORs 2 into the status word (the reference's table indexing raises there).
#include "kernels.hpp"
#include "rope.hpp"

namespace cie {

template <int DTYPE, int D>
__global__ __launch_bounds__(256) void rope_kernel(const RopeParams p) {
  constexpr uint32_t UPR = D / 16;  // chunk pairs per row
  constexpr int HALF = D / 2;
  const uint32_t stride = gridDim.x * 256u;
  bool bad = false;
  for (uint32_t u = blockIdx.x * 256u + threadIdx.x; u < p.total; u += stride) {
    const uint32_t row = u / UPR, j = u % UPR;
    const uint32_t bh = fdiv(row, p.ldiv);
    const int l = (int)(row - bh * (uint32_t)p.L);
    const uint32_t b = fdiv(bh, p.hdiv);
    const int h = (int)(bh - b * (uint32_t)p.H);
    const int pos = p.pos ? p.pos[(int64_t)b * p.pos_bs + l] : l;
    const bool ok = pos >= 0 && pos < p.tab.rows;
    bad |= !ok;
    const int64_t tr = (ok ? (int64_t)pos : 0) * HALF + 8 * j;
    const uint16_t* x = p.x + (int64_t)b * p.xs0 + (int64_t)h * p.xs1 + (int64_t)l * p.xs2 + 8 * j;
    u32x4 lo = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(x));  // streamed once
    u32x4 hi = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(x + HALF));
    rope8<DTYPE>(lo, hi, tab8(p.tab.cos + tr), tab8(p.tab.sin + tr));
    if (!ok) lo = hi = u32x4{0x7fff7fffu, 0x7fff7fffu, 0x7fff7fffu, 0x7fff7fffu};
    uint16_t* o = p.out + (int64_t)b * p.os0 + (int64_t)h * p.os1 + (int64_t)l * p.os2 + 8 * j;
    *reinterpret_cast<u32x4*>(o) = lo;  // cached: attention reads the rotated rows next
    *reinterpret_cast<u32x4*>(o + HALF) = hi;
  }
  if (p.status && __builtin_amdgcn_ballot_w64(bad) != 0 && (threadIdx.x & 63) == 0) atomicOr(p.status, 2u);
}

template <int DTYPE>
static hipError_t launch_rope_d(const RopeParams& p, int D, int grid, hipStream_t stream) {
  switch (D) {
    case 16: hipLaunchKernelGGL((rope_kernel<DTYPE, 16>), dim3(grid), dim3(256), 0, stream, p); break;
    case 32: hipLaunchKernelGGL((rope_kernel<DTYPE, 32>), dim3(grid), dim3(256), 0, stream, p); break;
    case 64: hipLaunchKernelGGL((rope_kernel<DTYPE, 64>), dim3(grid), dim3(256), 0, stream, p); break;
    case 128: hipLaunchKernelGGL((rope_kernel<DTYPE, 128>), dim3(grid), dim3(256), 0, stream, p); break;
    case 256: hipLaunchKernelGGL((rope_kernel<DTYPE, 256>), dim3(grid), dim3(256), 0, stream, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_rope(const RopeParams& p, int dtype, int D, hipStream_t stream) {
  if (p.total == 0) return hipSuccess;
  // one pair per thread up to 64K workgroups, grid-stride beyond
  const int grid = (int)std::min<uint32_t>(65536u, (p.total + 255u) / 256u);
  return dtype == 0 ? launch_rope_d<0>(p, D, grid, stream) : launch_rope_d<1>(p, D, grid, stream);
}

}  // namespace cie
