// The steady-state pipeline step of the head_dim-64 head-pair prefill kernel
// (flash_fwd_r64_kernel), rebuilt in a loop with its parts switched on one at
// a time, so that what each part costs, and how far the full step can run
// at all, is measured rather than estimated.
//
// One step of one wave, as in the kernel: 64 query rows (two row groups of
// 32) against a 32-key tile at head_dim 64, fp16:
//   QK   8 MFMAs 32x32x16 for S(t+1) = K . Q^T (four k-blocks, two row groups)
//   SM   the softmax of S(t): 32 fma (fp32 scale and -m) + 32 v_exp_f32 + 16
//        packs to fp16, interleaved with the QK MFMAs (four scores after each)
//   SUM  8 row-sum MFMAs 4x4x4 (A all ones) over the packed p (their sums are
//        used only by the check below, so the two go together)
//   (always) the fragment reads: 4 ds_read_b128 of K, 8 ds_read_b64_tr_b16
//        of V (without them the compiler would hoist the MFMAs of constant
//        operands out of the loop)
//   CHK  the lazy-max check: one cross-half sum per row group, a ballot and a
//        branch (never taken here)
//   PV   8 MFMAs 32x32x16 for O += V^T . P^T (two 16-key blocks, two output
//        tiles, two row groups)
//   BAR  one workgroup barrier per step
//   CPY  the tile copies: every wave moves 2 KiB of tile t+3 with
//        global_load_lds_dwordx4 into a four-stage ring, after waiting for
//        tile t+1 (tile t+2 still in flight), as the kernel does (the
//        source, 256 KiB per group of 32 workgroups, stays in L2: the
//        kernel's K/V come from HBM and L2)
//   PRIO the QK/softmax phase at raised wave priority, as in the kernel
// Four-wave workgroups, two per CU (two waves per SIMD, as the kernel), or
// one per CU; a four-stage ring as the kernel's, or eight stages; the copy
// source L2-resident or a 64 MiB region every workgroup walks through. All LDS addresses stay inside the workgroup's 32 KiB; the
// global source is sized for the grid; the exponent inputs stay below zero.
//
// Each configuration first runs back to back for ~0.2 s (clock settle), then
// one launch is timed (HIP events) while wave 0 of workgroup 0 reads the
// shader-clock and 100 MHz real-time counters around its loop, and every
// wave records its own shader cycles for the loop. Printed per row: kernel
// time, clock, the SIMD time per wave-step (kernel time x clock over the
// steps of the SIMD's waves), a wave's own loop cycles per step (shorter
// than the SIMD time when the two workgroups of a CU do not run the whole
// loop side by side), and the useful MFMA work (16 MFMAs of 32x32x16 per
// wave and step) per kernel time: against the MFMA-only row, in TFLOP/s and
// as a fraction of the 2516.6 TFLOP/s dense fp16 peak.
//
// Built by build_lib.py (custom-inference-engine_amd/_build/prefill_step);
// run through benchmarks/prefill_step.py.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <algorithm>
#include <vector>

#include "common.hpp"

using namespace cie;

#define CHECK(x)                                                                          \
  do {                                                                                    \
    hipError_t e_ = (x);                                                                  \
    if (e_ != hipSuccess) {                                                               \
      std::fprintf(stderr, "HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); \
      std::exit(1);                                                                       \
    }                                                                                     \
  } while (0)

enum : unsigned {
  QK = 1u,
  SM = 2u,
  SUM = 4u,
  CHK = 16u,
  PV = 32u,
  BAR = 64u,
  CPY = 128u,
  PRIO = 256u,
  NOEXP = 512u,  // SM with a v_max in place of each v_exp_f32 (same data flow)
  FAR = 1024u,   // CPY from a 64 MiB source: L2 misses that the Infinity Cache serves
};

constexpr int kIters = 2000;  // steps per wave (even)
constexpr int kStage = 4096;     // fp16 elements of one K + V tile stage (8 KiB: 32 keys x 64 x 2 tensors)
constexpr int kSrcTiles = 32;    // tiles of the copy source per group of 32 workgroups
constexpr int kFarTiles = 8192;  // tiles of the FAR source (64 MiB)

// NSTG ring stages of 8 KiB: 4 as the kernel (tile t+1 waited for, t+2 in
// flight), 8 for three tiles in flight.
template <unsigned F, int OCC, int NSTG>
__global__ __launch_bounds__(256, OCC) void step_kernel(float* out, long long* cyc, long long* clk,
                                                        const uint16_t* src, float c) {
  using E = Elt<0>;
  constexpr int kStages = NSTG;
  __shared__ __attribute__((aligned(16))) uint16_t ring[kStages * kStage];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int i = threadIdx.x; i < kStages * kStage; i += 256) ring[i] = (uint16_t)(0x2000 + (i & 63));  // small fp16
  __syncthreads();

  // Q fragments (two row groups x four k-blocks), small values
  u32x4 qf[2][4];
#pragma unroll
  for (int rg = 0; rg < 2; ++rg)
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const uint32_t h = E::pack2(0.01f * (float)(lane % 7 + kk), 0.01f * (float)(rg + 1));
      qf[rg][kk] = u32x4{h, h, h, h};
    }
  const u32x2 sum_ones = {E::pack2(1.f, 1.f), E::pack2(1.f, 1.f)};
  f32x16 sc[2], sn[2], acc[2][2];
#pragma unroll
  for (int rg = 0; rg < 2; ++rg) {
#pragma unroll
    for (int e = 0; e < 16; ++e) sc[rg][e] = 0.01f * (float)(e + lane % 5);
    sn[rg] = f32x16{};
    acc[rg][0] = acc[rg][1] = f32x16{};
  }
  float nm[2] = {-0.5f, -0.25f};
  float l[2] = {0.f, 0.f};
  u32x4 pb[2][2];
#pragma unroll
  for (int rg = 0; rg < 2; ++rg) pb[rg][0] = pb[rg][1] = u32x4{0x3c00u, 0x3c00u, 0x3c00u, 0x3c00u};

  const uint32_t ring_lds = lds_addr_of(ring);
  int taken = 0;

  // One step: sc holds S(t) (its softmax is computed), S(t+1) goes to sn; the
  // loop runs two steps per iteration with the two score sets swapping roles,
  // as the kernel's unrolled loop does (no register moves between steps).
  auto step = [&](const int it, f32x16* sc, f32x16* sn) __attribute__((always_inline)) {
    // K(t+1) is read from stage (it + 1) % 4, V(t) from stage it % 4; the
    // copies refill stage (it + 3) % 4, whose tile t-1 no wave reads any more
    // once every wave has passed this step's barrier
    const int st = it % kStages, st1 = (it + 1) % kStages;
    // tile t+1 landed, this wave's copies of tiles t+2 .. t+NSTG-2 still in flight
    if constexpr ((F & CPY) != 0) vm_wait<2 * (NSTG - 3)>();
    if constexpr ((F & BAR) != 0) __syncthreads();
    if constexpr ((F & CPY) != 0) {
      // this wave's two 1 KiB pieces of tile t+NSTG-1
      const size_t tile = (F & FAR) != 0 ? (size_t)((blockIdx.x * 37u + (unsigned)it) % kFarTiles)
                                         : (size_t)((blockIdx.x >> 5) * kSrcTiles + it % kSrcTiles);
      const void* base = uniform_ptr(src + tile * kStage);
      const uint32_t dst = ring_lds + 2u * (uint32_t)(((it + NSTG - 1) % kStages) * kStage) + 2048u * (uint32_t)wave;
      dma16_sv(base, (uint32_t)(2048 * wave + 16 * lane), dst);
      dma16_sv(base, (uint32_t)(2048 * wave + 1024 + 16 * lane), dst + 1024u);
    }
    if constexpr ((F & PRIO) != 0) __builtin_amdgcn_s_setprio(1);
    f32x4 tsm[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
    {
      const uint16_t* ks = ring + st1 * kStage;
      u32x4 ka[4];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        ka[kk] = *reinterpret_cast<const u32x4*>(ks + 8 * lane + 512 * kk);
      }
      // S(t+1) starts from zero when its softmax is computed; without the
      // softmax the scores accumulate, so the QK^T MFMAs stay live
      if constexpr ((F & SM) != 0) {
#pragma unroll
        for (int rg = 0; rg < 2; ++rg) sn[rg] = f32x16{};
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int kk = i / 2, rgq = i % 2;
        if constexpr ((F & QK) != 0) sn[rgq] = E::mfma(ka[kk], qf[rgq][kk], sn[rgq]);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr ((F & SM) != 0) {
#pragma unroll
          for (int e = 4 * i; e < 4 * i + 4; ++e) {
            const int rg = e / 16, ee = e % 16;
            const float x = fmaf(sc[rg][ee], c, nm[rg]);  // below zero: scores are small, nm < 0
            float p;
            if constexpr ((F & NOEXP) != 0) p = fmaxf(x, -1.f);
            else p = exp2_fast(x);
            sc[rg][ee] = p;
            if (ee & 1) {
              const uint32_t pk = E::pack2(sc[rg][ee - 1], sc[rg][ee]);
              asm volatile("" ::"v"(pk));
              pb[rg][ee >> 3][(ee & 7) >> 1] = pk;
            }
            if constexpr ((F & SUM) != 0) {
              if ((ee & 3) == 3) {
                const int cb = ee >> 3, w = (ee & 7) >> 1;
                tsm[rg] = E::mfma4(sum_ones, u32x2{pb[rg][cb][w - 1], pb[rg][cb][w]}, tsm[rg]);
              }
            }
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if constexpr ((F & PRIO) != 0) __builtin_amdgcn_s_setprio(0);
    if constexpr ((F & CHK) != 0) {
      const float t0 = xhalf_sum(tsm[0][0]), t1 = xhalf_sum(tsm[1][0]);
      if (__builtin_amdgcn_ballot_w64(!(t0 <= 1e30f) || !(t1 <= 1e30f))) {
        nm[0] -= 1.f;  // never: the sums stay finite and far below the trigger
        ++taken;
      }
      l[0] += t0;
      l[1] += t1;
    }
    if constexpr ((F & PV) != 0) {
      const uint16_t* vs = ring + st * kStage + 2048;
      u32x4 va[2][2];
#pragma unroll
      for (int cc = 0; cc < 2; ++cc)
#pragma unroll
        for (int dt = 0; dt < 2; ++dt) {
          const int f = 2 * cc + dt;
          const u32x2 lo = lds_read_tr16(vs + 4 * lane + 512 * f);
          const u32x2 hi = lds_read_tr16(vs + 4 * lane + 512 * f + 256);
          va[dt][cc] = u32x4{lo[0], lo[1], hi[0], hi[1]};
        }
#pragma unroll
      for (int cc = 0; cc < 2; ++cc)
#pragma unroll
        for (int rg = 0; rg < 2; ++rg)
#pragma unroll
          for (int dt = 0; dt < 2; ++dt) acc[rg][dt] = E::mfma(va[dt][cc], pb[rg][cc], acc[rg][dt]);
    }
  };

  const long long c0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
#pragma nounroll
  for (int it = 0; it < kIters; it += 2) {
    step(it, sc, sn);
    step(it + 1, sn, sc);
  }
  vm_wait<0>();
  const long long c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();

  float r = l[0] + l[1] + (float)taken;
#pragma unroll
  for (int rg = 0; rg < 2; ++rg)
#pragma unroll
    for (int e = 0; e < 16; ++e) r += sc[rg][e] + sn[rg][e] + acc[rg][0][e] + acc[rg][1][e];
  out[blockIdx.x * 256 + threadIdx.x] = r;
  if (lane == 0) cyc[blockIdx.x * 4 + wave] = c1 - c0;
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    clk[0] = c1 - c0;
    clk[1] = r1 - r0;
  }
}

struct Bufs {
  float* out;
  long long* cyc;
  long long* clk;
  const uint16_t* src;
  int cus;
};

static double g_base_tflops = 0.0;

template <unsigned F, int OCC, int NSTG = 4>
static void run(const char* name, const Bufs& b) {
  const int grid = b.cus * OCC;
  const float c = 0.18033688f;  // (1/8) log2 e, the head_dim-64 scale
  hipEvent_t w0, w1;
  CHECK(hipEventCreate(&w0));
  CHECK(hipEventCreate(&w1));
  float settled = 0.f;
  while (settled < 200.f) {
    CHECK(hipEventRecord(w0));
    for (int i = 0; i < 8; ++i)
      hipLaunchKernelGGL((step_kernel<F, OCC, NSTG>), dim3(grid), dim3(256), 0, 0, b.out, b.cyc, b.clk, b.src, c);
    CHECK(hipGetLastError());
    CHECK(hipEventRecord(w1));
    CHECK(hipEventSynchronize(w1));
    float ms = 0.f;
    CHECK(hipEventElapsedTime(&ms, w0, w1));
    settled += ms;
  }
  CHECK(hipEventRecord(w0));
  hipLaunchKernelGGL((step_kernel<F, OCC, NSTG>), dim3(grid), dim3(256), 0, 0, b.out, b.cyc, b.clk, b.src, c);
  CHECK(hipGetLastError());
  CHECK(hipEventRecord(w1));
  CHECK(hipDeviceSynchronize());
  float ms = 0.f;
  CHECK(hipEventElapsedTime(&ms, w0, w1));
  CHECK(hipEventDestroy(w0));
  CHECK(hipEventDestroy(w1));
  std::vector<long long> cyc((size_t)grid * 4);
  long long clk[2];
  CHECK(hipMemcpy(cyc.data(), b.cyc, cyc.size() * sizeof(long long), hipMemcpyDeviceToHost));
  CHECK(hipMemcpy(clk, b.clk, sizeof(clk), hipMemcpyDeviceToHost));
  double s = 0.0;
  for (long long v : cyc) s += (double)v;
  const double own = s / (double)cyc.size() / kIters;  // a wave's own loop cycles per step
  const double ghz = clk[1] > 0 ? (double)clk[0] / (double)clk[1] * 0.1 : 0.0;
  // SIMD time per step: kernel time over the OCC waves of a SIMD x kIters steps
  const double simd_cycles = (double)ms * 1e-3 * ghz * 1e9 / ((double)kIters * OCC);
  // useful work: 16 MFMAs 32x32x16 (32768 FLOP each) per wave and step, 4 SIMDs per CU
  const double tflops = 16.0 * 32768.0 * OCC * kIters * 4.0 * b.cus / ((double)ms * 1e-3) / 1e12;
  const double frac = tflops / 2516.6;
  if (g_base_tflops == 0.0) g_base_tflops = tflops;
  std::printf("| %s | %d | %.3f | %.2f | %.0f | %.0f | %.2f | %.0f | %.3f |\n", name, OCC, ms, ghz, simd_cycles, own,
              tflops / g_base_tflops, tflops, frac);
}

int main() {
  Bufs b{};
  int dev = 0;
  CHECK(hipGetDevice(&dev));
  CHECK(hipDeviceGetAttribute(&b.cus, hipDeviceAttributeMultiprocessorCount, dev));
  const int max_grid = b.cus * 2;
  CHECK(hipMalloc(&b.out, (size_t)max_grid * 256 * sizeof(float)));
  CHECK(hipMalloc(&b.cyc, (size_t)max_grid * 4 * sizeof(long long)));
  CHECK(hipMalloc(&b.clk, 2 * sizeof(long long)));
  uint16_t* src;
  const size_t src_elems = std::max((size_t)((max_grid + 31) / 32) * kSrcTiles, (size_t)kFarTiles) * kStage;
  CHECK(hipMalloc(&src, src_elems * sizeof(uint16_t)));
  CHECK(hipMemset(src, 0x20, src_elems * sizeof(uint16_t)));
  b.src = src;
  std::printf("%d CUs, 256-thread workgroups, %d steps per wave\n\n", b.cus, kIters);
  std::printf("| step content | workgroups / CU | kernel ms | clock GHz | SIMD cycles per wave-step | a wave's own cycles per step | MFMA rate vs first row | TFLOP/s | fraction of the 2516.6 TFLOP/s peak |\n");
  std::printf("|---|---:|---:|---:|---:|---:|---:|---:|---:|\n");
  constexpr unsigned MM = QK | PV;
  constexpr unsigned FULL = QK | SM | SUM | CHK | PV | BAR | CPY | PRIO;
  run<MM, 2>("16 MFMA (8 QK^T, 8 P.V) with their LDS fragment reads", b);
  run<MM | SM, 2>("+ softmax: 32 fma, 32 exp2, 16 packs", b);
  run<MM | SM | SUM | CHK, 2>("+ 8 row-sum MFMAs 4x4x4 and the lazy-max check", b);
  run<MM | SM | SUM | CHK | BAR, 2>("+ one barrier per step", b);
  run<MM | SM | SUM | CHK | BAR | CPY, 2>("+ tile copies and their wait", b);
  run<FULL, 2>("+ raised priority of the QK^T phase (the full step)", b);
  run<FULL & ~BAR, 2>("full step without the barrier", b);
  run<FULL & ~PRIO, 2>("full step without the priority raise", b);
  run<FULL | NOEXP, 2>("full step, v_exp_f32 replaced by v_max", b);
  run<FULL, 1>("full step, one wave per SIMD", b);
  run<FULL, 2, 8>("full step, 8-stage ring (three tiles in flight)", b);
  run<FULL | FAR, 2>("full step, copies from a 64 MiB source", b);
  run<FULL | FAR, 2, 8>("full step, copies from a 64 MiB source, 8-stage ring", b);
  CHECK(hipFree(src));
  CHECK(hipFree(b.out));
  CHECK(hipFree(b.cyc));
  CHECK(hipFree(b.clk));
  return 0;
}
