// Issue rates of the instructions the prefill step is made of, on gfx950:
// v_exp_f32, v_fma_f32, v_mfma_f32_32x32x16_f16, and mixes of them, so that
// "does X overlap Y" is a measurement. One workgroup of 64 * W threads per
// CU (W waves per SIMD over the 4 SIMDs); every lane runs CH independent
// chains of each instruction for ITERS iterations, so latency is hidden and
// the time per iteration is the issue cost of the mix. Each mix first runs
// back to back for ~0.2 s (the clock needs milliseconds of load to leave its
// idle level), then one timed launch: the table gives its duration (HIP
// events), the shader clock it ran at (wave 0 of workgroup 0 reads the
// shader-clock counter and the 100 MHz real-time counter around its loop)
// and the SIMD time per iteration, duration / (ITERS * W) with the W waves
// of a SIMD taking turns, in ns and in shader cycles.
//
// Built by build_lib.py (custom-inference-engine_amd/_build/vector_rates);
// run through benchmarks/vector_rates.py.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

#define CHECK(x)                                                                       \
  do {                                                                                 \
    hipError_t e_ = (x);                                                               \
    if (e_ != hipSuccess) {                                                            \
      std::fprintf(stderr, "HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); \
      std::exit(1);                                                                    \
    }                                                                                  \
  } while (0)

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int CH = 8;       // independent VALU chains per lane
constexpr int NACC = 4;     // independent MFMA accumulators per wave
constexpr int ITERS = 16384;

// NE exps, NF fmas (per chain) and NM MFMAs per iteration.
template <int NE, int NF, int NM>
__global__ __launch_bounds__(1024) void mix_kernel(float* out, long long* clk) {
  float a[CH], b[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    a[i] = -0.001f * (float)(threadIdx.x + i);
    b[i] = 0.5f + 0.001f * (float)i;
  }
  f16x8 x;
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = (_Float16)(0.001f * (float)(threadIdx.x % 7 + i));
  f32x16 acc[NACC];
#pragma unroll
  for (int j = 0; j < NACC; ++j) acc[j] = f32x16{};
  const long long c0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < ITERS; ++it) {
#pragma unroll
    for (int m = 0; m < NM; ++m) acc[m % NACC] = __builtin_amdgcn_mfma_f32_32x32x16_f16(x, x, acc[m % NACC], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < CH; ++i) {
#pragma unroll
      for (int e = 0; e < NE; ++e) a[i] = __builtin_amdgcn_exp2f(a[i]) - 1.0f;  // stays in (-1, 0]
#pragma unroll
      for (int f = 0; f < NF; ++f) b[i] = __builtin_fmaf(b[i], 0.999f, 0.0001f);
    }
  }
  const long long c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    clk[0] = c1 - c0;
    clk[1] = r1 - r0;
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < CH; ++i) s += a[i] + b[i];
#pragma unroll
  for (int j = 0; j < NACC; ++j) s += acc[j][threadIdx.x % 16];
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

template <int NE, int NF, int NM>
static void run(const char* name, int waves_per_simd, int cus, float* out, long long* clk) {
  const int threads = 256 * waves_per_simd;
  hipEvent_t w0, w1;
  CHECK(hipEventCreate(&w0));
  CHECK(hipEventCreate(&w1));
  float settled = 0.f;
  while (settled < 200.f) {  // ~0.2 s of back-to-back launches
    CHECK(hipEventRecord(w0));
    for (int i = 0; i < 8; ++i) hipLaunchKernelGGL((mix_kernel<NE, NF, NM>), dim3(cus), dim3(threads), 0, 0, out, clk);
    CHECK(hipGetLastError());
    CHECK(hipEventRecord(w1));
    CHECK(hipEventSynchronize(w1));
    float ms = 0.f;
    CHECK(hipEventElapsedTime(&ms, w0, w1));
    settled += ms;
  }
  CHECK(hipEventDestroy(w0));
  CHECK(hipEventDestroy(w1));
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  CHECK(hipEventRecord(e0));
  hipLaunchKernelGGL((mix_kernel<NE, NF, NM>), dim3(cus), dim3(threads), 0, 0, out, clk);
  CHECK(hipGetLastError());
  CHECK(hipEventRecord(e1));
  CHECK(hipDeviceSynchronize());
  float ms = 0.f;
  CHECK(hipEventElapsedTime(&ms, e0, e1));
  long long c[2];
  CHECK(hipMemcpy(c, clk, sizeof(c), hipMemcpyDeviceToHost));
  const double ghz = c[1] > 0 ? (double)c[0] / (double)c[1] * 0.1 : 0.0;  // real-time counter: 100 MHz
  const double ns = (double)ms * 1e6 / ((double)ITERS * waves_per_simd);  // SIMD time per iteration
  std::printf("| %s | %d | %d | %d | %d | %.3f | %.2f | %.2f | %.1f |\n", name, waves_per_simd, NE * CH, NF * CH, NM, ms,
              ghz, ns, ns * ghz);
  CHECK(hipEventDestroy(e0));
  CHECK(hipEventDestroy(e1));
}

int main() {
  int dev = 0, cus = 0;
  CHECK(hipGetDevice(&dev));
  CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  float* out;
  long long* clk;
  CHECK(hipMalloc(&out, (size_t)cus * 1024 * sizeof(float)));
  CHECK(hipMalloc(&clk, 2 * sizeof(long long)));
  std::printf("%d CUs, one workgroup per CU, %d iterations\n\n", cus, ITERS);
  std::printf("| mix per iteration (per wave) | waves / SIMD | exp | fma | MFMA 32x32x16 | kernel ms | clock GHz | SIMD ns per iteration | SIMD cycles per iteration |\n");
  std::printf("|---|---:|---:|---:|---:|---:|---:|---:|---:|\n");
  for (int w : {2, 4}) {
    run<1, 0, 0>("8 exp2 (+8 sub)", w, cus, out, clk);
    run<0, 1, 0>("8 fma", w, cus, out, clk);
    run<0, 4, 0>("32 fma", w, cus, out, clk);
    run<1, 4, 0>("8 exp2 (+8 sub) + 32 fma", w, cus, out, clk);
    run<0, 0, 4>("4 MFMA", w, cus, out, clk);
    run<1, 0, 4>("4 MFMA + 8 exp2 (+8 sub)", w, cus, out, clk);
    run<2, 0, 4>("4 MFMA + 16 exp2 (+16 sub)", w, cus, out, clk);
    run<0, 4, 4>("4 MFMA + 32 fma", w, cus, out, clk);
  }
  CHECK(hipFree(out));
  CHECK(hipFree(clk));
  return 0;
}
