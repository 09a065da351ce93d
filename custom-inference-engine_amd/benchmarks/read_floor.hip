// Floor of a streaming read on one MI355X: how long a short kernel that does
// nothing but read S bytes takes, launch, ramp and drain included. The paged
// attention pair and the INT8 decode-size GEMV read a few tens to a few
// hundred MB per call; this is the time the same bytes cost with no
// arithmetic, no block table and no second pass.
//
// Each thread reads 16-byte chunks with non-temporal loads (grid-stride, four
// loads in flight per thread) and folds them into one word that is stored
// only on an impossible value, so the loads stay. Every size is read from a
// rotation of buffer copies spanning more than 512 MiB, so no copy is still in
// the 256 MiB Infinity Cache when it is read again. Per size and grid: 64
// untimed launches, then 320 timed back to back on one stream (HIP events);
// for the 16 MiB size also a HIP graph of 20 launches replayed 20 times.
//
// Built by build_lib.py (custom-inference-engine_amd/_build/read_floor);
// run through benchmarks/read_floor.py. Arguments: sizes in bytes (default:
// the byte counts of the bench's INT8 GEMV weights and paged workloads).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <vector>

#define CHECK(x)                                                                          \
  do {                                                                                    \
    hipError_t e_ = (x);                                                                  \
    if (e_ != hipSuccess) {                                                               \
      std::fprintf(stderr, "HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); \
      std::exit(1);                                                                       \
    }                                                                                     \
  } while (0)

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kUnroll = 4;

__global__ __launch_bounds__(256) void read_kernel(const u32x4* __restrict__ src, size_t n16, uint32_t* out) {
  const size_t tid = blockIdx.x * 256ull + threadIdx.x, nt = (size_t)gridDim.x * 256ull;
  uint32_t acc = 0;
  for (size_t i = tid; i < n16; i += nt * kUnroll) {
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const size_t j = i + (size_t)u * nt;
      v[u] = j < n16 ? __builtin_nontemporal_load(src + j) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  if (acc == 0x9e3779b9u) out[blockIdx.x] = acc;  // never for the fill below: keeps the loads
}

static float time_launches(const u32x4* buf, size_t copies, size_t n16, int grid, uint32_t* out, int n) {
  hipEvent_t a, b;
  CHECK(hipEventCreate(&a));
  CHECK(hipEventCreate(&b));
  for (int i = 0; i < 64; ++i)
    hipLaunchKernelGGL(read_kernel, dim3(grid), dim3(256), 0, 0, buf + (i % copies) * n16, n16, out);
  CHECK(hipGetLastError());
  CHECK(hipEventRecord(a));
  for (int i = 0; i < n; ++i)
    hipLaunchKernelGGL(read_kernel, dim3(grid), dim3(256), 0, 0, buf + (i % copies) * n16, n16, out);
  CHECK(hipGetLastError());
  CHECK(hipEventRecord(b));
  CHECK(hipEventSynchronize(b));
  float ms = 0.f;
  CHECK(hipEventElapsedTime(&ms, a, b));
  CHECK(hipEventDestroy(a));
  CHECK(hipEventDestroy(b));
  return ms * 1e3f / (float)n;  // us per launch
}

static float time_graph(const u32x4* buf, size_t copies, size_t n16, int grid, uint32_t* out) {
  hipStream_t s;
  CHECK(hipStreamCreate(&s));
  hipGraph_t g;
  hipGraphExec_t ge;
  CHECK(hipStreamBeginCapture(s, hipStreamCaptureModeGlobal));
  for (int i = 0; i < 20; ++i)
    hipLaunchKernelGGL(read_kernel, dim3(grid), dim3(256), 0, s, buf + (i % copies) * n16, n16, out);
  CHECK(hipStreamEndCapture(s, &g));
  CHECK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
  for (int i = 0; i < 5; ++i) CHECK(hipGraphLaunch(ge, s));
  hipEvent_t a, b;
  CHECK(hipEventCreate(&a));
  CHECK(hipEventCreate(&b));
  CHECK(hipEventRecord(a, s));
  for (int i = 0; i < 20; ++i) CHECK(hipGraphLaunch(ge, s));
  CHECK(hipEventRecord(b, s));
  CHECK(hipEventSynchronize(b));
  float ms = 0.f;
  CHECK(hipEventElapsedTime(&ms, a, b));
  CHECK(hipEventDestroy(a));
  CHECK(hipEventDestroy(b));
  CHECK(hipGraphExecDestroy(ge));
  CHECK(hipGraphDestroy(g));
  CHECK(hipStreamDestroy(s));
  return ms * 1e3f / 400.f;
}

int main(int argc, char** argv) {
  std::vector<size_t> sizes;
  for (int i = 1; i < argc; ++i) sizes.push_back((size_t)std::strtoull(argv[i], nullptr, 10));
  if (sizes.empty()) sizes = {16777216, 79574520, 149889040, 299759632};
  const int grids[] = {256, 512, 1024, 2048, 4096};
  uint32_t* out;
  CHECK(hipMalloc(&out, 4096 * sizeof(uint32_t)));
  std::printf("| bytes | grid (x 256 threads) | us per launch | GB/s | fraction of 8 TB/s |\n");
  std::printf("|---:|---:|---:|---:|---:|\n");
  for (const size_t S0 : sizes) {
    const size_t S = S0 / 16 * 16, n16 = S / 16;
    if (n16 == 0) continue;
    const size_t copies = (size_t)(512ull << 20) / S + 1;  // rotation spans more than 512 MiB
    u32x4* buf;
    CHECK(hipMalloc(&buf, S * copies));
    CHECK(hipMemset(buf, 1, S * copies));
    float best = 1e30f;
    int best_grid = 0;
    for (const int grid : grids) {
      const float us = time_launches(buf, copies, n16, grid, out, 320);
      const double gbs = (double)S / (us * 1e-6) / 1e9;
      std::printf("| %zu | %d | %.2f | %.0f | %.3f |\n", S, grid, us, gbs, gbs / 8000.0);
      if (us < best) best = us, best_grid = grid;
    }
    const double gbs = (double)S / (best * 1e-6) / 1e9;
    std::printf("| %zu | best (%d) | **%.2f** | **%.0f** | **%.3f** |\n", S, best_grid, best, gbs, gbs / 8000.0);
    if (S <= (size_t)(32u << 20)) {
      const float gus = time_graph(buf, copies, n16, best_grid, out);
      const double ggbs = (double)S / (gus * 1e-6) / 1e9;
      std::printf("| %zu | graph replay (%d) | %.2f | %.0f | %.3f |\n", S, best_grid, gus, ggbs, ggbs / 8000.0);
    }
    CHECK(hipFree(buf));
  }
  CHECK(hipFree(out));
  return 0;
}
