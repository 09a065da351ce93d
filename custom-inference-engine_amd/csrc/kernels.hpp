// Kernel parameter blocks and launcher declarations (host + device visible).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "common.hpp"

namespace cie {

// The GPU a launch is sized for: its compute units, and its XCDs (2^xcd_shift
// of them), over which workgroup ids are dispatched round-robin, each XCD
// with its own L2. On gfx950 an XCD has 32 active CUs: 8 XCDs and 256 CUs as
// one partition (an MI355X), fewer when the GPU is partitioned.
struct DeviceShape {
  int cus;
  int xcd_shift;
};
constexpr int kDefaultCUs = 256;  // an unpartitioned MI355X
DeviceShape shape_for_cus(int cus);
// The current device's shape, queried once per device; the MI355X's when no
// device can be queried (size and argument checks on a host without a GPU).
// Thread-safe.
DeviceShape device_shape();

// Rotary tables of the kernels that apply RoPE: cos, sin of shape (rows, D/2),
// contiguous, elements of type dt (kTabF16, kTabBF16 or kTabF32).
// cos == nullptr: no rotation.
constexpr int kTabF16 = 0, kTabBF16 = 1, kTabF32 = 2;
struct RopeTables {
  const void* cos;
  const void* sin;
  int rows;
  int dt;
};

// Dense attention. Strides are in elements; head_dim stride is 1.
struct FlashParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  int64_t qs0, qs1, qs2;  // batch, head, row
  int64_t ks0, ks1, ks2;
  int64_t vs0, vs1, vs2;
  int64_t os0, os1, os2;
  int B, Hq, Hk, Lq, Lk, group;
  int n_mt;  // query tiles of 128 rows (the launcher recounts them for kernels with other tiles)
  int n_wg;  // B * Hq * n_mt
  float scale_log2;  // |scale| * log2(e), never below 1e-30
  uint32_t q_sign;   // 0x80008000 flips the sign of q when the caller's scale is negative
  int causal;
  RopeTables rope;        // rotate q rows as they are loaded: row i of batch b at position q_pos0[b] + i
  const int32_t* q_pos0;  // [B] or nullptr (position = row)
  int cus;                // compute units of the device (kernel choice)
  int xcd_shift;          // log2 of its XCDs (workgroup placement)
};

// Prefill kernel a launch takes (launch_flash); cie_prefill_kernel reports it.
enum FlashKernel { kFlash32 = 0, kFlashR64Heads = 1, kFlashR64Rows = 2, kFlashIl = 3 };
FlashKernel flash_kernel_choice(const FlashParams& p, int D);

// Paged attention over a (num_blocks, block_size, Hk, D) pool.
//
// Work split: the kv heads form NG groups of Hg heads; for every group the
// 32-token tiles of all sequences, concatenated in batch order, are cut into
// min(Wg, tiles) equal contiguous ranges, one per workgroup (id = j * NG +
// group). A sequence covered by more than one range leaves partial states in
// the workspace that a second kernel merges.
struct PagedParams {
  const uint16_t* q;
  const uint16_t* kc;
  const uint16_t* vc;
  uint16_t* o;
  const int32_t* bt;
  const int32_t* lens;
  int4* info;    // [NG][B] pieces of each sequence: first range, count, slot side of piece 0
  float* slots;  // [Wg][NG][2][NWV][Rt][D + 2] partial (acc, m, l) of split sequences
  int64_t qs0, qs1, qs2;
  int64_t ks0, ks1, ks2;  // block, offset, head
  int64_t vs0, vs1, vs2;
  int64_t os0, os1, os2;
  int B, Hq, Hk, Lq, group, R, Rt;  // R = group * Lq query rows per kv head, Rt = min(R, 32)
  int num_blocks, max_blocks, block_size;
  int ctx_limit;  // largest valid context length
  int narrow;     // pool offsets < 2^31 elements, ids and block/offset strides < 2^24
  uint32_t ks0_24, ks1_24, vs0_24, vs1_24;
  FastDiv bsdiv;
  FastDiv rtdiv, nwvdiv, ngdiv;  // item decomposition of the merge pass
  int xcd_runs;   // ranges of a head group in contiguous runs per XCD (paged_xcd_runs)
  int xcd_shift;  // log2 of the device's XCDs
  int mtab_cap;   // > 0: the merge pass takes its sequences from the plan's merge table (capacity per XCD)
  int plan_mtab;  // offset of that table in the plan (int32 elements)
  int Hg, NG, n_qt, NWV, NCH, NST, Wg;
  float scale_log2;  // |scale| * log2(e), never below 1e-30
  uint32_t q_sign;   // 0x80008000 flips the sign of q when the caller's scale is negative
  int causal;
  RopeTables rope;  // rotate q row i of sequence b at position lens[b] - Lq + i as it is loaded
  // Fused append (kn != nullptr): the Lq newest tokens of sequence b are rows
  // b * Lq + i of kn / vn ((B * Lq, Hk, D), strides kns0 / vns0 per token,
  // kns1 / vns1 per head). Attention reads them from there, and the
  // workgroup whose range holds a new token writes it into the pool.
  const uint16_t* kn;
  const uint16_t* vn;
  int64_t kns0, kns1, vns0, vns1;
  // Host-built plan (paged_plan.cpp), or nullptr: the schedule is then
  // derived on the device from lens and bt. Offsets in int32 elements.
  const int32_t* plan;
  int plan_ranges, plan_entries, plan_ids, plan_empty;
  int plan_split;  // split sequences the caller says the plan has (checked against its header)
};

constexpr int kPagedTile = 32;         // tokens per tile
constexpr int kPagedIds = 384;         // block ids of one workgroup's range staged in LDS
constexpr int kPagedEntries = 32;      // sequences one workgroup's range may touch
constexpr int kPagedMaxWaves = 8;      // waves per workgroup (head_dim 256: paged_max_waves)
// Waves per paged workgroup at head_dim D. At D = 256 a wave's accumulators
// and q fragments need more than the 256 registers it has when two waves
// share a SIMD, so those workgroups have at most four waves (one per SIMD)
// and at most 128 query rows per kv head.
__host__ __device__ constexpr int paged_max_waves(int D) { return D == 256 ? 4 : kPagedMaxWaves; }
constexpr int kPagedLdsBudget = 150 * 1024;

// Launch geometry of a paged call; a pure function of the arguments, so the
// workspace query and the launch agree.
struct PagedGeom {
  int ok;            // 0: shape not supported (error text in err)
  const char* err;
  int Hq, D;         // the shape's query heads and head_dim
  DeviceShape dev;   // the GPU the launch is sized for
  int R, Rt, n_qt;
  int Hg, NG, NWV;   // kv heads per workgroup, head groups, waves per workgroup
  int NCH;           // 16-byte chunks per token row of a head group (Hg * D / 8)
  int NST;           // LDS stages
  int Wg;            // workgroups per head group
  size_t lds_bytes;  // dynamic LDS per workgroup
  size_t info_bytes, slot_bytes;  // workspace parts
};
PagedGeom paged_geometry(int B, int Hq, int Hk, int Lq, int D, int ctx_limit, int block_size, DeviceShape dev);

// Host-built plan of a paged launch (see paged_plan.cpp for the layout).
constexpr int32_t kPlanMagic = 0x43504c33;  // "CPL3"
constexpr int kPlanHeader = 16;             // header ints
// Header fields (int32 indices): every argument the plan's layout, ranges
// and validated block ids depend on, compared by the launch before it reads
// anything else of the plan.
enum PlanHeader {
  kPlMagic = 0, kPlW = 1, kPlNT = 2, kPlWg = 3, kPlEmpty = 4, kPlSplit = 5, kPlB = 6, kPlAppend = 7,
  kPlNG = 8, kPlLq = 9, kPlD = 10, kPlNumBlocks = 11, kPlBlockSize = 12, kPlMaxBlocks = 13, kPlCtxLimit = 14,
  kPlHq = 15
};
constexpr int kPlanRangeInts = 8;           // ints per range row
struct PlanLayout {
  size_t ranges, entries, ids, info, empty, mtab;  // section offsets (int32 elements)
  size_t ints;                                     // total size
};
// The main pass places the ranges of a head group on the XCDs in contiguous
// runs (workgroup ids are dispatched round-robin over the XCDs, and each XCD
// keeps what its workgroups wrote in its L2 across the kernel boundary), and
// the plan's merge table hands each split sequence's merge work to the XCD
// holding its pieces: mtab[x][i] (x < kMaxXcds, i < merge_table_cap(...)) is
// the i-th sequence merged on XCD x as 4 ints: b * NG + gh, then the
// sequence's piece descriptor (first range, pieces, slot side of piece 0),
// so a merge workgroup reads its whole schedule in one load; {-1, 0, 0, 0}
// when unused (lists of XCDs the device does not have stay empty).
constexpr int kMaxXcds = 8;
// Sequences per XCD list over 2^xcd_shift XCDs: every split sequence fits,
// with one to spare.
__host__ __device__ inline int merge_cap(int split_units, int xcd_shift) {
  return ((split_units + (1 << xcd_shift) - 1) >> xcd_shift) + 1;
}
__host__ __device__ inline int merge_table_cap(int B, int NG, int xcd_shift) { return merge_cap(B * NG, xcd_shift); }
// The placement (and the merge table) is used when the main pass has one
// workgroup per CU or fewer (verify-like shapes: partial states of ~20 query
// rows per kv head, merge reads from L2 3.8 % faster on verify_b8); with two
// workgroups per CU (decode-like) contiguous runs cost the main pass more
// than the merge saves (decode_b32 +1.2 us), and ranges alternate head
// groups over the workgroup ids instead.
inline bool paged_xcd_runs(const PagedGeom& g) { return (int64_t)g.NG * g.Wg <= g.dev.cus; }
// XCD of main-pass workgroup `logical` (the order of xcd_logical) when the
// grid has n workgroups over 2^xcd_shift XCDs.
inline int xcd_of_logical(int64_t logical, int64_t n, int xcd_shift) {
  const int nx = 1 << xcd_shift;
  const int64_t base = n >> xcd_shift, extra = n & (nx - 1);
  for (int x = 0; x < nx - 1; ++x)
    if (logical < (x + 1) * base + std::min<int64_t>(x + 1, extra)) return x;
  return nx - 1;
}

// Workgroup `block` of an n-workgroup grid, renumbered so that each XCD
// (block % 2^xcd_shift, the round-robin dispatch) holds a contiguous run of
// logical ids: XCD x takes ids [start_x, start_x + count_x), the counts in
// XCD order. A bijection of [0, n) for every n.
__device__ __forceinline__ int xcd_logical(int block, int n, int xcd_shift) {
  const int mask = (1 << xcd_shift) - 1;
  const int xcd = block & mask, slot = block >> xcd_shift;
  return xcd * (n >> xcd_shift) + min(xcd, n & mask) + slot;
}
PlanLayout paged_plan_layout(const PagedGeom& g, int B, int max_blocks);
// Fills P (layout L) from host lengths and block tables; returns the number
// of sequences split across workgroups (>= 0), or -1 when the geometry's
// bounds are violated.
int build_paged_plan(int32_t* P, const PagedGeom& g, const PlanLayout& L, const int32_t* lens,
                     const int32_t* bt, int64_t bt_stride, int B, int Lq, int num_blocks, int block_size,
                     int max_blocks, int ctx_limit, int append);

// Paged KV append: new token rows (T, Hk, D) into the pool through block tables.
struct AppendParams {
  const uint16_t* k_new;
  const uint16_t* v_new;
  uint16_t* kc;
  uint16_t* vc;
  const int32_t* bt;      // [B][max_blocks]
  const int32_t* cu_new;  // [B + 1] prefix offsets of each sequence's rows in k_new / v_new
  const int32_t* start;   // [B] position of each sequence's first new token
  uint32_t* status;       // optional: set to 1 when a position or block id is out of range
  int64_t ns0, ns1;       // k_new strides (token, head); head_dim stride 1
  int64_t ms0, ms1;       // v_new strides
  int64_t ks0, ks1, ks2;  // k pool strides (block, offset, head)
  int64_t vs0, vs1, vs2;
  int num_blocks, max_blocks, block_size;
  uint32_t cpr;           // 16-byte chunks per token row (Hk * D / 8)
  uint32_t lg_cph;        // log2 of chunks per head row (D / 8)
  FastDiv cprdiv, bsdiv;
  // RoPE on K (rope.cos != nullptr): token i of sequence b is rotated at
  // position start[b] + i before it is written; a position outside the
  // table writes neither K nor V of that token and ORs 2 into status.
  RopeTables rope;
  FastDiv updiv;          // chunk pairs per token row (cpr / 2)
  uint16_t* k_out;        // optional dense copy of the rotated K rows, (T, Hk, D)
  int64_t os0, os1;       // k_out strides (token, head)
};

// Standalone RoPE of x (B, H, L, D) into out (may be x itself).
struct RopeParams {
  const uint16_t* x;
  uint16_t* out;
  int64_t xs0, xs1, xs2;
  int64_t os0, os1, os2;
  const int32_t* pos;  // nullptr: position = row index l; else pos[b * pos_bs + l]
  int64_t pos_bs;
  RopeTables tab;
  uint32_t* status;    // optional: 2 ORed in when a position is outside the table
  int B, H, L;
  int HG;              // heads one thread rotates: kRopeHeads, or 1 for launches too small to fill the GPU
  int NHG;             // head groups: ceil(H / HG)
  uint32_t total;      // B * NHG * L * D / 16 (one thread per chunk pair of a head group)
  FastDiv ldiv, hgdiv;
};
constexpr int kRopeHeads = 8;  // heads one thread rotates (they share the position's table row)
constexpr int64_t kRopeGroupMin = (int64_t)512 * 256 * kRopeHeads;  // chunk pairs from which 8-head threads still give 512 workgroups

// INT8-weight GEMM: y (M, N) = (x (M, K) . w (N, K)^T) * scales[n] (+ bias[n]).
struct I8GemmParams {
  const uint16_t* x;      // fp16 / bf16, row stride xs elements, unit column stride
  const int8_t* w;        // row stride wsr bytes
  const void* scales;     // (N,) fp16 / bf16 / fp32 (scale_dtype 0 / 1 / 2)
  const uint16_t* bias;   // (N,) in x's dtype, or nullptr
  uint16_t* y;            // row stride ys elements
  float* partial;         // fp32 partial tiles when splits > 1 (lane order, see int8_gemm.hip)
  int64_t xs, wsr, ys;
  int M, N, K, scale_dtype;
  int n_tiles, m_tiles, splits, ksteps, m_pad, n_pad;
  int xcd_shift;          // log2 of the device's XCDs
};

// Launch geometry of an INT8 GEMM; a pure function of (M, N, K), so the
// workspace query and the launch agree.
struct I8Geom {
  int gemv;                // 1: weight-streaming MFMA kernel (M <= 64), 2: VALU dot kernel (M = 1),
                           // 3: row-streaming dot kernel (M <= 2, activations staged in LDS); one launch
  int kw2;                 // tiled kernel: two K-waves per workgroup (eight waves)
  DeviceShape dev;         // the GPU the launch is sized for
  int mt;                  // 32-row activation tiles per workgroup
  int nst;                 // LDS ring stages
  int m_tiles, n_tiles, ksteps, splits, m_pad, n_pad;
  size_t workspace_bytes;  // split-K partials (0 when splits == 1)
  size_t lds_bytes;
};
I8Geom int8_gemm_geometry(int M, int N, int K, DeviceShape dev);

// Raises a kernel's dynamic-LDS limit to `bytes` on the current device, once
// per (kernel, device): the attribute is a property of the kernel as loaded
// on a device, so a process that launches on several GPUs sets it on each.
// Thread-safe.
hipError_t set_dynamic_lds(const void* kernel, int bytes);

hipError_t launch_flash(const FlashParams& p, int dtype, int D, hipStream_t stream);
hipError_t launch_int8_gemm(const I8GemmParams& p, const I8Geom& g, int dtype, hipStream_t stream);
hipError_t launch_kv_append(const AppendParams& p, int B, int max_new, int dtype, int D, hipStream_t stream);
hipError_t launch_rope(const RopeParams& p, int dtype, int D, hipStream_t stream);
// merge: launch the merge pass of split sequences (false only when a plan
// says no sequence is split)
hipError_t launch_paged(const PagedParams& p, int dtype, int D, size_t lds_bytes, bool merge, hipStream_t stream);

// Bytes of the static device workspace behind cie_paged_fwd_noalloc.
constexpr size_t kPagedScratchBytes = (size_t)16 << 20;
// Device address of that workspace on the current device, looked up once
// per device (the host-side symbol is not a device address). Thread-safe.
hipError_t paged_scratch_ptr(void** ptr);

}  // namespace cie
