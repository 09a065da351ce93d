// Kernel parameter blocks and launcher declarations (host + device visible).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "common.hpp"

namespace cie {

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
  int n_mt;  // query tiles of 128 rows
  int n_wg;  // B * Hq * n_mt
  float scale_log2;  // |scale| * log2(e), never below 1e-30
  uint32_t q_sign;   // 0x80008000 flips the sign of q when the caller's scale is negative
  int causal;
};

// Paged attention over a (num_blocks, block_size, Hk, D) pool.
struct PagedParams {
  const uint16_t* q;
  const uint16_t* kc;
  const uint16_t* vc;
  uint16_t* o;
  const int32_t* bt;
  const int32_t* lens;
  float* ws_acc;  // [B*Hq*Lq*n_splits][D] unnormalised partial outputs
  float* ws_ml;   // [B*Hq*Lq*n_splits][2]  (running max, row sum)
  int64_t qs0, qs1, qs2;
  int64_t ks0, ks1, ks2;  // block, offset, head
  int64_t vs0, vs1, vs2;
  int64_t os0, os1, os2;
  int B, Hq, Hk, Lq, group, R;  // R = group * Lq query rows per kv head
  int num_blocks, max_blocks, block_size;
  int narrow;  // every pool element offset < 2^31, ids and block/offset strides < 2^24
  uint32_t ks0_24, ks1_24, vs0_24, vs1_24;
  FastDiv bsdiv;
  int split_len, n_splits, n_qt;
  float scale_log2;  // |scale| * log2(e), never below 1e-30
  uint32_t q_sign;   // 0x80008000 flips the sign of q when the caller's scale is negative
  int causal;
};

constexpr int kPagedWaves = 4;
constexpr int kPagedTile = 32;             // keys per wave iteration
constexpr int kPagedMaxSplitBlocks = 528;  // block ids of one split staged in LDS
constexpr int kPagedReduceChunk = 256;      // split weights staged per reduction step

// Split length (multiple of kPagedWaves * kPagedTile) for a paged launch.
int paged_split_len(int B, int Hk, int n_qt, int max_ctx, int block_size);

hipError_t launch_flash(const FlashParams& p, int dtype, int D, hipStream_t stream);
hipError_t launch_paged(const PagedParams& p, int dtype, int D, hipStream_t stream);

}  // namespace cie
