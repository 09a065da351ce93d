// Paged decode / speculative-verify attention for gfx950.
//
// Replaces the reference's per-layer gather-then-dense sequence
// (engine/model/block.py:56-71: cache.gather -> index_select of the whole
// history, engine/cache/kv_cache.py:141-165, then the dense Triton kernel):
// K and V are read once, straight out of the (num_blocks, block_size, Hk, D)
// pool through the int32 block table.
//
// Memory path. A workgroup owns a group of Hg kv heads (Hg * D <= 256, so a
// token's rows of the group are at most 512 contiguous bytes of the pool)
// and one wave per (kv head, query tile). Each 32-token tile of K and of V is
// copied global -> LDS by 16-byte direct-to-LDS loads, every load instruction
// covering whole contiguous token rows of the group: pool blocks stream at
// close to copy bandwidth, where per-head 128-byte rows scattered 1 KiB apart
// do not. The tile is stored token-major with the 16-byte chunks of each
// token row XOR-swizzled (row_swizzle), so the per-head fragment reads below
// are bank-conflict-free. NST stages rotate; the copies of the next NST-1
// tiles are in flight while one tile is computed. The pool copies are
// non-temporal (read once; decode_b32 ran 9 % faster than with cached
// copies, which displaced the block tables and lengths). (Groups of 512-byte rows
// give 32 KiB stages, four of them, against two 64 KiB stages for 1 KiB
// rows: verify_b8 ran 9 % faster, decode_b32 the same.)
//
// Per tile and wave (one kv head, up to 32 query rows r = g * Lq + i: query
// head kvh * group + g, new token i):
//   S^T[32 keys x 32 rows] = K_tile . Q^T    A operand: ds_read_b128 of a token row
//   online softmax in registers (one v_permlane32_swap per reduction)
//   O^T += V^T_tile . P^T                    A operand: ds_read_b64_tr_b16 turns the
//                                             token-major V tile into key-contiguous V^T
//
// Work split (stream-K over sequences). For a head group, the 32-token tiles
// of all sequences are concatenated in batch order and cut into equal
// contiguous ranges, one per workgroup, so every workgroup streams the same
// number of bytes whatever the context lengths. A sequence inside one range
// is written directly. A sequence cut across ranges leaves one partial state
// (acc, m, l) per piece in the workspace plus a piece descriptor, and
// paged_merge_kernel combines the pieces in piece order (the kernel boundary
// makes the partials visible; no counters or device-wide fences).
//
// Invalid input is never dereferenced: a context length outside
// [0, ctx_limit] or a block id outside [0, num_blocks) makes that sequence's
// output NaN.
#include <climits>
#include <map>
#include <mutex>
#include <type_traits>

#include "kernels.hpp"
#include "rope.hpp"

namespace cie {

#ifdef CIE_TIMELINE
__device__ unsigned long long paged_timeline[kTimelineMaxWg * kTimelineSlots];  // benchmarks/timeline.py
#endif

constexpr float kLazyRescalePaged = 8.0f;

// Lambdas of the kernel are inlined: the arrays they touch stay in registers.
#define CIE_PAGED_INLINE __attribute__((always_inline))

template <int D>
struct PagedCfg {
  static constexpr int KK = D / 16;                 // MFMA steps over head_dim
  static constexpr int DT = D >= 32 ? D / 32 : 1;   // 32-row output tiles
  static constexpr int S = D / 8;                   // 16-byte chunks per head row
  static constexpr int DPW = D / 16;                // 1 KiB copies per issuing wave, tensor and tile
  static constexpr int QPRE = D <= 64 ? 3 : (D == 128 ? 1 : 0);  // sequences with q loaded up front
  static constexpr int QARR = QPRE > 0 ? QPRE : 1;
  static constexpr int MU = D <= 64 ? 4 : (D == 128 ? 2 : 1);    // pieces loaded together by a merge
};

// Swizzle of the 16-byte chunks of token row t in a tile with nch chunks per
// row: the family of chunk_swizzle applied to rows of nch chunks.
__device__ __forceinline__ int row_swizzle(int nch, int t) {
  return nch >= 16 ? bitrev4(t & 15) : nch == 8 ? bitrev3((t >> 1) & 7) : nch == 4 ? ((t >> 2) & 3) : ((t >> 3) & 1);
}

// Inclusive prefix sum over the 64 lanes: DPP row shifts within each row of
// 16 lanes, then the row totals broadcast forward (row_bcast:15 into rows 1
// and 3, row_bcast:31 into rows 2 and 3). Lanes whose DPP source lies
// outside the row, and rows outside the row mask, add the old value 0.
__device__ __forceinline__ int wave_incl_scan(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return x;
}

// floor(n / d) for n < 2^63, 0 < d < 2^31: a 32-bit division whenever n fits
// in 32 bits (always, unless tiles x workgroups reaches 2^32).
__device__ __forceinline__ int div_small(uint64_t n, uint32_t d) {
  return n <= 0xffffffffull ? (int)((uint32_t)n / d) : (int)(n / d);
}

// The plan header names the launch it was built for: every argument its
// layout, ranges and validated block ids depend on, and the split count the
// caller passes with it. Anything else of the plan is read only after this
// check. The 16 header ints are loaded together and compared without
// short-circuit branches: one memory round trip, where a chain of compare-
// and-branch steps waits for each field's load in turn.
template <int D>
__device__ __forceinline__ bool plan_matches(const PagedParams& p) {
  const int4* P4 = reinterpret_cast<const int4*>(p.plan);  // the plan is 16-byte aligned
  int32_t h[kPlanHeader];
#pragma unroll
  for (int i = 0; i < kPlanHeader / 4; ++i) {
    const int4 v = P4[i];
    h[4 * i] = v.x, h[4 * i + 1] = v.y, h[4 * i + 2] = v.z, h[4 * i + 3] = v.w;
  }
  bool ok = h[kPlMagic] == kPlanMagic;
  ok &= h[kPlWg] == p.Wg;
  ok &= h[kPlB] == p.B;
  ok &= h[kPlAppend] == (p.kn ? 1 : 0);
  ok &= h[kPlSplit] == p.plan_split;
  ok &= h[kPlNG] == p.NG;
  ok &= h[kPlLq] == p.Lq;
  ok &= h[kPlD] == D;
  ok &= h[kPlNumBlocks] == p.num_blocks;
  ok &= h[kPlBlockSize] == p.block_size;
  ok &= h[kPlMaxBlocks] == p.max_blocks;
  ok &= h[kPlCtxLimit] == p.ctx_limit;
  ok &= h[kPlHq] == p.Hq;
  return ok;
}

__device__ __forceinline__ bool ctx_valid(const PagedParams& p, int ctx) {
  // with a fused append the Lq new tokens are part of every valid context
  return ctx >= (p.kn ? p.Lq : 0) && ctx <= p.ctx_limit && (ctx == 0 || p.num_blocks > 0);
}

// Range index of tile x when nt tiles are cut into wg <= nt ranges
// [floor(j nt / wg), floor((j+1) nt / wg)).
__device__ __forceinline__ int range_of(int x, int nt, int wg) {
  return div_small((uint64_t)(x + 1) * (uint32_t)wg - 1, (uint32_t)nt);
}

template <int DPW>
__device__ __forceinline__ void wait_tiles_ahead(int ahead) {
  // vmcnt counts the 2 * DPW copies of every tile issued after the one needed
  if constexpr (6 * DPW < 64) {
    if (ahead >= 3) { vm_wait<6 * DPW>(); return; }
  }
  if constexpr (4 * DPW < 64) {
    if (ahead == 2) { vm_wait<4 * DPW>(); return; }
  }
  if (ahead == 1) { vm_wait<2 * DPW>(); return; }
  vm_wait<0>();
}

// Writes this lane's half (columns [hl * D/2, (hl+1) * D/2)) of one output
// row with a constant 16-bit pattern.
template <int D>
__device__ __forceinline__ void fill_row_half(uint16_t* row, int hl, uint32_t bits2) {
#pragma unroll
  for (int d = hl * (D / 2); d < (hl + 1) * (D / 2); d += 8)
    *reinterpret_cast<u32x4*>(row + d) = u32x4{bits2, bits2, bits2, bits2};
}

// Stores acc * inv (MFMA C layout of O^T: this lane holds row l32, columns
// 32 dt + 8 g4 + 4 hl + 0..3) as one output row.
template <int DTYPE, int D>
__device__ __forceinline__ void store_row(uint16_t* row, const f32x16* acc, float inv, int hl) {
  using E = Elt<DTYPE>;
  constexpr int DT = PagedCfg<D>::DT;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int d = 32 * dt + 8 * g4 + 4 * hl;
      if (D >= 32 || d < D) {
        const u32x2 w = {E::pack2(acc[dt][4 * g4] * inv, acc[dt][4 * g4 + 1] * inv),
                         E::pack2(acc[dt][4 * g4 + 2] * inv, acc[dt][4 * g4 + 3] * inv)};
        *reinterpret_cast<u32x2*>(row + d) = w;
      }
    }
  }
}

// APPEND: the fused-append variant (p.kn set), a separate instantiation so
// the plain kernel carries none of its registers or branches.
template <int DTYPE, int D, bool APPEND>
__global__ __launch_bounds__(64 * paged_max_waves(D)) void paged_fwd_kernel(const PagedParams p) {
  CIE_STAMP(paged_timeline, 0);  // entry
  CIE_STAMP_WHERE(paged_timeline, 5);
  warm_kernargs<sizeof(PagedParams)>();
  using C = PagedCfg<D>;
  using E = Elt<DTYPE>;
  extern __shared__ __attribute__((aligned(16))) uint16_t ring[];
  __shared__ int32_t sbt[kPagedIds];
  __shared__ int32_t ent[kPagedEntries][8];  // b, ctx, tt_lo, n, idbase, blk_lo, pre, pieces

  // Range j of head group gh. With xcd_runs the ranges of a head group go to
  // the XCDs in contiguous runs (workgroups are dispatched round-robin over
  // the XCDs), so the pieces of a split sequence are mostly written through
  // one XCD's L2, where the merge pass then finds them (merge_table_cap);
  // otherwise consecutive workgroup ids alternate head groups.
  int gh, j;
  if (p.xcd_runs) {
    const int logical = xcd_logical(blockIdx.x, p.NG * p.Wg, p.xcd_shift);
    gh = logical / p.Wg;
    j = logical - gh * p.Wg;
  } else {
    gh = blockIdx.x % p.NG;
    j = blockIdx.x / p.NG;
  }
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave index, uniform
  const int lane = threadIdx.x & 63, l32 = lane & 31, hl = lane >> 5;
  const int hh = w % p.Hg, qt = w / p.Hg;
  const int kvh = gh * p.Hg + hh;
  const bool issuer = qt == 0;  // the qt = 0 waves copy the tiles all waves read

  // Query row of this lane.
  const int r = qt * 32 + l32;
  const bool rv = r < p.R;
  const int g = rv ? r / p.Lq : 0;
  const int i = rv ? r - g * p.Lq : 0;
  const int hq = kvh * p.group + g;
  const uint32_t nan2 = 0x7fff7fffu;  // NaN in both fp16 and bf16

  const uint32_t sbt_lds = lds_addr_of(sbt);
  int ne = 0, nid = 0, S0 = 0, T = 0;
  if (p.plan) {
    // ---- schedule from the host-built plan: this range's row, then its
    // entries and block ids (already validated) copied straight into LDS ----
    // The range row is loaded beside the header, in the same round trip (the
    // launch checked that the buffer holds every offset of its layout, so a
    // row of a plan for other arguments is still inside it); it is used only
    // when the header matches.
    const int32_t* P = p.plan;
    const int32_t* row = P + p.plan_ranges + kPlanRangeInts * j;  // 16-byte aligned
    const int4 r03 = *reinterpret_cast<const int4*>(row);        // first entry, entries, first id, ids
    const int2 r45 = *reinterpret_cast<const int2*>(row + 4);    // S0, T
    const bool ok = plan_matches<D>(p);
    // selects, not a branch: a branch would let the compiler sink the row's
    // loads behind the header check
    ne = ok ? min(r03.y, kPagedEntries) : 0;
    nid = ok ? min(r03.w, kPagedIds) : 0;
    S0 = ok ? r45.x : 0;
    T = ok ? r45.y : 0;
    if (j == 0) {
      // sequences without tiles (zeros for an empty history, NaN for an
      // invalid length); every sequence NaN when the plan is not this launch's
      const int nz = ok ? min(P[4], p.B) : p.B;
      const int32_t* Z = P + p.plan_empty;
      for (int z = 0; z < nz; ++z) {
        const int bz = ok ? Z[2 * z] : z;
        const bool zvalid = ok && Z[2 * z + 1] != 0;
        if (rv && (uint32_t)bz < (uint32_t)p.B)
          fill_row_half<D>(p.o + (int64_t)bz * p.os0 + hq * p.os1 + (int64_t)i * p.os2, hl, zvalid ? 0u : nan2);
      }
    }
    if (w == 0 && T > 0) {
      const int32_t* es = P + p.plan_entries + 8 * r03.x;
      const uint32_t ent_lds = lds_addr_of(ent);
      for (int x0 = 0; x0 < 8 * ne; x0 += 64)
        if (x0 + lane < 8 * ne) dma4(es + x0 + lane, ent_lds + 4u * (uint32_t)x0);
      const int32_t* is = P + p.plan_ids + r03.z;
      for (int x0 = 0; x0 < nid; x0 += 64)
        if (x0 + lane < nid) dma4(is + x0 + lane, sbt_lds + 4u * (uint32_t)x0);
      vm_wait<0>();
    }
  } else {
  // ---- schedule: every wave derives it from the context lengths ----------
  // ctx0, incl0: this lane's length and inclusive tile prefix among the
  // first 64 sequences, reused below
  int NT = 0, ctx0 = 0, incl0 = 0;
  for (int b0 = 0; b0 < p.B; b0 += 64) {
    const int b = b0 + lane;
    const int ctx = b < p.B ? p.lens[b] : 0;
    const int incl = wave_incl_scan(ctx_valid(p, ctx) ? (ctx + kPagedTile - 1) / kPagedTile : 0);
    if (b0 == 0) ctx0 = ctx, incl0 = incl;
    NT += __builtin_amdgcn_readlane(incl, 63);
  }
  // W <= NT ranges, so none is empty: every range a sequence spans holds one
  // of its pieces (workgroups j >= W have nothing to do).
  const int W = min(p.Wg, NT);
  S0 = j < W ? div_small((uint64_t)j * (uint32_t)NT, (uint32_t)W) : NT;
  const int S1 = j < W ? div_small((uint64_t)(j + 1) * (uint32_t)NT, (uint32_t)W) : NT;

  int carry = 0;
  for (int b0 = 0; b0 < p.B; b0 += 64) {
    if (j != 0 && carry >= S1) break;
    const int b = b0 + lane;
    const int ctx = b0 == 0 ? ctx0 : (b < p.B ? p.lens[b] : 0);
    const bool valid = ctx_valid(p, ctx);
    const int t = valid ? (ctx + kPagedTile - 1) / kPagedTile : 0;
    const int incl = b0 == 0 ? incl0 : wave_incl_scan(t);
    const int pre = carry + incl - t;
    carry += __builtin_amdgcn_readlane(incl, 63);
    if (j == 0) {
      // Sequences without tiles: zeros for an empty history, NaN for an
      // invalid length. The first workgroup of each head group writes them.
      uint64_t zm = __builtin_amdgcn_ballot_w64(b < p.B && t == 0);
      while (zm) {
        const int zl = __builtin_ctzll(zm);
        zm &= zm - 1;
        const int zvalid = __shfl((int)valid, zl);
        if (rv) fill_row_half<D>(p.o + (int64_t)(b0 + zl) * p.os0 + hq * p.os1 + (int64_t)i * p.os2, hl,
                                 zvalid ? 0u : nan2);
      }
    }
    if (j == 0 && w == 0 && b < p.B && t == 0)
      p.info[(int64_t)gh * p.B + b] = int4{0, 0, 0, 0};  // nothing to merge
    const bool ov = t > 0 && pre < S1 && pre + t > S0;
    int tt_lo = 0, n = 0, blk_lo = 0, nids = 0;
    if (ov) {
      tt_lo = max(S0 - pre, 0);
      const int tt_hi = min(S1 - pre, t);
      n = tt_hi - tt_lo;
      blk_lo = (int)fdiv((uint32_t)(kPagedTile * tt_lo), p.bsdiv);
      const int blk_hi = (int)fdiv((uint32_t)(min(ctx, kPagedTile * tt_hi) - 1), p.bsdiv);
      nids = blk_hi - blk_lo + 1;
    }
    const int ids_incl = wave_incl_scan(nids);
    const uint64_t om = __builtin_amdgcn_ballot_w64(ov);
    if (w == 0 && ov) {
      const int e = ne + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(om >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)om, 0));
      const int j0 = range_of(pre, NT, W), j1 = range_of(pre + t - 1, NT, W);
      ent[e][0] = b;
      ent[e][1] = ctx;
      ent[e][2] = tt_lo;
      ent[e][3] = n;
      ent[e][4] = nid + ids_incl - nids;
      ent[e][5] = blk_lo;
      ent[e][6] = pre;
      ent[e][7] = j1 - j0 + 1;
      // The range holding a sequence's first tile describes its pieces for
      // the merge pass: first range, piece count, slot side of piece 0.
      if (pre >= S0) p.info[(int64_t)gh * p.B + b] = int4{j, j1 - j0 + 1, pre > S0 ? 1 : 0, 0};
    }
    ne += __builtin_popcountll(om);
    nid += __builtin_amdgcn_readlane(ids_incl, 63);
  }
  T = S1 - S0;

  // Stage the block ids of the range in LDS (one direct-to-LDS dword per id);
  // ids outside [0, num_blocks) become -1 (never dereferenced, poison the piece).
  if (w == 0 && T > 0) {
    for (int e = 0; e < ne; ++e) {
      // entry fields are wave-uniform; readfirstlane keeps the address math scalar
      const int b = __builtin_amdgcn_readfirstlane(ent[e][0]), ctx = __builtin_amdgcn_readfirstlane(ent[e][1]);
      const int tt_lo = __builtin_amdgcn_readfirstlane(ent[e][2]), n = __builtin_amdgcn_readfirstlane(ent[e][3]);
      const int idb = __builtin_amdgcn_readfirstlane(ent[e][4]), blk_lo = __builtin_amdgcn_readfirstlane(ent[e][5]);
      const int blk_hi = (int)fdiv((uint32_t)(min(ctx, kPagedTile * (tt_lo + n)) - 1), p.bsdiv);
      const int cnt = blk_hi - blk_lo + 1;
      const int32_t* src = p.bt + (int64_t)b * p.max_blocks + blk_lo;
      for (int x0 = 0; x0 < cnt; x0 += 64) {
        const uint32_t dst = sbt_lds + 4u * (uint32_t)(idb + x0);
        if (x0 + lane < cnt) dma4(src + x0 + lane, dst);
      }
    }
    vm_wait<0>();
    for (int x = lane; x < nid; x += 64)
      if ((uint32_t)sbt[x] >= (uint32_t)p.num_blocks) sbt[x] = -1;
  }
  }  // device-derived schedule
  __syncthreads();
  CIE_STAMP(paged_timeline, 1);  // schedule in LDS
  CIE_STAMP_VALUE(paged_timeline, 6, T);
  CIE_STAMP_VALUE(paged_timeline, 7, ne);
  if (T == 0) return;

  // ---- per-lane constants -------------------------------------------------
  const int NCH = p.NCH, NST = p.NST;
  const int lg_nch = __builtin_ctz(NCH);
  const int TILE_EL = kPagedTile * NCH * 8;  // elements of one tensor tile
  const int STAGE_EL = 2 * TILE_EL;

  // Copies: load i of this wave moves LDS chunk P = 64 (hh DPW + i) + lane of
  // the tile, i.e. token P / NCH, stored chunk P % NCH, which holds chunk
  // (P % NCH) ^ row_swizzle(token) of the token's group row.
  int ltok[C::DPW];
  int32_t goffk[C::DPW], goffv[C::DPW];  // head + column offsets (the host bounds them below 2^31)
  // Fused append: the chunk's (head, column) within a new-token row, kept as
  // the chunk index only; the offsets are formed on the few tiles that hold
  // new tokens (keeping them as 64-bit offsets pushed the kernel past the
  // register file, and the spill reloads waited for every copy in flight).
  constexpr int NA = APPEND ? C::DPW : 1;
  int nch_of[NA];
#pragma unroll
  for (int x = 0; x < C::DPW; ++x) {
    const int P = 64 * (hh * C::DPW + x) + lane;
    const int tk = P >> lg_nch;
    const int c = (P & (NCH - 1)) ^ row_swizzle(NCH, tk);
    const int hd = c / C::S, dc = c % C::S;
    ltok[x] = tk;
    goffk[x] = (gh * p.Hg + hd) * (int32_t)p.ks2 + 8 * dc;
    if constexpr (APPEND) nch_of[x] = c;
    goffv[x] = (gh * p.Hg + hd) * (int32_t)p.vs2 + 8 * dc;
  }
  // Fragment reads: K row l32 (chunk 2 kk + hl of head hh), V^T rows.
  const int swk = row_swizzle(NCH, l32);
  const int rq = lane & 15, gq = lane >> 4;
  int swv[2][2];
#pragma unroll
  for (int cc = 0; cc < 2; ++cc) {
    swv[cc][0] = row_swizzle(NCH, 16 * cc + 4 * hl + (rq >> 2));
    swv[cc][1] = row_swizzle(NCH, 16 * cc + 4 * hl + (rq >> 2) + 8);
  }

  const uint32_t ring_lds = lds_addr_of(ring);  // byte address of stage 0

  // Issue cursor.
  int ie = 0, i_base = 0, i_end = __builtin_amdgcn_readfirstlane(ent[0][3]);
  int i_b = __builtin_amdgcn_readfirstlane(ent[0][0]);
  int i_ctx = __builtin_amdgcn_readfirstlane(ent[0][1]), i_ttlo = __builtin_amdgcn_readfirstlane(ent[0][2]);
  int i_idb = __builtin_amdgcn_readfirstlane(ent[0][4]), i_blk = __builtin_amdgcn_readfirstlane(ent[0][5]);
  int i_stage = 0;
  auto issue = [&](int k) {
    if (k == i_end) {
      ++ie;
      i_base = i_end;
      i_end += __builtin_amdgcn_readfirstlane(ent[ie][3]);
      i_ctx = __builtin_amdgcn_readfirstlane(ent[ie][1]);
      i_ttlo = __builtin_amdgcn_readfirstlane(ent[ie][2]);
      i_idb = __builtin_amdgcn_readfirstlane(ent[ie][4]);
      i_blk = __builtin_amdgcn_readfirstlane(ent[ie][5]);
      i_b = __builtin_amdgcn_readfirstlane(ent[ie][0]);
    }
    const int tbase = kPagedTile * (i_ttlo + k - i_base);
    const uint32_t st = ring_lds + 2u * (uint32_t)(i_stage * STAGE_EL) + 1024u * (uint32_t)(hh * C::DPW);
    i_stage = i_stage + 1 == NST ? 0 : i_stage + 1;
    if (APPEND && tbase + kPagedTile > i_ctx - p.Lq) {
      // a tile holding new tokens: those rows come from kn / vn, the rest
      // from the pool (per-lane addresses)
#pragma unroll
      for (int x = 0; x < C::DPW; ++x) {
        const int tk = min(tbase + ltok[x], i_ctx - 1);
        const uint16_t *sk, *sv;
        if (tk >= i_ctx - p.Lq) {
          const int64_t row = (int64_t)i_b * p.Lq + (tk - (i_ctx - p.Lq));
          int c = nch_of[APPEND ? x : 0];
          asm volatile("" : "+v"(c));  // keeps the offset arithmetic on this path (not hoisted and kept live)
          const int hd = gh * p.Hg + c / C::S, col = 8 * (c % C::S);
          sk = p.kn + row * p.kns0 + (int64_t)hd * p.kns1 + col;
          sv = p.vn + row * p.vns0 + (int64_t)hd * p.vns1 + col;
        } else {
          const int blk = (int)fdiv((uint32_t)tk, p.bsdiv);
          const int off = tk - blk * p.block_size;
          const int bid = max(sbt[i_idb + blk - i_blk], 0);
          sk = p.kc + (int64_t)bid * p.ks0 + (int64_t)off * p.ks1 + goffk[x];
          sv = p.vc + (int64_t)bid * p.vs0 + (int64_t)off * p.vs1 + goffv[x];
        }
        dma16_at_nt(sk, st + 1024u * x);
        dma16_at_nt(sv, st + 2u * TILE_EL + 1024u * x);
      }
      return;
    }
    int bid[C::DPW], off[C::DPW];
#pragma unroll
    for (int x = 0; x < C::DPW; ++x) {  // all block-id reads in flight together
      const int tk = min(tbase + ltok[x], i_ctx - 1);
      const int blk = (int)fdiv((uint32_t)tk, p.bsdiv);
      off[x] = tk - blk * p.block_size;
      bid[x] = max(sbt[i_idb + blk - i_blk], 0);
    }
    if (p.narrow) {
#pragma unroll
      for (int x = 0; x < C::DPW; ++x) {
        // whole 32-bit element offsets (the narrow path bounds them below 2^31),
        // added to the pool base once: no per-lane 64-bit pointers stay live
        const uint32_t ek = __umul24(bid[x], p.ks0_24) + __umul24(off[x], p.ks1_24) + (uint32_t)goffk[x];
        const uint32_t ev = __umul24(bid[x], p.vs0_24) + __umul24(off[x], p.vs1_24) + (uint32_t)goffv[x];
        dma16_at_nt(p.kc + ek, st + 1024u * x);
        dma16_at_nt(p.vc + ev, st + 2u * TILE_EL + 1024u * x);
      }
    } else {
#pragma unroll
      for (int x = 0; x < C::DPW; ++x) {
        dma16_at_nt(p.kc + (int64_t)bid[x] * p.ks0 + (int64_t)off[x] * p.ks1 + goffk[x], st + 1024u * x);
        dma16_at_nt(p.vc + (int64_t)bid[x] * p.vs0 + (int64_t)off[x] * p.vs1 + goffv[x], st + 2u * TILE_EL + 1024u * x);
      }
    }
  };

  // q rows of the first QPRE sequences, then the first tiles; the wait below
  // covers the q loads only (the tile copies issued after them stay in flight)
  const uint16_t* qrow = p.q + hq * p.qs1 + (int64_t)i * p.qs2;
  u32x4 qpre[C::QARR][C::KK];
#pragma unroll
  for (int e = 0; e < C::QPRE; ++e) {
    const int b = e < ne ? ent[e][0] : 0;
#pragma unroll
    for (int kk = 0; kk < C::KK; ++kk) qpre[e][kk] = load16(qrow + b * p.qs0 + 16 * kk + 8 * hl, rv && e < ne);
  }
  const int pro = min(NST - 1, T);
  if (issuer) {
    for (int k = 0; k < pro; ++k) issue(k);
    wait_tiles_ahead<C::DPW>(pro);
  } else {
    vm_wait<0>();
  }
  if (p.rope.cos) {  // RoPE fused into the load: row i at position ctx - Lq + i
#pragma unroll
    for (int e = 0; e < C::QPRE; ++e)
      if (e < ne)  // wave-uniform: preload slots past the range's sequences hold zeros and are never used
        rope_q_lane<DTYPE, D>(qpre[e], p.rope, ent[e][1] - p.Lq + i, rv, hl);
  }
#pragma unroll
  for (int e = 0; e < C::QPRE; ++e)
#pragma unroll
    for (int kk = 0; kk < C::KK; ++kk) qpre[e][kk] ^= u32x4{p.q_sign, p.q_sign, p.q_sign, p.q_sign};

  // Compute cursor and the running state of the current sequence piece.
  int ce = -1, c_base = 0, c_end = 0, c_stage = 0;
  int c_b = 0, c_ctx = 0, c_ttlo = 0, lim = 0, lim_min = 0;
  bool poison = false;
  u32x4 qf[C::KK];
  f32x16 acc[C::DT];
  float m = -INFINITY, l = 0.f;
  const float c = p.scale_log2;

  // First tile of the next sequence piece. FIRST: the piece of the range's
  // first tile, set up before the tile loop, so the q rows preloaded for it
  // are dead inside the loop when no later piece uses them (QPRE = 1).
  auto begin_piece = [&](const int n, auto FIRST) CIE_PAGED_INLINE {
    {
      ++ce;
      c_base = n;
      c_end = n + ent[ce][3];
      c_b = ent[ce][0];
      c_ctx = ent[ce][1];
      c_ttlo = ent[ce][2];
      {
        const int idb = ent[ce][4], blk_lo = ent[ce][5];
        const int blk_hi = (int)fdiv((uint32_t)(min(c_ctx, kPagedTile * (c_ttlo + ent[ce][3])) - 1), p.bsdiv);
        bool bad = false;
        for (int x = lane; x < blk_hi - blk_lo + 1; x += 64) bad |= sbt[idb + x] < 0;
        poison = __builtin_amdgcn_ballot_w64(bad) != 0;
      }
      if (decltype(FIRST)::value && C::QPRE > 0) {
#pragma unroll
        for (int kk = 0; kk < C::KK; ++kk) qf[kk] = qpre[0][kk];
      } else if (!decltype(FIRST)::value && C::QPRE > 1 && ce < C::QPRE) {
#pragma unroll
        for (int e = 1; e < C::QPRE; ++e)
          if (e == ce)
#pragma unroll
            for (int kk = 0; kk < C::KK; ++kk) qf[kk] = qpre[e][kk];
      } else {
#pragma unroll
        for (int kk = 0; kk < C::KK; ++kk) qf[kk] = load16(qrow + c_b * p.qs0 + 16 * kk + 8 * hl, rv);
        if (p.rope.cos) rope_q_lane<DTYPE, D>(qf, p.rope, c_ctx - p.Lq + i, rv, hl);
#pragma unroll
        for (int kk = 0; kk < C::KK; ++kk) qf[kk] ^= u32x4{p.q_sign, p.q_sign, p.q_sign, p.q_sign};
      }
#pragma unroll
      for (int dt = 0; dt < C::DT; ++dt) acc[dt] = f32x16{};
      m = -INFINITY;
      l = 0.f;
      // Last key visible to this row: the Lq new tokens are the newest Lq
      // positions of the context (bottom-right causal alignment).
      lim = p.causal ? c_ctx - p.Lq + i : c_ctx - 1;
      lim_min = p.causal ? c_ctx - p.Lq : c_ctx - 1;
    }
  };
  begin_piece(0, std::true_type{});

  for (int n = 0; n < T; ++n) {
    if (issuer) {
      if (n + NST - 1 < T) issue(n + NST - 1);
      wait_tiles_ahead<C::DPW>(min(NST - 1, T - 1 - n));
    }
    __syncthreads();  // tile n is in LDS for every wave
    if (n == 0) CIE_STAMP(paged_timeline, 2);  // first tile in LDS

    if (n > 0 && n == c_end) begin_piece(n, std::false_type{});

    const uint16_t* kst = ring + c_stage * STAGE_EL;
    const uint16_t* vst = kst + TILE_EL;
    c_stage = c_stage + 1 == NST ? 0 : c_stage + 1;
    const int t0 = kPagedTile * (c_ttlo + n - c_base);
    if (APPEND && p.rope.cos && t0 + kPagedTile > c_ctx - p.Lq) {
      // fused append with RoPE: the new K rows of this tile arrived
      // unrotated from kn; rotate them in LDS at their positions (pairs of
      // 16-byte chunks j, j + D/16 of each head, found through the row
      // swizzle), then publish the rotated tile
      const int first = max(c_ctx - p.Lq, t0), last = min(c_ctx, t0 + kPagedTile);
      const int items = (last - first) * p.Hg * (D / 16);
      for (int u = threadIdx.x; u < items; u += blockDim.x) {
        const int tr = u / (p.Hg * (D / 16)), rem = u - tr * p.Hg * (D / 16);
        const int hd = rem / (D / 16), jj = rem - hd * (D / 16);
        const int pos = first + tr, t = pos - t0;
        const int sw = row_swizzle(NCH, t);
        uint16_t* rowp = const_cast<uint16_t*>(kst) + (t << lg_nch) * 8;
        u32x4* lo = reinterpret_cast<u32x4*>(rowp + ((hd * C::S + jj) ^ sw) * 8);
        u32x4* hi = reinterpret_cast<u32x4*>(rowp + ((hd * C::S + jj + C::S / 2) ^ sw) * 8);
        u32x4 a = *lo, b = *hi;
        const bool ok = pos < p.rope.rows;
        const int64_t tr0 = (ok ? (int64_t)pos : 0) * (D / 2) + 8 * jj;
        rope_apply8<DTYPE>(a, b, rope_load(p.rope, tr0), p.rope.dt);
        if (!ok) a = b = u32x4{0x7fff7fffu, 0x7fff7fffu, 0x7fff7fffu, 0x7fff7fffu};
        *lo = a;
        *hi = b;
      }
      __syncthreads();
    }

    f32x16 sc = f32x16{};
#pragma unroll
    for (int kk = 0; kk < C::KK; ++kk) {
      const int pos = (hh * C::S + 2 * kk + hl) ^ swk;
      const u32x4 a = *reinterpret_cast<const u32x4*>(kst + ((l32 << lg_nch) + pos) * 8);
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
      for (int x = 0; x < 4; ++x) pb[cc][x] = E::pack2(sc[8 * cc + 2 * x], sc[8 * cc + 2 * x + 1]);

    // V^T fragments: lane (group gq, r = rq) points at token k0 + r/4, dims
    // d0 + 4 (r % 4); the transpose read hands lane l the four keys k0..k0+3
    // of dim 32 dt + lane % 32.
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) {
      int d = 32 * dt + 16 * (gq & 1) + 4 * (rq & 3);
      if (D < 32) d = min(d, D - 4);  // rows >= D of O^T are discarded
      const int chunk = hh * C::S + (d >> 3), within = d & 7;
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
        const int tlo = 16 * cc + 4 * hl + (rq >> 2);
        const int thi = tlo + 8;
        const u32x2 lo = lds_read_tr16(vst + ((tlo << lg_nch) + (chunk ^ swv[cc][0])) * 8 + within);
        const u32x2 hi = lds_read_tr16(vst + ((thi << lg_nch) + (chunk ^ swv[cc][1])) * 8 + within);
        acc[dt] = E::mfma(u32x4{lo[0], lo[1], hi[0], hi[1]}, pb[cc], acc[dt]);
      }
    }

    if (n == c_end - 1) {  // last tile of the piece
      const float l_tot = xhalf_sum(l);
      if (ent[ce][7] == 1 || !p.slots) {
        // (no partial-state space: the caller's plan said nothing is split,
        // which this plan contradicts; the rows are NaN rather than partial)
        const float inv = poison || ent[ce][7] != 1 ? __builtin_nanf("") : 1.f / l_tot;
        if (rv) store_row<DTYPE, D>(p.o + (int64_t)c_b * p.os0 + hq * p.os1 + (int64_t)i * p.os2, acc, inv, hl);
      } else {
        // Piece of a split sequence: side 1 if it starts inside this range.
        const int side = ent[ce][6] > S0 ? 1 : 0;
        float* sl = p.slots + ((((int64_t)j * p.NG + gh) * 2 + side) * p.NWV + w) * p.Rt * (D + 2);
        const float pz = poison ? __builtin_nanf("") : 1.f;
        if (rv) {
#pragma unroll
          for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
              const int d = 32 * dt + 8 * g4 + 4 * hl;
              if (D >= 32 || d < D)
                *reinterpret_cast<float4*>(sl + l32 * D + d) =
                    float4{acc[dt][4 * g4] * pz, acc[dt][4 * g4 + 1] * pz, acc[dt][4 * g4 + 2] * pz,
                           acc[dt][4 * g4 + 3] * pz};
            }
          if (hl == 0) *reinterpret_cast<float2*>(sl + p.Rt * D + 2 * l32) = float2{m * pz, l_tot * pz};
        }
      }
    }
    __syncthreads();  // every wave is done with this stage before it is refilled
  }

  CIE_STAMP(paged_timeline, 3);  // tile loop done

  // Fused append: the new tokens inside this range go into the pool, the
  // head group's rows of each (16-byte chunks over the whole workgroup).
  // Nothing in this launch reads those pool rows (the tiles holding them
  // took the rows from kn / vn), so no ordering is needed.
  if (APPEND) {
    const int cpr = p.Hg * (D / 8);  // chunks of one tensor per token row of the head group
    const bool rot = p.rope.cos != nullptr;
    for (int e = 0; e < ne; ++e) {
      const int ctx = ent[e][1], tt_lo = ent[e][2], n = ent[e][3], idb = ent[e][4], blk_lo = ent[e][5];
      const int lo = max(ctx - p.Lq, kPagedTile * tt_lo), hi = min(ctx, kPagedTile * (tt_lo + n));
      const int b = ent[e][0];
      for (int u = threadIdx.x; u < (hi > lo ? hi - lo : 0) * cpr * 2; u += blockDim.x) {
        const int tsr = u / (2 * cpr), rem = u - tsr * 2 * cpr;
        const int tensor = rem / cpr, c = rem - tensor * cpr;
        const int pos = lo + tsr;
        const int blk = (int)fdiv((uint32_t)pos, p.bsdiv);
        const int bid = sbt[idb + blk - blk_lo];
        if (bid < 0) continue;  // invalid block id: the output is NaN, nothing is written
        // a position outside the rotary tables: NaN output rows, neither K nor
        // V written (as the rotating append leaves the pool)
        if (rot && pos >= p.rope.rows) continue;
        const int off = pos - blk * p.block_size;
        const int h = gh * p.Hg + c / (D / 8), d = 8 * (c % (D / 8));
        const int64_t row = (int64_t)b * p.Lq + (pos - (ctx - p.Lq));
        if (tensor == 0 && rot) {
          // K rotated at its position: the thread of the pair's first chunk writes both
          if (d >= D / 2) continue;
          const uint16_t* src = p.kn + row * p.kns0 + (int64_t)h * p.kns1 + d;
          u32x4 a = *reinterpret_cast<const u32x4*>(src), bb = *reinterpret_cast<const u32x4*>(src + D / 2);
          rope_apply8<DTYPE>(a, bb, rope_load(p.rope, (int64_t)pos * (D / 2) + d), p.rope.dt);
          uint16_t* dst = const_cast<uint16_t*>(p.kc) + (int64_t)bid * p.ks0 + (int64_t)off * p.ks1 +
                          (int64_t)h * p.ks2 + d;
          *reinterpret_cast<u32x4*>(dst) = a;
          *reinterpret_cast<u32x4*>(dst + D / 2) = bb;
        } else if (tensor == 0)
          *reinterpret_cast<u32x4*>(const_cast<uint16_t*>(p.kc) + (int64_t)bid * p.ks0 + (int64_t)off * p.ks1 +
                                    (int64_t)h * p.ks2 + d) =
              *reinterpret_cast<const u32x4*>(p.kn + row * p.kns0 + (int64_t)h * p.kns1 + d);
        else
          *reinterpret_cast<u32x4*>(const_cast<uint16_t*>(p.vc) + (int64_t)bid * p.vs0 + (int64_t)off * p.vs1 +
                                    (int64_t)h * p.vs2 + d) =
              *reinterpret_cast<const u32x4*>(p.vn + row * p.vns0 + (int64_t)h * p.vns1 + d);
      }
    }
  }

  CIE_STAMP(paged_timeline, 4);  // end
}

// Second pass: combines the pieces of every split sequence. Eight lanes
// share one (sequence, head group, wave slot, row, 4 columns) item; lane t of
// the eight combines pieces t, t + 8, ... (all its loads issued together,
// unconditionally, at addresses clamped to the last piece), then the eight
// partial states are combined by a fixed butterfly, so the result does not
// depend on timing. The piece descriptor written by the first pass says
// where the pieces are.
constexpr int kMergeLanes = 8;
constexpr int kMergeBatch = 4;  // pieces per lane per batch

__device__ __forceinline__ void merge_state(float& M, float& L, float4& A, float m2, float l2, float4 a2) {
  const float Mn = maxf(M, m2);
  const float wo = rescale_weight(M, Mn), wn = rescale_weight(m2, Mn);
  L = L * wo + l2 * wn;
  A.x = A.x * wo + a2.x * wn;
  A.y = A.y * wo + a2.y * wn;
  A.z = A.z * wo + a2.z * wn;
  A.w = A.w * wo + a2.w * wn;
  M = Mn;
}

// Value of lane (lane ^ OFF) for OFF = 1, 2, 4, by DPP: quad permutations for
// 1 and 2, the two row rotations by 4 (row_ror:12 reads lane + 4, row_ror:4
// reads lane - 4 within each row of 16) for 4.
template <int OFF>
__device__ __forceinline__ float lane_xor(float x) {
  const int v = __float_as_int(x);
  if constexpr (OFF == 1) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(v, 0xb1, 0xf, 0xf, false));  // quad_perm [1,0,3,2]
  } else if constexpr (OFF == 2) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(v, 0x4e, 0xf, 0xf, false));  // quad_perm [2,3,0,1]
  } else {
    static_assert(OFF == 4, "lane_xor: 1, 2 or 4");
    const int up = __builtin_amdgcn_mov_dpp(v, 0x12c, 0xf, 0xf, false);  // row_ror:12
    const int dn = __builtin_amdgcn_mov_dpp(v, 0x124, 0xf, 0xf, false);  // row_ror:4
    return __int_as_float((threadIdx.x & 4) ? dn : up);
  }
}

template <int OFF>
__device__ __forceinline__ void butterfly_step(int t, float& M, float& L, float4& A) {
  const float m2 = lane_xor<OFF>(M), l2 = lane_xor<OFF>(L);
  const float4 a2 = {lane_xor<OFF>(A.x), lane_xor<OFF>(A.y), lane_xor<OFF>(A.z), lane_xor<OFF>(A.w)};
  // the lower lane of each pair keeps its own state first: same order in both lanes
  if (t & OFF) {
    float Mx = m2, Lx = l2;
    float4 Ax = a2;
    merge_state(Mx, Lx, Ax, M, L, A);
    M = Mx, L = Lx, A = Ax;
  } else {
    merge_state(M, L, A, m2, l2, a2);
  }
}

template <int DTYPE, int D>
__global__ __launch_bounds__(256) void paged_merge_kernel(const PagedParams p) {
  using E = Elt<DTYPE>;
  constexpr int Q4 = D / 4;
  static_assert(kMergeLanes == 8, "the butterfly below covers eight lanes");
  warm_kernargs<sizeof(PagedParams)>();
  // thread index < 2^31 (paged_geometry bounds the merge grid): 32-bit
  // decomposition, invariant divisors by multiply-shift. With the plan's
  // merge table, workgroup (XCD x, slot s) takes part s % wpu of the x-th
  // list's sequence s / wpu; otherwise the sequences follow the grid.
  uint32_t tid = blockIdx.x * 256u + threadIdx.x;
  // a plan built for other arguments: the main pass has written NaN rows,
  // and the offsets of its descriptors and merge table may lie past its end
  if (p.plan && !plan_matches<D>(p)) return;
  int unit = -1;
  int4 minf = {0, 0, 0, 0};  // the table entry's piece descriptor
  if (p.mtab_cap > 0) {
    const uint32_t per_unit = (uint32_t)p.NWV * p.Rt * Q4 * kMergeLanes;
    const uint32_t wpu = (per_unit + 255) / 256;
    const uint32_t slot = blockIdx.x >> p.xcd_shift, ui = slot / wpu;
    const int xcd = (int)(blockIdx.x & ((1u << p.xcd_shift) - 1));
    if (ui < (uint32_t)p.mtab_cap) {
      const int4 e = reinterpret_cast<const int4*>(p.plan + p.plan_mtab)
          [(int64_t)xcd * merge_table_cap(p.B, p.NG, p.xcd_shift) + ui];
      unit = e.x;
      minf = int4{e.y, e.z, e.w, 0};
    }
    if (unit < 0 || unit >= p.B * p.NG) return;  // an unused (or invalid) entry: the whole workgroup idles
    tid = (slot - ui * wpu) * 256u + threadIdx.x;
  }
  const int t = (int)(tid % kMergeLanes);
  uint32_t item = tid / kMergeLanes;
  const int d4 = (int)(item % Q4);
  item /= Q4;
  uint32_t qn = fdiv(item, p.rtdiv);
  const int row = (int)(item - qn * (uint32_t)p.Rt);
  item = qn;
  qn = fdiv(item, p.nwvdiv);
  const int w = (int)(item - qn * (uint32_t)p.NWV);
  item = qn;
  int gh, b;
  bool in;
  if (unit >= 0) {  // item is 0 within the sequence's threads
    gh = unit % p.NG;
    b = unit / p.NG;
    in = item == 0;
  } else {
    qn = fdiv(item, p.ngdiv);
    gh = (int)(item - qn * (uint32_t)p.NG);
    b = (int)qn;
    in = b < p.B;
  }
  // Items of one wave belong to at most a few sequences; lanes past the end
  // or without work still take part in the shuffles below.
  const int4 inf = unit >= 0 ? minf : (in ? p.info[(int64_t)gh * p.B + b] : int4{0, 0, 0, 0});
  const int pieces = inf.y;
  const int hh = w % p.Hg, qt = w / p.Hg;
  const int r = qt * 32 + row;
  // a descriptor that does not name ranges of this launch is ignored
  const bool described = inf.x >= 0 && pieces <= p.Wg && inf.x <= p.Wg - pieces;
  const bool act = in && pieces > 1 && r < p.R && described;
  const int64_t slot_floats = (int64_t)p.Rt * (D + 2);

  float M = -INFINITY, L = 0.f;
  float4 A = {0.f, 0.f, 0.f, 0.f};
  if (act) {
    for (int k0 = t; k0 < pieces; k0 += kMergeLanes * kMergeBatch) {
      float2 ml[kMergeBatch];
      float4 a[kMergeBatch];
#pragma unroll
      for (int u = 0; u < kMergeBatch; ++u) {
        const int k = min(k0 + kMergeLanes * u, pieces - 1);
        const int side = k == 0 ? inf.z : 0;
        const float* sl = p.slots + ((((int64_t)(inf.x + k) * p.NG + gh) * 2 + side) * p.NWV + w) * slot_floats;
        ml[u] = *reinterpret_cast<const float2*>(sl + (int64_t)p.Rt * D + 2 * row);
        a[u] = *reinterpret_cast<const float4*>(sl + row * D + 4 * d4);
      }
#pragma unroll
      for (int u = 0; u < kMergeBatch; ++u)
        if (k0 + kMergeLanes * u < pieces) merge_state(M, L, A, ml[u].x, ml[u].y, a[u]);
    }
  }
  butterfly_step<1>(t, M, L, A);
  butterfly_step<2>(t, M, L, A);
  butterfly_step<4>(t, M, L, A);
  if (!act || t != 0) return;
  const int g = r / p.Lq, i = r - g * p.Lq;
  const int hq = (gh * p.Hg + hh) * p.group + g;
  const float inv = 1.f / L;
  uint16_t* orow = p.o + (int64_t)b * p.os0 + hq * p.os1 + (int64_t)i * p.os2;
  *reinterpret_cast<u32x2*>(orow + 4 * d4) = u32x2{E::pack2(A.x * inv, A.y * inv), E::pack2(A.z * inv, A.w * inv)};
}

PagedGeom paged_geometry(int B, int Hq, int Hk, int Lq, int D, int ctx_limit, int block_size, DeviceShape dev) {
  PagedGeom g{};
  g.ok = 0;
  g.Hq = Hq;
  g.D = D;
  g.dev = dev;
  if (B < 1 || Hq < 1 || Hk < 1 || Lq < 1 || Hq % Hk || block_size < 1 || ctx_limit < 0 ||
      !(D == 16 || D == 32 || D == 64 || D == 128 || D == 256)) {
    g.err = "invalid shape";
    return g;
  }
  g.R = (Hq / Hk) * Lq;
  g.n_qt = (g.R + 31) / 32;
  g.Rt = std::min(32, g.R);
  const int maxw = paged_max_waves(D);
  if (g.n_qt > maxw) {
    g.err = D == 256 ? "more than 128 query rows per kv head (num_heads / num_kv_heads * new tokens) at head_dim 256"
                     : "more than 256 query rows per kv head (num_heads / num_kv_heads * new tokens)";
    return g;
  }
  g.Hg = 1;
  for (int h = 1; h <= Hk; ++h)
    if (Hk % h == 0 && h * D <= 256 && h * g.n_qt <= maxw) g.Hg = h;
  g.NG = Hk / g.Hg;
  g.NWV = g.Hg * g.n_qt;
  g.NCH = g.Hg * D / 8;
  const size_t stage = (size_t)2 * kPagedTile * g.NCH * 16;  // K and V tiles
  const int dpw = D / 16;
  // Ring budget: decode-like shapes (few query rows per kv head, little
  // compute per tile) run best as two workgroups per CU with two stages
  // each; verify-like ones as one workgroup with three (decode_b32 -3 %,
  // verify_b8 -1.4 % against four stages for both).
  const size_t budget = g.R <= 8 ? 75 * 1024 : 100 * 1024;
  int nst = (int)std::min<size_t>(4, std::min<size_t>(budget, kPagedLdsBudget) / stage);
  nst = std::min(std::max(nst, 2), 1 + 31 / dpw);  // 2 * dpw * (nst - 1) copies fit vmcnt
  g.NST = nst;
  g.lds_bytes = (size_t)nst * stage;
  const size_t static_lds = sizeof(int32_t) * (kPagedIds + 8 * kPagedEntries) + 16;
  int wpc = (int)((160 * 1024) / (g.lds_bytes + static_lds));
  wpc = std::max(1, std::min(wpc, 16 / g.NWV));
  const int64_t nt_upper = (int64_t)B * ((ctx_limit + kPagedTile - 1) / kPagedTile);
  const int ids_per_tile = (kPagedTile + block_size - 1) / block_size + 2;
  const int tcap = std::min(kPagedEntries, kPagedIds / ids_per_tile);
  int64_t wg = std::max<int64_t>(1, (int64_t)dev.cus * wpc / g.NG);
  wg = std::min<int64_t>(wg, std::max<int64_t>(1, nt_upper));
  wg = std::max<int64_t>(wg, (nt_upper + tcap - 1) / tcap);
  if (wg * g.NG > INT_MAX) {
    g.err = "problem too large for one launch";
    return g;
  }
  g.Wg = (int)wg;
  if ((int64_t)B * g.NG * g.NWV * g.Rt * (D / 4) * kMergeLanes >= ((int64_t)1 << 31)) {
    g.err = "problem too large for one launch";
    return g;
  }
  g.info_bytes = ((size_t)g.NG * B * sizeof(int4) + 255) / 256 * 256;
  g.slot_bytes = (size_t)g.NG * g.Wg * 2 * g.NWV * g.Rt * (D + 2) * sizeof(float);
  g.ok = 1;
  return g;
}

template <int DTYPE, int D>
static hipError_t launch_paged_t(const PagedParams& p, size_t lds, bool merge, hipStream_t stream) {
  const void* fn = p.kn ? reinterpret_cast<const void*>(&paged_fwd_kernel<DTYPE, D, true>)
                        : reinterpret_cast<const void*>(&paged_fwd_kernel<DTYPE, D, false>);
  const hipError_t attr = set_dynamic_lds(fn, kPagedLdsBudget);
  if (attr != hipSuccess) return attr;
  const int64_t n_wg = (int64_t)p.NG * p.Wg;
  if (p.kn)
    hipLaunchKernelGGL((paged_fwd_kernel<DTYPE, D, true>), dim3((unsigned)n_wg), dim3(64 * p.NWV), lds, stream, p);
  else
    hipLaunchKernelGGL((paged_fwd_kernel<DTYPE, D, false>), dim3((unsigned)n_wg), dim3(64 * p.NWV), lds, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !merge) return e;
  const int64_t per_unit = (int64_t)p.NWV * p.Rt * (D / 4) * kMergeLanes;
  const int64_t n_merge = p.mtab_cap > 0 ? ((int64_t)p.mtab_cap << p.xcd_shift) * ((per_unit + 255) / 256)
                                         : ((int64_t)p.B * p.NG * per_unit + 255) / 256;
  hipLaunchKernelGGL((paged_merge_kernel<DTYPE, D>), dim3((unsigned)n_merge), dim3(256), 0, stream, p);
  return hipGetLastError();
}

template <int DTYPE>
static hipError_t launch_paged_d(const PagedParams& p, int D, size_t lds, bool merge, hipStream_t stream) {
  switch (D) {
    case 16: return launch_paged_t<DTYPE, 16>(p, lds, merge, stream);
    case 32: return launch_paged_t<DTYPE, 32>(p, lds, merge, stream);
    case 64: return launch_paged_t<DTYPE, 64>(p, lds, merge, stream);
    case 128: return launch_paged_t<DTYPE, 128>(p, lds, merge, stream);
    case 256: return launch_paged_t<DTYPE, 256>(p, lds, merge, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_paged(const PagedParams& p, int dtype, int D, size_t lds, bool merge, hipStream_t stream) {
  return dtype == 0 ? launch_paged_d<0>(p, D, lds, merge, stream) : launch_paged_d<1>(p, D, lds, merge, stream);
}

// Static workspace of the allocation-free paged entry: one copy per GPU,
// loaded with the code object and held until the process ends. Every call
// on a device shares it, so calls that overlap on one device race; nothing
// in it needs to start at zero (the main pass writes every piece descriptor
// the merge pass reads, and every partial state before its descriptor).
static __device__ __align__(256) unsigned char paged_scratch[kPagedScratchBytes];

hipError_t paged_scratch_ptr(void** ptr) {
  static std::mutex mu;
  static std::map<int, void*> per_device;  // the array's address on each device
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(mu);
  auto it = per_device.find(dev);
  if (it == per_device.end()) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(paged_scratch));  // with `dev` current
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    it = per_device.emplace(dev, p).first;
  }
  *ptr = it->second;
  return hipSuccess;
}

}  // namespace cie

#ifdef CIE_TIMELINE
// timeline build only: the stamps of the last paged_fwd_kernel launch
extern "C" int cie_timeline_paged(void* host, size_t bytes) {
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(cie::paged_timeline), bytes, 0, hipMemcpyDeviceToHost);
}
#endif
