// Host-built work plan of the paged attention kernels.
//
// Without a plan every workgroup of paged_fwd_kernel derives its share of
// the work on the device: it reads all context lengths, scans them, cuts the
// concatenated 32-token tiles into equal ranges and fetches the block ids of
// its range -- three dependent memory round trips before its first KV tile
// is requested. The engine already knows the lengths and block tables on the
// host when it prepares a step (the reference's BlockTable lists,
// engine/cache/block_table.py:16-18, and the lengths it appends,
// engine/cache/kv_cache.py:138-139), so it can build the same schedule once
// per step, upload it with the step's other metadata and let every layer's
// launch read its range directly: one round trip (the range row), then the
// entries and block ids of the range by direct-to-LDS copies.
//
// The schedule is the one the device derives (same ranges, same pieces, same
// arithmetic order), so planned and unplanned launches give bit-identical
// results.
//
// Layout (int32), offsets fixed by the launch geometry so the launch knows
// them without reading the plan:
//   header   kPlanHeader ints (PlanHeader): magic, W, NT, Wg, empties,
//            split sequences, B, append flag, then the arguments the layout
//            and the validated ids depend on: NG, Lq, D, num_blocks,
//            block_size, max_blocks, ctx_limit, Hq. A launch compares them
//            all with its own before it reads anything else of the plan.
//   ranges   Wg rows of kPlanRangeInts: first entry, entries, first id, ids,
//            S0 (first tile), T (tiles)
//   entries  (Wg + B) rows of 8: b, ctx, tt_lo, n, idb (from the range's
//            first id), blk_lo, pre (tiles before the sequence), pieces
//   ids      B * max_blocks + 2 * Wg block ids of the ranges, in range
//            order; an id outside [0, num_blocks) is stored as -1
//   info     NG * B int4: first range, pieces, slot side of piece 0 (the
//            merge pass's piece descriptors), zero for unsplit sequences
//   empty    B rows of 2: sequences without tiles (b, 1 if the history is
//            empty, 0 if its length is invalid)
//   mtab     (int4 aligned) kMaxXcds lists of merge_table_cap(B, NG,
//            xcd_shift) entries of 4 ints: the split sequences (b * NG + gh,
//            then its info descriptor) whose merge runs on each XCD,
//            {-1, 0, 0, 0} past the end (and in the lists of XCDs the device
//            does not have);
//            each goes to the XCD that ran its middle piece (its partial
//            states are in that XCD's L2), or, when that list holds
//            merge_cap(split sequences) already, to the shortest list
#include <algorithm>
#include <cstring>
#include <vector>

#include "kernels.hpp"

namespace cie {

PlanLayout paged_plan_layout(const PagedGeom& g, int B, int max_blocks) {
  PlanLayout L{};
  L.ranges = kPlanHeader;
  L.entries = L.ranges + (size_t)kPlanRangeInts * g.Wg;
  L.ids = L.entries + (size_t)8 * (g.Wg + B);
  L.info = L.ids + (size_t)B * max_blocks + (size_t)2 * g.Wg;
  L.info = (L.info + 3) / 4 * 4;  // int4 aligned
  L.empty = L.info + (size_t)4 * g.NG * B;
  L.mtab = (L.empty + (size_t)2 * B + 3) / 4 * 4;  // int4 aligned
  L.ints = L.mtab + (size_t)4 * kMaxXcds * merge_table_cap(B, g.NG, g.dev.xcd_shift);
  return L;
}

// Tile ranges exactly as paged_fwd_kernel cuts them: W = min(Wg, NT) ranges
// [floor(j NT / W), floor((j+1) NT / W)).
static int64_t range_start(int64_t j, int64_t NT, int64_t W) { return j * NT / W; }
static int range_of(int64_t x, int64_t NT, int64_t W) { return (int)(((x + 1) * W - 1) / NT); }

int build_paged_plan(int32_t* P, const PagedGeom& g, const PlanLayout& L, const int32_t* lens,
                     const int32_t* bt, int64_t bt_stride, int B, int Lq, int num_blocks, int block_size,
                     int max_blocks, int ctx_limit, int append) {
  std::memset(P, 0, L.ints * sizeof(int32_t));
  // tiles per sequence (0 for an empty history or an invalid length)
  std::vector<int> tiles(B), valid(B);
  int64_t NT = 0;
  for (int b = 0; b < B; ++b) {
    const int ctx = lens[b];
    valid[b] = ctx >= (append ? Lq : 0) && ctx <= ctx_limit && (ctx == 0 || num_blocks > 0);
    tiles[b] = valid[b] ? (ctx + kPagedTile - 1) / kPagedTile : 0;
    NT += tiles[b];
  }
  const int64_t W = std::min<int64_t>(g.Wg, NT);
  int32_t* R = P + L.ranges;
  int32_t* E = P + L.entries;
  int32_t* I = P + L.ids;
  int32_t* F = P + L.info;
  int32_t* Z = P + L.empty;
  int ne_total = 0, nid_total = 0, split = 0, n_empty = 0;
  for (int b = 0; b < B; ++b)
    if (tiles[b] == 0) {
      Z[2 * n_empty] = b;
      Z[2 * n_empty + 1] = valid[b] ? 1 : 0;
      ++n_empty;
    }
  // first tile of every sequence in the concatenation
  std::vector<int64_t> pre(B + 1, 0);
  for (int b = 0; b < B; ++b) pre[b + 1] = pre[b] + tiles[b];
  for (int b = 0; b < B; ++b)
    if (tiles[b] > 0 && range_of(pre[b] + tiles[b] - 1, NT, W) > range_of(pre[b], NT, W)) ++split;
  int b0 = 0;  // first sequence that may overlap the current range
  for (int64_t j = 0; j < W; ++j) {
    const int64_t S0 = range_start(j, NT, W), S1 = range_start(j + 1, NT, W);
    int32_t* row = R + (size_t)kPlanRangeInts * j;
    row[0] = ne_total;
    row[2] = nid_total;
    row[4] = (int32_t)S0;
    row[5] = (int32_t)(S1 - S0);
    while (b0 < B && pre[b0] + tiles[b0] <= S0) ++b0;
    int ne = 0, nid = 0;
    for (int b = b0; b < B && pre[b] < S1; ++b) {
      const int t = tiles[b];
      if (t == 0 || pre[b] + t <= S0) continue;
      if (ne >= kPagedEntries) return -1;  // the geometry bounds this; never reached
      const int ctx = lens[b];
      const int tt_lo = (int)std::max<int64_t>(S0 - pre[b], 0);
      const int tt_hi = (int)std::min<int64_t>(S1 - pre[b], t);
      const int blk_lo = kPagedTile * tt_lo / block_size;
      const int blk_hi = (std::min(ctx, kPagedTile * tt_hi) - 1) / block_size;
      const int nids = blk_hi - blk_lo + 1;
      if (nid + nids > kPagedIds) return -1;
      const int j0 = range_of(pre[b], NT, W), j1 = range_of(pre[b] + t - 1, NT, W);
      int32_t* e = E + (size_t)8 * (ne_total + ne);
      e[0] = b;
      e[1] = ctx;
      e[2] = tt_lo;
      e[3] = tt_hi - tt_lo;
      e[4] = nid;
      e[5] = blk_lo;
      e[6] = (int32_t)pre[b];
      e[7] = j1 - j0 + 1;
      for (int x = 0; x < nids; ++x) {
        const int id = bt[(int64_t)b * bt_stride + blk_lo + x];
        I[nid_total + nid + x] = (id >= 0 && id < num_blocks) ? id : -1;
      }
      if (pre[b] >= S0)  // the range holding the first tile describes the pieces
        for (int gh = 0; gh < g.NG; ++gh) {
          int32_t* f = F + (size_t)4 * ((size_t)gh * B + b);
          f[0] = (int32_t)j;
          f[1] = j1 - j0 + 1;
          f[2] = pre[b] > S0 ? 1 : 0;
        }
      ++ne;
      nid += nids;
    }
    row[1] = ne;
    row[3] = nid;
    ne_total += ne;
    nid_total += nid;
  }
  // merge table (launches placed in XCD runs only): every split sequence of
  // every head group, on the XCD of its middle piece when that list has room
  {
    const int xs = g.dev.xcd_shift, nx = 1 << xs;
    const int cap_t = merge_table_cap(B, g.NG, xs), cap = merge_cap(split * g.NG, xs);
    int32_t* T = P + L.mtab;
    for (int i = 0; i < kMaxXcds * cap_t; ++i) T[4 * i] = -1;  // (the descriptor ints stay 0)
    if (paged_xcd_runs(g)) {
      int cnt[kMaxXcds] = {0, 0, 0, 0, 0, 0, 0, 0};
      const int64_t n = (int64_t)g.NG * g.Wg;
      for (int b = 0; b < B; ++b)
        for (int gh = 0; gh < g.NG; ++gh) {
          const int32_t* f = F + (size_t)4 * ((size_t)gh * B + b);
          if (tiles[b] == 0 || f[1] <= 1) continue;
          int x = xcd_of_logical((int64_t)gh * g.Wg + f[0] + f[1] / 2, n, xs);
          if (cnt[x] >= cap) x = (int)(std::min_element(cnt, cnt + nx) - cnt);
          int32_t* t = T + (size_t)4 * (x * cap_t + cnt[x]++);
          t[0] = b * g.NG + gh;
          t[1] = f[0];
          t[2] = f[1];
          t[3] = f[2];
        }
    }
  }
  P[kPlMagic] = kPlanMagic;
  P[kPlW] = (int32_t)W;
  P[kPlNT] = (int32_t)NT;
  P[kPlWg] = g.Wg;
  P[kPlEmpty] = n_empty;
  P[kPlSplit] = split;
  P[kPlB] = B;
  P[kPlAppend] = append ? 1 : 0;
  P[kPlNG] = g.NG;
  P[kPlLq] = Lq;
  P[kPlD] = g.D;
  P[kPlNumBlocks] = num_blocks;
  P[kPlBlockSize] = block_size;
  P[kPlMaxBlocks] = max_blocks;
  P[kPlCtxLimit] = ctx_limit;
  P[kPlHq] = g.Hq;
  return split;
}

}  // namespace cie
