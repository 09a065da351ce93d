"""Host-side integer math the kernels rely on, checked on the CPU.

* FastDiv (csrc/common.hpp: make_fastdiv / fdiv): q = (umulhi(n, mul) + n) >> shift
  must equal n // d for every divisor the paged kernel may see (block sizes)
  and every token index below 2^31.
* The prefill grid's XCD-aware remap (csrc/flash_fwd.hip) must be a bijection
  from workgroup ids onto (batch, kv head, query tile, group member).
"""

from __future__ import annotations

import itertools
import random


def make_fastdiv(d: int) -> tuple[int, int]:
    s = 0
    while (1 << s) < d:
        s += 1
    return (((1 << 32) * ((1 << s) - d)) // d + 1) & 0xFFFFFFFF, s


def fdiv(n: int, mul: int, s: int) -> int:
    return (((n * mul) >> 32) + n) >> s


def test_fastdiv_exact():
    rng = random.Random(0)
    for d in list(range(1, 300)) + [1023, 1024, 4096, 65535, 100000, 2**20 + 7]:
        mul, s = make_fastdiv(d)
        assert mul < 2**32
        for n in list(range(0, 3000)) + [rng.randrange(0, 2**31) for _ in range(500)] + [2**31 - 1]:
            assert fdiv(n, mul, s) == n // d, (d, n)


def _remap(N, n_mt, G, Hk, B):
    seen = set()
    for bid in range(N):
        xcd, slot = bid & 7, bid >> 3
        logical = xcd * (N >> 3) + min(xcd, N & 7) + slot
        assert 0 <= logical < N
        per = n_mt * G
        grp, rem = divmod(logical, per)
        mt, g = n_mt - 1 - rem // G, rem % G
        b, kvh = divmod(grp, Hk)
        assert 0 <= mt < n_mt and 0 <= g < G and 0 <= kvh < Hk and 0 <= b < B
        seen.add((b, kvh, mt, g))
    return len(seen) == N


def test_prefill_grid_remap_is_bijective():
    for B, Hk, G, n_mt in itertools.product([1, 2, 3, 4], [1, 2, 3, 8], [1, 2, 4, 7], [1, 2, 5, 16, 33]):
        assert _remap(n_mt * B * Hk * G, n_mt, G, Hk, B)


# ---------------------------------------------------------------- paged launch geometry and schedule
#
# Python mirror of paged_geometry() and of the per-workgroup schedule the
# paged kernel derives from the context lengths (csrc/paged_fwd.hip).

TILE, IDS, ENTRIES, MAX_WAVES, CUS, LDS_BUDGET = 32, 384, 32, 8, 256, 150 * 1024


def paged_geometry(B, Hq, Hk, Lq, D, ctx_limit, bs):
    R = (Hq // Hk) * Lq
    n_qt = (R + 31) // 32
    Rt = min(32, R)
    if n_qt > MAX_WAVES:
        return None
    Hg = max(h for h in range(1, Hk + 1) if Hk % h == 0 and h * D <= 256 and h * n_qt <= MAX_WAVES)
    NG, NWV, NCH = Hk // Hg, Hg * n_qt, Hg * D // 8
    stage = 2 * TILE * NCH * 16
    dpw = D // 16
    budget = 75 * 1024 if R <= 8 else 100 * 1024
    nst = min(max(min(4, min(budget, LDS_BUDGET) // stage), 2), 1 + 31 // dpw)
    lds = nst * stage
    static = 4 * (IDS + 8 * ENTRIES) + 16
    wpc = max(1, min((160 * 1024) // (lds + static), 16 // NWV))
    nt_upper = B * ((ctx_limit + TILE - 1) // TILE)
    tcap = min(ENTRIES, IDS // ((TILE + bs - 1) // bs + 2))
    wg = max(1, CUS * wpc // NG)
    wg = min(wg, max(1, nt_upper))
    wg = max(wg, -(-nt_upper // tcap))
    cnt = (NG * B * 16 + 255) // 256 * 256
    slots = NG * wg * 2 * NWV * Rt * (D + 2) * 4
    return dict(R=R, Rt=Rt, n_qt=n_qt, Hg=Hg, NG=NG, NWV=NWV, NCH=NCH, NST=nst, Wg=wg, lds=lds,
                ws=cnt + slots, tcap=tcap, dpw=dpw)


def range_of(x, nt, wg):
    return ((x + 1) * wg - 1) // nt


def schedule(lens, ctx_limit, bs, wg):
    """Entries (b, tt_lo, n, pre, pieces, side) and staged block ids of every
    workgroup range, as the kernel derives them."""
    tiles = [(c + TILE - 1) // TILE if 0 <= c <= ctx_limit else 0 for c in lens]
    pre = [sum(tiles[:b]) for b in range(len(lens))]
    NT = sum(tiles)
    W = min(wg, NT)  # no empty range
    out = []
    for j in range(wg):
        S0, S1 = (j * NT // W, (j + 1) * NT // W) if j < W else (NT, NT)
        ents, nid = [], 0
        for b, t in enumerate(tiles):
            if t == 0 or not (pre[b] < S1 and pre[b] + t > S0):
                continue
            tt_lo = max(S0 - pre[b], 0)
            tt_hi = min(S1 - pre[b], t)
            blk_lo = (TILE * tt_lo) // bs
            blk_hi = (min(lens[b], TILE * tt_hi) - 1) // bs
            pieces = range_of(pre[b] + t - 1, NT, W) - range_of(pre[b], NT, W) + 1
            side = 1 if pre[b] > S0 else 0
            ents.append((b, tt_lo, tt_hi - tt_lo, pre[b], pieces, side))
            nid += blk_hi - blk_lo + 1
        out.append((S0, S1, ents, nid))
    return out, tiles, pre, NT, W


def test_paged_workspace_matches_library():
    from engine import _lib

    lib = _lib.load()
    rng = random.Random(3)
    for _ in range(300):
        D = rng.choice([16, 32, 64, 128, 256])
        Hk = rng.choice([1, 2, 4, 8, 16])
        Hq = Hk * rng.choice([1, 2, 4, 8])
        Lq = rng.choice([1, 2, 5, 8, 16])
        bs = rng.choice([1, 4, 8, 16, 32, 64])
        mb = rng.randrange(1, 300)
        B = rng.randrange(1, 80)
        mc = rng.choice([0, rng.randrange(1, mb * bs + 1)])
        limit = min(mc, mb * bs) if mc > 0 else mb * bs
        g = paged_geometry(B, Hq, Hk, Lq, D, limit, bs)
        got = lib.cie_paged_workspace_bytes(B, Hq, Hk, Lq, D, mc, bs, mb)
        assert got == (g["ws"] if g else 0), (B, Hq, Hk, Lq, D, mc, bs, mb)


def test_paged_schedule_covers_every_tile_once_within_lds_bounds():
    rng = random.Random(4)
    for trial in range(200):
        bs = rng.choice([1, 2, 8, 16, 32, 48])
        B = rng.randrange(1, 70)
        limit = rng.choice([64, 500, 4096])
        lens = [rng.choice([0, rng.randrange(1, limit + 1), limit, limit + 7, -1]) for _ in range(B)]
        g = paged_geometry(B, 32, 8, rng.choice([1, 5]), 64, limit, bs)
        wg = g["Wg"] if trial % 2 else 4 * g["Wg"] + 3  # also far more ranges than tiles
        sched, tiles, pre, NT, W = schedule(lens, limit, bs, wg)
        seen = [[0] * t for t in tiles]
        slots = set()
        pieces_seen = {}
        for j, (S0, S1, ents, nid) in enumerate(sched):
            assert sum(e[2] for e in ents) == S1 - S0
            assert S1 - S0 <= g["tcap"] and len(ents) <= ENTRIES and nid <= IDS
            for (b, tt_lo, n, p0, pieces, side) in ents:
                assert n >= 1
                for tt in range(tt_lo, tt_lo + n):
                    seen[b][tt] += 1
                if pieces > 1:
                    assert (j, side) not in slots
                    slots.add((j, side))
                    # the merger recomputes this piece's slot from (b, k)
                    k = j - range_of(p0, NT, W)
                    jk = range_of(p0, NT, W) + k
                    side_m = 1 if (k == 0 and p0 > jk * NT // W) else 0
                    assert (jk, side_m) == (j, side)
                    pieces_seen.setdefault(b, []).append(j)
        assert all(c == 1 for row in seen for c in row)
        for b, js in pieces_seen.items():
            p0, t = pre[b], tiles[b]
            assert js == list(range(range_of(p0, NT, W), range_of(p0 + t - 1, NT, W) + 1))
