"""The host-built paged attention plan (cie_paged_plan) on the CPU.

The plan must hold exactly the schedule paged_fwd_kernel derives on the
device from the context lengths (ranges of the concatenated 32-token tiles,
the sequences and block ids of every range, the piece descriptors of the
merge pass), so that planned and unplanned launches compute the same thing.
This file restates that schedule in Python, independently of the C builder,
and checks the plan against it and against its invariants: every tile of
every valid sequence in exactly one range, ranges of equal size within one
tile, block ids validated like the device path validates them."""

from __future__ import annotations

import pytest
import torch

from engine import _lib
from engine.attention import device_cus, paged_plan_fill, paged_plan_ints

TILE = 32


def _xcds():
    """XCDs of the device the plan is sized for: 32 active CUs per gfx950
    XCD, at most 8, a power of two."""
    n = min(max(device_cus() // 32, 1), 8)
    return 1 << (n.bit_length() - 1)


def _geometry(Hq, Hk, Lq, D):
    """Head grouping of the launch: the largest divisor Hg of Hk with
    Hg * D <= 256 and Hg * query tiles <= 8 waves (4 at D = 256); NG = Hk / Hg groups."""
    R = (Hq // Hk) * Lq
    n_qt = -(-R // 32)
    maxw = 4 if D == 256 else 8
    Hg = max(h for h in range(1, Hk + 1) if Hk % h == 0 and h * D <= 256 and h * n_qt <= maxw)
    return Hk // Hg


def _restated(lens, bt, num_blocks, bs, ctx_limit, Lq, append, Wg):
    """The device schedule of paged_fwd_kernel, restated."""
    B = len(lens)
    valid = [(c >= (Lq if append else 0)) and c <= ctx_limit and (c == 0 or num_blocks > 0) for c in lens]
    tiles = [-(-c // TILE) if v else 0 for c, v in zip(lens, valid)]
    NT = sum(tiles)
    W = min(Wg, NT)
    pre = [sum(tiles[:b]) for b in range(B)]
    rng = lambda x: ((x + 1) * W - 1) // NT  # noqa: E731  range index of tile x
    ranges = []
    for j in range(W):
        S0, S1 = j * NT // W, (j + 1) * NT // W
        ents, ids = [], []
        for b in range(B):
            t = tiles[b]
            if t == 0 or pre[b] >= S1 or pre[b] + t <= S0:
                continue
            tt_lo, tt_hi = max(S0 - pre[b], 0), min(S1 - pre[b], t)
            blk_lo, blk_hi = TILE * tt_lo // bs, (min(lens[b], TILE * tt_hi) - 1) // bs
            ents.append((b, lens[b], tt_lo, tt_hi - tt_lo, len(ids), blk_lo, pre[b],
                         rng(pre[b] + t - 1) - rng(pre[b]) + 1))
            ids += [x if 0 <= x < num_blocks else -1 for x in bt[b][blk_lo:blk_hi + 1]]
        ranges.append((S0, S1 - S0, ents, ids))
    info = {}
    for b in range(B):
        if tiles[b]:
            j0 = rng(pre[b])
            # piece 0 takes slot side 1 when the sequence starts inside its first range
            info[b] = (j0, rng(pre[b] + tiles[b] - 1) - j0 + 1, 1 if pre[b] > j0 * NT // W else 0)
        else:
            info[b] = (0, 0, 0)
    empty = [(b, 1 if valid[b] else 0) for b in range(B) if tiles[b] == 0]
    split = sum(1 for b in range(B) if info[b][1] > 1)
    return W, NT, ranges, info, empty, split


def _build(lens, bt, Hq, Hk, Lq, D, num_blocks, bs, max_context=None, append=False):
    B, mb = bt.shape
    n = paged_plan_ints(B, Hq, Hk, Lq, D, bs, mb, max_context)
    assert n > 0
    out = torch.full((n,), 12345, dtype=torch.int32)
    split, key = paged_plan_fill(out, torch.tensor(lens, dtype=torch.int32), bt, Hq=Hq, Hk=Hk, Lq=Lq, D=D,
                                 num_blocks=num_blocks, block_size=bs, max_context=max_context, for_append=append)
    return out, split, key


def _check(lens, bt, Hq, Hk, Lq, D, num_blocks, bs, max_context=None, append=False):
    P, split, key = _build(lens, bt, Hq, Hk, Lq, D, num_blocks, bs, max_context, append)
    B, mb = bt.shape
    ctx_limit = min(max_context, mb * bs) if max_context else mb * bs
    Wg = int(P[3])
    NG = _geometry(Hq, Hk, Lq, D)
    W, NT, ranges, info, empty, split_ref = _restated(lens, bt.tolist(), num_blocks, bs, ctx_limit, Lq, append, Wg)
    assert int(P[0]) == 0x43504C33 and int(P[1]) == W and int(P[2]) == NT and int(P[6]) == B
    assert int(P[7]) == (1 if append else 0)
    assert split == split_ref == int(P[5])
    # the rest of the header: every argument the layout and the validated ids
    # depend on, compared by the launch (NG, Lq, D, num_blocks, block_size,
    # max_blocks, the context bound, Hq)
    assert P[8:16].tolist() == [NG, Lq, D, num_blocks, bs, mb, ctx_limit, Hq]
    off_r = 16
    off_e = off_r + 8 * Wg
    off_i = off_e + 8 * (Wg + B)
    off_f = (off_i + B * mb + 2 * Wg + 3) // 4 * 4
    off_z = off_f + 4 * NG * B
    covered = {}
    for j in range(Wg):
        row = P[off_r + 8 * j: off_r + 8 * j + 8].tolist()
        if j >= W:
            assert row[1] == 0 and row[5] == 0
            continue
        S0, T, ents, ids = ranges[j]
        assert (row[4], row[5], row[1], row[3]) == (S0, T, len(ents), len(ids)), j
        got = [tuple(P[off_e + 8 * (row[0] + e): off_e + 8 * (row[0] + e) + 8].tolist()) for e in range(row[1])]
        assert got == ents, j
        assert P[off_i + row[2]: off_i + row[2] + row[3]].tolist() == ids, j
        for b, ctx, tt_lo, n, *_ in got:
            for t in range(tt_lo, tt_lo + n):
                covered[(b, t)] = covered.get((b, t), 0) + 1
    # every tile of every sequence with tiles lies in exactly one range, ranges within one tile of each other
    for (b, t), c in covered.items():
        assert c == 1, (b, t)
    assert sum(1 for _ in covered) == NT
    sizes = [ranges[j][1] for j in range(W)]
    assert not sizes or max(sizes) - min(sizes) <= 1
    for gh in range(NG):
        for b in range(B):
            f = P[off_f + 4 * (gh * B + b): off_f + 4 * (gh * B + b) + 3].tolist()
            assert tuple(f) == info[b], (gh, b, f, info[b])
    n_empty = int(P[4])
    assert [tuple(P[off_z + 2 * z: off_z + 2 * z + 2].tolist()) for z in range(n_empty)] == empty
    # merge table: 8 lists of cap_t entries (those of XCDs the device does not
    # have stay empty); every split sequence of every head group exactly
    # once, each list at most merge_cap(split * NG) long, each sequence on the
    # XCD that ran its middle piece unless that list was full
    nx = _xcds()
    off_m = (off_z + 2 * B + 3) // 4 * 4
    cap_t = (B * NG + nx - 1) // nx + 1
    cap = (split * NG + nx - 1) // nx + 1
    assert P.numel() == off_m + 4 * 8 * cap_t
    n_wg = NG * Wg
    base, extra = n_wg // nx, n_wg % nx

    def xcd_of(logical):  # the main pass's XCD of range j of head group gh (logical = gh Wg + j)
        return next(x for x in range(nx) if logical < (x + 1) * base + min(x + 1, extra)) if logical < n_wg else nx - 1

    placed, fallbacks = {}, 0
    for x in range(8):
        ent = P[off_m + 4 * x * cap_t: off_m + 4 * (x + 1) * cap_t].reshape(cap_t, 4).tolist()
        lst = [e[0] for e in ent]
        used = [u for u in lst if u >= 0]
        assert lst == used + [-1] * (cap_t - len(used)) and len(used) <= cap, (x, lst)
        assert x < nx or not used
        for u, e in zip(used, ent):
            assert u not in placed, u
            placed[u] = x
            # each entry carries its sequence's piece descriptor (the info rows)
            assert tuple(e[1:]) == info[u // NG], (x, e, info[u // NG])
        assert all(e == [-1, 0, 0, 0] for e in ent[len(used):]), (x, ent)
    # (only launches of one workgroup per CU or fewer place ranges in XCD runs
    # and fill the table; the others merge in grid order)
    runs = NG * Wg <= device_cus()
    want = {b * NG + gh for b in range(B) for gh in range(NG) if info[b][1] > 1} if runs else set()
    assert set(placed) == want
    for u, x in placed.items():
        b, gh = u // NG, u % NG
        j0, pieces, _ = info[b]
        fallbacks += xcd_of(gh * Wg + j0 + pieces // 2) != x
    assert fallbacks <= len(want) // 2, fallbacks  # most sequences land where their pieces are
    return P, split


def _tables(lens, bs, seed, extra=3):
    g = torch.Generator().manual_seed(seed)
    need = [-(-c // bs) for c in lens]
    nb = sum(need) + extra
    perm = torch.randperm(nb, generator=g)
    bt = torch.zeros(len(lens), max(need + [1]), dtype=torch.int32)
    p = 0
    for b, n in enumerate(need):
        bt[b, :n] = perm[p:p + n].int()
        p += n
    return bt, nb


@pytest.mark.parametrize("seed", range(6))
def test_plan_matches_restated_schedule_random(seed):
    g = torch.Generator().manual_seed(100 + seed)
    B = int(torch.randint(1, 70, (1,), generator=g))
    lens = torch.randint(0, 3000, (B,), generator=g).tolist()
    bs = [16, 3, 32, 7, 16, 1][seed]
    bt, nb = _tables(lens, bs, seed)
    Hq, Hk, Lq, D = [(32, 8, 1, 64), (8, 2, 5, 128), (16, 4, 3, 16), (4, 4, 1, 256), (32, 8, 5, 64), (8, 1, 2, 32)][seed]
    _check(lens, bt, Hq, Hk, Lq, D, nb, bs)


def test_plan_workload_shapes():
    from benchmarks import workloads

    for name in ("decode_b32", "verify_b8"):
        c = workloads.WORKLOADS[name]()
        B, Hq, Lq, D = c.q.shape
        nb, bs, Hk, _ = c.k_pool.shape
        P, split = _check(c.context_lens.tolist(), c.block_tables, Hq, Hk, Lq, D, nb, bs,
                          int(c.context_lens.max()))
        assert split > 0  # these shapes split sequences across workgroups


def test_plan_invalid_lengths_and_ids_and_append_validity():
    lens = [40, 0, 10_000, 33, 2, 17]  # an empty history, one longer than the table allows
    bt, nb = _tables([40, 0, 16, 33, 2, 17], 16, seed=3)
    bt[3, 1] = nb + 5  # an id outside the pool
    bt[0, 0] = -2
    P, _ = _check(lens, bt, 8, 2, 1, 64, nb, 16)
    # for the fused append, a context shorter than its Lq new tokens is invalid too
    _check([40, 0, 3, 33, 2, 17], bt, 8, 2, 5, 64, nb, 16, append=True)


def test_plan_without_split_sequences():
    lens = [32] * 40 + [5, 0]  # one tile each: no range holds part of a sequence
    bt, nb = _tables(lens, 16, seed=4)
    P, split = _check(lens, bt, 8, 2, 1, 64, nb, 16)
    assert split == 0


def test_plan_argument_errors():
    lib = _lib.load()
    bt = torch.zeros(2, 4, dtype=torch.int32)
    lens = torch.tensor([10, 20], dtype=torch.int32)
    n = paged_plan_ints(2, 8, 2, 1, 64, 16, 4)
    out = torch.zeros(n, dtype=torch.int32)
    # too small a buffer, a row stride below the table width, an unsupported shape
    assert lib.cie_paged_plan(out.data_ptr(), 16, lens.data_ptr(), bt.data_ptr(), 4, 2, 8, 2, 1, 64, 10, 16, 4,
                              0, 0) == _lib.CIE_EWORKSPACE
    assert lib.cie_paged_plan(out.data_ptr(), n * 4, lens.data_ptr(), bt.data_ptr(), 2, 2, 8, 2, 1, 64, 10, 16, 4,
                              0, 0) == _lib.CIE_EINVAL
    assert lib.cie_paged_plan(out.data_ptr(), n * 4, lens.data_ptr(), bt.data_ptr(), 4, 2, 8, 3, 1, 64, 10, 16, 4,
                              0, 0) == _lib.CIE_EINVAL
    assert paged_plan_ints(2, 8, 2, 65 * 4, 64, 16, 4) == 0  # more than 256 query rows per kv head
    assert paged_plan_ints(2, 8, 2, 33, 256, 16, 4) == 0  # more than 128 at head_dim 256
