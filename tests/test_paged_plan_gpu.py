"""GPU parity of planned paged attention (a host-built work plan,
cie_paged_plan + cie_paged_fwd_ex) against the unplanned launch that derives
the same schedule on the device (cie_paged_fwd and its append / RoPE
variants): the same ranges, pieces and arithmetic, so outputs and pools must
be equal bit for bit; and against the oracle (the reference's gather then
dense attention, engine/model/block.py:56-71) within tolerance."""

from __future__ import annotations

import ctypes
import math

import pytest
import torch

from engine import _lib
from engine.attention import paged_attention, paged_plan
from oracle import paged_attention_ref
from test_flash_gpu import TOL, assert_close
from test_paged_gpu import make_paged

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _both(q, kp, vp, bt, lt, **kw):
    B, Hq, Lq, D = q.shape
    nb, bs, Hk, _ = kp.shape
    args = [t.to(DEV) for t in (q, kp, vp, bt, lt)]
    plain = paged_attention(*args, causal=True, **kw)
    pl = paged_plan(lt, bt, Hq=Hq, Hk=Hk, Lq=Lq, D=D, num_blocks=nb, block_size=bs,
                    max_context=kw.get("max_context"), device=DEV)
    planned = paged_attention(*args, causal=True, plan=pl, **kw)
    return plain.cpu(), planned.cpu(), pl


@pytest.mark.parametrize("name", ["decode_b32", "verify_b8", "decode_b32_d128", "verify_b8_d128"])
def test_workloads_planned_equal_unplanned(name):
    from benchmarks import workloads

    c = workloads.WORKLOADS[name]()
    plain, planned, pl = _both(c.q, c.k_pool, c.v_pool, c.block_tables, c.context_lens,
                               max_context=int(c.context_lens.max()))
    assert pl.split > 0
    assert torch.equal(planned, plain)
    ref = paged_attention_ref(c.q, c.k_pool, c.v_pool, c.block_tables, c.context_lens, causal=True)
    assert_close(planned, ref, TOL[c.q.dtype], name)


@pytest.mark.parametrize("B,Lq", [(3000, 1), (1200, 4)])
def test_many_short_sequences_planned_equal_unplanned(B, Lq):
    """Thousands of sequences of 1-40 tokens: a workgroup range then covers
    many sequences, up to the per-range cap of sequences the launch geometry
    keeps (more ranges than CUs when needed), most sequences end inside a
    range and a few are split -- against the oracle, planned and unplanned
    bit-identical."""
    g = torch.Generator().manual_seed(B + Lq)
    lens = (torch.randint(Lq, 41, (B,), generator=g)).tolist()
    q, kp, vp, bt, lt = make_paged(lens, Lq, 64, torch.float16, 16, Hq=8, Hk=2, seed=B, vscale=0.5)
    plain, planned, _ = _both(q, kp, vp, bt, lt)
    assert torch.equal(planned, plain)
    ref = paged_attention_ref(q, kp, vp, bt, lt, causal=True)
    assert_close(planned, ref, TOL[torch.float16], f"B={B} Lq={Lq}")


@pytest.mark.parametrize("Lq,bs,D,dtype", [(1, 16, 64, torch.float16), (5, 3, 128, torch.bfloat16),
                                           (3, 16, 16, torch.float16), (2, 7, 256, torch.bfloat16),
                                           (1, 1, 32, torch.float16)])
def test_ragged_and_invalid_planned_equal_unplanned(Lq, bs, D, dtype):
    # empty history, lengths below / around tile and block boundaries, an invalid
    # length (longer than the table allows) and an invalid block id
    lens = [0, Lq, 31 + Lq, 33, 700, 2049, 95, 1024 + Lq, 5000]
    q, kp, vp, bt, lt = make_paged(lens[:-1] + [64], Lq, D, dtype, bs, Hq=8, Hk=2, seed=D + bs, vscale=0.5)
    lt[-1] = 5000  # beyond max_blocks * block_size of its row
    bt[4, 2] = kp.shape[0] + 7
    plain, planned, _ = _both(q, kp, vp, bt, lt)
    assert torch.equal(torch.isnan(planned), torch.isnan(plain))
    assert torch.equal(planned.nan_to_num(7.0), plain.nan_to_num(7.0))
    assert torch.isnan(planned[4]).all() and torch.isnan(planned[8]).all()
    assert (planned[0] == 0).all()


def test_plan_without_split_skips_the_merge():
    lens = [32] * 48 + [7]  # one tile per sequence
    q, kp, vp, bt, lt = make_paged(lens, 1, 64, torch.float16, 16, Hq=32, Hk=8, seed=3)
    plain, planned, pl = _both(q, kp, vp, bt, lt)
    assert pl.split == 0
    assert torch.equal(planned, plain)


@pytest.mark.parametrize("rope", [False, True])
@pytest.mark.parametrize("Lq,dtype", [(1, torch.float16), (5, torch.bfloat16)])
def test_planned_fused_append_equals_unplanned(Lq, dtype, rope):
    from engine.model.rope import RotaryEmbedding

    lens = [Lq, 40 + Lq, 700, 2049, 4096, 33]
    q, kp, vp, bt, lt = make_paged(lens, Lq, 64, dtype, 16, Hq=8, Hk=2, seed=Lq, vscale=0.5)
    g = torch.Generator().manual_seed(9)
    kn = torch.randn(len(lens) * Lq, 2, 64, generator=g).to(dtype)
    vn = (torch.randn(len(lens) * Lq, 2, 64, generator=g) * 0.5).to(dtype)
    kw = {"rope": RotaryEmbedding(64, 8192).to(DEV).tables} if rope else {}
    outs, pools = [], []
    for planned in (False, True):
        kd, vd = kp.to(DEV), vp.to(DEV)
        pl = paged_plan(lt, bt, Hq=8, Hk=2, Lq=Lq, D=64, num_blocks=kp.shape[0], block_size=16,
                        for_append=True, device=DEV) if planned else None
        o = paged_attention(q.to(DEV), kd, vd, bt.to(DEV), lt.to(DEV), causal=True,
                            new_kv=(kn.to(DEV), vn.to(DEV)), plan=pl, **kw)
        outs.append(o.cpu())
        pools.append((kd.cpu(), vd.cpu()))
    assert torch.equal(outs[0], outs[1])
    assert torch.equal(pools[0][0], pools[1][0]) and torch.equal(pools[0][1], pools[1][1])


def _launch_ex(lib, args, o, plan, split, *, Hq, Hk, Lq, D, nb, bs, mb, max_context):
    """cie_paged_fwd_ex straight through the C ABI (no Python key check)."""
    st = [_lib.strides(t) for t in (args[0], args[1], args[2], o)]
    none3 = (ctypes.c_int64 * 3)(0, 0, 1)
    ws = torch.empty(16 << 20, dtype=torch.uint8, device=DEV)
    rc = lib.cie_paged_fwd_ex(args[0].data_ptr(), None, None, args[1].data_ptr(), args[2].data_ptr(), None, None,
                              plan.data_ptr(), plan.numel() * plan.element_size(), split, o.data_ptr(),
                              ws.data_ptr(), ws.numel(),
                              st[0], none3, none3, st[1], st[2], st[3], args[0].shape[0], Hq, Hk, Lq, D, nb, bs,
                              mb, max_context, ctypes.c_float(1.0 / math.sqrt(D)), 1, 0, None, None, 0, 0,
                              _lib.stream_handle(torch.device(DEV)))
    _lib.check(rc)
    torch.cuda.synchronize()


# one argument of the plan builder changed per case: (field, builder overrides, plan_split offset)
_MISMATCHES = [
    ("append", dict(for_append=True), 0),
    ("B", dict(rows=1), 0),
    ("Hq", dict(Hq=4), 0),
    ("Lq", dict(Lq=2), 0),
    ("head_dim", dict(D=32), 0),
    ("num_blocks", dict(num_blocks_add=7), 0),
    ("block_size", dict(block_size=8), 0),
    ("max_blocks", dict(extra_col=True), 0),
    ("max_context", dict(max_context=301), 0),
    ("head groups", dict(Hq=8, Hk=8), 0),
    ("split count", dict(), 1),
]


@pytest.mark.parametrize("field,over,dsplit", _MISMATCHES, ids=[m[0] for m in _MISMATCHES])
def test_plan_for_other_arguments_gives_nan(field, over, dsplit):
    """Through the C ABI a plan is checked against the launch on the device
    (its header): a plan built with any one argument different from the
    launch's, or passed with another split count, is read no further and
    every output row is NaN (the Python layer refuses such a plan by its key
    before that)."""
    Hq, Hk, Lq, D, bs = 8, 2, 1, 64, 16
    q, kp, vp, bt, lt = make_paged([40, 300], Lq, D, torch.float16, bs, Hq=Hq, Hk=Hk, seed=5)
    nb, mb = kp.shape[0], bt.shape[1]
    args = [t.to(DEV) for t in (q, kp, vp, bt, lt)]
    lib = _lib.load()
    # the matching plan: the same result as the unplanned launch
    good = paged_plan(lt, bt, Hq=Hq, Hk=Hk, Lq=Lq, D=D, num_blocks=nb, block_size=bs, device=DEV)
    assert good.split > 0  # the 300-token sequence is split, so the merge pass runs
    o = torch.zeros_like(args[0])
    _launch_ex(lib, args, o, good.data, good.split, Hq=Hq, Hk=Hk, Lq=Lq, D=D, nb=nb, bs=bs, mb=mb, max_context=0)
    assert torch.equal(o, paged_attention(*args, causal=True))
    with pytest.raises(ValueError):  # the Python layer checks the key
        paged_attention(*args, plan=paged_plan(lt, bt, Hq=Hq, Hk=Hk, Lq=Lq, D=D, num_blocks=nb, block_size=bs,
                                               for_append=True, device=DEV))
    rows = over.get("rows", 2)
    btp = bt[:rows]
    if over.get("extra_col"):
        btp = torch.cat([btp, torch.zeros(rows, 1, dtype=torch.int32)], dim=1)
    bad = paged_plan(lt[:rows], btp, Hq=over.get("Hq", Hq), Hk=over.get("Hk", Hk), Lq=over.get("Lq", Lq),
                     D=over.get("D", D), num_blocks=nb + over.get("num_blocks_add", 0),
                     block_size=over.get("block_size", bs), max_context=over.get("max_context"),
                     for_append=over.get("for_append", False), device=DEV)
    # a buffer smaller than this launch's plan is refused before any launch;
    # padded to that size (zeros past the plan) it reaches the header check
    need = lib.cie_paged_plan_bytes(q.shape[0], Hq, Hk, Lq, D, 0, bs, mb)
    data = bad.data
    if data.numel() * 4 < need:
        o = torch.zeros_like(args[0])
        with pytest.raises(ValueError, match="plan"):
            _launch_ex(lib, args, o, data, bad.split + dsplit, Hq=Hq, Hk=Hk, Lq=Lq, D=D, nb=nb, bs=bs, mb=mb,
                       max_context=0)
        assert not o.any()
        data = torch.zeros(need // 4, dtype=torch.int32, device=DEV)
        data[:bad.data.numel()] = bad.data
    o = torch.zeros_like(args[0])
    _launch_ex(lib, args, o, data, bad.split + dsplit, Hq=Hq, Hk=Hk, Lq=Lq, D=D, nb=nb, bs=bs, mb=mb,
               max_context=0)
    assert torch.isnan(o).all(), field


def test_plan_buffer_smaller_than_the_launch_is_refused():
    """plan_bytes below cie_paged_plan_bytes for the call's arguments:
    CIE_EINVAL before any launch, the output untouched."""
    Hq, Hk, Lq, D, bs = 8, 2, 1, 64, 16
    q, kp, vp, bt, lt = make_paged([40, 300], Lq, D, torch.float16, bs, Hq=Hq, Hk=Hk, seed=5)
    nb, mb = kp.shape[0], bt.shape[1]
    args = [t.to(DEV) for t in (q, kp, vp, bt, lt)]
    lib = _lib.load()
    good = paged_plan(lt, bt, Hq=Hq, Hk=Hk, Lq=Lq, D=D, num_blocks=nb, block_size=bs, device=DEV)
    assert good.data.numel() * 4 == lib.cie_paged_plan_bytes(2, Hq, Hk, Lq, D, 0, bs, mb)
    o = torch.zeros_like(args[0])
    with pytest.raises(ValueError, match="plan"):
        _launch_ex(lib, args, o, good.data[:-1], good.split, Hq=Hq, Hk=Hk, Lq=Lq, D=D, nb=nb, bs=bs, mb=mb,
                   max_context=0)
    assert not o.any()


def test_attention_section_with_step_plan_equals_without():
    """A decode step and a verify step through attention_section, with the
    plan built by prepare_step(num_heads=...) and without it."""
    from engine.cache import KVCacheConfig, PagedKVCache
    from engine.model import attention_section

    for L, dtype in ((1, torch.float16), (4, torch.bfloat16)):
        B, Hq, Hk, D = 5, 8, 2, 64
        outs = []
        for use_plan in (False, True):
            cache = PagedKVCache(KVCacheConfig(1, Hk, D, 400, 16, dtype, DEV))
            g = torch.Generator().manual_seed(L)
            tables = [cache.new_sequence() for _ in range(B)]
            for t, n in zip(tables, [50, 0, 300, 1000, 17]):
                if n:
                    cache.append(0, t, torch.randn(n, Hk, D, generator=g).to(dtype).to(DEV),
                                 torch.randn(n, Hk, D, generator=g).to(dtype).to(DEV))
            q = torch.randn(B, Hq, L, D, generator=g).to(dtype).to(DEV)
            k = torch.randn(B, Hk, L, D, generator=g).to(dtype).to(DEV)
            v = torch.randn(B, Hk, L, D, generator=g).to(dtype).to(DEV)
            step = cache.prepare_step(tables, L, num_heads=Hq if use_plan else None)
            assert (step.plan is not None) == use_plan
            outs.append((attention_section(q, k, v, 0, cache, step).cpu(), cache.k[0].cpu(), cache.v[0].cpu()))
        for a, b in zip(outs[0], outs[1]):
            assert torch.equal(a, b)


@pytest.mark.parametrize("name", ["decode_b32", "verify_b8"])
def test_workloads_are_bit_identical_run_to_run(name):
    """The split sequences' pieces are fixed by the schedule and merged in
    piece order by a fixed butterfly, so repeated launches (planned and
    unplanned, into fresh outputs, with other launches between them) give
    the same bits."""
    from benchmarks import workloads

    c = workloads.WORKLOADS[name]()
    B, Hq, Lq, D = c.q.shape
    nb, bs, Hk, _ = c.k_pool.shape
    mc = int(c.context_lens.max())
    args = [t.to(DEV) for t in (c.q, c.k_pool, c.v_pool, c.block_tables, c.context_lens)]
    pl = paged_plan(c.context_lens, c.block_tables, Hq=Hq, Hk=Hk, Lq=Lq, D=D, num_blocks=nb, block_size=bs,
                    max_context=mc, device=DEV)
    first = paged_attention(*args, causal=True, plan=pl, max_context=mc)
    for _ in range(3):
        other = torch.randn(B, Hq, Lq, D, device=DEV).to(c.q.dtype)  # a different launch in between
        paged_attention(other, *args[1:], causal=True, max_context=mc)
        assert torch.equal(paged_attention(*args, causal=True, plan=pl, max_context=mc), first)
        assert torch.equal(paged_attention(*args, causal=True, max_context=mc), first)
