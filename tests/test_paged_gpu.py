"""GPU parity of the paged decode / verify kernel (engine.attention.paged_attention
-> cie_paged_fwd) against the CPU oracle (gather through the block table, then
the dense fp32 reference, exactly as the reference engine's Attention.forward
does), plus the engine.cache behaviour tests on the GPU."""

from __future__ import annotations

import pytest
import torch

from benchmarks import workloads
from engine.attention import flash_attention, paged_attention
from engine.cache import BlockTable, KVCacheConfig, PagedKVCache, block_table_tensor
from oracle import paged_attention_ref
from test_flash_gpu import TOL, assert_close

pytestmark = pytest.mark.gpu
DEV = "cuda"


def make_paged(lens, Lq, D, dtype, bs, Hq=8, Hk=2, seed=0, extra=5, vscale=1.0):
    g = torch.Generator().manual_seed(seed)
    B = len(lens)
    nblk = [-(-L // bs) for L in lens]
    nb = sum(nblk) + extra
    perm = torch.randperm(nb, generator=g)
    kp = torch.randn(nb, bs, Hk, D, generator=g).to(dtype)
    vp = (torch.randn(nb, bs, Hk, D, generator=g) * vscale).to(dtype)
    bt = torch.zeros(B, max(nblk + [1]), dtype=torch.int32)
    pos = 0
    for b in range(B):
        bt[b, :nblk[b]] = perm[pos:pos + nblk[b]].int()
        pos += nblk[b]
    q = torch.randn(B, Hq, Lq, D, generator=g).to(dtype)
    return q, kp, vp, bt, torch.tensor(lens, dtype=torch.int32)


def run(q, kp, vp, bt, lens, causal=True, **kw):
    return paged_attention(q.to(DEV), kp.to(DEV), vp.to(DEV), bt.to(DEV), lens.to(DEV), causal=causal, **kw)


def test_workload_decode_b32():
    c = workloads.decode_b32()
    out = run(c.q, c.k_pool, c.v_pool, c.block_tables, c.context_lens)
    ref = paged_attention_ref(c.q, c.k_pool, c.v_pool, c.block_tables, c.context_lens, causal=True)
    assert_close(out, ref, 2e-3, "decode_b32")


def test_workload_verify_b8():
    c = workloads.verify_b8()
    out = run(c.q, c.k_pool, c.v_pool, c.block_tables, c.context_lens)
    ref = paged_attention_ref(c.q, c.k_pool, c.v_pool, c.block_tables, c.context_lens, causal=True)
    assert_close(out, ref, 1e-2, "verify_b8")


@pytest.mark.parametrize("name,tol", [("decode_b32_d128", 2e-3), ("verify_b8_d128", 1e-2)])
def test_workloads_at_head_dim_128(name, tol):
    c = workloads.WORKLOADS[name]()
    out = run(c.q, c.k_pool, c.v_pool, c.block_tables, c.context_lens)
    ref = paged_attention_ref(c.q, c.k_pool, c.v_pool, c.block_tables, c.context_lens, causal=True)
    assert_close(out, ref, tol, name)


@pytest.mark.parametrize("bs", [1, 3, 8, 16, 32])
@pytest.mark.parametrize("D", [16, 64, 128, 256])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_sweep_block_size_head_dim(bs, D, dtype):
    lens = [1, 5, 37, 129, 300, 0, 2]
    for Lq, causal in ((1, True), (3, True), (2, False)):
        q, kp, vp, bt, ln = make_paged(lens, Lq, D, dtype, bs, seed=bs * 7 + D + Lq, vscale=0.5)
        out = run(q, kp, vp, bt, ln, causal=causal)
        ref = paged_attention_ref(q, kp, vp, bt, ln, causal=causal)
        assert_close(out, ref, TOL[dtype], f"bs={bs} D={D} {dtype} Lq={Lq} causal={causal}")


def test_context_shorter_than_new_tokens_and_empty():
    q, kp, vp, bt, ln = make_paged([0, 2, 6], 4, 64, torch.float16, 4, seed=3)
    out = run(q, kp, vp, bt, ln, causal=True)
    ref = paged_attention_ref(q, kp, vp, bt, ln, causal=True)
    assert (out[0] == 0).all()                       # no history -> zeros
    assert torch.isnan(out[1, :, :2].float()).all()  # rows with no visible key -> NaN
    assert_close(out, ref, 2e-3, "short contexts")


@pytest.mark.parametrize("Hq,Hk,Lq", [(32, 2, 3), (16, 1, 5), (8, 8, 1)])
def test_query_tiles_and_group_sizes(Hq, Hk, Lq):
    # group * Lq > 32 needs several query tiles per kv head
    q, kp, vp, bt, ln = make_paged([50, 333, 1000], Lq, 64, torch.float16, 16, Hq=Hq, Hk=Hk, seed=Hq + Lq)
    out = run(q, kp, vp, bt, ln, causal=True)
    ref = paged_attention_ref(q, kp, vp, bt, ln, causal=True)
    assert_close(out, ref, 2e-3, f"Hq={Hq} Hk={Hk} Lq={Lq}")


def test_long_contexts_split_and_max_context_hint():
    lens = [9000, 17, 4100, 8192]
    q, kp, vp, bt, ln = make_paged(lens, 2, 128, torch.bfloat16, 16, seed=21, vscale=0.5)
    ref = paged_attention_ref(q, kp, vp, bt, ln, causal=True)
    a = run(q, kp, vp, bt, ln)
    b = run(q, kp, vp, bt, ln, max_context=max(lens))
    assert_close(a, ref, 1e-2, "split, table bound")
    assert_close(b, ref, 1e-2, "split, max_context hint")


def test_wide_pool_offsets():
    """A pool view whose blocks lie 2^24 elements apart inside one larger
    allocation (block stride >= 2^24, element offsets past 2^31 for block ids
    >= 128): the launcher takes the 64-bit address path; the result equals
    the oracle over the same blocks, planned and unplanned."""
    from engine.attention import paged_plan

    nb, bs, Hk, D, Lq = 136, 16, 2, 64, 3
    lens = [1000, 700]
    q, kp, vp, bt, ln = make_paged(lens, Lq, D, torch.float16, bs, Hq=8, Hk=Hk, seed=77,
                                   extra=nb - sum(-(-c // bs) for c in lens), vscale=0.5)
    assert kp.shape[0] == nb
    # make sure the tables use blocks past 2^31 elements (ids >= 128)
    used = set(bt[0, :-(-lens[0] // bs)].tolist()) | set(bt[1, :-(-lens[1] // bs)].tolist())
    high = [i for i in range(128, nb) if i not in used]
    if not any(i >= 128 for i in used):
        bt[0, 0] = high[0]
    stride = 1 << 24
    views = []
    for pool in (kp, vp):
        big = torch.zeros(nb, stride, dtype=pool.dtype, device=DEV)
        view = big[:, :bs * Hk * D].view(nb, bs, Hk, D)
        view.copy_(pool.to(DEV))
        assert view.stride(0) == stride
        views.append(view)
    ref = paged_attention_ref(q, kp, vp, bt, ln, causal=True)
    args = (q.to(DEV), views[0], views[1], bt.to(DEV), ln.to(DEV))
    out = paged_attention(*args, causal=True).cpu()
    assert_close(out, ref, 2e-3, "wide offsets")
    pl = paged_plan(ln, bt, Hq=8, Hk=Hk, Lq=Lq, D=D, num_blocks=nb, block_size=bs, max_context=max(lens), device=DEV)
    planned = paged_attention(*args, causal=True, max_context=max(lens), plan=pl).cpu()
    assert torch.equal(planned, out)
    del views, args
    torch.cuda.empty_cache()


def test_context_beyond_hint_is_poisoned_not_truncated():
    lens = [3000, 100]
    q, kp, vp, bt, ln = make_paged(lens, 1, 64, torch.float16, 16, seed=22)
    out = run(q, kp, vp, bt, ln, max_context=600)
    ref = paged_attention_ref(q, kp, vp, bt, ln, causal=True)
    assert torch.isnan(out[0].float()).all()
    assert_close(out[1:], ref[1:], 2e-3, "other sequence unaffected")


def test_invalid_block_id_poisons_only_that_sequence():
    q, kp, vp, bt, ln = make_paged([40, 40], 1, 64, torch.float16, 16, seed=23)
    bt_bad = bt.clone()
    bt_bad[0, 1] = kp.shape[0] + 1000
    out = run(q, kp, vp, bt_bad, ln)
    ref = paged_attention_ref(q, kp, vp, bt, ln, causal=True)
    assert torch.isnan(out[0].float()).all()
    assert_close(out[1:], ref[1:], 2e-3, "valid sequence")


def test_block_relabelling_is_bitwise_invariant():
    q, kp, vp, bt, ln = make_paged([700, 45, 1290], 5, 64, torch.bfloat16, 16, seed=24, extra=11)
    base = run(q, kp, vp, bt, ln)
    relabel = torch.randperm(kp.shape[0], generator=torch.Generator().manual_seed(5))
    kp2, vp2 = torch.empty_like(kp), torch.empty_like(vp)
    kp2[relabel] = kp
    vp2[relabel] = vp
    out = run(q, kp2, vp2, relabel[bt.long()].int(), ln)
    assert torch.equal(out, base)


def test_decode_matches_last_prefill_row():
    # incremental decode == last row of the full causal prefill over the same keys
    L, Hq, Hk, D = 301, 8, 2, 64
    g = torch.Generator().manual_seed(25)
    q = torch.randn(1, Hq, L, D, generator=g).half()
    k = torch.randn(1, Hk, L, D, generator=g).half()
    v = torch.randn(1, Hk, L, D, generator=g).half()
    full = flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), causal=True)
    cache = PagedKVCache(KVCacheConfig(1, Hk, D, num_blocks=64, block_size=16, dtype=torch.float16, device=DEV))
    seq = cache.new_sequence()
    cache.append(0, seq, k[0].transpose(0, 1).to(DEV), v[0].transpose(0, 1).to(DEV))
    dec = cache.attend(0, q[:, :, -1:].to(DEV), [seq])
    ver = cache.attend(0, q[:, :, -5:].to(DEV), [seq])
    assert_close(dec, full[:, :, -1:].float(), 2e-3, "decode vs prefill last row")
    assert_close(ver, full[:, :, -5:].float(), 2e-3, "verify vs prefill last 5 rows")


def test_cache_attend_equals_gather_then_dense():
    Hq, Hk, D = 8, 2, 64
    cache = PagedKVCache(KVCacheConfig(2, Hk, D, num_blocks=40, block_size=8, dtype=torch.bfloat16, device=DEV))
    g = torch.Generator().manual_seed(26)
    seqs = []
    for L in (13, 70, 1):
        s = cache.new_sequence()
        for layer in range(2):
            cache.append(layer, s, torch.randn(L, Hk, D, generator=g).bfloat16().to(DEV),
                         torch.randn(L, Hk, D, generator=g).bfloat16().to(DEV), start=0)
        seqs.append(s)
    q = torch.randn(3, Hq, 1, D, generator=g).bfloat16().to(DEV)
    out = cache.attend(1, q, seqs)
    for b, s in enumerate(seqs):
        gk, gv = cache.gather(1, s)
        dense = flash_attention(q[b:b + 1], gk.transpose(0, 1).unsqueeze(0), gv.transpose(0, 1).unsqueeze(0),
                                causal=True)
        assert_close(out[b:b + 1], dense.float(), 1e-2, f"seq {b}")


# the reference's KV-cache behaviour tests (tests/cache/test_kv_cache.py) on the GPU

def _cache(num_blocks=8, block_size=4):
    return PagedKVCache(KVCacheConfig(2, 2, 16, num_blocks=num_blocks, block_size=block_size,
                                      dtype=torch.float16, device=DEV))


def test_gpu_append_gather_fork_rollback():
    cache = _cache()
    seq = cache.new_sequence()
    k = torch.randn(6, 2, 16, device=DEV, dtype=torch.float16)
    v = torch.randn(6, 2, 16, device=DEV, dtype=torch.float16)
    cache.append(0, seq, k, v)
    gk, gv = cache.gather(0, seq)
    assert torch.equal(gk, k) and torch.equal(gv, v)
    forked = cache.fork(seq)
    cache.append(0, seq, k[:1], v[:1])
    assert seq.length == 7 and forked.length == 6
    assert torch.equal(cache.gather(0, forked)[0], k)
    free_before = len(cache._free)
    cache.rollback(seq, 2)
    assert seq.length == 2 and len(cache._free) == free_before + 1


def test_block_table_tensor_on_device():
    bt, lens = block_table_tensor([BlockTable(4, [3, 1], 6)], DEV)
    assert bt.is_cuda and bt.dtype == torch.int32 and bt.tolist() == [[3, 1]] and lens.tolist() == [6]
