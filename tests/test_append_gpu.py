"""GPU parity of the paged KV append (engine.cache.kv_append / PagedKVCache.append
-> cie_kv_append) against the oracle's restatement of the reference's append
loop (engine/cache/kv_cache.py:128-136). The bar is bit-exactness of both
pools: append moves bytes and computes nothing."""

from __future__ import annotations

import pytest
import torch

from engine.cache import BlockTable, KVCacheConfig, PagedKVCache, kv_append
from oracle import append_ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _pool(nb, bs, Hk, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    kp = torch.randn(nb, bs, Hk, D, generator=g).to(dtype)
    vp = torch.randn(nb, bs, Hk, D, generator=g).to(dtype)
    return kp, vp


def _batch(lens, starts, bs, Hk, D, dtype, seed, extra=4):
    """Random disjoint block tables covering [start, start + len) per sequence."""
    g = torch.Generator().manual_seed(seed)
    need = [-(-(s + n) // bs) for s, n in zip(starts, lens)]
    nb = sum(need) + extra
    perm = torch.randperm(nb, generator=g).tolist()
    tables, pos = [], 0
    for n in need:
        tables.append(perm[pos:pos + n])
        pos += n
    width = max(need + [1])
    bt = torch.full((len(lens), width), -7, dtype=torch.int32)  # padding never read
    for b, ids in enumerate(tables):
        bt[b, :len(ids)] = torch.tensor(ids, dtype=torch.int32)
    T = sum(lens)
    k = torch.randn(T, Hk, D, generator=g).to(dtype)
    v = torch.randn(T, Hk, D, generator=g).to(dtype)
    return nb, tables, bt, k, v


def _expected(kp, vp, tables, starts, lens, k, v):
    ek, ev = kp.clone(), vp.clone()
    row = 0
    for ids, s0, n in zip(tables, starts, lens):
        append_ref(ek, ev, ids, s0, k[row:row + n], v[row:row + n])
        row += n
    return ek, ev


def _run(kp, vp, bt, k, v, lens, starts, status=None):
    kd, vd = kp.to(DEV), vp.to(DEV)
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32, device=DEV)
    kv_append(k.to(DEV), v.to(DEV), kd, vd, bt.to(DEV), cu, torch.tensor(starts, dtype=torch.int32, device=DEV),
              max_new=max(lens + [0]), status=status)
    return kd.cpu(), vd.cpu()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bs,Hk,D", [(16, 8, 64), (1, 2, 16), (32, 4, 128), (8, 1, 256), (3, 8, 32)])
def test_batched_append_is_bit_exact(dtype, bs, Hk, D):
    lens = [1, 37, 0, 5, 64, 16]
    starts = [0, 3, 9, 15, 1, 16]
    nb, tables, bt, k, v = _batch(lens, starts, bs, Hk, D, dtype, seed=bs + D)
    kp, vp = _pool(nb, bs, Hk, D, dtype, seed=1)
    ek, ev = _expected(kp, vp, tables, starts, lens, k, v)
    gk, gv = _run(kp, vp, bt, k, v, lens, starts)
    assert torch.equal(gk, ek) and torch.equal(gv, ev)


def test_workload_sized_prefill_and_decode_appends():
    # prefill: 4 sequences x 2048 tokens; decode: 32 sequences x 1 token at ragged ends
    for lens, starts in (([2048] * 4, [0] * 4), ([1] * 32, [(97 * b) % 4096 for b in range(32)])):
        nb, tables, bt, k, v = _batch(lens, starts, 16, 8, 64, torch.float16, seed=len(lens))
        kp, vp = _pool(nb, 16, 8, 64, torch.float16, seed=2)
        ek, ev = _expected(kp, vp, tables, starts, lens, k, v)
        gk, gv = _run(kp, vp, bt, k, v, lens, starts)
        assert torch.equal(gk, ek) and torch.equal(gv, ev)


def test_strided_sources_and_pool_views():
    lens, starts = [20, 7], [5, 0]
    nb, tables, bt, k, v = _batch(lens, starts, 16, 4, 64, torch.float16, seed=5)
    kp, vp = _pool(nb, 16, 4, 64, torch.float16, seed=3)
    ek, ev = _expected(kp, vp, tables, starts, lens, k, v)
    # k, v as views of a wider (T, 2 * Hk, D) buffer; pools as views with padded heads
    kw = torch.zeros(k.shape[0], 8, 64, dtype=k.dtype)
    kw[:, ::2] = k
    big_k = torch.zeros(nb, 16, 6, 64, dtype=kp.dtype, device=DEV)
    big_v = torch.zeros(nb, 16, 6, 64, dtype=vp.dtype, device=DEV)
    big_k[:, :, :4] = kp.to(DEV)
    big_v[:, :, :4] = vp.to(DEV)
    cu = torch.tensor([0, 20, 27], dtype=torch.int32, device=DEV)
    kv_append(kw.to(DEV)[:, ::2], v.to(DEV), big_k[:, :, :4], big_v[:, :, :4], bt.to(DEV), cu,
              torch.tensor(starts, dtype=torch.int32, device=DEV), max_new=20)
    assert torch.equal(big_k[:, :, :4].cpu(), ek) and torch.equal(big_v[:, :, :4].cpu(), ev)
    assert (big_k[:, :, 4:] == 0).all() and (big_v[:, :, 4:] == 0).all()


def test_out_of_range_ids_and_positions_are_skipped_and_reported():
    lens, starts = [6, 6, 6], [0, 0, 0]
    nb, tables, bt, k, v = _batch(lens, starts, 4, 2, 16, torch.float16, seed=9)
    kp, vp = _pool(nb, 4, 2, 16, torch.float16, seed=4)
    bad = bt.clone()
    bad[1, 1] = nb + 100  # second block of sequence 1 is out of range
    status = torch.zeros(1, dtype=torch.int32, device=DEV)
    gk, gv = _run(kp, vp, bad, k, v, lens, starts, status=status)
    assert int(status.item()) == 1
    # sequences 0 and 2 written; sequence 1 written only in its valid first block
    ek, ev = _expected(kp, vp, [tables[0], tables[2]], [0, 0], [6, 6],
                       torch.cat([k[:6], k[12:]]), torch.cat([v[:6], v[12:]]))
    append_ref(ek, ev, tables[1][:1], 0, k[6:10], v[6:10])
    assert torch.equal(gk, ek) and torch.equal(gv, ev)
    # a clean launch leaves the status word alone
    status.zero_()
    _run(kp, vp, bt, k, v, lens, starts, status=status)
    assert int(status.item()) == 0


def test_cache_append_matches_reference_semantics():
    cfg = KVCacheConfig(num_layers=2, num_kv_heads=4, head_dim=64, num_blocks=40, block_size=16,
                        dtype=torch.bfloat16, device=DEV)
    cache = PagedKVCache(cfg)
    ref_k = [torch.zeros(40, 16, 4, 64, dtype=torch.bfloat16) for _ in range(2)]
    ref_v = [torch.zeros(40, 16, 4, 64, dtype=torch.bfloat16) for _ in range(2)]
    g = torch.Generator().manual_seed(12)
    t = cache.new_sequence()
    for L, start in ((37, None), (1, None), (5, 20), (16, None)):
        k = torch.randn(L, 4, 64, generator=g).to(torch.bfloat16)
        v = torch.randn(L, 4, 64, generator=g).to(torch.bfloat16)
        s0 = t.length if start is None else start
        cache.append(1, t, k.to(DEV), v.to(DEV), start=start)
        append_ref(ref_k[1], ref_v[1], t.blocks, s0, k, v)
        assert t.length == max(s0 + L, t.length)
    assert torch.equal(cache.k[1].cpu(), ref_k[1]) and torch.equal(cache.v[1].cpu(), ref_v[1])
    assert (cache.k[0] == 0).all()


def test_append_batch_then_paged_attention_equals_gather_path():
    from engine.attention import flash_attention

    cfg = KVCacheConfig(num_layers=1, num_kv_heads=2, head_dim=64, num_blocks=64, block_size=16,
                        dtype=torch.float16, device=DEV)
    cache = PagedKVCache(cfg)
    g = torch.Generator().manual_seed(13)
    tables = [cache.new_sequence() for _ in range(3)]
    lens = [70, 5, 33]
    k = torch.randn(sum(lens), 2, 64, generator=g).half().to(DEV)
    v = torch.randn(sum(lens), 2, 64, generator=g).half().to(DEV)
    cache.append_batch(0, tables, k, v, lens)
    q = torch.randn(3, 8, 1, 64, generator=g).half().to(DEV)
    out = cache.attend(0, q, tables)
    for b, t in enumerate(tables):
        kd, vd = cache.gather(0, t)
        ref = flash_attention(q[b:b + 1], kd.transpose(0, 1).unsqueeze(0).contiguous(),
                              vd.transpose(0, 1).unsqueeze(0).contiguous(), causal=True)
        assert (out[b:b + 1].float() - ref.float()).abs().max().item() <= 2e-3
        row = sum(lens[:b])
        assert torch.equal(kd, k[row:row + lens[b]]) and torch.equal(vd, v[row:row + lens[b]])


@pytest.mark.parametrize("L,dtype", [(1, torch.float16), (5, torch.bfloat16)])
def test_attention_section_matches_reference_per_sequence_path(L, dtype):
    """engine.model.attention_section (batched, paged) against the reference's
    per-sequence sequence of block.py:56-75 on the oracle: append_ref, then
    gather_ref of the whole history, then flash_attention_ref with causal=True
    and scale 1/sqrt(D), transposed to (L, Hq * D)."""
    import math

    from engine.model import attention_section
    from oracle import flash_attention_ref, gather_ref

    B, Hq, Hk, D, bs = 4, 8, 2, 64, 16
    cfg = KVCacheConfig(num_layers=2, num_kv_heads=Hk, head_dim=D, num_blocks=80, block_size=bs,
                        dtype=dtype, device=DEV)
    cache = PagedKVCache(cfg)
    g = torch.Generator().manual_seed(40 + L)
    tables = [cache.new_sequence() for _ in range(B)]
    hist = [37, 0, 100, 16]
    # existing history (layer 1), written through the cache's own append
    for t, n in zip(tables, hist):
        if n:
            cache.append(1, t, torch.randn(n, Hk, D, generator=g).to(dtype).to(DEV),
                         torch.randn(n, Hk, D, generator=g).to(dtype).to(DEV))
    ref_k = cache.k[1].cpu().float()
    ref_v = cache.v[1].cpu().float()
    starts = [t.length for t in tables]
    q = torch.randn(B, Hq, L, D, generator=g).to(dtype)
    k = torch.randn(B, Hk, L, D, generator=g).to(dtype)
    v = torch.randn(B, Hk, L, D, generator=g).to(dtype)
    step = cache.prepare_step(tables, L, starts)
    out = attention_section(q.to(DEV), k.to(DEV), v.to(DEV), 1, cache, step)
    assert out.shape == (B, L, Hq * D)
    tol = 2e-3 if dtype == torch.float16 else 1e-2
    for b, t in enumerate(tables):
        append_ref(ref_k, ref_v, t.blocks, starts[b], k[b].transpose(0, 1).float(), v[b].transpose(0, 1).float())
        kd = gather_ref(ref_k, t.blocks, t.length).transpose(0, 1).unsqueeze(0)
        vd = gather_ref(ref_v, t.blocks, t.length).transpose(0, 1).unsqueeze(0)
        ref = flash_attention_ref(q[b:b + 1].float(), kd, vd, causal=True, scale=1.0 / math.sqrt(D))
        ref = ref.transpose(1, 2).reshape(1, L, Hq * D)
        err = (out[b:b + 1].float().cpu() - ref).abs().max().item()
        assert err <= tol, (b, err)
    assert torch.equal(cache.k[1].cpu().float(), ref_k) and torch.equal(cache.v[1].cpu().float(), ref_v)
