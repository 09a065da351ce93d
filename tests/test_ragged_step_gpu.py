"""GPU parity of ragged and long steps through the attention section against
the reference's per-sequence order of operations on the oracle (block.py:
53-71: rotate q and k at positions start..start+c-1, append, gather the
whole history, causal attention with scale 1/sqrt(D)).

* attention_section_rows: a prefill chunk over a history next to decode
  tokens, a fresh prefill and a sequence with no new tokens in one step;
  with and without the model's RoPE tables, and with the new tokens written
  below a sequence's end (positions that differ from context_len - c + i);
* attention_section with L new tokens per sequence over a history and more
  query rows per kv head than one paged launch takes (256; 128 at head_dim
  256): the split launches.

PagedKVCache.gather is replaced by a function that raises, so a path that
falls back to gathering the history fails."""

from __future__ import annotations

import math

import pytest
import torch

from engine.cache import KVCacheConfig, PagedKVCache
from engine.model import attention_section, attention_section_rows
from engine.model.rope import RotaryEmbedding
from oracle import append_ref, flash_attention_ref, gather_ref, rope_ref

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.float16: 2e-3, torch.bfloat16: 1e-2}


@pytest.fixture
def no_gather(monkeypatch):
    def refuse(*a, **k):
        raise AssertionError("the attention section gathered a history")

    monkeypatch.setattr(PagedKVCache, "gather", refuse)


def _cache(Hk, D, dtype, hist, g, num_blocks=400, bs=16):
    cache = PagedKVCache(KVCacheConfig(num_layers=1, num_kv_heads=Hk, head_dim=D, num_blocks=num_blocks,
                                       block_size=bs, dtype=dtype, device=DEV))
    tables = [cache.new_sequence() for _ in hist]
    for t, n in zip(tables, hist):
        if n:
            cache.append(0, t, torch.randn(n, Hk, D, generator=g).to(dtype).to(DEV),
                         torch.randn(n, Hk, D, generator=g).to(dtype).to(DEV))
    return cache, tables


def _reference(ref_k, ref_v, tables, starts, counts, q, k, v, tabs):
    """Per sequence, the reference's order on the oracle. q (T, Hq, D),
    k / v (T, Hk, D) packed rows; tabs = (cos, sin) on the host or None.
    Returns (T, Hq * D) fp32, NaN rows for nothing."""
    Hq, D = q.shape[1], q.shape[2]
    out = torch.empty(q.shape[0], Hq * D)
    r0 = 0
    for t, s0, c in zip(tables, starts, counts):
        if c == 0:
            continue
        qb = q[r0:r0 + c].transpose(0, 1).unsqueeze(0)
        kb = k[r0:r0 + c].transpose(0, 1).unsqueeze(0)
        if tabs is not None:
            pos = torch.arange(s0, s0 + c)
            qb, kb = rope_ref(qb, tabs[0], tabs[1], pos), rope_ref(kb, tabs[0], tabs[1], pos)
        append_ref(ref_k, ref_v, t.blocks, s0, kb[0].transpose(0, 1).float(), v[r0:r0 + c].float())
        kh = gather_ref(ref_k, t.blocks, t.length).transpose(0, 1).unsqueeze(0)
        vh = gather_ref(ref_v, t.blocks, t.length).transpose(0, 1).unsqueeze(0)
        o = flash_attention_ref(qb.float(), kh, vh, causal=True, scale=1.0 / math.sqrt(D))
        out[r0:r0 + c] = o[0].transpose(0, 1).reshape(c, Hq * D)
        r0 += c
    return out


@pytest.mark.parametrize("rope,below_end", [(False, False), (True, False), (True, True), (False, True)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_ragged_step_matches_reference_order(dtype, rope, below_end, no_gather):
    Hq, Hk, D = 8, 2, 64  # 4 query heads per kv head: launches of at most 64 tokens
    hist = [500, 40, 1200, 0, 77, 300, 9]
    counts = [300, 1, 1, 130, 5, 0, 64]  # a prefill chunk over a history, decode, a fresh prefill, none
    g = torch.Generator().manual_seed(7 + int(rope) + 2 * int(below_end))
    cache, tables = _cache(Hk, D, dtype, hist, g)
    starts = [h - 3 if below_end and c and h >= 3 else h for h, c in zip(hist, counts)]
    emb = RotaryEmbedding(D, 4096)
    tabs = (emb.cos, emb.sin) if rope else None
    emb = emb.to(DEV)
    ref_k, ref_v = cache.k[0].cpu().float(), cache.v[0].cpu().float()
    T = sum(counts)
    q = torch.randn(T, Hq, D, generator=g).to(dtype)
    k = torch.randn(T, Hk, D, generator=g).to(dtype)
    v = torch.randn(T, Hk, D, generator=g).to(dtype)
    step = cache.prepare_step(tables, counts, starts)
    assert step.num_new == -1 and step.aligned == (not below_end)
    out = attention_section_rows(q.to(DEV), k.to(DEV), v.to(DEV), 0, cache, step,
                                 rope=emb.tables if rope else None)
    assert out.shape == (T, Hq * D)
    ref = _reference(ref_k, ref_v, tables, starts, counts, q, k, v, tabs)
    err = (out.float().cpu() - ref).abs().max().item()
    assert err <= TOL[dtype], err
    assert torch.equal(cache.k[0].cpu().float(), ref_k) and torch.equal(cache.v[0].cpu().float(), ref_v)
    # a second layer call of the same step reuses the step's launch list and gives the same rows
    n_cached = len(step.cache)
    cache2, tables2 = _cache(Hk, D, dtype, hist, torch.Generator().manual_seed(7 + int(rope) + 2 * int(below_end)))
    step2 = cache2.prepare_step(tables2, counts, starts)
    step2.cache.update(step.cache)
    out2 = attention_section_rows(q.to(DEV), k.to(DEV), v.to(DEV), 0, cache2, step2,
                                  rope=emb.tables if rope else None)
    assert len(step2.cache) == n_cached and torch.equal(out2.cpu(), out.cpu())


@pytest.mark.parametrize("L,Hq,Hk,D,dtype", [(96, 8, 2, 64, torch.float16), (300, 4, 4, 128, torch.bfloat16),
                                            (257, 2, 2, 32, torch.float16), (40, 8, 2, 256, torch.float16)])
def test_long_uniform_step_over_history_matches_reference_order(L, Hq, Hk, D, dtype, no_gather):
    """(Hq/Hk) * L above paged_max_rows(D) (256; 128 at head_dim 256):
    attention_section splits the chunk into launches."""
    from engine.attention import paged_max_rows

    assert (Hq // Hk) * L > paged_max_rows(D)
    hist = [200, 31, 1000]
    g = torch.Generator().manual_seed(L)
    cache, tables = _cache(Hk, D, dtype, hist, g)
    emb = RotaryEmbedding(D, 4096)
    tabs = (emb.cos, emb.sin)
    emb = emb.to(DEV)
    ref_k, ref_v = cache.k[0].cpu().float(), cache.v[0].cpu().float()
    B = len(hist)
    q = torch.randn(B, Hq, L, D, generator=g).to(dtype)
    k = torch.randn(B, Hk, L, D, generator=g).to(dtype)
    v = torch.randn(B, Hk, L, D, generator=g).to(dtype)
    step = cache.prepare_step(tables, L, num_heads=Hq)
    assert not step.fresh and step.plan is None  # no single launch covers this shape
    qv, kv_, vv = (x.transpose(1, 2).contiguous().to(DEV).transpose(1, 2) for x in (q, k, v))
    out = attention_section(qv, kv_, vv, 0, cache, step, rope=emb.tables)
    assert out.shape == (B, L, Hq * D)
    pack = lambda x: x.transpose(1, 2).reshape(B * L, x.shape[1], D)  # noqa: E731
    ref = _reference(ref_k, ref_v, tables, hist, [L] * B, pack(q), pack(k), pack(v), tabs)
    err = (out.float().cpu().view(B * L, Hq * D) - ref).abs().max().item()
    assert err <= TOL[dtype], err
    assert torch.equal(cache.k[0].cpu().float(), ref_k) and torch.equal(cache.v[0].cpu().float(), ref_v)


def test_uniform_step_through_rows_equals_attention_section(no_gather):
    """A decode step through attention_section_rows equals attention_section's
    fused path bit for bit (the same kernels on the same rows)."""
    Hq, Hk, D, dtype = 8, 2, 64, torch.float16
    hist = [50, 0, 300, 1000, 17]
    outs = []
    for rows in (False, True):
        g = torch.Generator().manual_seed(3)
        cache, tables = _cache(Hk, D, dtype, hist, g)
        B, L = len(hist), 1
        q = torch.randn(B, Hq, L, D, generator=g).to(dtype).to(DEV)
        k = torch.randn(B, Hk, L, D, generator=g).to(dtype).to(DEV)
        v = torch.randn(B, Hk, L, D, generator=g).to(dtype).to(DEV)
        step = cache.prepare_step(tables, L)
        if rows:
            o = attention_section_rows(q[:, :, 0], k[:, :, 0], v[:, :, 0], 0, cache, step)
        else:
            o = attention_section(q, k, v, 0, cache, step).view(B, Hq * D)
        outs.append((o.cpu(), cache.k[0].cpu(), cache.v[0].cpu()))
    for a, b in zip(*outs):
        assert torch.equal(a, b)
