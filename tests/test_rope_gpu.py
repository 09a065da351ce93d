"""GPU parity of the rotary embedding paths against the oracle's restatement
of the reference's apply_rotary_ref (kernels/ref/rope_apply_ref.py:22-53):

* rope_apply (cie_rope_apply): bit-exact, every head_dim and dtype,
  positions None / (L,) / (B, L), strided and in-place;
* the rotary KV append (cie_kv_append_rope): pools and the dense rotated K
  bit-exact against append_ref of rope_ref(k);
* RoPE fused into the query loads of flash and paged attention: bit-identical
  to rope_apply followed by the plain kernel (the same deterministic kernel
  on the same rotated q), and within the attention tolerance of the oracle;
* the attention section with RoPE against the reference's per-sequence
  order of operations on the oracle (block.py:53-71)."""

from __future__ import annotations

import math

import pytest
import torch

from engine.attention import prefill_kernel
from prefill_dispatch import batch_for_two_row_groups
from engine.attention import flash_attention, paged_attention
from engine.cache import KVCacheConfig, PagedKVCache, kv_append
from engine.model.rope import RotaryEmbedding, build_rope_cache, rope_apply
from oracle import append_ref, flash_attention_ref, gather_ref, rope_ref

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.float16: 2e-3, torch.bfloat16: 1e-2}


def _tables(n, D, theta=10000.0, tdt=torch.float32):
    """cos, sin on the host and on the GPU, in table dtype tdt: fp32 as
    built, or cast as the reference engine casts RotaryEmbedding's buffers
    (engine/runtime.py:35-37)."""
    c, s = build_rope_cache(n, D, theta)
    c, s = c.to(tdt), s.to(tdt)
    return c, s, c.to(DEV), s.to(DEV)


def _tdt(kind, dtype):
    """Table dtype for x of `dtype`: fp32, the same 16-bit type, or the other one."""
    return {"fp32": torch.float32, "same": dtype,
            "other": torch.bfloat16 if dtype == torch.float16 else torch.float16}[kind]


@pytest.mark.parametrize("tables", ["fp32", "same", "other"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D", [16, 32, 64, 128, 256])
def test_rope_apply_bit_exact(D, dtype, tables):
    B, H, L = 2, 3, 37
    c, s, cd, sd = _tables(4096, D, tdt=_tdt(tables, dtype))
    g = torch.Generator().manual_seed(D)
    x = (torch.randn(B, H, L, D, generator=g) * 3).to(dtype)
    pos1 = torch.randint(0, 4096, (L,), generator=g)
    pos2 = torch.randint(0, 4096, (B, L), generator=g)
    for pos in (None, pos1, pos2):
        got = rope_apply(x.to(DEV), cd, sd, None if pos is None else pos.to(DEV))
        assert torch.equal(got.cpu(), rope_ref(x, c, s, pos)), pos


def test_rope_apply_strided_in_place_and_module():
    D = 64
    c, s, cd, sd = _tables(512, D)
    g = torch.Generator().manual_seed(3)
    base = torch.randn(2, 9, 6, D, generator=g).half()
    want = rope_ref(base[:, ::2], c, s, torch.arange(100, 106))
    xd = base.to(DEV)
    view = xd[:, ::2]  # strided heads
    rope_apply(view, cd, sd, torch.arange(100, 106, device=DEV), out=view)
    assert torch.equal(xd[:, ::2].cpu(), want)
    assert torch.equal(xd[:, 1::2].cpu(), base[:, 1::2])  # untouched
    emb = RotaryEmbedding(D, 512).to(DEV)
    x = torch.randn(1, 4, 5, D, generator=g).bfloat16()
    assert torch.equal(emb.apply(x.to(DEV), torch.tensor([0, 1, 2, 3, 4], device=DEV)).cpu(),
                       rope_ref(x, c, s, torch.arange(5)))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_module_after_reference_engine_cast(dtype):
    """RotaryEmbedding whose buffers went through the reference engine's cast
    (cast_non_quantized_params: every floating buffer to the activation
    dtype) rotates bit-identically to apply_rotary_ref with those tables."""
    D = 64
    emb = RotaryEmbedding(D, 1024)
    for name, b in list(emb.named_buffers(recurse=False)):
        if b.is_floating_point():
            setattr(emb, name, b.to(dtype))
    c, s = emb.cos.clone(), emb.sin.clone()
    emb = emb.to(DEV)
    assert emb.cos.dtype == dtype
    g = torch.Generator().manual_seed(4)
    x = (torch.randn(2, 4, 33, D, generator=g) * 2).to(dtype)
    pos = torch.randint(0, 1024, (2, 33), generator=g)
    got = emb.apply(x.to(DEV), pos.to(DEV)).cpu()
    assert torch.equal(got, rope_ref(x, c, s, pos))
    # the reference's expression, evaluated by torch on these 16-bit tensors
    cc, ss = c[pos].reshape(2, 1, 33, D // 2), s[pos].reshape(2, 1, 33, D // 2)
    x1, x2 = x[..., :D // 2], x[..., D // 2:]
    assert torch.equal(got, torch.cat([x1 * cc - x2 * ss, x1 * ss + x2 * cc], -1))


def test_rope_apply_out_of_range_positions():
    D = 32
    _, _, cd, sd = _tables(16, D)
    x = torch.randn(1, 2, 3, D).half().to(DEV)
    status = torch.zeros(1, dtype=torch.int32, device=DEV)
    y = rope_apply(x, cd, sd, torch.tensor([0, 16, 5], device=DEV), status=status)
    assert int(status.item()) == 2
    assert torch.isnan(y[:, :, 1].float()).all() and torch.isfinite(y[:, :, [0, 2]].float()).all()


def _batch_tables(lens, starts, bs, seed, extra=4):
    g = torch.Generator().manual_seed(seed)
    need = [-(-(s0 + n) // bs) for s0, n in zip(starts, lens)]
    nb = sum(need) + extra
    perm = torch.randperm(nb, generator=g).tolist()
    tables, p = [], 0
    for n in need:
        tables.append(perm[p:p + n])
        p += n
    bt = torch.zeros(len(lens), max(need), dtype=torch.int32)
    for b, ids in enumerate(tables):
        bt[b, :len(ids)] = torch.tensor(ids, dtype=torch.int32)
    return nb, tables, bt


@pytest.mark.parametrize("tables", ["fp32", "same"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("Hk,D", [(8, 64), (2, 16), (4, 128), (1, 256)])
def test_rotary_append_bit_exact(Hk, D, dtype, tables):
    bs = 16
    lens, starts = [1, 37, 0, 64, 5], [0, 3, 9, 100, 15]
    c, s, cd, sd = _tables(1024, D, tdt=_tdt(tables, dtype))
    nb, tables, bt = _batch_tables(lens, starts, bs, seed=D)
    g = torch.Generator().manual_seed(Hk)
    kp = torch.randn(nb, bs, Hk, D, generator=g).to(dtype)
    vp = torch.randn(nb, bs, Hk, D, generator=g).to(dtype)
    T = sum(lens)
    k = torch.randn(T, Hk, D, generator=g).to(dtype)
    v = torch.randn(T, Hk, D, generator=g).to(dtype)
    ek, ev, ekr = kp.clone(), vp.clone(), torch.empty_like(k)
    row = 0
    for ids, s0, n in zip(tables, starts, lens):
        kr = rope_ref(k[row:row + n].transpose(0, 1).unsqueeze(0), c, s, torch.arange(s0, s0 + n))
        kr = kr[0].transpose(0, 1)
        ekr[row:row + n] = kr
        append_ref(ek, ev, ids, s0, kr, v[row:row + n])
        row += n
    kd, vd = kp.to(DEV), vp.to(DEV)
    k_out = torch.zeros(T, Hk, D, dtype=dtype, device=DEV)
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32, device=DEV)
    status = torch.zeros(1, dtype=torch.int32, device=DEV)
    kv_append(k.to(DEV), v.to(DEV), kd, vd, bt.to(DEV), cu, torch.tensor(starts, dtype=torch.int32, device=DEV),
              max_new=max(lens), status=status, rope=(cd, sd), k_out=k_out)
    assert int(status.item()) == 0
    assert torch.equal(kd.cpu(), ek) and torch.equal(vd.cpu(), ev)
    assert torch.equal(k_out.cpu(), ekr)


def test_rotary_append_position_outside_table_writes_nothing():
    D, bs = 64, 4
    _, _, cd, sd = _tables(6, D)  # positions 0..5 only
    nb, tables, bt = _batch_tables([4, 4], [0, 4], bs, seed=1)
    kd = torch.zeros(nb, bs, 2, D, dtype=torch.float16, device=DEV)
    vd = torch.zeros_like(kd)
    k = torch.ones(8, 2, D, dtype=torch.float16, device=DEV)
    status = torch.zeros(1, dtype=torch.int32, device=DEV)
    cu = torch.tensor([0, 4, 8], dtype=torch.int32, device=DEV)
    kv_append(k, k, kd, vd, bt.to(DEV), cu, torch.tensor([0, 4], dtype=torch.int32, device=DEV), max_new=4,
              status=status, rope=(cd, sd))
    assert int(status.item()) == 2
    # sequence 1: positions 4, 5 written, 6, 7 not
    blk = tables[1][1]
    assert (vd[blk, :2] == 1).all() and (vd[blk, 2:] == 0).all() and (kd[blk, 2:] == 0).all()


@pytest.mark.parametrize("tables", ["fp32", "same"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_flash_with_fused_q_rope_two_row_groups(dtype, tables):
    """head_dim 64 with enough work runs the two-row-group kernel, which
    rotates the q rows of both its row groups (two query heads) as they are
    loaded: equal bit for bit to rope_apply then the same launch, and to the
    oracle, over a batch of 2 problems repeated (positions from 0 and 300)."""
    B0, Hq, Hk, L, D = 2, 8, 2, 200, 64
    c, s, cd, sd = _tables(2048, D, tdt=_tdt(tables, dtype))
    g = torch.Generator().manual_seed(77)
    q = torch.randn(B0, Hq, L, D, generator=g).to(dtype)
    k = torch.randn(B0, Hk, L, D, generator=g).to(dtype)
    v = torch.randn(B0, Hk, L, D, generator=g).to(dtype)
    pos0 = torch.tensor([0, 300], dtype=torch.int32)
    kr = torch.cat([rope_ref(k[b:b + 1], c, s, torch.arange(int(pos0[b]), int(pos0[b]) + L)) for b in range(B0)])
    qr = torch.cat([rope_ref(q[b:b + 1], c, s, torch.arange(int(pos0[b]), int(pos0[b]) + L)) for b in range(B0)])
    ref = flash_attention_ref(qr.float(), kr.float(), v.float(), causal=True)
    R = (batch_for_two_row_groups(Hq, L, L, True) + B0 - 1) // B0  # copies of the 2-problem batch
    B = B0 * R
    assert prefill_kernel(B, Hq, Hk, L, L, D, True, dtype) == "r64_heads"
    rep = lambda t: t.repeat(R, *([1] * (t.dim() - 1)))  # noqa: E731
    qd, krd, vd, pd = rep(q).to(DEV), rep(kr).to(DEV), rep(v).to(DEV), rep(pos0).to(DEV)
    fused = flash_attention(qd, krd, vd, causal=True, rope=(cd, sd), q_pos0=pd)
    qrd = rep(qr).to(DEV)
    assert torch.equal(fused, flash_attention(qrd, krd, vd, causal=True))
    assert (fused.float().cpu() - rep(ref)).abs().max().item() <= TOL[dtype]


def _equal_or_both_nan(a, b):
    """NaN in the same places and equal bit for bit everywhere else."""
    an, bn = torch.isnan(a), torch.isnan(b)
    return torch.equal(an, bn) and torch.equal(a[~an], b[~bn])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_flash_fused_q_rope_positions_past_the_table(dtype):
    """Through the two-row-group kernel: a row whose position lies past the
    rotary tables comes out NaN (the reference's table indexing raises there)
    and every other row is what rope_apply then the same launch gives."""
    B0, Hq, Hk, L, D, rows = 2, 8, 2, 200, 64, 1024
    _, _, cd, sd = _tables(rows, D)
    g = torch.Generator().manual_seed(5)
    q = torch.randn(B0, Hq, L, D, generator=g).to(dtype)
    k = (torch.randn(B0, Hk, L, D, generator=g) * 0.125).to(dtype)
    v = torch.randn(B0, Hk, L, D, generator=g).to(dtype)
    pos0 = torch.tensor([0, rows - 150], dtype=torch.int32)  # batch 1: rows 150.. lie past the table
    R = (batch_for_two_row_groups(Hq, L, L, True) + B0 - 1) // B0
    assert prefill_kernel(B0 * R, Hq, Hk, L, L, D, True, dtype) == "r64_heads"
    rep = lambda t: t.repeat(R, *([1] * (t.dim() - 1)))  # noqa: E731
    qd, kd, vd, pd = rep(q).to(DEV), rep(k).to(DEV), rep(v).to(DEV), rep(pos0).to(DEV)
    fused = flash_attention(qd, kd, vd, causal=True, rope=(cd, sd), q_pos0=pd)
    pos = pd[:, None].long() + torch.arange(L, device=DEV)[None]
    unfused = flash_attention(rope_apply(qd, cd, sd, pos), kd, vd, causal=True)
    assert _equal_or_both_nan(fused, unfused)
    nan_rows = torch.isnan(fused.float()).all(-1)
    assert torch.equal(nan_rows, (pos >= rows)[:, None, :].expand_as(nan_rows))
    assert torch.isfinite(fused.float()[~nan_rows]).all()


@pytest.mark.parametrize("Lq,dtype", [(1, torch.float16), (5, torch.bfloat16)])
def test_paged_fused_q_rope_positions_past_the_table(Lq, dtype):
    """Paged: new-token rows at positions past the rotary tables come out NaN,
    the others equal rope_apply then the same launch."""
    Hq, Hk, D, bs, rows = 8, 2, 64, 16, 1024
    ctx = [40, rows + 6, 5 + Lq, rows + Lq - 1, 333]
    B = len(ctx)
    _, _, cd, sd = _tables(rows, D)
    nb, _, bt = _batch_tables(ctx, [0] * B, bs, seed=Lq)
    g = torch.Generator().manual_seed(Lq)
    kp = torch.randn(nb, bs, Hk, D, generator=g).to(dtype)
    vp = torch.randn(nb, bs, Hk, D, generator=g).to(dtype)
    q = torch.randn(B, Hq, Lq, D, generator=g).to(dtype)
    qd, kd, vd, btd = q.to(DEV), kp.to(DEV), vp.to(DEV), bt.to(DEV)
    ld = torch.tensor(ctx, dtype=torch.int32, device=DEV)
    fused = paged_attention(qd, kd, vd, btd, ld, causal=True, rope=(cd, sd))
    pos = torch.stack([torch.arange(n - Lq, n) for n in ctx]).to(DEV)
    unfused = paged_attention(rope_apply(qd, cd, sd, pos), kd, vd, btd, ld, causal=True)
    assert _equal_or_both_nan(fused, unfused)
    nan_rows = torch.isnan(fused.float()).all(-1)
    assert torch.equal(nan_rows, (pos >= rows)[:, None, :].expand_as(nan_rows))
    assert nan_rows.any() and not nan_rows.all()


@pytest.mark.parametrize("tables", ["fp32", "same"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D", [16, 64, 128])
def test_flash_with_fused_q_rope(D, dtype, tables):
    B, Hq, Hk, L = 2, 8, 2, 200
    c, s, cd, sd = _tables(2048, D, tdt=_tdt(tables, dtype))
    g = torch.Generator().manual_seed(11 + D)
    q = torch.randn(B, Hq, L, D, generator=g).to(dtype)
    k = torch.randn(B, Hk, L, D, generator=g).to(dtype)
    v = torch.randn(B, Hk, L, D, generator=g).to(dtype)
    pos0 = torch.tensor([0, 300], dtype=torch.int32)
    kr = torch.cat([rope_ref(k[b:b + 1], c, s, torch.arange(int(pos0[b]), int(pos0[b]) + L)) for b in range(B)])
    qr = torch.cat([rope_ref(q[b:b + 1], c, s, torch.arange(int(pos0[b]), int(pos0[b]) + L)) for b in range(B)])
    qd, krd, vd = q.to(DEV), kr.to(DEV), v.to(DEV)
    fused = flash_attention(qd, krd, vd, causal=True, rope=(cd, sd), q_pos0=pos0.to(DEV))
    # the same kernel on q rotated by rope_apply
    qrd = torch.empty_like(qd)
    for b in range(B):
        qrd[b:b + 1] = rope_apply(qd[b:b + 1], cd, sd, torch.arange(int(pos0[b]), int(pos0[b]) + L, device=DEV))
    assert torch.equal(qrd.cpu(), qr)
    unfused = flash_attention(qrd, krd, vd, causal=True)
    assert torch.equal(fused, unfused)
    ref = flash_attention_ref(qr.float(), kr.float(), v.float(), causal=True)
    assert (fused.float().cpu() - ref).abs().max().item() <= TOL[dtype]
    # default positions 0..L-1
    f0 = flash_attention(qd, krd, vd, causal=True, rope=(cd, sd))
    assert torch.equal(f0[0], fused[0])


@pytest.mark.parametrize("tables", ["fp32", "same"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("Lq,D", [(1, 64), (5, 128), (1, 16), (3, 256)])
def test_paged_with_fused_q_rope(Lq, D, dtype, tables):
    Hq, Hk, bs = 8, 2, 16
    ctx = [40, 1000, 5, 333, 17 + Lq]
    B = len(ctx)
    c, s, cd, sd = _tables(2048, D, tdt=_tdt(tables, dtype))
    nb, tables, bt = _batch_tables(ctx, [0] * B, bs, seed=Lq + D)
    g = torch.Generator().manual_seed(D)
    kp = torch.randn(nb, bs, Hk, D, generator=g).to(dtype)
    vp = torch.randn(nb, bs, Hk, D, generator=g).to(dtype)
    q = torch.randn(B, Hq, Lq, D, generator=g).to(dtype)
    lens = torch.tensor(ctx, dtype=torch.int32)
    qd, kd, vd, btd, ld = q.to(DEV), kp.to(DEV), vp.to(DEV), bt.to(DEV), lens.to(DEV)
    fused = paged_attention(qd, kd, vd, btd, ld, causal=True, rope=(cd, sd))
    pos = torch.stack([torch.arange(n - Lq, n) for n in ctx])
    qr = rope_apply(qd, cd, sd, pos.to(DEV))
    assert torch.equal(qr.cpu(), rope_ref(q, c, s, pos))
    assert torch.equal(fused, paged_attention(qr, kd, vd, btd, ld, causal=True))
    for b in range(B):
        kh = gather_ref(kp.float(), tables[b], ctx[b]).transpose(0, 1).unsqueeze(0)
        vh = gather_ref(vp.float(), tables[b], ctx[b]).transpose(0, 1).unsqueeze(0)
        ref = flash_attention_ref(qr[b:b + 1].float().cpu(), kh, vh, causal=True)
        assert (fused[b:b + 1].float().cpu() - ref).abs().max().item() <= TOL[dtype]


@pytest.mark.parametrize("cast", [False, True])
@pytest.mark.parametrize("L,dtype", [(1, torch.float16), (4, torch.bfloat16), (96, torch.float16)])
def test_attention_section_with_rope_matches_reference_order(L, dtype, cast):
    """Prefill (fresh sequences, L=96), decode (L=1) and verify (L=4) through
    attention_section with un-rotated q, k and the model's tables, against
    the reference's per-sequence order on the oracle: rotate q and k at
    positions start..start+L-1 (block.py:53-54), append (:57-64), gather
    (:65), causal attention with scale 1/sqrt(D) (:69-71)."""
    from engine.model import attention_section

    B, Hq, Hk, D, bs = 3, 8, 2, 64, 16
    emb = RotaryEmbedding(D, 4096)
    if cast:  # the reference engine's cast of every floating buffer (engine/runtime.py:35-37)
        for name, b in list(emb.named_buffers(recurse=False)):
            setattr(emb, name, b.to(dtype))
    c, s = emb.cos, emb.sin
    emb = emb.to(DEV)
    cache = PagedKVCache(KVCacheConfig(num_layers=1, num_kv_heads=Hk, head_dim=D, num_blocks=120, block_size=bs,
                                       dtype=dtype, device=DEV))
    g = torch.Generator().manual_seed(60 + L)
    tables = [cache.new_sequence() for _ in range(B)]
    hist = [0, 0, 0] if L == 96 else [50, 0, 300]
    for t, n in zip(tables, hist):
        if n:
            cache.append(0, t, torch.randn(n, Hk, D, generator=g).to(dtype).to(DEV),
                         torch.randn(n, Hk, D, generator=g).to(dtype).to(DEV))
    ref_k, ref_v = cache.k[0].cpu().float(), cache.v[0].cpu().float()
    starts = [t.length for t in tables]
    q = torch.randn(B, Hq, L, D, generator=g).to(dtype)
    k = torch.randn(B, Hk, L, D, generator=g).to(dtype)
    v = torch.randn(B, Hk, L, D, generator=g).to(dtype)
    step = cache.prepare_step(tables, L)
    # q, k, v as the model makes them: transposed views of (B, L, H, D) projections (block.py:50-52)
    qv, kv_, vv = (x.transpose(1, 2).contiguous().to(DEV).transpose(1, 2) for x in (q, k, v))
    out = attention_section(qv, kv_, vv, 0, cache, step, rope=emb.tables)
    assert out.shape == (B, L, Hq * D)
    for b, t in enumerate(tables):
        pos = torch.arange(starts[b], starts[b] + L)
        qr = rope_ref(q[b:b + 1], c, s, pos)
        kr = rope_ref(k[b:b + 1], c, s, pos)
        append_ref(ref_k, ref_v, t.blocks, starts[b], kr[0].transpose(0, 1).float(), v[b].transpose(0, 1).float())
        kh = gather_ref(ref_k, t.blocks, t.length).transpose(0, 1).unsqueeze(0)
        vh = gather_ref(ref_v, t.blocks, t.length).transpose(0, 1).unsqueeze(0)
        ref = flash_attention_ref(qr.float(), kh, vh, causal=True, scale=1.0 / math.sqrt(D))
        ref = ref.transpose(1, 2).reshape(1, L, Hq * D)
        assert (out[b:b + 1].float().cpu() - ref).abs().max().item() <= TOL[dtype], b
    assert torch.equal(cache.k[0].cpu().float(), ref_k) and torch.equal(cache.v[0].cpu().float(), ref_v)
