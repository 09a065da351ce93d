"""GPU parity of the fused append + paged attention (engine.attention.paged_attention
with new_kv -> cie_paged_fwd_append) against the two-step path it replaces:
cie_kv_append of the new tokens (the reference's append loop,
engine/cache/kv_cache.py:128-136) followed by cie_paged_fwd (the reference's
gather + attend, engine/model/block.py:57-71). The bar is bit-exactness of
both pools and of the output: the fused launch reads the same values and
runs the same arithmetic; the oracle check confirms the result too. With
RoPE the reference rotates q and k first (engine/model/block.py:53-54); the
fused pair rotates the new K rows itself, bit-identical to the rotating
append."""

from __future__ import annotations

import pytest
import torch

from engine.attention import paged_attention
from engine.cache import kv_append
from oracle import paged_attention_ref
from test_flash_gpu import TOL, assert_close
from test_paged_gpu import make_paged

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _two_step(q, kp, vp, bt, lens, k_new, v_new, Lq, **kw):
    """kv_append of the Lq newest tokens, then paged_attention (the reference's order)."""
    kd, vd = kp.to(DEV), vp.to(DEV)
    B = q.shape[0]
    cu = torch.arange(0, B * Lq + 1, Lq, dtype=torch.int32, device=DEV)
    starts = (lens - Lq).to(torch.int32).to(DEV)
    kv_append(k_new.to(DEV), v_new.to(DEV), kd, vd, bt.to(DEV), cu, starts, max_new=Lq)
    out = paged_attention(q.to(DEV), kd, vd, bt.to(DEV), lens.to(DEV), causal=True, **kw)
    return out.cpu(), kd.cpu(), vd.cpu()


def _fused(q, kp, vp, bt, lens, k_new, v_new, **kw):
    kd, vd = kp.to(DEV), vp.to(DEV)
    out = paged_attention(q.to(DEV), kd, vd, bt.to(DEV), lens.to(DEV), causal=True,
                          new_kv=(k_new.to(DEV), v_new.to(DEV)), **kw)
    return out.cpu(), kd.cpu(), vd.cpu()


def _new_rows(B, Lq, Hk, D, dtype, seed, vscale=0.5):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(B * Lq, Hk, D, generator=g).to(dtype),
            (torch.randn(B * Lq, Hk, D, generator=g) * vscale).to(dtype))


@pytest.mark.parametrize("Lq", [1, 5])
@pytest.mark.parametrize("bs", [3, 16])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fused_append_equals_append_then_attend(Lq, bs, D, dtype):
    # lengths include the Lq new tokens; several split across workgroups, new
    # tokens straddling block and 32-token tile boundaries
    lens = [Lq, 31 + Lq, 33, 700, 2049, 4096, 95, 1024 + Lq]
    # V scaled by 1/2 keeps bf16 output rounding inside the tolerance, as in the other paged tests
    q, kp, vp, bt, lt = make_paged(lens, Lq, D, dtype, bs, Hq=8, Hk=2, seed=D + bs + Lq, vscale=0.5)
    k_new, v_new = _new_rows(len(lens), Lq, 2, D, dtype, seed=7 + Lq)
    o2, k2, v2 = _two_step(q, kp, vp, bt, lt, k_new, v_new, Lq)
    o1, k1, v1 = _fused(q, kp, vp, bt, lt, k_new, v_new)
    assert torch.equal(k1, k2) and torch.equal(v1, v2), "pool after the fused append differs"
    assert torch.equal(o1, o2), (o1.float() - o2.float()).abs().max().item()
    # and against the oracle over the appended pool
    ref = paged_attention_ref(q.float(), k2.float(), v2.float(), bt, lt, causal=True)
    assert_close(o1, ref, TOL[dtype], f"fused append Lq={Lq} bs={bs} D={D} {dtype}")


def test_fused_append_workload_shapes():
    """decode_b32- and verify_b8-like shapes (32 / 8 sequences, 32 q / 8 kv heads)."""
    for B, Lq, dtype, seed in ((32, 1, torch.float16, 2), (8, 5, torch.bfloat16, 3)):
        g = torch.Generator().manual_seed(seed)
        lens = torch.randint(256, 4097, (B,), generator=g).tolist()
        q, kp, vp, bt, lt = make_paged(lens, Lq, 64, dtype, 16, Hq=32, Hk=8, seed=seed)
        k_new, v_new = _new_rows(B, Lq, 8, 64, dtype, seed=seed + 100)
        o2, k2, v2 = _two_step(q, kp, vp, bt, lt, k_new, v_new, Lq)
        o1, k1, v1 = _fused(q, kp, vp, bt, lt, k_new, v_new)
        assert torch.equal(k1, k2) and torch.equal(v1, v2)
        assert torch.equal(o1, o2)


def test_fused_append_invalid_context_and_block_id():
    Lq, D, dtype = 5, 64, torch.float16
    lens = [40, 3, 300]  # sequence 1 is shorter than its Lq new tokens: invalid here
    q, kp, vp, bt, lt = make_paged(lens, Lq, D, dtype, 16, seed=11)
    bt[2, 18] = kp.shape[0] + 3  # the block holding sequence 2's newest tokens is out of range
    k_new, v_new = _new_rows(len(lens), Lq, 2, D, dtype, seed=12)
    o1, k1, v1 = _fused(q, kp, vp, bt, lt, k_new, v_new)
    assert torch.isnan(o1[1]).all() and torch.isnan(o1[2]).all()
    assert not torch.isnan(o1[0]).any()
    # sequence 0's new tokens were written; nothing of sequences 1 and 2 outside valid blocks
    # (one sequence alone splits differently, so compare within tolerance)
    o2, k2, v2 = _two_step(q[:1], kp, vp, bt[:1], lt[:1], k_new[:Lq], v_new[:Lq], Lq)
    assert_close(o1[:1], o2, TOL[dtype], "valid sequence next to invalid ones")
    b0_blocks = set(bt[0, :3].tolist())
    for blk in range(kp.shape[0]):
        if blk in b0_blocks or blk in set(bt[2, :18].tolist()):
            continue  # appended (sequence 0) or holding sequence 2's valid older rows
        assert torch.equal(k1[blk], kp[blk]) and torch.equal(v1[blk], vp[blk]), blk


@pytest.mark.parametrize("tables", ["fp32", "cast"])
@pytest.mark.parametrize("Lq", [1, 5])
@pytest.mark.parametrize("D", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fused_append_with_rope_equals_rotating_append_then_attend(Lq, D, dtype, tables):
    """q and k_new un-rotated: the fused pair rotates the new K rows in LDS
    and on their way into the pool, bit-identical to kv_append(rope=) then
    paged_attention(rope=); with fp32 tables and with tables cast to the
    activation dtype as the reference engine casts them
    (engine/runtime.py:35-37). Every head_dim covers one swizzle family of
    the in-LDS rotation."""
    from engine.model.rope import RotaryEmbedding

    emb = RotaryEmbedding(D, 8192)
    if tables == "cast":
        for name, b in list(emb.named_buffers(recurse=False)):
            setattr(emb, name, b.to(dtype))
    emb = emb.to(DEV)
    lens = [Lq, 40 + Lq, 700, 2049, 4096, 33]
    q, kp, vp, bt, lt = make_paged(lens, Lq, D, dtype, 16, Hq=8, Hk=2, seed=D + Lq, vscale=0.5)
    k_new, v_new = _new_rows(len(lens), Lq, 2, D, dtype, seed=21 + Lq)
    kd, vd = kp.to(DEV), vp.to(DEV)
    B = len(lens)
    cu = torch.arange(0, B * Lq + 1, Lq, dtype=torch.int32, device=DEV)
    kv_append(k_new.to(DEV), v_new.to(DEV), kd, vd, bt.to(DEV), cu, (lt - Lq).to(DEV), max_new=Lq, rope=emb.tables)
    o2 = paged_attention(q.to(DEV), kd, vd, bt.to(DEV), lt.to(DEV), causal=True, rope=emb.tables).cpu()
    o1, k1, v1 = _fused(q, kp, vp, bt, lt, k_new, v_new, rope=emb.tables)
    assert torch.equal(k1, kd.cpu()) and torch.equal(v1, vd.cpu()), "pool after the rotating fused append differs"
    assert torch.equal(o1, o2), (o1.float() - o2.float()).abs().max().item()


def test_fused_append_with_rope_position_outside_table_writes_nothing():
    """New tokens whose positions lie outside the rotary tables: their query
    rows are NaN and neither their K nor their V reaches the pool, as the
    rotating append leaves the pool (kv_append(rope=) writes neither). Rows
    of the same sequence whose positions are inside see only keys inside."""
    from engine.model.rope import build_rope_cache

    Lq, D, dtype = 5, 64, torch.float16
    lens = [40, 300]  # sequence 1's new tokens sit at positions 295..299; the tables hold 0..296
    q, kp, vp, bt, lt = make_paged(lens, Lq, D, dtype, 16, seed=31)
    k_new, v_new = _new_rows(len(lens), Lq, 2, D, dtype, seed=32)
    cos, sin = build_rope_cache(297, D)
    o1, k1, v1 = _fused(q, kp, vp, bt, lt, k_new, v_new, rope=(cos.to(DEV), sin.to(DEV)))
    assert not torch.isnan(o1[0]).any()
    assert not torch.isnan(o1[1, :, :2]).any() and torch.isnan(o1[1, :, 2:]).all()
    for pos in range(295, 300):
        blk, off = int(bt[1, pos // 16]), pos % 16
        if pos < 297:  # inside the tables: written
            assert torch.equal(v1[blk, off], v_new[Lq + pos - 295])
        else:  # outside: the pool keeps its old rows
            assert torch.equal(k1[blk, off], kp[blk, off]) and torch.equal(v1[blk, off], vp[blk, off]), pos


def test_fused_append_rejects_pools_it_cannot_write_in_place():
    """The fused append writes the pools in place: a pool view the kernels
    cannot address directly (here 8-byte aligned) is rejected rather than
    copied, which would drop the appended tokens."""
    q, kp, vp, bt, lt = make_paged([40], 1, 64, torch.float16, 16)
    k_new, v_new = _new_rows(1, 1, 2, 64, torch.float16, seed=1)
    nb = kp.shape[0]
    flat_k = torch.zeros(kp.numel() + 4, dtype=torch.float16, device=DEV)
    flat_v = torch.zeros_like(flat_k)
    kd = flat_k[4:].view(nb, 16, 2, 64)  # 8 bytes past a 16-byte boundary
    vd = flat_v[4:].view(nb, 16, 2, 64)
    kd.copy_(kp.to(DEV))
    vd.copy_(vp.to(DEV))
    with pytest.raises(ValueError):
        paged_attention(q.to(DEV), kd, vd, bt.to(DEV), lt.to(DEV), new_kv=(k_new.to(DEV), v_new.to(DEV)))
    # without the append the same views are read through a copy, correctly
    out = paged_attention(q.to(DEV), kd, vd, bt.to(DEV), lt.to(DEV))
    ref = paged_attention_ref(q.float(), kp.float(), vp.float(), bt, lt, causal=True)
    assert_close(out.cpu(), ref, TOL[torch.float16], "misaligned pool read through a copy")


def test_fused_append_rejects_bad_shapes():
    q, kp, vp, bt, lt = make_paged([40], 1, 64, torch.float16, 16)
    k_new, v_new = _new_rows(1, 1, 2, 64, torch.float16, seed=1)
    with pytest.raises(ValueError):
        paged_attention(q.to(DEV), kp.to(DEV), vp.to(DEV), bt.to(DEV), lt.to(DEV),
                        new_kv=(k_new[:, :1].to(DEV), v_new.to(DEV)))
    with pytest.raises(ValueError):
        paged_attention(q.to(DEV), kp.to(DEV), vp.to(DEV), bt.to(DEV), lt.to(DEV),
                        new_kv=(k_new.to(DEV), v_new.to(DEV).float()))
