"""Host logic of engine.cache on the CPU device: the reference's block-table
known answers (tests/cache/test_block_table.py:8-29) and its KV-cache
behaviour tests (tests/cache/test_kv_cache.py:16-77), plus the int32 device
block-table packing the paged kernel reads."""

from __future__ import annotations

import pytest
import torch

from engine.cache import BlockTable, KVCacheConfig, PagedKVCache, block_table_tensor
from oracle import gather_ref


def test_logical_to_physical():
    t = BlockTable(block_size=4, blocks=[10, 11, 12], length=9)
    assert t.logical_to_physical(0) == (10, 0)
    assert t.logical_to_physical(3) == (10, 3)
    assert t.logical_to_physical(4) == (11, 0)
    assert t.logical_to_physical(8) == (12, 0)


def test_clone_independent():
    t = BlockTable(block_size=2, blocks=[1, 2], length=4)
    c = t.clone()
    c.blocks.append(3)
    c.length = 5
    assert t.blocks == [1, 2] and t.length == 4


def test_truncate_drops_blocks():
    t = BlockTable(block_size=2, blocks=[1, 2, 3], length=6)
    t.truncate(3)
    assert t.length == 3 and t.blocks == [1, 2]


def test_num_blocks_needed():
    t = BlockTable(block_size=16)
    assert [t.num_blocks_needed(n) for n in (0, 1, 16, 17, 32)] == [0, 1, 1, 2, 2]


def make_cache(num_blocks=8, block_size=4, layers=2, heads=2, dim=16, dtype=torch.float16):
    return PagedKVCache(KVCacheConfig(num_layers=layers, num_kv_heads=heads, head_dim=dim,
                                      num_blocks=num_blocks, block_size=block_size, dtype=dtype, device="cpu"))


def test_bytes_required():
    cfg = KVCacheConfig(num_layers=3, num_kv_heads=8, head_dim=64, num_blocks=10, block_size=16,
                        dtype=torch.bfloat16, device="cpu")
    assert cfg.bytes_required() == 2 * 3 * 10 * 16 * 8 * 64 * 2


def test_append_and_gather_roundtrip():
    torch.manual_seed(0)
    cache = make_cache()
    seq = cache.new_sequence()
    k = torch.randn(6, 2, 16, dtype=torch.float16)
    v = torch.randn(6, 2, 16, dtype=torch.float16)
    cache.append(0, seq, k, v)
    gk, gv = cache.gather(0, seq)
    assert torch.equal(gk, k) and torch.equal(gv, v) and seq.length == 6


def test_append_spans_multiple_blocks():
    cache = make_cache(block_size=2)
    seq = cache.new_sequence()
    k = torch.randn(5, 2, 16, dtype=torch.float16)
    v = torch.randn(5, 2, 16, dtype=torch.float16)
    cache.append(0, seq, k, v)
    assert len(seq.blocks) == 3
    gk, gv = cache.gather(0, seq)
    assert torch.equal(gk, k) and torch.equal(gv, v)
    # the pool layout: token t at pool[blocks[t // bs], t % bs]
    assert torch.equal(gather_ref(cache.k[0], seq.blocks, seq.length), k)


def test_append_at_explicit_start_overwrites():
    cache = make_cache(block_size=4)
    seq = cache.new_sequence()
    cache.append(0, seq, torch.zeros(6, 2, 16, dtype=torch.float16), torch.zeros(6, 2, 16, dtype=torch.float16))
    upd = torch.ones(2, 2, 16, dtype=torch.float16)
    cache.append(0, seq, upd, upd, start=3)
    gk, _ = cache.gather(0, seq)
    assert seq.length == 6
    assert (gk[3:5] == 1).all() and (gk[:3] == 0).all() and (gk[5] == 0).all()


def test_free_sequence_returns_blocks():
    cache = make_cache(num_blocks=4, block_size=2)
    seq = cache.new_sequence()
    cache.append(0, seq, torch.randn(4, 2, 16, dtype=torch.float16), torch.randn(4, 2, 16, dtype=torch.float16))
    assert len(cache._free) == 2
    cache.free_sequence(seq)
    assert len(cache._free) == 4 and seq.length == 0


def test_out_of_blocks():
    cache = make_cache(num_blocks=1, block_size=2)
    seq = cache.new_sequence()
    with pytest.raises(RuntimeError, match="out of blocks"):
        cache.append(0, seq, torch.randn(3, 2, 16, dtype=torch.float16), torch.randn(3, 2, 16, dtype=torch.float16))


def test_dtype_mismatch_rejected():
    cache = make_cache()
    seq = cache.new_sequence()
    with pytest.raises(ValueError):
        cache.append(0, seq, torch.randn(1, 2, 16), torch.randn(1, 2, 16))


def test_fork_is_deep_copy():
    cache = make_cache()
    seq = cache.new_sequence()
    cache.append(0, seq, torch.randn(3, 2, 16, dtype=torch.float16), torch.randn(3, 2, 16, dtype=torch.float16))
    forked = cache.fork(seq)
    gk0, _ = cache.gather(0, seq)
    gkf, _ = cache.gather(0, forked)
    assert torch.equal(gk0, gkf) and set(forked.blocks).isdisjoint(seq.blocks)
    cache.append(0, seq, torch.randn(1, 2, 16, dtype=torch.float16), torch.randn(1, 2, 16, dtype=torch.float16))
    assert seq.length == 4 and forked.length == 3
    gkf2, _ = cache.gather(0, forked)
    assert torch.equal(gkf, gkf2)


def test_rollback_frees_blocks():
    cache = make_cache(num_blocks=4, block_size=2)
    seq = cache.new_sequence()
    cache.append(0, seq, torch.randn(4, 2, 16, dtype=torch.float16), torch.randn(4, 2, 16, dtype=torch.float16))
    assert len(cache._free) == 2
    cache.rollback(seq, new_length=2)
    assert seq.length == 2 and len(cache._free) == 3


def test_block_table_tensor_packing():
    tabs = [BlockTable(4, [7, 2, 5], 10), BlockTable(4, [], 0), BlockTable(4, [1], 3)]
    bt, lens = block_table_tensor(tabs, "cpu")
    assert bt.dtype == torch.int32 and lens.dtype == torch.int32
    assert bt.tolist() == [[7, 2, 5], [0, 0, 0], [1, 0, 0]]
    assert lens.tolist() == [10, 0, 3]
    bt2, _ = block_table_tensor(tabs, "cpu", max_blocks=5)
    assert bt2.shape == (3, 5)
    with pytest.raises(ValueError):
        block_table_tensor(tabs, "cpu", max_blocks=2)
