"""Paged K/V storage shared across sequences.

API and pool layout follow the reference's ``engine/cache/kv_cache.py``:

* ``KVCacheConfig`` (:10-31) with ``bytes_required`` = 2 * layers * blocks *
  block_size * Hk * D * element size;
* per layer one K and one V pool of shape ``(num_blocks, block_size, Hk, D)``
  (:55-63), zero-initialised, so element (bid, off, h, d) sits at
  ``((bid * block_size + off) * Hk + h) * D + d``;
* a LIFO free list (:64, 76-82), ``new_sequence`` / ``free_sequence``,
  ``append`` (:102-139), ``gather`` (:141-165), ``fork`` (:169-185),
  ``rollback`` (:187-194), ``stats`` (:196-210).

Added for the paged kernel: :func:`block_table_tensor`, which packs host
block tables into the int32 ``(B, max_blocks)`` / ``(B,)`` device format
``paged_attention`` reads, and :meth:`PagedKVCache.attend`, which runs it on
one layer's pools.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Sequence

import torch

from engine.cache.block_table import BlockTable


@dataclass
class KVCacheConfig:
    num_layers: int
    num_kv_heads: int
    head_dim: int
    num_blocks: int
    block_size: int
    dtype: torch.dtype = torch.float16
    device: torch.device | str = "cuda"

    def bytes_required(self) -> int:
        """K + V bytes over all layers."""
        elt = torch.empty((), dtype=self.dtype).element_size()
        return 2 * self.num_layers * self.num_blocks * self.block_size * self.num_kv_heads * self.head_dim * elt


def block_table_tensor(
    tables: Sequence[BlockTable],
    device: torch.device | str,
    max_blocks: int | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Pack block tables for ``paged_attention``.

    Returns ``(block_tables int32 (B, max_blocks), context_lens int32 (B,))``
    on ``device`` (one host-to-device copy each). Unused trailing entries of a
    row are 0; they are never read because ``context_lens`` bounds every row.
    """
    width = max([len(t.blocks) for t in tables] + [1]) if max_blocks is None else max_blocks
    bt = torch.zeros((len(tables), width), dtype=torch.int32)
    for i, t in enumerate(tables):
        if len(t.blocks) > width:
            raise ValueError(f"sequence {i} holds {len(t.blocks)} blocks, more than max_blocks={width}")
        if t.blocks:
            bt[i, :len(t.blocks)] = torch.tensor(t.blocks, dtype=torch.int32)
    lens = torch.tensor([t.length for t in tables], dtype=torch.int32)
    return bt.to(device), lens.to(device)


class PagedKVCache:
    """Block-based K/V storage. Sequences own a :class:`BlockTable`; ``fork``
    deep-copies a sequence into fresh blocks so speculative rejection can roll
    back without disturbing the parent."""

    def __init__(self, cfg: KVCacheConfig):
        self.cfg = cfg
        device = torch.device(cfg.device)
        if device.type == "cuda":
            free, _ = torch.cuda.mem_get_info(device)
            need = cfg.bytes_required()
            if need > free:
                raise RuntimeError(
                    f"PagedKVCache would need {need / 2**30:.2f} GiB but only "
                    f"{free / 2**30:.2f} GiB free on {device}")
        shape = (cfg.num_blocks, cfg.block_size, cfg.num_kv_heads, cfg.head_dim)
        self.k = [torch.zeros(shape, dtype=cfg.dtype, device=device) for _ in range(cfg.num_layers)]
        self.v = [torch.zeros(shape, dtype=cfg.dtype, device=device) for _ in range(cfg.num_layers)]
        self._free: list[int] = list(range(cfg.num_blocks))

    @property
    def device(self) -> torch.device:
        return self.k[0].device

    @property
    def dtype(self) -> torch.dtype:
        return self.k[0].dtype

    # block allocator (LIFO: the most recently freed block is reused first)

    def _alloc_block(self) -> int:
        if not self._free:
            raise RuntimeError("KV cache out of blocks")
        return self._free.pop()

    def _free_block(self, block_id: int) -> None:
        self._free.append(block_id)

    def new_sequence(self) -> BlockTable:
        return BlockTable(block_size=self.cfg.block_size)

    def free_sequence(self, table: BlockTable) -> None:
        for bid in table.blocks:
            self._free_block(bid)
        table.blocks.clear()
        table.length = 0

    # write / read

    def _validate(self, t: torch.Tensor) -> None:
        if t.device != self.device or t.dtype != self.dtype:
            raise ValueError(
                f"tensor device/dtype ({t.device}/{t.dtype}) does not match "
                f"cache ({self.device}/{self.dtype})")

    def append(self, layer: int, table: BlockTable, k: torch.Tensor, v: torch.Tensor,
               start: int | None = None) -> None:
        """Write ``k``, ``v`` of shape (L, Hk, D) at positions start..start+L-1
        (default: after the current end), allocating blocks as needed and
        extending ``table.length`` when the write passes the end."""
        L = k.shape[0]
        assert v.shape[0] == L
        self._validate(k)
        self._validate(v)
        if start is None:
            start = table.length
        end = start + L
        while len(table.blocks) < table.num_blocks_needed(end):
            table.blocks.append(self._alloc_block())
        bs = self.cfg.block_size
        done = 0
        while done < L:
            bid, off = table.logical_to_physical(start + done)
            n = min(bs - off, L - done)
            self.k[layer][bid, off:off + n] = k[done:done + n]
            self.v[layer][bid, off:off + n] = v[done:done + n]
            done += n
        table.length = max(table.length, end)

    def gather(self, layer: int, table: BlockTable) -> tuple[torch.Tensor, torch.Tensor]:
        """Dense (L, Hk, D) copies of one sequence's K and V history."""
        L = table.length
        Hk, D = self.cfg.num_kv_heads, self.cfg.head_dim
        if L == 0:
            empty = self.k[layer].new_zeros((0, Hk, D))
            return empty, empty.clone()
        idx = torch.tensor(table.blocks, dtype=torch.long, device=self.device)
        k = self.k[layer].index_select(0, idx).reshape(-1, Hk, D)[:L]
        v = self.v[layer].index_select(0, idx).reshape(-1, Hk, D)[:L]
        return k, v

    def attend(self, layer: int, q: torch.Tensor, tables: Sequence[BlockTable],
               causal: bool = True, scale: float | None = None) -> torch.Tensor:
        """``paged_attention`` of q (B, Hq, Lq, D) over the sequences'
        histories in this layer's pools (no gather)."""
        from engine.attention import paged_attention

        bt, lens = block_table_tensor(tables, self.device)
        max_ctx = max([t.length for t in tables] + [1])
        return paged_attention(q, self.k[layer], self.v[layer], bt, lens, causal=causal,
                               scale=scale, max_context=max_ctx)

    # speculative fork / rollback

    def fork(self, table: BlockTable) -> BlockTable:
        """New table whose K/V are a deep copy of ``table``'s, in fresh blocks."""
        n = len(table.blocks)
        fresh = [self._alloc_block() for _ in range(n)]
        if n:
            src = torch.tensor(table.blocks, dtype=torch.long, device=self.device)
            dst = torch.tensor(fresh, dtype=torch.long, device=self.device)
            for layer in range(self.cfg.num_layers):
                self.k[layer].index_copy_(0, dst, self.k[layer].index_select(0, src))
                self.v[layer].index_copy_(0, dst, self.v[layer].index_select(0, src))
        return BlockTable(block_size=self.cfg.block_size, blocks=fresh, length=table.length)

    def rollback(self, table: BlockTable, new_length: int) -> None:
        """Truncate to ``new_length`` tokens and free the blocks it no longer needs."""
        assert new_length <= table.length
        keep = table.num_blocks_needed(new_length)
        for bid in table.blocks[keep:]:
            self._free_block(bid)
        del table.blocks[keep:]
        table.length = new_length

    def stats(self) -> None:
        total = self.cfg.num_blocks
        free = len(self._free)
        print(f"Cache Memory Footprint: {self.cfg.bytes_required()}")
        print(f"Total Blocks: {total}")
        print(f"Allocated Blocks: {total - free}")
        print(f"Freed Blocks: {free}")
