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

Added for the paged kernels: :func:`block_table_tensor`, which packs host
block tables into the int32 ``(B, max_blocks)`` / ``(B,)`` device format the
kernels read; :func:`kv_append`, the batched device write of new tokens
(``cie_kv_append``); :meth:`PagedKVCache.append_batch`, its per-layer use for
many sequences; :meth:`PagedKVCache.prepare_step` / :meth:`append_step`,
which upload a step's metadata once for all layers (:class:`StepBatch`);
and :meth:`PagedKVCache.attend`, which runs
``paged_attention`` on one layer's pools. On a CUDA device ``append`` writes
through ``cie_kv_append`` (the reference's per-block slice loop,
kv_cache.py:128-136, becomes one launch); a cache on the CPU device keeps the
reference's slice copies, since no kernel runs there.
"""

from __future__ import annotations

from dataclasses import dataclass, field
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


@dataclass
class StepBatch:
    """Device-resident metadata of one engine step for B sequences
    (:meth:`PagedKVCache.prepare_step`), read by every layer's append and
    paged attention: int32 block tables (B, max_blocks), context lengths (B,)
    including the step's new tokens, row offsets ``cu_new`` (B+1,) of the
    new tokens and their start positions (B,). ``num_new`` is the number of
    new tokens of every sequence, or -1 when the counts differ (a ragged
    step: a prefill chunk next to decode tokens); ``new_counts`` holds them
    per sequence. ``max_context`` bounds ``context_lens``."""
    block_tables: torch.Tensor
    context_lens: torch.Tensor
    cu_new: torch.Tensor
    starts: torch.Tensor
    num_new: int
    max_context: int
    tables: tuple = ()           # the host BlockTables, in batch order
    starts_host: tuple = ()      # host copies of starts and context lengths
    lengths_host: tuple = ()
    plan: object = None          # engine.attention.PagedPlan of the step's paged launches, or None
    new_counts: tuple = ()       # new tokens per sequence (host)
    cache: dict = field(default_factory=dict, repr=False)  # device index tensors of ragged steps, built once

    @property
    def total_new(self) -> int:
        return sum(self.new_counts)

    @property
    def max_new(self) -> int:
        return max(self.new_counts + (0,))

    def plan_for(self, append: bool):
        """The step's paged-attention plan if it was built for a launch with
        (``append``) or without the fused append, else None."""
        if self.plan is not None and self.plan.key[-1] == append:
            return self.plan
        return None

    @property
    def fresh(self) -> bool:
        """Every sequence holds exactly this step's tokens (a prefill from
        position 0): attention needs only the new K/V, no history."""
        return all(s0 == 0 and n == c for s0, n, c in zip(self.starts_host, self.lengths_host, self.new_counts))

    @property
    def aligned(self) -> bool:
        """The new tokens are the newest of every sequence (start + count ==
        context length), so their positions are context_len - count + i, as
        the paged kernel's fused RoPE assumes."""
        return all(s0 + c == n for s0, n, c in zip(self.starts_host, self.lengths_host, self.new_counts))


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


def kv_append(k_new: torch.Tensor, v_new: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
              block_tables: torch.Tensor, cu_new: torch.Tensor, start: torch.Tensor,
              max_new: int, status: torch.Tensor | None = None, *,
              rope: tuple[torch.Tensor, torch.Tensor] | None = None,
              k_out: torch.Tensor | None = None) -> None:
    """Write new tokens of B sequences into one layer's pools on the GPU.

    k_new / v_new: (T, Hk, D); the rows of sequence b are
    ``cu_new[b] .. cu_new[b+1]-1`` (int32 (B+1,), device) and go to positions
    ``start[b] + i`` (int32 (B,), device) through ``block_tables`` (int32
    (B, max_blocks), device, already holding the needed blocks). ``max_new``
    bounds the per-sequence count. ``status`` (optional int32/uint32 (1,),
    device) gets 1 ORed in if a position or block id was out of range; those
    tokens are not written.

    ``rope``: (cos, sin) tables; k_new is then un-rotated and each K row is
    rotated at its position before it is written (bit-identical to
    ``rope_apply`` on k first); a position outside the tables writes neither
    K nor V of the token and ORs 2 into status. ``k_out`` (T, Hk, D) then
    also receives the rotated rows.
    """
    from engine import _lib

    for name, t in (("k_new", k_new), ("v_new", v_new), ("k_cache", k_cache), ("v_cache", v_cache),
                    ("block_tables", block_tables), ("cu_new", cu_new), ("start", start)):
        if not t.is_cuda or t.device != k_cache.device:
            raise RuntimeError(f"kv_append requires CUDA tensors on one device ({name})")
    if k_new.dtype != k_cache.dtype or v_new.dtype != k_cache.dtype or v_cache.dtype != k_cache.dtype:
        raise ValueError("kv_append: new tokens and pools must share a dtype")
    if k_new.dim() != 3 or tuple(v_new.shape) != tuple(k_new.shape):
        raise ValueError(f"kv_append expects k_new, v_new of shape (T, Hk, D), got {tuple(k_new.shape)}, "
                         f"{tuple(v_new.shape)}")
    nb, bs, Hk, D = k_cache.shape
    if tuple(v_cache.shape) != tuple(k_cache.shape) or k_new.shape[1:] != (Hk, D):
        raise ValueError(f"kv_append: pool {tuple(k_cache.shape)} does not match tokens {tuple(k_new.shape)}")
    if k_cache.dtype not in _lib.DTYPE_CODES:
        raise ValueError(f"attention kernels expect FP16 or BF16 Q/K/V, got {k_cache.dtype}")
    B = start.shape[0]
    bt = block_tables.to(torch.int32).contiguous()
    cu = cu_new.to(torch.int32).contiguous()
    st = start.to(torch.int32).contiguous()
    if bt.dim() != 2 or bt.shape[0] != B or cu.shape[0] != B + 1:
        raise ValueError("kv_append: block_tables must be (B, max_blocks) and cu_new (B + 1,)")
    if k_new.stride(-1) != 1 or v_new.stride(-1) != 1:
        k_new, v_new = k_new.contiguous(), v_new.contiguous()
    lib = _lib.load()
    args = (k_new.data_ptr(), v_new.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
            _lib.strides3(k_new), _lib.strides3(v_new), _lib.strides(k_cache), _lib.strides(v_cache),
            bt.data_ptr(), cu.data_ptr(), st.data_ptr(), status.data_ptr() if status is not None else None,
            B, k_new.shape[0], int(max_new), Hk, D, nb, bs, bt.shape[1], _lib.DTYPE_CODES[k_cache.dtype])
    if rope is None and k_out is not None:
        raise ValueError("kv_append: k_out is only written together with rope")
    with torch.cuda.device(k_cache.device):
        if rope is None:
            rc = lib.cie_kv_append(*args, _lib.stream_handle(k_cache.device))
        else:
            from engine.attention import rope_args

            out_p, out_st = None, None
            if k_out is not None:
                if not k_out.is_cuda or k_out.device != k_cache.device or k_out.dtype != k_cache.dtype \
                        or tuple(k_out.shape) != tuple(k_new.shape) or k_out.stride(-1) != 1:
                    raise ValueError(f"kv_append: k_out must match k_new {tuple(k_new.shape)} on the pool's device")
                out_p, out_st = k_out.data_ptr(), _lib.strides3(k_out)
            rc = lib.cie_kv_append_rope(*args, *rope_args(rope, D, k_cache.device), out_p, out_st,
                                        _lib.stream_handle(k_cache.device))
    _lib.check(rc)


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
        if L and self.device.type == "cuda":
            # one launch; block ids, row offsets and start travel in one small copy
            first = start // self.cfg.block_size
            ids = table.blocks[first:table.num_blocks_needed(end)]
            meta = torch.tensor(ids + [0, L, start % self.cfg.block_size], dtype=torch.int32).to(self.device)
            n = len(ids)
            kv_append(k, v, self.k[layer], self.v[layer], meta[:n].view(1, n), meta[n:n + 2], meta[n + 2:n + 3],
                      max_new=L)
        elif L:
            bs = self.cfg.block_size
            done = 0
            while done < L:
                bid, off = table.logical_to_physical(start + done)
                n = min(bs - off, L - done)
                self.k[layer][bid, off:off + n] = k[done:done + n]
                self.v[layer][bid, off:off + n] = v[done:done + n]
                done += n
        table.length = max(table.length, end)

    def prepare_step(self, tables: Sequence[BlockTable], num_new: int | Sequence[int],
                     starts: Sequence[int] | None = None, max_blocks: int | None = None, *,
                     num_heads: int | None = None, fused_append: bool | None = None) -> "StepBatch":
        """Host side of one engine step for a batch: allocate the blocks the
        ``num_new`` tokens of every sequence need (one count for all, or one
        per sequence for a ragged step; at ``starts[b]``, default each
        table's end), extend the lengths, and upload everything the step's
        kernels read (block tables, context lengths, the row offsets and
        start positions of the new tokens) in ONE host-to-device copy. Every
        layer's :meth:`append_step` and ``paged_attention`` of the step
        reuses it, so no layer touches the host.

        ``num_heads`` (the model's query heads): also build the work plan of
        the step's paged attention launches on the host (``cie_paged_plan``)
        and upload it in the same copy, so that no layer's launch derives
        its schedule on the device. ``fused_append``: plan for the launch
        with the append fused in (default: when the new tokens are the newest
        of every sequence, the case ``attention_section`` fuses)."""
        if self.device.type != "cuda":
            raise RuntimeError("prepare_step requires a CUDA cache")
        starts = [t.length for t in tables] if starts is None else list(starts)
        counts = [int(num_new)] * len(tables) if isinstance(num_new, int) else [int(c) for c in num_new]
        if len(starts) != len(tables) or len(counts) != len(tables) or any(c < 0 for c in counts) \
                or any(s < 0 for s in starts):
            raise ValueError(f"bad step: {len(tables)} tables, starts {starts}, new tokens {num_new}")
        uniform = len(set(counts)) <= 1
        num_new = counts[0] if counts and uniform else (0 if not counts else -1)
        for t, s0, c in zip(tables, starts, counts):
            while len(t.blocks) < t.num_blocks_needed(s0 + c):
                t.blocks.append(self._alloc_block())
            t.length = max(t.length, s0 + c)
        B = len(tables)
        width = max([len(t.blocks) for t in tables] + [1]) if max_blocks is None else max_blocks
        lengths = tuple(t.length for t in tables)
        max_context = max(lengths + (1,))
        o = B * width
        meta = o + 3 * B + 1
        n_plan = 0
        if num_heads is not None and num_new > 0:  # a plan covers one launch shape: uniform steps only
            from engine.attention import paged_plan_ints

            n_plan = paged_plan_ints(B, num_heads, self.cfg.num_kv_heads, num_new, self.cfg.head_dim,
                                     self.cfg.block_size, width, max_context)
        p0 = (meta + 3) // 4 * 4  # 16-byte aligned plan
        host = torch.zeros(p0 + n_plan if n_plan else meta, dtype=torch.int32)
        for i, t in enumerate(tables):
            if len(t.blocks) > width:
                raise ValueError(f"sequence {i} holds {len(t.blocks)} blocks, more than max_blocks={width}")
            if t.blocks:
                host[i * width:i * width + len(t.blocks)] = torch.tensor(t.blocks, dtype=torch.int32)
        host[o:o + B] = torch.tensor(lengths, dtype=torch.int32)
        cu = [0]
        for c in counts:
            cu.append(cu[-1] + c)
        host[o + B:o + 2 * B + 1] = torch.tensor(cu, dtype=torch.int32)
        host[o + 2 * B + 1:meta] = torch.tensor(starts, dtype=torch.int32)
        split = key = None
        if n_plan:
            from engine.attention import paged_plan_fill

            append = all(s0 + c == n for s0, n, c in zip(starts, lengths, counts)) if fused_append is None \
                else fused_append
            split, key = paged_plan_fill(host[p0:p0 + n_plan], host[o:o + B], host[:o].view(B, width),
                                         Hq=num_heads, Hk=self.cfg.num_kv_heads, Lq=num_new, D=self.cfg.head_dim,
                                         num_blocks=self.cfg.num_blocks, block_size=self.cfg.block_size,
                                         max_context=max_context, for_append=append)
        dev = host.to(self.device)
        plan = None
        if n_plan:
            from engine.attention import PagedPlan, _plan_fingerprint

            plan = PagedPlan(dev[p0:p0 + n_plan], split, key,
                             _plan_fingerprint(host[o:o + B], host[:o].view(B, width)))
        return StepBatch(block_tables=dev[:o].view(B, width), context_lens=dev[o:o + B],
                         cu_new=dev[o + B:o + 2 * B + 1], starts=dev[o + 2 * B + 1:meta], num_new=num_new,
                         max_context=max_context, tables=tuple(tables), starts_host=tuple(starts),
                         lengths_host=lengths, plan=plan, new_counts=tuple(counts))

    def append_step(self, layer: int, step: "StepBatch", k: torch.Tensor, v: torch.Tensor, *,
                    rope: tuple[torch.Tensor, torch.Tensor] | None = None,
                    k_out: torch.Tensor | None = None) -> None:
        """Write one layer's new K/V rows of a prepared step: k, v are
        (total new tokens, Hk, D), the rows of sequence b consecutive. One
        ``cie_kv_append`` launch; no host work, no host-to-device copy, so a
        step's layers can be captured in one HIP graph. ``rope`` / ``k_out``
        as in :func:`kv_append` (K rotated at its position on the way in)."""
        self._validate(k)
        self._validate(v)
        if k.shape[0] != step.total_new or v.shape[0] != k.shape[0]:
            raise ValueError(f"append_step expects {step.total_new} rows, got {k.shape[0]}, {v.shape[0]}")
        kv_append(k, v, self.k[layer], self.v[layer], step.block_tables, step.cu_new, step.starts,
                  max_new=step.max_new, rope=rope, k_out=k_out)

    def append_batch(self, layer: int, tables: Sequence[BlockTable], k: torch.Tensor, v: torch.Tensor,
                     lengths: Sequence[int], starts: Sequence[int] | None = None,
                     block_tables: torch.Tensor | None = None) -> None:
        """``append`` for many sequences in one launch: k, v are (T, Hk, D)
        with the rows of ``tables[b]`` consecutive (``lengths[b]`` of them),
        written at ``starts[b]`` (default: each table's end). Blocks are
        allocated on the host first; ``block_tables`` (the device table of
        ``block_table_tensor``, e.g. shared by all layers of a step) is built
        when not given."""
        self._validate(k)
        self._validate(v)
        if self.device.type != "cuda":
            raise RuntimeError("append_batch requires a CUDA cache")
        starts = [t.length for t in tables] if starts is None else list(starts)
        for t, s0, n in zip(tables, starts, lengths):
            while len(t.blocks) < t.num_blocks_needed(s0 + n):
                t.blocks.append(self._alloc_block())
        if block_tables is None:
            block_tables, _ = block_table_tensor(tables, self.device)
        cu = [0]
        for n in lengths:
            cu.append(cu[-1] + n)
        meta = torch.tensor(cu + starts, dtype=torch.int32).to(self.device)
        B = len(tables)
        kv_append(k, v, self.k[layer], self.v[layer], block_tables, meta[:B + 1], meta[B + 1:],
                  max_new=max(list(lengths) + [0]))
        for t, s0, n in zip(tables, starts, lengths):
            t.length = max(t.length, s0 + n)

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
