"""The attention section of the reference's ``Attention.forward``
(``engine/model/block.py:56-75``) on the paged path, for a batch.

The reference, per layer and for one sequence (``B == 1`` is asserted at
``block.py:48``): appends the rotated k, v of the new tokens at
``positions[0]`` (``:57-64``), gathers the whole history into dense tensors
(``:65-67``, ``kv_cache.py:141-165``), runs causal ``flash_attention`` with
scale ``1/sqrt(head_dim)`` (``:69-71``) and returns ``(1, L, Hq * D)``
(``:72-74``) for the output projection. :func:`attention_section` does the
same for B sequences with one ``cie_kv_append`` launch and one paged
attention launch that reads K/V in place; the Q/K/V projections, RoPE and the
output projection around it are unchanged.
"""

from __future__ import annotations

import math
from typing import Sequence

import torch

from engine.attention import paged_attention
from engine.cache import BlockTable, PagedKVCache


def attention_section(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, layer_idx: int, cache: PagedKVCache,
                      tables: Sequence[BlockTable], starts: Sequence[int],
                      step_tables: tuple[torch.Tensor, torch.Tensor]) -> torch.Tensor:
    """q: (B, Hq, L, D), k/v: (B, Hk, L, D), after RoPE: the L new tokens of
    each sequence, at positions ``starts[b] + 0..L-1``. ``step_tables`` is
    ``cache.prepare_step(tables, L, starts)``, made once per engine step
    before the first layer (it allocates the blocks and extends the lengths,
    so the history includes the new tokens as in the reference, which appends
    before it attends). Returns (B, L, Hq * D)."""
    B, Hq, L, D = q.shape
    if len(tables) != B or k.shape[0] != B or v.shape[0] != B:
        raise ValueError(f"{len(tables)} block tables for q of batch {B}")
    Hk = k.shape[1]
    bt, lens = step_tables
    # append (block.py:57-64): the rows of sequence b are consecutive in (B*L, Hk, D)
    k_rows = k.transpose(1, 2).reshape(B * L, Hk, D)
    v_rows = v.transpose(1, 2).reshape(B * L, Hk, D)
    cache.append_batch(layer_idx, tables, k_rows, v_rows, [L] * B, starts=starts, block_tables=bt)
    # attend in place (replaces gather + flash_attention, block.py:65-71)
    max_ctx = max([t.length for t in tables] + [1])
    out = paged_attention(q, cache.k[layer_idx], cache.v[layer_idx], bt, lens, causal=True,
                          scale=1.0 / math.sqrt(D), max_context=max_ctx)
    # (block.py:72-74)
    return out.transpose(1, 2).reshape(B, L, Hq * D)
