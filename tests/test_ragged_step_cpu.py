"""Host logic of the ragged / long-step attention section on the CPU.

attention_section_rows and the long-chunk branch of attention_section run
paged attention per group of sequences with equal counts of new tokens, in
launches of at most 256 query rows per kv head: chunk [i0, i1) of a
sequence's c new tokens is launched as the i1 - i0 newest tokens of a
context of length ctx - c + i1. Checked here:

* the launch list covers every new-token row exactly once, with the block
  table row of its own sequence and that context length;
* the splitting identity itself on the oracle: the chunks' causal attention
  (the reference's bottom-right mask, kernels/ref/flash_attention_ref.py:
  35-39) equals the whole block's, row for row -- a wrong length (ctx - c +
  i0, or ctx) fails it."""

from __future__ import annotations

import pytest
import torch

from engine.cache import StepBatch
from engine.model.block import _launches
from oracle import flash_attention_ref


def _step(counts, lengths, width=4):
    B = len(counts)
    bt = torch.arange(B * width, dtype=torch.int32).view(B, width)
    cu = [0]
    for c in counts:
        cu.append(cu[-1] + c)
    return StepBatch(block_tables=bt, context_lens=torch.tensor(lengths, dtype=torch.int32),
                     cu_new=torch.tensor(cu, dtype=torch.int32),
                     starts=torch.tensor([n - c for n, c in zip(lengths, counts)], dtype=torch.int32),
                     num_new=-1, max_context=max(lengths), starts_host=tuple(n - c for n, c in zip(lengths, counts)),
                     lengths_host=tuple(lengths), new_counts=tuple(counts))


@pytest.mark.parametrize("counts,chunk", [([300, 1, 1, 0, 5, 700, 64, 1], 64), ([4, 4, 4], 256), ([1], 1),
                                          ([129, 128, 127, 0], 32), ([0, 0], 8)])
def test_launches_cover_every_row_once(counts, chunk):
    lengths = [c + 37 * b for b, c in enumerate(counts)]
    step = _step(counts, lengths)
    launches = _launches(step, chunk, torch.device("cpu"))
    cu = [0]
    for c in counts:
        cu.append(cu[-1] + c)
    seen = {}
    for tables, rows, lens, Lsub in launches:
        assert 1 <= Lsub <= chunk and rows.numel() == tables.shape[0] * Lsub == lens.shape[0] * Lsub
        for j in range(tables.shape[0]):
            b = int(tables[j, 0]) // 4
            assert torch.equal(tables[j], step.block_tables[b])
            r = rows[j * Lsub:(j + 1) * Lsub].tolist()
            i1 = r[-1] - cu[b] + 1
            assert r == list(range(cu[b] + i1 - Lsub, cu[b] + i1))  # consecutive rows of sequence b
            assert int(lens[j]) == lengths[b] - counts[b] + i1
            for x in r:
                seen[x] = seen.get(x, 0) + 1
    assert sorted(seen) == list(range(sum(counts))) and all(n == 1 for n in seen.values())
    # one launch per (count, chunk) pair
    assert len(launches) == sum(-(-c // chunk) for c in set(counts) if c)


@pytest.mark.parametrize("c,hist,chunk", [(300, 200, 64), (97, 0, 32), (5, 1000, 2)])
def test_chunked_causal_rows_equal_the_whole_block(c, hist, chunk):
    g = torch.Generator().manual_seed(c)
    ctx = hist + c
    q = torch.randn(1, 4, c, 32, generator=g)
    k = torch.randn(1, 2, ctx, 32, generator=g)
    v = torch.randn(1, 2, ctx, 32, generator=g)
    whole = flash_attention_ref(q, k, v, causal=True)
    parts = []
    for i0 in range(0, c, chunk):
        i1 = min(c, i0 + chunk)
        n = ctx - c + i1  # the chunk's context length
        parts.append(flash_attention_ref(q[:, :, i0:i1], k[:, :, :n], v[:, :, :n], causal=True))
    assert torch.allclose(torch.cat(parts, dim=2), whole, atol=1e-6, rtol=0)
    # a planted mistake: the chunk's length taken as ctx - c + i0 shifts every mask by the chunk size
    i0, i1 = 0, min(c, chunk)
    wrong = flash_attention_ref(q[:, :, i0:i1], k[:, :, :ctx - c + i0 + 1], v[:, :, :ctx - c + i0 + 1],
                                causal=True)
    if i1 - i0 > 1:
        assert not torch.allclose(wrong.nan_to_num(9.0), whole[:, :, i0:i1], atol=1e-3)
