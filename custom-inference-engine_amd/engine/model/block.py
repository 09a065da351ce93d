"""The attention section of the reference's ``Attention.forward``
(``engine/model/block.py:53-75``) on the paged path, for a batch.

The reference, per layer and for one sequence (``B == 1`` is asserted at
``block.py:48``): rotates q and k at ``positions`` (``:53-54``), appends
the rotated k and v at ``positions[0]`` (``:57-64``), gathers the whole
history into dense tensors (``:65-67``, ``kv_cache.py:141-165``), runs
causal ``flash_attention`` with scale ``1/sqrt(head_dim)`` (``:69-71``) and
returns ``(1, L, Hq * D)`` (``:72-74``) for the output projection.
:func:`attention_section` does the same for B sequences of L new tokens
each, with RoPE fused into the kernels when the model's tables are given:

* a prefill of fresh sequences (every history is just the new tokens):
  one rotary append that also returns the rotated K densely, then prefill
  attention over the new tokens with q rotated as it is loaded;
* decode / verify ((Hq/Hk) * L <= 256 query rows per kv head, 128 at
  head_dim 256: ``paged_max_rows``): one rotary append, then paged attention
  reading K/V in place with q rotated as it is loaded;
* a long chunk on top of a history (more query rows per kv head): the rotary
  append, then paged attention in launches of at most that many rows per kv
  head (see below) -- the history is never gathered.

:func:`attention_section_rows` takes a ragged step (a different number of
new tokens per sequence, e.g. a prefill chunk next to decode tokens) as
packed rows: one append for all, then paged attention per group of
sequences with equal counts, long groups again split into launches.

Splitting is exact: the Lq new tokens of a sequence of context length ctx
sit at positions ctx - Lq .. ctx - 1 (the reference appends before it
attends, block.py:57-65), and row i sees keys <= ctx - Lq + i. Rows i0 ..
i1 - 1 alone are the i1 - i0 newest tokens of a context of length
ctx - Lq + i1, for which the paged kernel's rule and RoPE positions give
the same keys and positions.

The Q/K/V projections and the output projection around it are unchanged.
"""

from __future__ import annotations

import math

import torch

from engine.attention import flash_attention, paged_attention, paged_max_rows
from engine.cache import PagedKVCache, StepBatch


def attention_section(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, layer_idx: int, cache: PagedKVCache,
                      step: StepBatch, rope: tuple[torch.Tensor, torch.Tensor] | None = None,
                      fuse_append: bool = True) -> torch.Tensor:
    """q: (B, Hq, L, D), k/v: (B, Hk, L, D): the L new tokens of each
    sequence, at positions ``starts[b] + 0..L-1``, after RoPE when ``rope``
    is None, before it when ``rope`` is the model's (cos, sin) tables
    (``RotaryEmbedding.tables``). ``step`` is ``cache.prepare_step(tables,
    L, starts)``, made once per engine step before the first layer: it
    allocates the blocks, extends the lengths (so the history includes the
    new tokens, as in the reference, which appends before it attends) and
    holds the step's device metadata. Returns (B, L, Hq * D).

    With ``fuse_append`` (default) a step whose new tokens are the newest of
    every sequence appends inside the paged attention launch pair
    (``paged_attention(new_kv=..., rope=rope)``), bit-identical to
    ``append_step`` followed by ``paged_attention``."""
    B, Hq, L, D = q.shape
    if step.context_lens.shape[0] != B or k.shape[0] != B or v.shape[0] != B or step.num_new != L:
        raise ValueError(f"step of {step.context_lens.shape[0]} sequences x {step.num_new} tokens "
                         f"for q of shape {tuple(q.shape)}")
    Hk = k.shape[1]
    scale = 1.0 / math.sqrt(D)
    # the kernels write (B, L, Hq, D) directly: the reference's
    # transpose(1, 2).contiguous() of the output (block.py:72-74) is free
    out_rows = torch.empty((B, L, Hq, D), dtype=q.dtype, device=q.device)
    out = out_rows.transpose(1, 2)
    # the rows of sequence b are consecutive in (B*L, Hk, D)
    k_rows = k.transpose(1, 2).reshape(B * L, Hk, D)
    v_rows = v.transpose(1, 2).reshape(B * L, Hk, D)

    if step.fresh:
        # history == the new tokens: attend over them directly (the gathered
        # history of the reference is bit-identical to them)
        if rope is None:
            cache.append_step(layer_idx, step, k_rows, v_rows)
            flash_attention(q, k, v, causal=True, scale=scale, out=out)
        else:
            k_rot = torch.empty_like(k_rows)
            cache.append_step(layer_idx, step, k_rows, v_rows, rope=rope, k_out=k_rot)
            flash_attention(q, k_rot.view(B, L, Hk, D).transpose(1, 2), v, causal=True, scale=scale, rope=rope,
                            out=out)  # positions 0..L-1
    elif (Hq // Hk) * L <= paged_max_rows(D) and fuse_append and step.aligned:
        cache._validate(k_rows)
        cache._validate(v_rows)
        paged_attention(q, cache.k[layer_idx], cache.v[layer_idx], step.block_tables, step.context_lens,
                        causal=True, scale=scale, max_context=step.max_context, rope=rope, out=out,
                        new_kv=(k_rows, v_rows), plan=step.plan_for(True))
    elif (Hq // Hk) * L <= paged_max_rows(D):
        cache.append_step(layer_idx, step, k_rows, v_rows, rope=rope)
        q_rope = rope
        if rope is not None and not step.aligned:
            # positions start + i differ from context_len - L + i: rotate q first
            from engine.model.rope import rope_apply

            pos = step.starts[:, None] + torch.arange(L, device=q.device, dtype=torch.int32)[None, :]
            q, q_rope = rope_apply(q, rope[0], rope[1], positions=pos), None
        paged_attention(q, cache.k[layer_idx], cache.v[layer_idx], step.block_tables, step.context_lens,
                        causal=True, scale=scale, max_context=step.max_context, rope=q_rope, out=out,
                        plan=step.plan_for(False))
    else:
        cache.append_step(layer_idx, step, k_rows, v_rows, rope=rope)
        _paged_rows(q.transpose(1, 2).reshape(B * L, Hq, D), layer_idx, cache, step, rope,
                    out_rows.view(B * L, Hq, D))
    return out_rows.view(B, L, Hq * D)


def attention_section_rows(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, layer_idx: int,
                           cache: PagedKVCache, step: StepBatch,
                           rope: tuple[torch.Tensor, torch.Tensor] | None = None) -> torch.Tensor:
    """The attention section for a step of any shape, ragged ones included:
    q (T, Hq, D), k / v (T, Hk, D) hold the new tokens of all sequences as
    packed rows, sequence b's ``step.new_counts[b]`` rows consecutive (the
    layout of ``step.cu_new``), at positions ``starts[b] + i``, un-rotated
    when ``rope`` is given. ``step`` is ``cache.prepare_step(tables,
    counts)``. Returns (T, Hq * D), row for row. One append for every
    sequence, then paged attention per group of sequences with equal
    counts, in launches of at most ``paged_max_rows(D)`` query rows per kv
    head."""
    T, Hq, D = q.shape
    Hk = k.shape[1]
    if T != step.total_new or k.shape[0] != T or v.shape[0] != T or k.shape[1:] != (Hk, D) \
            or tuple(v.shape) != tuple(k.shape):
        raise ValueError(f"step of {step.total_new} new tokens for q {tuple(q.shape)}, k {tuple(k.shape)}, "
                         f"v {tuple(v.shape)}")
    out = torch.empty((T, Hq, D), dtype=q.dtype, device=q.device)
    cache.append_step(layer_idx, step, k, v, rope=rope)
    _paged_rows(q, layer_idx, cache, step, rope, out)
    return out.view(T, Hq * D)


def _paged_rows(q_rows: torch.Tensor, layer_idx: int, cache: PagedKVCache, step: StepBatch,
                rope: tuple[torch.Tensor, torch.Tensor] | None, out_rows: torch.Tensor) -> None:
    """Paged attention of the packed new-token rows of ``step`` (already
    appended) over each sequence's history, into ``out_rows`` (T, Hq, D).
    Sequences are grouped by their count of new tokens; a group's tokens go
    in chunks of at most ``paged_max_rows(D) // (Hq / Hk)`` per launch, chunk
    [i0, i1) as the newest tokens of a context of length ctx - count + i1.
    The device index tensors of each launch are built on the first call of
    the step and reused by every layer."""
    T, Hq, D = q_rows.shape
    Hk = cache.cfg.num_kv_heads
    scale = 1.0 / math.sqrt(D)
    dev = q_rows.device
    if rope is not None and not step.aligned:
        # positions start + i differ from context_len - count + i: rotate q first
        from engine.model.rope import rope_apply

        key = ("positions",)
        if key not in step.cache:
            pos = [s0 + i for s0, c in zip(step.starts_host, step.new_counts) for i in range(c)]
            step.cache[key] = torch.tensor(pos, dtype=torch.int32).to(dev)
        q_rows = rope_apply(q_rows.transpose(0, 1).unsqueeze(0), rope[0], rope[1],
                            positions=step.cache[key])[0].transpose(0, 1)
        rope = None
    chunk = max(1, paged_max_rows(D) // (Hq // Hk))
    key = ("launches", chunk)
    if key not in step.cache:
        step.cache[key] = _launches(step, chunk, dev)
    for tables, rows, lens, Lsub in step.cache[key]:
        qs = q_rows[rows].view(-1, Lsub, Hq, D).transpose(1, 2)
        o = paged_attention(qs, cache.k[layer_idx], cache.v[layer_idx], tables, lens,
                            causal=True, scale=scale, max_context=step.max_context, rope=rope)
        out_rows[rows] = o.transpose(1, 2).reshape(-1, Hq, D)


def _launches(step: StepBatch, chunk: int, dev: torch.device) -> list:
    """(block tables (B', max_blocks), packed row indices (B' * Lsub,),
    context lengths (B',), Lsub) of every launch of a step; the indices are
    uploaded in one copy."""
    groups: dict[int, list[int]] = {}
    for b, c in enumerate(step.new_counts):
        if c > 0:
            groups.setdefault(c, []).append(b)
    cu = [0]
    for c in step.new_counts:
        cu.append(cu[-1] + c)
    parts, shapes = [], []
    for c, seqs in sorted(groups.items()):
        for i0 in range(0, c, chunk):
            i1 = min(c, i0 + chunk)
            rows = [cu[b] + i for b in seqs for i in range(i0, i1)]
            lens = [step.lengths_host[b] - c + i1 for b in seqs]
            parts += [seqs, rows, lens]
            shapes.append((len(seqs), i1 - i0))
    if not shapes:
        return []
    flat = torch.tensor([x for part in parts for x in part], dtype=torch.int64).to(dev)
    out, p = [], 0
    for n, Lsub in shapes:
        tables = step.block_tables[flat[p:p + n]]
        rows = flat[p + n:p + n + n * Lsub]
        lens = flat[p + n + n * Lsub:p + 2 * n + n * Lsub].to(torch.int32)
        out.append((tables, rows, lens, Lsub))
        p += 2 * n + n * Lsub
    return out
