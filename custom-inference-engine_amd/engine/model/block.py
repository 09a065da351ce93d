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
* decode / verify ((Hq/Hk) * L <= 256 query rows per kv head): one rotary
  append, then paged attention reading K/V in place with q rotated as it
  is loaded;
* anything else (a long chunk on top of a history): the rotary append,
  then the reference's own structure per sequence on the GPU kernels
  (gather, prefill attention).

The Q/K/V projections and the output projection around it are unchanged.
"""

from __future__ import annotations

import math

import torch

from engine.attention import flash_attention, paged_attention
from engine.cache import PagedKVCache, StepBatch

_PAGED_MAX_ROWS = 256  # query rows per kv head one paged launch takes


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
    elif (Hq // Hk) * L <= _PAGED_MAX_ROWS and fuse_append and step.aligned:
        cache._validate(k_rows)
        cache._validate(v_rows)
        paged_attention(q, cache.k[layer_idx], cache.v[layer_idx], step.block_tables, step.context_lens,
                        causal=True, scale=scale, max_context=step.max_context, rope=rope, out=out,
                        new_kv=(k_rows, v_rows), plan=step.plan_for(True))
    elif (Hq // Hk) * L <= _PAGED_MAX_ROWS:
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
        if rope is not None:
            from engine.model.rope import rope_apply

            pos = step.starts[:, None] + torch.arange(L, device=q.device, dtype=torch.int32)[None, :]
            q = rope_apply(q, rope[0], rope[1], positions=pos)
        for b, t in enumerate(step.tables):
            kd, vd = cache.gather(layer_idx, t)
            flash_attention(q[b:b + 1], kd.transpose(0, 1).unsqueeze(0), vd.transpose(0, 1).unsqueeze(0),
                            causal=True, scale=scale, out=out[b:b + 1])
    return out_rows.view(B, L, Hq * D)
