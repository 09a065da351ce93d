"""The reference's end-to-end parity contracts, restated at the level of the
attention section (the part of the model this library replaces).

The reference checks them on a whole model:

* tests/model/test_transformer_forward.py:32-46 -- feeding the tokens one
  at a time through the KV cache gives the last-step logits of feeding them
  all at once (atol 1e-3);
* tests/decode/test_speculative.py:25-37 -- speculative decoding gives
  exactly the base loop's tokens, which exercises a verify of gamma + 1
  tokens, the rollback of the rejected ones (engine/cache/kv_cache.py:
  187-194) and the next verify writing over the rolled-back positions.

Here the "model" is two attention sections chained by fixed random
projections (q, k, v from the hidden rows, a residual output projection),
RoPE on, as engine/model/block.py:44-75 chains them per layer: the same
token rows must come out of every schedule -- one prefill, single-token
steps, chunked steps, and verify / rollback / re-verify -- within the
tolerance of the dtype (the schedules run different kernels: the prefill
kernel over the new tokens, the paged kernel over the pool with the append
fused in). The projections run in fp32 and round to the activation dtype,
as the reference's half-precision linears do.
"""

from __future__ import annotations

import math

import pytest
import torch

from engine.cache import KVCacheConfig, PagedKVCache
from engine.model import attention_section
from engine.model.rope import build_rope_cache
from oracle import flash_attention_ref
from oracle.rope_ref import rope_ref

pytestmark = pytest.mark.gpu
DEV = "cuda"
Hq, Hk, D, LAYERS, BS = 8, 2, 64, 2, 16
HID = Hq * D
TOL = {torch.float16: 2e-3, torch.bfloat16: 1e-2}


class TwoLayerSections:
    """Token embeddings and per-layer projections (fixed by a seed); a forward
    of some new tokens of every sequence through both layers' sections."""

    def __init__(self, dtype, seed=0, vocab=97):
        g = torch.Generator().manual_seed(seed)
        s = 1.0 / math.sqrt(HID)
        self.dtype = dtype
        # hidden rows of size ~0.1 (so that one rounding step of the residual
        # stays far below the tolerance), q and k of size ~1 (scores of
        # standard deviation ~1, as in the seeded workloads), v ~0.1
        self.emb = (torch.randn(vocab, HID, generator=g) * 0.1).to(DEV)
        self.w = [[(torch.randn(HID, n, generator=g) * (s * f)).to(DEV)
                   for n, f in ((Hq * D, 10.0), (Hk * D, 10.0), (Hk * D, 1.0), (HID, 1.0))]
                  for _ in range(LAYERS)]
        cos, sin = build_rope_cache(512, D)
        self.rope = (cos.to(DEV), sin.to(DEV))

    def cache(self, num_blocks=64):
        return PagedKVCache(KVCacheConfig(LAYERS, Hk, D, num_blocks, BS, self.dtype, DEV))

    def forward(self, tokens, cache, tables, plan=False):
        """tokens: (B, L) ids, the next L tokens of every sequence. Returns
        the last layer's hidden rows (B, L, HID) in the activation dtype."""
        B, L = tokens.shape
        step = cache.prepare_step(tables, L, num_heads=Hq if plan else None)
        x = self.emb[tokens.to(DEV)].to(self.dtype)
        for layer, (wq, wk, wv, wo) in enumerate(self.w):
            xf = x.float()
            q = (xf @ wq).to(self.dtype).view(B, L, Hq, D).transpose(1, 2)
            k = (xf @ wk).to(self.dtype).view(B, L, Hk, D).transpose(1, 2)
            v = (xf @ wv).to(self.dtype).view(B, L, Hk, D).transpose(1, 2)
            a = attention_section(q, k, v, layer, cache, step, rope=self.rope)
            x = (xf + a.float() @ wo).to(self.dtype)
        return x

    def forward_ref(self, tokens):
        """The same two layers for whole sequences (B, N) from position 0, on
        the CPU oracle: RoPE by the restated reference, fp32 attention."""
        B, N = tokens.shape
        cos, sin = (t.cpu() for t in self.rope)
        x = self.emb[tokens.to(DEV)].to(self.dtype).cpu()
        for wq, wk, wv, wo in self.w:
            wq, wk, wv, wo = (w.cpu() for w in (wq, wk, wv, wo))
            xf = x.float()
            q = (xf @ wq).to(self.dtype).view(B, N, Hq, D).transpose(1, 2)
            k = (xf @ wk).to(self.dtype).view(B, N, Hk, D).transpose(1, 2)
            v = (xf @ wv).to(self.dtype).view(B, N, Hk, D).transpose(1, 2)
            pos = torch.arange(N)
            q, k = rope_ref(q, cos, sin, pos), rope_ref(k, cos, sin, pos)
            a = flash_attention_ref(q, k, v, causal=True).transpose(1, 2).reshape(B, N, HID)
            x = (xf + a.float() @ wo).to(self.dtype)
        return x


def _close(a, b, tol, what, ulps=0):
    """max |a - b| <= tol, plus ``ulps`` units in the last place of b's
    dtype per element (for values that are the rounded output of a
    projection of inputs that already differ within tol)."""
    a, b32 = a.float().cpu(), b.float().cpu()
    rel = ulps * {torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}.get(b.dtype, 0.0)
    excess = (a - b32).abs() - tol - rel * b32.abs()
    err = float((a - b32).abs().max())
    assert float(excess.max()) <= 0, f"{what}: max abs difference {err:.3e} > {tol:.1e} (+{ulps} ulp)"
    return err


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("plan", [False, True])
def test_incremental_steps_match_one_prefill(dtype, plan):
    """tests/model/test_transformer_forward.py:32-46 at the section level:
    40 tokens of two sequences fed at once, one at a time, and as a
    25-token prefill followed by three 5-token steps give the same rows
    (checked on every row of the last layer, not only the last)."""
    model = TwoLayerSections(dtype, seed=1)
    g = torch.Generator().manual_seed(2)
    N = 40
    tokens = torch.randint(0, 97, (2, N), generator=g)

    cache = model.cache()
    tables = [cache.new_sequence() for _ in range(2)]
    full = model.forward(tokens, cache, tables, plan)
    assert [t.length for t in tables] == [N, N]
    _close(full, model.forward_ref(tokens), TOL[dtype], "one prefill against the oracle")

    cache = model.cache()
    tables = [cache.new_sequence() for _ in range(2)]
    inc = torch.cat([model.forward(tokens[:, i:i + 1], cache, tables, plan) for i in range(N)], dim=1)
    _close(inc, full, TOL[dtype], "single-token steps")

    cache = model.cache()
    tables = [cache.new_sequence() for _ in range(2)]
    parts = [model.forward(tokens[:, :25], cache, tables, plan)]
    parts += [model.forward(tokens[:, i:i + 5], cache, tables, plan) for i in (25, 30, 35)]
    _close(torch.cat(parts, dim=1), full, TOL[dtype], "prefill then 5-token steps")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("plan", [False, True])
def test_verify_rollback_reverify_equals_fresh_prefill(dtype, plan):
    """tests/decode/test_speculative.py:25-37 at the section level: after a
    46-token prefill, a verify of gamma + 1 = 4 draft tokens (positions
    46..49, across a block boundary), a rollback to the accepted prefix
    (sequence 0 keeps 2 of them, sequence 1 all 4; engine/cache/kv_cache.py:
    187-194 frees the block past it) and a second verify of 4 new tokens
    that writes over the rolled-back positions must give the rows a fresh
    prefill of the final sequences gives, and leave the same K / V in the
    pool at every live position."""
    model = TwoLayerSections(dtype, seed=3)
    g = torch.Generator().manual_seed(4)
    P = 46
    prompt = torch.randint(0, 97, (2, P), generator=g)
    draft1 = torch.randint(0, 97, (2, 4), generator=g)
    draft2 = torch.randint(0, 97, (2, 4), generator=g)
    accepted = [2, 4]

    cache = model.cache(num_blocks=12)
    tables = [cache.new_sequence() for _ in range(2)]
    model.forward(prompt, cache, tables, plan)
    model.forward(draft1, cache, tables, plan)  # verify: positions 46..49
    assert [len(t.blocks) for t in tables] == [4, 4]
    free_before = len(cache._free)
    for t, a in zip(tables, accepted):
        cache.rollback(t, P + a)
    assert [t.length for t in tables] == [48, 50] and [len(t.blocks) for t in tables] == [3, 4]
    assert len(cache._free) == free_before + 1  # sequence 0's fourth block went back to the free list
    # the second verify starts at each sequence's accepted length; sequence 0
    # rewrites positions 48.. (its rolled-back block comes back from the free list)
    out = model.forward(draft2, cache, tables, plan)

    finals = [torch.cat([prompt[b], draft1[b, :accepted[b]], draft2[b]]) for b in range(2)]
    for b in range(2):
        ref_cache = model.cache()
        ref_tables = [ref_cache.new_sequence()]
        fresh = model.forward(finals[b][None], ref_cache, ref_tables, plan)
        n = finals[b].numel()
        _close(out[b], fresh[0, n - 4:], TOL[dtype], f"re-verify rows of sequence {b}")
        # live K / V of every layer equal the fresh prefill's
        for layer in range(LAYERS):
            for pool, ref_pool in ((cache.k[layer], ref_cache.k[layer]), (cache.v[layer], ref_cache.v[layer])):
                got = torch.cat([pool[i] for i in tables[b].blocks]).reshape(-1, Hk, D)[:n]
                want = torch.cat([ref_pool[i] for i in ref_tables[0].blocks]).reshape(-1, Hk, D)[:n]
                if layer == 0:  # layer 0's K / V depend on the token embeddings alone: bit for bit
                    assert torch.equal(got, want), (b, layer)
                else:  # projections of layer inputs equal within the tolerance: two ulps of slack
                    _close(got, want, TOL[dtype], f"layer {layer} pool of sequence {b}", ulps=2)
