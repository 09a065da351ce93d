"""Pins the CPU oracle before anything is checked against it.

Each oracle function is checked against something other than itself:
* the reference's own known-answer tests for this path
  (tests/kernels/test_flash_attention_ref.py:11-39,
  tests/cache/test_block_table.py:8-13);
* the fp64 brute force (independent construction: loops, explicit max-shifted
  exponentials, no matmul / softmax routine);
* torch's scaled_dot_product_attention with an explicit bottom-right mask;
* closed forms (GQA head mapping, bottom-right alignment, scale, row sums,
  row 0 of a causal prefill, decode == last prefill row);
* planted mistakes in copies of the oracle, which at least one check must catch.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import (
    attention_brute_f64,
    attention_rows_ref,
    flash_attention_ref,
    flash_attention_ref_chunked,
    gather_ref,
    logical_to_physical_ref,
    paged_attention_brute_f64,
    paged_attention_ref,
)


def _same(a, b, atol):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    assert a.shape == b.shape
    na, nb = np.isnan(a), np.isnan(b)
    assert (na == nb).all(), "NaN pattern differs"
    if (~na).any():
        assert np.abs(a[~na] - b[~na]).max() <= atol


# ---------------------------------------------------------------- reference known answers

@pytest.mark.parametrize("B,H,Lq,Lk,D", [(1, 2, 4, 4, 8), (2, 4, 8, 16, 16)])
def test_matches_manual_softmax(B, H, Lq, Lk, D):
    torch.manual_seed(0)
    q, k, v = torch.randn(B, H, Lq, D), torch.randn(B, H, Lk, D), torch.randn(B, H, Lk, D)
    out = flash_attention_ref(q, k, v)
    expected = torch.softmax(q @ k.transpose(-2, -1) / math.sqrt(D), dim=-1) @ v
    assert torch.allclose(out, expected, atol=1e-5)


def test_causal_mask_blocks_future():
    torch.manual_seed(0)
    q, k, v = torch.randn(1, 1, 4, 8), torch.randn(1, 1, 4, 8), torch.randn(1, 1, 4, 8)
    assert not torch.allclose(flash_attention_ref(q, k, v), flash_attention_ref(q, k, v, causal=True))


def test_gqa_broadcast_shape():
    out = flash_attention_ref(torch.randn(1, 4, 3, 8), torch.randn(1, 2, 3, 8), torch.randn(1, 2, 3, 8))
    assert out.shape == (1, 4, 3, 8)


def test_block_table_known_answers():
    blocks = [10, 11, 12]
    assert logical_to_physical_ref(blocks, 4, 0) == (10, 0)
    assert logical_to_physical_ref(blocks, 4, 3) == (10, 3)
    assert logical_to_physical_ref(blocks, 4, 4) == (11, 0)
    assert logical_to_physical_ref(blocks, 4, 8) == (12, 0)


# ---------------------------------------------------------------- brute force and library

CASES = [
    # B, H, Hk, Lq, Lk, D, causal
    (1, 2, 2, 4, 4, 16, True),
    (2, 4, 2, 3, 9, 16, True),    # Lq < Lk: prefill over a cache
    (1, 4, 1, 5, 5, 8, False),
    (2, 6, 3, 1, 7, 16, True),    # decode row
    (1, 4, 2, 6, 3, 16, True),    # Lq > Lk: first rows see nothing -> NaN
    (1, 2, 1, 3, 0, 16, True),    # empty history -> zeros
    (1, 2, 2, 2, 11, 32, False),
]


@pytest.mark.parametrize("B,H,Hk,Lq,Lk,D,causal", CASES)
def test_ref_matches_brute_f64(B, H, Hk, Lq, Lk, D, causal):
    g = torch.Generator().manual_seed(B * 100 + Lq * 10 + Lk)
    q = torch.randn(B, H, Lq, D, generator=g)
    k = torch.randn(B, Hk, Lk, D, generator=g)
    v = torch.randn(B, Hk, Lk, D, generator=g)
    _same(flash_attention_ref(q, k, v, causal=causal), attention_brute_f64(q, k, v, causal=causal), 2e-6)
    _same(flash_attention_ref_chunked(q, k, v, causal=causal, q_chunk=2),
          attention_brute_f64(q, k, v, causal=causal), 2e-6)


@pytest.mark.parametrize("Lq,Lk", [(7, 7), (3, 12), (1, 5)])
def test_ref_matches_sdpa_bottom_right(Lq, Lk):
    g = torch.Generator().manual_seed(7)
    q = torch.randn(2, 8, Lq, 32, generator=g)
    k = torch.randn(2, 2, Lk, 32, generator=g)
    v = torch.randn(2, 2, Lk, 32, generator=g)
    i = torch.arange(Lq).unsqueeze(-1)
    j = torch.arange(Lk).unsqueeze(0)
    allowed = j <= (Lk - Lq + i)
    lib = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=allowed, enable_gqa=True)
    assert torch.allclose(flash_attention_ref(q, k, v, causal=True), lib, atol=1e-5)


@pytest.mark.parametrize("Lq,Lk,causal", [(9, 9, True), (4, 13, True), (7, 3, True), (5, 8, False), (3, 0, True)])
def test_rows_ref_matches_full(Lq, Lk, causal):
    g = torch.Generator().manual_seed(Lq * 31 + Lk)
    q = torch.randn(2, 6, Lq, 16, generator=g)
    k = torch.randn(2, 3, Lk, 16, generator=g)
    v = torch.randn(2, 3, Lk, 16, generator=g)
    rows = [Lq - 1, 0, Lq // 2]
    full = attention_brute_f64(q, k, v, causal=causal)
    _same(attention_rows_ref(q, k, v, rows, causal=causal), full[:, :, rows], 2e-6)


def test_chunked_matches_unchunked():
    g = torch.Generator().manual_seed(3)
    q = torch.randn(2, 8, 37, 16, generator=g).half()
    k = torch.randn(2, 2, 50, 16, generator=g).half()
    v = torch.randn(2, 2, 50, 16, generator=g).half()
    for causal in (True, False):
        ref = flash_attention_ref(q.float(), k.float(), v.float(), causal=causal)
        for chunk in (1, 5, 16, 64):
            got = flash_attention_ref_chunked(q, k, v, causal=causal, q_chunk=chunk)
            assert torch.allclose(got, ref, atol=1e-6)


# ---------------------------------------------------------------- closed forms + planted mistakes

def closed_form_failures(fn) -> list[str]:
    """Runs the closed-form battery on an attention function with the
    oracle's signature; returns the names of the checks it fails."""
    fails = []
    g = torch.Generator().manual_seed(11)
    B, H, Hk, D = 2, 8, 2, 16
    group = H // Hk

    # GQA: V of kv head j is the constant j+1 -> query head h outputs h//group + 1
    q = torch.randn(B, H, 5, D, generator=g)
    k = torch.randn(B, Hk, 9, D, generator=g)
    v = torch.ones(B, Hk, 9, D) * torch.arange(1, Hk + 1).view(1, Hk, 1, 1)
    out = fn(q, k, v, causal=True)
    want = (torch.arange(H) // group + 1).float().view(1, H, 1, 1).expand_as(out)
    if not torch.allclose(out, want, atol=1e-5):
        fails.append("gqa_mapping")

    # bottom-right alignment: k = 0 (uniform weights), v[j] = j -> row i = (Lk-Lq+i)/2
    Lq, Lk = 4, 10
    q = torch.randn(1, 2, Lq, D, generator=g)
    k = torch.zeros(1, 2, Lk, D)
    v = torch.arange(Lk).float().view(1, 1, Lk, 1).expand(1, 2, Lk, D).contiguous()
    out = fn(q, k, v, causal=True)
    want = ((Lk - Lq + torch.arange(Lq)).float() / 2).view(1, 1, Lq, 1).expand_as(out)
    if not torch.allclose(out, want, atol=1e-5):
        fails.append("bottom_right")

    # scale: two keys with q.k0 = a, q.k1 = 0; v0 = 1, v1 = 0 -> sigmoid(scale * a)
    a = 3.0
    q = torch.zeros(1, 1, 1, D)
    q[..., 0] = 1.0
    k = torch.zeros(1, 1, 2, D)
    k[0, 0, 0, 0] = a
    v = torch.zeros(1, 1, 2, D)
    v[0, 0, 0, :] = 1.0
    for scale in (None, 0.37):
        s = 1.0 / math.sqrt(D) if scale is None else scale
        out = fn(q, k, v, causal=False, scale=scale)
        if abs(float(out[0, 0, 0, 0]) - 1.0 / (1.0 + math.exp(-s * a))) > 1e-6:
            fails.append(f"scale_{scale}")

    # rows sum to one: v = 1 -> output 1 wherever a key is visible
    q = torch.randn(1, 4, 6, D, generator=g)
    k = torch.randn(1, 2, 8, D, generator=g)
    out = fn(q, k, torch.ones(1, 2, 8, D), causal=True)
    if not torch.allclose(out, torch.ones_like(out), atol=1e-5):
        fails.append("row_sum")

    # causal prefill row 0 sees only key 0
    q = torch.randn(1, 4, 6, D, generator=g)
    k = torch.randn(1, 2, 6, D, generator=g)
    v = torch.randn(1, 2, 6, D, generator=g)
    out = fn(q, k, v, causal=True)
    if not torch.allclose(out[0, :, 0], v[0, torch.arange(4) // 2, 0], atol=1e-6):
        fails.append("causal_row0")

    # decode == last row of prefill; Lq = 1 causal == full
    q = torch.randn(1, 4, 6, D, generator=g)
    full = fn(q, k, v, causal=True)
    dec = fn(q[:, :, -1:], k, v, causal=True)
    if not torch.allclose(full[:, :, -1:], dec, atol=1e-6):
        fails.append("decode_vs_prefill")
    if not torch.allclose(dec, fn(q[:, :, -1:], k, v, causal=False), atol=1e-6):
        fails.append("lq1_causal_eq_full")
    return fails


def _mutant(kind):
    def fn(q, k, v, causal=False, scale=None):
        B, H, Lq, D = q.shape
        Hk, Lk = k.shape[1], k.shape[2]
        if H != Hk:
            if kind == "gqa_tile":
                k, v = k.repeat(1, H // Hk, 1, 1), v.repeat(1, H // Hk, 1, 1)
            else:
                k, v = k.repeat_interleave(H // Hk, 1), v.repeat_interleave(H // Hk, 1)
        if scale is None:
            scale = 1.0 if kind == "no_scale" else 1.0 / math.sqrt(D)
        s = q @ k.transpose(-2, -1) * scale
        if causal:
            i = torch.arange(Lq).unsqueeze(-1)
            j = torch.arange(Lk).unsqueeze(0)
            if kind == "top_left":
                hide = j > i
            elif kind == "off_by_one":
                hide = j >= (Lk - Lq + i)
            else:
                hide = j > (Lk - Lq + i)
            s = s.masked_fill(hide, float("-inf"))
        p = torch.softmax(s, -2 if kind == "softmax_over_queries" else -1)
        if kind == "unnormalised":
            p = torch.exp(s - s.amax(-1, keepdim=True))
        return p @ (k if kind == "k_for_v" else v)
    return fn


def test_oracle_passes_closed_forms():
    assert closed_form_failures(flash_attention_ref) == []
    assert closed_form_failures(lambda *a, **kw: torch.from_numpy(attention_brute_f64(*a, **kw)).float()) == []


@pytest.mark.parametrize("kind", ["gqa_tile", "top_left", "off_by_one", "no_scale", "unnormalised",
                                  "softmax_over_queries", "k_for_v"])
def test_planted_mistakes_are_caught(kind):
    assert closed_form_failures(_mutant(kind)), f"mutant {kind} passed every check"


def test_nan_rows_and_empty_history():
    q = torch.randn(1, 2, 5, 16)
    k = torch.randn(1, 1, 3, 16)
    v = torch.randn(1, 1, 3, 16)
    out = flash_attention_ref(q, k, v, causal=True)
    assert torch.isnan(out[:, :, :2]).all() and not torch.isnan(out[:, :, 2:]).any()
    empty = flash_attention_ref(q, k[:, :, :0], v[:, :, :0], causal=True)
    assert (empty == 0).all()


# ---------------------------------------------------------------- paged composition

def _pool_case(seed, B=3, Hq=4, Hk=2, D=16, bs=4, Lq=2, lens=(5, 9, 2), extra_blocks=3):
    g = torch.Generator().manual_seed(seed)
    nblk = [-(-L // bs) for L in lens]
    nb = sum(nblk) + extra_blocks
    perm = torch.randperm(nb, generator=g)
    kp = torch.randn(nb, bs, Hk, D, generator=g)
    vp = torch.randn(nb, bs, Hk, D, generator=g)
    bt = torch.zeros(B, max(nblk), dtype=torch.int32)
    pos = 0
    for b in range(B):
        bt[b, :nblk[b]] = perm[pos:pos + nblk[b]].int()
        pos += nblk[b]
    q = torch.randn(B, Hq, Lq, D, generator=g)
    return q, kp, vp, bt, torch.tensor(lens, dtype=torch.int32)


def test_gather_follows_block_table():
    q, kp, vp, bt, lens = _pool_case(1)
    for b in range(bt.shape[0]):
        L = int(lens[b])
        got = gather_ref(kp, bt[b], L)
        for t in range(L):
            bid, off = logical_to_physical_ref(bt[b].tolist(), kp.shape[1], t)
            assert torch.equal(got[t], kp[bid, off])
    assert gather_ref(kp, bt[0], 0).shape == (0, kp.shape[2], kp.shape[3])


def test_gather_matches_index_select_form():
    # the reference's gather: index_select over whole blocks, reshape, slice to L
    q, kp, vp, bt, lens = _pool_case(2)
    for b in range(bt.shape[0]):
        L = int(lens[b])
        n = -(-L // kp.shape[1])
        dense = kp.index_select(0, bt[b, :n].long()).reshape(-1, kp.shape[2], kp.shape[3])[:L]
        assert torch.equal(gather_ref(kp, bt[b], L), dense)


@pytest.mark.parametrize("causal", [True, False])
def test_paged_ref_matches_brute_and_dense(causal):
    q, kp, vp, bt, lens = _pool_case(3)
    got = paged_attention_ref(q, kp, vp, bt, lens, causal=causal)
    _same(got, paged_attention_brute_f64(q, kp, vp, bt, lens, causal=causal), 2e-6)
    for b in range(q.shape[0]):
        L = int(lens[b])
        kd = gather_ref(kp, bt[b], L).transpose(0, 1).unsqueeze(0)
        vd = gather_ref(vp, bt[b], L).transpose(0, 1).unsqueeze(0)
        _same(got[b:b + 1], flash_attention_ref(q[b:b + 1], kd, vd, causal=causal), 1e-6)


def test_paged_ref_invariant_to_block_relabelling():
    q, kp, vp, bt, lens = _pool_case(4)
    base = paged_attention_ref(q, kp, vp, bt, lens)
    g = torch.Generator().manual_seed(99)
    relabel = torch.randperm(kp.shape[0], generator=g)  # old id -> new id
    kp2 = torch.empty_like(kp)
    vp2 = torch.empty_like(vp)
    kp2[relabel] = kp
    vp2[relabel] = vp
    bt2 = relabel[bt.long()].int()
    _same(paged_attention_ref(q, kp2, vp2, bt2, lens), base, 0)


# ---------------------------------------------------------------- append

def test_append_ref_round_trips_through_gather_and_spans_blocks():
    from oracle import append_ref

    g = torch.Generator().manual_seed(31)
    bs, Hk, D = 4, 2, 16
    kp = torch.zeros(9, bs, Hk, D)
    vp = torch.zeros(9, bs, Hk, D)
    blocks = [7, 2, 5, 0]
    k = torch.randn(11, Hk, D, generator=g)
    v = torch.randn(11, Hk, D, generator=g)
    append_ref(kp, vp, blocks, 3, k, v)  # starts mid-block, spans 4 blocks
    assert torch.equal(gather_ref(kp, blocks, 14)[3:], k)
    assert torch.equal(gather_ref(vp, blocks, 14)[3:], v)
    # positions before start untouched, blocks outside the table untouched
    assert (gather_ref(kp, blocks, 3) == 0).all()
    assert (kp[[1, 3, 4, 6, 8]] == 0).all()
    # every element lands where logical_to_physical says (independent form)
    for t in range(11):
        bid, off = blocks[(3 + t) // bs], (3 + t) % bs
        assert torch.equal(kp[bid, off], k[t]) and torch.equal(vp[bid, off], v[t])


def test_append_ref_explicit_start_overwrites():
    # the reference's "append at start < length rewrites" behaviour (tests/cache/test_kv_cache.py:52-77)
    from oracle import append_ref

    bs, Hk, D = 4, 1, 16
    kp = torch.zeros(3, bs, Hk, D)
    vp = torch.zeros(3, bs, Hk, D)
    blocks = [2, 0]
    first = torch.ones(6, Hk, D)
    append_ref(kp, vp, blocks, 0, first, first)
    patch = torch.full((2, Hk, D), 5.0)
    append_ref(kp, vp, blocks, 3, patch, -patch)
    got = gather_ref(kp, blocks, 6)
    assert torch.equal(got[:3], first[:3]) and torch.equal(got[3:5], patch) and torch.equal(got[5:], first[5:])
    assert torch.equal(gather_ref(vp, blocks, 6)[3:5], -patch)
