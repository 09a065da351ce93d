"""GPU parity of the prefill kernel (engine.attention.flash_attention ->
cie_flash_fwd) against the CPU oracle.

Bar: max |out - ref| <= 2e-3 for fp16 and <= 1e-2 for bf16, where ref is the
fp32 oracle evaluated on the same rounded inputs; NaN patterns must agree.
"""

from __future__ import annotations

import math

import pytest
import torch

from benchmarks import workloads
from engine.attention import flash_attention
from oracle import attention_rows_ref, flash_attention_ref, flash_attention_ref_chunked
from engine.attention import prefill_kernel
from prefill_dispatch import batch_for_two_row_groups, replicate

pytestmark = pytest.mark.gpu

TOL = {torch.float16: 2e-3, torch.bfloat16: 1e-2}
DEV = "cuda"


def assert_close(out: torch.Tensor, ref: torch.Tensor, tol: float, what: str = "") -> float:
    out = out.float().cpu()
    ref = ref.float().cpu()
    assert out.shape == ref.shape, (out.shape, ref.shape)
    n_out, n_ref = torch.isnan(out), torch.isnan(ref)
    assert torch.equal(n_out, n_ref), f"{what}: NaN pattern differs ({int(n_out.sum())} vs {int(n_ref.sum())})"
    ok = ~n_ref
    err = float((out[ok] - ref[ok]).abs().max()) if ok.any() else 0.0
    assert err <= tol, f"{what}: max abs error {err:.3e} > {tol:.1e}"
    return err


def _inputs(B, H, Hk, Lq, Lk, D, dtype, seed, vscale=1.0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, Lq, D, generator=g).to(dtype)
    k = torch.randn(B, Hk, Lk, D, generator=g).to(dtype)
    v = (torch.randn(B, Hk, Lk, D, generator=g) * vscale).to(dtype)
    return q, k, v


def test_reference_kernel_case():
    # the reference's kernel test: fp16 (2,4,64,64,64), causal, seed 0
    torch.manual_seed(0)
    q = torch.randn(2, 4, 64, 64, device=DEV, dtype=torch.float16)
    k = torch.randn(2, 4, 64, 64, device=DEV, dtype=torch.float16)
    v = torch.randn(2, 4, 64, 64, device=DEV, dtype=torch.float16)
    out = flash_attention(q, k, v, causal=True)
    ref = flash_attention_ref(q.cpu().float(), k.cpu().float(), v.cpu().float(), causal=True)
    assert out.dtype == torch.float16 and out.shape == q.shape and out.is_contiguous()
    assert_close(out, ref, 2e-3, "reference case")


SHAPES = [
    # B, H, Hk, Lq, Lk
    (1, 4, 2, 77, 77),      # ragged single tile
    (2, 8, 2, 33, 200),     # prefill over a cache (Lq < Lk)
    (1, 4, 4, 130, 130),    # MHA, two query tiles
    (1, 6, 3, 300, 311),    # several tiles, ragged key tail
]


@pytest.mark.parametrize("D", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("shape", SHAPES)
def test_sweep(D, dtype, causal, shape):
    B, H, Hk, Lq, Lk = shape
    q, k, v = _inputs(B, H, Hk, Lq, Lk, D, dtype, seed=D + Lq + Lk, vscale=0.5)
    out = flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), causal=causal)
    ref = flash_attention_ref(q.float(), k.float(), v.float(), causal=causal)
    assert_close(out, ref, TOL[dtype], f"D={D} {dtype} causal={causal} {shape}")


@pytest.mark.parametrize("L", [1, 31, 32, 33, 64, 65, 96, 97, 128, 160, 161, 192, 193, 224])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [True, False])
def test_d128_every_tile_count(L, dtype, causal):
    """D=128 streams 32-key tiles and publishes them two per workgroup
    barrier: 1..7 tiles, full and ragged, cover both barrier parities at
    the last tile and every prologue length."""
    q, k, v = _inputs(1, 4, 2, L, L, 128, dtype, seed=1000 + L, vscale=0.5)
    out = flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), causal=causal)
    ref = flash_attention_ref(q.float(), k.float(), v.float(), causal=causal)
    assert_close(out, ref, TOL[dtype], f"D=128 L={L} {dtype} causal={causal}")


@pytest.mark.parametrize("Lq,Lk", [(129, 129), (160, 160), (191, 191), (192, 192), (255, 255), (256, 256),
                                   (257, 257), (300, 311), (383, 383), (384, 384), (385, 385), (511, 511),
                                   (512, 512), (513, 513), (200, 1000), (520, 70)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("H,Hk", [(4, 2), (3, 3)])
def test_d64_two_row_group_kernel(Lq, Lk, dtype, causal, H, Hk):
    """D=64 launches with enough work run two 32-row groups per wave over
    32-key tiles in a four-stage ring: the same rows of two query heads (even
    group size, 128-row workgroups) or 64 rows of one head (odd group size,
    256-row workgroups). One problem is repeated over a batch large enough to
    take that kernel and every copy is checked against the oracle: 1..33
    tiles, full and ragged query and key tails, waves with no rows, a
    history longer than the chunk and more queries than keys (NaN rows under
    the causal rule)."""
    q, k, v = _inputs(1, H, Hk, Lq, Lk, 64, dtype, seed=2000 + Lq + Lk, vscale=0.5)
    ref = flash_attention_ref(q.float(), k.float(), v.float(), causal=causal)
    B = batch_for_two_row_groups(H, Lq, Lk, causal)
    out = flash_attention(replicate(q, B).to(DEV), replicate(k, B).to(DEV), replicate(v, B).to(DEV), causal=causal)
    assert_close(out, replicate(ref, B), TOL[dtype], f"D=64 Lq={Lq} Lk={Lk} {dtype} causal={causal} B={B}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_more_queries_than_keys_gives_nan_rows(dtype):
    q, k, v = _inputs(1, 4, 2, 150, 20, 64, dtype, seed=5, vscale=0.5)
    out = flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), causal=True)
    ref = flash_attention_ref(q.float(), k.float(), v.float(), causal=True)
    assert torch.isnan(ref[:, :, :130]).all()
    assert_close(out, ref, TOL[dtype], "Lq > Lk")


def test_empty_history_gives_zeros():
    q, k, v = _inputs(1, 4, 2, 5, 0, 64, torch.float16, seed=6)
    out = flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), causal=True)
    assert (out == 0).all()


def test_empty_query():
    q, k, v = _inputs(1, 4, 2, 0, 9, 64, torch.float16, seed=7)
    out = flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), causal=True)
    assert out.shape == (1, 4, 0, 64)


def test_strided_views_match_contiguous():
    # the call-site layout: gathered (N, Hk, D) history viewed as (1, Hk, N, D)
    g = torch.Generator().manual_seed(8)
    N, Hk, H, D, L = 97, 2, 8, 64, 97
    hist_k = torch.randn(N, Hk, D, generator=g).half().to(DEV)
    hist_v = torch.randn(N, Hk, D, generator=g).half().to(DEV)
    q = torch.randn(1, L, H, D, generator=g).half().to(DEV).transpose(1, 2)  # (1, H, L, D) view
    kv_k = hist_k.transpose(0, 1).unsqueeze(0)
    kv_v = hist_v.transpose(0, 1).unsqueeze(0)
    assert not kv_k.is_contiguous() and not q.is_contiguous()
    out = flash_attention(q, kv_k, kv_v, causal=True, scale=1.0 / math.sqrt(D))
    out_c = flash_attention(q.contiguous(), kv_k.contiguous(), kv_v.contiguous(), causal=True)
    assert torch.equal(out, out_c)


@pytest.mark.parametrize("D", [64, 128])
def test_huge_row_stride_uses_wide_copies(D):
    """K and V rows 2^25 elements apart (views into one 2.7 GB allocation
    each): a tile of rows spans more than 2^31 bytes, so the kernels form
    64-bit per-lane addresses instead of 32-bit offsets from a tile base; the
    result equals the oracle and the same data laid out contiguously, bit
    for bit."""
    g = torch.Generator().manual_seed(D)
    H, Hk, L = 4, 2, 40
    q = torch.randn(1, H, L, D, generator=g).half()
    k = torch.randn(1, Hk, L, D, generator=g).half()
    v = torch.randn(1, Hk, L, D, generator=g).half()
    stride = 1 << 25
    views = []
    for t in (k, v):
        big = torch.zeros(L, stride, dtype=t.dtype, device=DEV)
        view = big[:, :Hk * D].view(L, Hk, D).permute(1, 0, 2).unsqueeze(0)
        view.copy_(t.to(DEV))
        assert view.stride(2) == stride
        views.append(view)
    out = flash_attention(q.to(DEV), views[0], views[1], causal=True).cpu()
    dense = flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), causal=True).cpu()
    ref = flash_attention_ref(q.float(), k.float(), v.float(), causal=True)
    assert_close(out, ref, 2e-3, f"D={D} huge row stride")
    assert torch.equal(out, dense)
    del views
    torch.cuda.empty_cache()

@pytest.mark.parametrize("D,B,Lq,Lk", [(64, 2, 100, 140), (64, 2, 300, 340), (64, 64, 300, 340), (64, 32, 1024, 1024),
                                      (128, 2, 100, 140)])
def test_gqa_equals_expanded_mha_bitwise(D, B, Lq, Lk):
    """GQA indexes the shared kv head instead of copying it. At D=64 with
    enough work (B = 64 and 32 here) it runs head pairs where the expanded
    MHA (group size 1) runs 64-row waves of one head; the launcher decides
    from B * Hq alone, and both give every row the same bits."""
    if D == 64 and B >= 32:
        assert prefill_kernel(B, 8, 2, Lq, Lk, D, True) == "r64_heads"
    q, k, v = _inputs(B, 8, 2, Lq, Lk, D, torch.float16, seed=9)
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    gqa = flash_attention(q, k, v, causal=True)
    mha = flash_attention(q, k.repeat_interleave(4, 1), v.repeat_interleave(4, 1), causal=True)
    assert torch.equal(gqa, mha)


@pytest.mark.parametrize("D,L", [(64, 96), (64, 300), (128, 96)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_nan_query_row_stays_in_its_row(D, L, dtype):
    """A NaN in one query row makes that row NaN and no other, as the
    reference's per-row softmax does (the row sums run on the matrix pipe
    and must not mix rows: rows r and r + 16 of a wave once shared an MFMA
    column, where 0 x NaN = NaN)."""
    q, k, v = _inputs(1, 4, 2, L, L, D, dtype, seed=23)
    qn = q.clone()
    qn[0, 1, 0, 3] = float("nan")
    qn[0, 2, 37, 0] = float("nan")
    if L > 128:  # the other head of a pair, and row group 1 of a 64-row wave
        qn[0, 3, 64 + 33, 5] = float("nan")
    ref = flash_attention_ref(qn.float(), k.float(), v.float(), causal=True)
    B = batch_for_two_row_groups(4, L, L, True) if L > 128 else 1  # D=64: the two-row-group kernel
    q, qn, k, v = (replicate(x, B).to(DEV) for x in (q, qn, k, v))
    clean = flash_attention(q, k, v, causal=True)
    out = flash_attention(qn, k, v, causal=True)
    assert_close(out, replicate(ref, B), TOL[dtype], f"nan rows D={D} L={L} {dtype}")  # includes the NaN pattern
    if D == 128 or L > 128:  # the slow path there acts per row: the other rows keep their bits
        keep = ~torch.isnan(replicate(ref, B)).any(dim=-1)
        assert torch.equal(out.cpu()[keep], clean.cpu()[keep])


@pytest.mark.parametrize("D,span", [(128, 32), (64, 64)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_rows_do_not_depend_on_their_wave(D, span, dtype):
    """head_dim 128 (32-row waves) and head_dim 64 over more than 128 query
    rows (waves of 32 rows of both query heads here): a row whose scores rise
    across tiles takes the lazy-max slow path; the other rows (1..span-1 of
    both heads, its own wave included) keep their arithmetic, so their
    outputs are bit-identical to a run in which no row takes it."""
    L = 320
    g = torch.Generator().manual_seed(21)
    u = torch.randn(D, generator=g)
    u = u / u.norm()
    q = torch.randn(1, 2, L, D, generator=g) * 0.3
    k = torch.randn(1, 1, L, D, generator=g) * 0.3
    k += (torch.arange(L, dtype=torch.float32) / 32.0 * 20.0 * math.sqrt(D) / (3.0 * math.log2(math.e)))[None, None, :, None] * u
    v = torch.randn(1, 1, L, D, generator=g) * 0.5
    quiet = q.clone()
    loud = q.clone()
    loud[:, :, 0] += 3.0 * u  # row 0 (and its wave's slow path) rises with the keys
    ref = flash_attention_ref(loud.to(dtype).float(), k.to(dtype).float(), v.to(dtype).float(), causal=False)
    B = batch_for_two_row_groups(2, L, L, False) if D == 64 else 1  # D=64: the two-row-group kernel
    k, v = (replicate(x, B).to(dtype).to(DEV) for x in (k, v))
    outs = [flash_attention(replicate(x, B).to(dtype).to(DEV), k, v, causal=False) for x in (quiet, loud)]
    assert torch.equal(outs[0][:, :, 1:span], outs[1][:, :, 1:span])
    assert_close(outs[1], replicate(ref, B), TOL[dtype], f"loud row {dtype}")


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("pattern", ["rising", "spikes", "falling"])
def test_row_max_changes_across_tiles(D, dtype, pattern):
    """Scores whose row max moves by many log2 units from tile to tile: the
    kernel keeps a reference max per row and recomputes it only when a tile's
    probabilities outgrow it (rising scores do so on every tile; spikes on a
    few; falling never), so each pattern takes a different path."""
    g = torch.Generator().manual_seed(D + len(pattern))
    B, H, Hk, L = 1, 4, 2, 640
    u = torch.randn(D, generator=g)
    u = u / u.norm()
    q = (torch.randn(B, H, L, D, generator=g) * 0.3 + 3.0 * u).to(dtype)
    k = torch.randn(B, Hk, L, D, generator=g) * 0.3
    pos = torch.arange(L, dtype=torch.float32)
    c = math.log2(math.e) / math.sqrt(D)  # log2 units of score per unit of q.k
    if pattern == "rising":      # +20 log2 units of score per 64 keys
        k += (pos / 64.0 * 20.0 / (3.0 * c))[None, None, :, None] * u
    elif pattern == "spikes":    # a few keys, each 5-20 log2 units above the ones before
        for j, h in ((5, 10.0), (150, 20.0), (151, 20.0), (400, 30.0), (639, 40.0)):
            k[:, :, j] += h * u
    else:                        # the first keys dominate
        k += ((L - pos) / L * 4.0)[None, None, :, None] * u
    k = k.to(dtype)
    v = (torch.randn(B, Hk, L, D, generator=g) * 0.5).to(dtype)
    for causal in (True, False):
        ref = flash_attention_ref(q.float(), k.float(), v.float(), causal=causal)
        # D=64: also repeated over a batch that takes the two-row-group kernel
        for R in (1, batch_for_two_row_groups(H, L, L, causal)) if D == 64 else (1,):
            out = flash_attention(replicate(q, R).to(DEV), replicate(k, R).to(DEV), replicate(v, R).to(DEV), causal=causal)
            assert_close(out, replicate(ref, R), TOL[dtype], f"{pattern} D={D} {dtype} causal={causal} B={R}")


def test_deterministic():
    q, k, v = _inputs(1, 8, 2, 257, 257, 128, torch.bfloat16, seed=10)
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    assert torch.equal(flash_attention(q, k, v, causal=True), flash_attention(q, k, v, causal=True))


def test_headline_workload_is_bit_identical_run_to_run():
    """prefill_s2048 on the head-pair kernel, three more launches with another
    launch between each: the same bits (every row's arithmetic is fixed; no
    cross-workgroup reduction)."""
    c = workloads.prefill_s2048(DEV)
    assert prefill_kernel(4, 32, 8, 2048, 2048, 64, True, torch.float16) == "r64_heads"
    first = flash_attention(c.q, c.k, c.v, causal=True)
    for _ in range(3):
        flash_attention(c.k.repeat_interleave(4, dim=1), c.k, c.v, causal=True)
        assert torch.equal(flash_attention(c.q, c.k, c.v, causal=True), first)


def test_explicit_scale():
    q, k, v = _inputs(1, 4, 2, 64, 64, 64, torch.float16, seed=11)
    out = flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), causal=False, scale=0.05)
    ref = flash_attention_ref(q.float(), k.float(), v.float(), causal=False, scale=0.05)
    assert_close(out, ref, 2e-3, "scale=0.05")


def test_boundary_errors_match_reference_types():
    q = torch.randn(1, 2, 4, 16, device=DEV, dtype=torch.float16)
    with pytest.raises(ValueError):
        flash_attention(q.float(), q.float(), q.float())
    bad = torch.randn(1, 2, 4, 24, device=DEV, dtype=torch.float16)
    with pytest.raises(ValueError):
        flash_attention(bad, bad, bad)
    small = torch.randn(1, 2, 4, 8, device=DEV, dtype=torch.float16)
    with pytest.raises(ValueError):
        flash_attention(small, small, small)
    with pytest.raises(ValueError):
        flash_attention(q, q[:, :1].repeat(1, 3, 1, 1)[:, :3], q[:, :1].repeat(1, 3, 1, 1)[:, :3])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_workload_prefill_s128(dtype):
    # the CPU-oracle workload, run on the GPU in fp16 and bf16
    case = workloads.prefill_s128()
    q, k, v = case.q.to(dtype), case.k.to(dtype), case.v.to(dtype)
    out = flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), causal=True)
    ref = flash_attention_ref(q.float(), k.float(), v.float(), causal=True)
    assert_close(out, ref, TOL[dtype], f"prefill_s128 {dtype}")


def test_workload_prefill_s2048():
    case = workloads.prefill_s2048()
    out = flash_attention(case.q.to(DEV), case.k.to(DEV), case.v.to(DEV), causal=True)
    ref = flash_attention_ref_chunked(case.q, case.k, case.v, causal=True, q_chunk=1024)
    assert_close(out, ref, 2e-3, "prefill_s2048")


@pytest.mark.parametrize("Lq,Lk", [(65536, 65536), (300, 65536)])
def test_long_sequences_sampled_rows(Lq, Lk):
    """64 K keys, fp16, head_dim 64, 8 / 2 heads, causal: a prefill of all of
    them (the head-pair kernel, 4 * 16 * 512 items) and a 300-row chunk at
    the end of the history (bottom-right mask: row i sees keys <= Lk - Lq +
    i), checked on sampled rows against the oracle, with row and key
    offsets past 2^16 and the element offsets of K / V past 2^22."""
    g = torch.Generator().manual_seed(Lq)
    q = (torch.randn(1, 8, Lq, 64, generator=g) / 8).half()
    k = (torch.randn(1, 2, Lk, 64, generator=g) / 8).half()
    v = torch.randn(1, 2, Lk, 64, generator=g).half()
    out = flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), causal=True).cpu()
    assert not torch.isnan(out).any()
    rows = sorted({0, 1, Lq // 2, Lq - 2, Lq - 1} | set(torch.randint(0, Lq, (11,), generator=g).tolist()))
    ref = attention_rows_ref(q, k, v, rows, causal=True)
    assert_close(out[:, :, rows], ref, 2e-3, f"Lq={Lq} Lk={Lk} sampled rows")


def test_workload_prefill_s16384_sampled_rows():
    case = workloads.prefill_s16384()
    out = flash_attention(case.q.to(DEV), case.k.to(DEV), case.v.to(DEV), causal=True).cpu()
    assert not torch.isnan(out).any()
    # causal row 0 attends to key 0 alone: P = 1 exactly, so the row is V[kv(h), 0] bit for bit
    assert torch.equal(out[0, :, 0], case.v[0, torch.arange(32) // 4, 0])
    g = torch.Generator().manual_seed(123)
    rows = [1, 127, 128, 129, 4095, 8191, 16383] + torch.randint(0, 16384, (25,), generator=g).tolist()
    ref = attention_rows_ref(case.q, case.k, case.v, rows, causal=True)
    assert_close(out[:, :, rows], ref, 1e-2, "prefill_s16384 sampled rows")
