"""A decode / verify step's attention sections captured in one HIP graph
(torch.cuda.CUDAGraph) and replayed: every replay, with new token data copied
into the captured input buffers and the program's own eager work and
synchronisations between replays, must equal the eager section bit for bit
(both run the same deterministic kernels; the append at fixed positions is
idempotent, so the eager run after a replay rewrites the same rows). The
eager section itself is checked against the oracle in test_append_gpu.py."""

from __future__ import annotations

import pytest
import torch

from engine.attention import prefill_kernel
from prefill_dispatch import batch_for_two_row_groups
from engine.cache import KVCacheConfig, PagedKVCache
from engine.model import attention_section

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("L,dtype", [(1, torch.float16), (4, torch.bfloat16)])
def test_graph_replays_equal_eager(L, dtype):
    B, Hq, Hk, D, layers = 6, 16, 4, 64, 2
    cache = PagedKVCache(KVCacheConfig(num_layers=layers, num_kv_heads=Hk, head_dim=D, num_blocks=200,
                                       block_size=16, dtype=dtype, device=DEV))
    g = torch.Generator().manual_seed(70 + L)
    tables = [cache.new_sequence() for _ in range(B)]
    for t, n in zip(tables, [300, 17, 0, 129, 64, 500]):
        if n:
            for layer in range(layers):
                cache.append(layer, t, torch.randn(n, Hk, D, generator=g).to(dtype).to(DEV),
                             torch.randn(n, Hk, D, generator=g).to(dtype).to(DEV), start=0)
    step = cache.prepare_step(tables, L)
    q = torch.zeros(layers, B, Hq, L, D, dtype=dtype, device=DEV)
    k = torch.zeros(layers, B, Hk, L, D, dtype=dtype, device=DEV)
    v = torch.zeros(layers, B, Hk, L, D, dtype=dtype, device=DEV)

    def run():
        return [attention_section(q[i], k[i], v[i], i, cache, step) for i in range(layers)]

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()  # warm-up outside the capture (workspace, library load)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = run()
    for rep in range(3):
        for x in (q, k, v):
            x.copy_(torch.randn(x.shape, generator=g).to(dtype))
        graph.replay()
        torch.cuda.synchronize()
        got = [o.clone() for o in outs]
        want = run()
        torch.cuda.synchronize()
        for i in range(layers):
            assert torch.isfinite(got[i].float()).all()
            assert torch.equal(got[i], want[i]), (rep, i, (got[i].float() - want[i].float()).abs().max().item())


def test_out_argument_writes_views_in_place():
    """flash_attention / paged_attention with ``out`` = a transposed view of a
    (B, L, H, D) buffer write exactly what they return without it."""
    from engine.attention import flash_attention, paged_attention
    from engine.cache import block_table_tensor

    g = torch.Generator().manual_seed(90)
    B, Hq, Hk, L, D = 2, 8, 2, 70, 64
    q = torch.randn(B, Hq, L, D, generator=g).half().to(DEV)
    k = torch.randn(B, Hk, L, D, generator=g).half().to(DEV)
    v = torch.randn(B, Hk, L, D, generator=g).half().to(DEV)
    rows = torch.full((B, L, Hq, D), 7.0, dtype=torch.float16, device=DEV)
    got = flash_attention(q, k, v, causal=True, out=rows.transpose(1, 2))
    assert got.data_ptr() == rows.data_ptr()
    assert torch.equal(rows.transpose(1, 2), flash_attention(q, k, v, causal=True))
    # 200 rows over a batch that takes the head_dim-64 two-row-group kernel
    Lr = 200
    Br = batch_for_two_row_groups(Hq, Lr, Lr, True)
    assert prefill_kernel(Br, Hq, Hk, Lr, Lr, D, True) == "r64_heads"
    qr, kr, vr = (torch.randn(Br, h, Lr, D, generator=g).half().to(DEV) for h in (Hq, Hk, Hk))
    big = torch.full((Br, Lr, Hq, D), 7.0, dtype=torch.float16, device=DEV)
    flash_attention(qr, kr, vr, causal=True, out=big.transpose(1, 2))
    assert torch.equal(big.transpose(1, 2), flash_attention(qr, kr, vr, causal=True))
    cache = PagedKVCache(KVCacheConfig(num_layers=1, num_kv_heads=Hk, head_dim=D, num_blocks=64, block_size=16,
                                       dtype=torch.float16, device=DEV))
    tables = [cache.new_sequence() for _ in range(B)]
    for b, t in enumerate(tables):
        cache.append(0, t, k[b].transpose(0, 1), v[b].transpose(0, 1))
    bt, lens = block_table_tensor(tables, DEV)
    q1 = q[:, :, :3]
    rows = torch.zeros((B, 3, Hq, D), dtype=torch.float16, device=DEV)
    paged_attention(q1, cache.k[0], cache.v[0], bt, lens, out=rows.transpose(1, 2))
    assert torch.equal(rows.transpose(1, 2), paged_attention(q1, cache.k[0], cache.v[0], bt, lens))
    with pytest.raises(ValueError):
        flash_attention(q, k, v, out=torch.empty(B, Hq, L, D + 4, dtype=torch.float16, device=DEV)[..., :D])
