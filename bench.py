"""Benchmark of the MI355X attention hot path.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--no-extra]

Headline (one JSON line on stdout): causal GQA prefill attention, B=4, S=2048,
32 q / 8 kv heads, head_dim 64, fp16, inputs N(0,1)/8 (seed 1), in TFLOP/s of
algorithmic work (4 B Hq D S(S+1)/2 FLOP per step). A step is one
``engine.attention.flash_attention`` call on inputs already resident in HBM.

The same line carries
  roofline      the prefill kernel's achieved TFLOP/s (algorithmic FLOP per
                launch / average launch duration from HIP events on the launch
                stream) against the dense fp16 MFMA peak, and against that
                peak at the GFX clock the kernel holds under back-to-back
                launches (amdsmi; null where it is not available);
  cpu_baseline  the fp32 oracle (the reference's naive algorithm) timed on the
                host cores on the same workload;
  extra         the other workloads: paged decode (B=32, fp16) and speculative
                verify (B=8, Lq=5, bf16) in GB/s against the 8 TB/s HBM peak,
                timed while rotating over >= 512 MiB of KV pool copies so the
                256 MiB Infinity Cache cannot hold them (back-to-back
                launches; the planned calls also captured in a HIP graph and
                replayed, as an engine step runs them); the paged KV append
                of a prefill (4 x 2048 tokens) and of a decode step (32 x 1
                token) in GB/s of bytes read + written; RoPE of the
                prefill's q (4 x 32 x 2048 x 64) in GB/s; one layer's
                attention section of that prefill with RoPE fused against
                rope_apply first; one layer's attention section of a decode
                step (batched append + paged attention; eager, HIP-graph
                replay, with RoPE fused or applied first) beside the
                reference's per-sequence append / gather / dense
                structure; the INT8-weight GEMM at the reference's
                benchmark shapes (64 and 512 x 4096 x 4096) in TFLOP/s and
                GB/s; and the S=16384 D=128 bf16 prefill in TFLOP/s.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(REPO, "custom-inference-engine_amd")
for _p in (REPO, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_MFMA_F16_TFLOPS = 2516.6  # 256 CU x 2.4 GHz x 4096 FLOP/clk, dense fp16/bf16
PEAK_HBM_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="run only a 256 MiB copy (counter calibration), the prefill kernel and the "
                         "paged decode / verify pairs, for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs")
    ap.add_argument("--probe", default="",
                    help="comma-separated workloads (prefill_s2048, prefill_s16384, decode_b32, verify_b8): "
                         "run only the 256 MiB calibration copy and three launches of each, for rocprofv3 "
                         "--pmc counter runs")
    return ap.parse_args()


TRAFFIC_SUMMARY = os.path.join(REPO, "profiles", "flash_fwd_prefill_s2048_traffic.txt")


def traffic_from_summary():
    """HBM bytes per launch of the prefill kernel from the committed counter
    summary (FETCH_SIZE + WRITE_SIZE, each scaled by the counter's reading for
    a copy of known size), or None when no summary is committed."""
    try:
        for line in open(TRAFFIC_SUMMARY):
            if line.startswith("traffic_bytes_per_launch:"):
                return float(line.split(":", 1)[1])
    except OSError:
        return None
    return None


def traffic_probe(names=("prefill_s2048", "decode_b32", "verify_b8")):
    """The calibration copy, then three launches of each named workload
    (paged ones on distinct pool copies): short runs for counter passes."""
    import torch

    from benchmarks import workloads

    dev = torch.device("cuda:0")
    x = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    y = torch.empty_like(x)
    for _ in range(3):
        y.copy_(x)  # 256 MiB read + 256 MiB written per dispatch
    torch.cuda.synchronize()
    del x, y
    for name in names:
        case = workloads.WORKLOADS[name]()
        launch = FlashLaunch(case, dev) if name.startswith("prefill") else PagedLaunch(case, dev, planned=True)
        for i in range(3):
            launch(i)
        torch.cuda.synchronize()
        del launch
        torch.cuda.empty_cache()
        print(f"probe {name} done", flush=True)


class FlashLaunch:
    """Pre-bound cie_flash_fwd call (no per-call Python allocation)."""

    def __init__(self, case, dev):
        import torch
        from engine import _lib

        self.lib = _lib.load()
        self.q, self.k, self.v = case.q.to(dev), case.k.to(dev), case.v.to(dev)
        self.o = torch.empty_like(self.q)
        B, H, M, D = self.q.shape
        Hk, N = self.k.shape[1], self.k.shape[2]
        self._keep = [_lib.strides(t) for t in (self.q, self.k, self.v, self.o)]
        self.args = (self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(), self.o.data_ptr(),
                     *self._keep, B, H, Hk, M, N, D, ctypes.c_float(1.0 / math.sqrt(D)), 1,
                     _lib.DTYPE_CODES[self.q.dtype])
        self.dev = self.q.device
        self.flops = case.flops

    def __call__(self, i=0):
        rc = self.lib.cie_flash_fwd(*self.args, _stream(self.dev))
        if rc:
            from engine import _lib
            _lib.check(rc)


class PagedLaunch:
    """Pre-bound paged attention call rotating over `copies` KV pool copies:
    cie_paged_fwd (schedule derived on the device from the lengths), or with
    `planned` cie_paged_fwd_ex reading a work plan built on the host from the
    same lengths and block tables and uploaded beforehand, as an engine step
    does once for all its layers."""

    def __init__(self, case, dev, min_bytes=512 << 20, planned=False):
        import torch
        from engine import _lib
        from engine.attention import paged_plan

        self.lib = _lib.load()
        self.q = case.q.to(dev)
        pool_bytes = 2 * case.k_pool.numel() * case.k_pool.element_size()
        self.copies = max(1, -(-min_bytes // pool_bytes))
        self.pools = [(case.k_pool.to(dev), case.v_pool.to(dev)) for _ in range(self.copies)]
        self.bt = case.block_tables.to(dev).contiguous()
        self.lens = case.context_lens.to(dev)
        self.o = torch.empty_like(self.q)
        B, Hq, Lq, D = self.q.shape
        nb, bs, Hk, _ = case.k_pool.shape
        mb = self.bt.shape[1]
        mc = int(case.context_lens.max())
        ws = self.lib.cie_paged_workspace_bytes(B, Hq, Hk, Lq, D, mc, bs, mb)
        self.ws = torch.empty(max(ws, 16), dtype=torch.uint8, device=dev)
        self._keep = [_lib.strides(t) for t in (self.q, self.pools[0][0], self.pools[0][1], self.o)]
        self.planned = planned
        if planned:
            self.plan = paged_plan(case.context_lens, case.block_tables, Hq=Hq, Hk=Hk, Lq=Lq, D=D, num_blocks=nb,
                                   block_size=bs, max_context=mc, device=dev)
            self._none3 = (ctypes.c_int64 * 3)(0, 0, 1)
            self.tail = (None, None, self.plan.data.data_ptr(), self.plan.data.numel() * 4, self.plan.split,
                         self.o.data_ptr(),
                         self.ws.data_ptr(), ws, self._keep[0], self._none3, self._none3, *self._keep[1:],
                         B, Hq, Hk, Lq, D, nb, bs, mb, mc, ctypes.c_float(1.0 / math.sqrt(D)), 1,
                         _lib.DTYPE_CODES[self.q.dtype], None, None, 0, 0)
        else:
            self.tail = (self.bt.data_ptr(), self.lens.data_ptr(), self.o.data_ptr(), self.ws.data_ptr(), ws,
                         *self._keep, B, Hq, Hk, Lq, D, nb, bs, mb, mc, ctypes.c_float(1.0 / math.sqrt(D)), 1,
                         _lib.DTYPE_CODES[self.q.dtype])
        self.dev = dev
        self.ptrs = [(k.data_ptr(), v.data_ptr()) for k, v in self.pools]
        self.bytes = case.bytes
        self.flops = case.flops

    def __call__(self, i=0):
        kp, vp = self.ptrs[i % self.copies]
        if self.planned:
            rc = self.lib.cie_paged_fwd_ex(self.q.data_ptr(), None, None, kp, vp, *self.tail, _stream(self.dev))
        else:
            rc = self.lib.cie_paged_fwd(self.q.data_ptr(), kp, vp, *self.tail, _stream(self.dev))
        if rc:
            from engine import _lib
            _lib.check(rc)


class AppendLaunch:
    """Pre-bound cie_kv_append: B sequences x L new tokens (Hk=8, D=64, fp16,
    block_size 16) into a pool whose blocks are a random permutation, rotating
    over copies of the sources and pools that together exceed `min_bytes` so
    the Infinity Cache cannot hold them."""

    def __init__(self, B, L, dev, seed=6, min_bytes=512 << 20):
        import torch
        from engine import _lib

        self.lib = _lib.load()
        g = torch.Generator().manual_seed(seed)
        Hk, D, bs = 8, 64, 16
        starts = torch.randint(0, 4096, (B,), generator=g, dtype=torch.int32)
        need = [-(-(int(s) + L) // bs) for s in starts]
        nb = sum(need)
        perm = torch.randperm(nb, generator=g).to(torch.int32)
        width = max(need)
        bt = torch.zeros(B, width, dtype=torch.int32)
        pos = 0
        for b, n in enumerate(need):
            bt[b, :n] = perm[pos:pos + n]
            pos += n
        T = B * L
        k = torch.randn(T, Hk, D, generator=g).half()
        v = torch.randn(T, Hk, D, generator=g).half()
        per_copy = 2 * T * Hk * D * 2 + 2 * nb * bs * Hk * D * 2
        self.copies = max(1, -(-min_bytes // per_copy))
        self.bufs = []
        for _ in range(self.copies):
            kc = torch.zeros(nb, bs, Hk, D, dtype=torch.float16, device=dev)
            self.bufs.append((k.to(dev), v.to(dev), kc, torch.zeros_like(kc)))
        self.bt = bt.to(dev)
        self.cu = torch.arange(0, T + 1, L, dtype=torch.int32).to(dev)
        self.st = starts.to(dev)
        k0, v0, kc0, vc0 = self.bufs[0]
        self._keep = [_lib.strides3(k0), _lib.strides3(v0), _lib.strides(kc0), _lib.strides(vc0)]
        self.ptrs = [tuple(t.data_ptr() for t in bufs) for bufs in self.bufs]
        self.tail = (*self._keep, self.bt.data_ptr(), self.cu.data_ptr(), self.st.data_ptr(), None,
                     B, T, L, Hk, D, nb, bs, width, 0)
        self.dev = dev
        self.bytes = 2 * 2 * T * Hk * D * 2  # K and V rows, read once and written once

    def __call__(self, i=0):
        rc = self.lib.cie_kv_append(*self.ptrs[i % self.copies], *self.tail, _stream(self.dev))
        if rc:
            from engine import _lib
            _lib.check(rc)


class RopeLaunch:
    """Pre-bound cie_rope_apply, in place, on q of the prefill_s2048 shape
    (4 x 32 heads x 2048 rows x 64, fp16) at positions 0..2047, rotating over
    copies that together exceed `min_bytes` (Infinity Cache)."""

    def __init__(self, dev, B=4, H=32, L=2048, D=64, min_bytes=512 << 20):
        import torch
        from engine import _lib
        from engine.model.rope import build_rope_cache

        self.lib = _lib.load()
        cos, sin = build_rope_cache(4096, D)
        self.cos, self.sin = cos.to(dev), sin.to(dev)
        per = B * H * L * D * 2
        self.copies = max(1, -(-min_bytes // per))
        x = torch.randn(B, H, L, D).half().to(dev)
        self.bufs = [x.clone() for _ in range(self.copies)]
        self._st = _lib.strides(x)
        self.tail = (self._st, self._st, None, 0, self.cos.data_ptr(), self.sin.data_ptr(), 4096, 2, None,
                     B, H, L, D, 0)
        self.dev = dev
        self.bytes = 2 * per  # read once, written once (the fp32 tables: 0.5 MiB more, from L2)

    def __call__(self, i=0):
        t = self.bufs[i % self.copies]
        rc = self.lib.cie_rope_apply(t.data_ptr(), t.data_ptr(), *self.tail, _stream(self.dev))
        if rc:
            from engine import _lib
            _lib.check(rc)


class Int8Launch:
    """Pre-bound cie_int8_matmul at the reference's benchmark shapes
    (benchmarks/bench_int8_matmul.py:14: M x 4096 x 4096, fp16 activations,
    per-channel fp16 scales), rotating over weight copies that together
    exceed `min_bytes` so the Infinity Cache cannot hold them."""

    def __init__(self, M, dev, N=4096, K=4096, min_bytes=512 << 20):
        import torch
        from engine import _lib

        self.lib = _lib.load()
        g = torch.Generator().manual_seed(12)
        w = torch.randint(-128, 128, (N, K), generator=g, dtype=torch.int8)
        self.copies = max(1, -(-min_bytes // (N * K)))
        self.ws_ = [w.to(dev) for _ in range(self.copies)]
        self.x = torch.randn(M, K, generator=g).half().to(dev)
        self.s = (torch.rand(N, generator=g) * 0.01).half().to(dev)
        self.y = torch.empty(M, N, dtype=torch.float16, device=dev)
        nbytes = int(self.lib.cie_int8_matmul_workspace_bytes(M, N, K))
        self.work = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=dev)
        self.args_tail = (self.s.data_ptr(), None, self.y.data_ptr(), K, K, N, M, N, K, 0, 0,
                          self.work.data_ptr(), self.work.numel())
        self.dev = dev
        self.flops = 2.0 * M * N * K
        self.bytes = N * K + M * K * 2 + M * N * 2 + N * 2  # weights, x, y, scales: each once

    def __call__(self, i=0):
        rc = self.lib.cie_int8_matmul(self.x.data_ptr(), self.ws_[i % self.copies].data_ptr(), *self.args_tail,
                                      _stream(self.dev))
        if rc:
            from engine import _lib
            _lib.check(rc)


def prefill_section_times(dev, iters=10):
    """One layer's attention section for a prefill of 4 fresh sequences x
    2048 tokens (32/8 heads, D=64, fp16) with RoPE: fused (rotary append that
    also returns the rotated K, Q rotated in the prefill kernel's load)
    against rotating q and k first with rope_apply and running the plain
    section (append + prefill attention)."""
    import torch

    from engine.cache import KVCacheConfig, PagedKVCache
    from engine.model import attention_section
    from engine.model.rope import RotaryEmbedding, rope_apply

    B, L, Hq, Hk, D = 4, 2048, 32, 8, 64
    emb = RotaryEmbedding(D, 4096).to(dev)
    cache = PagedKVCache(KVCacheConfig(1, Hk, D, B * L // 16 + 8, 16, torch.float16, dev))
    tables = [cache.new_sequence() for _ in range(B)]
    step = cache.prepare_step(tables, L)
    g = torch.Generator().manual_seed(8)
    # transposed views of (B, L, H, D) projections, as the model makes them (block.py:50-52)
    q = (torch.randn(B, L, Hq, D, generator=g) / 8).half().to(dev).transpose(1, 2)
    k = torch.randn(B, L, Hk, D, generator=g).half().to(dev).transpose(1, 2)
    v = torch.randn(B, L, Hk, D, generator=g).half().to(dev).transpose(1, 2)

    def fused(i=0):
        attention_section(q, k, v, 0, cache, step, rope=emb.tables)

    def unfused(i=0):
        qr = rope_apply(q, emb.cos, emb.sin)
        kr = rope_apply(k, emb.cos, emb.sin)
        attention_section(qr, kr, v, 0, cache, step)

    def plain(i=0):
        attention_section(q, k, v, 0, cache, step)

    # GPU time of each section: captured in a HIP graph and replayed
    res = {}
    for name, fn in (("fused_us", fused), ("rope_apply_then_section_us", unfused), ("no_rope_us", plain)):
        gr = _captured(fn)
        res[name] = round(event_time_ms(lambda i=0: gr.replay(), iters, 2) * 1e3, 1)
        del gr
    del cache
    torch.cuda.empty_cache()
    res["rope_cost_fused_us"] = round(res["fused_us"] - res["no_rope_us"], 1)
    res["rope_cost_unfused_us"] = round(res["rope_apply_then_section_us"] - res["no_rope_us"], 1)
    return res


def _captured(fn):
    """fn captured once in a HIP graph (after one eager warm-up on a side stream)."""
    import torch

    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(g):
        fn()
    return g


def decode_step_times(dev, iters=20):
    """One layer's attention section for a decode step of the decode_b32 shape
    (32 sequences, contexts 256..4096, 32/8 heads, D=64, fp16): the batched
    paged path (the append fused into the paged attention launch pair; also
    timed as a separate append launch before it) against the
    reference's per-sequence structure (append, gather of the whole history,
    dense causal attention; engine/model/block.py:57-71), both on the GPU."""
    import torch

    from engine.attention import flash_attention
    from engine.cache import KVCacheConfig, PagedKVCache
    from engine.model import attention_section

    g = torch.Generator().manual_seed(2)
    ctx = torch.randint(256, 4097, (32,), generator=g).tolist()
    nb = sum(-(-(c + 1) // 16) for c in ctx) + 64
    cache = PagedKVCache(KVCacheConfig(1, 8, 64, nb, 16, torch.float16, dev))
    tables = [cache.new_sequence() for _ in ctx]
    for t, c in zip(tables, ctx):
        cache.prepare_step([t], c - 1)  # history of c - 1 tokens (pool contents are irrelevant to timing)
    step = cache.prepare_step(tables, 1)  # the new token of this step
    starts = [t.length - 1 for t in tables]
    # transposed views of (B, L, H, D) projections, as the model makes them (block.py:50-52)
    q = torch.randn(32, 1, 32, 64, generator=g).half().to(dev).transpose(1, 2)
    k = torch.randn(32, 1, 8, 64, generator=g).half().to(dev).transpose(1, 2)
    v = torch.randn(32, 1, 8, 64, generator=g).half().to(dev).transpose(1, 2)

    from engine.model.rope import RotaryEmbedding, rope_apply

    emb = RotaryEmbedding(64, 8192).to(dev)

    def paged(i=0):
        attention_section(q, k, v, 0, cache, step)

    def paged_two_launch(i=0):
        attention_section(q, k, v, 0, cache, step, fuse_append=False)

    def paged_rope(i=0):
        attention_section(q, k, v, 0, cache, step, rope=emb.tables)

    def paged_rope_unfused(i=0):
        pos = step.context_lens[:, None] - 1
        attention_section(rope_apply(q, emb.cos, emb.sin, pos), rope_apply(k, emb.cos, emb.sin, pos), v, 0, cache,
                          step)


    # the same section captured once in a HIP graph and replayed (no host work per layer)
    graph = _captured(paged)
    graph_two = _captured(paged_two_launch)
    graph_rope = _captured(paged_rope)
    graph_rope_unfused = _captured(paged_rope_unfused)

    def per_sequence(i=0):
        for b, t in enumerate(tables):
            cache.append(0, t, k[b].transpose(0, 1), v[b].transpose(0, 1), start=starts[b])
            kd, vd = cache.gather(0, t)
            flash_attention(q[b:b + 1], kd.transpose(0, 1).unsqueeze(0), vd.transpose(0, 1).unsqueeze(0),
                            causal=True, scale=0.125)

    t_paged = event_time_ms(paged, iters, 3)
    t_graph = event_time_ms(lambda i=0: graph.replay(), iters, 3)
    t_graph_two = event_time_ms(lambda i=0: graph_two.replay(), iters, 3)
    t_graph_rope = event_time_ms(lambda i=0: graph_rope.replay(), iters, 3)
    t_graph_rope_unfused = event_time_ms(lambda i=0: graph_rope_unfused.replay(), iters, 3)
    t_ref = event_time_ms(per_sequence, max(3, iters // 4), 1)
    del graph, graph_two, graph_rope, graph_rope_unfused, cache
    torch.cuda.empty_cache()
    return {"us": round(t_paged * 1e3, 2), "graph_replay_us": round(t_graph * 1e3, 2),
            "graph_replay_append_then_paged_us": round(t_graph_two * 1e3, 2),
            "graph_replay_rope_fused_us": round(t_graph_rope * 1e3, 2),
            "graph_replay_rope_apply_then_section_us": round(t_graph_rope_unfused * 1e3, 2),
            "per_sequence_gather_path_us": round(t_ref * 1e3, 1), "speedup": round(t_ref / t_paged, 1)}


def _stream(dev):
    """The current HIP stream (the capture stream while a graph is captured)."""
    import torch

    return torch.cuda.current_stream(dev).cuda_stream


def graph_time_ms(fn, n_inner=20, reps=20):
    """Per-call device time of a kernel shorter than one host launch: n_inner
    calls (rotating over their buffer copies) captured in one HIP graph, the
    graph replayed back to back after a settle phase. Eager timing of such a
    kernel measures the Python launch path instead of the GPU."""
    import torch

    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(n_inner):
            fn(i)
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(g):
        for i in range(n_inner):
            fn(i)
    ms = event_time_ms(lambda i=0: g.replay(), reps, 3)
    del g
    return ms / n_inner


SETTLE_S = 0.3  # seconds of untimed back-to-back work before a measurement
PEAK_CLOCK_GHZ = 2.4  # the clock the spec peak assumes


def gfx_clock_ghz(fn, seconds=0.8, skip=0.3):
    """Median GFX clock (GHz) while fn runs back to back for `seconds`, from
    the GPU metrics table (amdsmi, ~20 samples per second; the first `skip`
    seconds dropped while the clock settles). None when amdsmi is not
    available. The clock a kernel holds under load sets what fraction of the
    spec peak (which assumes 2.4 GHz) it can reach."""
    import threading

    import torch

    try:
        import amdsmi

        amdsmi.amdsmi_init()
        handle = amdsmi.amdsmi_get_processor_handles()[0]
    except Exception:  # noqa: BLE001 (no amdsmi, or no device it can open)
        return None
    samples = []
    stop = threading.Event()

    def sampler():
        while not stop.is_set():
            try:
                v = amdsmi.amdsmi_get_gpu_metrics_info(handle).get("current_gfxclk")
            except Exception:  # noqa: BLE001
                v = None
            if isinstance(v, list):  # per-XCD values
                v = max((x for x in v if isinstance(x, int) and x not in (0xFFFF, 0xFFFFFFFF)), default=None)
            if isinstance(v, int) and v not in (0xFFFF, 0xFFFFFFFF):
                samples.append((time.perf_counter(), v))
            time.sleep(0.05)

    th = threading.Thread(target=sampler, daemon=True)
    t0 = time.perf_counter()
    th.start()
    i = 0
    while time.perf_counter() - t0 < seconds:
        for _ in range(8):
            fn(i)
            i += 1
        torch.cuda.synchronize()
    stop.set()
    th.join()
    sel = sorted(v for t, v in samples if t - t0 >= skip)
    return sel[len(sel) // 2] / 1000.0 if sel else None


def settle(fn, seconds=SETTLE_S):
    """Run fn back-to-back, untimed, for about `seconds`: the GPU needs a few
    milliseconds of sustained load before its clock reaches the level it
    holds under continuous work (the first 40 prefill launches after idle
    run 10-15 % slower than the following ones)."""
    import torch

    t_end = time.perf_counter() + seconds
    i = 0
    while time.perf_counter() < t_end:
        for _ in range(8):
            fn(i)
            i += 1
        torch.cuda.synchronize()


def event_time_ms(fn, n, warmup, trials=3, mark=None):
    """Median over trials of (HIP-event time of n back-to-back launches) / n,
    after `warmup` launches and a settle phase. `mark` (optional): called at
    the start of each trial, its results collected in `event_time_ms.marks`."""
    import torch

    for i in range(warmup):
        fn(i)
    settle(fn)
    torch.cuda.synchronize()
    res = []
    event_time_ms.marks = []
    for _ in range(trials):
        if mark is not None:
            event_time_ms.marks.append(mark())
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        for i in range(n):
            fn(i)
        b.record()
        torch.cuda.synchronize()
        res.append(a.elapsed_time(b) / n)
    return statistics.median(res)


def _timed(fn, runs, min_run_s=0.25):
    """fn() once untimed, then the median over `runs` timed runs of the wall
    time per call, each run repeating fn enough times to last about
    `min_run_s` (a single call of a small case is too short for the clock).
    Returns (seconds per call, calls per run)."""
    t0 = time.perf_counter()
    fn()
    reps = max(1, math.ceil(min_run_s / max(time.perf_counter() - t0, 1e-6)))
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        times.append((time.perf_counter() - t0) / reps)
    return statistics.median(times), reps


def cpu_baselines(names=("prefill_s128", "prefill_s2048", "decode_b32", "verify_b8", "prefill_s16384")):
    """The reference's CPU path (kernels/ref/flash_attention_ref.py:8-56: fp32
    up-cast, repeat_interleave GQA, full score matrix, bottom-right mask,
    softmax, P.V), restated by the oracle, on every host core this process may
    use, for each workload: the prefill cases as one call over the whole
    batch (the S=16384 case chunked over query blocks, on a bounded sample),
    the paged cases per sequence as the reference's engine runs them
    (engine/model/block.py:56-71: gather the history through the block
    table, then attend). Each figure is in its workload's GPU unit (TFLOP/s
    of algorithmic work, or GB/s of algorithmic bytes)."""
    import torch
    from benchmarks import workloads
    from oracle import flash_attention_ref, flash_attention_ref_chunked, gather_ref

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    out = {}
    for name in names:
        c = workloads.WORKLOADS[name]()
        if name.startswith("prefill"):
            q, k, v = c.q.float(), c.k.float(), c.v.float()
            if name == "prefill_s16384":
                # bounded sample: batch 0, kv head 0 with its 4 query heads (1/8 of the work), every
                # query row, chunked over 2048-row query blocks (the full score matrix is 34 GB)
                qs, ks, vs = q[:, :4], k[:, :1], v[:, :1]
                t, _ = _timed(lambda: flash_attention_ref_chunked(qs, ks, vs, causal=True, q_chunk=2048), 1)
                flops = c.flops / 8
                sample = (f"kv head 0 with its 4 query heads over all 16384 rows (1/8 of the workload), "
                          f"fp32 oracle chunked over 2048-row query blocks, 1 run, {t:.2f} s")
            else:
                t, reps = _timed(lambda: flash_attention_ref(q, k, v, causal=True), 3)
                flops = c.flops
                sample = (f"full {name} workload through the unchunked fp32 oracle, median of 3 runs of {reps} "
                          f"call(s), {t * 1e3:.2f} ms per call")
            out[name] = {"value": round(flops / t / 1e12, 6), "unit": "TFLOP/s", "cores": torch.get_num_threads(),
                         "kind": "port", "sample": sample}
        else:
            B, Hq, Lq, D = c.q.shape
            lens = c.context_lens.tolist()

            def per_sequence():
                for b in range(B):
                    kd = gather_ref(c.k_pool, c.block_tables[b], lens[b]).float().transpose(0, 1).unsqueeze(0)
                    vd = gather_ref(c.v_pool, c.block_tables[b], lens[b]).float().transpose(0, 1).unsqueeze(0)
                    flash_attention_ref(c.q[b:b + 1].float(), kd, vd, causal=True)

            t, reps = _timed(per_sequence, 3)
            out[name] = {"value": round(c.bytes / t / 1e9, 4), "unit": "GB/s", "cores": torch.get_num_threads(),
                         "kind": "port",
                         "sample": f"full {name} workload, per sequence: gather through the block table, then "
                                   f"the fp32 oracle with Lq={Lq}; median of 3 runs of {reps} call(s), "
                                   f"{t * 1e3:.2f} ms per call"}
    return out


def main():
    args = parse()
    if args.traffic_probe:
        traffic_probe()
        return
    if args.probe:
        traffic_probe(tuple(n for n in args.probe.split(",") if n))
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; run with --gpus 1"}))
        sys.exit(2)
    import torch

    from benchmarks import workloads
    from engine.attention import flash_attention, prefill_kernel

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    case = workloads.prefill_s2048()
    q, k, v = case.q.to(dev), case.k.to(dev), case.v.to(dev)

    # Launches of the prefill kernel are counted in launch order, so a kernel
    # trace of this run can pick out the timed ones. The library names the
    # kernel this shape takes (on an MI355X the head-pair kernel: one
    # workgroup per 128-row query tile and pair of query heads).
    B_, H_, S_, D_ = case.q.shape
    kind = prefill_kernel(B_, H_, case.k.shape[1], S_, case.k.shape[2], D_, True, case.q.dtype)
    n_mt = (S_ + 127) // 128
    kernel_names = {
        "r64_heads": ("cie::flash_fwd_r64_kernel<0, 64, true>", "flash_fwd_r64_kernel<fp16, D=64, head pairs>",
                      n_mt * B_ * H_ // 2),
        "r64_rows": ("cie::flash_fwd_r64_kernel<0, 64, false>", "flash_fwd_r64_kernel<fp16, D=64, 64-row waves>",
                     ((S_ + 255) // 256) * B_ * H_),
        "flash_fwd": ("cie::flash_fwd_kernel<0, 64>", "flash_fwd_kernel<fp16, D=64>", n_mt * B_ * H_),
    }
    trace_name, roof_name, prefill_wg = kernel_names[kind]
    launches = [0]

    def headline(i=0):
        flash_attention(q, k, v, causal=True)
        launches[0] += 1

    # headline: K steps of the public entry point (after an untimed clock settle and W warmup steps)
    settle(headline)
    for _ in range(args.warmup):
        headline()
    torch.cuda.synchronize()
    first_timed = launches[0]
    t0 = time.perf_counter()
    for _ in range(args.steps):
        headline()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall / args.steps * 1e3
    value = case.flops / (ms_per_step / 1e3) / 1e12

    # roofline of the prefill kernel: event-timed back-to-back launches
    fl = FlashLaunch(case, dev)

    def roof(i=0):
        fl(i)
        launches[0] += 1

    n_roof = max(20, args.steps)
    kern_ms = event_time_ms(roof, n_roof, 3, mark=lambda: launches[0])
    print("[bench-launches] " + json.dumps({
        "kernel": trace_name, "workgroups": prefill_wg, "workload": "prefill_s2048",
        "headline_steps": [first_timed, args.steps],
        "roofline_trials": [[m, n_roof] for m in event_time_ms.marks]}), file=sys.stderr, flush=True)
    achieved = case.flops / (kern_ms / 1e3) / 1e12
    roof = {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_MFMA_F16_TFLOPS, "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_MFMA_F16_TFLOPS, 4), "traffic": traffic_from_summary(),
            "kernel": roof_name, "kernel_us": round(kern_ms * 1e3, 2)}
    # the clock the kernel holds under back-to-back load, and the fraction of
    # the peak at that clock (the spec peak assumes 2.4 GHz)
    ghz = gfx_clock_ghz(fl)
    roof["clock_ghz"] = ghz
    roof["frac_at_clock"] = round(achieved / (PEAK_MFMA_F16_TFLOPS * ghz / PEAK_CLOCK_GHZ), 4) if ghz else None

    extra = {}
    if not args.no_extra:
        # the paged workloads, and the same shapes at head_dim 128
        for name in ("decode_b32", "verify_b8", "decode_b32_d128", "verify_b8_d128"):
            c = workloads.WORKLOADS[name]()
            # with the host-built plan (what an engine step uses, uploaded once for all layers) and
            # with the schedule derived on the device from the lengths alone
            pl = PagedLaunch(c, dev, planned=True)
            ms = event_time_ms(pl, 40 * pl.copies, 2 * pl.copies)
            gbs = c.bytes / (ms / 1e3) / 1e9
            # the same planned calls captured in a HIP graph (as an engine's decode step runs them)
            ms_graph = graph_time_ms(pl, n_inner=max(20, pl.copies))
            gbs_graph = c.bytes / (ms_graph / 1e3) / 1e9
            split = pl.plan.split
            del pl
            pd = PagedLaunch(c, dev)
            ms_dev = event_time_ms(pd, 40 * pd.copies, 2 * pd.copies)
            gbs_dev = c.bytes / (ms_dev / 1e3) / 1e9
            extra[name] = {"GB/s": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "us": round(ms * 1e3, 2),
                           "schedule": "host plan", "split_sequences": split,
                           "graph_replay": {"GB/s": round(gbs_graph, 1), "frac_hbm": round(gbs_graph / PEAK_HBM_GBS, 4),
                                            "us": round(ms_graph * 1e3, 2)},
                           "device_schedule": {"GB/s": round(gbs_dev, 1), "frac_hbm": round(gbs_dev / PEAK_HBM_GBS, 4),
                                               "us": round(ms_dev * 1e3, 2)},
                           "bytes": int(c.bytes), "pool_copies": pd.copies,
                           "dtype": "fp16" if c.q.dtype == torch.float16 else "bf16"}
            del pd
        for name, (B, L) in (("append_prefill_b4_l2048", (4, 2048)), ("append_decode_b32", (32, 1))):
            al = AppendLaunch(B, L, dev)
            ms = graph_time_ms(al, n_inner=max(20, al.copies))
            gbs = al.bytes / (ms / 1e3) / 1e9
            extra[name] = {"GB/s": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "us": round(ms * 1e3, 2),
                           "bytes": int(al.bytes), "copies": al.copies, "dtype": "fp16", "timing": "graph replay"}
            del al
        rl = RopeLaunch(dev)
        ms = graph_time_ms(rl, n_inner=rl.copies)
        gbs = rl.bytes / (ms / 1e3) / 1e9
        extra["rope_q_prefill_b4_s2048"] = {"GB/s": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM_GBS, 4),
                                            "us": round(ms * 1e3, 2), "bytes": int(rl.bytes), "copies": rl.copies,
                                            "dtype": "fp16", "timing": "graph replay"}
        del rl
        extra["prefill_section_b4_s2048_rope"] = prefill_section_times(dev)
        for M in (1, 4, 16, 64, 512):
            il = Int8Launch(M, dev)
            ms = graph_time_ms(il, n_inner=il.copies)
            gbs = il.bytes / (ms / 1e3) / 1e9
            tfs = il.flops / (ms / 1e3) / 1e12
            extra[f"int8_matmul_m{M}_n4096_k4096"] = {
                "us": round(ms * 1e3, 2), "TFLOP/s": round(tfs, 2), "frac_mfma": round(tfs / PEAK_MFMA_F16_TFLOPS, 4),
                "GB/s": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "weight_copies": il.copies,
                "dtype": "fp16 x int8", "timing": "graph replay"}
            del il
        extra["decode_step_b32_one_layer"] = decode_step_times(dev)
        c5 = workloads.prefill_s16384()
        f5 = FlashLaunch(c5, dev)
        ms = event_time_ms(f5, 5, 1)
        t5 = c5.flops / (ms / 1e3) / 1e12
        ghz5 = gfx_clock_ghz(f5, seconds=2.0, skip=0.5)
        extra["prefill_s16384"] = {"TFLOP/s": round(t5, 2), "frac_mfma": round(t5 / PEAK_MFMA_F16_TFLOPS, 4),
                                   "us": round(ms * 1e3, 1), "dtype": "bf16", "clock_ghz": ghz5,
                                   "frac_mfma_at_clock": round(t5 / (PEAK_MFMA_F16_TFLOPS * ghz5 / PEAK_CLOCK_GHZ), 4)
                                   if ghz5 else None}
        del f5
        # the CPU-oracle case (fp32 on the host) run on the GPU with its tensors cast to fp16
        c1 = workloads.prefill_s128(dtype=torch.float16)
        f1 = FlashLaunch(c1, dev)
        ms = graph_time_ms(f1, n_inner=20)
        t1 = c1.flops / (ms / 1e3) / 1e12
        extra["prefill_s128"] = {"TFLOP/s": round(t1, 3), "frac_mfma": round(t1 / PEAK_MFMA_F16_TFLOPS, 5),
                                 "us": round(ms * 1e3, 2), "dtype": "fp16", "timing": "graph replay",
                                 "note": "32 workgroups: latency-bound, far too small to fill 256 CUs"}
        del f1
        torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu_baseline:
        cpus = cpu_baselines() if not args.no_extra else cpu_baselines(("prefill_s2048",))
        cpu = cpus.pop("prefill_s2048")
        for name, base in cpus.items():
            extra.setdefault(name, {})["cpu_baseline"] = base

    line = {
        "metric": "prefill attention TFLOP/s + paged-decode KV GB/s (% roofline) on 1 MI355X",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {"workload": "prefill_s2048", "B": 4, "S": 2048, "Hq": 32, "Hk": 8, "head_dim": 64,
                   "causal": True, "flop_per_step": case.flops},
        "roofline": roof,
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
