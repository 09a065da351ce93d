"""Per-workgroup timelines of the head-pair prefill kernel and of the paged
decode / verify kernel, from the library's timeline build.

    python3 custom-inference-engine_amd/build_lib.py --timeline
    cd custom-inference-engine_amd && python3 -m benchmarks.timeline [workload ...]
    (default: prefill_s2048 decode_b32 verify_b8)

The timeline build (CIE_TIMELINE) has thread 0 of every workgroup write
s_memrealtime stamps (100 MHz) at fixed points of its life, plus where it
ran (XCC_ID, HW_ID) and its amount of work. Each workload runs back to back
(the prefill 400 times; the paged ones with the host-built plan, rotating
over pool copies that together exceed 512 MiB, as the bench does), and the
stamps of the last launch are read back and summarised:

- prefill: entry -> q rows in registers -> first K/V tile in LDS -> loop
  start -> loop end -> stores issued, per workgroup (percentiles), the time
  per 32-key step, the gap between a workgroup's last store and the next
  workgroup's start on its CU, and the share of the span each CU holds 0, 1
  or 2 workgroups;
- paged: entry -> schedule in LDS -> first tile in LDS -> tile loop done ->
  end, per workgroup, and the spread of the workgroups' ends by XCD.
"""

from __future__ import annotations

import ctypes
import os
import sys

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(PKG, "libcie_attn_timeline.so")
os.environ["CIE_ATTN_LIB"] = LIB  # read when engine._lib is imported

import numpy as np  # noqa: E402
import torch  # noqa: E402

from benchmarks import workloads  # noqa: E402
from engine import _lib  # noqa: E402
from engine.attention import flash_attention, paged_attention, paged_plan, prefill_kernel  # noqa: E402

SLOTS = 8
MAX_WG = 16384
TICK_US = 0.01  # s_memrealtime: 100 MHz


def _read(fn, nwg: int) -> np.ndarray:
    buf = np.zeros(MAX_WG * SLOTS, dtype=np.uint64)
    rc = fn(ctypes.c_void_p(buf.ctypes.data), ctypes.c_size_t(buf.nbytes))
    if rc != 0:
        raise RuntimeError(f"timeline copy failed ({rc})")
    return buf[: nwg * SLOTS].reshape(nwg, SLOTS).astype(np.int64)


def _cu_key(where: np.ndarray) -> np.ndarray:
    hw = where & 0xFFFFFFFF
    xcc = (where >> 32) & 0xF
    return xcc * 1000 + ((hw >> 13) & 0x7) * 100 + ((hw >> 12) & 1) * 16 + ((hw >> 8) & 0xF)


def _pct(x: np.ndarray, ps=(5, 50, 95)) -> str:
    return " / ".join(f"{np.percentile(x, p):.2f}" for p in ps)


def prefill(name: str, dev) -> None:
    c = workloads.WORKLOADS[name]()
    q, k, v = c.q.to(dev), c.k.to(dev), c.v.to(dev)
    out = torch.empty_like(q)
    B, Hq, S, _ = q.shape
    if prefill_kernel(B, Hq, c.k.shape[1], S, S, q.shape[-1], True, q.dtype) != "r64_heads":
        print(f"## {name}: not the head-pair kernel; skipped\n")
        return
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    n = 400
    for i in range(n):
        if i == n - 20:
            e0.record()
        flash_attention(q, k, v, causal=True, out=out)
    e1.record()
    torch.cuda.synchronize()
    nwg = B * Hq // 2 * ((S + 127) // 128)
    t = _read(_lib.load().cie_timeline_flash, nwg)
    t0 = t[:, 0].min()
    us = lambda i: (t[:, i] - t0) * TICK_US  # noqa: E731
    st, lp, le, en, qd, ft = us(0), us(1), us(2), us(3), us(6), us(7)
    ntl = t[:, 4]
    key = _cu_key(t[:, 5])
    span = en.max() - st.min()
    print(f"## {name}: {nwg} workgroups, {e0.elapsed_time(e1) / 20 * 1e3:.1f} us per launch (last 20), "
          f"stamped span {span:.1f} us\n")
    print("| interval (us, p5 / p50 / p95) | value |")
    print("|---|---:|")
    print(f"| entry -> q rows in registers | {_pct(qd - st)} |")
    print(f"| -> first K/V tile in LDS | {_pct(ft - qd)} |")
    print(f"| -> loop start (first QK^T, row max) | {_pct(lp - ft)} |")
    print(f"| loop | {_pct(le - lp)} |")
    print(f"| loop per 32-key step | {_pct((le - lp) / np.maximum(ntl, 1))} |")
    print(f"| loop end -> stores issued | {_pct(en - le)} |")
    gaps, occ = [], np.zeros(4)
    grid = np.linspace(0, span, 2001)
    for cu in np.unique(key):
        m = key == cu
        s_, e_ = st[m], en[m]
        act = ((grid[:, None] >= s_[None, :]) & (grid[:, None] < e_[None, :])).sum(1)
        for j in range(4):
            occ[j] += (np.minimum(act, 3) == j).sum()
        ends = np.sort(e_)
        for s1 in np.sort(s_)[2:]:
            prev = ends[ends <= s1]
            if len(prev):
                gaps.append(s1 - prev.max())
    occ /= occ.sum()
    if gaps:
        print(f"| a workgroup's last store -> the next start on its CU | {_pct(np.array(gaps))} |")
    print(f"\nLoops are {(le - lp).sum() / (en - st).sum():.3f} of the workgroups' lifetimes; the CUs hold "
          f"0 / 1 / 2 workgroups for {occ[0]:.3f} / {occ[1]:.3f} / {occ[2]:.3f} of the span.\n")


def paged(name: str, dev) -> None:
    c = workloads.WORKLOADS[name]()
    B, Hq, Lq, D = c.q.shape
    nb, bs, Hk, _ = c.k_pool.shape
    pool_bytes = 2 * c.k_pool.numel() * c.k_pool.element_size()
    copies = max(1, -(-(512 << 20) // pool_bytes))
    pools = [(c.k_pool.to(dev), c.v_pool.to(dev)) for _ in range(copies)]
    q, bt, ln = c.q.to(dev), c.block_tables.to(dev), c.context_lens.to(dev)
    mc = int(c.context_lens.max())
    plan = paged_plan(c.context_lens, c.block_tables, Hq=Hq, Hk=Hk, Lq=Lq, D=D, num_blocks=nb, block_size=bs,
                      max_context=mc, device=dev)
    out = torch.empty_like(q)
    n = 40 * copies
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for i in range(n):
        if i == n - 2 * copies:
            e0.record()
        kp, vp = pools[i % copies]
        paged_attention(q, kp, vp, bt, ln, causal=True, max_context=mc, plan=plan, out=out)
    e1.record()
    torch.cuda.synchronize()
    hdr = plan.data.cpu()
    nwg = int(hdr[3]) * int(hdr[8])  # ranges x head groups
    t = _read(_lib.load().cie_timeline_paged, nwg)
    live = t[:, 6] > 0  # workgroups with tiles
    t0 = t[:, 0].min()
    us = lambda i: (t[:, i] - t0) * TICK_US  # noqa: E731
    st, sc, ft, le, en = us(0), us(1), us(2), us(3), us(4)
    xcc = (t[:, 5] >> 32) & 0xF
    print(f"## {name}: {nwg} workgroups ({int(live.sum())} with tiles), "
          f"{e0.elapsed_time(e1) / (2 * copies) * 1e3:.1f} us per call (pair, last {2 * copies})\n")
    print("| time from the first entry (us, p5 / p50 / p95) | value |")
    print("|---|---:|")
    print(f"| entry | {_pct(st[live])} |")
    print(f"| schedule in LDS | {_pct(sc[live])} |")
    print(f"| first tile in LDS | {_pct(ft[live])} |")
    print(f"| tile loop done | {_pct(le[live])} |")
    print(f"| end (last {en[live].max():.2f}) | {_pct(en[live])} |")
    print(f"| tiles per workgroup | {_pct(t[live, 6].astype(float))} |")
    per_xcd = [f"{en[live & (xcc == x)].mean():.1f}" for x in np.unique(xcc[live])]
    print(f"\nMean end by XCD (us): {', '.join(per_xcd)}; correlation of a workgroup's end with its "
          f"first tile's arrival: {np.corrcoef(ft[live], en[live])[0, 1]:.2f}.\n")


def main(names: list[str]) -> None:
    if not os.path.exists(LIB):
        sys.stderr.write(f"{LIB} missing: run custom-inference-engine_amd/build_lib.py --timeline first\n")
        raise SystemExit(1)
    dev = torch.device("cuda:0")
    for name in names:
        (prefill if name.startswith("prefill") else paged)(name, dev)
        torch.cuda.empty_cache()


if __name__ == "__main__":
    main(sys.argv[1:] or ["prefill_s2048", "decode_b32", "verify_b8"])
