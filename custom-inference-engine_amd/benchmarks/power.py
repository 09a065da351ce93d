"""Board power and GFX clock while a prefill workload runs back to back.

    python3 -m benchmarks.power [workload ...]   (default: prefill_s2048 prefill_s16384)

For each workload: launches of the public prefill entry point run back to
back for a few seconds while a thread samples the GPU's metrics table
(amdsmi, ~20 Hz: current socket power, current GFX clock, GFX activity,
hotspot temperature); the first 0.5 s of each phase (clock and power
settling) is dropped. Prints one markdown row per phase (medians over the
samples) and the kernel time per launch over the phase (HIP events), then
an idle row, and the board's power cap as amdsmi reports it. A workload
whose power sits at the cap while its clock falls below the peak is
power-bound.
"""

from __future__ import annotations

import sys
import threading
import time

import torch

from benchmarks import workloads
from engine.attention import flash_attention

SETTLE_S = 0.5
SAMPLE_S = 0.05


def _median(xs: list) -> float | None:
    xs = sorted(x for x in xs if isinstance(x, (int, float)) and x not in (0xFFFF, 0xFFFFFFFF))
    return xs[len(xs) // 2] if xs else None


def _metric(m: dict, key: str):
    v = m.get(key)
    if isinstance(v, list):  # per-XCD values: the largest valid one
        v = [x for x in v if isinstance(x, (int, float)) and x not in (0xFFFF, 0xFFFFFFFF)]
        v = max(v) if v else None
    return v


def main(names: list[str]) -> None:
    import amdsmi

    amdsmi.amdsmi_init()
    handle = amdsmi.amdsmi_get_processor_handles()[0]
    samples: list[tuple[float, dict]] = []
    stop = threading.Event()

    def sampler() -> None:
        while not stop.is_set():
            samples.append((time.time(), amdsmi.amdsmi_get_gpu_metrics_info(handle)))
            time.sleep(SAMPLE_S)

    th = threading.Thread(target=sampler, daemon=True)
    th.start()
    dev = torch.device("cuda:0")
    phases = []
    for name in names:
        c = workloads.WORKLOADS[name]()
        q, k, v = c.q.to(dev), c.k.to(dev), c.v.to(dev)
        out = torch.empty_like(q)
        flash_attention(q, k, v, causal=True, out=out)
        torch.cuda.synchronize()
        per_sync = max(1, int(2e-3 / max(c.flops / 1e15, 1e-9)))  # ~2 ms of launches between host checks
        secs = 3.0 if c.flops < 1e12 else 4.0
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.time()
        e0.record()
        n = 0
        while time.time() - t0 < secs:
            for _ in range(per_sync):
                flash_attention(q, k, v, causal=True, out=out)
            n += per_sync
            torch.cuda.synchronize()
        e1.record()
        torch.cuda.synchronize()
        phases.append((name, t0 + SETTLE_S, time.time(), e0.elapsed_time(e1) / n * 1e3, c.flops))
        del q, k, v, out
        time.sleep(SETTLE_S)
    t_idle = time.time()
    time.sleep(1.0)
    phases.append(("idle", t_idle + 0.2, time.time(), None, None))
    stop.set()
    th.join()

    try:  # raw fields (amdsmi reports microwatts)
        print(f"power cap: {amdsmi.amdsmi_get_power_cap_info(handle)}\n")
    except Exception as e:  # noqa: BLE001 (an amdsmi without the query)
        print(f"power cap: not reported ({e})\n")
    print("| phase | samples | socket power W | GFX clock MHz | GFX activity % | hotspot C | us per launch | TFLOP/s |")
    print("|---|---:|---:|---:|---:|---:|---:|---:|")
    for name, a, b, us, flops in phases:
        sel = [m for t, m in samples if a <= t <= b]
        cols = [_median([_metric(m, key) for m in sel])
                for key in ("current_socket_power", "current_gfxclk", "average_gfx_activity", "temperature_hotspot")]
        cols = ["-" if x is None else str(x) for x in cols]
        tf = f"{flops / (us * 1e-6) / 1e12:.1f}" if us else "-"
        print(f"| {name} | {len(sel)} | {' | '.join(cols)} | {us:.1f} | {tf} |" if us else
              f"| {name} | {len(sel)} | {' | '.join(cols)} | - | - |")


if __name__ == "__main__":
    main(sys.argv[1:] or ["prefill_s2048", "prefill_s16384"])
