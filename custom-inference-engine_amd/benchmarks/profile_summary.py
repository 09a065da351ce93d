"""Text summaries of rocprofv3 output for the profiles kept with the sources.

    python -m benchmarks.profile_summary trace TRACE_CSV BENCH_STDOUT BENCH_STDERR
    python -m benchmarks.profile_summary mfma COUNTER_CSV [COUNTER_CSV ...]
    python -m benchmarks.profile_summary traffic FETCH_CSV WRITE_CSV

(run with ``custom-inference-engine_amd`` on ``PYTHONPATH``). Each prints
a markdown summary on stdout.

trace
    ``rocprofv3 --kernel-trace --stats --output-format csv`` of ``bench.py``:
    per-kernel statistics of the whole run, then the launches of the prefill
    kernel that the bench timed, picked out by the launch numbers bench.py
    prints on stderr (``[bench-launches] {...}``), set against the bench's
    own ``ms_per_step`` and ``roofline.kernel_us`` from its JSON line.
mfma
    ``rocprofv3 --pmc`` passes over ``bench.py --probe ...``: MFMA busy cycles
    per SIMD against the shader cycles of the dispatch, i.e. MFMA
    utilisation at the clock the kernel ran at, and the clock itself.
traffic
    ``--pmc FETCH_SIZE`` and ``--pmc WRITE_SIZE`` passes over ``bench.py
    --traffic-probe``: HBM bytes per dispatch, each counter scaled by what it
    reads for the probe's 256 MiB copy.
"""

from __future__ import annotations

import collections
import csv
import json
import statistics
import sys

XCDS = 8            # accelerator complex dies of one MI355X; GRBM_GUI_ACTIVE is summed over them
SIMDS = 256 * 4     # 256 CUs x 4 SIMDs; SQ_VALU_MFMA_BUSY_CYCLES is summed over them
COPY_BYTES = 256 << 20
PROBE_WORKLOADS = {1024: "prefill_s2048", 4096: "prefill_s16384"}  # by workgroup count
# head_dim 64 runs the head-pair kernel (prefill_s2048), head_dim 128 the interleaved one
PREFILL_KERNELS = ("cie::flash_fwd_kernel", "cie::flash_fwd_r64_kernel", "cie::flash_fwd_il_kernel")


def _grid(r: dict) -> tuple[int, int]:
    """(workgroups, threads per workgroup) of a trace or counter row."""
    if "Grid_Size_X" in r:
        wg = int(r["Workgroup_Size_X"]) * int(r["Workgroup_Size_Y"]) * int(r["Workgroup_Size_Z"])
        grid = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
    else:
        wg, grid = int(r["Workgroup_Size"]), int(r["Grid_Size"])
    return grid // wg, wg


def _name(r: dict) -> str:
    n = r["Kernel_Name"]
    if n.startswith("void cie::"):
        n = n[len("void "):].split("(")[0]
    return n


def _dur_us(r: dict) -> float:
    return (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3


def _stats(v: list[float]) -> str:
    return f"{statistics.mean(v):.2f} | {statistics.median(v):.2f} | {min(v):.2f} | {max(v):.2f}"


def trace(trace_csv: str, bench_stdout: str, bench_stderr: str) -> None:
    rows = sorted(csv.DictReader(open(trace_csv)), key=lambda r: int(r["Start_Timestamp"]))
    line = json.loads(next(ln for ln in open(bench_stdout) if ln.startswith("{")))
    marks = json.loads(next(ln for ln in open(bench_stderr) if ln.startswith("[bench-launches] "))
                       .split(" ", 1)[1])
    groups = collections.defaultdict(list)
    for r in rows:
        groups[(_name(r), *_grid(r))].append(_dur_us(r))
    total = sum(sum(v) for v in groups.values())
    print("All dispatches of the run, by kernel and launch grid (durations: end - start, us; calls include")
    print("warm-up, clock-settle and untimed launches):\n")
    print("| kernel | workgroups x threads | calls | avg us | median us | min us | max us | % time |")
    print("|---|---:|---:|---:|---:|---:|---:|---:|")
    for (name, wg, thr), v in sorted(groups.items(), key=lambda kv: -sum(kv[1]))[:20]:
        print(f"| `{name[:100]}` | {wg} x {thr} | {len(v)} | {_stats(v)} | {100 * sum(v) / total:.2f} |")

    kern = [r for r in rows if _name(r) == marks["kernel"] and _grid(r)[0] == marks["workgroups"]]
    a, k = marks["headline_steps"]
    head = kern[a:a + k]
    print(f"\nLaunches of `{marks['kernel']}` with {marks['workgroups']} workgroups "
          f"({marks['workload']}), numbered in launch order: {len(kern)} in the run.\n")
    print("| region (launch numbers from bench.py) | launches | avg us | median us | min us | max us |")
    print("|---|---:|---:|---:|---:|---:|")
    hd = [_dur_us(r) for r in head]
    print(f"| headline steps [{a}, {a + k}) | {len(hd)} | {_stats(hd)} |")
    tr_all = []
    for m, n in marks["roofline_trials"]:
        tr = [_dur_us(r) for r in kern[m:m + n]]
        tr_all += tr
        print(f"| roofline trial [{m}, {m + n}) | {len(tr)} | {_stats(tr)} |")
    span = (int(head[-1]["End_Timestamp"]) - int(head[0]["Start_Timestamp"])) / 1e3 / len(head)
    flops = line["config"]["flop_per_step"]
    peak = line["roofline"]["peak"]
    print("\nAgainst the bench's JSON line of the same run:\n")
    print(f"- bench `ms_per_step` (host wall clock over the {k} headline steps): {line['ms_per_step'] * 1e3:.2f} us")
    print(f"- trace, headline steps: first start to last end / {k} = {span:.2f} us; "
          f"mean kernel duration {statistics.mean(hd):.2f} us")
    print(f"- bench `roofline.kernel_us` (HIP events, median of 3 trials): {line['roofline']['kernel_us']:.2f} us")
    print(f"- trace, roofline trials: mean kernel duration {statistics.mean(tr_all):.2f} us")
    fr = flops / (statistics.mean(tr_all) * 1e-6) / 1e12 / peak
    print(f"- frac recomputed from the trace: {flops:.6g} FLOP / {statistics.mean(tr_all):.2f} us / "
          f"{peak} TFLOP/s = {fr:.4f} (bench `roofline.frac`: {line['roofline']['frac']})")


def _counter_rows(paths: list[str]) -> dict:
    out = collections.OrderedDict()
    for path in paths:
        for r in csv.DictReader(open(path)):
            key = (path, r["Dispatch_Id"])
            d = out.setdefault(key, {"name": _name(r), "grid": _grid(r), "dur_us": _dur_us(r)})
            d[r["Counter_Name"]] = float(r["Counter_Value"])
    return out


def mfma(paths: list[str]) -> None:
    rows = [d for d in _counter_rows(paths).values() if d["name"].startswith(PREFILL_KERNELS)]
    print("| dispatch | workload | us | MFMA instr | MFMA busy / SIMD (cycles) | shader cycles per XCD "
          "| clock GHz | MFMA busy | fp16+bf16 MOPS x 512 (GFLOP) |")
    print("|---|---|---:|---:|---:|---:|---:|---:|---:|")
    per = collections.defaultdict(list)
    for d in rows:
        if "SQ_VALU_MFMA_BUSY_CYCLES" not in d or "GRBM_GUI_ACTIVE" not in d:
            continue
        wl = PROBE_WORKLOADS.get(d["grid"][0], "?")
        cyc = d["GRBM_GUI_ACTIVE"] / XCDS
        busy = d["SQ_VALU_MFMA_BUSY_CYCLES"] / SIMDS
        ghz = cyc / (d["dur_us"] * 1e3)
        mops = d.get("SQ_INSTS_VALU_MFMA_MOPS_F16", 0.0) + d.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", 0.0)
        per[wl].append((busy / cyc, ghz, d["dur_us"]))
        print(f"| `{d['name']}` | {wl} | {d['dur_us']:.1f} | {d.get('SQ_INSTS_MFMA', 0):.0f} | {busy:.0f} | {cyc:.0f} "
              f"| {ghz:.3f} | {100 * busy / cyc:.1f} % | {mops * 512 / 1e9:.2f} |")
    print()
    for wl, v in per.items():
        u = statistics.mean(x[0] for x in v)
        g = statistics.mean(x[1] for x in v)
        print(f"- {wl}: MFMA busy {100 * u:.1f} % of the shader cycles at {g:.2f} GHz; against the spec peak "
              f"(2.4 GHz) that is {100 * u * g / 2.4:.1f} % of the dense MFMA rate")
    # instruction mix and issue state per wave, where those counters were collected
    # (every pass runs the same probe, so the n-th dispatch of a workload is the same launch)
    merged = collections.defaultdict(dict)
    seen = collections.Counter()
    for path in paths:
        seen.clear()
        for d in _counter_rows([path]).values():
            if not d["name"].startswith(PREFILL_KERNELS):
                continue
            wl = PROBE_WORKLOADS.get(d["grid"][0], "?")
            key = (wl, seen[wl])
            seen[wl] += 1
            merged[key].update(d)
    keys = ("SQ_INSTS_VALU", "SQ_INSTS_MFMA", "SQ_INSTS_SALU", "SQ_INSTS_LDS", "SQ_WAVE_CYCLES",
            "SQ_ACTIVE_INST_ANY", "SQ_ACTIVE_INST_VALU", "SQ_WAIT_INST_ANY", "SQ_WAIT_INST_LDS", "SQ_LDS_BANK_CONFLICT")
    rows = [(k, d) for k, d in sorted(merged.items()) if all(x in d for x in keys)]
    if rows:
        print("\nPer wave (counter / waves of the dispatch; the issue-state counters as a share of "
              "SQ_WAVE_CYCLES, which counts in the same units):\n")
        print("| workload | VALU instr | MFMA instr | SALU instr | LDS instr | active any | active VALU "
              "| waiting on a dependency | waiting on LDS | LDS bank conflicts |")
        print("|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|")
        for (wl, i), d in rows:
            waves = d["grid"][0] * d["grid"][1] / 64
            wc = d["SQ_WAVE_CYCLES"]
            print(f"| {wl} #{i} | {d['SQ_INSTS_VALU'] / waves:.0f} | {d['SQ_INSTS_MFMA'] / waves:.0f} "
                  f"| {d['SQ_INSTS_SALU'] / waves:.0f} | {d['SQ_INSTS_LDS'] / waves:.0f} "
                  f"| {100 * d['SQ_ACTIVE_INST_ANY'] / wc:.1f} % | {100 * d['SQ_ACTIVE_INST_VALU'] / wc:.1f} % "
                  f"| {100 * d['SQ_WAIT_INST_ANY'] / wc:.1f} % | {100 * d['SQ_WAIT_INST_LDS'] / wc:.1f} % "
                  f"| {d['SQ_LDS_BANK_CONFLICT']:.0f} |")


def _largest(v: list[float]) -> list[float]:
    top = max(v)
    return [x for x in v if x >= 0.9 * top]


def traffic(fetch_csv: str, write_csv: str) -> None:
    f = _counter_rows([fetch_csv])
    w = _counter_rows([write_csv])
    fl = [d for d in f.values()]
    wl = [d for d in w.values()]
    # the probe's three 256 MiB copies: the largest copy dispatches (the
    # workloads' host-to-device uploads are copy dispatches too)
    copies_f = _largest([d["FETCH_SIZE"] for d in fl if "copyBuffer" in d["name"]])
    copies_w = _largest([d["WRITE_SIZE"] for d in wl if "copyBuffer" in d["name"]])
    sf = COPY_BYTES / 1024 / statistics.mean(copies_f)
    sw = COPY_BYTES / 1024 / statistics.mean(copies_w)
    print(f"Calibration: the 256 MiB copy reads {COPY_BYTES // 1024} KiB; FETCH_SIZE reports "
          f"{statistics.mean(copies_f):.2f} KiB (scale {sf:.5f}), WRITE_SIZE {statistics.mean(copies_w):.2f} KiB "
          f"(scale {sw:.5f}).\n")
    print("| dispatch | workgroups | FETCH_SIZE KiB | WRITE_SIZE KiB | fetch bytes | write bytes |")
    print("|---|---:|---:|---:|---:|---:|")
    for df, dw in zip(fl, wl):
        if not df["name"].startswith("cie::"):
            continue
        print(f"| `{df['name']}` | {df['grid'][0]} | {df['FETCH_SIZE']:.2f} | {dw['WRITE_SIZE']:.2f} "
              f"| {df['FETCH_SIZE'] * sf * 1024:.0f} | {dw['WRITE_SIZE'] * sw * 1024:.0f} |")


def main(argv: list[str]) -> None:
    cmd, args = argv[0], argv[1:]
    if cmd == "trace":
        trace(*args)
    elif cmd == "mfma":
        mfma(args)
    elif cmd == "traffic":
        traffic(*args)
    else:
        raise SystemExit(__doc__)


if __name__ == "__main__":
    main(sys.argv[1:])
