"""Builds libcie_attn.so (the gfx950 attention library) in-tree.

    python custom-inference-engine_amd/build_lib.py              # the library
    python custom-inference-engine_amd/build_lib.py --timeline   # its timeline build

Every source is compiled for gfx950 with hipcc (objects under ``_build/``,
compiled in parallel) and linked into ``custom-inference-engine_amd/libcie_attn.so``,
which the Python layer loads with ctypes. Packed-FP32 VALU instructions are
disabled for all device code.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
INCLUDE = os.path.join(REPO, "include")
BUILD = os.path.join(PKG_DIR, "_build")
LIB_PATH = os.path.join(PKG_DIR, "libcie_attn.so")
TIMELINE_LIB_PATH = os.path.join(PKG_DIR, "libcie_attn_timeline.so")
# stand-alone microbenchmarks (benchmarks/<name>.hip -> _build/<name>), not part of the library
BENCH_TOOLS = ("vector_rates", "read_floor", "prefill_step")

SOURCES = ["capi.cpp", "paged_plan.cpp", "flash_fwd.hip", "paged_fwd.hip", "kv_append.hip", "rope.hip",
           "int8_gemm.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in VGPRs: the online-softmax rescale multiplies them on the VALU
    "-Xarch_device", "-mllvm=-amdgpu-mfma-vgpr-form=1",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature; that warning is noise
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{err}\n{res.stdout}")
    if err.strip():
        sys.stderr.write(err + "\n")


def _build_lib(out: str, objdir: str, defines: list[str]) -> None:
    os.makedirs(objdir, exist_ok=True)
    objs = []
    cmds = []
    for src in SOURCES:
        obj = os.path.join(objdir, os.path.splitext(src)[0] + ".o")
        lang = ["-x", "hip"] if src.endswith(".hip") else []
        cmds.append([HIPCC, *COMMON, *defines, *lang, "-c", os.path.join(CSRC, src), "-o", obj])
        objs.append(obj)
    with ThreadPoolExecutor(max_workers=min(len(cmds), os.cpu_count() or 1)) as ex:
        list(ex.map(_run, cmds))
    tmp = out + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp])
    os.replace(tmp, out)


def build(verbose: bool = False) -> str:
    """Compile every source and link the shared library; returns its path."""
    os.makedirs(BUILD, exist_ok=True)
    _build_lib(LIB_PATH, BUILD, [])
    # the microbenchmarks behind benchmarks/vector_rates.py, read_floor.py and prefill_step.py
    tools = [[HIPCC, *COMMON, "-x", "hip", os.path.join(PKG_DIR, "benchmarks", t + ".hip"), "-o", os.path.join(BUILD, t)]
             for t in BENCH_TOOLS]
    with ThreadPoolExecutor(max_workers=len(tools)) as ex:
        list(ex.map(_run, tools))
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


def build_timeline(verbose: bool = False) -> str:
    """The library once more with CIE_TIMELINE defined (per-workgroup stamps of
    the head-pair prefill and paged kernels, read by benchmarks/timeline.py);
    a measurement build, next to the product library, never loaded by it."""
    _build_lib(TIMELINE_LIB_PATH, os.path.join(BUILD, "timeline"), ["-DCIE_TIMELINE"])
    if verbose:
        print(f"built {TIMELINE_LIB_PATH}")
    return TIMELINE_LIB_PATH


if __name__ == "__main__":
    if "--timeline" in sys.argv[1:]:
        build_timeline(verbose=True)
    else:
        build(verbose=True)
