"""The head_dim-64 head-pair prefill step in isolation: its parts (MFMAs,
softmax, row sums, LDS fragment reads, lazy-max check, barrier, tile copies,
wave priority) switched on one at a time in a loop of 2000 steps per wave.

    python3 -m benchmarks.prefill_step

Runs the microbenchmark that build_lib.py compiles from prefill_step.hip
(``_build/prefill_step``) and prints its markdown table: per row the shader
cycles per step and wave, the MFMA rate against the MFMA-only row, and the
equivalent fraction of the dense fp16 peak at the clock the row ran at.
"""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(os.path.dirname(HERE), "_build", "prefill_step")


def main() -> int:
    if not os.path.exists(BIN):
        sys.stderr.write(f"{BIN} missing: run custom-inference-engine_amd/build_lib.py first\n")
        return 1
    return subprocess.run([BIN]).returncode


if __name__ == "__main__":
    sys.exit(main())
