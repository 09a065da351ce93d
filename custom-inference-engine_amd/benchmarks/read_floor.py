"""Floor of a streaming read: the time a kernel that only reads S bytes
takes on the GPU, for the byte counts of the bench's INT8 decode-size GEMV
(16 MiB of weights) and its paged workloads (verify_b8, decode_b32 and the
head_dim-128 decode).

    python3 -m benchmarks.read_floor [bytes ...]

Runs the microbenchmark that build_lib.py compiles from read_floor.hip
(``_build/read_floor``) and prints its markdown table: per size, each grid,
the best one, and for the 16 MiB size a HIP-graph replay.
"""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(os.path.dirname(HERE), "_build", "read_floor")


def main() -> int:
    if not os.path.exists(BIN):
        sys.stderr.write(f"{BIN} missing: run custom-inference-engine_amd/build_lib.py first\n")
        return 1
    return subprocess.run([BIN, *sys.argv[1:]]).returncode


if __name__ == "__main__":
    sys.exit(main())
