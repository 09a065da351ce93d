"""Issue rates of the prefill step's instructions on the GPU (v_exp_f32,
v_fma_f32, v_mfma_f32_32x32x16_f16 and mixes of them).

    python3 -m benchmarks.vector_rates

Runs the microbenchmark that build_lib.py compiles from vector_rates.hip
(``_build/vector_rates``) and prints its markdown table. Reading it: a mix
whose cycles per iteration equal the sum of its parts' shares one issue
resource; one that takes the larger of them overlaps.
"""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(os.path.dirname(HERE), "_build", "vector_rates")


def main() -> int:
    if not os.path.exists(BIN):
        sys.stderr.write(f"{BIN} missing: run custom-inference-engine_amd/build_lib.py first\n")
        return 1
    return subprocess.run([BIN]).returncode


if __name__ == "__main__":
    sys.exit(main())
