"""CPU oracle for the attention hot path.

TEST INFRASTRUCTURE ONLY. Nothing in the shipped package imports this module:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker (or, for the baseline, as the
thing timed on the host CPU). The product path goes through the HIP library
and fails loudly when it is missing.

Contents
--------
``attention_ref``  fp32 torch restatement of the reference's
                   ``kernels/ref/flash_attention_ref.py:8-56`` plus the paged
                   composition (``engine/cache/kv_cache.py:141-165`` gather,
                   ``engine/cache/block_table.py:23-26`` block math) and the
                   append loop (``engine/cache/kv_cache.py:128-136``).
``rope_ref``       fp32 torch restatement of the reference's rotary tables
                   and rotation (``kernels/ref/rope_apply_ref.py:6-53``).
``int8_ref``       fp32 torch restatement of the reference's INT8 weight
                   path (``kernels/ref/int8_matmul_ref.py``,
                   ``kernels/int8_matmul.py``, ``engine/quant/calibrate.py``).
``brute``          fp64 numpy brute force written independently of the
                   above (explicit per-row max-subtracted exponentials).

Pinning: every function here is checked in ``tests/test_oracle.py`` against
the reference's own known answers (``tests/kernels/test_flash_attention_ref.py``,
``tests/cache/test_block_table.py``, ``tests/kernels/test_rope_ref.py``,
``tests/model/test_rope.py``, ``tests/kernels/test_int8_matmul_ref.py``),
against the fp64 brute force, against
``torch.nn.functional.scaled_dot_product_attention`` with an explicit
bottom-right mask, against closed-form special cases, and against planted
mistakes that those checks must catch. No function is "parity unpinned".
"""

from oracle.attention_ref import (  # noqa: F401
    append_ref,
    attention_rows_ref,
    flash_attention_ref,
    flash_attention_ref_chunked,
    gather_ref,
    logical_to_physical_ref,
    paged_attention_ref,
)
from oracle.brute import attention_brute_f64, paged_attention_brute_f64  # noqa: F401
from oracle.rope_ref import build_rope_cache_ref, rope_ref  # noqa: F401
from oracle.int8_ref import (  # noqa: F401
    calibrate_weight_ref,
    dequantize_int8_ref,
    int8_matmul_kernel_order_ref,
    int8_matmul_ref,
)
