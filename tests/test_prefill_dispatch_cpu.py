"""The prefill launcher's kernel choice (cie_prefill_kernel) on the CPU.

The GPU tests that target the head_dim-64 two-row-group kernel ask the
library which kernel a shape takes; here an independent restatement of the
launcher's rule (tests/prefill_dispatch.py) is checked against the library's
own answer over a sweep of shapes and device sizes, so a change of either
shows up as a disagreement, and the query is checked for the kernels every
head_dim takes."""

from __future__ import annotations

import itertools

import pytest
import torch

from engine import _lib
from engine.attention import device_cus, prefill_kernel
from prefill_dispatch import TWO_ROW_GROUP_KERNELS, two_row_group_kernel_runs


@pytest.mark.parametrize("cus", [256, 128, 64, 32, 304])
def test_restated_rule_agrees_with_the_library(cus):
    Bs = [1, 2, 3, 4, 8, 16, 32, 64]
    Ls = [(128, 128), (129, 129), (200, 1000), (256, 256), (512, 512), (1024, 1024), (2048, 2048),
          (4096, 4096), (300, 40), (1536, 1536)]
    heads = [(32, 8), (32, 32), (28, 4), (8, 2), (3, 3), (16, 16)]
    n_r64 = 0
    for B, (Lq, Lk), (H, Hk), causal in itertools.product(Bs, Ls, heads, (True, False)):
        got = prefill_kernel(B, H, Hk, Lq, Lk, 64, causal, torch.float16, cu_count=cus)
        want = two_row_group_kernel_runs(B, H, Lq, Lk, causal, cus=cus)
        assert (got in TWO_ROW_GROUP_KERNELS) == want, (B, H, Hk, Lq, Lk, causal, cus, got)
        if want:
            # head pairs when the group size is even, else 64-row waves of one head
            assert got == ("r64_heads" if (H // Hk) % 2 == 0 else "r64_rows")
            n_r64 += 1
    assert n_r64 > 20  # the sweep reaches both sides of the rule


def test_workload_kernels():
    # prefill_s2048 (B=4, S=2048, 32/8 heads, D=64) takes head pairs on an
    # MI355X; prefill_s16384 (D=128) the interleaved kernel; prefill_s128 the
    # 32-row kernel (too little work for two row groups)
    assert prefill_kernel(4, 32, 8, 2048, 2048, 64, True, torch.float16, cu_count=256) == "r64_heads"
    assert prefill_kernel(1, 32, 8, 16384, 16384, 128, True, torch.bfloat16, cu_count=256) == "il"
    assert prefill_kernel(1, 32, 8, 128, 128, 64, True, torch.float16, cu_count=256) == "flash_fwd"
    for D in (16, 32, 256):
        assert prefill_kernel(64, 32, 8, 4096, 4096, D, True, torch.float16, cu_count=256) == "flash_fwd"


def test_query_rejects_what_the_launch_rejects():
    lib = _lib.load()
    assert lib.cie_prefill_kernel(1, 4, 2, 10, 10, 48, 1, 0, 0) == _lib.CIE_EHEADDIM
    assert lib.cie_prefill_kernel(1, 4, 3, 10, 10, 64, 1, 0, 0) == _lib.CIE_EINVAL
    assert lib.cie_prefill_kernel(1, 4, 2, 10, 10, 64, 1, 7, 0) == _lib.CIE_EDTYPE
    assert lib.cie_prefill_kernel(-1, 4, 2, 10, 10, 64, 1, 0, 0) == _lib.CIE_EINVAL


def test_device_cus_without_a_gpu():
    # no device to query here: launches are sized for an unpartitioned MI355X
    if not torch.cuda.is_available():
        assert device_cus() == 256
    assert device_cus() > 0
