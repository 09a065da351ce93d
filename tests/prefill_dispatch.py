"""Which prefill kernel a head_dim-64 launch takes, for the GPU tests that
must reach the two-row-group kernel with small problems (by repeating one
problem over a batch).

The GPU tests ask the library itself (``cie_prefill_kernel``, through
``engine.attention.prefill_kernel``); ``two_row_group_kernel_runs`` restates
the launcher's rule independently, and a CPU test checks that the two agree
over a sweep of shapes and compute-unit counts."""

from __future__ import annotations

from engine.attention import prefill_kernel

TWO_ROW_GROUP_KERNELS = ("r64_heads", "r64_rows")


def two_row_group_kernel_runs(B, H, Lq, Lk, causal, cus=256):
    """Whether a head_dim-64 launch takes the two-row-group kernel: restates
    the launcher's rule (r64_pays, csrc/flash_fwd.hip) -- at least one item of
    B * H / 2 per 128-row query tile for each of the 2 * cus workgroup slots
    and, causal, the longest item (32 keys a step, plus 4) within 1.6x the
    average work per slot."""
    if Lq <= 128:
        return False
    slots = 2 * cus
    n_mt = (Lq + 127) // 128
    items = B * H // 2
    if n_mt * items < slots:
        return False
    if not causal:
        return True
    work = longest = 0
    for mt in range(n_mt):
        kend = max(0, min(Lk, Lk - Lq + min(Lq, 128 * (mt + 1))))
        st = (kend + 31) // 32 + 4
        work += st
        longest = max(longest, st)
    return longest * slots * 10 <= 16 * work * items


def batch_for_two_row_groups(H, Lq, Lk, causal):
    """The smallest batch whose head_dim-64 launch the library runs on the
    two-row-group kernel (on the current device)."""
    for B in range(1, 1025):
        if prefill_kernel(B, H, H, Lq, Lk, 64, causal) in TWO_ROW_GROUP_KERNELS:
            return B
    raise AssertionError("no batch size reaches the two-row-group kernel")


def replicate(x, B):
    """x (1, ...) repeated B times along the batch: every copy is an independent
    item of the launch and must give the same outputs."""
    return x.expand(B, *x.shape[1:]).contiguous()
