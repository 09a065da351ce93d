"""Which prefill kernel a head_dim-64 launch takes, for the GPU tests that
must reach the two-row-group kernel with small problems (by repeating one
problem over a batch)."""

from __future__ import annotations


def two_row_group_kernel_runs(B, H, Lq, Lk, causal):
    """Whether a head_dim-64 launch takes the two-row-group kernel: restates
    the launcher's rule (r64_pays, csrc/flash_fwd.hip) -- at least one item of
    B * H / 2 per 128-row query tile for each of the 512 workgroup slots and,
    causal, the longest item (32 keys a step, plus 4) within 1.6x the
    average work per slot."""
    if Lq <= 128:
        return False
    n_mt = (Lq + 127) // 128
    items = B * H // 2
    if n_mt * items < 512:
        return False
    if not causal:
        return True
    work = longest = 0
    for mt in range(n_mt):
        kend = max(0, min(Lk, Lk - Lq + min(Lq, 128 * (mt + 1))))
        st = (kend + 31) // 32 + 4
        work += st
        longest = max(longest, st)
    return longest * 512 * 10 <= 16 * work * items


def batch_for_two_row_groups(H, Lq, Lk, causal):
    """The smallest batch whose launch takes the two-row-group kernel."""
    for B in range(1, 1025):
        if two_row_group_kernel_runs(B, H, Lq, Lk, causal):
            return B
    raise AssertionError("no batch size reaches the two-row-group kernel")


def replicate(x, B):
    """x (1, ...) repeated B times along the batch: every copy is an independent
    item of the launch and must give the same outputs."""
    return x.expand(B, *x.shape[1:]).contiguous()
