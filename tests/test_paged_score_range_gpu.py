"""GPU parity of the paged decode / verify kernels on peaked attention:
scores of standard deviation 4-6 (fp16) and about 2.3 (bf16, head_dim 128)
instead of the ~1 of the seeded workloads.

The paged kernel applies the softmax scale (times log2 e) to the fp32 score
accumulator, as the reference's dense kernel does after its fp32 dot
(kernels/flash_attention.py:98), and the contexts here are long enough that
every sequence is cut across workgroup ranges, so the merge of fp32 partial
states (acc, m, l) in piece order runs on every output row: large scores
stress both the exponent arithmetic and the rescaling of the partial states
to a common maximum.

Bar: max |out - ref| <= 2e-3 (fp16) / 1e-2 (bf16) against the oracle
(gather through the block table, then the fp32 reference), on the same
rounded inputs.
"""

from __future__ import annotations

import pytest
import torch

from engine.attention import paged_attention, paged_plan
from oracle import paged_attention_ref
from test_flash_gpu import assert_close
from test_paged_gpu import make_paged

pytestmark = pytest.mark.gpu
DEV = "cuda"

LENS = [3000, 1500, 4097, 700]  # a few hundred 32-token tiles per head group: every sequence splits


def _peaked(Lq, D, dtype, sigma, seed, Hq=32, Hk=8):
    """q and the K pool ~ N(0, sigma^2), the V pool ~ N(0, 1), rounded to dtype."""
    q, kp, vp, bt, ln = make_paged(LENS, Lq, D, torch.float32, 16, Hq=Hq, Hk=Hk, seed=seed)
    return (q * sigma).to(dtype), (kp * sigma).to(dtype), vp.to(dtype), bt, ln


@pytest.mark.parametrize("planned", [False, True])
@pytest.mark.parametrize("sigma", [2.0, 2.5])
@pytest.mark.parametrize("Lq", [1, 5])
def test_fp16_d64_peaked_scores(Lq, sigma, planned):
    q, kp, vp, bt, ln = _peaked(Lq, 64, torch.float16, sigma, seed=int(10 * sigma) + Lq)
    ref = paged_attention_ref(q, kp, vp, bt, ln, causal=True)
    kw = {}
    if planned:  # the host-built schedule (same ranges and pieces as the device's)
        kw["max_context"] = int(ln.max())
        kw["plan"] = paged_plan(ln, bt, Hq=32, Hk=8, Lq=Lq, D=64, num_blocks=kp.shape[0], block_size=16,
                                max_context=kw["max_context"], device=DEV)
    out = paged_attention(q.to(DEV), kp.to(DEV), vp.to(DEV), bt.to(DEV), ln.to(DEV), causal=True, **kw)
    assert_close(out, ref, 2e-3, f"fp16 D=64 Lq={Lq} sigma={sigma} planned={planned}")


@pytest.mark.parametrize("Lq", [1, 5])
def test_bf16_d128_peaked_scores(Lq):
    q, kp, vp, bt, ln = _peaked(Lq, 128, torch.bfloat16, 1.5, seed=40 + Lq)
    ref = paged_attention_ref(q, kp, vp, bt, ln, causal=True)
    out = paged_attention(q.to(DEV), kp.to(DEV), vp.to(DEV), bt.to(DEV), ln.to(DEV), causal=True)
    assert_close(out, ref, 1e-2, f"bf16 D=128 Lq={Lq} sigma=1.5")
