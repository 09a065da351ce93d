"""The committed fixtures of tests/golden/ (written by tests/golden/make_golden.py
from the fp64 brute force): the oracle reproduces them on the CPU, and the HIP
kernels reproduce them on the GPU within the parity bar (max-abs 2e-3 fp16,
1e-2 bf16, against the fp64 outputs on the same rounded inputs).
"""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch

from oracle import flash_attention_ref, logical_to_physical_ref, paged_attention_ref

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = {"f16": 2e-3, "bf16": 1e-2}


def _load_values(arr: np.ndarray, dtype: str) -> torch.Tensor:
    if dtype == "f16":
        return torch.from_numpy(arr.astype(np.float16))
    return torch.from_numpy(arr.view(np.int16).copy()).view(torch.bfloat16)


def _cases(fname: str) -> dict[str, dict[str, np.ndarray]]:
    data = np.load(os.path.join(GOLDEN, fname))
    out: dict[str, dict[str, np.ndarray]] = {}
    for key in data.files:
        name, field = key.split("__")
        out.setdefault(name, {})[field] = data[key]
    return out


PREFILL = _cases("prefill_cases.npz")
PAGED = _cases("paged_cases.npz")


def _prefill_inputs(c):
    dt = str(c["dtype"])
    return [_load_values(c[n], dt) for n in ("q", "k", "v")], bool(c["causal"]), dt


def _paged_inputs(c):
    dt = str(c["dtype"])
    q, kp, vp = (_load_values(c[n], dt) for n in ("q", "k_pool", "v_pool"))
    bt = torch.from_numpy(c["block_tables"].astype(np.int32))
    lens = torch.from_numpy(c["context_lens"].astype(np.int32))
    return q, kp, vp, bt, lens, bool(c["causal"]), dt


def _check(out: torch.Tensor, want: np.ndarray, tol: float, what: str) -> None:
    out = out.double().cpu().numpy()
    assert out.shape == want.shape, (what, out.shape, want.shape)
    assert np.array_equal(np.isnan(out), np.isnan(want)), f"{what}: NaN pattern differs"
    ok = ~np.isnan(want)
    err = float(np.abs(out[ok] - want[ok]).max()) if ok.any() else 0.0
    assert err <= tol, f"{what}: max abs error {err:.3e} > {tol:.1e}"


# ------------------------------------------------------------------ CPU: oracle

def test_block_table_known_answers():
    from engine.cache import BlockTable

    ka = json.load(open(os.path.join(GOLDEN, "block_table_known_answers.json")))
    table = BlockTable(ka["block_size"], list(ka["blocks"]), 9)
    for pos, want in ka["positions"].items():
        assert list(logical_to_physical_ref(ka["blocks"], ka["block_size"], int(pos))) == want
        assert list(table.logical_to_physical(int(pos))) == want


@pytest.mark.parametrize("name", sorted(PREFILL))
def test_oracle_reproduces_prefill_fixture(name):
    c = PREFILL[name]
    (q, k, v), causal, _ = _prefill_inputs(c)
    _check(flash_attention_ref(q.float(), k.float(), v.float(), causal=causal), c["out"], 2e-6, name)


@pytest.mark.parametrize("name", sorted(PAGED))
def test_oracle_reproduces_paged_fixture(name):
    q, kp, vp, bt, lens, causal, _ = _paged_inputs(PAGED[name])
    got = paged_attention_ref(q.float(), kp.float(), vp.float(), bt, lens, causal=causal)
    _check(got, PAGED[name]["out"], 2e-6, name)


def test_oracle_reproduces_s128_workload_rows():
    from benchmarks import workloads

    g = np.load(os.path.join(GOLDEN, "prefill_s128_rows.npz"))
    case = workloads.prefill_s128()
    q, k, v = (t.double().numpy() for t in (case.q, case.k, case.v))
    # the seeded inputs are the ones the fixture was made from
    np.testing.assert_allclose([q.sum(), np.abs(q).sum()], g["checksum_q"], rtol=1e-12)
    np.testing.assert_allclose([k.sum(), np.abs(k).sum()], g["checksum_k"], rtol=1e-12)
    np.testing.assert_allclose([v.sum(), np.abs(v).sum()], g["checksum_v"], rtol=1e-12)
    assert np.array_equal(q[0, 0, 0, :8], g["head_q"])
    out = flash_attention_ref(case.q, case.k, case.v, causal=True)
    _check(out[:, :, g["rows"]], g["out_rows"], 2e-6, "prefill_s128")


# ------------------------------------------------------------------ GPU: kernels

@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(PREFILL))
def test_kernel_reproduces_prefill_fixture(name):
    from engine.attention import flash_attention

    c = PREFILL[name]
    (q, k, v), causal, dt = _prefill_inputs(c)
    out = flash_attention(q.cuda(), k.cuda(), v.cuda(), causal=causal)
    _check(out, c["out"], TOL[dt], name)


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(PAGED))
def test_kernel_reproduces_paged_fixture(name):
    from engine.attention import paged_attention

    q, kp, vp, bt, lens, causal, dt = _paged_inputs(PAGED[name])
    out = paged_attention(q.cuda(), kp.cuda(), vp.cuda(), bt.cuda(), lens.cuda(), causal=causal)
    _check(out, PAGED[name]["out"], TOL[dt], name)


@pytest.mark.gpu
@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_kernel_s128_workload_rows(dt):
    """The fp32 workload run in fp16 / bf16: against the fixture's fp64 rows
    computed on the unrounded inputs the error also holds the input rounding
    (1.4e-3 fp16, 9.5e-3 bf16 for the oracle itself), so the kernel is held to
    the bar against the oracle on the rounded inputs and to 3x the bar against
    the fixture."""
    from benchmarks import workloads
    from engine.attention import flash_attention

    g = np.load(os.path.join(GOLDEN, "prefill_s128_rows.npz"))
    case = workloads.prefill_s128()
    tdt = torch.float16 if dt == "f16" else torch.bfloat16
    q, k, v = (t.to(tdt) for t in (case.q, case.k, case.v))
    out = flash_attention(q.cuda(), k.cuda(), v.cuda(), causal=True)
    ref = flash_attention_ref(q.float(), k.float(), v.float(), causal=True)
    _check(out, ref.double().numpy(), TOL[dt], "s128 vs oracle")
    _check(out[:, :, g["rows"]], g["out_rows"], 3 * TOL[dt], "s128 vs fixture")
