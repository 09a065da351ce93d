"""Pins the oracle's restatement of the reference's INT8 weight path
(oracle/int8_ref.py) and checks, on the CPU, the package's quantizer, the
Int8Linear mirror and the argument validation of cie_int8_matmul.

Pinning: the reference's own known answers
(tests/kernels/test_int8_matmul_ref.py:9-45, tests/quant/test_int8_linear.py),
a float64 brute force of sum_k x[m,k] * w[n,k] * s[n], exact integer cases,
the agreement of the reference order (dequantize, then matmul) with the
production kernel's order (matmul, then scale; bias after rounding), and
planted mistakes that these checks must catch."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import calibrate_weight_ref, dequantize_int8_ref, int8_matmul_kernel_order_ref, int8_matmul_ref


def _quantized(out_f, in_f, seed=0):
    torch.manual_seed(seed)
    w_fp = torch.randn(out_f, in_f)
    scales = (w_fp.abs().amax(dim=1) / 127.0).clamp_min(1e-8)
    w_int8 = (w_fp / scales.unsqueeze(-1)).round().clamp(-128, 127).to(torch.int8)
    return w_fp, w_int8, scales


# ---- the reference's known answers -----------------------------------------


def test_per_channel_roundtrip_within_one_step():
    w_fp, w_int8, scales = _quantized(16, 32)
    assert (dequantize_int8_ref(w_int8, scales) - w_fp).abs().max() < scales.max() * 1.1


def test_matmul_matches_dequantized_fp():
    _, w_int8, scales = _quantized(8, 16)
    x = torch.randn(4, 16)
    y = int8_matmul_ref(x, w_int8, scales)
    assert torch.allclose(y, x @ dequantize_int8_ref(w_int8, scales).t(), atol=1e-5)


def test_grouped_quantization():
    torch.manual_seed(0)
    out_f, in_f, gs = 4, 32, 8
    w_fp = torch.randn(out_f, in_f)
    groups = w_fp.view(out_f, in_f // gs, gs)
    scales = (groups.abs().amax(dim=-1) / 127.0).clamp_min(1e-8)
    w_int8 = (groups / scales.unsqueeze(-1)).round().clamp(-128, 127).to(torch.int8).view(out_f, in_f)
    assert (dequantize_int8_ref(w_int8, scales, group_size=gs) - w_fp).abs().max() < scales.max() * 1.1


# ---- independent checks ------------------------------------------------------


def _brute_f64(x, w_int8, scales, bias=None):
    xm, wm, sv = x.double().numpy(), w_int8.numpy().astype(np.float64), scales.double().numpy()
    M, K = xm.shape
    N = wm.shape[0]
    y = np.zeros((M, N))
    for m in range(M):
        for n in range(N):
            y[m, n] = sum(xm[m, k] * wm[n, k] for k in range(K)) * sv[n]
    if bias is not None:
        y = y + bias.double().numpy()[None, :]
    return y


def int8_failures(ref, kernel_order) -> list[str]:
    bad = []
    g = torch.Generator().manual_seed(3)
    # 1. brute force (fp32 result of the oracle, fp64 truth)
    x = torch.randn(5, 64, generator=g)
    _, w, s = _quantized(7, 64, seed=1)
    if np.abs(ref(x, w, s).double().numpy() - _brute_f64(x, w, s)).max() > 1e-4:
        bad.append("brute force")
    # 2. exact integers: small integer x, power-of-two scales -> exact sums
    xi = torch.randint(-4, 5, (9, 128), generator=g).float().half()
    wi = torch.randint(-128, 128, (12, 128), generator=g).to(torch.int8)
    si = (2.0 ** -torch.randint(4, 9, (12,), generator=g).float()).half()
    exact = torch.tensor(_brute_f64(xi, wi, si)).half()
    if not (torch.equal(ref(xi, wi, si), exact) and torch.equal(kernel_order(xi, wi, si), exact)):
        bad.append("exact integers")
    # 3. both orders agree to the output rounding
    xh = torch.randn(6, 256, generator=g).half()
    _, w2, s2 = _quantized(20, 256, seed=2)
    a, b = ref(xh, w2, s2.half()).float(), kernel_order(xh, w2, s2.half()).float()
    if ((a - b).abs() > 2e-3 * (a.abs() + 1)).any():
        bad.append("orders agree")
    # 4. bias after the rounded product, in the output dtype (kernel order):
    # acc = 1024 + fp16(0.4) = 1024.3999 rounds to 1024 (fp16 spacing 1 there),
    # then + fp16(0.3) = 1024.3 -> 1024; adding the bias first would give 1025
    xb = torch.zeros(1, 64).half()
    xb[0, 0], xb[0, 1] = 1024.0, 0.4
    wb = torch.zeros(1, 64, dtype=torch.int8)
    wb[0, 0] = wb[0, 1] = 1
    sb, bb = torch.tensor([1.0]).half(), torch.tensor([0.3]).half()
    if kernel_order(xb, wb, sb, bb).item() != 1024.0:
        bad.append("bias order")
    return bad


def test_oracle_passes_every_check():
    assert int8_failures(int8_matmul_ref, int8_matmul_kernel_order_ref) == []


MUTANTS = {
    "scale ignored": (lambda x, w, s, b=None: int8_matmul_ref(x, w, torch.ones_like(s), bias=b),
                      lambda x, w, s, b=None: int8_matmul_kernel_order_ref(x, w, torch.ones_like(s), b)),
    "one scale for every channel": (
        lambda x, w, s, b=None: int8_matmul_ref(x, w, s.float().mean().expand(s.shape), bias=b),
        lambda x, w, s, b=None: int8_matmul_kernel_order_ref(x, w, s.float().mean().expand(s.shape), b)),
    "bias before rounding": (int8_matmul_ref,
                             lambda x, w, s, b=None: int8_matmul_ref(x, w, s, bias=b)),
    "unsigned weights": (lambda x, w, s, b=None: int8_matmul_ref(x, w.view(torch.uint8).to(torch.int16), s, bias=b),
                         lambda x, w, s, b=None: int8_matmul_kernel_order_ref(x, w.view(torch.uint8).to(torch.int16),
                                                                              s, b)),
    "fp16 accumulation": (lambda x, w, s, b=None: (x.half() @ (w.half() * s.half()[:, None]).t()).to(x.dtype),
                          lambda x, w, s, b=None: (x.half() @ (w.half() * s.half()[:, None]).t()).to(x.dtype)),
}


@pytest.mark.parametrize("name", sorted(MUTANTS))
def test_planted_mistakes_are_caught(name):
    assert int8_failures(*MUTANTS[name]), f"mutant '{name}' passed every check"


def test_calibrate_ref_properties():
    torch.manual_seed(4)
    w = torch.randn(32, 96) * torch.linspace(0.01, 10, 32)[:, None]
    q, s = calibrate_weight_ref(w)
    assert q.dtype == torch.int8 and s.dtype == torch.float16
    assert (q.abs().amax(dim=1) == 127).all()  # the largest weight of a row maps to +-127
    assert ((q.float() * s.float()[:, None] - w).abs() <= s.float()[:, None] * 0.51 + 1e-3 * w.abs()).all()


# ---- the package's host side ------------------------------------------------


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_package_calibration_equals_reference_scheme(dtype):
    from engine.quant import calibrate_weight

    torch.manual_seed(5)
    w = (torch.randn(64, 128) * 0.05).to(dtype)
    q, s = calibrate_weight(w)
    rq, rs = calibrate_weight_ref(w)
    assert torch.equal(q, rq) and torch.equal(s, rs)
    q2, s2 = calibrate_weight(w, per_channel=False)
    rq2, rs2 = calibrate_weight_ref(w, per_channel=False)
    assert torch.equal(q2, rq2) and torch.equal(s2, rs2)


def test_int8_linear_shapes_and_cpu_refusal():
    # tests/quant/test_int8_linear.py:24-29
    from engine.quant import Int8Linear

    qlin = Int8Linear(16, 8, bias=False)
    assert qlin.weight_int8.shape == (8, 16) and qlin.scales.shape == (8,) and qlin.bias is None
    with pytest.raises(RuntimeError):
        qlin(torch.randn(2, 16).half())


# ---- C ABI validation (no compute call) ------------------------------------

FAKE = 1 << 20


def _call(**over):
    from engine import _lib

    a = dict(x=FAKE, w=FAKE, s=FAKE, b=None, y=FAKE, xs=4096, wsr=4096, ys=4096, M=128, N=4096, K=4096,
             dtype=0, sdt=0, ws=FAKE, wsb=1 << 30)
    a.update(over)
    return _lib.load().cie_int8_matmul(a["x"], a["w"], a["s"], a["b"], a["y"], a["xs"], a["wsr"], a["ys"], a["M"],
                                       a["N"], a["K"], a["dtype"], a["sdt"], a["ws"], a["wsb"], None)


@pytest.mark.parametrize("over,code", [
    (dict(dtype=2), -3), (dict(sdt=3), -3), (dict(K=0), -1), (dict(M=-1), -1), (dict(K=100, xs=100), -1),
    (dict(x=0), -1), (dict(w=FAKE + 4), -1), (dict(s=0), -1), (dict(s=FAKE + 1), -1), (dict(b=FAKE + 1), -1),
    (dict(xs=4100), -1), (dict(wsr=4104), -1), (dict(ys=100), -1), (dict(y=FAKE + 4), -1), (dict(ws=0), -4), (dict(wsb=16), -4),
])
def test_int8_matmul_rejects_bad_arguments(over, code):
    from engine import _lib

    assert _call(**over) == code
    assert _lib.last_error()


def test_int8_matmul_empty_and_workspace_query():
    from engine import _lib

    lib = _lib.load()
    assert _call(M=0, x=0, y=0) == 0
    assert lib.cie_int8_matmul_workspace_bytes(64, 4096, 4096) == 0       # decode shapes stream the weights
    assert lib.cie_int8_matmul_workspace_bytes(128, 4096, 4096) > 0       # few tiles: split K
    assert lib.cie_int8_matmul_workspace_bytes(4096, 4096, 4096) == 0     # enough tiles: no split
    assert lib.cie_int8_matmul_workspace_bytes(64, 4096, 100) == 0        # any K; streaming needs none
    assert lib.cie_int8_matmul_workspace_bytes(128, 4096, 4100) > 0       # any K; split like K = 4096
