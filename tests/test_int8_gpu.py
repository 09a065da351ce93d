"""GPU parity of the INT8-weight GEMM (engine.quant.int8_matmul ->
cie_int8_matmul) against the oracle's restatement of the reference
(oracle/int8_ref.py <- kernels/int8_matmul.py, kernels/ref/int8_matmul_ref.py).

* the reference's own test case (tests/kernels/test_triton_kernels.py:25-41:
  M=64, N=128, K=64, fp16, seed 0) at its tolerance, 1e-3;
* bit-exactness at full sizes where the arithmetic is exact: integer
  activations in [-4, 4] and power-of-two scales make every fp32 sum exact,
  so any summation order gives the same result and the output must equal
  the oracle's bit for bit -- at the reference's benchmark shapes
  (64 / 512 x 4096 x 4096, benchmarks/bench_int8_matmul.py:14) and ragged
  ones, split-K and not, with and without bias;
* random activations against the oracle within the output rounding
  (|y - ref| <= atol + rtol |ref|: fp16 1e-3 + 2e-3 |ref|, bf16 1e-2 + 1.6e-2 |ref|);
* Int8Linear against the float layer it quantizes
  (tests/quant/test_int8_linear.py:9-21: relative error < 5 %)."""

from __future__ import annotations

import pytest
import torch

from engine.quant import Int8Linear, int8_matmul, int8_matmul_workspace_bytes, quantize_linear
from oracle import int8_matmul_kernel_order_ref, int8_matmul_ref

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.float16: (1e-3, 2e-3), torch.bfloat16: (1e-2, 1.6e-2)}


def test_reference_test_case():
    torch.manual_seed(0)
    M, N, K = 64, 128, 64
    w_fp = torch.randn(N, K)
    scales = (w_fp.abs().amax(dim=1) / 127.0).clamp_min(1e-8)
    w_int8 = (w_fp / scales.unsqueeze(-1)).round().clamp(-128, 127).to(torch.int8)
    x = torch.randn(M, K, dtype=torch.float16, device=DEV)
    y = int8_matmul(x, w_int8.to(DEV), scales.to(DEV).to(torch.float16))
    ref = int8_matmul_ref(x.cpu(), w_int8, scales.to(torch.float16))
    assert (y.cpu() - ref).abs().max() < 1e-3


def _exact_case(M, N, K, dtype, seed, bias):
    g = torch.Generator().manual_seed(seed)
    x = torch.randint(-4, 5, (M, K), generator=g).to(dtype)
    w = torch.randint(-128, 128, (N, K), generator=g).to(torch.int8)
    s = (2.0 ** -torch.randint(6, 10, (N,), generator=g).float()).to(torch.float16)
    b = (torch.randn(N, generator=g) * 4).to(dtype) if bias else None
    return x, w, s, b


@pytest.mark.parametrize("M,N,K", [(64, 4096, 4096), (512, 4096, 4096), (1, 4096, 4096), (33, 300, 640),
                                   (100, 127, 64), (2048, 4096, 256), (515, 1000, 1024), (16, 11008, 4096),
                                   (32, 4096, 11008), (5, 96, 64), (31, 1000, 2112),
                                   # small M: ragged N, K tails within a step
                                   (2, 300, 640), (3, 1001, 2112), (4, 130, 1088), (1, 7, 64), (1, 11008, 4096),
                                   # M = 1, 2 with the whole activation rows in LDS (K = 32768, 16384), and
                                   # past it (the kernels that read the activations from L2)
                                   (1, 64, 32768), (1, 80, 32800), (2, 64, 16384), (2, 48, 16448),
                                   # the streaming kernel at 8 / 16 / 32 / 64 staged rows, K tails within a pass
                                   (8, 4096, 4096), (12, 520, 1216), (40, 333, 1088), (64, 1000, 4160), (65, 512, 1024),
                                   # any K (the reference masks the K tail, kernels/int8_matmul.py:43-50):
                                   # K below one step of each kernel, K tails of 4 / 32 / 36 past a step,
                                   # rows not 16-byte aligned (K = 100, 4100, 17: padded copies)
                                   (1, 32, 32), (1, 17, 8), (1, 4096, 100), (1, 300, 4100), (2, 64, 32),
                                   (3, 300, 96), (12, 520, 100), (40, 333, 4100), (64, 128, 32), (64, 96, 17),
                                   (65, 512, 4100), (512, 1024, 4100), (100, 127, 96), (300, 96, 32), (2048, 256, 100),
                                   (130, 4096, 4132),
                                   # the eight-wave tiled kernel (one workgroup per CU): two K
                                   # splits with a K tail, one split over 64 steps
                                   (256, 4096, 1060), (512, 2048, 4096)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_exact_arithmetic_is_bit_exact(M, N, K, dtype):
    for bias in (False, True):
        x, w, s, b = _exact_case(M, N, K, dtype, seed=M + N + K, bias=bias)
        y = int8_matmul(x.to(DEV), w.to(DEV), s.to(DEV), bias=None if b is None else b.to(DEV))
        want = int8_matmul_kernel_order_ref(x, w, s, b)
        assert torch.equal(y.cpu(), want), (M, N, K, bias, (y.cpu().float() - want.float()).abs().max().item())


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,N,K", [(1, 512, 4096), (3, 256, 1600), (7, 256, 512), (64, 1024, 2048), (300, 384, 4096),
                                   (1, 512, 100), (33, 256, 4100), (300, 384, 96), (5, 64, 32)])
def test_random_activations_within_rounding(M, N, K, dtype):
    g = torch.Generator().manual_seed(M * 7 + K)
    x = torch.randn(M, K, generator=g).to(dtype)
    w_fp = torch.randn(N, K, generator=g) * 0.02
    s = (w_fp.abs().amax(dim=1) / 127.0).clamp_min(1e-8)
    w = (w_fp / s[:, None]).round().clamp(-128, 127).to(torch.int8)
    s = s.to(torch.float16)
    y = int8_matmul(x.to(DEV), w.to(DEV), s.to(DEV)).cpu().float()
    ref = int8_matmul_ref(x, w, s).float()
    atol, rtol = TOL[dtype]
    assert ((y - ref).abs() <= atol + rtol * ref.abs()).all(), (y - ref).abs().max().item()


def test_layouts_scale_dtypes_and_shapes():
    g = torch.Generator().manual_seed(9)
    B, L, K, N = 2, 5, 256, 192
    x = torch.randint(-3, 4, (B, L, K), generator=g).half()
    w = torch.randint(-128, 128, (N, K), generator=g).to(torch.int8)
    s = 2.0 ** -torch.randint(5, 8, (N,), generator=g).float()
    want = int8_matmul_kernel_order_ref(x.reshape(-1, K), w, s.half()).reshape(B, L, N)
    for sd in (torch.float16, torch.bfloat16, torch.float32):  # powers of two: exact in each
        y = int8_matmul(x.to(DEV), w.to(DEV), s.to(sd).to(DEV))
        assert y.shape == (B, L, N) and torch.equal(y.cpu(), want)
    # strided activations (a column slice of a wider buffer) and a strided weight view
    wide = torch.zeros(B * L, K + 64).half()
    wide[:, 32:32 + K] = x.reshape(-1, K)
    wbig = torch.zeros(N, K + 128, dtype=torch.int8)
    wbig[:, :K] = w
    y = int8_matmul(wide.to(DEV)[:, 32:32 + K], wbig.to(DEV)[:, :K], s.half().to(DEV))
    assert torch.equal(y.cpu(), want.reshape(-1, N))
    assert int8_matmul_workspace_bytes(1, N, 4096) == 0   # weight streaming: one launch, no workspace
    assert int8_matmul_workspace_bytes(64, N, 4096) == 0  # weight streaming up to M = 64
    assert int8_matmul_workspace_bytes(128, N, 4096) > 0  # split K


@pytest.mark.parametrize("M", [1, 2])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_decode_rows_layouts_bias_and_scale_dtypes(M, dtype):
    """The row-streaming kernel of one or two activation rows: strided
    activation rows (a column slice of a wider buffer, rows further apart
    than K), a strided weight view, a bias, every scale dtype, a K tail past
    the last 128-k step and N not a multiple of its 8 rows per workgroup --
    bit for bit against the reference order in exact arithmetic."""
    g = torch.Generator().manual_seed(20 + M)
    K, N = 4160, 203
    x = torch.randint(-3, 4, (M, K), generator=g).to(dtype)
    w = torch.randint(-128, 128, (N, K), generator=g).to(torch.int8)
    s = 2.0 ** -torch.randint(5, 8, (N,), generator=g).float()
    bias = (torch.randint(-64, 64, (N,), generator=g).float() / 4).to(dtype)
    want = int8_matmul_kernel_order_ref(x, w, s.to(dtype), bias)
    wide = torch.zeros(M, K + 96, dtype=dtype)
    wide[:, 48:48 + K] = x
    wbig = torch.zeros(N, K + 64, dtype=torch.int8)
    wbig[:, :K] = w
    for sd in (torch.float16, torch.bfloat16, torch.float32):  # powers of two: exact in each
        y = int8_matmul(wide.to(DEV)[:, 48:48 + K], wbig.to(DEV)[:, :K], s.to(sd).to(DEV), bias.to(DEV))
        assert y.shape == (M, N) and torch.equal(y.cpu(), want), (M, dtype, sd)


def test_int8_linear_close_to_float_layer():
    # tests/quant/test_int8_linear.py:9-21
    torch.manual_seed(0)
    lin = torch.nn.Linear(64, 32, bias=True).to(device=DEV, dtype=torch.float16)
    qlin = quantize_linear(lin).to(DEV)
    assert isinstance(qlin, Int8Linear)
    x = torch.randn(4, 64, device=DEV, dtype=torch.float16)
    y_fp = lin(x)
    y_q = qlin(x)
    assert y_q.shape == y_fp.shape
    assert (y_q - y_fp).abs().max().item() / y_fp.abs().max().item() < 0.05
    # and it is the oracle's result for the quantized weights
    ref = int8_matmul_kernel_order_ref(x.cpu(), qlin.weight_int8.cpu(), qlin.scales.cpu(), qlin.bias.detach().cpu())
    atol, rtol = TOL[torch.float16]
    assert ((y_q.cpu().float() - ref.float()).abs() <= atol + rtol * ref.float().abs()).all()


@pytest.mark.parametrize("M", [1, 8])
def test_reference_tiny_model_layers(M):
    """Every Int8Linear of the reference's tiny test model
    (tests/conftest.py:30-43: hidden 32, 2 heads of 16, intermediate 64,
    vocab 32): q/k/v/o 32 -> 32, gate/up 32 -> 64, down 64 -> 32, lm head
    32 -> 32; a decode token (M = 1) and an 8-token prefill, against the
    oracle at the reference's tolerance."""
    torch.manual_seed(M)
    for fin, fout in ((32, 32), (32, 64), (64, 32)):
        lin = torch.nn.Linear(fin, fout, bias=False).to(device=DEV, dtype=torch.float16)
        qlin = quantize_linear(lin).to(DEV)
        x = torch.randn(1, M, fin, device=DEV, dtype=torch.float16)
        y = qlin(x)
        assert y.shape == (1, M, fout)
        ref = int8_matmul_ref(x.cpu().reshape(M, fin), qlin.weight_int8.cpu(), qlin.scales.cpu())
        assert (y.cpu().reshape(M, fout).float() - ref.float()).abs().max().item() < 1e-3


def test_repeated_calls_are_deterministic():
    x, w, s, _ = _exact_case(64, 2048, 4096, torch.float16, seed=1, bias=False)
    xr = torch.randn(64, 4096).half().to(DEV)
    wd, sd = w.to(DEV), s.to(DEV)
    a = int8_matmul(xr, wd, sd)
    for _ in range(3):
        assert torch.equal(int8_matmul(xr, wd, sd), a)
