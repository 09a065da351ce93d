"""fp32 torch restatement of the reference's INT8 weight path.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference functions restated here:

* ``kernels/ref/int8_matmul_ref.py:6-23`` -> :func:`dequantize_int8_ref`:
  per-channel ``w.float() * s[:, None]`` (:15-16) or per-group, each group
  of ``group_size`` inputs of a row with its own scale (:17-23).
* ``kernels/ref/int8_matmul_ref.py:26-47`` -> :func:`int8_matmul_ref`:
  ``x.float() @ dequantize(w).T`` (+ ``bias.float()``), cast to x's dtype
  (:43-47).
* ``kernels/int8_matmul.py:65-110`` -> :func:`int8_matmul_kernel_order_ref`:
  the order the production kernel uses -- the fp32 sum of the exact
  products first, times the channel scale (:56-57), rounded to x's dtype,
  then ``+ bias`` in x's dtype (:107-109). Both orders agree to fp32
  rounding; the second is what the GPU kernel restates.
* ``engine/quant/calibrate.py:6-24`` -> :func:`calibrate_weight_ref`.
"""

from __future__ import annotations

import torch


def dequantize_int8_ref(w_int8: torch.Tensor, scales: torch.Tensor, group_size: int | None = None) -> torch.Tensor:
    if group_size is None or scales.ndim == 1:
        return w_int8.float() * scales.float()[:, None]
    rows, cols = w_int8.shape
    assert cols % group_size == 0
    groups = cols // group_size
    assert scales.shape == (rows, groups)
    return (w_int8.float().reshape(rows, groups, group_size) * scales.float()[:, :, None]).reshape(rows, cols)


def int8_matmul_ref(x: torch.Tensor, w_int8: torch.Tensor, scales: torch.Tensor, group_size: int | None = None,
                    bias: torch.Tensor | None = None) -> torch.Tensor:
    y = x.float() @ dequantize_int8_ref(w_int8, scales, group_size).t()
    if bias is not None:
        y = y + bias.float()
    return y.to(x.dtype)


def int8_matmul_kernel_order_ref(x: torch.Tensor, w_int8: torch.Tensor, scales: torch.Tensor,
                                 bias: torch.Tensor | None = None) -> torch.Tensor:
    acc = x.float() @ w_int8.float().t()
    y = (acc * scales.float()[None, :]).to(x.dtype)
    if bias is not None:
        y = y + bias.to(y.dtype)
    return y


def calibrate_weight_ref(w: torch.Tensor, per_channel: bool = True) -> tuple[torch.Tensor, torch.Tensor]:
    amax = w.abs().amax(dim=1) if per_channel else w.abs().amax().expand(w.shape[0])
    scales = amax.clamp_min(1e-8) / 127.0
    q = torch.clamp(torch.round(w / scales[:, None]), -128, 127).to(torch.int8)
    return q, scales.to(torch.float16)
