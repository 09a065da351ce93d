"""Offline weight quantization (host side, not the hot path): the same
symmetric per-channel scheme as the reference's
``engine/quant/calibrate.py:6-24``, so that a model quantized here and there
holds the same int8 weights and fp16 scales."""

from __future__ import annotations

import torch


def calibrate_weight(w: torch.Tensor, symmetric: bool = True,
                     per_channel: bool = True) -> tuple[torch.Tensor, torch.Tensor]:
    """(w_int8 (out, in), scales fp16 (out,)): scale = max |w| / 127 per row
    (or over the whole matrix), w_int8 = clamp(round(w / scale), -128, 127)."""
    if w.ndim != 2:
        raise ValueError("weight must be 2-D (out, in)")
    if not symmetric:
        raise NotImplementedError("only symmetric quantization implemented")
    amax = w.abs().amax(dim=1) if per_channel else w.abs().amax().expand(w.shape[0])
    scales = amax.clamp_min(1e-8) / 127.0
    w_int8 = (w / scales.unsqueeze(-1)).round().clamp(-128, 127).to(torch.int8)
    return w_int8, scales.to(torch.float16)
