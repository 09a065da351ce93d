"""fp32 torch restatement of the reference's rotary position embedding.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference functions restated here:

* ``kernels/ref/rope_apply_ref.py:6-19`` -> :func:`build_rope_cache_ref`:
  per pair i the inverse frequency ``1 / theta ** (2i / D)`` in fp32 (:16),
  the angle table ``outer(position, inv_freq)`` (:17-18), then its cos and
  sin (:19), each of shape (max_seq_len, D/2).
* ``kernels/ref/rope_apply_ref.py:22-53`` -> :func:`rope_ref`: positions
  default to 0..L-1 (:36-37) and index the tables as (L,) or (B, L)
  (:38-47); the halves x1 = x[..., :D/2], x2 = x[..., D/2:] (:49-50) become
  x1*c - x2*s and x1*s + x2*c (:51-52), joined and cast back to x's dtype
  (:53). With fp16/bf16 x and fp32 tables every product and the
  difference / sum are fp32 operations, each rounded, as written here.
"""

from __future__ import annotations

import torch


def build_rope_cache_ref(max_seq_len: int, head_dim: int, theta: float = 10000.0) -> tuple[torch.Tensor, torch.Tensor]:
    """(cos, sin) fp32 tables of shape (max_seq_len, head_dim // 2)."""
    assert head_dim % 2 == 0
    exponents = torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim
    inv_freq = 1.0 / (theta ** exponents)
    angles = torch.outer(torch.arange(max_seq_len, dtype=torch.float32), inv_freq)
    return angles.cos(), angles.sin()


def rope_ref(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
             positions: torch.Tensor | None = None) -> torch.Tensor:
    """Rotate x (B, H, L, D) at ``positions`` ((L,), (B, L) or None for
    0..L-1). Returns x's dtype."""
    B, H, L, D = x.shape
    half = D // 2
    pos = torch.arange(L) if positions is None else positions.long().cpu()
    c = cos.cpu()[pos]
    s = sin.cpu()[pos]
    # (L, half) -> broadcast over batch and heads; (B, L, half) -> over heads
    c = c.reshape(1, 1, L, half) if pos.dim() == 1 else c.reshape(B, 1, L, half)
    s = s.reshape(1, 1, L, half) if pos.dim() == 1 else s.reshape(B, 1, L, half)
    x1 = x[..., :half].float()
    x2 = x[..., half:].float()
    first = x1 * c - x2 * s
    second = x1 * s + x2 * c
    return torch.cat((first, second), dim=-1).to(x.dtype)
