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
  (:53). The element type of that arithmetic is torch's result type of x
  and the tables:
    - fp32 tables (as ``build_rope_cache`` makes them), or fp16 x with bf16
      tables and the reverse (torch promotes that pair to fp32): every
      product and the difference / sum are fp32 operations, each rounded,
      and only the final cast rounds to x's type;
    - tables of x's own 16-bit type, which is what the reference engine
      runs with: ``cast_non_quantized_params`` (engine/runtime.py:22-37,
      called at :124, engine/model/loader.py:128 and the reference's
      tests/conftest.py:62) casts every floating buffer, RotaryEmbedding's
      cos / sin included, to the activation dtype. Each product and the
      difference / sum is then a half (or bfloat16) operation: computed in
      fp32 and rounded to the 16-bit type, as written here.
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


def rope_arith_dtype(x_dtype: torch.dtype, table_dtype: torch.dtype) -> torch.dtype:
    """Element type of the rotation's products and sums: the table's type
    when it equals x's 16-bit type, fp32 otherwise (fp32 tables, or a mixed
    fp16 / bf16 pair, which torch promotes to fp32)."""
    if table_dtype == x_dtype and x_dtype in (torch.float16, torch.bfloat16):
        return x_dtype
    return torch.float32


def rope_ref(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
             positions: torch.Tensor | None = None) -> torch.Tensor:
    """Rotate x (B, H, L, D) at ``positions`` ((L,), (B, L) or None for
    0..L-1). Returns x's dtype."""
    B, H, L, D = x.shape
    half = D // 2
    pos = torch.arange(L) if positions is None else positions.long().cpu()
    adt = rope_arith_dtype(x.dtype, cos.dtype)
    c = cos.cpu()[pos].float()
    s = sin.cpu()[pos].float()
    # (L, half) -> broadcast over batch and heads; (B, L, half) -> over heads
    c = c.reshape(1, 1, L, half) if pos.dim() == 1 else c.reshape(B, 1, L, half)
    s = s.reshape(1, 1, L, half) if pos.dim() == 1 else s.reshape(B, 1, L, half)
    x1 = x[..., :half].float()
    x2 = x[..., half:].float()

    def r(t):  # one operation's result in the arithmetic type (fp32 products of 16-bit values are exact)
        return t.to(adt).float()

    first = r(r(x1 * c) - r(x2 * s))
    second = r(r(x1 * s) + r(x2 * c))
    return torch.cat((first, second), dim=-1).to(x.dtype)
