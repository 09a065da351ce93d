"""Rotary position embedding: the drop-in for the reference's
``engine/model/rope.py`` (``RotaryEmbedding``, :9-19) and the table builder it
uses (``kernels/ref/rope_apply_ref.py:6-19``).

The tables are built exactly as the reference builds them (fp32, on the host,
at construction) so that every rotation below is bit-identical to the
reference's ``apply_rotary_ref``. The rotation itself runs in
``libcie_attn.so``: :func:`rope_apply` (``cie_rope_apply``), or fused into
the KV append (K) and the attention kernels' query loads (Q) through the
``rope=`` arguments of ``kv_append``, ``flash_attention`` and
``paged_attention``.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from engine import _lib
from engine.attention import _check_dtype, _check_head_dim, _kernel_layout, rope_args


def build_rope_cache(max_seq_len: int, head_dim: int, theta: float = 10000.0,
                     device: torch.device | str = "cpu",
                     dtype: torch.dtype = torch.float32) -> tuple[torch.Tensor, torch.Tensor]:
    """(cos, sin), each (max_seq_len, head_dim / 2): angle p * theta^(-2i/D)
    for position p and pair i, computed in fp32 with the same operations as
    the reference (kernels/ref/rope_apply_ref.py:13-19), hence the same
    bits."""
    if head_dim % 2:
        raise ValueError("head_dim must be even for RoPE")
    device = torch.device(device)
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, device=device, dtype=torch.float32) / head_dim))
    t = torch.arange(max_seq_len, device=device, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    return freqs.cos().to(dtype), freqs.sin().to(dtype)


def rope_apply(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, positions: torch.Tensor | None = None,
               out: torch.Tensor | None = None, status: torch.Tensor | None = None) -> torch.Tensor:
    """RoPE of x (B, H, L, D) on the GPU, as ``apply_rotary_ref``
    (kernels/ref/rope_apply_ref.py:22-53): positions (L,), (B, L) or None
    (0..L-1); cos / sin the (rows, D/2) tables on x's device, fp32 or cast
    to fp16 / bf16 (then rotated with 16-bit arithmetic, as torch does when
    the reference engine casts the model's buffers). Returns
    ``out`` (a new tensor by default; ``out=x`` rotates in place). A position
    outside the tables gives a NaN row and ORs 2 into ``status`` (optional
    int32 (1,) on the device) where the reference's indexing raises."""
    if not x.is_cuda:
        raise RuntimeError("rope_apply requires CUDA tensors")
    if x.dim() != 4:
        raise ValueError(f"rope_apply expects x of shape (B, H, L, D), got {tuple(x.shape)}")
    B, H, L, D = x.shape
    _check_head_dim(D)
    _check_dtype(x)
    cos_p, sin_p, rows, tdt = rope_args((cos, sin), D, x.device)
    pos_p, pos_bs = None, 0
    if positions is not None:
        if positions.dim() == 1 and positions.shape[0] == L:
            pos_bs = 0
        elif positions.dim() == 2 and tuple(positions.shape) == (B, L):
            pos_bs = L
        else:
            raise ValueError(f"positions must be (L,) or (B, L) for x {tuple(x.shape)}, got {tuple(positions.shape)}")
        positions = positions.to(device=x.device, dtype=torch.int32).contiguous()
        pos_p = positions.data_ptr()
    src = _kernel_layout(x)
    if out is None:
        out = torch.empty((B, H, L, D), dtype=x.dtype, device=x.device)
    elif tuple(out.shape) != (B, H, L, D) or out.dtype != x.dtype or out.device != x.device:
        raise ValueError("rope_apply: out must match x")
    dst = _kernel_layout(out)
    lib = _lib.load()
    with torch.cuda.device(x.device):
        rc = lib.cie_rope_apply(src.data_ptr(), dst.data_ptr(), _lib.strides(src), _lib.strides(dst), pos_p, pos_bs,
                                cos_p, sin_p, rows, tdt, status.data_ptr() if status is not None else None,
                                B, H, L, D, _lib.DTYPE_CODES[x.dtype], _lib.stream_handle(x.device))
    _lib.check(rc)
    if dst is not out:
        out.copy_(dst)
    return out


class RotaryEmbedding(nn.Module):
    """RoPE with a precomputed cos/sin cache (engine/model/rope.py:9-19).
    ``apply`` runs the gfx950 kernel; ``tables`` is the (cos, sin) pair the
    fused paths take as ``rope=``."""

    def __init__(self, head_dim: int, max_seq_len: int, theta: float = 10000.0):
        super().__init__()
        cos, sin = build_rope_cache(max_seq_len, head_dim, theta=theta)
        self.register_buffer("cos", cos, persistent=False)
        self.register_buffer("sin", sin, persistent=False)

    @property
    def tables(self) -> tuple[torch.Tensor, torch.Tensor]:
        return self.cos, self.sin

    def apply(self, x: torch.Tensor, positions: torch.Tensor | None = None) -> torch.Tensor:
        return rope_apply(x, self.cos, self.sin, positions=positions)
