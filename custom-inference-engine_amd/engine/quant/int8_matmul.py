"""INT8-weight matmul on the GPU: the drop-in for the reference's
``kernels.int8_matmul.int8_matmul`` (``kernels/int8_matmul.py:65-110``).

Same signature, checks and result: ``y = x @ (w_int8 * scales[:, None]).T``
with fp32 accumulation, in x's dtype, plus ``bias`` added in x's dtype
afterwards (``:107-109``). Runs ``cie_int8_matmul`` (the gfx950 kernel of
``libcie_attn.so``); there is no fallback.
"""

from __future__ import annotations

import torch

from engine import _lib

_SCALE_CODES = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}
# One split-K workspace per (device, stream); an outgrown one is retired, not
# freed, since a HIP graph captured earlier may still write to it.
_WORKSPACES: dict[tuple[int, int], torch.Tensor] = {}
_RETIRED_WORKSPACES: list[torch.Tensor] = []


def int8_matmul_workspace_bytes(M: int, N: int, K: int) -> int:
    """Device workspace (bytes) an ``int8_matmul`` of this shape needs (the
    split-K partial sums; 0 when K is not split)."""
    return int(_lib.load().cie_int8_matmul_workspace_bytes(M, N, K))


def _aligned_rows(t: torch.Tensor, elems: int) -> torch.Tensor:
    """``t`` (rows, K) with 16-byte aligned rows (row stride a multiple of
    ``elems`` elements, unit column stride): ``t`` itself when it already is,
    else a copy into a buffer whose rows are padded to that multiple."""
    if t.stride(1) == 1 and t.stride(0) % elems == 0 and t.data_ptr() % 16 == 0 and t.stride(0) >= t.shape[1]:
        return t
    rows, K = t.shape
    buf = torch.empty((rows, -(-K // elems) * elems), dtype=t.dtype, device=t.device)
    buf[:, :K] = t
    return buf[:, :K]


def _workspace(device: torch.device, stream: int, nbytes: int) -> torch.Tensor | None:
    if nbytes == 0:
        return None
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        if ws is not None:
            _RETIRED_WORKSPACES.append(ws)
        ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


def int8_matmul(x: torch.Tensor, w_int8: torch.Tensor, scales: torch.Tensor,
                bias: torch.Tensor | None = None) -> torch.Tensor:
    """Per-channel INT8 x FP16/BF16 matmul: x (..., K), w_int8 (N, K) int8,
    scales (N,), optional bias (N,). Returns (..., N) in x's dtype."""
    if not x.is_cuda:
        raise RuntimeError("int8_matmul requires CUDA tensors")
    if scales.ndim != 1:
        raise ValueError("int8_matmul expects per-channel scales with shape (N,)")
    if not (w_int8.is_cuda and scales.is_cuda) or w_int8.device != x.device or scales.device != x.device:
        raise RuntimeError("int8_matmul requires x, w_int8 and scales on the same CUDA device")
    if w_int8.dtype != torch.int8 or w_int8.dim() != 2:
        raise ValueError(f"w_int8 must be a 2-d int8 tensor, got {w_int8.dtype} {tuple(w_int8.shape)}")
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"int8_matmul expects FP16 or BF16 activations, got {x.dtype}")
    N, K = w_int8.shape
    if x.shape[-1] != K:
        raise ValueError(f"in_features mismatch: x has {x.shape[-1]}, w_int8 has {K}")
    if scales.shape[0] != N:
        raise ValueError(f"scales must have shape ({N},), got {tuple(scales.shape)}")
    if K < 1:
        raise ValueError(f"in_features must be positive, got {K}")
    # the kernels read rows in 16-byte pieces: rows that do not start 16-byte
    # aligned (e.g. K = 100 int8 weights) are copied into padded rows first;
    # any K is accepted, its tail past the kernels' step is masked as the
    # reference masks it (kernels/int8_matmul.py:43-50)
    x2 = _aligned_rows(x.reshape(-1, K), 8)
    w = _aligned_rows(w_int8, 16)
    s = scales if scales.dtype in _SCALE_CODES else scales.float()
    s = s.contiguous()
    b = None
    if bias is not None:
        if bias.shape != (N,) or not bias.is_cuda or bias.device != x.device:
            raise ValueError(f"bias must be a ({N},) tensor on x's device")
        b = bias.to(x.dtype).contiguous()
    M = x2.shape[0]
    y = torch.empty((M, N), dtype=x.dtype, device=x.device)
    lib = _lib.load()
    stream = _lib.stream_handle(x.device)
    ws_bytes = int(lib.cie_int8_matmul_workspace_bytes(M, N, K)) if M > 0 and N > 0 else 0
    ws = _workspace(x.device, stream, ws_bytes)
    with torch.cuda.device(x.device):
        rc = lib.cie_int8_matmul(x2.data_ptr(), w.data_ptr(), s.data_ptr(), b.data_ptr() if b is not None else None,
                                 y.data_ptr(), x2.stride(0), w.stride(0), y.stride(0), M, N, K,
                                 _lib.DTYPE_CODES[x.dtype], _SCALE_CODES[s.dtype],
                                 ws.data_ptr() if ws is not None else None,
                                 ws.numel() if ws is not None else 0, stream)
    _lib.check(rc)
    return y.reshape(*x.shape[:-1], N)
