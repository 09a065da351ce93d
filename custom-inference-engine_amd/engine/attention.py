"""Attention entry points: the drop-in for the reference's ``engine/attention.py``.

``flash_attention`` keeps the reference signature and argument checks
(``engine/attention.py:6-32``) and runs the gfx950 prefill kernel of
``libcie_attn.so``. ``paged_attention`` is the added entry that attends
straight out of the paged KV pool (``engine/cache/kv_cache.py:55``) through
int32 block tables, replacing ``cache.gather`` + dense attention
(``engine/model/block.py:56-71``).

Both accept fp16 and bf16 (the reference accepts fp16 only,
``engine/attention.py:24-25``); scores, softmax and accumulation run in fp32.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import torch

from engine import _lib

_DTYPES = (torch.float16, torch.bfloat16)


def _check_head_dim(D: int) -> None:
    if D & (D - 1):
        raise ValueError(f"head_dim must be power of 2, got {D}")
    if D < 16:
        raise ValueError(f"head_dim must be >= 16, got {D}")
    if D > 256:
        raise ValueError(f"head_dim must be <= 256, got {D}")


def _check_dtype(t: torch.Tensor) -> None:
    if t.dtype not in _DTYPES:
        raise ValueError(f"attention kernels expect FP16 or BF16 Q/K/V, got {t.dtype}")


def _kernel_layout(t: torch.Tensor) -> torch.Tensor:
    """Return ``t`` unchanged when the kernels can read it in place (unit
    head_dim stride, 16-byte aligned rows); otherwise a contiguous copy."""
    ok = t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all(
        t.shape[i] == 1 or t.stride(i) % 8 == 0 for i in range(t.dim() - 1))
    if ok:
        return t
    return t.clone(memory_format=torch.contiguous_format)


def _output(out: torch.Tensor | None, shape: tuple[int, ...], q: torch.Tensor) -> torch.Tensor:
    """A new contiguous output, or the caller's after checking that the
    kernels can write it in place."""
    if out is None:
        return torch.empty(shape, dtype=q.dtype, device=q.device)
    if tuple(out.shape) != shape or out.dtype != q.dtype or out.device != q.device:
        raise ValueError(f"out must be {shape} {q.dtype} on {q.device}, got {tuple(out.shape)} {out.dtype}")
    if _kernel_layout(out) is not out:
        raise ValueError("out needs a unit last stride, 16-byte aligned rows and outer strides in multiples of 8")
    return out


def rope_args(rope: tuple[torch.Tensor, torch.Tensor], D: int, device: torch.device) -> tuple[int, int, int, int]:
    """Validate RoPE tables (cos, sin: (rows, D/2), contiguous, on ``device``,
    fp32 as ``RotaryEmbedding`` builds them or fp16 / bf16 as the reference
    engine's ``cast_non_quantized_params`` leaves them) and return their
    pointers, row count and table dtype code for the library."""
    cos, sin = rope
    for name, t in (("cos", cos), ("sin", sin)):
        if not t.is_cuda or t.device != device:
            raise RuntimeError(f"rope {name} table must be on {device}")
        if t.dtype not in _lib.TABLE_DTYPE_CODES or t.dim() != 2 or t.shape[1] != D // 2 or not t.is_contiguous():
            raise ValueError(f"rope {name} table must be contiguous fp32, fp16 or bf16 (rows, {D // 2}), got "
                             f"{t.dtype} {tuple(t.shape)}")
    if cos.shape != sin.shape or cos.shape[0] < 1 or cos.dtype != sin.dtype:
        raise ValueError(f"rope tables differ or are empty: {tuple(cos.shape)} {cos.dtype}, "
                         f"{tuple(sin.shape)} {sin.dtype}")
    for t in (cos, sin):
        if t.data_ptr() % 16:
            raise ValueError("rope tables must start 16-byte aligned")
    return cos.data_ptr(), sin.data_ptr(), int(cos.shape[0]), _lib.TABLE_DTYPE_CODES[cos.dtype]


def flash_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    causal: bool = False,
    scale: float | None = None,
    *,
    rope: tuple[torch.Tensor, torch.Tensor] | None = None,
    q_pos0: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Flash attention on the GPU.

    Shapes: q (B, H, M, D); k/v (B, Hk, N, D) with H % Hk == 0 (GQA: query
    head h reads kv head h // (H // Hk)). ``causal`` masks bottom-right
    aligned: row i sees keys j <= N - M + i. ``scale`` defaults to
    1/sqrt(D). Returns a new contiguous (B, H, M, D) tensor in q's dtype.

    ``rope`` (keyword only, not in the reference's signature): (cos, sin)
    tables; q is then un-rotated and row i of batch b is rotated at position
    ``q_pos0[b] + i`` (int32 (B,) on the device; default 0) inside the
    kernel, bit-identical to ``rope_apply`` on q first. k must already be
    rotated. ``out``: an existing (B, H, M, D) tensor (any strides with a
    unit last stride, e.g. the transposed view of a (B, M, H, D) buffer) to
    write instead of a new one.
    """
    if not q.is_cuda:
        raise RuntimeError("flash_attention requires CUDA tensors")
    if not (k.is_cuda and v.is_cuda) or k.device != q.device or v.device != q.device:
        raise RuntimeError("flash_attention requires q, k, v on the same CUDA device")
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("flash_attention expects 4-d q (B,H,M,D) and k/v (B,Hk,N,D)")
    D = q.shape[-1]
    _check_head_dim(D)
    _check_dtype(q)
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError(f"q, k, v must share a dtype, got {q.dtype}, {k.dtype}, {v.dtype}")
    B, H, M, _ = q.shape
    Bk, Hk, N, Dk = k.shape
    if tuple(v.shape) != tuple(k.shape) or Bk != B or Dk != D:
        raise ValueError(f"shape mismatch: q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)}")
    if Hk < 1 or H % Hk:
        raise ValueError(f"num_heads {H} must be a multiple of num_kv_heads {Hk}")
    if scale is None:
        scale = 1.0 / math.sqrt(D)

    lib = _lib.load()
    q, k, v = _kernel_layout(q), _kernel_layout(k), _kernel_layout(v)
    out = _output(out, (B, H, M, D), q)
    with torch.cuda.device(q.device):
        if rope is None:
            rc = lib.cie_flash_fwd(
                q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                _lib.strides(q), _lib.strides(k), _lib.strides(v), _lib.strides(out),
                B, H, Hk, M, N, D, float(scale), 1 if causal else 0,
                _lib.DTYPE_CODES[q.dtype], _lib.stream_handle(q.device))
        else:
            cos_p, sin_p, rows, tdt = rope_args(rope, D, q.device)
            pos_p = None
            if q_pos0 is not None:
                if not q_pos0.is_cuda or q_pos0.device != q.device or q_pos0.dtype != torch.int32 \
                        or q_pos0.shape != (B,) or not q_pos0.is_contiguous():
                    raise ValueError("q_pos0 must be a contiguous int32 (B,) tensor on q's device")
                pos_p = q_pos0.data_ptr()
            rc = lib.cie_flash_fwd_rope(
                q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                _lib.strides(q), _lib.strides(k), _lib.strides(v), _lib.strides(out),
                B, H, Hk, M, N, D, float(scale), 1 if causal else 0,
                _lib.DTYPE_CODES[q.dtype], cos_p, sin_p, rows, tdt, pos_p, _lib.stream_handle(q.device))
    _lib.check(rc)
    return out


_PREFILL_KERNELS = {0: "flash_fwd", 1: "r64_heads", 2: "r64_rows", 3: "il"}


def prefill_kernel(B: int, Hq: int, Hk: int, Lq: int, Lk: int, D: int, causal: bool = True,
                   dtype: torch.dtype = torch.float16, cu_count: int = 0) -> str:
    """Name of the prefill kernel :func:`flash_attention` runs for this shape
    (``cie_prefill_kernel``): ``"flash_fwd"`` (32 query rows per wave),
    ``"r64_heads"`` / ``"r64_rows"`` (head_dim 64, two 32-row groups per
    wave: the same rows of two query heads, or 64 rows of one head) or
    ``"il"`` (head_dim 128, interleaved MFMA / softmax stream). ``cu_count``:
    compute units to size for, 0 for the current device."""
    rc = _lib.load().cie_prefill_kernel(B, Hq, Hk, Lq, Lk, D, 1 if causal else 0, _lib.DTYPE_CODES[dtype],
                                        int(cu_count))
    if rc < 0:
        _lib.check(rc)
    return _PREFILL_KERNELS[rc]


def device_cus() -> int:
    """Compute units of the current device, as the library sizes its
    launches for it (``cie_device_cus``)."""
    return int(_lib.load().cie_device_cus())


def _plan_fingerprint(context_lens: torch.Tensor, block_tables: torch.Tensor) -> int:
    """A cheap hash of host lengths and block-table rows (the bytes a plan is
    built from)."""
    import zlib

    return zlib.crc32(block_tables.numpy().tobytes(), zlib.crc32(context_lens.numpy().tobytes()))


@dataclass(frozen=True)
class PagedPlan:
    """A host-built work plan of paged attention (``cie_paged_plan``): the
    share of every workgroup, the block ids it reads and the piece
    descriptors of the merge pass, for one launch shape and one set of
    context lengths and block tables. ``data`` is the int32 plan (on the
    device for a launch), ``split`` the number of sequences split across
    workgroups, ``key`` the launch shape it was built for, ``fingerprint``
    a hash of the host lengths and block tables it was built from (see
    :meth:`built_from`)."""
    data: torch.Tensor
    split: int
    key: tuple
    fingerprint: int = 0

    def built_from(self, context_lens: torch.Tensor, block_tables: torch.Tensor) -> bool:
        """Whether the plan was built from these host lengths and tables (a
        launch with a plan reads neither: a plan of an earlier step with the
        same shape would attend over that step's lengths and blocks)."""
        lens = context_lens.to(torch.int32).contiguous()
        bt = block_tables.to(torch.int32).contiguous()
        return self.fingerprint == _plan_fingerprint(lens, bt)


def paged_max_rows(head_dim: int) -> int:
    """Query rows per kv head ((num_heads / num_kv_heads) x new tokens) that
    one paged launch takes: 256, or 128 at head_dim 256 (a workgroup holds
    up to 8 waves of 32 rows, 4 at head_dim 256, whose waves need the whole
    register file of a SIMD)."""
    return 128 if head_dim == 256 else 256


def paged_plan_ints(B: int, Hq: int, Hk: int, Lq: int, D: int, block_size: int, max_blocks_per_seq: int,
                    max_context: int | None = None) -> int:
    """int32 elements of a plan for this launch shape (0 if unsupported)."""
    return int(_lib.load().cie_paged_plan_bytes(B, Hq, Hk, Lq, D, int(max_context or 0), block_size,
                                                max_blocks_per_seq)) // 4


def paged_plan_fill(out: torch.Tensor, context_lens: torch.Tensor, block_tables: torch.Tensor, *, Hq: int,
                    Hk: int, Lq: int, D: int, num_blocks: int, block_size: int, max_context: int | None = None,
                    for_append: bool = False) -> tuple[int, tuple]:
    """Fill ``out`` (a contiguous host int32 tensor of at least
    :func:`paged_plan_ints` elements) with the plan of a launch over host
    ``context_lens`` (B,) and ``block_tables`` (B, max_blocks), int32.
    Returns (split sequences, key)."""
    B, max_blocks = block_tables.shape
    lens = context_lens.to(torch.int32).contiguous()
    bt = block_tables.to(torch.int32).contiguous()
    if lens.is_cuda or bt.is_cuda or out.is_cuda:
        raise ValueError("paged plans are built from host tensors")
    if lens.shape != (B,) or out.dtype != torch.int32 or not out.is_contiguous():
        raise ValueError("paged_plan_fill: context_lens must be (B,) and out a contiguous int32 tensor")
    mc = int(max_context or 0)
    rc = _lib.load().cie_paged_plan(out.data_ptr(), out.numel() * 4, lens.data_ptr(), bt.data_ptr(),
                                    bt.stride(0), B, Hq, Hk, Lq, D, num_blocks, block_size, max_blocks, mc,
                                    1 if for_append else 0)
    if rc < 0:
        _lib.check(rc)
    return rc, (B, Hq, Hk, Lq, D, num_blocks, block_size, max_blocks, mc, bool(for_append))


def paged_plan(context_lens: torch.Tensor, block_tables: torch.Tensor, *, Hq: int, Hk: int, Lq: int, D: int,
               num_blocks: int, block_size: int, max_context: int | None = None, for_append: bool = False,
               device: torch.device | str = "cuda") -> PagedPlan:
    """Build a plan on the host and copy it to ``device``. ``for_append``:
    the plan is for a launch with ``new_kv`` (whose contexts must count
    their Lq new tokens)."""
    B, max_blocks = block_tables.shape
    n = paged_plan_ints(B, Hq, Hk, Lq, D, block_size, max_blocks, max_context)
    if n == 0:
        raise ValueError("paged_plan: unsupported shape")
    host = torch.empty(n, dtype=torch.int32)
    lens = context_lens.cpu().to(torch.int32).contiguous()
    bt = block_tables.cpu().to(torch.int32).contiguous()
    split, key = paged_plan_fill(host, lens, bt, Hq=Hq, Hk=Hk, Lq=Lq, D=D, num_blocks=num_blocks,
                                 block_size=block_size, max_context=max_context, for_append=for_append)
    return PagedPlan(host.to(device), split, key, _plan_fingerprint(lens, bt))


def paged_workspace_bytes(B: int, Hq: int, Hk: int, Lq: int, D: int, block_size: int,
                          max_blocks_per_seq: int, max_context: int | None = None) -> int:
    """Device workspace (bytes) a :func:`paged_attention` call of this shape
    needs: per-sequence piece descriptors and the partial states of
    sequences split across workgroups."""
    return int(_lib.load().cie_paged_workspace_bytes(
        B, Hq, Hk, Lq, D, int(max_context or 0), block_size, max_blocks_per_seq))


# Workspaces, one per (device, stream): calls on one stream run in order, so
# they can share it. A workspace outgrown by a larger call is retired, never
# freed: a HIP graph captured earlier may still hold its address, and its
# replays must not write into memory the caching allocator has handed to
# another tensor.
_WORKSPACES: dict[tuple[int, int], torch.Tensor] = {}
_RETIRED_WORKSPACES: list[torch.Tensor] = []


def _cached_workspace(device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        if ws is not None:
            _RETIRED_WORKSPACES.append(ws)
        ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


def paged_attention(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    causal: bool = True,
    scale: float | None = None,
    max_context: int | None = None,
    workspace: torch.Tensor | None = None,
    *,
    rope: tuple[torch.Tensor, torch.Tensor] | None = None,
    out: torch.Tensor | None = None,
    new_kv: tuple[torch.Tensor, torch.Tensor] | None = None,
    plan: PagedPlan | None = None,
) -> torch.Tensor:
    """Attention of the newest ``Lq`` tokens of each sequence over its paged
    KV history.

    q: (B, Hq, Lq, D). k_cache / v_cache: one layer's pool,
    (num_blocks, block_size, Hk, D). block_tables: int32 (B, max_blocks),
    row b = the physical block ids of sequence b in logical order.
    context_lens: int32 (B,), tokens in the pool per sequence including the
    Lq new ones (the reference appends before attending). With ``causal``
    new token i sees positions <= context_len - Lq + i. ``max_context`` (an
    upper bound of context_lens; a longer context yields NaN) lets the launch
    size its work split tighter than max_blocks * block_size. ``workspace``:
    a caller-owned uint8 device buffer of at least
    :func:`paged_workspace_bytes` bytes; by default a cached per-(device,
    stream) buffer is used. Equal to ``flash_attention`` over ``cache.gather``
    per sequence. Returns (B, Hq, Lq, D) in q's dtype.

    ``rope``: (cos, sin) tables; q is then un-rotated and row i of sequence
    b is rotated at position ``context_lens[b] - Lq + i`` as it is loaded,
    bit-identical to ``rope_apply`` on q first. ``out``: an existing
    (B, Hq, Lq, D) tensor to write, as in :func:`flash_attention`.

    ``new_kv``: (k_new, v_new), each (B * Lq, Hk, D) with row b * Lq + i =
    new token i of sequence b, not yet in the pool. The append happens in the
    same launch pair (``cie_paged_fwd_append``): attention reads those rows
    directly and writes them into the pool at positions
    ``context_lens[b] - Lq + i``, so the pool and the result equal
    ``kv_append`` followed by ``paged_attention`` bit for bit. Every context
    must count its Lq new tokens (a shorter one gives NaN rows). With
    ``rope`` k_new is un-rotated too and is rotated at those positions, as
    ``kv_append(rope=)`` would (``cie_paged_fwd_append_rope``).

    ``plan``: a :class:`PagedPlan` built on the host for exactly these
    lengths, block tables and shape (:func:`paged_plan`, or
    ``PagedKVCache.prepare_step``); the launch then reads every workgroup's
    share of the work from it instead of deriving it on the device
    (``cie_paged_fwd_ex``), with the same result bit for bit. With a plan,
    ``block_tables`` and ``context_lens`` are checked for shape only and not
    read: the plan carries the lengths and validated block ids it was built
    from, so a plan of another step with the same shape attends over that
    step's sequences (:meth:`PagedPlan.built_from` checks host copies). The
    shape is checked here (its key) and by the launch (the plan's header).
    """
    for name, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache),
                    ("block_tables", block_tables), ("context_lens", context_lens)):
        if not t.is_cuda or t.device != q.device:
            raise RuntimeError(f"paged_attention requires CUDA tensors on one device ({name})")
    if q.dim() != 4 or k_cache.dim() != 4 or v_cache.dim() != 4:
        raise ValueError("paged_attention expects q (B,Hq,Lq,D) and pools (num_blocks,block_size,Hk,D)")
    D = q.shape[-1]
    _check_head_dim(D)
    _check_dtype(q)
    if k_cache.dtype != q.dtype or v_cache.dtype != q.dtype:
        raise ValueError(f"q and the KV pool must share a dtype, got {q.dtype}, {k_cache.dtype}, {v_cache.dtype}")
    if tuple(k_cache.shape) != tuple(v_cache.shape) or k_cache.shape[-1] != D:
        raise ValueError(f"pool shape mismatch: k {tuple(k_cache.shape)}, v {tuple(v_cache.shape)}, head_dim {D}")
    B, Hq, Lq, _ = q.shape
    num_blocks, block_size, Hk, _ = k_cache.shape
    if Hk < 1 or Hq % Hk:
        raise ValueError(f"num_heads {Hq} must be a multiple of num_kv_heads {Hk}")
    if block_tables.dim() != 2 or block_tables.shape[0] != B:
        raise ValueError(f"block_tables must be (B, max_blocks), got {tuple(block_tables.shape)}")
    if context_lens.dim() != 1 or context_lens.shape[0] != B:
        raise ValueError(f"context_lens must be (B,), got {tuple(context_lens.shape)}")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    if new_kv is not None:
        k_new, v_new = new_kv
        for name, t in (("k_new", k_new), ("v_new", v_new)):
            if not t.is_cuda or t.device != q.device:
                raise RuntimeError(f"paged_attention requires CUDA tensors on one device ({name})")
            if tuple(t.shape) != (B * Lq, Hk, D) or t.dtype != q.dtype:
                raise ValueError(f"{name} must be ({B * Lq}, {Hk}, {D}) in {q.dtype}, got {tuple(t.shape)} {t.dtype}")
        k_new, v_new = _kernel_layout(k_new), _kernel_layout(v_new)

    lib = _lib.load()
    bt = block_tables.to(torch.int32).contiguous()
    lens = context_lens.to(torch.int32).contiguous()
    max_blocks = bt.shape[1]
    q = _kernel_layout(q)
    if new_kv is not None and (_kernel_layout(k_cache) is not k_cache or _kernel_layout(v_cache) is not v_cache):
        # the fused append writes the pools in place: a copy would drop the new tokens
        raise ValueError("paged_attention(new_kv=...) needs pools with a unit last stride, 16-byte aligned rows "
                         "and outer strides in multiples of 8 elements")
    k_cache, v_cache = _kernel_layout(k_cache), _kernel_layout(v_cache)
    mc = int(max_context or 0)
    ws_bytes = int(lib.cie_paged_workspace_bytes(B, Hq, Hk, Lq, D, mc, block_size, max_blocks))
    stream = _lib.stream_handle(q.device)
    if workspace is None:
        workspace = _cached_workspace(q.device, stream, ws_bytes)
    elif not workspace.is_cuda or workspace.device != q.device:
        raise RuntimeError("paged_attention: workspace must be on the query's CUDA device")
    ws_have = workspace.numel() * workspace.element_size()
    out = _output(out, (B, Hq, Lq, D), q)
    args = (q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), bt.data_ptr(), lens.data_ptr(),
            out.data_ptr(), workspace.data_ptr(), ws_have,
            _lib.strides(q), _lib.strides(k_cache), _lib.strides(v_cache), _lib.strides(out),
            B, Hq, Hk, Lq, D, num_blocks, block_size, max_blocks, mc,
            float(scale), 1 if causal else 0, _lib.DTYPE_CODES[q.dtype])
    if plan is not None:
        key = (B, Hq, Hk, Lq, D, num_blocks, block_size, max_blocks, mc, new_kv is not None)
        if plan.key != key or not plan.data.is_cuda or plan.data.device != q.device:
            raise ValueError(f"paged_attention: the plan was built for {plan.key}, this call is {key}")
        none3 = (ctypes.c_int64 * 3)(0, 0, 1)
        kn = (k_new.data_ptr(), v_new.data_ptr()) if new_kv is not None else (None, None)
        kst = (_lib.strides3(k_new), _lib.strides3(v_new)) if new_kv is not None else (none3, none3)
        rp = rope_args(rope, D, q.device) if rope is not None else (None, None, 0, 0)
        with torch.cuda.device(q.device):
            rc = lib.cie_paged_fwd_ex(q.data_ptr(), *kn, k_cache.data_ptr(), v_cache.data_ptr(), None, None,
                                      plan.data.data_ptr(), plan.data.numel() * plan.data.element_size(),
                                      plan.split, out.data_ptr(),
                                      workspace.data_ptr() if plan.split else None, ws_have if plan.split else 0,
                                      _lib.strides(q), *kst, _lib.strides(k_cache), _lib.strides(v_cache),
                                      _lib.strides(out), *args[12:], *rp, stream)
        _lib.check(rc)
        return out
    with torch.cuda.device(q.device):
        if new_kv is not None:
            fargs = (q.data_ptr(), k_new.data_ptr(), v_new.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                     bt.data_ptr(), lens.data_ptr(), out.data_ptr(), workspace.data_ptr(), ws_have,
                     _lib.strides(q), _lib.strides3(k_new), _lib.strides3(v_new), _lib.strides(k_cache),
                     _lib.strides(v_cache), _lib.strides(out), *args[12:])
            if rope is None:
                rc = lib.cie_paged_fwd_append(*fargs, stream)
            else:
                rc = lib.cie_paged_fwd_append_rope(*fargs, *rope_args(rope, D, q.device), stream)
        elif rope is None:
            rc = lib.cie_paged_fwd(*args, stream)
        else:
            rc = lib.cie_paged_fwd_rope(*args, *rope_args(rope, D, q.device), stream)
    _lib.check(rc)
    return out
