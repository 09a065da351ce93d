"""fp32 torch restatement of the reference attention oracle and paged gather.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference functions restated here:

* ``kernels/ref/flash_attention_ref.py:8-56`` -> :func:`flash_attention_ref`
  (fp32 up-cast :27-30, GQA by ``repeat_interleave`` :32-37, default scale
  ``1/sqrt(D)`` :39-40, bottom-right causal mask ``j > Lk-Lq+i`` :44-49,
  additive mask after the causal fill :51-52, softmax + PV :54-55, cast back
  to the input dtype :56).
* ``engine/cache/block_table.py:23-26`` -> :func:`logical_to_physical_ref`.
* ``engine/cache/kv_cache.py:141-165`` -> :func:`gather_ref` (dense
  ``(L, Hk, D)`` history of one sequence; ``L == 0`` gives empty tensors).
* ``engine/model/block.py:56-71`` -> :func:`paged_attention_ref`: the
  reference appends the new tokens first and then attends causally over the
  whole gathered history, so ``context_lens`` includes the ``Lq`` new tokens.
"""

from __future__ import annotations

import math

import torch


def flash_attention_ref(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    mask: torch.Tensor | None = None,
    causal: bool = False,
    scale: float | None = None,
) -> torch.Tensor:
    """Naive scaled-dot-product attention computed in fp32.

    q: (B, H, Lq, D); k, v: (B, Hk, Lk, D) with H % Hk == 0. Query head ``h``
    reads kv head ``h // (H // Hk)``. Returns (B, H, Lq, D) in q's dtype.
    Rows with no visible key (causal with Lq > Lk) come out NaN, as the
    reference's softmax over an all ``-inf`` row does; Lk == 0 gives zeros.
    """
    out_dtype = q.dtype
    qf, kf, vf = q.float(), k.float(), v.float()
    B, H, Lq, D = qf.shape
    Hk, Lk = kf.shape[1], kf.shape[2]
    if H != Hk:
        if H % Hk:
            raise ValueError(f"num_heads {H} must be a multiple of num_kv_heads {Hk}")
        group = H // Hk
        kf = kf.repeat_interleave(group, dim=1)
        vf = vf.repeat_interleave(group, dim=1)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    scores = torch.matmul(qf, kf.transpose(-2, -1)) * scale
    if causal:
        rows = torch.arange(Lq).unsqueeze(-1)
        cols = torch.arange(Lk).unsqueeze(0)
        hidden = cols > (Lk - Lq + rows)
        scores = scores.masked_fill(hidden.to(scores.device), float("-inf"))
    if mask is not None:
        scores = scores + mask
    probs = torch.softmax(scores, dim=-1)
    return torch.matmul(probs, vf).to(out_dtype)


def flash_attention_ref_chunked(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    causal: bool = False,
    scale: float | None = None,
    q_chunk: int = 2048,
) -> torch.Tensor:
    """:func:`flash_attention_ref` evaluated one (batch, kv group, query block)
    at a time so that long sequences fit in host memory.

    Each query row's softmax only involves its own score row, so splitting the
    query axis (keeping the absolute row index for the bottom-right mask) and
    the head axis gives the same numbers as the unchunked form. Output is
    fp32 regardless of the input dtype.
    """
    B, H, Lq, D = q.shape
    Hk, Lk = k.shape[1], k.shape[2]
    group = H // Hk
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    out = torch.empty(B, H, Lq, D, dtype=torch.float32)
    cols = torch.arange(Lk)
    for b in range(B):
        for kh in range(Hk):
            kf = k[b, kh].float()
            vf = v[b, kh].float()
            qs = q[b, kh * group:(kh + 1) * group].float()  # (group, Lq, D)
            for r0 in range(0, Lq, q_chunk):
                r1 = min(Lq, r0 + q_chunk)
                # keys beyond the last visible column of this block never
                # contribute; trimming them is exact
                kend = Lk if not causal else max(0, min(Lk, Lk - Lq + r1))
                s = torch.matmul(qs[:, r0:r1], kf[:kend].transpose(0, 1)) * scale
                if causal:
                    rows = torch.arange(r0, r1).unsqueeze(-1)
                    s = s.masked_fill(cols[:kend].unsqueeze(0) > (Lk - Lq + rows), float("-inf"))
                if kend == 0 and Lk > 0:
                    out[b, kh * group:(kh + 1) * group, r0:r1] = float("nan")
                    continue
                p = torch.softmax(s, dim=-1)
                out[b, kh * group:(kh + 1) * group, r0:r1] = torch.matmul(p, vf[:kend])
    return out


def attention_rows_ref(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    rows,
    causal: bool = False,
    scale: float | None = None,
) -> torch.Tensor:
    """fp32 outputs of the listed absolute query rows only, all heads:
    returns (B, H, len(rows), D). Row ``i`` keeps its place in the
    bottom-right mask (sees keys ``j <= Lk - Lq + i``), so this equals
    ``flash_attention_ref(...)[:, :, rows]`` at a fraction of the cost when
    the full problem is too large for the host."""
    B, H, Lq, D = q.shape
    Hk, Lk = k.shape[1], k.shape[2]
    group = H // Hk
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    rows = [int(r) for r in rows]
    out = torch.empty(B, H, len(rows), D, dtype=torch.float32)
    for n, i in enumerate(rows):
        kend = Lk if not causal else max(0, min(Lk, Lk - Lq + i + 1))
        if Lk == 0:
            out[:, :, n] = 0.0
            continue
        if kend == 0:
            out[:, :, n] = float("nan")
            continue
        kf = k[:, :, :kend].float().repeat_interleave(group, dim=1)
        vf = v[:, :, :kend].float().repeat_interleave(group, dim=1)
        s = torch.matmul(q[:, :, i:i + 1].float(), kf.transpose(-2, -1)) * scale
        out[:, :, n] = torch.matmul(torch.softmax(s, dim=-1), vf)[:, :, 0]
    return out


def logical_to_physical_ref(blocks, block_size: int, pos: int) -> tuple[int, int]:
    """Block math of the reference's ``BlockTable.logical_to_physical``:
    position ``pos`` lives in physical block ``blocks[pos // bs]`` at offset
    ``pos % bs``."""
    return int(blocks[pos // block_size]), pos % block_size


def gather_ref(pool: torch.Tensor, blocks, length: int) -> torch.Tensor:
    """Dense ``(length, Hk, D)`` history of one sequence from a pool of shape
    ``(num_blocks, block_size, Hk, D)``, position by position through the
    block table."""
    nb, bs, Hk, D = pool.shape
    if length == 0:
        return pool.new_zeros((0, Hk, D))
    blocks = torch.as_tensor(blocks, dtype=torch.long).cpu()
    pos = torch.arange(length)
    phys = blocks[pos // bs]
    off = pos % bs
    return pool.cpu()[phys, off]


def paged_attention_ref(
    q: torch.Tensor,
    k_pool: torch.Tensor,
    v_pool: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    causal: bool = True,
    scale: float | None = None,
) -> torch.Tensor:
    """Attention of ``q`` (B, Hq, Lq, D) against each sequence's paged
    history, computed as gather-then-dense exactly as the reference's
    ``Attention.forward`` does. Returns fp32 (B, Hq, Lq, D)."""
    B, Hq, Lq, D = q.shape
    out = torch.empty(B, Hq, Lq, D, dtype=torch.float32)
    bt = block_tables.cpu()
    lens = context_lens.cpu()
    for b in range(B):
        L = int(lens[b])
        kd = gather_ref(k_pool, bt[b], L).float().transpose(0, 1).unsqueeze(0)
        vd = gather_ref(v_pool, bt[b], L).float().transpose(0, 1).unsqueeze(0)
        out[b] = flash_attention_ref_chunked(q[b:b + 1].cpu(), kd, vd, causal=causal, scale=scale)[0]
    return out


def append_ref(k_pool: torch.Tensor, v_pool: torch.Tensor, blocks, start: int, k: torch.Tensor,
               v: torch.Tensor) -> None:
    """In-place write of ``k``, ``v`` (L, Hk, D) at positions start..start+L-1
    of the sequence whose physical blocks are ``blocks``; the slice loop of
    ``engine/cache/kv_cache.py:128-136`` (one slice assignment per block
    spanned, ``take = min(bs - off, L - src_off)``). Block allocation
    (``:122-125``) is the caller's: ``blocks`` must already cover the range."""
    bs = k_pool.shape[1]
    L = k.shape[0]
    src = 0
    pos = start
    while src < L:
        bid, off = logical_to_physical_ref(blocks, bs, pos)
        take = min(bs - off, L - src)
        k_pool[bid, off:off + take] = k[src:src + take]
        v_pool[bid, off:off + take] = v[src:src + take]
        pos += take
        src += take
