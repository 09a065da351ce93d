"""The allocation-free paged entry (cie_paged_fwd_noalloc, workspace in a
static device array of the library) against cie_paged_fwd with a caller
workspace: the same kernels on the same arguments, so the outputs must be
equal bit for bit, call after call -- here a decode-shaped call followed by
a smaller verify-shaped one, which reuses the array the first call left
behind. Also checked against the oracle, and the size limit is rejected
before any HIP call."""

from __future__ import annotations

import ctypes
import math

import pytest
import torch

from engine import _lib
from oracle import paged_attention_ref
from test_paged_gpu import make_paged

DEV = "cuda"
TOL = {torch.float16: 2e-3, torch.bfloat16: 1e-2}


def _args(q, kp, vp, bt, lens, o):
    B, Hq, Lq, D = q.shape
    nb, bs, Hk, _ = kp.shape
    keep = [_lib.strides(t) for t in (q, kp, vp, o)]
    head = (q.data_ptr(), kp.data_ptr(), vp.data_ptr(), bt.data_ptr(), lens.data_ptr(), o.data_ptr())
    tail = (B, Hq, Hk, Lq, D, nb, bs, bt.shape[1], int(lens.max()), ctypes.c_float(1.0 / math.sqrt(D)), 1,
            _lib.DTYPE_CODES[q.dtype], _lib.stream_handle(q.device))
    return head, keep, tail


def _both(lens, Lq, D, dtype, Hq, Hk, seed):
    q, kp, vp, bt, lt = make_paged(lens, Lq, D, dtype, 16, Hq=Hq, Hk=Hk, seed=seed, vscale=0.5)
    qd, kd, vd, btd, ld = (t.to(DEV) for t in (q, kp, vp, bt, lt))
    lib = _lib.load()
    o_ws = torch.full_like(qd, float("nan"))
    o_na = torch.full_like(qd, float("nan"))
    head, keep, tail = _args(qd, kd, vd, btd, ld, o_ws)
    B, _, _, _ = q.shape
    nbytes = lib.cie_paged_workspace_bytes(B, Hq, Hk, Lq, D, int(lt.max()), 16, bt.shape[1])
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=DEV)
    rc = lib.cie_paged_fwd(*head, ws.data_ptr(), nbytes, *keep, *tail)
    _lib.check(rc)
    head_na = head[:5] + (o_na.data_ptr(),)
    rc = lib.cie_paged_fwd_noalloc(*head_na, *keep, *tail)
    _lib.check(rc)
    torch.cuda.synchronize()
    ref = paged_attention_ref(q.float(), kp.float(), vp.float(), bt, lt, causal=True)
    return o_ws.cpu(), o_na.cpu(), ref, nbytes


@pytest.mark.gpu
def test_noalloc_equals_caller_workspace_on_consecutive_calls():
    g = torch.Generator().manual_seed(2)
    # 1. decode-shaped: 32 sequences, 32 q / 8 kv heads, contexts 256..4096 (many split across workgroups)
    lens = torch.randint(256, 4097, (32,), generator=g).tolist()
    o_ws, o_na, ref, n1 = _both(lens, 1, 64, torch.float16, 32, 8, seed=5)
    assert n1 > 0
    assert torch.equal(o_na, o_ws)
    assert (o_na.float() - ref).abs().max().item() <= TOL[torch.float16]
    # 2. smaller, verify-shaped: 4 sequences x 5 new tokens, bf16, other head counts; it uses less of the
    #    static array than the first call, whose partial states stay behind it
    lens = [40, 1000, 5, 333]
    o_ws, o_na, ref, n2 = _both(lens, 5, 64, torch.bfloat16, 8, 2, seed=6)
    assert 0 < n2 < n1
    assert torch.equal(o_na, o_ws)
    assert (o_na.float() - ref).abs().max().item() <= TOL[torch.bfloat16]


def test_noalloc_rejects_shapes_beyond_the_static_workspace():
    lib = _lib.load()
    st = (ctypes.c_int64 * 4)(4096, 64, 64, 1)
    pool = (ctypes.c_int64 * 4)(8192, 512, 64, 1)
    # 4096 sequences x 64 rows per kv head at D = 256: the partial states alone exceed 16 MiB
    need = lib.cie_paged_workspace_bytes(4096, 64, 8, 8, 256, 65536, 16, 4096)
    assert need > 16 << 20
    rc = lib.cie_paged_fwd_noalloc(1 << 20, 1 << 20, 1 << 20, 1 << 20, 1 << 20, 1 << 20, st, pool, pool, st,
                                   4096, 64, 8, 8, 256, 100, 16, 4096, 65536, 0.0625, 1, 0, None)
    assert rc == _lib.CIE_EWORKSPACE and "static workspace" in _lib.last_error()
