"""C ABI of libcie_attn.so on the CPU: the library loads, exports exactly what
include/cie_attn.h declares, and rejects bad arguments with the documented
status codes before touching the GPU (no compute call is made here)."""

from __future__ import annotations

import ctypes
import os
import re

import pytest
import torch

from engine import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "cie_attn.h")


def _declared() -> set[str]:
    text = open(HEADER).read()
    return set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(cie_\w+)\s*\(", text, re.M))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _declared()
    assert declared == set(_lib.EXPORTED_SYMBOLS)
    for name in declared:
        assert hasattr(lib, name), name


def test_abi_version():
    assert _lib.load().cie_abi_version() == _lib.ABI_VERSION


def _st(*s):
    return (ctypes.c_int64 * 4)(*s)


FAKE = 1 << 20  # aligned, never dereferenced: validation fails first


def _flash(**over):
    args = dict(q=FAKE, k=FAKE, v=FAKE, o=FAKE, qs=_st(8192, 1024, 64, 1), ks=_st(8192, 1024, 64, 1),
                vs=_st(8192, 1024, 64, 1), os_=_st(8192, 1024, 64, 1), B=1, Hq=8, Hk=2, Lq=16, Lk=16,
                D=64, scale=0.125, causal=1, dtype=0)
    args.update(over)
    lib = _lib.load()
    return lib.cie_flash_fwd(args["q"], args["k"], args["v"], args["o"], args["qs"], args["ks"], args["vs"],
                             args["os_"], args["B"], args["Hq"], args["Hk"], args["Lq"], args["Lk"], args["D"],
                             args["scale"], args["causal"], args["dtype"], None)


@pytest.mark.parametrize("D", [0, 8, 48, 100, 512])
def test_flash_rejects_head_dim(D):
    assert _flash(D=D) == _lib.CIE_EHEADDIM
    assert "head_dim" in _lib.last_error()
    with pytest.raises(ValueError):
        _lib.check(_lib.CIE_EHEADDIM)


@pytest.mark.parametrize("dtype", [-1, 2, 7])
def test_flash_rejects_dtype(dtype):
    assert _flash(dtype=dtype) == _lib.CIE_EDTYPE


@pytest.mark.parametrize("over", [
    dict(Hq=6, Hk=4),                 # H % Hk
    dict(Hk=0),
    dict(Lq=-1),
    dict(B=-2),
    dict(q=FAKE + 2),                 # misaligned
    dict(o=0),                        # NULL output
    dict(qs=_st(8192, 1024, 64, 2)),  # head_dim stride != 1
    dict(ks=_st(8192, 1024, 60, 1)),  # row stride not 16-byte multiple
    dict(vs=_st(8192, -1024, 64, 1)),
    dict(scale=float("inf")),
])
def test_flash_rejects_bad_arguments(over):
    assert _flash(**over) == _lib.CIE_EINVAL
    assert _lib.last_error()


def test_flash_empty_problem_is_a_no_op():
    assert _flash(Lq=0, q=0, o=0) == _lib.CIE_OK
    assert _flash(B=0) == _lib.CIE_OK


def _paged(**over):
    args = dict(q=FAKE, kc=FAKE, vc=FAKE, bt=FAKE, lens=FAKE, o=FAKE, ws=FAKE, ws_bytes=1 << 30,
                qs=_st(2048, 64, 64, 1), ks=_st(8192, 512, 64, 1), vs=_st(8192, 512, 64, 1),
                os_=_st(2048, 64, 64, 1), B=4, Hq=32, Hk=8, Lq=1, D=64, nb=100, bs=16, mb=25, mc=0,
                scale=0.125, causal=1, dtype=0)
    args.update(over)
    a = args
    return _lib.load().cie_paged_fwd(a["q"], a["kc"], a["vc"], a["bt"], a["lens"], a["o"], a["ws"], a["ws_bytes"],
                                     a["qs"], a["ks"], a["vs"], a["os_"], a["B"], a["Hq"], a["Hk"], a["Lq"], a["D"],
                                     a["nb"], a["bs"], a["mb"], a["mc"], a["scale"], a["causal"], a["dtype"], None)


@pytest.mark.parametrize("over,code", [
    (dict(D=24), _lib.CIE_EHEADDIM),
    (dict(dtype=3), _lib.CIE_EDTYPE),
    (dict(Hq=30), _lib.CIE_EINVAL),
    (dict(bs=0), _lib.CIE_EINVAL),
    (dict(bt=0), _lib.CIE_EINVAL),
    (dict(kc=FAKE + 8), _lib.CIE_EINVAL),
    (dict(ws=0), _lib.CIE_EWORKSPACE),
    (dict(ws_bytes=16), _lib.CIE_EWORKSPACE),
    (dict(mb=1 << 28, bs=16), _lib.CIE_EINVAL),
    # the kv heads of one token spanning 2^31 elements (per-lane head offsets are 32-bit)
    (dict(ks=_st(8 << 32, 8 << 29, 1 << 29, 1)), _lib.CIE_EINVAL),
    (dict(vs=_st(8 << 32, 8 << 29, 1 << 29, 1)), _lib.CIE_EINVAL),
])
def test_paged_rejects_bad_arguments(over, code):
    assert _paged(**over) == code
    assert _lib.last_error()


def _paged_append(rope=False, **over):
    args = dict(q=FAKE, kn=FAKE, vn=FAKE, kc=FAKE, vc=FAKE, bt=FAKE, lens=FAKE, o=FAKE, ws=FAKE, ws_bytes=1 << 30,
                qs=_st(2048, 64, 64, 1), kns=_st(512, 64, 1, 0), vns=_st(512, 64, 1, 0),
                ks=_st(8192, 512, 64, 1), vs=_st(8192, 512, 64, 1),
                os_=_st(2048, 64, 64, 1), B=4, Hq=32, Hk=8, Lq=1, D=64, nb=100, bs=16, mb=25, mc=0,
                scale=0.125, causal=1, dtype=0)
    args.update(over)
    a = args
    head = (a["q"], a["kn"], a["vn"], a["kc"], a["vc"], a["bt"], a["lens"], a["o"], a["ws"], a["ws_bytes"],
            a["qs"], a["kns"], a["vns"], a["ks"], a["vs"], a["os_"], a["B"], a["Hq"], a["Hk"], a["Lq"], a["D"],
            a["nb"], a["bs"], a["mb"], a["mc"], a["scale"], a["causal"], a["dtype"])
    lib = _lib.load()
    if rope:
        return lib.cie_paged_fwd_append_rope(*head, FAKE, FAKE, 4096, 2, None)
    return lib.cie_paged_fwd_append(*head, None)


@pytest.mark.parametrize("rope", [False, True])
@pytest.mark.parametrize("over,code", [
    (dict(kn=0), _lib.CIE_EINVAL),
    (dict(vn=0), _lib.CIE_EINVAL),
    (dict(kn=FAKE + 8), _lib.CIE_EINVAL),                  # not 16-byte aligned
    (dict(kns=_st(500, 64, 1, 0)), _lib.CIE_EINVAL),       # token stride not a multiple of 8
    (dict(D=24), _lib.CIE_EHEADDIM),
    (dict(ws_bytes=16), _lib.CIE_EWORKSPACE),
])
def test_paged_append_rejects_bad_arguments(rope, over, code):
    """The fused append entries validate before any launch (no GPU needed)."""
    assert _paged_append(rope=rope, **over) == code
    assert _lib.last_error()


def test_paged_workspace_size():
    lib = _lib.load()
    # counters for every (head group, sequence) plus partial slots
    small = lib.cie_paged_workspace_bytes(4, 32, 8, 1, 64, 32, 16, 2)
    assert small >= 256
    n = lib.cie_paged_workspace_bytes(32, 32, 8, 1, 64, 4096, 16, 256)
    assert n > small
    # the max_context hint never increases the requirement
    assert lib.cie_paged_workspace_bytes(32, 32, 8, 1, 64, 1024, 16, 256) <= n
    assert lib.cie_paged_workspace_bytes(0, 32, 8, 1, 64, 4096, 16, 256) == 0
    # more than 256 query rows per kv head is not supported
    assert lib.cie_paged_workspace_bytes(2, 32, 8, 65, 64, 4096, 16, 256) == 0
    assert _paged(Lq=65) == _lib.CIE_EINVAL
    # at head_dim 256, more than 128
    assert lib.cie_paged_workspace_bytes(2, 32, 8, 32, 256, 4096, 16, 256) > 0
    assert lib.cie_paged_workspace_bytes(2, 32, 8, 33, 256, 4096, 16, 256) == 0
    assert _paged(Lq=33, D=256, qs=_st(8448 * 4, 8448, 256, 1), os_=_st(8448 * 4, 8448, 256, 1)) == _lib.CIE_EINVAL


def test_error_codes_map_to_reference_exception_types():
    with pytest.raises(ValueError):
        _lib.check(_lib.CIE_EDTYPE)
    with pytest.raises(ValueError):
        _lib.check(_lib.CIE_EINVAL)
    with pytest.raises(RuntimeError):
        _lib.check(_lib.CIE_ELAUNCH)
    _lib.check(_lib.CIE_OK)


def test_python_boundary_requires_gpu_tensors():
    from engine.attention import flash_attention, paged_attention

    q = torch.randn(1, 2, 4, 16, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="requires CUDA tensors"):
        flash_attention(q, q, q)
    with pytest.raises(RuntimeError):
        paged_attention(q, q, q, torch.zeros(1, 1, dtype=torch.int32), torch.zeros(1, dtype=torch.int32))
