"""ctypes binding of ``libcie_attn.so`` (declared in ``include/cie_attn.h``).

The library is loaded on first use, after ``torch`` so that the HIP runtime
torch already mapped (soname ``libamdhip64.so.7``) is the one the library binds
to and torch's stream handles are valid in it. There is no fallback: if the
library is missing or refuses a launch, the call raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.environ.get("CIE_ATTN_LIB", os.path.join(PKG_ROOT, "libcie_attn.so"))
ABI_VERSION = 3

CIE_OK = 0
CIE_EINVAL = -1
CIE_EHEADDIM = -2
CIE_EDTYPE = -3
CIE_EWORKSPACE = -4
CIE_ELAUNCH = -5

DTYPE_CODES = {torch.float16: 0, torch.bfloat16: 1}
TABLE_DTYPE_CODES = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}

EXPORTED_SYMBOLS = (
    "cie_abi_version",
    "cie_last_error",
    "cie_device_cus",
    "cie_prefill_kernel",
    "cie_flash_fwd",
    "cie_paged_workspace_bytes",
    "cie_paged_fwd",
    "cie_paged_fwd_noalloc",
    "cie_paged_plan_bytes",
    "cie_paged_plan",
    "cie_paged_fwd_ex",
    "cie_kv_append",
    "cie_rope_apply",
    "cie_flash_fwd_rope",
    "cie_paged_fwd_rope",
    "cie_paged_fwd_append",
    "cie_paged_fwd_append_rope",
    "cie_kv_append_rope",
    "cie_int8_matmul_workspace_bytes",
    "cie_int8_matmul",
)


class NativeLibraryError(RuntimeError):
    """The attention library could not be loaded or rejected a call."""


_lib = None
_lock = threading.Lock()

_i64p = ctypes.POINTER(ctypes.c_int64)
_vp = ctypes.c_void_p
_i = ctypes.c_int


def _declare(lib: ctypes.CDLL) -> None:
    lib.cie_abi_version.argtypes = []
    lib.cie_abi_version.restype = _i
    lib.cie_last_error.argtypes = []
    lib.cie_last_error.restype = ctypes.c_char_p
    lib.cie_device_cus.argtypes = []
    lib.cie_device_cus.restype = _i
    lib.cie_prefill_kernel.argtypes = [_i, _i, _i, _i, _i, _i, _i, _i, _i]
    lib.cie_prefill_kernel.restype = _i
    lib.cie_flash_fwd.argtypes = [_vp, _vp, _vp, _vp, _i64p, _i64p, _i64p, _i64p,
                                  _i, _i, _i, _i, _i, _i, ctypes.c_float, _i, _i, _vp]
    lib.cie_flash_fwd.restype = _i
    lib.cie_paged_workspace_bytes.argtypes = [_i, _i, _i, _i, _i, _i, _i, _i]
    lib.cie_paged_workspace_bytes.restype = ctypes.c_size_t
    lib.cie_paged_fwd.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t,
                                  _i64p, _i64p, _i64p, _i64p,
                                  _i, _i, _i, _i, _i, _i, _i, _i, _i,
                                  ctypes.c_float, _i, _i, _vp]
    lib.cie_paged_fwd.restype = _i
    lib.cie_paged_fwd_noalloc.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _i64p, _i64p, _i64p, _i64p,
                                          _i, _i, _i, _i, _i, _i, _i, _i, _i, ctypes.c_float, _i, _i, _vp]
    lib.cie_paged_fwd_noalloc.restype = _i
    lib.cie_paged_plan_bytes.argtypes = [_i, _i, _i, _i, _i, _i, _i, _i]
    lib.cie_paged_plan_bytes.restype = ctypes.c_size_t
    lib.cie_paged_plan.argtypes = [_vp, ctypes.c_size_t, _vp, _vp, ctypes.c_int64, _i, _i, _i, _i, _i, _i, _i, _i,
                                   _i, _i]
    lib.cie_paged_plan.restype = _i
    lib.cie_paged_fwd_ex.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t, _i, _vp, _vp,
                                     ctypes.c_size_t,
                                     _i64p, _i64p, _i64p, _i64p, _i64p, _i64p,
                                     _i, _i, _i, _i, _i, _i, _i, _i, _i, ctypes.c_float, _i, _i,
                                     _vp, _vp, _i, _i, _vp]
    lib.cie_paged_fwd_ex.restype = _i
    lib.cie_kv_append.argtypes = [_vp, _vp, _vp, _vp, _i64p, _i64p, _i64p, _i64p, _vp, _vp, _vp, _vp,
                                  _i, _i, _i, _i, _i, _i, _i, _i, _i, _vp]
    lib.cie_kv_append.restype = _i
    lib.cie_rope_apply.argtypes = [_vp, _vp, _i64p, _i64p, _vp, ctypes.c_int64, _vp, _vp, _i, _i, _vp,
                                   _i, _i, _i, _i, _i, _vp]
    lib.cie_rope_apply.restype = _i
    lib.cie_flash_fwd_rope.argtypes = [_vp, _vp, _vp, _vp, _i64p, _i64p, _i64p, _i64p,
                                       _i, _i, _i, _i, _i, _i, ctypes.c_float, _i, _i, _vp, _vp, _i, _i, _vp, _vp]
    lib.cie_flash_fwd_rope.restype = _i
    lib.cie_paged_fwd_rope.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t,
                                       _i64p, _i64p, _i64p, _i64p,
                                       _i, _i, _i, _i, _i, _i, _i, _i, _i,
                                       ctypes.c_float, _i, _i, _vp, _vp, _i, _i, _vp]
    lib.cie_paged_fwd_rope.restype = _i
    lib.cie_paged_fwd_append.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t,
                                         _i64p, _i64p, _i64p, _i64p, _i64p, _i64p,
                                         _i, _i, _i, _i, _i, _i, _i, _i, _i,
                                         ctypes.c_float, _i, _i, _vp]
    lib.cie_paged_fwd_append.restype = _i
    lib.cie_paged_fwd_append_rope.argtypes = lib.cie_paged_fwd_append.argtypes[:-1] + [_vp, _vp, _i, _i, _vp]
    lib.cie_paged_fwd_append_rope.restype = _i
    lib.cie_kv_append_rope.argtypes = [_vp, _vp, _vp, _vp, _i64p, _i64p, _i64p, _i64p, _vp, _vp, _vp, _vp,
                                       _i, _i, _i, _i, _i, _i, _i, _i, _i, _vp, _vp, _i, _i, _vp, _i64p, _vp]
    lib.cie_kv_append_rope.restype = _i
    lib.cie_int8_matmul_workspace_bytes.argtypes = [_i, _i, _i]
    lib.cie_int8_matmul_workspace_bytes.restype = ctypes.c_size_t
    lib.cie_int8_matmul.argtypes = [_vp, _vp, _vp, _vp, _vp, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                                    _i, _i, _i, _i, _i, _vp, ctypes.c_size_t, _vp]
    lib.cie_int8_matmul.restype = _i


def load() -> ctypes.CDLL:
    """Load (once) and return the library handle."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise NativeLibraryError(
                    f"{LIB_PATH} is not built; run `python custom-inference-engine_amd/build_lib.py`")
            lib = ctypes.CDLL(LIB_PATH)
            _declare(lib)
            ver = lib.cie_abi_version()
            if ver != ABI_VERSION:
                raise NativeLibraryError(f"libcie_attn ABI {ver}, expected {ABI_VERSION}")
            _lib = lib
    return _lib


def last_error() -> str:
    return load().cie_last_error().decode()


def check(rc: int) -> None:
    """Raise the reference's exception type for a failing status code."""
    if rc == CIE_OK:
        return
    msg = last_error()
    if rc in (CIE_EHEADDIM, CIE_EDTYPE, CIE_EINVAL):
        raise ValueError(msg)
    raise NativeLibraryError(msg)


def strides(t: torch.Tensor) -> ctypes.Array:
    """Element strides of a 4-d tensor; a size-1 dimension's stride is never
    multiplied by a non-zero index, so it is passed as 0."""
    st = [0 if t.shape[i] == 1 else t.stride(i) for i in range(3)] + [t.stride(3)]
    return (ctypes.c_int64 * 4)(*st)


def strides3(t: torch.Tensor) -> ctypes.Array:
    """Element strides of a (T, Hk, D) tensor (size-1 dimensions as 0)."""
    st = [0 if t.shape[i] == 1 else t.stride(i) for i in range(2)] + [t.stride(2)]
    return (ctypes.c_int64 * 3)(*st)


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream
