"""ctypes binding of the gfx950 C ABI (include/laprune_hip.h).

The library is ``laprune_amd/_lib/liblaprune_hip.so`` built in-tree by
``laprune_amd.build``.  Loading is lazy; :func:`lib` raises ``RuntimeError``
when the library is absent or a call fails, so no caller can silently take a
non-HIP path.  Device pointers come from torch tensors; the stream is the
current torch stream of the tensor's device.
"""
from __future__ import annotations

import ctypes as C
import os
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "liblaprune_hip.so"

# status codes
LAP_OK = 0
LAP_ERR_INVALID = 1
LAP_ERR_UNSUPPORTED = 2
LAP_ERR_HIP = 3
LAP_ERR_WORKSPACE = 4

# dtype codes
F32, F16, BF16, U8, I8, I32, I64 = range(7)
LUT_HMK, LUT_GMKG = 0, 1
KEY_F16, KEY_BF16 = 0, 1
SELECT_PER_HEAD = 0x10  # key_mode flag: one top-k per query head

_TORCH_DTYPE = {
    torch.float32: F32,
    torch.float16: F16,
    torch.bfloat16: BF16,
    torch.uint8: U8,
    torch.int8: I8,
    torch.int32: I32,
    torch.int64: I64,
}

vp, i32, i64, f32, sz = C.c_void_p, C.c_int, C.c_int64, C.c_float, C.c_size_t
psz = C.POINTER(C.c_size_t)
pint = C.POINTER(C.c_int)
pu32 = C.POINTER(C.c_uint32)

# name -> argtypes; every function returns int status
SIGNATURES = {
    "lap_abi_version": [],
    "lap_device_info": [pint, pint, pint],
    "lap_lut_build": [vp, i32, i64, vp, i32, i32, i32, i32, i32, i32, i32, vp, vp],
    "lap_lut_score_grouped": [vp, i32, vp, i64, i64, i32, i32, i32, i32, i32, vp, vp],
    "lap_lut_score_gqa": [vp, vp, i64, i64, i32, i32, i32, i32, i32, i32, i32, vp, i32, vp, vp],
    "lap_lut_score_mha": [vp, i32, vp, i32, i32, i32, i32, i32, vp, vp],
    "lap_aq_lut_direct": [vp, vp, i32, vp, i32, i32, i32, i32, i32, i32, vp, vp],
    "lap_topk_workspace_size": [i32, i32, psz],
    "lap_topk_select": [vp, i64, i32, i32, i32, i32, i32, i32, i32, vp, i32, vp, sz, vp],
    "lap_retrieve_workspace_size": [i32, i32, psz],
    "lap_retrieve_topk": [vp, vp, i64, i64, i64, i32, i32, i32, i32, i32, i32, i32, vp, vp,
                          i32, vp, sz, vp],
    "lap_retrieve_score": [vp, vp, i64, i64, i64, i32, i32, i32, i32, i32, i32, vp, vp, sz, vp],
    "lap_retrieve_select": [i32, i32, i32, i32, i32, i32, vp, i32, vp, sz, vp],
    "lap_retrieve_select_heads": [i32, i32, i32, i32, i32, i32, vp, i32, vp, sz, vp],
    "lap_rope_append": [vp, i64, i64, vp, i64, i64, vp, i64, i64, vp, vp, i64, i32, i32, i32,
                        i32, i32, vp, vp, i64, i64, i64, vp, i64, i64, i64, i32, vp, vp],
    "lap_retrieve_topk_ragged": [vp, vp, i64, i64, i64, i32, i32, i32, vp, i32, i32, vp, vp, i32,
                                 vp, sz, vp],
    "lap_topk_select_ragged": [vp, i64, i32, i32, i32, i32, vp, i32, i32, vp, i32, vp, sz, vp],
    "lap_gqa_gather_kv": [vp, vp, i32, i32, i32, i32, i32, i64, i64, i64, i64, i64, i64, vp,
                          i32, i32, i32, i32, vp, vp, vp],
    "lap_attn_decode_workspace_size": [i32, i32, i32, i32, psz],
    "lap_sparse_attn_decode": [vp, i64, i64, vp, vp, i32, i32, i32, i32, i32, i32, i64, i64,
                               i64, i64, i64, i64, vp, i32, i32, i32, i32, i32, i32, f32, vp,
                               vp, sz, vp],
    "lap_sparse_attn_decode_ragged": [vp, i64, i64, vp, vp, i32, i32, i32, i32, i32, i32, i64,
                                      i64, i64, i64, i64, i64, vp, i32, i32, i32, vp, i32, i32,
                                      f32, vp, vp, sz, vp],
    "lap_dense_attn_decode": [vp, i64, i64, vp, vp, i32, i32, i32, i32, i32, i32, i64, i64,
                              i64, i64, i64, i64, f32, vp, vp, sz, vp],
    "lap_decode_step_workspace_size": [i32, i32, i32, i32, i32, i32, i32, psz],
    "lap_decode_step": [vp, vp, i64, i64, i64, i32, i32, i32, i32, i32, i32, i32, vp, i32, i32,
                        i32, i32, vp, i64, i64, vp, vp, i32, i32, i32, i32, i32, i32, i64, i64,
                        i64, i64, i64, i64, f32, vp, i32, vp, vp, sz, vp],
    "lap_decode_step_status": [vp, sz, pu32, pu32],
    "lap_decode_step_noalloc_status": [pu32, pu32],
    "lap_decode_step_noalloc_reset": [vp],
    "lap_decode_step_noalloc": [vp, vp, i64, i64, i64, i32, i32, i32, i32, i32, i32, i32, vp, i32,
                                i32, i32, i32, vp, i64, i64, vp, vp, i32, i32, i32, i32, i32, i32,
                                i64, i64, i64, i64, i64, i64, f32, vp, i32, vp, vp],
    "lap_encode_prep_size": [i32, i32, i32, psz],
    "lap_aq_reconstruct": [vp, i32, i32, i32, vp, i32, i64, i32, vp, vp],
    "lap_encode_prepare": [vp, i32, i32, i32, vp, sz, vp],
    "lap_encode_greedy": [vp, i64, i32, i32, vp, i32, i32, vp, sz, vp, i64, vp, vp],
    "lap_encode_keys": [vp, i32, i64, i64, i64, i32, i32, i32, i32, i32, vp, i32, i32, vp, sz,
                        vp, i64, i64, i64, vp, vp],
    "lap_encode_keys_ranges": [vp, i32, i64, i64, i64, i32, i32, vp, i32, i32, i32, vp, i32, i32,
                               vp, sz, vp, i64, i64, i64, vp],
    "lap_floor_empty": [i32, i32, vp],
    "lap_floor_stream": [vp, vp, i64, i64, i32, i32, i32, vp, vp],
}

_lock = threading.Lock()
_lib = None


class NativeError(RuntimeError):
    """A C-ABI call returned a non-zero status."""

    def __init__(self, fn: str, status: int, msg: str):
        super().__init__(msg or f"{fn} failed with status {status}")
        self.fn = fn
        self.status = status


def _load():
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"laprune_amd HIP library not built: {LIB_PATH} is missing "
                "(run `python -c 'import __graft_entry__ as g; g.build()'`)")
        lib = C.CDLL(str(LIB_PATH))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = C.c_int
        lib.lap_last_error.argtypes = []
        lib.lap_last_error.restype = C.c_char_p
        _lib = lib
        return lib


def lib():
    """The loaded library (raises RuntimeError if it cannot be loaded)."""
    return _load()


def available() -> bool:
    try:
        _load()
        return True
    except (RuntimeError, OSError):
        return False


def call(name: str, *args) -> None:
    """Invoke a C-ABI function; raise RuntimeError with its message on failure."""
    L = _load()
    st = getattr(L, name)(*args)
    if st != LAP_OK:
        msg = L.lap_last_error().decode("utf-8", "replace")
        raise NativeError(name, st, msg)


def size_query(name: str, *args) -> int:
    out = C.c_size_t(0)
    call(name, *args, C.byref(out))
    return int(out.value)


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _TORCH_DTYPE[dt]
    except KeyError:
        raise RuntimeError(f"dtype {dt} is not served by the HIP path") from None


def ptr(t: torch.Tensor | None):
    return None if t is None else C.c_void_p(t.data_ptr())


u32 = C.c_uint32
byref = C.byref


def stream_of(t: torch.Tensor):
    return C.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def require_cuda(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError("tensors must be on CUDA (ROCm) devices")


def device_info() -> tuple[int, int, int]:
    a, b, c = C.c_int(0), C.c_int(0), C.c_int(0)
    call("lap_device_info", C.byref(a), C.byref(b), C.byref(c))
    return a.value, b.value, c.value


def loaded_from() -> str:
    return os.fspath(LIB_PATH)
