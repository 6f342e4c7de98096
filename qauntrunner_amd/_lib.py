"""ctypes binding of libqr_attn.so (the C ABI declared in include/qr_attn.h).

The shared library is built in-tree by ``__graft_entry__.build()`` (hipcc,
gfx950).  There is no fallback: if the library is missing or cannot be
loaded, every entry point raises.
"""
from __future__ import annotations

import atexit
import ctypes
import os
import sys
import weakref

_HERE = os.path.dirname(os.path.abspath(__file__))
# QR_ATTN_LIB selects another build of the same library (the sanitizer builds of the host code)
LIB_PATH = os.environ.get("QR_ATTN_LIB") or os.path.join(_HERE, "libqr_attn.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "qr_attn.h")

PAGE_TOKENS = 256

DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2
DTYPES = {"f32": DTYPE_F32, "f16": DTYPE_F16, "bf16": DTYPE_BF16}

# weight-row formats: QuantFormat values (Dtypes.cs:6-26)
FORMATS = {"F32": 0, "F16": 1, "BF16": 2, "Q4_0": 3, "Q8_0": 4, "Q4_K": 6, "Q6_K": 7}

QR_OK = 0
QR_ERR_INVALID_ARGUMENT = -1
QR_ERR_OUT_OF_RANGE = -2
QR_ERR_OUT_OF_MEMORY = -3
QR_ERR_HIP = -4
QR_ERR_NOT_RESIDENT = -5


class QrError(Exception):
    """Base class of every error reported by libqr_attn."""

    status = None


class QrInvalidArgument(QrError, ValueError):
    status = QR_ERR_INVALID_ARGUMENT


class QrOutOfRange(QrError, IndexError):
    status = QR_ERR_OUT_OF_RANGE


class QrOutOfMemory(QrError, MemoryError):
    status = QR_ERR_OUT_OF_MEMORY


class QrHipError(QrError, RuntimeError):
    status = QR_ERR_HIP


class QrNotResident(QrError, LookupError):
    status = QR_ERR_NOT_RESIDENT


_ERRORS = {c.status: c for c in (QrInvalidArgument, QrOutOfRange, QrOutOfMemory, QrHipError, QrNotResident)}

_p = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float
_ip = ctypes.POINTER(ctypes.c_int)
_llp = ctypes.POINTER(ctypes.c_longlong)
_pp = ctypes.POINTER(ctypes.c_void_p)

# name -> argtypes (every function returns int unless listed in _RESTYPES)
SIGNATURES = {
    "qr_abi_version": [],
    "qr_last_error": [],
    "qr_status_name": [_i],
    "qr_kv_create": [_pp, _i, _i, _i, _i, _i, _i, _i],
    "qr_kv_destroy": [_p],
    "qr_kv_reserve": [_p, _i],
    "qr_kv_append": [_p, _i, _i, _i, _p, _i, _p, _i],
    "qr_kv_append_range": [_p, _i, _i, _i, _i, _p, _p, _i],
    "qr_kv_append_range_dev": [_p, _i, _i, _i, _i, _p, _p, _i, _p],
    "qr_kv_append_rope": [_p, _i, _i, _i, _p, _p, _p, _f],
    "qr_kv_append_rope_dev": [_p, _i, _i, _i, _i, _p, _p, _p, _f, _p],
    "qr_kv_append_rope_step_dev": [_p, _i, _i, _p, _p, _p, _p, _f, _p],
    "qr_kv_attention_step_dev": [_p, _i, _p, _i, _p, _p, _p, _f, _p],
    "qr_kv_append_rope_chunk_step_dev": [_p, _i, _i, _i, _p, _p, _p, _p, _f, _p],
    "qr_kv_attention_chunk_step_dev": [_p, _i, _i, _i, _p, _p, _i, _p, _f, _p],
    "qr_mla_append_step_dev": [_p, _i, _i, _p, _p, _i, _p],
    "qr_mla_attention_step_dev": [_p, _i, _p, _i, _p, _p, _f, _p, _p],
    "qr_mla_attend_absorbed_step_dev": [_p, _i, _p, _i, _i, _i, _p, _p, _i, _p, _p],
    "qr_kv_attention": [_p, _i, _i, _i, _p, _p, _f],
    "qr_kv_attention_batch": [_p, _i, _p, _i, _p, _p, _p, _f],
    "qr_kv_attention_dev": [_p, _i, _p, _i, _p, _p, _p, _f, _p],
    "qr_kv_attention_dev_noalloc": [_p, _i, _p, _i, _p, _p, _p, _f, _p],
    "qr_kv_attention_chunk": [_p, _i, _i, _i, _i, _p, _i, _p, _f],
    "qr_kv_attention_chunk_dev": [_p, _i, _i, _i, _i, _p, _i, _p, _f, _p],
    "qr_kv_set_split_event": [_p, _p],
    "qr_kv_decode_plan": [_p, _i, _p, _i, _p, _ip, _ip],
    "qr_kv_reset": [_p, _i],
    "qr_kv_truncate": [_p, _i, _i],
    "qr_kv_seq_len": [_p, _i, _ip],
    "qr_kv_bytes_used": [_p, _llp],
    "qr_kv_bytes_per_token": [_p, _llp],
    "qr_kv_read": [_p, _i, _i, _i, _i, _p, _p],
    "qr_mla_create": [_pp, _i, _i, _i, _i, _i],
    "qr_mla_create_latent": [_pp, _i, _i, _i, _i],
    "qr_mla_set_rope": [_p, _i],
    "qr_mla_max_seq": [_p, _ip],
    "qr_mla_destroy": [_p],
    "qr_mla_reserve": [_p, _i],
    "qr_mla_append": [_p, _i, _i, _p, _i],
    "qr_mla_append_range": [_p, _i, _i, _i, _p, _i],
    "qr_mla_append_range_dev": [_p, _i, _i, _i, _p, _i, _p],
    "qr_mla_attention": [_p, _i, _i, _i, _p, _p, _f, _p],
    "qr_mla_attention_dev": [_p, _i, _i, _i, _p, _p, _f, _p, _p],
    "qr_mla_reset": [_p],
    "qr_mla_truncate": [_p, _i],
    "qr_mla_seq_len": [_p, _ip],
    "qr_mla_bytes_used": [_p, _llp],
    "qr_mla_page_count": [_p, _i, _ip],
    "qr_mla_read_page": [_p, _i, _i, _p],
    "qr_mla_attend_absorbed": [_p, _i, _i, _i, _i, _i, _p, _p, _p],
    "qr_mla_attend_absorbed_dev": [_p, _i, _i, _i, _i, _i, _p, _p, _i, _p, _p],
    "qr_weight_row_bytes": [_i, _i, _llp],
    "qr_weight_create": [_pp, _i, ctypes.c_longlong, _i, _p],
    "qr_weight_destroy": [_p],
    "qr_weight_data": [_p, _pp],
    "qr_mla_q_absorb_dev": [_p, _i, _i, _i, _i, _i, _i, _i, _p, _p, _p],
    "qr_mla_wuv_dev": [_p, _i, _i, _i, _i, _i, _i, _p, _p, _p],
    "qr_matvec_dev": [_p, _i, ctypes.c_longlong, _i, _i, _p, _p, _p],
    "qr_matvec_group_dev": [_i, _p, _p, _i, _i, _i, _p, _p, _p],
    "qr_matvec": [_p, _i, _p, _p],
    "qr_model_open": [_pp, ctypes.c_char_p],
    "qr_model_close": [_p],
    "qr_model_tensor_count": [_p, _ip],
    "qr_model_tensor_name": [_p, _i, ctypes.c_char_p, _i],
    "qr_model_tensor_info": [_p, ctypes.c_char_p, _ip, _ip, _llp, _i, _llp],
    "qr_model_read": [_p, ctypes.c_char_p, _p, ctypes.c_longlong],
    "qr_model_set_prefetch": [_p, ctypes.c_longlong],
    "qr_model_begin": [_p, _i],
    "qr_model_acquire": [_p, ctypes.c_char_p, _i, _p, _pp],
    "qr_model_release": [_p, _i, _p],
    "qr_model_wait_layer": [_p, _i],
    "qr_model_make_resident": [_p],
    "qr_model_stats": [_p, _llp, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double), _ip, _ip],
}
_RESTYPES = {"qr_last_error": ctypes.c_char_p, "qr_status_name": ctypes.c_char_p}

_lib = None


def load():
    """Loads libqr_attn.so once; raises if it was not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with __graft_entry__.build()")
        lib = ctypes.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = _RESTYPES.get(name, ctypes.c_int)
        _lib = lib
    return _lib


def check(status: int) -> None:
    """Raises the QrError subclass of a non-zero status with the library's message."""
    if status == QR_OK:
        return
    lib = load()
    msg = lib.qr_last_error().decode(errors="replace")
    name = lib.qr_status_name(status).decode()
    raise _ERRORS.get(status, QrError)(f"{name}: {msg}")


# ---------------------------------------------------------------- handle lifetime
# Objects that own a library handle (caches, weights, model stores).  They are closed
# explicitly from an atexit hook, which runs while the HIP runtime is still whole; a
# finalizer that runs later, during interpreter shutdown, does nothing (the process exit
# reclaims the memory), so no hipFree or stream destroy reaches a runtime that is already
# tearing itself down.
_live = weakref.WeakSet()


def track(obj) -> None:
    """Registers an object with a close() method for the exit-time close."""
    _live.add(obj)


def finalizing() -> bool:
    return sys.is_finalizing()


@atexit.register
def _close_all() -> None:
    for obj in list(_live):
        try:
            obj.close()
        except Exception:
            pass
