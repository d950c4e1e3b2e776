"""ctypes binding of libmiikv.so (the C ABI declared in include/miikv.h).

``import torch`` happens first so that the HIP runtime torch ships
(``libamdhip64.so.7``) is the one libmiikv resolves to: device pointers and
streams are then shared between torch and the library.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must precede loading libmiikv, see module docstring)

from .build import LIB

MIIKV_OK = 0
MIIKV_EINVAL = 1
MIIKV_EUNSUPPORTED = 2
MIIKV_EWORKSPACE = 3

LAYOUT_CONTIGUOUS = 0
LAYOUT_PAGED = 1

KV_FP16_FP16 = 0
KV_Q8_FP16 = 1
KV_FP16_Q8 = 2
KV_Q8_Q8 = 3
SUFFIX_TILES_CURRENT = 1  # MIIKV_SUFFIX_TILES_CURRENT
SUFFIX_EXACT = 2  # MIIKV_SUFFIX_EXACT

DTYPE_F16 = 0
DTYPE_F32 = 1


class MiikvView(ctypes.Structure):
    _fields_ = [
        ("k_codes", ctypes.c_void_p),
        ("k_scales", ctypes.c_void_p),
        ("v_codes", ctypes.c_void_p),
        ("v_scales", ctypes.c_void_p),
        ("layout", ctypes.c_uint32),
        ("quant_mode", ctypes.c_uint32),
        ("kv_heads", ctypes.c_uint32),
        ("head_dim", ctypes.c_uint32),
        ("page_tokens", ctypes.c_uint32),
        ("num_pages", ctypes.c_uint32),
        ("block_table", ctypes.c_void_p),
        ("table_stride", ctypes.c_uint32),
        ("reserved", ctypes.c_uint32),
    ]


class MiikvSegment(ctypes.Structure):
    _fields_ = [("dst", ctypes.c_void_p), ("src", ctypes.c_void_p), ("bytes", ctypes.c_uint64)]


DECODE_STATE_BYTES = 64
PREFILL_STATE_BYTES = 64

# Every symbol include/miikv.h declares, with (restype, argtypes).
_P = ctypes.c_void_p
_U32 = ctypes.c_uint32
_U64 = ctypes.c_uint64
_VP = ctypes.POINTER(MiikvView)
SIGNATURES = {
    "miikv_abi_version": (_U32, []),
    "miikv_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "miikv_plane_bytes": (ctypes.c_int, [_VP, ctypes.POINTER(_U64), ctypes.POINTER(_U64)]),
    "miikv_append_f16": (ctypes.c_int, [_VP, _P, _P, _U32, _U32, _U32, _P, _P, _P]),
    "miikv_append_batch_f16": (ctypes.c_int, [_VP, _P, _P, _U32, _P, _P]),
    "miikv_append_f32": (ctypes.c_int, [_VP, _P, _P, _P, _U32, _U32, _U32, ctypes.c_float,
                                         ctypes.c_float, _P, _P, _P]),
    "miikv_decode_workspace_bytes": (_U64, [_VP, _U32, _U32, _U32]),
    "miikv_workspace_init": (ctypes.c_int, [_P, _U64, _P]),
    "miikv_decode_attn": (ctypes.c_int, [_VP, _P, _U32, _U32, ctypes.c_float, _U32, _P, _P, _U32,
                                          _P, _P, _P, _P, _U64, _P]),
    "miikv_decode_attn_q8_1": (ctypes.c_int, [_VP, _P, _U32, _U32, ctypes.c_float, _U32, _P, _P, _U32,
                                               _P, _P, _P, _P, _P, _U64, _P]),
    "miikv_decode_append_attn": (ctypes.c_int, [_VP, _P, _P, _P, _U32, _U32, ctypes.c_float, _U32, _P, _P,
                                                 _U32, _P, _P, _P, _P, _P, _U64, _P]),
    "miikv_export_canonical": (ctypes.c_int, [_VP, _U32, _U32, _U32, _P, _P, _P, _P, _P]),
    "miikv_import_canonical": (ctypes.c_int, [_VP, _U32, _U32, _U32, _P, _P, _P, _P, _P]),
    "miikv_decode_append_attn_f32": (ctypes.c_int, [_VP, _P, _P, _P, ctypes.c_float, ctypes.c_float, _P, _U32, _U32,
                                                     ctypes.c_float, _U32, _P, _P, _U32, _P, _P, _P, _P, _P, _U64,
                                                     _P]),
    "miikv_decode_scratch_max_bytes": (ctypes.c_uint64, []),
    "miikv_decode_append_attn_noalloc": (ctypes.c_int, [_VP, _P, _P, _P, _U32, _U32, ctypes.c_float, _U32, _P,
                                                         _P, _U32, _P, _P, _P, _P, _P]),
    "miikv_registry_create": (ctypes.c_void_p, [_P, _U32, _U32, ctypes.c_char_p, ctypes.c_char_p]),
    "miikv_registry_destroy": (None, [_P]),
    "miikv_registry_count": (_U32, [_P]),
    "miikv_registry_save": (ctypes.c_int, [_P, _P, _U32, _P, _U32, ctypes.c_uint64, _P]),
    "miikv_registry_lookup": (ctypes.c_int, [_P, _P, _U32, ctypes.c_char_p, ctypes.c_char_p, _U32, _P, _P]),
    "miikv_registry_fork": (ctypes.c_int, [_P, _U32, _P, _U32, _P, _P, _P]),
    "miikv_registry_release": (ctypes.c_int, [_P, _U32, _P]),
    "miikv_registry_evict_lru": (ctypes.c_int, [_P, _P, _P]),
    "miikv_registry_info": (ctypes.c_int, [_P, _U32, _P, _P, _P, _P, _U32]),
    "miikv_registry_set_layout_version": (ctypes.c_int, [_P, _U32, _U32]),
    "miikv_export_dequant": (ctypes.c_int, [_VP, _U32, _U32, _U32, _P, _P, _P]),
    "miikv_copy_pages": (ctypes.c_int, [_VP, _P, _P, _U32, _P]),
    "miikv_copy_segments": (ctypes.c_int, [_P, _U32, _P]),
    "miikv_decode_state_advance": (ctypes.c_int, [_P, _P, _U32, _P, _U32, _P]),
    "miikv_clone_state": (ctypes.c_int, [_P, _P, _U64, _U32, _P]),
    "miikv_stream_read": (ctypes.c_int, [_P, _U64, _P, _U32, _P]),
    "miikv_suffix_workspace_bytes": (_U64, [_VP, _U32, _U32]),
    "miikv_suffix_workspace_bytes_ex": (_U64, [_VP, _U32, _U32, _U32]),
    "miikv_pool_create": (_P, [_U32]),
    "miikv_pool_destroy": (None, [_P]),
    "miikv_pool_alloc": (ctypes.c_int32, [_P]),
    "miikv_pool_ref": (ctypes.c_int, [_P, ctypes.c_int32]),
    "miikv_pool_unref": (ctypes.c_int, [_P, ctypes.c_int32]),
    "miikv_pool_refcount": (_U32, [_P, ctypes.c_int32]),
    "miikv_pool_free_pages": (_U32, [_P]),
    "miikv_pool_fork": (ctypes.c_int, [_P, _P, _U32, _U32, _U32, _P, _P, _P, _P]),
    "miikv_pool_fork_n": (ctypes.c_int, [_P, _P, _U32, _U32, _U32, _P, _U32, _P, _P, _P, _P]),
    "miikv_pool_prepare_append": (ctypes.c_int, [_P, _P, _U32, _U32, _U32, _P, _P, _P]),
    "miikv_pool_release": (ctypes.c_int, [_P, _P, _U32, _U32]),
    "miikv_token_hash": (_U64, [_P, ctypes.c_size_t]),
    "miikv_prefix_create": (_P, [ctypes.c_char_p, ctypes.c_char_p]),
    "miikv_prefix_destroy": (None, [_P]),
    "miikv_prefix_save": (ctypes.c_int, [_P, _P, ctypes.c_size_t]),
    "miikv_prefix_check": (ctypes.c_int, [_P, _P, ctypes.c_size_t, ctypes.c_char_p, ctypes.c_char_p]),
    "miikv_prefix_clear": (None, [_P]),
    "miikv_prefix_length": (_U32, [_P]),
    "miikv_prefix_hash": (_U64, [_P]),
    "miikv_prefix_set_layout_version": (None, [_P, _U32]),
    "miikv_session_kv_mode": (_U32, [_U32]),
    "miikv_session_filename": (ctypes.c_int, [_U64, _U32, ctypes.c_char_p, ctypes.c_size_t]),
    "miikv_session_save": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, _P, _U32, _P,
                                           _U32, _U32, _P, _P, _U32, _P]),
    "miikv_session_inspect": (ctypes.c_int, [ctypes.c_char_p, _P, _P, _U32]),
    "miikv_session_load": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, _P, _U32, _U32,
                                           _P, _P, _U32, _P, _U32, _P, _P]),
    "miikv_session_find": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, _P,
                                           ctypes.c_size_t, ctypes.c_char_p, ctypes.c_size_t, _P]),
    "miikv_suffix_attn": (ctypes.c_int, [_VP, _P, _U32, _U32, ctypes.c_float, _U32, _U32, _U32, _P,
                                          _P, _P, _P, _P, _U64, _P]),
    "miikv_suffix_append_attn": (ctypes.c_int, [_VP, _P, _P, _P, _U32, _U32, ctypes.c_float, _U32, _U32, _U32,
                                                 _P, _P, _P, _P, _P, _U64, _P]),
    "miikv_suffix_attn_ex": (ctypes.c_int, [_VP, _P, _P, _P, _U32, _U32, ctypes.c_float, _U32, _U32, _U32,
                                             _P, _U32, _P, _P, _P, _P, _U64, _P]),
}

_lib = None


class MiikvError(RuntimeError):
    def __init__(self, fn: str, status: int):
        self.status = status
        msg = lib().miikv_status_string(status).decode()
        super().__init__(f"{fn} failed with status {status} ({msg})")


def lib() -> ctypes.CDLL:
    """Load libmiikv.so; raise loudly if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            raise RuntimeError(
                f"{LIB} is missing: build it with `python -m miinfer_amd.build` "
                "(or __graft_entry__.build()); there is no CPU fallback")
        l = ctypes.CDLL(LIB)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def check(fn: str, status: int) -> None:
    if status != MIIKV_OK:
        raise MiikvError(fn, status)


def call(fn: str, *args) -> None:
    check(fn, getattr(lib(), fn)(*args))
