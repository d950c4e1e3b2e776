"""Persistent session files (.miinfer) over the C ABI: save / inspect / load /
find, the reference's PersistentSession
(include/miinfer/prefill_v2/persistent_session.hpp:36-67) for caches of every quant mode
(kv_quant_mode: the reference's 0 for FP16_FP16; 4, 5, 6 for the modes with q8_0-32 planes).
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from ._lib import MiikvError, lib
from .kv import KvCache, _stream
from .reuse import RecurrentStates

SESSION_VERSION = 20260928
KV_FP16_FP16 = 0
KV_Q8_0_32 = 4
KV_Q8_0_32_FP16 = 5
KV_FP16_Q8_0_32 = 6


class SessionHeader(ctypes.Structure):
    """PersistentSessionHeader (persistent_session.hpp:18-34), packed, 157 bytes."""
    _pack_ = 1
    _fields_ = [
        ("magic", ctypes.c_char * 4),
        ("version", ctypes.c_uint32),
        ("model_id", ctypes.c_char * 64),
        ("quantization", ctypes.c_char * 32),
        ("prefix_length", ctypes.c_uint32),
        ("token_hash", ctypes.c_uint64),
        ("gdn_layers", ctypes.c_uint32),
        ("gdn_state_bytes", ctypes.c_uint64),
        ("gqa_layers", ctypes.c_uint32),
        ("kv_quant_mode", ctypes.c_uint8),
        ("kv_bytes", ctypes.c_uint64),
        ("tokens_bytes", ctypes.c_uint64),
        ("created_timestamp", ctypes.c_uint64),
    ]


def session_filename(token_hash: int, prefix_length: int) -> str:
    buf = ctypes.create_string_buffer(64)
    if lib().miikv_session_filename(token_hash, prefix_length, buf, 64) != 0:
        raise MiikvError("miikv_session_filename", 1)
    return buf.value.decode()


def _views(caches: list[KvCache]):
    arr = (type(caches[0]._view) * len(caches))()
    for i, c in enumerate(caches):
        arr[i] = c._view
    return arr


def _segments(states: RecurrentStates | None):
    """(pointers, bytes, count): per GDN layer its state, then its conv history."""
    if states is None or states.layers == 0:
        return None, None, 0
    ptrs, sizes = [], []
    for i in range(states.layers):
        for t in (states.state(i), states.conv(i)):
            ptrs.append(t.data_ptr())
            sizes.append(t.numel() * t.element_size())
    n = len(ptrs)
    return (ctypes.c_void_p * n)(*ptrs), (ctypes.c_uint64 * n)(*sizes), n


def save_session(path: str, model_id: str, quantization: str, tokens, caches: list[KvCache],
                 states: RecurrentStates | None = None, seq: int = 0, stream=None) -> None:
    t = np.ascontiguousarray(tokens, np.uint32)
    ptrs, sizes, n = _segments(states)
    r = lib().miikv_session_save(path.encode(), model_id.encode(), quantization.encode(),
                                 t.ctypes.data_as(ctypes.c_void_p), t.size, _views(caches), len(caches),
                                 seq, ptrs, sizes, n, _stream(stream))
    if r != 0:
        raise MiikvError("miikv_session_save", r)


def inspect_session(path: str, with_tokens: bool = False):
    """(SessionHeader, tokens or None), or None if the file is not a session."""
    h = SessionHeader()
    if not lib().miikv_session_inspect(path.encode(), ctypes.byref(h), None, 0):
        return None
    if not with_tokens:
        return h, None
    toks = np.zeros(h.prefix_length, np.uint32)
    if not lib().miikv_session_inspect(path.encode(), ctypes.byref(h), toks.ctypes.data_as(ctypes.c_void_p),
                                       toks.size):
        return None
    return h, toks


def load_session(path: str, model_id: str, quantization: str, caches: list[KvCache],
                 states: RecurrentStates | None = None, seq: int = 0, max_tokens: int | None = None,
                 stream=None):
    """Tokens of the loaded prefix (np.uint32), or None if the file does not match.
    On success the states' position is set to the prefix length."""
    cap = max_tokens if max_tokens is not None else caches[0].capacity
    toks = np.zeros(cap, np.uint32)
    plen = ctypes.c_uint32(0)
    ptrs, sizes, n = _segments(states)
    r = lib().miikv_session_load(path.encode(), model_id.encode(), quantization.encode(), _views(caches),
                                 len(caches), seq, ptrs, sizes, n, toks.ctypes.data_as(ctypes.c_void_p), cap,
                                 ctypes.byref(plen), _stream(stream))
    if r < 0:
        raise MiikvError("miikv_session_load", r)
    if r == 0:
        return None
    if states is not None:
        states.position = plen.value
    return toks[:plen.value]


def find_session(session_dir: str, model_id: str, quantization: str, prompt):
    """(path, prefix_length) of the longest saved prefix of prompt, or None."""
    p = np.ascontiguousarray(prompt, np.uint32)
    out = ctypes.create_string_buffer(4096)
    plen = ctypes.c_uint32(0)
    if not lib().miikv_session_find(session_dir.encode(), model_id.encode(), quantization.encode(),
                                    p.ctypes.data_as(ctypes.c_void_p), p.size, out, 4096, ctypes.byref(plen)):
        return None
    return out.value.decode(), plen.value
