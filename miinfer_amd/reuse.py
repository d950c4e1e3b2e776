"""Prefix-state reuse over the C ABI: page pool + copy-on-write forks for paged
q8_0 caches, recurrent-state (GDN) checkpoints and clones, and the prefix
fingerprint / match policy of ReusableContext
(include/miinfer/prefill_v2/reusable_context.hpp:17-129).
"""
from __future__ import annotations

import ctypes
import enum

import numpy as np
import torch

from ._lib import call, lib
from .kv import KvCache, _on_stream, _ptr, _stream


class MatchResult(enum.IntEnum):
    """Order of ReusableContext::MatchResult (reusable_context.hpp:91-99)."""
    EXACT_MATCH = 0
    PREFIX_MISMATCH = 1
    MODEL_MISMATCH = 2
    QUANTIZATION_MISMATCH = 3
    EMPTY_CACHE = 4
    PROMPT_SHORTER_THAN_PREFIX = 5
    VERSION_MISMATCH = 6


def _i32p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


class PagePool:
    """Reference-counted physical pages of a paged cache (host bookkeeping)."""

    def __init__(self, num_pages: int):
        self._h = lib().miikv_pool_create(num_pages)
        if not self._h:
            raise ValueError("invalid page count")
        self.num_pages = num_pages

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            lib().miikv_pool_destroy(h)
            self._h = None

    def alloc(self) -> int:
        page = lib().miikv_pool_alloc(self._h)
        if page < 0:
            raise MemoryError("page pool exhausted")
        return page

    def refcount(self, page: int) -> int:
        return int(lib().miikv_pool_refcount(self._h, page))

    @property
    def free_pages(self) -> int:
        return int(lib().miikv_pool_free_pages(self._h))

    def fork(self, parent_row: np.ndarray, length: int, page_tokens: int):
        """Child row sharing the parent's full pages; returns (child_row, [(src, dst)])."""
        parent_row = np.ascontiguousarray(parent_row, np.int32)
        child = np.full_like(parent_row, -1)
        src = np.zeros(1, np.int32)
        dst = np.zeros(1, np.int32)
        n = ctypes.c_uint32(0)
        call("miikv_pool_fork", self._h, _i32p(parent_row), parent_row.size, length, page_tokens,
             _i32p(child), _i32p(src), _i32p(dst), ctypes.byref(n))
        return child, [(int(src[0]), int(dst[0]))] if n.value else []

    def fork_many(self, parent_row: np.ndarray, length: int, page_tokens: int, n: int):
        """n children of one parent in one call: (child_rows [n, len(parent_row)],
        [(src, dst)] copy-on-write page pairs)."""
        parent_row = np.ascontiguousarray(parent_row, np.int32)
        rows = np.full((n, parent_row.size), -1, np.int32)
        src = np.zeros(max(n, 1), np.int32)
        dst = np.zeros(max(n, 1), np.int32)
        nc = ctypes.c_uint32(0)
        done = ctypes.c_uint32(0)
        r = lib().miikv_pool_fork_n(self._h, _i32p(parent_row), length, page_tokens, n, _i32p(rows),
                                    parent_row.size, _i32p(src), _i32p(dst), ctypes.byref(nc),
                                    ctypes.byref(done))
        if r != 0:
            raise MemoryError(f"page pool exhausted after {done.value} of {n} forks")
        return rows, list(zip(src[:nc.value].tolist(), dst[:nc.value].tolist()))

    def prepare_append(self, row: np.ndarray, position: int, page_tokens: int):
        """Make the page receiving `position` writable (new page or copy-on-write);
        updates `row` in place and returns the [(src, dst)] page copies to run."""
        assert row.dtype == np.int32 and row.flags["C_CONTIGUOUS"]
        src = np.zeros(1, np.int32)
        dst = np.zeros(1, np.int32)
        n = ctypes.c_uint32(0)
        call("miikv_pool_prepare_append", self._h, _i32p(row), row.size, position, page_tokens,
             _i32p(src), _i32p(dst), ctypes.byref(n))
        return [(int(src[0]), int(dst[0]))] if n.value else []

    def release(self, row: np.ndarray, length: int, page_tokens: int) -> None:
        row = np.ascontiguousarray(row, np.int32)
        call("miikv_pool_release", self._h, _i32p(row), length, page_tokens)


def run_page_copies(cache: KvCache, copies, stream=None) -> None:
    """Execute [(src, dst)] physical page copies on the device in one launch."""
    if not copies:
        return
    dev = cache.k_codes.device
    with _on_stream(stream):  # the page lists live until the copy has run on `stream`
        src = torch.tensor([c[0] for c in copies], dtype=torch.int32, device=dev)
        dst = torch.tensor([c[1] for c in copies], dtype=torch.int32, device=dev)
    cache.copy_pages(src, dst, stream)


class RecurrentStates:
    """Device recurrent state of `layers` GDN layers: per layer a state tensor and a
    conv state, held in one contiguous buffer so a checkpoint or a fork clone is one
    launch (RecurrentLayerStateStorage, include/miinfer/prefill_v2/state.hpp:16-53)."""

    def __init__(self, layers: int, state_elems: int, conv_elems: int, device="cuda"):
        self.layers = layers
        self.state_elems = state_elems
        self.conv_elems = conv_elems
        per = state_elems + conv_elems
        pad = (-per) % 4  # keep each layer 16-byte aligned
        self.stride = per + pad
        self.buf = torch.zeros(layers * self.stride, dtype=torch.float32, device=device)
        self.position = 0

    def state(self, layer: int) -> torch.Tensor:
        o = layer * self.stride
        return self.buf[o:o + self.state_elems]

    def conv(self, layer: int) -> torch.Tensor:
        o = layer * self.stride + self.state_elems
        return self.buf[o:o + self.conv_elems]

    def reset(self) -> None:
        self.buf.zero_()
        self.position = 0

    @property
    def nbytes(self) -> int:
        return self.buf.numel() * 4


def clone_states(src: RecurrentStates, dsts: list[RecurrentStates], stream=None) -> None:
    """Byte-clone src into every destination in one launch (reads src once)."""
    if not dsts:
        return
    for d in dsts:
        if d.buf.numel() != src.buf.numel():
            raise ValueError("state layouts differ")
    ptrs = torch.tensor([d.buf.data_ptr() for d in dsts], dtype=torch.int64,
                        device=src.buf.device)
    call("miikv_clone_state", _ptr(ptrs), _ptr(src.buf), src.nbytes, len(dsts), _stream(stream))
    (torch.cuda.current_stream() if stream is None else stream).synchronize()
    for d in dsts:
        d.position = src.position


class PrefixContext:
    """A saved prefix: fingerprint + recurrent-state checkpoint
    (ReusableContext, src/prefill_v2/reusable_context.cpp:130-207)."""

    def __init__(self, model_id: str = "Qwen3.8-27B", quantization: str = "Q4_K_M"):
        self._h = lib().miikv_prefix_create(model_id.encode(), quantization.encode())
        self.checkpoint: RecurrentStates | None = None

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            lib().miikv_prefix_destroy(h)
            self._h = None

    def save(self, tokens, states: RecurrentStates | None = None) -> None:
        t = np.ascontiguousarray(tokens, np.uint32)
        if t.size and states is not None:
            if self.checkpoint is None or self.checkpoint.buf.numel() != states.buf.numel():
                self.checkpoint = RecurrentStates(states.layers, states.state_elems,
                                                  states.conv_elems, device=states.buf.device)
            clone_states(states, [self.checkpoint])  # capture
        call("miikv_prefix_save", self._h, t.ctypes.data_as(ctypes.c_void_p), t.size)

    def check_match(self, prompt, model_id: str, quantization: str) -> MatchResult:
        p = np.ascontiguousarray(prompt, np.uint32)
        return MatchResult(lib().miikv_prefix_check(self._h, p.ctypes.data_as(ctypes.c_void_p),
                                                    p.size, model_id.encode(),
                                                    quantization.encode()))

    def restore(self, states: RecurrentStates) -> None:
        """restore_gdn_states (reusable_context.cpp:187-200): copy the checkpoint back and
        set the position to the prefix length."""
        if self.prefix_length == 0 or self.checkpoint is None:
            raise RuntimeError("no valid prefix to restore")
        clone_states(self.checkpoint, [states])
        states.position = self.prefix_length

    def clear(self) -> None:
        lib().miikv_prefix_clear(self._h)

    @property
    def prefix_length(self) -> int:
        return int(lib().miikv_prefix_length(self._h))

    @property
    def token_hash(self) -> int:
        return int(lib().miikv_prefix_hash(self._h))

    def _set_layout_version(self, v: int) -> None:
        lib().miikv_prefix_set_layout_version(self._h, v)


def token_hash(tokens) -> int:
    t = np.ascontiguousarray(tokens, np.uint32)
    return int(lib().miikv_token_hash(t.ctypes.data_as(ctypes.c_void_p), t.size))
