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

from ._lib import MIIKV_EWORKSPACE, call, check, lib
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
        if h and lib is not None:  # module globals may already be gone at interpreter exit
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
            # the forks completed before the pool ran out hold page references and fresh
            # pages: give them back, so a failed call leaves the pool as it found it
            for c in range(done.value):
                self.release(rows[c], length, page_tokens)
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
        """Drop the row's page references; its entries become -1 (in place)."""
        work = np.ascontiguousarray(row, np.int32)
        call("miikv_pool_release", self._h, _i32p(work), length, page_tokens)
        if work is not row:
            row[...] = work


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


class PrefixRegistry:
    """Several saved prefixes over one page pool (one block-table row shared by every
    attention layer's cache).  Each entry keeps the ReusableContext fingerprint
    (reusable_context.hpp:17-129), a pool reference on each page of its row and,
    optionally, a recurrent-state checkpoint; lookup picks the longest prefix that
    passes check_match's rule (reusable_context.cpp:155-185), fork gives a new
    session a row sharing the entry's pages (the partial last page copied) and
    restores the checkpoint.  A full registry evicts its least recently used entry."""

    def __init__(self, pool: PagePool, page_tokens: int = 256, max_entries: int = 16,
                 model_id: str = "Qwen3.8-27B", quantization: str = "Q4_K_M"):
        self.pool = pool
        self.page_tokens = page_tokens
        self.model_id = model_id
        self.quantization = quantization
        self._h = lib().miikv_registry_create(pool._h, page_tokens, max_entries, model_id.encode(),
                                              quantization.encode())
        if not self._h:
            raise ValueError("invalid registry geometry")
        self._checkpoints: dict[int, RecurrentStates] = {}
        self._next_tag = 1

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            lib().miikv_registry_destroy(h)
            self._h = None

    def __len__(self) -> int:
        return int(lib().miikv_registry_count(self._h))

    def save(self, tokens, row: np.ndarray, states: RecurrentStates | None = None) -> int:
        """Register tokens held by the pages of `row` (+ a checkpoint of `states`);
        returns the entry id.  Evicts least recently used entries while full."""
        t = np.ascontiguousarray(tokens, np.uint32)
        row = np.ascontiguousarray(row, np.int32)
        tag = self._next_tag
        eid = ctypes.c_uint32(0)
        while True:
            st = lib().miikv_registry_save(self._h, t.ctypes.data_as(ctypes.c_void_p), t.size, _i32p(row),
                                           row.size, tag, ctypes.byref(eid))
            if st != MIIKV_EWORKSPACE or len(self) == 0:  # EWORKSPACE: the registry is full
                break
            self.evict_lru()
        check("miikv_registry_save", st)
        info = self.info(eid.value)
        if info["tag"] == tag:  # a new entry (an existing one keeps its checkpoint)
            self._next_tag += 1
            if states is not None:
                ck = RecurrentStates(states.layers, states.state_elems, states.conv_elems,
                                     device=states.buf.device)
                clone_states(states, [ck])
                ck.position = t.size
                self._checkpoints[tag] = ck
        return eid.value

    def lookup(self, prompt, model_id: str | None = None, quantization: str | None = None,
               strict: bool = True):
        """(MatchResult, entry id, prefix length) of the longest matching entry."""
        p = np.ascontiguousarray(prompt, np.uint32)
        eid = ctypes.c_uint32(0)
        n = ctypes.c_uint32(0)
        r = lib().miikv_registry_lookup(self._h, p.ctypes.data_as(ctypes.c_void_p), p.size,
                                        (model_id or self.model_id).encode(),
                                        (quantization or self.quantization).encode(), int(strict),
                                        ctypes.byref(eid), ctypes.byref(n))
        return MatchResult(r), eid.value, n.value

    def fork(self, entry_id: int, row_capacity: int, states: RecurrentStates | None = None):
        """A session row from an entry: (child_row, [(src, dst)] page copies to run);
        restores the entry's checkpoint into `states` (restore_gdn_states,
        reusable_context.cpp:187-200)."""
        child = np.full(row_capacity, -1, np.int32)
        src = np.zeros(1, np.int32)
        dst = np.zeros(1, np.int32)
        n = ctypes.c_uint32(0)
        call("miikv_registry_fork", self._h, entry_id, _i32p(child), row_capacity, _i32p(src), _i32p(dst),
             ctypes.byref(n))
        if states is not None:
            info = self.info(entry_id)
            ck = self._checkpoints.get(info["tag"])
            if ck is None:
                raise RuntimeError("entry has no recurrent-state checkpoint")
            clone_states(ck, [states])
            states.position = info["length"]
        return child, [(int(src[0]), int(dst[0]))] if n.value else []

    def _drop_tag(self, tag: int) -> None:
        self._checkpoints.pop(tag, None)

    def release(self, entry_id: int) -> None:
        tag = ctypes.c_uint64(0)
        call("miikv_registry_release", self._h, entry_id, ctypes.byref(tag))
        self._drop_tag(tag.value)

    def evict_lru(self) -> int:
        eid = ctypes.c_uint32(0)
        tag = ctypes.c_uint64(0)
        call("miikv_registry_evict_lru", self._h, ctypes.byref(eid), ctypes.byref(tag))
        self._drop_tag(tag.value)
        return eid.value

    def evict_until_free(self, min_free_pages: int) -> list[int]:
        """Evict least recently used entries until the pool has min_free_pages free
        pages (or the registry is empty); returns the evicted ids."""
        out = []
        while self.pool.free_pages < min_free_pages and len(self):
            out.append(self.evict_lru())
        return out

    def info(self, entry_id: int) -> dict:
        length = ctypes.c_uint32(0)
        h = ctypes.c_uint64(0)
        tag = ctypes.c_uint64(0)
        call("miikv_registry_info", self._h, entry_id, ctypes.byref(length), ctypes.byref(h),
             ctypes.byref(tag), None, 0)
        pages = np.zeros(-(-length.value // self.page_tokens), np.int32)
        call("miikv_registry_info", self._h, entry_id, None, None, None, _i32p(pages), pages.size)
        return {"length": length.value, "hash": h.value, "tag": tag.value, "pages": pages}

    def _set_layout_version(self, entry_id: int, v: int) -> None:
        call("miikv_registry_set_layout_version", self._h, entry_id, v)
