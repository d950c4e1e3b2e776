"""Host-side objects over the miikv C ABI (device memory comes from torch).

``KvCache`` mirrors ``AttentionLayerKvCacheStorage``
(include/miinfer/prefill_v2/kv_cache.hpp:49-122, src/prefill_v2/kv_cache.cpp)
for the q8_0-32 mode, in contiguous or paged form; ``decode_attention`` mirrors
``launch_qwen35_tiled_online_attention_quant_dynamic``
(include/miinfer/qwen3_gpu_primitives.hpp:719-741).  Every compute call goes
through libmiikv; there is no fallback path.
"""
from __future__ import annotations

import contextlib
import ctypes
import math

import numpy as np
import torch

from . import _lib
from ._lib import MiikvView, call, lib

QBLOCK = 32


def _ptr(t: torch.Tensor | None) -> ctypes.c_void_p | None:
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _on_stream(stream):
    """Context for allocating a launch's temporaries: with a caller stream they are
    allocated while that stream is current, so the caching allocator does not hand
    their memory out again before the work queued on it has run."""
    return torch.cuda.stream(stream) if stream is not None else contextlib.nullcontext()


def _stream(stream) -> ctypes.c_void_p:
    s = torch.cuda.current_stream() if stream is None else stream
    return ctypes.c_void_p(s.cuda_stream)


def _u32(t: torch.Tensor) -> torch.Tensor:
    if t.dtype not in (torch.int32, torch.uint32):
        raise TypeError("expected an int32/uint32 device tensor")
    return t


class KvCache:
    """q8_0 (32-value block) K/V storage of one attention layer.

    Planes are ``[page][kv_head][slab]`` (see include/miikv.h for the slab
    tiling).  A contiguous cache is a single page of ``capacity`` tokens.
    """

    def __init__(self, kv_heads: int, head_dim: int, page_tokens: int, num_pages: int,
                 block_table: torch.Tensor | None = None, device="cuda", quant_mode: int = _lib.KV_Q8_Q8):
        if page_tokens % 64 != 0:
            raise ValueError("page_tokens must be a multiple of 64")
        if quant_mode not in (_lib.KV_FP16_FP16, _lib.KV_Q8_FP16, _lib.KV_FP16_Q8, _lib.KV_Q8_Q8):
            raise ValueError("unknown quant_mode")
        self.kv_heads = kv_heads
        self.head_dim = head_dim
        self.page_tokens = page_tokens
        self.num_pages = num_pages
        self.paged = block_table is not None
        self.block_table = block_table
        self.quant_mode = quant_mode
        # K / V planes: q8 codes + one fp16 scale per 32 values (KvCacheQuantMode Q8), or
        # fp16 rows without scales (the reference's FP16 modes, kv_cache.hpp:16-21)
        self.k_f16 = quant_mode in (_lib.KV_FP16_FP16, _lib.KV_FP16_Q8)
        self.v_f16 = quant_mode in (_lib.KV_FP16_FP16, _lib.KV_Q8_FP16)
        n = num_pages * kv_heads * page_tokens
        nb = n * (head_dim // QBLOCK)
        self.k_codes = torch.zeros(n * head_dim, dtype=torch.float16 if self.k_f16 else torch.int8, device=device)
        self.v_codes = torch.zeros(n * head_dim, dtype=torch.float16 if self.v_f16 else torch.int8, device=device)
        self.k_scales = None if self.k_f16 else torch.zeros(nb, dtype=torch.int16, device=device)
        self.v_scales = None if self.v_f16 else torch.zeros(nb, dtype=torch.int16, device=device)
        self._view = MiikvView()
        self._refresh_view()

    @classmethod
    def contiguous(cls, kv_heads: int, head_dim: int, capacity: int, device="cuda",
                   quant_mode: int = _lib.KV_Q8_Q8) -> "KvCache":
        return cls(kv_heads, head_dim, capacity, 1, None, device, quant_mode)

    @classmethod
    def paged_cache(cls, kv_heads: int, head_dim: int, num_pages: int, block_table: torch.Tensor,
                    page_tokens: int = 256, device="cuda", quant_mode: int = _lib.KV_Q8_Q8) -> "KvCache":
        return cls(kv_heads, head_dim, page_tokens, num_pages, block_table, device, quant_mode)

    def _refresh_view(self) -> None:
        v = self._view
        v.k_codes = self.k_codes.data_ptr()
        v.k_scales = None if self.k_scales is None else self.k_scales.data_ptr()
        v.v_codes = self.v_codes.data_ptr()
        v.v_scales = None if self.v_scales is None else self.v_scales.data_ptr()
        v.layout = _lib.LAYOUT_PAGED if self.paged else _lib.LAYOUT_CONTIGUOUS
        v.quant_mode = self.quant_mode
        v.kv_heads = self.kv_heads
        v.head_dim = self.head_dim
        v.page_tokens = self.page_tokens
        v.num_pages = self.num_pages
        if self.paged:
            bt = self.block_table
            if bt.dtype != torch.int32 or bt.dim() != 2 or not bt.is_contiguous():
                raise TypeError("block_table must be a contiguous int32 [batch, stride] tensor")
            # -1 marks an entry not backing any token yet (kernels only read entries
            # below each sequence's length; speculative reads clamp the index).
            if bt.numel() and (int(bt.min()) < -1 or int(bt.max()) >= self.num_pages):
                raise ValueError("block_table entries must lie in [0, num_pages) or be -1")
            v.block_table = bt.data_ptr()
            v.table_stride = bt.shape[1]
        else:
            v.block_table = None
            v.table_stride = 0

    def set_block_table(self, block_table: torch.Tensor) -> None:
        self.block_table = block_table
        self.paged = True
        self._refresh_view()

    @property
    def view(self):
        return ctypes.byref(self._view)

    @property
    def capacity(self) -> int:
        return self.page_tokens if not self.paged else self.block_table.shape[1] * self.page_tokens

    def reset(self) -> None:
        """Zero every plane (src/prefill_v2/kv_cache.cpp:99-130)."""
        for t in (self.k_codes, self.v_codes, self.k_scales, self.v_scales):
            if t is not None:
                t.zero_()

    def raw_tokens_bytes(self, tokens: int) -> int:
        """Bytes of the raw compact form of `tokens` tokens (kv_cache.cpp:214-225,
        with one fp16 scale per 32-value block)."""
        per = {False: self.head_dim + 2 * (self.head_dim // QBLOCK), True: 2 * self.head_dim}
        return tokens * self.kv_heads * (per[self.k_f16] + per[self.v_f16])

    # ---- append ----------------------------------------------------------
    def append(self, k: torch.Tensor, v: torch.Tensor, base_position: int = 0, seq: int = 0,
               prefill_state: torch.Tensor | None = None, decode_state: torch.Tensor | None = None,
               stream=None) -> None:
        """Quantize fp16 rows k, v [T, kv_heads, head_dim] into positions base_position.. ."""
        if k.dtype != torch.float16 or v.dtype != torch.float16:
            raise TypeError("append expects fp16 rows")
        if not (k.is_contiguous() and v.is_contiguous()):
            raise ValueError("rows must be contiguous")
        self._check_rows(k, v)
        self._check_seq(seq)
        for st in (prefill_state, decode_state):
            if st is not None and st.numel() * st.element_size() < 64:
                raise ValueError("device state must be a 64-byte buffer")
        t = k.shape[0]
        call("miikv_append_f16", self.view, _ptr(k), _ptr(v), t, base_position, seq,
             _ptr(prefill_state), _ptr(decode_state), _stream(stream))

    def append_f32(self, k: torch.Tensor, v: torch.Tensor, base_position: int = 0, seq: int = 0, *,
                   k_norm_weight: torch.Tensor | None = None, theta: float = 1.0e7, epsilon: float = 1.0e-6,
                   prefill_state: torch.Tensor | None = None, decode_state: torch.Tensor | None = None,
                   stream=None) -> None:
        """fp32 rows k, v [T, kv_heads, head_dim]; with k_norm_weight ([head_dim] fp32) K first
        gets RMSNorm * weight and RoPE on dims 0..63 at its position (the reference's fused
        store prologue)."""
        for t in (k, v):
            if t.dtype != torch.float32 or t.dim() != 3 or \
                    tuple(t.shape[1:]) != (self.kv_heads, self.head_dim) or not t.is_contiguous():
                raise ValueError(f"rows must be contiguous fp32 [T, {self.kv_heads}, {self.head_dim}]")
        if k.shape != v.shape:
            raise ValueError("k and v shapes differ")
        if k_norm_weight is not None and (k_norm_weight.dtype != torch.float32 or
                                          k_norm_weight.numel() != self.head_dim):
            raise ValueError("k_norm_weight must be fp32 [head_dim]")
        self._check_seq(seq)
        call("miikv_append_f32", self.view, _ptr(k), _ptr(v), _ptr(k_norm_weight), k.shape[0],
             base_position, seq, float(theta), float(epsilon), _ptr(prefill_state),
             _ptr(decode_state), _stream(stream))

    def append_batch(self, k: torch.Tensor, v: torch.Tensor, positions: torch.Tensor,
                     stream=None) -> None:
        """One row per sequence: k, v [B, kv_heads, head_dim]; positions [B] device."""
        self._check_rows(k, v)
        if positions.numel() < k.shape[0]:
            raise ValueError("one position per row is required")
        if self.paged and k.shape[0] > self.block_table.shape[0]:
            raise ValueError("more rows than block-table sequences")
        call("miikv_append_batch_f16", self.view, _ptr(k), _ptr(v), k.shape[0],
             _ptr(_u32(positions)), _stream(stream))

    def _check_rows(self, k: torch.Tensor, v: torch.Tensor) -> None:
        if k.dtype != torch.float16 or v.dtype != torch.float16:
            raise TypeError("rows must be fp16")
        if k.dim() != 3 or tuple(k.shape[1:]) != (self.kv_heads, self.head_dim) or \
                k.shape != v.shape or not (k.is_contiguous() and v.is_contiguous()):
            raise ValueError(f"rows must be contiguous [T, {self.kv_heads}, {self.head_dim}]")
        if k.device != self.k_codes.device or v.device != self.k_codes.device:
            raise ValueError("rows must live on the cache's device")

    def _check_seq(self, seq: int) -> None:
        if seq < 0 or (not self.paged and seq != 0) or \
                (self.paged and seq >= self.block_table.shape[0]):
            raise ValueError(f"sequence index {seq} out of range")

    # ---- canonical export / import ------------------------------------------
    def export_canonical(self, seq: int, t0: int, count: int, stream=None):
        """Return (k_codes, k_scales, v_codes, v_scales) canonical device tensors:
        codes [kv_heads, count, head_dim] int8, scales [kv_heads, count, head_dim/32] int16;
        an fp16 plane gives its rows [kv_heads, count, head_dim] fp16 and no scales (None)."""
        self._check_seq(seq)
        dev = self.k_codes.device
        shape = (self.kv_heads, count, self.head_dim)
        sshape = (self.kv_heads, count, self.head_dim // QBLOCK)
        kc = torch.empty(shape, dtype=torch.float16 if self.k_f16 else torch.int8, device=dev)
        vc = torch.empty(shape, dtype=torch.float16 if self.v_f16 else torch.int8, device=dev)
        ks = None if self.k_f16 else torch.empty(sshape, dtype=torch.int16, device=dev)
        vs = None if self.v_f16 else torch.empty(sshape, dtype=torch.int16, device=dev)
        call("miikv_export_canonical", self.view, seq, t0, count, _ptr(kc), _ptr(ks), _ptr(vc),
             _ptr(vs), _stream(stream))
        return kc, ks, vc, vs

    def export_dequant(self, seq: int, t0: int, count: int, keys: bool = True, values: bool = True,
                       stream=None):
        """Dequantised rows code * scale as fp32 device tensors [kv_heads, count, head_dim]
        (None for a plane not asked for)."""
        self._check_seq(seq)
        dev = self.k_codes.device
        shape = (self.kv_heads, count, self.head_dim)
        with _on_stream(stream):
            k = torch.empty(shape, dtype=torch.float32, device=dev) if keys else None
            v = torch.empty(shape, dtype=torch.float32, device=dev) if values else None
        call("miikv_export_dequant", self.view, seq, t0, count, _ptr(k), _ptr(v), _stream(stream))
        return k, v

    def download_key(self, tokens: int, seq: int = 0) -> np.ndarray:
        """Host fp32 keys [kv_heads, tokens, head_dim] of positions [0, tokens): the
        q8 branch of AttentionLayerKvCacheStorage::download_key
        (src/prefill_v2/kv_cache.cpp:132-170), float(code) * float(scale)."""
        if tokens > self.capacity:
            raise ValueError("tokens exceeds capacity")
        k, _ = self.export_dequant(seq, 0, tokens, values=False)
        return k.cpu().numpy()

    def download_value(self, tokens: int, seq: int = 0) -> np.ndarray:
        """Host fp32 values, as download_key (kv_cache.cpp:172-210)."""
        if tokens > self.capacity:
            raise ValueError("tokens exceeds capacity")
        _, v = self.export_dequant(seq, 0, tokens, keys=False)
        return v.cpu().numpy()

    def import_canonical(self, seq: int, t0: int, kc, ks, vc, vs, stream=None) -> None:
        self._check_seq(seq)
        count = kc.shape[1]
        nb = self.head_dim // QBLOCK
        planes = [(kc, self.head_dim, torch.float16 if self.k_f16 else torch.int8),
                  (vc, self.head_dim, torch.float16 if self.v_f16 else torch.int8)]
        if not self.k_f16:
            planes.append((ks, nb, torch.int16))
        if not self.v_f16:
            planes.append((vs, nb, torch.int16))
        for t, last, dt in planes:
            if t is None or tuple(t.shape) != (self.kv_heads, count, last) or t.dtype != dt or \
                    not t.is_contiguous():
                raise ValueError("canonical planes have the wrong shape or dtype")
        if self.k_f16:
            ks = None
        if self.v_f16:
            vs = None
        call("miikv_import_canonical", self.view, seq, t0, count, _ptr(kc), _ptr(ks), _ptr(vc),
             _ptr(vs), _stream(stream))

    # ---- raw compact download / upload -----------------------------------
    def download_raw(self, tokens: int, seq: int = 0) -> bytes:
        """Compact raw bytes of tokens [0, tokens): per kv head [K codes | K scales], then
        the same for V (packing order of src/prefill_v2/kv_cache.cpp:227-297)."""
        kc, ks, vc, vs = self.export_canonical(seq, 0, tokens)
        parts = []
        for codes, scales in ((kc, ks), (vc, vs)):
            c = codes.cpu().numpy()
            s = None if scales is None else scales.cpu().numpy()
            for h in range(self.kv_heads):
                parts.append(c[h].tobytes())
                if s is not None:
                    parts.append(s[h].tobytes())
        return b"".join(parts)

    def upload_raw(self, raw: bytes, tokens: int, seq: int = 0) -> None:
        """Inverse of download_raw (src/prefill_v2/kv_cache.cpp:299-369)."""
        import numpy as np
        if len(raw) != self.raw_tokens_bytes(tokens):
            raise ValueError("raw size does not match tokens")
        d, nb, hk = self.head_dim, self.head_dim // QBLOCK, self.kv_heads
        buf = np.frombuffer(raw, dtype=np.uint8)
        off = 0
        out = []
        for f16 in (self.k_f16, self.v_f16):
            if f16:  # fp16 rows per kv head, no scales
                c = np.empty((hk, tokens, d), np.float16)
                for h in range(hk):
                    c[h] = buf[off:off + tokens * d * 2].view(np.float16).reshape(tokens, d)
                    off += tokens * d * 2
                out += [torch.from_numpy(c).to(self.k_codes.device), None]
                continue
            c = np.empty((hk, tokens, d), np.int8)
            s = np.empty((hk, tokens, nb), np.int16)
            for h in range(hk):
                c[h] = buf[off:off + tokens * d].view(np.int8).reshape(tokens, d)
                off += tokens * d
                s[h] = buf[off:off + tokens * nb * 2].view(np.int16).reshape(tokens, nb)
                off += tokens * nb * 2
            out += [torch.from_numpy(c).to(self.k_codes.device),
                    torch.from_numpy(s).to(self.k_codes.device)]
        self.import_canonical(seq, 0, out[0], out[1], out[2], out[3])

    # ---- page copies -----------------------------------------------------
    def copy_pages(self, src_pages: torch.Tensor, dst_pages: torch.Tensor, stream=None) -> None:
        if src_pages.dtype != torch.int32 or dst_pages.dtype != torch.int32 or \
                src_pages.numel() != dst_pages.numel():
            raise ValueError("page lists must be int32 of equal length")
        for t in (src_pages, dst_pages):
            if t.numel() and (int(t.min()) < 0 or int(t.max()) >= self.num_pages):
                raise ValueError("page index out of range")
        call("miikv_copy_pages", self.view, _ptr(src_pages), _ptr(dst_pages), src_pages.numel(),
             _stream(stream))


class DecodeWorkspace:
    """Caller-owned decode workspace (split partials + arrival counters)."""

    def __init__(self, cache: KvCache, q_heads: int, batch: int, max_context: int):
        self.bytes = int(lib().miikv_decode_workspace_bytes(cache.view, q_heads, batch,
                                                            max_context))
        if self.bytes == 0:
            raise ValueError("invalid decode geometry")
        self.buf = torch.empty(self.bytes, dtype=torch.uint8, device=cache.k_codes.device)
        call("miikv_workspace_init", _ptr(self.buf), self.bytes,
             _stream(None))


def decode_attention(cache: KvCache, q: torch.Tensor, scale: float | None = None, *,
                     lengths: torch.Tensor | None = None, decode_state: torch.Tensor | None = None,
                     max_context: int | None = None, gate: torch.Tensor | None = None,
                     out: torch.Tensor | None = None, gated_out: torch.Tensor | None = None,
                     gated_q8_1: torch.Tensor | None = None, k_new: torch.Tensor | None = None,
                     v_new: torch.Tensor | None = None,
                     workspace: DecodeWorkspace | None = None, stream=None):
    """Single-token GQA attention over the q8_0 cache.

    q: [batch, q_heads, head_dim] fp16 or fp32.  Context lengths come from
    `lengths` (device [batch]) or `decode_state` (position + 1).  With `gate`,
    `gated_q8_1` (uint8 [batch * q_heads * head_dim / 32, 36]) receives the gated
    output as Q8_1 blocks.  With k_new / v_new (fp16 [batch, kv_heads, head_dim]) the
    new token's row is stored at position L-1 in the same launch (fused append).
    Returns (out, gated_out)."""
    batch, q_heads, d = q.shape
    if d != cache.head_dim or not q.is_contiguous() or q.dtype not in (torch.float16,
                                                                        torch.float32):
        raise ValueError("q must be contiguous fp16/fp32 [batch, q_heads, head_dim]")
    if lengths is not None and (lengths.numel() < batch or lengths.dtype not in (torch.int32,
                                                                                 torch.uint32)):
        raise ValueError("lengths must be int32 with one entry per sequence")
    if decode_state is not None and decode_state.numel() * decode_state.element_size() < 64:
        raise ValueError("decode_state must be a 64-byte device buffer")
    if cache.paged and batch > cache.block_table.shape[0]:
        raise ValueError("batch exceeds the block-table rows")
    for t in (gate, out, gated_out):
        if t is not None and (tuple(t.shape) != (batch, q_heads, d) or t.dtype != torch.float32
                              or not t.is_contiguous()):
            raise ValueError("gate/out/gated_out must be contiguous fp32 [batch, q_heads, D]")
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    if max_context is None:
        max_context = cache.capacity
    with _on_stream(stream):
        if workspace is None:
            workspace = DecodeWorkspace(cache, q_heads, batch, max_context)
        elif workspace.bytes < int(lib().miikv_decode_workspace_bytes(cache.view, q_heads, batch,
                                                                       max_context)):
            raise ValueError("workspace too small for this geometry")
        if out is None and gate is None:
            out = torch.empty((batch, q_heads, d), dtype=torch.float32, device=q.device)
        if gate is not None and gated_out is None:
            gated_out = torch.empty((batch, q_heads, d), dtype=torch.float32, device=q.device)
    if gated_q8_1 is not None:
        if gate is None:
            raise ValueError("gated_q8_1 needs a gate")
        if gated_q8_1.dtype != torch.uint8 or not gated_q8_1.is_contiguous() or \
                gated_q8_1.numel() < batch * q_heads * (d // QBLOCK) * 36:
            raise ValueError("gated_q8_1 must be contiguous uint8 [batch*q_heads*D/32, 36]")
    qd = _lib.DTYPE_F16 if q.dtype == torch.float16 else _lib.DTYPE_F32
    if (k_new is None) != (v_new is None):
        raise ValueError("k_new and v_new go together")
    if k_new is not None:
        for t in (k_new, v_new):
            if t.dtype != torch.float16 or tuple(t.shape) != (batch, cache.kv_heads, d) or \
                    not t.is_contiguous():
                raise ValueError("k_new/v_new must be contiguous fp16 [batch, kv_heads, head_dim]")
        call("miikv_decode_append_attn", cache.view, _ptr(k_new), _ptr(v_new), _ptr(q), qd, q_heads,
             float(scale), batch, _ptr(lengths), _ptr(decode_state), max_context, _ptr(out), _ptr(gate),
             _ptr(gated_out), _ptr(gated_q8_1), _ptr(workspace.buf), workspace.bytes, _stream(stream))
        return out, gated_out
    call("miikv_decode_attn_q8_1", cache.view, _ptr(q), qd, q_heads, float(scale), batch,
         _ptr(lengths), _ptr(decode_state), max_context, _ptr(out), _ptr(gate), _ptr(gated_out),
         _ptr(gated_q8_1), _ptr(workspace.buf), workspace.bytes, _stream(stream))
    return out, gated_out


def suffix_attention(cache: KvCache, q: torch.Tensor, base_position: int, scale: float | None = None,
                     *, seq: int = 0, prefill_state: torch.Tensor | None = None,
                     gate: torch.Tensor | None = None, out: torch.Tensor | None = None,
                     gated_out: torch.Tensor | None = None, split: bool = True,
                     k_new: torch.Tensor | None = None, v_new: torch.Tensor | None = None,
                     workspace: torch.Tensor | None = None, tiles_current: bool = False, exact: bool = False,
                     stream=None):
    """Causal attention of a T-token suffix (rows already appended at base_position..)
    over the cache.  q: [T, q_heads, head_dim] fp16/fp32.  Returns (out, gated_out).
    With k_new / v_new (fp16 [T, kv_heads, head_dim]) the suffix's rows are quantised
    and stored in the same pass (fused append) instead of being appended first.

    The workspace holds the context's expanded fp16 tiles plus, for split-K, the
    partial records: split=True allocates suffix_workspace_bytes() (unless given);
    split=False allocates the tiles only, which runs one split.

    tiles_current (chunked prefill, with the same `workspace` for every chunk of one
    sequence and layer): the workspace's tiles of the keys below the base position
    are current from earlier calls, so only the new steps are expanded
    (MIIKV_SUFFIX_TILES_CURRENT).

    exact (MIIKV_SUFFIX_EXACT): the reference's fp32 products -- an fp32 query's low
    half kept and the key block scales applied in fp32 -- instead of the MFMA path's
    fp16 query and tiles: long suffixes over q8 planes on the exact-product MFMA kernel,
    short ones (and chunked prefill, other quant modes) as decodes; needs
    suffix_workspace_bytes(..., exact=True)."""
    t, q_heads, d = q.shape
    if d != cache.head_dim or not q.is_contiguous() or q.dtype not in (torch.float16,
                                                                        torch.float32):
        raise ValueError("q must be contiguous fp16/fp32 [T, q_heads, head_dim]")
    cache._check_seq(seq)
    for tns in (gate, out, gated_out):
        if tns is not None and (tuple(tns.shape) != (t, q_heads, d) or tns.dtype != torch.float32
                                or not tns.is_contiguous()):
            raise ValueError("gate/out/gated_out must be contiguous fp32 [T, q_heads, D]")
    if prefill_state is not None and prefill_state.numel() * prefill_state.element_size() < 64:
        raise ValueError("prefill_state must be a 64-byte device buffer")
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    qd = _lib.DTYPE_F16 if q.dtype == torch.float16 else _lib.DTYPE_F32
    with _on_stream(stream):
        if out is None and gate is None:
            out = torch.empty((t, q_heads, d), dtype=torch.float32, device=q.device)
        if gate is not None and gated_out is None:
            gated_out = torch.empty((t, q_heads, d), dtype=torch.float32, device=q.device)
        if workspace is None:
            if split or exact:
                need = suffix_workspace_bytes(cache, q_heads, t, exact=exact)
            else:
                bound = cache.capacity if prefill_state is not None else base_position + t
                need = cache.kv_heads * ((bound + 31) // 32) * 2 * d * 32 * 2
            workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    ws_bytes = workspace.numel() * workspace.element_size()
    if (k_new is None) != (v_new is None):
        raise ValueError("k_new and v_new go together")
    if k_new is not None:
        for tns in (k_new, v_new):
            if tns.dtype != torch.float16 or tuple(tns.shape) != (t, cache.kv_heads, d) or \
                    not tns.is_contiguous():
                raise ValueError("k_new/v_new must be contiguous fp16 [T, kv_heads, head_dim]")
    if tiles_current or exact:
        flags = (_lib.SUFFIX_TILES_CURRENT if tiles_current else 0) | (_lib.SUFFIX_EXACT if exact else 0)
        call("miikv_suffix_attn_ex", cache.view, _ptr(k_new), _ptr(v_new), _ptr(q), qd, q_heads, float(scale), t,
             base_position, seq, _ptr(prefill_state), flags, _ptr(out), _ptr(gate),
             _ptr(gated_out), _ptr(workspace), ws_bytes, _stream(stream))
        return out, gated_out
    if k_new is not None:
        call("miikv_suffix_append_attn", cache.view, _ptr(k_new), _ptr(v_new), _ptr(q), qd, q_heads,
             float(scale), t, base_position, seq, _ptr(prefill_state), _ptr(out), _ptr(gate),
             _ptr(gated_out), _ptr(workspace), ws_bytes, _stream(stream))
        return out, gated_out
    call("miikv_suffix_attn", cache.view, _ptr(q), qd, q_heads, float(scale), t, base_position,
         seq, _ptr(prefill_state), _ptr(out), _ptr(gate), _ptr(gated_out),
         _ptr(workspace), ws_bytes, _stream(stream))
    return out, gated_out


def suffix_workspace_bytes(cache: KvCache, q_heads: int, tokens: int, exact: bool = False) -> int:
    if exact:
        return int(lib().miikv_suffix_workspace_bytes_ex(cache.view, q_heads, tokens, _lib.SUFFIX_EXACT))
    return int(lib().miikv_suffix_workspace_bytes(cache.view, q_heads, tokens))


def make_decode_state(position: int, device="cuda", max_generated: int = 0x7fffffff) -> torch.Tensor:
    """A 64-byte device DeviceDecodeState with `position` set (current_token 0)."""
    st = torch.zeros(16, dtype=torch.int32, device=device)
    st[1] = position
    st[4] = max_generated
    return st


def advance_decode_state(state: torch.Tensor, token_output: torch.Tensor | None = None,
                         stop_tokens=(), stream=None) -> None:
    """Device-side step of a decode state (record token, stop flag, position += 1)."""
    import numpy as np
    st = np.ascontiguousarray(list(stop_tokens), np.uint32)
    cap = 0 if token_output is None else token_output.numel()
    call("miikv_decode_state_advance", _ptr(state), _ptr(token_output), cap,
         st.ctypes.data_as(ctypes.c_void_p) if st.size else None, st.size, _stream(stream))


def make_prefill_state(base_position: int, token_count: int, kv_capacity: int = 0,
                       device="cuda") -> torch.Tensor:
    st = torch.zeros(16, dtype=torch.int32, device=device)
    st[0] = base_position
    st[1] = token_count
    st[2] = base_position + token_count
    st[3] = kv_capacity
    return st


def copy_segments(segments: list[tuple[int, int, int]], stream=None, device="cuda") -> None:
    """Device-to-device copies [(dst_ptr, src_ptr, bytes)] in one launch."""
    import numpy as np
    arr = np.array(segments, dtype=np.uint64).reshape(-1, 3)
    dev = torch.from_numpy(arr.view(np.int64)).to(device)
    call("miikv_copy_segments", _ptr(dev), len(segments), _stream(stream))
    torch.cuda.current_stream().synchronize() if stream is None else stream.synchronize()


def clone_state(dsts: list[torch.Tensor], src: torch.Tensor, stream=None) -> None:
    """Byte-clone src into every tensor of dsts in one launch."""
    ptrs = torch.tensor([d.data_ptr() for d in dsts], dtype=torch.int64, device=src.device)
    nbytes = src.numel() * src.element_size()
    for d in dsts:
        if d.numel() * d.element_size() < nbytes:
            raise ValueError("destination smaller than source")
    call("miikv_clone_state", _ptr(ptrs), _ptr(src), nbytes, len(dsts), _stream(stream))
    # keep the pointer array alive until the copy has run
    (torch.cuda.current_stream() if stream is None else stream).synchronize()
