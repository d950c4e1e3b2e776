"""miinfer_amd — MI355X-native quantized KV-cache path (q8_0 append, split-K GQA
decode attention, suffix attention, prefix-state reuse) behind the C ABI in
include/miikv.h.  This package is the host-side mirror of the reference's
KV-cache / attention call surface; all compute runs in libmiikv.so (HIP,
gfx950) and fails loudly when that library is missing.
"""
from ._lib import MiikvError, lib  # noqa: F401
from .kv import (  # noqa: F401
    DecodeWorkspace,
    advance_decode_state,
    KvCache,
    clone_state,
    copy_segments,
    decode_attention,
    make_decode_state,
    make_prefill_state,
    suffix_attention,
    suffix_workspace_bytes,
)

__all__ = [
    "MiikvError", "lib", "advance_decode_state", "KvCache", "DecodeWorkspace", "decode_attention", "clone_state",
    "copy_segments", "make_decode_state", "make_prefill_state", "suffix_attention", "suffix_workspace_bytes",
]
