"""The C-ABI library on the host (no GPU): it loads, exports every symbol that
include/miikv.h declares, and rejects invalid arguments before launching
anything (the reference aborts instead: include/miinfer/hip_check.hpp:11-38)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "miikv.h")


def _declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(miikv_[a-z0-9_]+)\s*\(", text)))


def _lib():
    import torch  # noqa: F401  (shares its HIP runtime with the library)

    from miinfer_amd import _lib
    return _lib


def test_header_declares_the_boundary():
    syms = _declared_symbols()
    for must in ("miikv_append_f16", "miikv_decode_attn", "miikv_copy_pages", "miikv_clone_state",
                 "miikv_export_canonical", "miikv_decode_workspace_bytes"):
        assert must in syms


def test_library_exports_every_declared_symbol():
    L = _lib()
    lib = ctypes.CDLL(L.LIB)
    missing = [s for s in _declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing
    # and the Python binding knows each of them
    assert not [s for s in _declared_symbols() if s not in L.SIGNATURES]


def _view(**over):
    L = _lib()
    v = L.MiikvView()
    v.k_codes = v.v_codes = 0x1000
    v.k_scales = v.v_scales = 0x2000
    v.layout = L.LAYOUT_CONTIGUOUS
    v.quant_mode = L.KV_Q8_Q8
    v.kv_heads = 8
    v.head_dim = 128
    v.page_tokens = 4096
    v.num_pages = 1
    for k, val in over.items():
        setattr(v, k, val)
    return v


def test_version_and_status_strings():
    L = _lib()
    lib = L.lib()
    assert lib.miikv_abi_version() == 1
    assert lib.miikv_status_string(L.MIIKV_EINVAL) == b"invalid argument"


@pytest.mark.parametrize("over,status", [
    ({"head_dim": 64}, 2), ({"quant_mode": 7}, 1), ({"page_tokens": 100}, 1),
    # fp16 planes carry no scales; a q8 plane needs its scales
    ({"quant_mode": 0, "k_scales": None, "v_scales": None}, 0), ({"quant_mode": 1, "k_scales": None}, 1),
    ({"kv_heads": 0}, 1), ({"layout": 7}, 1), ({"num_pages": 2}, 1),
    ({"layout": 1, "num_pages": 4}, 1),  # paged without a block table
])
def test_plane_bytes_validation(over, status):
    L = _lib()
    cb, sb = ctypes.c_uint64(), ctypes.c_uint64()
    assert L.lib().miikv_plane_bytes(ctypes.byref(_view(**over)), ctypes.byref(cb),
                                     ctypes.byref(sb)) == status


def test_plane_bytes_geometry():
    L = _lib()
    cb, sb = ctypes.c_uint64(), ctypes.c_uint64()
    assert L.lib().miikv_plane_bytes(ctypes.byref(_view()), ctypes.byref(cb), ctypes.byref(sb)) == 0
    assert cb.value == 8 * 4096 * 128 and sb.value == 8 * 4096 * 4 * 2


def test_decode_rejects_before_launch():
    L = _lib()
    lib = L.lib()
    v = _view()
    ws = ctypes.c_void_p(0x3000)
    f = ctypes.c_float(0.1)
    # q_heads not a multiple of kv_heads
    assert lib.miikv_decode_attn(ctypes.byref(v), ctypes.c_void_p(0x10), 0, 30, f, 1,
                                 ctypes.c_void_p(0x20), None, 4096, ctypes.c_void_p(0x30), None,
                                 None, ws, 1 << 30, None) == L.MIIKV_EINVAL
    # max_context above the capacity
    assert lib.miikv_decode_attn(ctypes.byref(v), ctypes.c_void_p(0x10), 0, 32, f, 1,
                                 ctypes.c_void_p(0x20), None, 8192, ctypes.c_void_p(0x30), None,
                                 None, ws, 1 << 30, None) == L.MIIKV_EINVAL
    # no length source
    assert lib.miikv_decode_attn(ctypes.byref(v), ctypes.c_void_p(0x10), 0, 32, f, 1, None, None,
                                 4096, ctypes.c_void_p(0x30), None, None, ws, 1 << 30,
                                 None) == L.MIIKV_EINVAL
    # workspace too small
    need = lib.miikv_decode_workspace_bytes(ctypes.byref(v), 32, 1, 4096)
    assert need > 0
    assert lib.miikv_decode_attn(ctypes.byref(v), ctypes.c_void_p(0x10), 0, 32, f, 1,
                                 ctypes.c_void_p(0x20), None, 4096, ctypes.c_void_p(0x30), None,
                                 None, ws, need - 1, None) == L.MIIKV_EWORKSPACE
    # a gate without gated output
    assert lib.miikv_decode_attn(ctypes.byref(v), ctypes.c_void_p(0x10), 0, 32, f, 1,
                                 ctypes.c_void_p(0x20), None, 4096, ctypes.c_void_p(0x30),
                                 ctypes.c_void_p(0x40), None, ws, need, None) == L.MIIKV_EINVAL
    # more than 16 query heads per kv head (the MFMA's columns): not served by decode,
    # no workspace size; the suffix path (rows are (token, head) pairs) still serves it
    assert lib.miikv_decode_attn(ctypes.byref(v), ctypes.c_void_p(0x10), 0, 17 * 8, f, 1,
                                 ctypes.c_void_p(0x20), None, 4096, ctypes.c_void_p(0x30), None,
                                 None, ws, 1 << 30, None) == L.MIIKV_EUNSUPPORTED
    assert lib.miikv_decode_workspace_bytes(ctypes.byref(v), 17 * 8, 1, 4096) == 0
    assert lib.miikv_decode_workspace_bytes(ctypes.byref(v), 16 * 8, 1, 4096) > 0
    assert lib.miikv_suffix_workspace_bytes(ctypes.byref(v), 17 * 8, 4) > 0


def test_append_rejects_before_launch():
    L = _lib()
    lib = L.lib()
    v = _view()
    p = ctypes.c_void_p(0x10)
    assert lib.miikv_append_f16(ctypes.byref(v), p, p, 2, 4095, 0, None, None, None) == L.MIIKV_EINVAL
    assert lib.miikv_append_f16(ctypes.byref(v), p, p, 1, 0, 1, None, None, None) == L.MIIKV_EINVAL
    assert lib.miikv_append_f16(None, p, p, 1, 0, 0, None, None, None) == L.MIIKV_EINVAL
    assert lib.miikv_clone_state(p, p, 17, 2, None) == L.MIIKV_EINVAL  # not a multiple of 16
    assert lib.miikv_copy_segments(None, 3, None) == L.MIIKV_EINVAL


def test_workspace_bytes_scales_with_geometry():
    L = _lib()
    lib = L.lib()
    v = _view(page_tokens=32768)
    small = lib.miikv_decode_workspace_bytes(ctypes.byref(v), 32, 1, 4096)
    big = lib.miikv_decode_workspace_bytes(ctypes.byref(v), 32, 1, 32768)
    assert 0 < small <= big and big % 256 == 0
    assert lib.miikv_decode_workspace_bytes(ctypes.byref(v), 30, 1, 4096) == 0


def test_suffix_workspace_bytes_plan():
    """Suffix workspace: the expanded fp16 tiles of every 32-key step of the capacity
    (2*D*32 halves per step and kv head) plus, when the key range is split, one record
    per query row (token x head of the group), kv head and split: the row's normalised
    output in fp16 (2*D bytes) and its (m, l) pair in fp32 (8 bytes).  Short suffixes,
    which may run as a batch of decodes, get the tiles plus the decode records' room."""
    L = _lib()
    lib = L.lib()
    v = _view(page_tokens=8704, kv_heads=4, head_dim=256)
    tiles = 4 * (8704 // 32) * 2 * 256 * 32 * 2
    ws = lib.miikv_suffix_workspace_bytes(ctypes.byref(v), 24, 512)
    rec = 6 * (2 * 256 + 8)  # G = 6 rows per token
    assert ws > tiles and (ws - tiles) % (512 * 4 * rec) == 0
    assert 2 <= (ws - tiles) // (512 * 4 * rec) <= 64
    short = _view(page_tokens=256, kv_heads=4, head_dim=256)
    # 17 tokens (no packing: 17 decode row sets) run on the MFMA path, one split
    assert lib.miikv_suffix_workspace_bytes(ctypes.byref(short), 24, 17) == 4 * 8 * 2 * 256 * 32 * 2
    # 16 tokens may run as decodes (2 tokens per row set, or 16 row sets with a device
    # token count): the tiles (kept current for chunked prefill) plus the larger of
    # those plans' records
    dec = max(lib.miikv_decode_workspace_bytes(ctypes.byref(short), 24, 16, 256),
              lib.miikv_decode_workspace_bytes(ctypes.byref(short), 48, 8, 256))
    assert lib.miikv_suffix_workspace_bytes(ctypes.byref(short), 24, 16) == 4 * 8 * 2 * 256 * 32 * 2 + dec
    assert lib.miikv_suffix_workspace_bytes(ctypes.byref(v), 24, 0) == 0
    assert lib.miikv_suffix_workspace_bytes(ctypes.byref(v), 25, 512) == 0  # invalid heads


def test_fused_append_and_q8_1_decode_reject_before_launch():
    L = _lib()
    lib = L.lib()
    v = _view(page_tokens=256, kv_heads=4, head_dim=256)
    p = ctypes.c_void_p(0x3000)
    nan = float("nan")
    # theta / epsilon must be finite when the prologue runs
    assert lib.miikv_append_f32(ctypes.byref(v), p, p, p, 1, 0, 0, nan, 1e-6, None, None, None) == L.MIIKV_EINVAL
    assert lib.miikv_append_f32(ctypes.byref(v), p, p, p, 1, 0, 0, 1e7, nan, None, None, None) == L.MIIKV_EINVAL
    small = _view(page_tokens=256, kv_heads=4, head_dim=32)
    assert lib.miikv_append_f32(ctypes.byref(small), p, p, p, 1, 0, 0, 1e7, 1e-6, None, None, None) != L.MIIKV_OK
    assert lib.miikv_append_f32(ctypes.byref(v), p, p, None, 300, 0, 0, 1e7, 1e-6, None, None, None) == L.MIIKV_EINVAL
    lens = ctypes.c_void_p(0x4000)
    # Q8_1 output without a gate
    assert lib.miikv_decode_attn_q8_1(ctypes.byref(v), p, L.DTYPE_F16, 24, 0.0625, 1, lens, None, 256, p, None,
                                      None, p, p, 1 << 20, None) == L.MIIKV_EINVAL


def test_decode_state_advance_rejects_before_launch():
    L = _lib()
    lib = L.lib()
    p = ctypes.c_void_p(0x3000)
    stops = (ctypes.c_uint32 * 9)(*range(9))
    assert lib.miikv_decode_state_advance(None, None, 0, None, 0, None) == L.MIIKV_EINVAL
    assert lib.miikv_decode_state_advance(p, None, 0, stops, 9, None) == L.MIIKV_EINVAL
    assert lib.miikv_decode_state_advance(p, None, 0, None, 2, None) == L.MIIKV_EINVAL


def test_suffix_workspace_bytes_ex():
    """With MIIKV_SUFFIX_EXACT the workspace holds the tiles plus every token's decode
    records (at least the plain size); the flag needs <= 16 query heads per kv head;
    unknown flags give 0."""
    L = _lib()
    lib = L.lib()
    v = _view(page_tokens=8704, kv_heads=4, head_dim=256)
    base = lib.miikv_suffix_workspace_bytes(ctypes.byref(v), 24, 512)
    assert lib.miikv_suffix_workspace_bytes_ex(ctypes.byref(v), 24, 512, 0) == base
    assert lib.miikv_suffix_workspace_bytes_ex(ctypes.byref(v), 24, 512, L.SUFFIX_TILES_CURRENT) == base
    ex = lib.miikv_suffix_workspace_bytes_ex(ctypes.byref(v), 24, 512, L.SUFFIX_EXACT)
    tiles = 4 * (8704 // 32) * 2 * 256 * 32 * 2
    assert ex >= base and ex > tiles
    assert lib.miikv_suffix_workspace_bytes_ex(ctypes.byref(v), 24, 512, L.SUFFIX_EXACT | L.SUFFIX_TILES_CURRENT) == ex
    assert lib.miikv_suffix_workspace_bytes_ex(ctypes.byref(v), 24, 512, 4) == 0
    wide = _view(page_tokens=1024, kv_heads=1, head_dim=128)
    assert lib.miikv_suffix_workspace_bytes_ex(ctypes.byref(wide), 32, 64, L.SUFFIX_EXACT) == 0  # 32 heads per kv head
    assert lib.miikv_suffix_workspace_bytes_ex(ctypes.byref(wide), 32, 64, 0) > 0
