"""Persistent session file format on the host (no GPU): header layout, file
naming, inspect / find over synthetic files, and load rejecting mismatches
before touching device memory (src/prefill_v2/persistent_session.cpp:27-320)."""
import ctypes
import os
import struct

import numpy as np
import pytest


def _sess():
    import torch  # noqa: F401  (shares its HIP runtime with the library)

    from miinfer_amd import session
    return session


def _write(path, model="Qwen3.8-27B", quant="Q4_K_M", tokens=(1, 2, 3), gdn=b"", kv=b"", version=20260928,
           magic=b"MISS", mode=4, layers=(0, 0)):
    from miinfer_amd import lib
    t = np.asarray(tokens, np.uint32)
    h = struct.pack("<4sI64s32sIQIQIBQQQ", magic, version, model.encode(), quant.encode(), t.size,
                    lib().miikv_token_hash(t.ctypes.data_as(ctypes.c_void_p), t.size), layers[0], len(gdn),
                    layers[1], mode, len(kv), t.size * 4, 1234)
    with open(path, "wb") as f:
        f.write(h + t.tobytes() + gdn + kv)


def test_header_is_the_packed_reference_layout():
    s = _sess()
    H = s.SessionHeader
    assert ctypes.sizeof(H) == 157
    offs = {n: getattr(H, n).offset for n, _ in H._fields_}
    assert offs == {"magic": 0, "version": 4, "model_id": 8, "quantization": 72, "prefix_length": 104,
                    "token_hash": 108, "gdn_layers": 116, "gdn_state_bytes": 120, "gqa_layers": 128,
                    "kv_quant_mode": 132, "kv_bytes": 133, "tokens_bytes": 141, "created_timestamp": 149}


def test_session_filename_format():
    s = _sess()
    assert s.session_filename(0x0123456789abcdef, 32768) == "sess_0123456789abcdef_p32768.miinfer"
    assert s.session_filename(5, 7) == "sess_0000000000000005_p7.miinfer"


def test_inspect_reads_header_and_tokens(tmp_path):
    s = _sess()
    p = str(tmp_path / "a.miinfer")
    _write(p, tokens=[9, 8, 7, 6])
    h, toks = s.inspect_session(p, with_tokens=True)
    assert h.prefix_length == 4 and h.kv_quant_mode == 4 and h.model_id == b"Qwen3.8-27B"
    assert list(toks) == [9, 8, 7, 6]
    _write(p, version=20260927)
    assert s.inspect_session(p) is None
    _write(p, magic=b"MISX")
    assert s.inspect_session(p) is None
    assert s.inspect_session(str(tmp_path / "missing.miinfer")) is None


def test_find_picks_the_longest_matching_prefix(tmp_path):
    s = _sess()
    d = str(tmp_path)
    _write(os.path.join(d, "a.miinfer"), tokens=[1, 2, 3])
    _write(os.path.join(d, "b.miinfer"), tokens=[1, 2, 3, 4, 5])
    _write(os.path.join(d, "c.miinfer"), tokens=[1, 2, 9, 9, 9, 9])       # diverges
    _write(os.path.join(d, "d.miinfer"), tokens=[1, 2, 3, 4, 5, 6], model="other")
    _write(os.path.join(d, "e.txt"), tokens=[1, 2, 3, 4, 5, 6])            # not a session file
    _write(os.path.join(d, "f.miinfer"), tokens=[1, 2, 3, 4, 5, 6, 7, 8])  # longer than the prompt
    _write(os.path.join(d, "g.miinfer"), tokens=[1, 2, 3, 4, 5, 6], kv=b"\0" * 64)
    with open(os.path.join(d, "g.miinfer"), "r+b") as f:                 # truncated payload
        f.truncate(157 + 24 + 10)
    path, n = s.find_session(d, "Qwen3.8-27B", "Q4_K_M", [1, 2, 3, 4, 5, 6, 7])
    assert os.path.basename(path) == "b.miinfer" and n == 5
    assert s.find_session(d, "Qwen3.8-27B", "Q4_K_M", [7, 7, 7]) is None
    assert s.find_session(d, "Qwen3.8-27B", "Q8_0", [1, 2, 3, 4, 5]) is None
    assert s.find_session(str(tmp_path / "nope"), "Qwen3.8-27B", "Q4_K_M", [1]) is None


@pytest.mark.parametrize("case", ["model", "quant", "mode", "layers", "gdn_bytes", "hash", "truncated"])
def test_load_rejects_mismatch_before_device_writes(tmp_path, case):
    """Every mismatch is found on the host; the (fake) device pointers are never used."""
    import torch
    from miinfer_amd import KvCache, _lib  # noqa: F401
    s = _sess()
    L = _lib
    p = str(tmp_path / "s.miinfer")
    P, hk, d = 3, 2, 64
    layer_bytes = 2 * P * hk * (d + 2 * d // 32)
    kw = dict(tokens=[1, 2, 3], gdn=b"\0" * 16, kv=b"\0" * (2 * layer_bytes), layers=(1, 2))
    if case == "mode":
        kw["mode"] = 3
    if case == "gdn_bytes":
        kw["gdn"] = b"\0" * 8
    _write(p, **kw)
    if case == "hash":
        with open(p, "r+b") as f:
            f.seek(157)
            f.write(struct.pack("<I", 99))
    if case == "truncated":
        with open(p, "r+b") as f:
            f.truncate(157 + 12 + 16 + layer_bytes)
    v = L.MiikvView()
    v.k_codes = v.v_codes = 0x1000
    v.k_scales = v.v_scales = 0x2000
    v.layout = L.LAYOUT_CONTIGUOUS
    v.quant_mode = L.KV_Q8_Q8
    v.kv_heads, v.head_dim, v.page_tokens, v.num_pages = hk, d, 64, 1
    views = (L.MiikvView * 2)(v, v)
    segs = (ctypes.c_void_p * 2)(0x5000, 0x6000)
    sizes = (ctypes.c_uint64 * 2)(8, 8)
    toks = np.zeros(16, np.uint32)
    plen = ctypes.c_uint32(0)
    model = b"other" if case == "model" else b"Qwen3.8-27B"
    quant = b"Q8_0" if case == "quant" else b"Q4_K_M"
    n_layers = 1 if case == "layers" else 2
    r = L.lib().miikv_session_load(p.encode(), model, quant, views, n_layers, 0, segs, sizes, 2,
                                   toks.ctypes.data_as(ctypes.c_void_p), 16, ctypes.byref(plen), None)
    assert r == 0 and plen.value == 0


# Header fields the loader checks against the caller (offset, size), and the token
# payload; a change to any byte of them must be rejected before device memory is used.
_CHECKED = [(0, 4), (4, 4), (104, 4), (108, 8), (116, 4), (120, 8), (128, 4), (132, 1), (133, 8), (141, 8)]


@pytest.mark.parametrize("seed", range(4))
def test_load_rejects_random_corruption(tmp_path, seed):
    """Random byte changes in the checked header fields, the model / quantization
    strings and the tokens of a valid file: inspect / load reject every one before
    touching device memory (the device pointers here are fake), and never crash."""
    from miinfer_amd import _lib as L
    rng = np.random.default_rng(seed)
    P, hk, d = 3, 2, 64
    layer_bytes = 2 * P * hk * (d + 2 * d // 32)
    p = str(tmp_path / "s.miinfer")
    _write(p, tokens=[1, 2, 3], gdn=b"\0" * 16, kv=b"\0" * (2 * layer_bytes), layers=(1, 2))
    good = open(p, "rb").read()
    v = L.MiikvView()
    v.k_codes = v.v_codes = 0x1000
    v.k_scales = v.v_scales = 0x2000
    v.layout = L.LAYOUT_CONTIGUOUS
    v.quant_mode = L.KV_Q8_Q8
    v.kv_heads, v.head_dim, v.page_tokens, v.num_pages = hk, d, 64, 1
    views = (L.MiikvView * 2)(v, v)
    segs = (ctypes.c_void_p * 2)(0x5000, 0x6000)
    sizes = (ctypes.c_uint64 * 2)(8, 8)
    regions = _CHECKED + [(8, len("Qwen3.8-27B")), (72, len("Q4_K_M")), (157, 12)]
    for _ in range(200):
        off, size = regions[int(rng.integers(len(regions)))]
        data = bytearray(good)
        for _ in range(int(rng.integers(1, 3))):
            i = off + int(rng.integers(size))
            data[i] = (data[i] + int(rng.integers(1, 256))) % 256
        if bytes(data) == good:
            continue  # the changes cancelled: a valid file would go on to the (fake) device pointers
        with open(p, "wb") as f:
            f.write(bytes(data))
        toks = np.zeros(16, np.uint32)
        plen = ctypes.c_uint32(0)
        r = L.lib().miikv_session_load(p.encode(), b"Qwen3.8-27B", b"Q4_K_M", views, 2, 0, segs, sizes, 2,
                                       toks.ctypes.data_as(ctypes.c_void_p), 16, ctypes.byref(plen), None)
        assert r == 0 and plen.value == 0, (off, size)
        assert not np.any(toks)


def test_session_kv_mode_values():
    """File kv_quant_mode per view mode: FP16_FP16 keeps the reference's 0 (same raw bytes,
    kv_cache.hpp:16-21); the modes with q8_0-32 planes (one scale per 32 values, not per
    row as the reference's 1..3) get 4, 5, 6; unknown modes none."""
    from miinfer_amd import _lib as L
    f = L.lib().miikv_session_kv_mode
    assert [f(m) for m in (L.KV_FP16_FP16, L.KV_Q8_FP16, L.KV_FP16_Q8, L.KV_Q8_Q8, 9)] == [0, 5, 6, 4, 0xff]
