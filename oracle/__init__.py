"""CPU oracle for the quantized KV-cache path — TEST INFRASTRUCTURE ONLY.

ctypes bindings over ``libmiikv_oracle.so`` (built from ``miikv_oracle.c`` by
``make -C oracle``) plus numpy conveniences.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this package, and only as the checker: nothing in ``miinfer_amd`` imports it.

All caches handled here are canonical: codes ``[kv_heads][length][head_dim]``
int8 and scales ``[kv_heads][length][head_dim // 32]`` fp16 (as uint16 bits).
The C sources cite the reference file:line each function restates.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libmiikv_oracle.so")
_REF_PATH = os.path.join(_HERE, "_ref", "libmiikv_ref.so")
QBLOCK = 32

_f32p = ctypes.POINTER(ctypes.c_float)
_i8p = ctypes.POINTER(ctypes.c_int8)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_u32 = ctypes.c_uint32


def build(reference: str | None = None) -> None:
    """Compile the oracle (and the reference shim when ``reference`` exists)."""
    subprocess.run(["make", "-s", "-C", _HERE, "libmiikv_oracle.so"], check=True)
    if reference and os.path.isdir(reference):
        subprocess.run(["make", "-s", "-C", _HERE, "ref", f"REFERENCE={reference}"], check=True)


def _load() -> ctypes.CDLL:
    if not os.path.exists(_LIB_PATH):
        build()
    lib = ctypes.CDLL(_LIB_PATH)
    lib.miikv_oracle_f32_to_f16.restype = ctypes.c_uint16
    lib.miikv_oracle_f32_to_f16.argtypes = [ctypes.c_float]
    lib.miikv_oracle_f16_to_f32.restype = ctypes.c_float
    lib.miikv_oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
    lib.miikv_oracle_q8_0_block.argtypes = [_f32p, _i8p, _u16p]
    lib.miikv_oracle_quantize_rows_f16.argtypes = [_u16p, ctypes.c_size_t, _u32, _i8p, _u16p]
    lib.miikv_oracle_quantize_rows_f32.argtypes = [_f32p, ctypes.c_size_t, _u32, _i8p, _u16p]
    lib.miikv_oracle_rope_sincos.argtypes = [ctypes.c_float, ctypes.POINTER(ctypes.c_float),
                                             ctypes.POINTER(ctypes.c_float)]
    lib.miikv_oracle_k_norm_rope.argtypes = [_f32p, _f32p, _u32, _u32, ctypes.c_float, ctypes.c_float, _f32p]
    lib.miikv_oracle_q8_1_block.argtypes = [_f32p, ctypes.POINTER(ctypes.c_uint8)]
    lib.miikv_oracle_dequantize_rows.argtypes = [_i8p, _u16p, ctypes.c_size_t, _u32, _f32p]
    lib.miikv_oracle_attention_f32.argtypes = [_f32p, _f32p, _f32p, _u32, _u32, _u32, _u32, _u32,
                                               ctypes.c_float, _f32p, _f32p]
    lib.miikv_oracle_attention_q8.argtypes = [_f32p, _i8p, _u16p, _i8p, _u16p, _u32, _u32, _u32,
                                              _u32, _u32, ctypes.c_float, _f32p, _f32p]
    lib.miikv_oracle_suffix_attention_q8.argtypes = [_f32p, _i8p, _u16p, _i8p, _u16p, _u32, _u32,
                                                     _u32, _u32, _u32, _u32, ctypes.c_float,
                                                     _f32p, _f32p]
    lib.miikv_oracle_softmax.argtypes = [_f32p, _f32p, ctypes.c_size_t]
    lib.miikv_oracle_token_hash.restype = ctypes.c_uint64
    lib.miikv_oracle_token_hash.argtypes = [_u32p, ctypes.c_size_t]
    lib.miikv_oracle_time_attention_q8.restype = ctypes.c_double
    lib.miikv_oracle_time_attention_q8.argtypes = [_f32p, _i8p, _u16p, _i8p, _u16p, _u32, _u32,
                                                   _u32, _u32, _u32, ctypes.c_float, _f32p,
                                                   ctypes.c_int, ctypes.c_int, ctypes.c_int]
    return lib


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


def ref_lib() -> ctypes.CDLL | None:
    """The reference's own host primitives (``oracle/_ref``), or None if not built."""
    if not os.path.exists(_REF_PATH):
        return None
    r = ctypes.CDLL(_REF_PATH)
    r.miikv_ref_fp16_bits_to_float.restype = ctypes.c_float
    r.miikv_ref_fp16_bits_to_float.argtypes = [ctypes.c_uint16]
    r.miikv_ref_softmax.argtypes = [_f32p, _f32p, ctypes.c_size_t]
    return r


def _p(a: np.ndarray, t):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(t)


def _opt(a, t):
    return None if a is None else _p(a, t)


# ---- scalar / block helpers ------------------------------------------------

def f32_to_f16_bits(x: float) -> int:
    return int(lib().miikv_oracle_f32_to_f16(float(x)))


def f16_bits_to_f32(b: int) -> float:
    return float(lib().miikv_oracle_f16_to_f32(int(b)))


def q8_0_block(x: np.ndarray) -> tuple[np.ndarray, int]:
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert x.shape == (QBLOCK,)
    codes = np.zeros(QBLOCK, np.int8)
    scale = np.zeros(1, np.uint16)
    lib().miikv_oracle_q8_0_block(_p(x, _f32p), _p(codes, _i8p), _p(scale, _u16p))
    return codes, int(scale[0])


def quantize_rows(rows_f16: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """rows [..., head_dim] float16 -> (codes int8 same shape, scales uint16 [..., head_dim/32])."""
    rows = np.ascontiguousarray(rows_f16, dtype=np.float16)
    d = rows.shape[-1]
    n = rows.size // d
    codes = np.zeros(rows.shape, np.int8)
    scales = np.zeros(rows.shape[:-1] + (d // QBLOCK,), np.uint16)
    lib().miikv_oracle_quantize_rows_f16(_p(rows.view(np.uint16), _u16p), n, d,
                                         _p(codes, _i8p), _p(scales, _u16p))
    return codes, scales


def quantize_rows_f32(rows: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """rows [..., head_dim] float32 -> (codes int8, scales uint16 [..., head_dim/32])."""
    rows = np.ascontiguousarray(rows, dtype=np.float32)
    d = rows.shape[-1]
    codes = np.zeros(rows.shape, np.int8)
    scales = np.zeros(rows.shape[:-1] + (d // QBLOCK,), np.uint16)
    lib().miikv_oracle_quantize_rows_f32(_p(rows, _f32p), rows.size // d, d, _p(codes, _i8p), _p(scales, _u16p))
    return codes, scales


def rope_sincos(a: float):
    """(sin, cos) of a float32 angle with the prologue's float arithmetic."""
    s, c = ctypes.c_float(), ctypes.c_float()
    lib().miikv_oracle_rope_sincos(a, ctypes.byref(s), ctypes.byref(c))
    return s.value, c.value


def k_norm_rope(x: np.ndarray, w: np.ndarray, position: int, theta: float, eps: float) -> np.ndarray:
    """One K row after the reference's RMSNorm * weight and RoPE on dims 0..63."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    if x.size not in (64, 128, 256, 512):
        raise ValueError("head_dim must be a power of two in [64, 512] (the tree reduction)")
    out = np.zeros_like(x)
    lib().miikv_oracle_k_norm_rope(_p(x, _f32p), _p(w, _f32p), x.size, position, theta, eps, _p(out, _f32p))
    return out


def q8_1_blocks(x: np.ndarray) -> np.ndarray:
    """Rows of fp32 values (size % 32 == 0) -> uint8 [n_blocks, 36] Q8_1 blocks."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, QBLOCK)
    out = np.zeros((x.shape[0], 36), np.uint8)
    for i in range(x.shape[0]):
        lib().miikv_oracle_q8_1_block(_p(x[i], _f32p), out[i].ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)))
    return out


def dequantize_rows(codes: np.ndarray, scales: np.ndarray) -> np.ndarray:
    codes = np.ascontiguousarray(codes, np.int8)
    scales = np.ascontiguousarray(scales, np.uint16)
    d = codes.shape[-1]
    out = np.zeros(codes.shape, np.float32)
    lib().miikv_oracle_dequantize_rows(_p(codes, _i8p), _p(scales, _u16p), codes.size // d, d,
                                       _p(out, _f32p))
    return out


# ---- attention ---------------------------------------------------------------

def attention_f32(q, k, v, length, q_heads, kv_heads, head_dim, scale, gate=None):
    """q [q_heads, D]; k, v [kv_heads, stride_len, D] fp32."""
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    g = None if gate is None else np.ascontiguousarray(gate, np.float32)
    out = np.zeros((q_heads, head_dim), np.float32)
    lib().miikv_oracle_attention_f32(_p(q, _f32p), _p(k, _f32p), _p(v, _f32p), length,
                                     k.shape[1], q_heads, kv_heads, head_dim, scale,
                                     _opt(g, _f32p), _p(out, _f32p))
    return out


def attention_q8(q, k_codes, k_scales, v_codes, v_scales, length, q_heads, scale, gate=None):
    """Single-query attention over a canonical q8_0 cache. q [q_heads, D] fp32."""
    kv_heads, stride_len, d = k_codes.shape
    q = np.ascontiguousarray(q, np.float32)
    args = [np.ascontiguousarray(a) for a in (k_codes, k_scales, v_codes, v_scales)]
    g = None if gate is None else np.ascontiguousarray(gate, np.float32)
    out = np.zeros((q_heads, d), np.float32)
    lib().miikv_oracle_attention_q8(_p(q, _f32p), _p(args[0], _i8p), _p(args[1], _u16p),
                                    _p(args[2], _i8p), _p(args[3], _u16p), length, stride_len,
                                    q_heads, kv_heads, d, scale, _opt(g, _f32p), _p(out, _f32p))
    return out


def suffix_attention_q8(q, k_codes, k_scales, v_codes, v_scales, base_position, q_heads, scale,
                        gate=None):
    """q [T, q_heads, D]; the cache holds positions [0, base_position + T)."""
    kv_heads, stride_len, d = k_codes.shape
    t = q.shape[0]
    q = np.ascontiguousarray(q, np.float32)
    args = [np.ascontiguousarray(a) for a in (k_codes, k_scales, v_codes, v_scales)]
    g = None if gate is None else np.ascontiguousarray(gate, np.float32)
    out = np.zeros((t, q_heads, d), np.float32)
    lib().miikv_oracle_suffix_attention_q8(_p(q, _f32p), _p(args[0], _i8p), _p(args[1], _u16p),
                                           _p(args[2], _i8p), _p(args[3], _u16p), base_position,
                                           t, stride_len, q_heads, kv_heads, d, scale,
                                           _opt(g, _f32p), _p(out, _f32p))
    return out


def softmax(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros_like(x)
    lib().miikv_oracle_softmax(_p(x, _f32p), _p(out, _f32p), x.size)
    return out


def token_hash(tokens) -> int:
    t = np.ascontiguousarray(tokens, np.uint32)
    return int(lib().miikv_oracle_token_hash(_p(t, _u32p), t.size))


def time_attention_q8(q, k_codes, k_scales, v_codes, v_scales, length, q_heads, scale,
                      threads=1, warmup=3, reps=20) -> float:
    """Median seconds per single-query attention call on the host CPU."""
    kv_heads, stride_len, d = k_codes.shape
    q = np.ascontiguousarray(q, np.float32)
    args = [np.ascontiguousarray(a) for a in (k_codes, k_scales, v_codes, v_scales)]
    out = np.zeros((q_heads, d), np.float32)
    return float(lib().miikv_oracle_time_attention_q8(
        _p(q, _f32p), _p(args[0], _i8p), _p(args[1], _u16p), _p(args[2], _i8p),
        _p(args[3], _u16p), length, stride_len, q_heads, kv_heads, d, scale, _p(out, _f32p),
        threads, warmup, reps))
