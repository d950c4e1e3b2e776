"""Pins the CPU oracle before it is trusted as the checker (CPU only).

Each oracle function is checked against something it was not derived from:
the reference's own fixture and compiled host primitives (oracle/_ref), a
library routine (numpy fp16 conversion, scipy softmax), closed forms, or
published test vectors — chosen so that a plausible slip (wrong GQA map,
wrong rounding, dropped scale, transposed operand) fails.
"""
import os

import numpy as np
import pytest
from scipy.special import softmax as scipy_softmax

import oracle
from tests.helpers import randn_f16

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "m4a4")


# ---- fp16 conversions -------------------------------------------------------

def test_f16_decode_exhaustive_vs_numpy():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    expect = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_bits_to_f32(int(b)) for b in bits], np.float32)
    nan = np.isnan(expect)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), expect[~nan].view(np.uint32))


def test_f16_decode_exhaustive_vs_reference_build():
    ref = oracle.ref_lib()
    if ref is None:
        pytest.skip("oracle/_ref not built (reference checkout absent)")
    for b in range(65536):
        a = np.float32(oracle.f16_bits_to_f32(b)).view(np.uint32)
        r = np.float32(ref.miikv_ref_fp16_bits_to_float(b)).view(np.uint32)
        assert a == r, hex(b)


def test_f32_to_f16_rne_vs_numpy():
    rng = np.random.default_rng(7)
    # Random bit patterns cover every exponent (subnormal halves, overflow, NaN).
    x = rng.integers(0, 2**32, size=200_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    # Exact ties between two halves at several exponents, and the largest finite half.
    ties = np.array([1.0 + 2.0**-11, 1.0 + 3 * 2.0**-11, 2.0**-15 * (1 + 2.0**-11), 65504.0,
                     65520.0, 65519.99, 2.0**-25, 2.0**-24, 3 * 2.0**-26, -0.0], np.float32)
    x = np.concatenate([x, ties, -ties])
    expect = x.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f32_to_f16_bits(float(v)) for v in x], np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], expect[~nan])
    # NaN stays NaN (exponent all ones, non-zero mantissa)
    assert np.all((got[nan] & 0x7c00) == 0x7c00) and np.all((got[nan] & 0x3ff) != 0)


def test_f16_round_trip_identity():
    for b in range(0, 65536, 7):
        f = oracle.f16_bits_to_f32(b)
        if np.isnan(f):
            continue
        assert oracle.f32_to_f16_bits(f) == b


# ---- q8_0 block rule --------------------------------------------------------

def _f16_block(rng):
    return rng.standard_normal(32).astype(np.float32).astype(np.float16).astype(np.float32)


def test_q8_block_invariants_random():
    rng = np.random.default_rng(1)
    for _ in range(3000):
        x = _f16_block(rng) * np.float32(rng.choice([1e-3, 1.0, 40.0]))
        x = x.astype(np.float16).astype(np.float32)
        codes, sbits = oracle.q8_0_block(x)
        amax = np.float32(np.abs(x).max())
        scale = np.float32(amax / np.float32(127.0))
        # scale is fp16_rn(amax/127) (library conversion)
        assert sbits == int(np.array([scale], np.float32).astype(np.float16).view(np.uint16)[0])
        assert np.all(np.abs(codes.astype(np.int32)) <= 127)
        # the absmax element maps to +-127
        i = int(np.argmax(np.abs(x)))
        assert abs(int(codes[i])) == 127 and np.sign(codes[i]) == np.sign(x[i])
        # reconstruction error bounded by half a step (fp32 scale, small slack for 1/scale rounding)
        err = np.abs(x - codes.astype(np.float32) * scale)
        assert np.all(err <= 0.5 * scale * (1 + 1e-5) + 1e-30)


def test_q8_block_matches_vectorised_numpy_rule():
    """A numpy evaluation of the same rule on many blocks catches index/loop slips."""
    rng = np.random.default_rng(2)
    rows = randn_f16(rng, (512, 256))
    codes, scales = oracle.quantize_rows(rows)
    x = rows.astype(np.float32).reshape(-1, 32)
    amax = np.abs(x).max(axis=1)
    scale = np.where(amax > 0, amax / np.float32(127.0), np.float32(1.0)).astype(np.float32)
    inv = (np.float32(1.0) / scale).astype(np.float32)
    q = np.clip(np.rint((x * inv[:, None]).astype(np.float32)), -128, 127).astype(np.int8)
    assert np.array_equal(codes.reshape(-1, 32), q)
    assert np.array_equal(scales.reshape(-1), scale.astype(np.float16).view(np.uint16))


def test_q8_zero_block_keeps_reference_unit_scale():
    codes, sbits = oracle.q8_0_block(np.zeros(32, np.float32))
    assert sbits == 0x3C00 and not codes.any()  # scale 1.0h, codes 0 (qwen3_primitives.hip:7297-7299)


def test_q8_rounding_is_half_even_exhaustive():
    """amax = 127 gives scale = inv = 1 exactly, so code = rint(x): compare every fp16 value
    in [-127, 127] against Python's round-half-even."""
    halves = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    vals = halves[np.isfinite(halves) & (np.abs(halves) <= 127)]
    for start in range(0, vals.size, 31):
        chunk = vals[start:start + 31]
        x = np.zeros(32, np.float32)
        x[0] = 127.0
        x[1:1 + chunk.size] = chunk
        codes, sbits = oracle.q8_0_block(x)
        assert sbits == 0x3C00
        expect = [round(float(v)) for v in chunk]  # Python rounds half to even
        assert list(codes[1:1 + chunk.size]) == expect


def test_q8_ties_round_to_even_not_away():
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1:7] = [2.5, 3.5, -2.5, -3.5, 0.5, -0.5]
    codes, sbits = oracle.q8_0_block(x)
    assert sbits == 0x3C00
    # device rule (RNE): 2.5->2, 3.5->4, -2.5->-2, -3.5->-4, 0.5->0, -0.5->0.
    # The reference host test quantizer (std::round, half away from zero) would give 3, 4, -3,
    # -4, 1, -1: the oracle follows the device rule that the runtime stores.
    assert list(codes[1:7]) == [2, 4, -2, -4, 0, 0]


# ---- softmax / attention ------------------------------------------------------

def test_softmax_bitexact_vs_reference_build():
    ref = oracle.ref_lib()
    if ref is None:
        pytest.skip("oracle/_ref not built (reference checkout absent)")
    rng = np.random.default_rng(3)
    for n in (1, 2, 17, 4096):
        x = (rng.standard_normal(n) * 4).astype(np.float32)
        a = oracle.softmax(x)
        r = np.zeros_like(x)
        ref.miikv_ref_softmax(x.ctypes.data_as(oracle._f32p), r.ctypes.data_as(oracle._f32p), n)
        assert np.array_equal(a.view(np.uint32), r.view(np.uint32))


def test_softmax_vs_scipy():
    rng = np.random.default_rng(4)
    x = (rng.standard_normal(1000) * 6).astype(np.float32)
    np.testing.assert_allclose(oracle.softmax(x), scipy_softmax(x.astype(np.float64)), rtol=1e-6,
                               atol=1e-9)


def _load_fixture(p):
    f = lambda name: np.fromfile(os.path.join(GOLDEN, name), np.float32)
    return f(f"pos-{p}-17.f32").reshape(32, 128), f(f"pos-{p}-cache-k.f32").reshape(8, 128), \
        f(f"pos-{p}-cache-v.f32").reshape(8, 128), f(f"pos-{p}-19.f32").reshape(32, 128)


def test_attention_matches_reference_fixture_m4a4():
    """Layer-0 Qwen3-8B trace (32 q / 8 kv / D 128, the config-2 head shape): attention over
    positions 0..P must reproduce the captured output.  The reference checks this checkpoint
    at 2e-2 (tests/qwen3_kv_cache_test.cpp:32-42); the oracle is within 2e-4."""
    ks, vs = [], []
    for p in range(4):
        q, k, v, expect = _load_fixture(p)
        ks.append(k)
        vs.append(v)
        kc, vc = np.stack(ks, 1), np.stack(vs, 1)
        out = oracle.attention_f32(q, kc, vc, p + 1, 32, 8, 128, 1.0 / np.sqrt(128.0))
        assert np.abs(out - expect).max() < 2e-4, p
        # comparator mutations must be caught: wrong GQA map and a dropped scale
        if p >= 1:
            bad = oracle.attention_f32(q, kc[np.arange(8)[::-1]], vc[np.arange(8)[::-1]], p + 1,
                                       32, 8, 128, 1.0 / np.sqrt(128.0))
            assert np.abs(bad - expect).max() > 2e-3
            bad = oracle.attention_f32(q, kc, vc, p + 1, 32, 8, 128, 1.0)
            assert np.abs(bad - expect).max() > 2e-3


def _attention_f64(q, k, v, length, scale):
    hq, d = q.shape
    hk = k.shape[0]
    grp = hq // hk
    out = np.zeros((hq, d))
    for h in range(hq):
        kk = k[h // grp, :length].astype(np.float64)
        vv = v[h // grp, :length].astype(np.float64)
        p = scipy_softmax(kk @ q[h].astype(np.float64) * scale)
        out[h] = p @ vv
    return out


@pytest.mark.parametrize("hq,hk,d,length", [(32, 8, 128, 1), (32, 8, 128, 300), (24, 4, 256, 97),
                                            (4, 1, 128, 1000)])
def test_attention_q8_vs_float64(hq, hk, d, length):
    rng = np.random.default_rng(length + d)
    rows_k = randn_f16(rng, (hk, length, d))
    rows_v = randn_f16(rng, (hk, length, d))
    kc, ksc = oracle.quantize_rows(rows_k)
    vc, vsc = oracle.quantize_rows(rows_v)
    q = randn_f16(rng, (hq, d)).astype(np.float32)
    scale = 1.0 / np.sqrt(d)
    out = oracle.attention_q8(q, kc, ksc, vc, vsc, length, hq, scale)
    kdq = oracle.dequantize_rows(kc, ksc)
    vdq = oracle.dequantize_rows(vc, vsc)
    np.testing.assert_allclose(out, _attention_f64(q, kdq, vdq, length, scale), atol=2e-5)


def test_attention_closed_forms():
    rng = np.random.default_rng(5)
    d = 128
    rows_v = randn_f16(rng, (2, 50, d))
    vc, vsc = oracle.quantize_rows(rows_v)
    vdq = oracle.dequantize_rows(vc, vsc)
    # identical keys -> uniform weights -> mean of V
    k_row = randn_f16(rng, (1, 1, d))
    kc, ksc = oracle.quantize_rows(np.repeat(np.repeat(k_row, 50, 1), 2, 0))
    q = randn_f16(rng, (4, d)).astype(np.float32)
    out = oracle.attention_q8(q, kc, ksc, vc, vsc, 50, 4, 0.1)
    np.testing.assert_allclose(out[0], vdq[0].mean(0), atol=1e-5)
    np.testing.assert_allclose(out[3], vdq[1].mean(0), atol=1e-5)
    # length 1 -> the single V row, exactly
    out1 = oracle.attention_q8(q, kc, ksc, vc, vsc, 1, 4, 0.1)
    assert np.array_equal(out1[0], vdq[0, 0]) and np.array_equal(out1[2], vdq[1, 0])
    # gate multiplies by sigmoid
    g = rng.standard_normal((4, d)).astype(np.float32)
    outg = oracle.attention_q8(q, kc, ksc, vc, vsc, 50, 4, 0.1, gate=g)
    np.testing.assert_allclose(outg, out / (1 + np.exp(-g)), rtol=1e-6, atol=1e-7)


def test_suffix_attention_equals_per_token_decode():
    rng = np.random.default_rng(6)
    hq, hk, d, base, t = 6, 1, 256, 40, 9
    kc, ksc = oracle.quantize_rows(randn_f16(rng, (hk, base + t, d)))
    vc, vsc = oracle.quantize_rows(randn_f16(rng, (hk, base + t, d)))
    q = randn_f16(rng, (t, hq, d)).astype(np.float32)
    out = oracle.suffix_attention_q8(q, kc, ksc, vc, vsc, base, hq, 0.0625)
    for i in range(t):
        ref = oracle.attention_q8(q[i], kc, ksc, vc, vsc, base + i + 1, hq, 0.0625)
        assert np.array_equal(out[i], ref)
    # causality: changing a later row does not change earlier tokens
    kc2 = kc.copy()
    kc2[:, base + t - 1] = -kc2[:, base + t - 1]
    out2 = oracle.suffix_attention_q8(q, kc2, ksc, vc, vsc, base, hq, 0.0625)
    assert np.array_equal(out2[:-1], out[:-1]) and not np.array_equal(out2[-1], out[-1])


# ---- FNV-1a ----------------------------------------------------------------

def test_token_hash_published_vectors():
    # Published FNV-1a 64 test vectors; one byte per token widens identically.
    assert oracle.token_hash([]) == 0xCBF29CE484222325
    assert oracle.token_hash([ord("a")]) == 0xAF63DC4C8601EC8C
    assert oracle.token_hash([ord(c) for c in "foobar"]) == 0x85944171F73967E8


# ---- fused store prologue (RMSNorm * weight, RoPE on dims 0..63) -------------

def test_k_norm_rope_at_position_zero_is_rmsnorm():
    """Angle 0 leaves the pairs unrotated: the output is the float64 RMSNorm."""
    rng = np.random.default_rng(31)
    x = rng.standard_normal(256).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 256).astype(np.float32)
    got = oracle.k_norm_rope(x, w, 0, 1.0e7, 1.0e-6)
    x64 = x.astype(np.float64)
    expect = x64 / np.sqrt((x64 * x64).mean() + 1.0e-6) * w
    assert np.max(np.abs(got - expect)) < 2e-6


@pytest.mark.parametrize("d,pos,theta", [(256, 7, 1.0e7), (128, 1000, 1.0e4), (256, 65535, 1.0e6)])
def test_k_norm_rope_rotates_pairs_by_position_angles(d, pos, theta):
    """Pair i is rotated by its angle (cos/sin in float64), with the sign pattern of
    a rotation; pair norms are kept, and dims >= 64 are only normalised.  The angles
    follow the reference's convention of accumulating pos * s^i with s =
    theta^(-2/64) by repeated fp32 multiplication (qwen3_primitives.hip:636-648);
    they stay within 2^-20 relative of pos * theta^(-2i/64)."""
    rng = np.random.default_rng(pos)
    x = rng.standard_normal(d).astype(np.float32)
    w = np.ones(d, np.float32)
    got = oracle.k_norm_rope(x, w, pos, theta, 1.0e-6).astype(np.float64)
    n = oracle.k_norm_rope(x, w, 0, theta, 1.0e-6).astype(np.float64)
    step = np.float32(theta) ** np.float32(-2.0 / 64.0)
    ang = np.empty(32)
    a = np.float32(pos)
    for i in range(32):
        ang[i] = float(a)
        a = np.float32(a * step)
    ideal = pos * np.power(float(theta), -2.0 * np.arange(32) / 64.0)
    assert np.all(np.abs(ang - ideal) <= 2.0 ** -17 * np.maximum(ideal, 1.0))
    c, s = np.cos(ang), np.sin(ang)
    exp0 = n[:32] * c - n[32:64] * s
    exp1 = n[:32] * s + n[32:64] * c
    assert np.max(np.abs(got[:32] - exp0)) < 2e-5
    assert np.max(np.abs(got[32:64] - exp1)) < 2e-5
    assert np.allclose(got[:32] ** 2 + got[32:64] ** 2, n[:32] ** 2 + n[32:64] ** 2, rtol=1e-5, atol=1e-6)
    assert np.array_equal(got[64:], n[64:])


# ---- Q8_1 output blocks -------------------------------------------------------

def test_q8_1_block_closed_forms():
    rng = np.random.default_rng(32)
    x = rng.standard_normal(32).astype(np.float32)
    blk = oracle.q8_1_blocks(x)[0]
    d = blk[0:2].view(np.float16)[0]
    s = blk[2:4].view(np.float16)[0]
    q = blk[4:].view(np.int8).astype(np.int64)
    amax = np.abs(x).max()
    assert d == np.float16(amax / np.float32(127))
    assert abs(q[np.argmax(np.abs(x))]) == 127
    assert s == np.float16(np.float32(q.sum()) * (amax / np.float32(127)))
    # |x - q d| <= d/2 for every element (d in fp32)
    assert np.all(np.abs(x - q * (amax / 127.0)) <= amax / 127.0 / 2 + 1e-6)


def test_q8_1_rounds_half_away_and_zero_block():
    # x * (1/d) lands on .5 for these values: roundf goes away from zero (q8_0 goes to even)
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1], x[2], x[3], x[4] = 2.5, -2.5, 0.5, -1.5
    q = oracle.q8_1_blocks(x)[0][4:].view(np.int8)
    assert list(q[:5]) == [127, 3, -3, 1, -2]
    z = oracle.q8_1_blocks(np.zeros(32, np.float32))[0]
    assert not z.any()  # d = 0, inverse 0, all codes 0, s = 0


@pytest.mark.parametrize("d", [128, 256])
def test_k_norm_sum_of_squares_follows_the_reference_tree(d):
    """At position 0 the prologue is RMSNorm * weight; its sum of squares is reduced in
    the reference's LDS tree order (p[t] += p[t + stride], stride = D/2 .. 1,
    qwen3_primitives.hip:7257-7263), then value * (1 / sqrt(ss / D + eps)) * weight.
    Restated here with numpy float32 vector ops; a sequential sum differs in the last
    bits for some rows, which this catches."""
    rng = np.random.default_rng(d)
    seq_differs = 0
    for _ in range(50):
        x = (rng.standard_normal(d) * 3).astype(np.float32)
        w = rng.uniform(0.5, 1.5, d).astype(np.float32)
        p = x * x
        s = d // 2
        while s > 0:
            p[:s] = p[:s] + p[s:2 * s]
            s //= 2
        r = np.float32(1.0) / np.sqrt(p[0] / np.float32(d) + np.float32(1e-6))
        expect = (x * r) * w
        got = oracle.k_norm_rope(x, w, 0, 1.0e6, 1.0e-6)
        assert np.array_equal(got.view(np.uint32), expect.view(np.uint32))
        seq = np.float32(0)
        for v in x * x:
            seq = np.float32(seq + v)
        seq_differs += int(seq != p[0])
    assert seq_differs > 0  # the order is observable at this size


def test_rope_sincos_close_to_float64():
    """The prologue's sin/cos pair against float64 sin and cos of the same float32 angle,
    over the RoPE angle range (positions up to 131072 times step^i <= 1) and around multiples of
    pi/2, where the reduction matters: within 2.5 float32 ulps where |value| >= 1/16 and
    within 1e-7 absolute everywhere (libm's sinf/cosf are within half an ulp; a wrong
    quadrant, sign, reduction constant or polynomial coefficient is off by far more)."""
    rng = np.random.default_rng(7)
    angles = np.concatenate([
        rng.uniform(0, 131072, 4000), rng.uniform(0, 8, 2000),
        (np.arange(1, 83000, 83) * (np.pi / 2))[:1000] + rng.uniform(-1e-3, 1e-3, 1000),
        [0.0, 1e-8, 0.5, 1.0, 65535.0, 131071.0]]).astype(np.float32)
    worst_ulps, worst_abs = 0.0, 0.0
    for a in angles:
        s, c = oracle.rope_sincos(float(a))
        for got, exact in ((s, np.sin(np.float64(a))), (c, np.cos(np.float64(a)))):
            if abs(exact) >= 1.0 / 16:
                worst_ulps = max(worst_ulps, abs(got - exact) / float(np.spacing(np.float32(abs(exact)))))
            worst_abs = max(worst_abs, abs(got - exact))
    assert worst_ulps <= 2.5 and worst_abs <= 1e-7, (worst_ulps, worst_abs)


def test_library_rope_sincos_header_matches_the_oracle(tmp_path):
    """The kernels' rope_sincos (miinfer_amd/csrc/miikv_rope.h, included by every kernel
    that rotates keys) compiled for the host gives the oracle's bits at RoPE angles up
    to the largest supported position (131072) and around multiples of pi/2, so the
    device code and the oracle cannot drift apart unnoticed."""
    import ctypes
    import shutil
    import subprocess
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("no host C++ compiler")
    src = tmp_path / "rope_pin.cpp"
    src.write_text('#include "miikv_rope.h"\n'
                   'extern "C" void pin_rope(float a, float* s, float* c) { miikv::rope_sincos(a, s, c); }\n')
    so = tmp_path / "librope_pin.so"
    csrc = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "miinfer_amd", "csrc")
    subprocess.run([cxx, "-O2", "-ffp-contract=off", "-Wno-unknown-pragmas", "-shared", "-fPIC",
                    "-I", csrc, str(src), "-o", str(so)], check=True)
    lib = ctypes.CDLL(str(so))
    lib.pin_rope.argtypes = [ctypes.c_float, ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_float)]
    rng = np.random.default_rng(11)
    angles = np.concatenate([
        rng.uniform(0, 131072, 3000), rng.uniform(0, 8, 500),
        (np.arange(1, 83000, 83) * (np.pi / 2)) + rng.uniform(-1e-3, 1e-3, 1000),
        [0.0, 1e-8, 65535.0, 65536.0, 131071.0]]).astype(np.float32)
    s, c = ctypes.c_float(), ctypes.c_float()
    for a in angles:
        lib.pin_rope(float(a), ctypes.byref(s), ctypes.byref(c))
        es, ec = oracle.rope_sincos(float(a))
        assert (np.float32(s.value).view(np.uint32), np.float32(c.value).view(np.uint32)) == \
            (np.float32(es).view(np.uint32), np.float32(ec).view(np.uint32)), float(a)
