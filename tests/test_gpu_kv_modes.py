"""The four KV quant modes of KvCacheQuantMode (include/miinfer/prefill_v2/kv_cache.hpp:16-21)
on the GPU: FP16_FP16 (the reference's production default and the A/B control of its Q8
numbers), Q8_FP16, FP16_Q8 and Q8_Q8.  fp16 planes store the rows bit for bit, q8 planes
the oracle's codes; decode and suffix attention in every mode against the fp32 oracle over
the stored values; and the reference's own acceptance rule for the quantized modes against
FP16_FP16 (tests/qwen3_quant_kv_attention_test.cpp:255-281: cosine >= 0.999 for every Q8
mode, MAE <= 0.05 for Q8_Q8) on its shapes and N(0, 0.5) inputs."""
import math

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import assert_attention_close, randn_f16

pytestmark = pytest.mark.gpu

MODES = {"fp16_fp16": 0, "q8_fp16": 1, "fp16_q8": 2, "q8_q8": 3}


def _dev(a, gpu):
    return torch.from_numpy(np.ascontiguousarray(a)).to(gpu)


def _stored(x16, f16):
    """The values a plane holds for fp16 rows x16 [L, H, D]: the rows themselves (fp16
    plane) or the dequantised q8_0 codes, as [H, L, D] fp32."""
    xt = x16.transpose(1, 0, 2)
    if f16:
        return xt.astype(np.float32)
    c, s = oracle.quantize_rows(xt)
    return oracle.dequantize_rows(c, s)


def _flags(mode):
    return mode in (0, 2), mode in (0, 1)  # (k fp16, v fp16)


@pytest.mark.parametrize("mode", list(MODES))
def test_modes_store_export_raw(gpu, mode):
    import miinfer_amd as m
    md = MODES[mode]
    kf, vf = _flags(md)
    rng = np.random.default_rng(md)
    hk, d, n = 4, 256, 300
    cache = m.KvCache.contiguous(hk, d, 512, quant_mode=md)
    k = randn_f16(rng, (n, hk, d))
    v = randn_f16(rng, (n, hk, d))
    cache.append(_dev(k[:200], gpu), _dev(v[:200], gpu))
    cache.append(_dev(k[200:], gpu), _dev(v[200:], gpu), base_position=200)
    kc, ks, vc, vs = [None if t is None else t.cpu().numpy() for t in cache.export_canonical(0, 0, n)]
    for codes, scales, x, f16 in ((kc, ks, k, kf), (vc, vs, v, vf)):
        if f16:
            assert scales is None and codes.dtype == np.float16
            assert np.array_equal(codes.view(np.uint16), x.transpose(1, 0, 2).view(np.uint16))
        else:
            ec, es = oracle.quantize_rows(x.transpose(1, 0, 2))
            assert np.array_equal(codes, ec) and np.array_equal(scales.view(np.uint16), es)
    assert np.array_equal(cache.download_key(n), _stored(k, kf))
    assert np.array_equal(cache.download_value(n), _stored(v, vf))
    raw = cache.download_raw(n)
    assert len(raw) == cache.raw_tokens_bytes(n)
    other = m.KvCache.contiguous(hk, d, 512, quant_mode=md)
    other.upload_raw(raw, n)
    assert other.download_raw(n) == raw


@pytest.mark.parametrize("mode", list(MODES))
@pytest.mark.parametrize("hq,hk,d", [(32, 8, 128), (24, 4, 256)])
@pytest.mark.parametrize("length", [1, 33, 1000, 4097])
def test_modes_decode(gpu, mode, hq, hk, d, length):
    import miinfer_amd as m
    md = MODES[mode]
    kf, vf = _flags(md)
    rng = np.random.default_rng(length + md + d)
    cap = 4224
    cache = m.KvCache.contiguous(hk, d, cap, quant_mode=md)
    # older bytes past the context (a previous, longer sequence) must not leak in; fp16
    # planes get infinities there (p = 0 would not cancel them)
    junk = (randn_f16(rng, (cap, hk, d)) * np.float16(300)).astype(np.float16)
    if kf and vf:
        junk[:] = np.float16(np.inf)
    cache.append(_dev(junk, gpu), _dev(junk, gpu))
    k = randn_f16(rng, (length, hk, d))
    v = randn_f16(rng, (length, hk, d))
    cache.append(_dev(k, gpu), _dev(v, gpu))
    for qdt in (np.float16, np.float32):
        q = rng.standard_normal((1, hq, d)).astype(qdt)
        out, _ = m.decode_attention(cache, _dev(q, gpu), lengths=torch.tensor([length], dtype=torch.int32,
                                                                             device=gpu), max_context=cap)
        expect = oracle.attention_f32(q[0].astype(np.float32), _stored(k, kf), _stored(v, vf), length, hq, hk, d,
                                      1 / math.sqrt(d))
        assert_attention_close(out.cpu().numpy()[0], expect, f"{mode} L={length} q={qdt.__name__}")


@pytest.mark.parametrize("mode", ["fp16_fp16", "q8_fp16"])
def test_modes_decode_paged_batched(gpu, mode):
    import miinfer_amd as m
    md = MODES[mode]
    kf, vf = _flags(md)
    rng = np.random.default_rng(7 + md)
    hq, hk, d, pt = 24, 4, 256, 256
    lens = [1, 300, 5000, 257]
    pages = [(n + pt - 1) // pt for n in lens]
    stride, total = max(pages), sum(pages)
    perm = rng.permutation(total).astype(np.int32)
    table = np.zeros((len(lens), stride), np.int32)
    o = 0
    for s_, p_ in enumerate(pages):
        table[s_, :p_] = perm[o:o + p_]
        o += p_
    cache = m.KvCache.paged_cache(hk, d, total, _dev(table, gpu), page_tokens=pt, quant_mode=md)
    data = []
    for s_, n in enumerate(lens):
        k = randn_f16(rng, (n, hk, d))
        v = randn_f16(rng, (n, hk, d))
        cache.append(_dev(k, gpu), _dev(v, gpu), base_position=0, seq=s_)
        data.append((k, v))
    q = randn_f16(rng, (len(lens), hq, d))
    out, _ = m.decode_attention(cache, _dev(q, gpu), lengths=_dev(np.array(lens, np.int32), gpu),
                                max_context=stride * pt)
    out = out.cpu().numpy()
    for s_, n in enumerate(lens):
        k, v = data[s_]
        expect = oracle.attention_f32(q[s_].astype(np.float32), _stored(k, kf), _stored(v, vf), n, hq, hk, d,
                                      1 / math.sqrt(d))
        assert_attention_close(out[s_], expect, f"{mode} seq {s_}")


@pytest.mark.parametrize("mode", list(MODES))
def test_modes_suffix(gpu, mode):
    import miinfer_amd as m
    md = MODES[mode]
    kf, vf = _flags(md)
    rng = np.random.default_rng(40 + md)
    hq, hk, d, prefix, t = 24, 4, 256, 700, 64
    cache = m.KvCache.contiguous(hk, d, 1024, quant_mode=md)
    k = randn_f16(rng, (prefix + t, hk, d))
    v = randn_f16(rng, (prefix + t, hk, d))
    cache.append(_dev(k, gpu), _dev(v, gpu))
    q = randn_f16(rng, (t, hq, d))
    out, _ = m.suffix_attention(cache, _dev(q, gpu), prefix)
    out = out.cpu().numpy()
    ks, vs = _stored(k, kf), _stored(v, vf)
    for j in (0, 1, 31, 63):
        expect = oracle.attention_f32(q[j].astype(np.float32), ks, vs, prefix + j + 1, hq, hk, d, 1 / math.sqrt(d))
        assert_attention_close(out[j], expect, f"{mode} token {j}")
    if md != 3:  # the fused store writes q8 rows only
        with pytest.raises(m.MiikvError):
            m.suffix_attention(cache, _dev(q, gpu), prefix, k_new=_dev(k[prefix:], gpu), v_new=_dev(v[prefix:], gpu))


def _metrics(ref, test):
    ref = ref.astype(np.float64).ravel()
    test = test.astype(np.float64).ravel()
    diff = np.abs(ref - test)
    cos = float(ref @ test / (np.linalg.norm(ref) * np.linalg.norm(test) + 1e-12))
    return float(diff.max()), float(diff.mean()), cos


@pytest.mark.parametrize("prefix,suffix", [(64, 16), (512, 64), (4096, 128), (16384, 512)])
def test_quantized_modes_acceptance_rule(gpu, prefix, suffix):
    """The reference's qualification of the Q8 modes against FP16_FP16 on suffix attention
    (24q/4kv/D256, scale 1/16, q/gate/K/V N(0, 0.5), gated output): cosine >= 0.999 for
    Q8_FP16, FP16_Q8 and Q8_Q8, MAE <= 0.05 for Q8_Q8
    (tests/qwen3_quant_kv_attention_test.cpp:182-281)."""
    import miinfer_amd as m
    rng = np.random.default_rng(42)
    hq, hk, d = 24, 4, 256
    total = prefix + suffix
    cap = (total + 128 + 63) // 64 * 64  # the reference sizes total + 128; pages are multiples of 64
    k = (rng.standard_normal((total, hk, d)) * 0.5).astype(np.float32).astype(np.float16)
    v = (rng.standard_normal((total, hk, d)) * 0.5).astype(np.float32).astype(np.float16)
    q = (rng.standard_normal((suffix, hq, d)) * 0.5).astype(np.float32)
    gate = (rng.standard_normal((suffix, hq, d)) * 0.5).astype(np.float32)
    outs = {}
    for mode, md in MODES.items():
        cache = m.KvCache.contiguous(hk, d, cap, quant_mode=md)
        cache.append(_dev(k, gpu), _dev(v, gpu))
        _, g = m.suffix_attention(cache, _dev(q, gpu), prefix, 1.0 / 16.0, gate=_dev(gate, gpu))
        outs[mode] = g.cpu().numpy()
    ref = outs["fp16_fp16"]
    for mode in ("q8_fp16", "fp16_q8", "q8_q8"):
        mx, mae, cos = _metrics(ref, outs[mode])
        print(f"prefix={prefix} suffix={suffix} {mode}: max_abs={mx:.6f} mae={mae:.6f} cos={cos:.8f}")
        assert cos >= 0.999, (mode, cos)
        if mode == "q8_q8":
            assert mae <= 0.05, mae
