"""Fused append + decode (one launch pair): the new row lands in the cache with
the same bytes as miikv_append_f16, and attention covers it (oracle
tolerance, tests/helpers.py)."""
import math

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import assert_attention_close, randn_f16

pytestmark = pytest.mark.gpu


def _dev(a, gpu):
    return torch.from_numpy(np.ascontiguousarray(a)).to(gpu)


def _canon(cache, seq, n):
    out = cache.export_canonical(seq, 0, n)
    torch.cuda.synchronize()
    return [t.cpu().numpy() for t in out]


@pytest.mark.parametrize("hq,hk,d", [(32, 8, 128), (24, 4, 256)])
@pytest.mark.parametrize("length", [1, 2, 32, 33, 64, 65, 127, 128, 129, 1000, 4097])
def test_fused_append_decode_contiguous(gpu, hq, hk, d, length):
    import miinfer_amd as m
    rng = np.random.default_rng(length * 7 + d)
    cap = ((length + 127) // 128) * 128
    fused = m.KvCache.contiguous(hk, d, cap)
    plain = m.KvCache.contiguous(hk, d, cap)
    k = randn_f16(rng, (length, hk, d))
    v = randn_f16(rng, (length, hk, d))
    k.reshape(-1, 32)[-1] = 0.0  # a zero block in the new row
    # the slot of the new token holds older bytes (a previous sequence) in `fused`
    junk = randn_f16(rng, (length, hk, d)) * np.float16(50)
    fused.append(_dev(junk, gpu), _dev(junk, gpu))
    if length > 1:
        fused.append(_dev(k[:-1], gpu), _dev(v[:-1], gpu))
    plain.append(_dev(k, gpu), _dev(v, gpu))
    q = randn_f16(rng, (1, hq, d))
    gate = rng.standard_normal((1, hq, d)).astype(np.float32)
    lengths = torch.tensor([length], dtype=torch.int32, device=gpu)
    out, gated = m.decode_attention(fused, _dev(q, gpu), lengths=lengths, max_context=cap,
                                    gate=_dev(gate, gpu), out=torch.empty((1, hq, d), device=gpu),
                                    k_new=_dev(k[-1:], gpu), v_new=_dev(v[-1:], gpu))
    torch.cuda.synchronize()
    for a, b in zip(_canon(fused, 0, length), _canon(plain, 0, length)):
        assert np.array_equal(a, b)
    kc, ks = oracle.quantize_rows(k.transpose(1, 0, 2))
    vc, vs = oracle.quantize_rows(v.transpose(1, 0, 2))
    expect = oracle.attention_q8(q[0].astype(np.float32), kc, ks, vc, vs, length, hq, 1 / math.sqrt(d))
    assert_attention_close(out.cpu().numpy()[0], expect, f"L={length}")
    assert_attention_close(gated.cpu().numpy()[0], expect / (1 + np.exp(-gate[0])), "gated")


def test_fused_append_decode_state_and_fp32_query(gpu):
    import miinfer_amd as m
    rng = np.random.default_rng(3)
    hq, hk, d, length = 32, 8, 128, 777
    cache = m.KvCache.contiguous(hk, d, 1024)
    k = randn_f16(rng, (length, hk, d))
    v = randn_f16(rng, (length, hk, d))
    cache.append(_dev(k[:-1], gpu), _dev(v[:-1], gpu))
    q = rng.standard_normal((1, hq, d)).astype(np.float32)
    ds = m.make_decode_state(length - 1, device=gpu)
    out, _ = m.decode_attention(cache, _dev(q, gpu), decode_state=ds, max_context=1024,
                                k_new=_dev(k[-1:], gpu), v_new=_dev(v[-1:], gpu))
    torch.cuda.synchronize()
    kc, ks = oracle.quantize_rows(k.transpose(1, 0, 2))
    vc, vs = oracle.quantize_rows(v.transpose(1, 0, 2))
    expect = oracle.attention_q8(q[0], kc, ks, vc, vs, length, hq, 1 / math.sqrt(d))
    assert_attention_close(out.cpu().numpy()[0], expect, "fp32 q, decode state")


@pytest.mark.parametrize("hq,hk,d", [(24, 4, 256), (32, 8, 128)])
def test_fused_append_decode_paged_batched(gpu, hq, hk, d):
    import miinfer_amd as m
    rng = np.random.default_rng(hq * d)
    pt = 256
    lens = [1, 256, 257, 512, 3000, 1100]   # lengths include the new token
    pages = [(n + pt - 1) // pt for n in lens]
    stride = max(pages)
    total = sum(pages)
    perm = rng.permutation(total).astype(np.int32)
    table = np.zeros((len(lens), stride), np.int32)
    o = 0
    for s, p in enumerate(pages):
        table[s, :p] = perm[o:o + p]
        o += p
    cache = m.KvCache.paged_cache(hk, d, total, _dev(table, gpu), page_tokens=pt)
    refs, knew, vnew = [], [], []
    for s, n in enumerate(lens):
        k = randn_f16(rng, (n, hk, d))
        v = randn_f16(rng, (n, hk, d))
        if n > 1:
            cache.append(_dev(k[:-1], gpu), _dev(v[:-1], gpu), base_position=0, seq=s)
        knew.append(k[-1])
        vnew.append(v[-1])
        kc, ks = oracle.quantize_rows(k.transpose(1, 0, 2))
        vc, vs = oracle.quantize_rows(v.transpose(1, 0, 2))
        refs.append((kc, ks, vc, vs))
    q = randn_f16(rng, (len(lens), hq, d))
    out, _ = m.decode_attention(cache, _dev(q, gpu), lengths=_dev(np.array(lens, np.int32), gpu),
                                max_context=stride * pt, k_new=_dev(np.stack(knew), gpu),
                                v_new=_dev(np.stack(vnew), gpu))
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    for s, n in enumerate(lens):
        expect = oracle.attention_q8(q[s].astype(np.float32), *refs[s], n, hq, 1 / math.sqrt(d))
        assert_attention_close(out[s], expect, f"seq {s} L={n}")
        kc, ks, vc, vs = _canon(cache, s, n)
        assert np.array_equal(kc[:, n - 1], refs[s][0][:, n - 1])
        assert np.array_equal(ks[:, n - 1].view(np.uint16), refs[s][1][:, n - 1])
        assert np.array_equal(vc[:, n - 1], refs[s][2][:, n - 1])
        assert np.array_equal(vs[:, n - 1].view(np.uint16), refs[s][3][:, n - 1])


def test_fused_append_q8_1_epilogue_and_empty_sequence(gpu):
    """Fused append with the Q8_1 output blocks of the gated output, in a batch whose
    middle sequence is empty (L = 0): its outputs are zeros and no row is stored."""
    import miinfer_amd as m
    rng = np.random.default_rng(11)
    hq, hk, d, pt = 24, 4, 256, 256
    lens = [700, 0, 300]
    table = np.array([[0, 1, 2], [3, 4, 5], [6, 7, 8]], np.int32)
    cache = m.KvCache.paged_cache(hk, d, 9, _dev(table, gpu), page_tokens=pt)
    before = _canon(cache, 1, 1)
    refs, knew, vnew = [], [], []
    for s, n in enumerate(lens):
        k = randn_f16(rng, (max(n, 1), hk, d))
        v = randn_f16(rng, (max(n, 1), hk, d))
        if n > 1:
            cache.append(_dev(k[:-1], gpu), _dev(v[:-1], gpu), base_position=0, seq=s)
        knew.append(k[-1])
        vnew.append(v[-1])
        kc, ks = oracle.quantize_rows(k.transpose(1, 0, 2))
        vc, vs = oracle.quantize_rows(v.transpose(1, 0, 2))
        refs.append((kc, ks, vc, vs))
    q = randn_f16(rng, (len(lens), hq, d))
    gate = rng.standard_normal((len(lens), hq, d)).astype(np.float32)
    blocks = torch.zeros((len(lens) * hq * d // 32, 36), dtype=torch.uint8, device=gpu)
    out, gated = m.decode_attention(cache, _dev(q, gpu), lengths=_dev(np.array(lens, np.int32), gpu),
                                    max_context=3 * pt, gate=_dev(gate, gpu),
                                    out=torch.empty((len(lens), hq, d), device=gpu), gated_q8_1=blocks,
                                    k_new=_dev(np.stack(knew), gpu), v_new=_dev(np.stack(vnew), gpu))
    torch.cuda.synchronize()
    out, gated = out.cpu().numpy(), gated.cpu().numpy()
    for s, n in enumerate(lens):
        if n == 0:
            assert not out[s].any() and not gated[s].any()
            continue
        expect = oracle.attention_q8(q[s].astype(np.float32), *refs[s], n, hq, 1 / math.sqrt(d))
        assert_attention_close(out[s], expect, f"seq {s} L={n}")
    # Q8_1 blocks are the reference rule applied to the kernel's own gated output
    assert np.array_equal(blocks.cpu().numpy(), oracle.q8_1_blocks(gated.reshape(-1)))
    # the empty sequence's first slot keeps its bytes
    for a, b in zip(_canon(cache, 1, 1), before):
        assert np.array_equal(a, b)


@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("length", [1, 8193, 16384])
def test_decode_c2_16k_plan(gpu, fused, length):
    """Config 2 at its middle context: a 16384-token cache with max_context 16384 runs
    the plan the bench times there (two 32-token steps per wave, waves not interleaved)."""
    import miinfer_amd as m
    rng = np.random.default_rng(length + 16)
    hq, hk, d, cap = 32, 8, 128, 16384
    cache = m.KvCache.contiguous(hk, d, cap)
    k = randn_f16(rng, (length, hk, d))
    v = randn_f16(rng, (length, hk, d))
    n_cached = length - 1 if fused else length
    for t0 in range(0, n_cached, 8192):
        n = min(8192, n_cached - t0)
        cache.append(_dev(k[t0:t0 + n], gpu), _dev(v[t0:t0 + n], gpu), base_position=t0)
    q = randn_f16(rng, (1, hq, d))
    lens = torch.tensor([length], dtype=torch.int32, device=gpu)
    extra = dict(k_new=_dev(k[-1:], gpu), v_new=_dev(v[-1:], gpu)) if fused else {}
    out, _ = m.decode_attention(cache, _dev(q, gpu), lengths=lens, max_context=cap, **extra)
    torch.cuda.synchronize()
    kc, ks = oracle.quantize_rows(k.transpose(1, 0, 2))
    vc, vs = oracle.quantize_rows(v.transpose(1, 0, 2))
    if fused:
        got = _canon(cache, 0, length)
        assert np.array_equal(got[0][:, -1], kc[:, -1]) and np.array_equal(got[2][:, -1], vc[:, -1])
        assert np.array_equal(got[1][:, -1].view(np.uint16), ks[:, -1])
        assert np.array_equal(got[3][:, -1].view(np.uint16), vs[:, -1])
    expect = oracle.attention_q8(q[0].astype(np.float32), kc, ks, vc, vs, length, hq, 1 / math.sqrt(d))
    assert_attention_close(out.cpu().numpy()[0], expect, f"L={length} fused={fused}")


@pytest.mark.parametrize("hq,hk,d,length,theta", [(32, 8, 128, 32768, 1.0e6), (24, 4, 256, 1000, 1.0e7),
                                                  (24, 4, 256, 1, 1.0e7), (32, 8, 128, 33, 1.0e4)])
def test_decode_append_attn_f32_reference_step(gpu, hq, hk, d, length, theta):
    """miikv_decode_append_attn_f32: the reference's store arguments (fp32 rows, K-norm
    weight, theta, eps) fused into the decode launch pair.  The new row's bytes equal
    miikv_append_f32 with the same arguments (and so the oracle's prologue + q8 rule), and
    attention (fp32 query, gate, Q8_1 epilogue) matches the oracle."""
    import ctypes

    import miinfer_amd as m
    from miinfer_amd import _lib
    rng = np.random.default_rng(length + d)
    cap = max(64, (length + 63) // 64 * 64)
    fused = m.KvCache.contiguous(hk, d, cap)
    plain = m.KvCache.contiguous(hk, d, cap)
    k = randn_f16(rng, (length, hk, d))
    v = randn_f16(rng, (length, hk, d))
    for c in (fused, plain):
        if length > 1:
            for t0 in range(0, length - 1, 8192):
                n = min(8192, length - 1 - t0)
                c.append(_dev(k[t0:t0 + n], gpu), _dev(v[t0:t0 + n], gpu), base_position=t0)
    k32 = (rng.standard_normal((1, hk, d)) * 3).astype(np.float32)
    v32 = rng.standard_normal((1, hk, d)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, d).astype(np.float32)
    eps = 1.0e-6
    plain.append_f32(_dev(k32, gpu), _dev(v32, gpu), base_position=length - 1, k_norm_weight=_dev(w, gpu),
                     theta=theta, epsilon=eps)
    q = rng.standard_normal((1, hq, d)).astype(np.float32)
    gate = rng.standard_normal((1, hq, d)).astype(np.float32)
    ds = m.make_decode_state(length - 1, device=gpu)
    ws = m.DecodeWorkspace(fused, hq, 1, cap)
    out = torch.empty((1, hq, d), device=gpu)
    gated = torch.empty((1, hq, d), device=gpu)
    q81 = torch.zeros(hq * d // 32 * 36, dtype=torch.uint8, device=gpu)
    P = ctypes.c_void_p
    dk, dv, dw, dq, dg = (_dev(x, gpu) for x in (k32, v32, w, q, gate))
    st = _lib.lib().miikv_decode_append_attn_f32(
        fused.view, P(dk.data_ptr()), P(dv.data_ptr()), P(dw.data_ptr()), ctypes.c_float(theta),
        ctypes.c_float(eps), P(dq.data_ptr()), _lib.DTYPE_F32, hq, ctypes.c_float(1 / math.sqrt(d)), 1, None,
        P(ds.data_ptr()), cap, P(out.data_ptr()), P(dg.data_ptr()), P(gated.data_ptr()), P(q81.data_ptr()),
        P(ws.buf.data_ptr()), ws.bytes, P(torch.cuda.current_stream().cuda_stream))
    assert st == 0, st
    torch.cuda.synchronize()
    a, b = _canon(fused, 0, length), _canon(plain, 0, length)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)
    kn = oracle.k_norm_rope(k32[0, :, :].reshape(hk, d)[0], w, length - 1, theta, eps)  # one head spot check
    kc1, _ = oracle.quantize_rows_f32(kn[None, None])
    assert np.array_equal(a[0][0, length - 1], kc1[0, 0])
    kc, ks, vc, vs = b
    expect = oracle.attention_q8(q[0], kc, ks.view(np.uint16), vc, vs.view(np.uint16), length, hq, 1 / math.sqrt(d))
    assert_attention_close(out.cpu().numpy()[0], expect, f"L={length}")
    assert_attention_close(gated.cpu().numpy()[0], expect / (1 + np.exp(-gate[0])), "gated")
