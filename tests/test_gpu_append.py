"""q8_0 append: codes and scales bit-exact against the CPU oracle (GPU)."""
import numpy as np
import pytest
import torch

import oracle
from tests.helpers import randn_f16

pytestmark = pytest.mark.gpu


def _dev(a, gpu):
    return torch.from_numpy(np.ascontiguousarray(a)).to(gpu)


def _export_np(cache, seq, t0, count):
    kc, ks, vc, vs = cache.export_canonical(seq, t0, count)
    torch.cuda.synchronize()
    return (kc.cpu().numpy(), ks.cpu().numpy().view(np.uint16), vc.cpu().numpy(),
            vs.cpu().numpy().view(np.uint16))


def _edge_rows(rng, t, hk, d):
    """fp16 rows with the cases the rule must get exactly right."""
    rows = randn_f16(rng, (t, hk, d))
    flat = rows.reshape(-1, 32)
    flat[0] = 0.0                                            # zero block -> scale 1.0h
    flat[1] = np.float16(-0.0)
    flat[2, :] = np.arange(32, dtype=np.float16) - 15.5      # ties after scaling
    flat[2, 0] = 127.0
    flat[3, :] = np.float16(6.0e-8)                          # subnormal halves
    flat[4, :] = np.float16(60000.0)                         # near fp16 max
    flat[4, 1::2] = np.float16(-60000.0)
    flat[5, :] = rng.standard_normal(32).astype(np.float16) * np.float16(1e-3)
    return rows


@pytest.mark.parametrize("hk,d", [(8, 128), (4, 256)])
def test_append_contiguous_bitexact(gpu, hk, d):
    import miinfer_amd as m
    rng = np.random.default_rng(100 + d)
    cap, t = 512, 300
    cache = m.KvCache.contiguous(hk, d, cap)
    k = _edge_rows(rng, t, hk, d)
    v = randn_f16(rng, (t, hk, d))
    # a bulk append followed by single-row appends (the decode pattern)
    cache.append(_dev(k[:200], gpu), _dev(v[:200], gpu), base_position=0)
    for i in range(200, t):
        cache.append(_dev(k[i:i + 1], gpu), _dev(v[i:i + 1], gpu), base_position=i)
    kc, ks, vc, vs = _export_np(cache, 0, 0, t)
    ekc, eks = oracle.quantize_rows(k.transpose(1, 0, 2))
    evc, evs = oracle.quantize_rows(v.transpose(1, 0, 2))
    assert np.array_equal(kc, ekc) and np.array_equal(ks, eks)
    assert np.array_equal(vc, evc) and np.array_equal(vs, evs)


def test_append_device_state_variants(gpu):
    import miinfer_amd as m
    rng = np.random.default_rng(7)
    hk, d = 8, 128
    cache = m.KvCache.contiguous(hk, d, 256)
    k = randn_f16(rng, (70, hk, d))
    v = randn_f16(rng, (70, hk, d))
    # prefill state: device base 0, device count 64 (host bound 70 -> only 64 stored)
    ps = m.make_prefill_state(0, 64, 256, device=gpu)
    cache.append(_dev(k, gpu), _dev(v, gpu), prefill_state=ps)
    # decode state: one row at device position 64
    ds = m.make_decode_state(64, device=gpu)
    cache.append(_dev(k[64:65], gpu), _dev(v[64:65], gpu), decode_state=ds)
    kc, ks, vc, vs = _export_np(cache, 0, 0, 66)
    ekc, eks = oracle.quantize_rows(k[:65].transpose(1, 0, 2))
    assert np.array_equal(kc[:, :65], ekc) and np.array_equal(ks[:, :65], eks)
    # position 65 was never written: still zero from construction
    assert not kc[:, 65].any() and not ks[:, 65].any()


def test_append_paged_and_batch(gpu):
    import miinfer_amd as m
    rng = np.random.default_rng(9)
    hk, d, pt = 4, 256, 256
    batch, pages_per_seq = 3, 3
    perm = rng.permutation(batch * pages_per_seq).astype(np.int32).reshape(batch, pages_per_seq)
    table = _dev(perm, gpu)
    cache = m.KvCache.paged_cache(hk, d, batch * pages_per_seq, table, page_tokens=pt)
    lens = [700, 300, 513]
    rows = {}
    for s, n in enumerate(lens):
        k = randn_f16(rng, (n, hk, d))
        v = randn_f16(rng, (n, hk, d))
        rows[s] = (k, v)
        cache.append(_dev(k, gpu), _dev(v, gpu), base_position=0, seq=s)
    # one batched decode append per sequence at its current length
    kb = randn_f16(rng, (batch, hk, d))
    vb = randn_f16(rng, (batch, hk, d))
    cache.append_batch(_dev(kb, gpu), _dev(vb, gpu), _dev(np.array(lens, np.int32), gpu))
    for s, n in enumerate(lens):
        k = np.concatenate([rows[s][0], kb[s:s + 1]])
        v = np.concatenate([rows[s][1], vb[s:s + 1]])
        kc, ks, vc, vs = _export_np(cache, s, 0, n + 1)
        ekc, eks = oracle.quantize_rows(k.transpose(1, 0, 2))
        evc, evs = oracle.quantize_rows(v.transpose(1, 0, 2))
        assert np.array_equal(kc, ekc) and np.array_equal(ks, eks), s
        assert np.array_equal(vc, evc) and np.array_equal(vs, evs), s


def test_import_export_round_trip_and_raw(gpu):
    import miinfer_amd as m
    rng = np.random.default_rng(11)
    hk, d, n = 8, 128, 192
    cache = m.KvCache.contiguous(hk, d, 256)
    kc = rng.integers(-128, 128, (hk, n, d), dtype=np.int8)
    vc = rng.integers(-128, 128, (hk, n, d), dtype=np.int8)
    ks = rng.integers(0, 2**15, (hk, n, d // 32), dtype=np.int16)
    vs = rng.integers(0, 2**15, (hk, n, d // 32), dtype=np.int16)
    cache.import_canonical(0, 0, *[_dev(a, gpu) for a in (kc, ks, vc, vs)])
    got = _export_np(cache, 0, 0, n)
    assert np.array_equal(got[0], kc) and np.array_equal(got[2], vc)
    assert np.array_equal(got[1], ks.view(np.uint16)) and np.array_equal(got[3], vs.view(np.uint16))
    raw = cache.download_raw(n)
    assert len(raw) == cache.raw_tokens_bytes(n) == 2 * n * hk * (d + 2 * d // 32)
    other = m.KvCache.contiguous(hk, d, 256)
    other.upload_raw(raw, n)
    assert other.download_raw(n) == raw


def test_append_rejects_out_of_range(gpu):
    import miinfer_amd as m
    cache = m.KvCache.contiguous(8, 128, 128)
    k = torch.zeros((2, 8, 128), dtype=torch.float16, device=gpu)
    with pytest.raises(m.MiikvError):
        cache.append(k, k, base_position=127)  # 127 + 2 > capacity


@pytest.mark.parametrize("hk,d", [(8, 128), (4, 256)])
def test_append_f32_plain_bitexact(gpu, hk, d):
    """fp32 rows without the prologue: the q8_0 rule on the fp32 values, bit-exact."""
    import miinfer_amd as m
    rng = np.random.default_rng(200 + d)
    t = 130
    cache = m.KvCache.contiguous(hk, d, 192)
    k = (rng.standard_normal((t, hk, d)) * 3).astype(np.float32)
    v = rng.standard_normal((t, hk, d)).astype(np.float32)
    k.reshape(-1, 32)[0] = 0.0
    cache.append_f32(_dev(k, gpu), _dev(v, gpu), base_position=0)
    kc, ks, vc, vs = _export_np(cache, 0, 0, t)
    ek, eks = oracle.quantize_rows_f32(k.transpose(1, 0, 2))
    ev, evs = oracle.quantize_rows_f32(v.transpose(1, 0, 2))
    assert np.array_equal(kc, ek) and np.array_equal(ks, eks)
    assert np.array_equal(vc, ev) and np.array_equal(vs, evs)


@pytest.mark.parametrize("hk,d,theta,base", [(4, 256, 1.0e7, 1000), (8, 128, 1.0e4, 1000),
                                             (4, 256, 1.0e6, 60000)])
def test_append_f32_norm_rope_matches_oracle(gpu, hk, d, theta, base):
    """K gets RMSNorm * weight and RoPE at its position before quantisation, in the
    reference's order (LDS-tree sum of squares, value * r * weight, angle = position *
    step^i by repeated multiplication): K codes and scales bit-exact against the oracle
    (the square root and division are correctly rounded on both sides, the RoPE step is
    one host powf, and sin/cos use the same float arithmetic on both sides); V bit-exact."""
    import miinfer_amd as m
    rng = np.random.default_rng(300 + d + base)
    t = 70
    cache = m.KvCache.contiguous(hk, d, (base + t + 63) // 64 * 64)
    k = rng.standard_normal((t, hk, d)).astype(np.float32) * 4
    v = rng.standard_normal((t, hk, d)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, d).astype(np.float32)
    eps = 1.0e-6
    ps = m.make_prefill_state(base, t, device=gpu)
    # host base position for the first half, device state for the second
    cache.append_f32(_dev(k[:35], gpu), _dev(v[:35], gpu), base_position=base,
                     k_norm_weight=_dev(w, gpu), theta=theta, epsilon=eps)
    ps[0] = base + 35
    ps[1] = t - 35
    cache.append_f32(_dev(k[35:], gpu), _dev(v[35:], gpu), k_norm_weight=_dev(w, gpu), theta=theta,
                     epsilon=eps, prefill_state=ps)
    kc, ks, vc, vs = _export_np(cache, 0, base, t)
    kn = np.stack([[oracle.k_norm_rope(k[i, h], w, base + i, theta, eps) for h in range(hk)]
                   for i in range(t)])
    ek, eks = oracle.quantize_rows_f32(kn.transpose(1, 0, 2))
    ev, evs = oracle.quantize_rows_f32(v.transpose(1, 0, 2))
    assert np.array_equal(vc, ev) and np.array_equal(vs, evs)
    assert np.array_equal(kc, ek), int((kc != ek).sum())
    assert np.array_equal(ks, eks), int((ks != eks).sum())


@pytest.mark.parametrize("hk,d", [(8, 128), (4, 256)])
def test_append_tile_path_matches_row_path(gpu, hk, d):
    """Bulk appends send whole 32-token groups through the LDS-assembled tile kernel and
    the partial groups at either end through the per-row kernel: the bytes must equal
    the per-row kernel's alone (same arithmetic), for fp16 rows against the oracle too,
    on a contiguous cache and across page boundaries of a paged one, from unaligned
    starts."""
    import miinfer_amd as m
    rng = np.random.default_rng(400 + d)
    pt = 256
    table = _dev(np.array([[3, 0, 2]], np.int32), gpu)
    k16 = _edge_rows(rng, 400, hk, d)
    v16 = randn_f16(rng, (400, hk, d))
    k32 = rng.standard_normal((400, hk, d)).astype(np.float32) * 4
    v32 = rng.standard_normal((400, hk, d)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, d).astype(np.float32)

    def run(rows_only):
        # rows_only: chunks below the grouped store's 64-token minimum, so every row goes
        # through the per-row kernel
        step = 40 if rows_only else 400

        def put(cache, fn, k, v, base, **kw):
            for t0 in range(0, k.shape[0], step):
                fn(_dev(k[t0:t0 + step], gpu), _dev(v[t0:t0 + step], gpu), base_position=base + t0, **kw)

        out = []
        for layout in ("contiguous", "paged"):
            cache = (m.KvCache.contiguous(hk, d, 768) if layout == "contiguous"
                     else m.KvCache.paged_cache(hk, d, 4, table, page_tokens=pt))
            put(cache, cache.append, k16[:300], v16[:300], 45)
            put(cache, cache.append_f32, k32[:100], v32[:100], 345, k_norm_weight=_dev(w, gpu), theta=1.0e6,
                epsilon=1e-6)
            put(cache, cache.append_f32, k32[100:400], v32[100:400], 445)
            out.append(_export_np(cache, 0, 0, 745))
        return out

    tiled = run(False)
    rows = run(True)
    for a, b in zip(tiled, rows):
        for x, y in zip(a, b):
            assert np.array_equal(x, y)
    kc, ks, vc, vs = tiled[0]
    ekc, eks = oracle.quantize_rows(k16[:300].transpose(1, 0, 2))
    evc, evs = oracle.quantize_rows(v16[:300].transpose(1, 0, 2))
    assert np.array_equal(kc[:, 45:345], ekc) and np.array_equal(ks[:, 45:345], eks)
    assert np.array_equal(vc[:, 45:345], evc) and np.array_equal(vs[:, 45:345], evs)
    ek, eks = oracle.quantize_rows_f32(k32[100:400].transpose(1, 0, 2))
    assert np.array_equal(kc[:, 445:745], ek) and np.array_equal(ks[:, 445:745], eks)


@pytest.mark.parametrize("paged", [False, True])
def test_export_dequant_matches_oracle(gpu, paged):
    """miikv_export_dequant / download_key / download_value: float(code) * float(scale)
    rows, equal to the oracle's dequantisation of the oracle's codes (exact)."""
    import miinfer_amd as m
    rng = np.random.default_rng(21 + paged)
    hk, d, n = 4, 256, 700
    if paged:
        table = np.array([[2, 0, 1]], np.int32)
        cache = m.KvCache.paged_cache(hk, d, 3, torch.from_numpy(table).to(gpu), page_tokens=256)
    else:
        cache = m.KvCache.contiguous(hk, d, 768)
    k = rng.standard_normal((n, hk, d)).astype(np.float32).astype(np.float16)
    v = rng.standard_normal((n, hk, d)).astype(np.float32).astype(np.float16)
    cache.append(torch.from_numpy(k).to(gpu), torch.from_numpy(v).to(gpu))
    kc, ks = oracle.quantize_rows(k.transpose(1, 0, 2))
    vc, vs = oracle.quantize_rows(v.transpose(1, 0, 2))
    assert np.array_equal(cache.download_key(n), oracle.dequantize_rows(kc, ks))
    assert np.array_equal(cache.download_value(n), oracle.dequantize_rows(vc, vs))
    kd, vd = cache.export_dequant(0, 100, 300)
    torch.cuda.synchronize()
    assert np.array_equal(kd.cpu().numpy(), oracle.dequantize_rows(kc, ks)[:, 100:400])
    assert np.array_equal(vd.cpu().numpy(), oracle.dequantize_rows(vc, vs)[:, 100:400])
