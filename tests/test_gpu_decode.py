"""Split-K GQA decode attention over the q8_0 cache vs the fp32 oracle (GPU).

Tolerance: max-abs 2e-3 and relative 1e-2 (tests/helpers.py)."""
import math

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import assert_attention_close, randn_f16

pytestmark = pytest.mark.gpu


def _dev(a, gpu):
    return torch.from_numpy(np.ascontiguousarray(a)).to(gpu)


def _filled_contiguous(gpu, rng, hk, d, cap, n):
    import miinfer_amd as m
    cache = m.KvCache.contiguous(hk, d, cap)
    k = randn_f16(rng, (n, hk, d))
    v = randn_f16(rng, (n, hk, d))
    if n:
        cache.append(_dev(k, gpu), _dev(v, gpu))
    kc, ks = oracle.quantize_rows(k.transpose(1, 0, 2))
    vc, vs = oracle.quantize_rows(v.transpose(1, 0, 2))
    return cache, (kc, ks, vc, vs)


@pytest.mark.parametrize("length", [1, 2, 17, 63, 64, 65, 300, 1024, 4096])
def test_decode_c2_shape(gpu, length):
    import miinfer_amd as m
    hq, hk, d = 32, 8, 128
    rng = np.random.default_rng(length)
    cache, ref = _filled_contiguous(gpu, rng, hk, d, 4096, length)
    q = randn_f16(rng, (1, hq, d))
    lens = _dev(np.array([length], np.int32), gpu)
    out, _ = m.decode_attention(cache, _dev(q, gpu), lengths=lens, max_context=4096)
    torch.cuda.synchronize()
    expect = oracle.attention_q8(q[0].astype(np.float32), *ref, length, hq, 1 / math.sqrt(d))
    assert_attention_close(out[0].cpu().numpy(), expect, f"L={length}")


def test_decode_c2_32k_with_gate_and_state(gpu):
    import miinfer_amd as m
    hq, hk, d, length = 32, 8, 128, 32768
    rng = np.random.default_rng(2)
    cache, ref = _filled_contiguous(gpu, rng, hk, d, length, length)
    q = randn_f16(rng, (1, hq, d))
    gate = rng.standard_normal((1, hq, d)).astype(np.float32)
    ds = m.make_decode_state(length - 1, device=gpu)
    out, gated = m.decode_attention(cache, _dev(q, gpu), decode_state=ds, gate=_dev(gate, gpu),
                                    out=torch.empty((1, hq, d), device=gpu))
    torch.cuda.synchronize()
    expect = oracle.attention_q8(q[0].astype(np.float32), *ref, length, hq, 1 / math.sqrt(d))
    assert_attention_close(out[0].cpu().numpy(), expect, "32k")
    assert_attention_close(gated[0].cpu().numpy(), expect / (1 + np.exp(-gate[0])), "32k gated")


def test_decode_fp32_query(gpu):
    import miinfer_amd as m
    hq, hk, d, length = 32, 8, 128, 777
    rng = np.random.default_rng(3)
    cache, ref = _filled_contiguous(gpu, rng, hk, d, 1024, length)
    q = rng.standard_normal((1, hq, d)).astype(np.float32)  # not fp16-representable
    lens = _dev(np.array([length], np.int32), gpu)
    out, _ = m.decode_attention(cache, _dev(q, gpu), lengths=lens, max_context=1024)
    torch.cuda.synchronize()
    expect = oracle.attention_q8(q[0], *ref, length, hq, 1 / math.sqrt(d))
    assert_attention_close(out[0].cpu().numpy(), expect, "fp32 q")


def test_decode_replays_are_byte_identical(gpu):
    """The reference requires byte-identical replays
    (tests/qwen3_cached_attention_determinism_gpu_test.cpp:52-114); the arrival counters
    must also be left at zero for the next call."""
    import miinfer_amd as m
    hq, hk, d, length = 32, 8, 128, 5000
    rng = np.random.default_rng(4)
    cache, _ = _filled_contiguous(gpu, rng, hk, d, 8192, length)
    q = _dev(randn_f16(rng, (1, hq, d)), gpu)
    lens = _dev(np.array([length], np.int32), gpu)
    ws = m.DecodeWorkspace(cache, hq, 1, 8192)
    outs = []
    for _ in range(16):
        o, _ = m.decode_attention(cache, q, lengths=lens, max_context=8192, workspace=ws)
        outs.append(o.clone())
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o, outs[0])


def test_decode_zero_length_gives_zeros(gpu):
    import miinfer_amd as m
    cache, _ = _filled_contiguous(gpu, np.random.default_rng(5), 8, 128, 256, 10)
    q = torch.ones((1, 32, 128), dtype=torch.float16, device=gpu)
    out = torch.full((1, 32, 128), 7.0, device=gpu)
    m.decode_attention(cache, q, lengths=torch.zeros(1, dtype=torch.int32, device=gpu),
                       max_context=256, out=out)
    torch.cuda.synchronize()
    assert not out.any()


@pytest.mark.parametrize("hq,hk,d", [(24, 4, 256), (32, 8, 128)])
def test_decode_paged_batched(gpu, hq, hk, d):
    """Config-3 style: sequences of ragged length in 256-token pages behind a random table."""
    import miinfer_amd as m
    rng = np.random.default_rng(hq + d)
    pt = 256
    lens = [1, 255, 256, 257, 3000, 1100]
    pages = [(n + pt) // pt for n in lens]  # room for one more token
    stride = max(pages)
    total = sum(pages)
    perm = rng.permutation(total).astype(np.int32)
    table = np.zeros((len(lens), stride), np.int32)
    o = 0
    for s, p in enumerate(pages):
        table[s, :p] = perm[o:o + p]
        o += p
    cache = m.KvCache.paged_cache(hk, d, total, _dev(table, gpu), page_tokens=pt)
    refs = []
    for s, n in enumerate(lens):
        k = randn_f16(rng, (n, hk, d))
        v = randn_f16(rng, (n, hk, d))
        cache.append(_dev(k, gpu), _dev(v, gpu), base_position=0, seq=s)
        kc, ks = oracle.quantize_rows(k.transpose(1, 0, 2))
        vc, vs = oracle.quantize_rows(v.transpose(1, 0, 2))
        refs.append((kc, ks, vc, vs))
    q = randn_f16(rng, (len(lens), hq, d))
    max_ctx = stride * pt
    out, _ = m.decode_attention(cache, _dev(q, gpu), lengths=_dev(np.array(lens, np.int32), gpu),
                                max_context=max_ctx)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    for s, n in enumerate(lens):
        expect = oracle.attention_q8(q[s].astype(np.float32), *refs[s], n, hq, 1 / math.sqrt(d))
        assert_attention_close(out[s], expect, f"seq {s} L={n}")


def test_decode_q8_1_epilogue(gpu):
    """The Q8_1 blocks are exactly the reference rule applied to the kernel's own
    gated output (bit-exact), and that output matches the oracle."""
    import miinfer_amd as m
    rng = np.random.default_rng(77)
    hq, hk, d, length = 24, 4, 256, 3000
    cache, ref = _filled_contiguous(gpu, rng, hk, d, 3072, length)
    q = randn_f16(rng, (1, hq, d))
    gate = rng.standard_normal((1, hq, d)).astype(np.float32)
    blocks = torch.zeros((hq * d // 32, 36), dtype=torch.uint8, device=gpu)
    lengths = torch.tensor([length], dtype=torch.int32, device=gpu)
    _, gated = m.decode_attention(cache, _dev(q, gpu), lengths=lengths, gate=_dev(gate, gpu),
                                  gated_q8_1=blocks)
    torch.cuda.synchronize()
    g = gated.cpu().numpy()
    assert np.array_equal(blocks.cpu().numpy(), oracle.q8_1_blocks(g.reshape(-1)))
    expect = oracle.attention_q8(q[0].astype(np.float32), *ref, length, hq, 1 / math.sqrt(d))
    assert_attention_close(g[0], expect / (1 + np.exp(-gate[0])), "gated")


def test_decode_rejects_bad_arguments(gpu):
    import miinfer_amd as m
    cache, _ = _filled_contiguous(gpu, np.random.default_rng(6), 8, 128, 256, 4)
    q = torch.zeros((1, 30, 128), dtype=torch.float16, device=gpu)  # 30 % 8 != 0
    with pytest.raises((m.MiikvError, ValueError)):
        m.decode_attention(cache, q, lengths=torch.ones(1, dtype=torch.int32, device=gpu),
                           max_context=256)
    q = torch.zeros((1, 32, 128), dtype=torch.float16, device=gpu)
    with pytest.raises(m.MiikvError):  # max_context beyond capacity
        m.decode_attention(cache, q, lengths=torch.ones(1, dtype=torch.int32, device=gpu),
                           max_context=512)


def test_decode_batch_device_chosen_split(gpu):
    """A batch whose total context is large enough that the device raises the steps
    per wave above the host's floor (the lengths are only known on the device): the
    packed work items and the combine must agree on the split size."""
    import miinfer_amd as m
    rng = np.random.default_rng(31)
    hq, hk, d, pt = 32, 8, 128, 256
    lens = [60000, 1000, 30000, 9000, 1]
    pages = [(n + pt) // pt for n in lens]
    stride = max(pages)
    perm = rng.permutation(sum(pages)).astype(np.int32)
    table = np.zeros((len(lens), stride), np.int32)
    o = 0
    for s, p in enumerate(pages):
        table[s, :p] = perm[o:o + p]
        o += p
    cache = m.KvCache.paged_cache(hk, d, sum(pages), _dev(table, gpu), page_tokens=pt)
    refs = []
    for s, n in enumerate(lens):
        k = randn_f16(rng, (n, hk, d))
        v = randn_f16(rng, (n, hk, d))
        cache.append(_dev(k, gpu), _dev(v, gpu), base_position=0, seq=s)
        refs.append((oracle.quantize_rows(k.transpose(1, 0, 2)), oracle.quantize_rows(v.transpose(1, 0, 2))))
    q = randn_f16(rng, (len(lens), hq, d))
    out, _ = m.decode_attention(cache, _dev(q, gpu), lengths=_dev(np.array(lens, np.int32), gpu),
                                max_context=stride * pt)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    for s, n in enumerate(lens):
        (kc, ks), (vc, vs) = refs[s]
        expect = oracle.attention_q8(q[s].astype(np.float32), kc, ks, vc, vs, n, hq, 1 / math.sqrt(d))
        assert_attention_close(out[s], expect, f"seq {s} L={n}")


def test_decode_config3_full_size_fused_append(gpu):
    """Config 3 at full size, as bench.py runs it: 16 sequences of 24q/4kv/D256 with
    context lengths uniform in [1024, 65536] (seed 3), 256-token pages behind a random
    permutation table, one appended row per sequence in the same launch pair.  Every
    sequence's new row is checked byte for byte; the attention of four sequences (the
    longest and shortest among them) against the oracle."""
    import miinfer_amd as m
    hq, hk, d, pt, batch = 24, 4, 256, 256, 16
    rng = np.random.default_rng(3)
    lens = rng.integers(1024, 65536 + 1, size=batch)
    pages = [(int(n) + pt) // pt for n in lens]
    stride = max(pages)
    perm = rng.permutation(sum(pages)).astype(np.int32)
    table = np.zeros((batch, stride), np.int32)
    o = 0
    for b, p in enumerate(pages):
        table[b, :p] = perm[o:o + p]
        o += p
    cache = m.KvCache.paged_cache(hk, d, sum(pages), _dev(table, gpu), page_tokens=pt)
    gen = torch.Generator(device=gpu).manual_seed(0)
    kv = []
    for b, n in enumerate(lens):
        k = torch.randn((int(n), hk, d), device=gpu, generator=gen).half()
        v = torch.randn((int(n), hk, d), device=gpu, generator=gen).half()
        cache.append(k[:-1], v[:-1], base_position=0, seq=b)
        kv.append((k, v))
    q = randn_f16(rng, (batch, hq, d))
    knew = torch.stack([k[-1] for k, _ in kv]).contiguous()
    vnew = torch.stack([v[-1] for _, v in kv]).contiguous()
    out, _ = m.decode_attention(cache, _dev(q, gpu), lengths=_dev(lens.astype(np.int32), gpu),
                                max_context=stride * pt, k_new=knew, v_new=vnew)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    order = np.argsort(lens)
    for b in range(batch):
        n = int(lens[b])
        k, v = (t.cpu().numpy() for t in kv[b])
        kc, ks, vc, vs = _canon_tail(cache, b, n)
        ekc, eks = oracle.quantize_rows(k[-1:].transpose(1, 0, 2))
        evc, evs = oracle.quantize_rows(v[-1:].transpose(1, 0, 2))
        assert np.array_equal(kc, ekc) and np.array_equal(ks.view(np.uint16), eks)
        assert np.array_equal(vc, evc) and np.array_equal(vs.view(np.uint16), evs)
        if b in (order[0], order[1], order[-2], order[-1]):
            rk = oracle.quantize_rows(k.transpose(1, 0, 2))
            rv = oracle.quantize_rows(v.transpose(1, 0, 2))
            expect = oracle.attention_q8(q[b].astype(np.float32), *rk, *rv, n, hq, 1 / math.sqrt(d))
            assert_attention_close(out[b], expect, f"seq {b} L={n}")


def _canon_tail(cache, seq, n):
    """The last row (position n-1) of sequence `seq` in canonical form."""
    out = cache.export_canonical(seq, n - 1, 1)
    torch.cuda.synchronize()
    return [t.cpu().numpy() for t in out]


@pytest.mark.parametrize("length", [1, 129, 20000, 30001, 32768])
def test_decode_c2_capacity_32k_partial(gpu, length):
    """Config 2 shape planned for a 32768-token bound (4 steps per wave, the four waves
    of a workgroup interleaving their split's steps) at shorter contexts, so that
    splits end mid-way, some hold no key and the last step is masked.  With the fused
    append the new row (position length-1) is stored and scored in the same launch
    pair; the cache held junk at that position before."""
    import miinfer_amd as m
    hq, hk, d, cap = 32, 8, 128, 32768
    rng = np.random.default_rng(length + 11)
    k = randn_f16(rng, (length, hk, d))
    v = randn_f16(rng, (length, hk, d))
    cache = m.KvCache.contiguous(hk, d, cap)
    junk = randn_f16(rng, (1, hk, d)) * np.float16(50)
    if length > 1:
        cache.append(_dev(k[:-1], gpu), _dev(v[:-1], gpu))
    cache.append(_dev(junk, gpu), _dev(junk, gpu), base_position=length - 1)
    q = randn_f16(rng, (1, hq, d))
    lens = _dev(np.array([length], np.int32), gpu)
    out, _ = m.decode_attention(cache, _dev(q, gpu), lengths=lens, max_context=cap,
                                k_new=_dev(k[-1:], gpu), v_new=_dev(v[-1:], gpu))
    torch.cuda.synchronize()
    rk = oracle.quantize_rows(k.transpose(1, 0, 2))
    rv = oracle.quantize_rows(v.transpose(1, 0, 2))
    expect = oracle.attention_q8(q[0].astype(np.float32), *rk, *rv, length, hq, 1 / math.sqrt(d))
    assert_attention_close(out[0].cpu().numpy(), expect, f"L={length}")
    kc, ks, vc, vs = _canon_tail(cache, 0, length)
    assert np.array_equal(kc, rk[0][:, -1:]) and np.array_equal(ks.view(np.uint16), rk[1][:, -1:])
    assert np.array_equal(vc, rv[0][:, -1:]) and np.array_equal(vs.view(np.uint16), rv[1][:, -1:])


def test_side_stream_temporaries(gpu):
    """Helpers given a side stream allocate their temporaries on it: decode attention
    with an auto-allocated workspace and page copies run there and give the results of
    the default-stream calls."""
    import miinfer_amd as m
    from miinfer_amd import reuse
    rng = np.random.default_rng(11)
    hq, hk, d, pt = 24, 4, 256, 256
    table = np.array([[0, 1, 2], [3, 4, 5]], np.int32)
    cache = m.KvCache.paged_cache(hk, d, 8, _dev(table, gpu), page_tokens=pt)
    k = randn_f16(rng, (700, hk, d))
    v = randn_f16(rng, (700, hk, d))
    cache.append(_dev(k, gpu), _dev(v, gpu), base_position=0, seq=0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    reuse.run_page_copies(cache, [(0, 3), (1, 4), (2, 5)], stream=side)
    q = _dev(randn_f16(rng, (2, hq, d)), gpu)
    lens = torch.tensor([700, 700], dtype=torch.int32, device=gpu)
    out_side, _ = m.decode_attention(cache, q, lengths=lens, max_context=3 * pt, stream=side)
    side.synchronize()
    out_ref, _ = m.decode_attention(cache, q, lengths=lens, max_context=3 * pt)
    torch.cuda.synchronize()
    assert torch.equal(out_side, out_ref)
    kc, ks = oracle.quantize_rows(k.transpose(1, 0, 2))
    vc, vs = oracle.quantize_rows(v.transpose(1, 0, 2))
    for s in range(2):  # row 1 reads the copied pages
        expect = oracle.attention_q8(q[s].cpu().numpy().astype(np.float32), kc, ks, vc, vs, 700, hq,
                                     1 / math.sqrt(d))
        assert_attention_close(out_ref[s].cpu().numpy(), expect, f"row {s}")


@pytest.mark.parametrize("length", [131072, 100003])
def test_decode_128k_context(gpu, length):
    """Config 2 shape at a 131072-token capacity (16 steps per wave, 64 splits of 2048
    keys): the largest context tested; 100003 ends mid-split and mid-step."""
    import miinfer_amd as m
    hq, hk, d, cap = 32, 8, 128, 131072
    rng = np.random.default_rng(length)
    cache, ref = _filled_contiguous(gpu, rng, hk, d, cap, length)
    q = randn_f16(rng, (1, hq, d))
    lens = _dev(np.array([length], np.int32), gpu)
    out, _ = m.decode_attention(cache, _dev(q, gpu), lengths=lens, max_context=cap)
    torch.cuda.synchronize()
    expect = oracle.attention_q8(q[0].astype(np.float32), *ref, length, hq, 1 / math.sqrt(d))
    assert_attention_close(out[0].cpu().numpy(), expect, f"L={length}")


@pytest.mark.parametrize("length,cap", [(16384, 16384), (32768, 32768), (20001, 32768), (5000, 65536)])
def test_decode_d256_single_sequence_plans(gpu, length, cap):
    """24q/4kv/D256, one sequence: the plans of 2, 4 and 8 steps per wave (one workgroup
    per CU), full and partial contexts."""
    import miinfer_amd as m
    hq, hk, d = 24, 4, 256
    rng = np.random.default_rng(length + cap)
    cache, ref = _filled_contiguous(gpu, rng, hk, d, cap, length)
    q = randn_f16(rng, (1, hq, d))
    lens = _dev(np.array([length], np.int32), gpu)
    out, _ = m.decode_attention(cache, _dev(q, gpu), lengths=lens, max_context=cap)
    torch.cuda.synchronize()
    expect = oracle.attention_q8(q[0].astype(np.float32), *ref, length, hq, 1 / math.sqrt(d))
    assert_attention_close(out[0].cpu().numpy(), expect, f"L={length} cap={cap}")


# (hq, hk, d, length): 32q/8kv/D128 and 24q/4kv/D256 pair the query's lo parts into
# spare MFMA columns, as do the edges 8q/8kv (one head: columns 0 and 8) and 16q/2kv
# (eight heads: all 16 columns); 32q/2kv/D128 (16 heads per kv head) carries them as
# a second fragment set.
@pytest.mark.parametrize("hq,hk,d,length", [(32, 8, 128, 3000), (24, 4, 256, 2500), (32, 2, 128, 1800),
                                            (8, 8, 128, 2200), (16, 2, 256, 1300)])
def test_decode_fp32_query_low_parts_count(gpu, hq, hk, d, length):
    """An fp32 query enters as fp16 hi + lo parts.  The attention tolerance alone would
    not notice lost lo parts (they move the output by less than it), so: the result
    differs from the same query rounded to fp16, and is closer to the fp32 oracle."""
    import miinfer_amd as m
    rng = np.random.default_rng(hq + d + length)
    cache, ref = _filled_contiguous(gpu, rng, hk, d, ((length + 255) // 256) * 256, length)
    q32 = (rng.standard_normal((1, hq, d)) * 3).astype(np.float32)
    q16 = q32.astype(np.float16)
    lens = _dev(np.array([length], np.int32), gpu)
    scale = 2 / math.sqrt(d)  # sharper softmax: more weight on the scores
    o32, _ = m.decode_attention(cache, _dev(q32, gpu), lengths=lens, max_context=cache.capacity, scale=scale)
    o16, _ = m.decode_attention(cache, _dev(q16, gpu), lengths=lens, max_context=cache.capacity, scale=scale)
    torch.cuda.synchronize()
    o32, o16 = o32[0].cpu().numpy(), o16[0].cpu().numpy()
    expect = oracle.attention_q8(q32[0], *ref, length, hq, scale)
    assert_attention_close(o32, expect, "fp32 q")
    e32 = float(np.linalg.norm(o32 - expect))
    e16 = float(np.linalg.norm(o16 - expect))
    print(f"hq={hq} hk={hk} d={d}: |o32-ref|={e32:.3e} |o16-ref|={e16:.3e}")
    assert not np.array_equal(o32, o16)
    assert e32 < 0.5 * e16, (e32, e16)


# seeds 10-13 fix shapes with at least 16384 combine threads (the narrow combine
# whatever the record bound): 16 x 24q/4kv/D256 (config 3's shape), 24 x 32q/8kv/D128,
# 20 x 48q/8kv/D128, 12 x 64q/8kv/D256
_WIDE_BATCHES = {10: (256, 4, 6, 16), 11: (128, 8, 4, 24), 12: (128, 8, 6, 20), 13: (256, 8, 8, 12)}


@pytest.mark.parametrize("seed", range(14))
def test_decode_random_batches(gpu, seed):
    """Seeded random batches of paged decodes (batch, heads per kv head, head_dim, ragged
    lengths including 0 and 1, context bound, query dtype, gate): the plan's split
    size, the device's choice of steps per wave and the combine form (the wide one,
    or one thread per 4 outputs) all vary with them; every row against the oracle."""
    import miinfer_amd as m
    rng = np.random.default_rng(1000 + seed)
    d = int(rng.choice([128, 256]))
    hk = int(rng.choice([1, 2, 4, 8]))
    g = int(rng.choice([1, 2, 4, 6, 8]))
    hq = hk * g
    batch = int(rng.integers(1, 25))
    if seed in _WIDE_BATCHES:
        d, hk, g, batch = _WIDE_BATCHES[seed]
        hq = hk * g
    pt = 256
    lens = rng.integers(0, 2500, size=batch)
    lens[rng.random(batch) < 0.15] = 0
    lens[rng.random(batch) < 0.1] = 1
    pages = [max(1, (int(n) + pt) // pt) for n in lens]
    stride = max(pages) + int(rng.integers(0, 3))  # a context bound above the longest sequence
    total = sum(pages)
    perm = rng.permutation(total).astype(np.int32)
    table = np.zeros((batch, stride), np.int32)
    o = 0
    for s, p in enumerate(pages):
        table[s, :p] = perm[o:o + p]
        table[s, p:] = perm[o + p - 1]  # unused entries name a valid page
        o += p
    cache = m.KvCache.paged_cache(hk, d, total, _dev(table, gpu), page_tokens=pt)
    refs = []
    for s, n in enumerate(lens):
        n = int(n)
        k = randn_f16(rng, (n, hk, d))
        v = randn_f16(rng, (n, hk, d))
        if n:
            cache.append(_dev(k, gpu), _dev(v, gpu), base_position=0, seq=s)
        kc, ks = oracle.quantize_rows(k.transpose(1, 0, 2))
        vc, vs = oracle.quantize_rows(v.transpose(1, 0, 2))
        refs.append((kc, ks, vc, vs))
    f32 = bool(rng.integers(0, 2))
    q = rng.standard_normal((batch, hq, d)).astype(np.float32) if f32 else randn_f16(rng, (batch, hq, d))
    gate = rng.standard_normal((batch, hq, d)).astype(np.float32) if rng.integers(0, 2) else None
    out, gated = m.decode_attention(cache, _dev(q, gpu), lengths=_dev(lens.astype(np.int32), gpu),
                                    max_context=stride * pt, gate=None if gate is None else _dev(gate, gpu),
                                    out=torch.empty((batch, hq, d), device=gpu))
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    what = f"seed {seed}: batch {batch} {hq}q/{hk}kv/D{d} f32={f32} gate={gate is not None}"
    for s, n in enumerate(lens):
        if n == 0:
            assert not out[s].any(), what
            continue
        expect = oracle.attention_q8(q[s].astype(np.float32), *refs[s], int(n), hq, 1 / math.sqrt(d))
        assert_attention_close(out[s], expect, f"{what} seq {s} L={n}")
        if gate is not None:
            assert_attention_close(gated[s].cpu().numpy(), expect / (1 + np.exp(-gate[s])), f"{what} gated seq {s}")
