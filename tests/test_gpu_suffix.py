"""Suffix attention over a cached q8_0 prefix (MFMA) vs the fp32 oracle (GPU).

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


def _setup(gpu, rng, hq, hk, d, prefix, t, cap):
    import miinfer_amd as m
    cache = m.KvCache.contiguous(hk, d, cap)
    k = randn_f16(rng, (prefix + t, hk, d))
    v = randn_f16(rng, (prefix + t, hk, d))
    if prefix:
        cache.append(_dev(k[:prefix], gpu), _dev(v[:prefix], gpu), base_position=0)
    cache.append(_dev(k[prefix:], gpu), _dev(v[prefix:], gpu), base_position=prefix)  # the suffix rows
    kc, ks = oracle.quantize_rows(k.transpose(1, 0, 2))
    vc, vs = oracle.quantize_rows(v.transpose(1, 0, 2))
    return cache, (kc, ks, vc, vs)


@pytest.mark.parametrize("hq,hk,d,prefix,t", [(24, 4, 256, 300, 40), (32, 8, 128, 1000, 64),
                                              (24, 4, 256, 0, 17), (6, 1, 128, 64, 1),
                                              (24, 4, 256, 257, 33), (24, 4, 256, 5000, 3),
                                              (8, 8, 128, 3000, 130),
                                              # more query heads per kv head than decode's
                                              # 16 MFMA columns: the MFMA path only
                                              (34, 2, 128, 300, 9), (40, 2, 256, 100, 20),
                                              # split plans evenly divided over the
                                              # workgroup slots, ranges across row blocks
                                              (24, 4, 256, 2000, 100), (12, 2, 128, 600, 300)])
@pytest.mark.parametrize("split", [True, False])
def test_suffix_small(gpu, hq, hk, d, prefix, t, split):
    import miinfer_amd as m
    rng = np.random.default_rng(prefix + t + d)
    cap = ((prefix + t + 63) // 64) * 64
    cache, ref = _setup(gpu, rng, hq, hk, d, prefix, t, cap)
    q = randn_f16(rng, (t, hq, d))
    gate = rng.standard_normal((t, hq, d)).astype(np.float32)
    out, gated = m.suffix_attention(cache, _dev(q, gpu), prefix, gate=_dev(gate, gpu),
                                    out=torch.empty((t, hq, d), device=gpu), split=split)
    torch.cuda.synchronize()
    expect = oracle.suffix_attention_q8(q.astype(np.float32), *ref, prefix, hq, 1 / math.sqrt(d))
    assert_attention_close(out.cpu().numpy(), expect, "suffix")
    assert_attention_close(gated.cpu().numpy(), expect / (1 + np.exp(-gate)), "suffix gated")


@pytest.mark.parametrize("split", [True, False])
def test_suffix_config4_full_size_sampled_tokens(gpu, split):
    """Config 4: 512 suffix tokens over an 8192-token prefix (24q/4kv/D256); the oracle
    checks a sample of tokens (each is an independent causal row set)."""
    import miinfer_amd as m
    hq, hk, d, prefix, t = 24, 4, 256, 8192, 512
    rng = np.random.default_rng(4)
    cache, ref = _setup(gpu, rng, hq, hk, d, prefix, t, prefix + t)
    q = randn_f16(rng, (t, hq, d))
    if split:
        assert m.suffix_workspace_bytes(cache, hq, t) > 0
    out, _ = m.suffix_attention(cache, _dev(q, gpu), prefix, split=split)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    for tok in (0, 1, 63, 64, 255, 511):
        expect = oracle.attention_q8(q[tok].astype(np.float32), *ref, prefix + tok + 1, hq,
                                     1 / math.sqrt(d))
        assert_attention_close(out[tok], expect, f"token {tok}")


@pytest.mark.parametrize("split", [True, False])
def test_suffix_config4_fused_store_full_size(gpu, split):
    """Config 4 as bench.py times it: miikv_suffix_append_attn stores 512 fp16 suffix rows
    over an 8192-token prefix (24q/4kv/D256) and attends.  All 512 stored rows (codes and
    scales of every kv head, over slots that held other bytes) are bit-exact against the
    oracle's quantisation, and two tokens of every 32-token block of the suffix, token 511
    among them, match the oracle's attention."""
    import miinfer_amd as m
    hq, hk, d, prefix, t = 24, 4, 256, 8192, 512
    rng = np.random.default_rng(44)
    cap = prefix + t
    k = randn_f16(rng, (cap, hk, d))
    v = randn_f16(rng, (cap, hk, d))
    cache = m.KvCache.contiguous(hk, d, cap)
    junk = randn_f16(rng, (t, hk, d)) * np.float16(20)
    cache.append(_dev(junk, gpu), _dev(junk, gpu), base_position=prefix)  # older bytes in the slots
    cache.append(_dev(k[:prefix], gpu), _dev(v[:prefix], gpu), base_position=0)
    q16 = randn_f16(rng, (t, hq, d))
    out, _ = m.suffix_attention(cache, _dev(q16, gpu), prefix, split=split, k_new=_dev(k[prefix:], gpu),
                                v_new=_dev(v[prefix:], gpu))
    torch.cuda.synchronize()
    kc, ks = oracle.quantize_rows(k.transpose(1, 0, 2))
    vc, vs = oracle.quantize_rows(v.transpose(1, 0, 2))
    got = _canon_all(cache, 0, cap)
    for x, e, name in zip(got, (kc, ks.view(np.int16), vc, vs.view(np.int16)),
                          ("k codes", "k scales", "v codes", "v scales")):
        assert np.array_equal(x[:, prefix:], e[:, prefix:]), f"stored suffix {name}"
        assert np.array_equal(x[:, :prefix], e[:, :prefix]), f"prefix {name}"
    out = out.cpu().numpy()
    toks = sorted({32 * j + (7 * j) % 32 for j in range(16)} | {32 * j + 31 - (5 * j) % 16 for j in range(16)}
                  | {0, 511})
    for tok in toks:
        expect = oracle.attention_q8(q16[tok].astype(np.float32), kc, ks, vc, vs, prefix + tok + 1, hq,
                                     1 / math.sqrt(d))
        assert_attention_close(out[tok], expect, f"token {tok}")


# (t, extra): 100 tokens run on the MFMA path, 3 as a batch of decodes
@pytest.mark.parametrize("t,extra", [(100, 20), (3, 2)])
@pytest.mark.parametrize("split", [True, False])
def test_suffix_prefill_state_and_paged(gpu, split, t, extra):
    import miinfer_amd as m
    rng = np.random.default_rng(8)
    hq, hk, d, pt = 24, 4, 256, 256
    prefix = 700
    npages = (prefix + t + pt - 1) // pt
    table = _dev(rng.permutation(npages + 2)[:npages].astype(np.int32).reshape(1, npages), gpu)
    cache = m.KvCache.paged_cache(hk, d, npages + 2, table, page_tokens=pt)
    k = randn_f16(rng, (prefix + t, hk, d))
    v = randn_f16(rng, (prefix + t, hk, d))
    cache.append(_dev(k, gpu), _dev(v, gpu), base_position=0)
    kc, ks = oracle.quantize_rows(k.transpose(1, 0, 2))
    vc, vs = oracle.quantize_rows(v.transpose(1, 0, 2))
    q = randn_f16(rng, (t + extra, hq, d))  # host bound t + extra rows, device says t
    ps = m.make_prefill_state(prefix, t, device=gpu)
    out = torch.full((t + extra, hq, d), 5.0, device=gpu)
    m.suffix_attention(cache, _dev(q, gpu), 0, prefill_state=ps, out=out, split=split)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    expect = oracle.suffix_attention_q8(q[:t].astype(np.float32), kc, ks, vc, vs, prefix, hq,
                                        1 / math.sqrt(d))
    assert_attention_close(got[:t], expect, "paged suffix")
    assert np.all(got[t:] == 5.0)  # rows past the device token count untouched


def test_suffix_split_matches_unsplit(gpu):
    """Split-K and single-split results agree closely: same fp16 tiles and MFMAs; only the
    running max (and so the fp16 rounding of each probability) and the summation order
    differ.  Probabilities carry 2^-11 relative rounding, so 2e-4 absolute bounds it."""
    import miinfer_amd as m
    rng = np.random.default_rng(11)
    hq, hk, d, prefix, t = 32, 8, 128, 4000, 96
    cache, _ = _setup(gpu, rng, hq, hk, d, prefix, t, prefix + t + 64)
    q = _dev(randn_f16(rng, (t, hq, d)), gpu)
    a, _ = m.suffix_attention(cache, q, prefix, split=True)
    b, _ = m.suffix_attention(cache, q, prefix, split=False)
    torch.cuda.synchronize()
    assert torch.allclose(a, b, atol=2e-4, rtol=1e-3), (a - b).abs().max().item()


def test_suffix_workspace_too_small_is_rejected(gpu):
    """64 tokens (the MFMA path): a workspace holding just the context's tiles runs
    one split (same results as the full workspace within the split tolerance, and the
    oracle's); one byte less is rejected."""
    import miinfer_amd as m
    rng = np.random.default_rng(12)
    hq, hk, d, prefix, t = 24, 4, 256, 2048, 64
    cache, ref = _setup(gpu, rng, hq, hk, d, prefix, t, prefix + t)
    q16 = randn_f16(rng, (t, hq, d))
    q = _dev(q16, gpu)
    tiles = hk * ((prefix + t + 31) // 32) * 2 * d * 32 * 2
    assert m.suffix_workspace_bytes(cache, hq, t) > tiles
    out, _ = m.suffix_attention(cache, q, prefix, workspace=torch.empty(tiles, dtype=torch.uint8, device=gpu))
    torch.cuda.synchronize()
    expect = oracle.suffix_attention_q8(q16.astype(np.float32), *ref, prefix, hq, 1 / math.sqrt(d))
    assert_attention_close(out.cpu().numpy(), expect, "single split")
    with pytest.raises(m.MiikvError):
        m.suffix_attention(cache, q, prefix, workspace=torch.empty(tiles - 1, dtype=torch.uint8, device=gpu))


def _canon_all(cache, seq, n):
    out = cache.export_canonical(seq, 0, n)
    torch.cuda.synchronize()
    return [t.cpu().numpy() for t in out]


@pytest.mark.parametrize("hq,hk,d,prefix,t,split", [(24, 4, 256, 300, 40, True), (32, 8, 128, 1000, 64, True),
                                                    (24, 4, 256, 0, 17, False), (6, 1, 128, 64, 1, True),
                                                    (24, 4, 256, 257, 96, False), (8, 8, 128, 3000, 130, True)])
def test_suffix_fused_append_matches_append_then_attend(gpu, hq, hk, d, prefix, t, split):
    """miikv_suffix_append_attn stores the suffix rows with the bytes miikv_append_f16
    stores (the cache slots start with older bytes) and returns exactly the outputs of
    append followed by miikv_suffix_attn; the oracle checks the result."""
    import miinfer_amd as m
    rng = np.random.default_rng(prefix * 3 + t)
    cap = ((prefix + t + 63) // 64) * 64
    k = randn_f16(rng, (prefix + t, hk, d))
    v = randn_f16(rng, (prefix + t, hk, d))
    junk = randn_f16(rng, (cap, hk, d)) * np.float16(30)
    fused = m.KvCache.contiguous(hk, d, cap)
    plain = m.KvCache.contiguous(hk, d, cap)
    fused.append(_dev(junk, gpu), _dev(junk, gpu))
    for c in (fused, plain):
        if prefix:
            c.append(_dev(k[:prefix], gpu), _dev(v[:prefix], gpu), base_position=0)
    plain.append(_dev(k[prefix:], gpu), _dev(v[prefix:], gpu), base_position=prefix)
    q = _dev(randn_f16(rng, (t, hq, d)), gpu)
    a, _ = m.suffix_attention(fused, q, prefix, split=split, k_new=_dev(k[prefix:], gpu),
                              v_new=_dev(v[prefix:], gpu))
    b, _ = m.suffix_attention(plain, q, prefix, split=split)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    for x, y in zip(_canon_all(fused, 0, prefix + t), _canon_all(plain, 0, prefix + t)):
        assert np.array_equal(x, y)
    kc, ks = oracle.quantize_rows(k.transpose(1, 0, 2))
    vc, vs = oracle.quantize_rows(v.transpose(1, 0, 2))
    expect = oracle.suffix_attention_q8(q.cpu().numpy().astype(np.float32), kc, ks, vc, vs, prefix, hq,
                                        1 / math.sqrt(d))
    assert_attention_close(a.cpu().numpy(), expect, "fused suffix")


@pytest.mark.parametrize("t,extra", [(100, 20), (4, 3)])
def test_suffix_fused_append_paged_prefill_state(gpu, t, extra):
    """Paged cache, positions from a device prefill state (host bound larger than the
    device token count): rows past the device count are neither stored nor attended.
    4 + 3 tokens run as a batch of decodes after a plain append."""
    import miinfer_amd as m
    rng = np.random.default_rng(21)
    hq, hk, d, pt = 24, 4, 256, 256
    prefix = 700
    npages = (prefix + t + extra + pt - 1) // pt
    table = _dev(rng.permutation(npages + 2)[:npages].astype(np.int32).reshape(1, npages), gpu)
    k = randn_f16(rng, (prefix + t + extra, hk, d))
    v = randn_f16(rng, (prefix + t + extra, hk, d))
    fused = m.KvCache.paged_cache(hk, d, npages + 2, table, page_tokens=pt)
    plain = m.KvCache.paged_cache(hk, d, npages + 2, table, page_tokens=pt)
    for c in (fused, plain):
        c.append(_dev(k[:prefix], gpu), _dev(v[:prefix], gpu), base_position=0)
    plain.append(_dev(k[prefix:prefix + t], gpu), _dev(v[prefix:prefix + t], gpu), base_position=prefix)
    before = _canon_all(fused, 0, prefix + t + extra)
    q = _dev(randn_f16(rng, (t + extra, hq, d)), gpu)
    ps = m.make_prefill_state(prefix, t, device=gpu)
    a = torch.full((t + extra, hq, d), 5.0, device=gpu)
    b = torch.full((t + extra, hq, d), 5.0, device=gpu)
    m.suffix_attention(fused, q, 0, prefill_state=ps, out=a, k_new=_dev(k[prefix:], gpu),
                       v_new=_dev(v[prefix:], gpu))
    m.suffix_attention(plain, q, 0, prefill_state=ps, out=b)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    assert bool((a[t:] == 5.0).all())
    after = _canon_all(fused, 0, prefix + t + extra)
    for x, y, z in zip(after, _canon_all(plain, 0, prefix + t + extra), before):
        assert np.array_equal(x[:, :prefix + t], y[:, :prefix + t])
        assert np.array_equal(x[:, prefix + t:], z[:, prefix + t:])  # past the device count: untouched


@pytest.mark.parametrize("split", [True, False])
def test_suffix_blocks_near_the_fp16_maximum(gpu, split):
    """Blocks whose absmax sits within 0.8% of the fp16 maximum have scales above
    511.75; the suffix path clamps those scales so that its fp16 tiles stay finite
    (128 * 511.75 = 65504).  Keys and values hold such blocks here: the outputs stay
    finite and equal the oracle over the clamped scales (relative 1e-2), while the
    unclamped oracle differs by the clamp's factor on the affected values."""
    import miinfer_amd as m
    rng = np.random.default_rng(77)
    hq, hk, d, prefix, t = 24, 4, 256, 500, 40
    cache = m.KvCache.contiguous(hk, d, 576)
    k = randn_f16(rng, (prefix + t, hk, d))
    v = randn_f16(rng, (prefix + t, hk, d))
    big = np.float16(65504.0)
    v[::7, :, 32:64] = v[::7, :, 32:64] * np.float16(0.5)   # a block of each 7th row ...
    v[::7, :, 40] = big                                      # ... with absmax 65504: scale 515.5
    k[::11, :, 0:32] = k[::11, :, 0:32] * np.float16(0.01)
    k[::11, :, 3] = np.float16(-65504.0)                     # keys with a huge negative entry
    cache.append(_dev(k, gpu), _dev(v, gpu))
    kc, ks = oracle.quantize_rows(k.transpose(1, 0, 2))
    vc, vs = oracle.quantize_rows(v.transpose(1, 0, 2))
    q = randn_f16(rng, (t, hq, d)) * np.float16(0.01)
    out, _ = m.suffix_attention(cache, _dev(q, gpu), prefix, split=split)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.all(np.isfinite(got))
    f16 = lambda bits: bits.view(np.float16).astype(np.float32)
    clamp = lambda s: np.minimum(f16(s), np.float32(511.75)).astype(np.float16).view(np.uint16)
    assert (f16(vs) > 511.75).any() and (f16(ks) > 511.75).any()
    expect = oracle.suffix_attention_q8(q.astype(np.float32), kc, clamp(ks), vc, clamp(vs), prefix, hq,
                                        1 / math.sqrt(d))
    rel = np.linalg.norm(got - expect) / np.linalg.norm(expect)
    assert rel <= 1e-2, rel
    unclamped = oracle.suffix_attention_q8(q.astype(np.float32), kc, ks, vc, vs, prefix, hq, 1 / math.sqrt(d))
    assert np.abs(unclamped - expect).max() > 1.0  # the clamp is visible at this size


@pytest.mark.parametrize("t", [40, 4])  # the MFMA path; packed decodes
@pytest.mark.parametrize("split", [True, False])
def test_suffix_scores_climbing_far_past_the_first_step(gpu, split, t):
    """Keys deep in the context whose scores exceed every earlier score by ~100 (log2
    units) for some rows: the softmax must re-reference those rows (a fixed reference
    taken from the first keys would overflow fp16 probabilities)."""
    import miinfer_amd as m
    rng = np.random.default_rng(91)
    hq, hk, d, prefix = 24, 4, 256, 3000
    cap = ((prefix + t + 63) // 64) * 64
    k = randn_f16(rng, (prefix + t, hk, d))
    v = randn_f16(rng, (prefix + t, hk, d))
    q = randn_f16(rng, (t, hq, d))
    # key 1700 of kv head 0 and key 2900 of kv head 3 align with two query rows
    k[1700, 0] = (q[t - 1, 0].astype(np.float32) * 6).astype(np.float16)
    k[2900, 3] = (q[min(5, t - 1), 20].astype(np.float32) * 6).astype(np.float16)
    cache = m.KvCache.contiguous(hk, d, cap)
    cache.append(_dev(k, gpu), _dev(v, gpu))
    kc, ks = oracle.quantize_rows(k.transpose(1, 0, 2))
    vc, vs = oracle.quantize_rows(v.transpose(1, 0, 2))
    out, _ = m.suffix_attention(cache, _dev(q, gpu), prefix, split=split)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    expect = oracle.suffix_attention_q8(q.astype(np.float32), kc, ks, vc, vs, prefix, hq, 1 / math.sqrt(d))
    assert np.all(np.isfinite(got))
    # The aligned rows output (nearly) one value row, |x| up to ~4 rather than the
    # ~0.05 of an average over thousands of rows, so the bound is relative there:
    # fp16 tiles and fp16 split records each hold ~2^-11 of |x|.
    err = np.abs(got - expect)
    assert np.all(err <= 2e-3 + 2e-3 * np.abs(expect)), float((err - 2e-3 * np.abs(expect)).max())
    assert np.linalg.norm(got - expect) / np.linalg.norm(expect) <= 1e-2



@pytest.mark.parametrize("t", [1, 5, 9])
def test_suffix_short_on_a_second_sequence(gpu, t):
    """Short suffixes run as a batch of decodes: token t reads sequence `seq`'s block
    table row with context P + t + 1.  Two sequences share the page pool; the suffix
    of sequence 1 must read its own pages only."""
    import miinfer_amd as m
    rng = np.random.default_rng(31 + t)
    hq, hk, d, pt = 24, 4, 256, 256
    prefix = 1500
    per = (prefix + t + pt - 1) // pt
    perm = rng.permutation(2 * per + 3)[:2 * per].astype(np.int32)
    table = _dev(perm.reshape(2, per), gpu)
    cache = m.KvCache.paged_cache(hk, d, 2 * per + 3, table, page_tokens=pt)
    other = randn_f16(rng, (prefix + t, hk, d))
    cache.append(_dev(other, gpu), _dev(other, gpu), base_position=0, seq=0)
    k = randn_f16(rng, (prefix + t, hk, d))
    v = randn_f16(rng, (prefix + t, hk, d))
    cache.append(_dev(k, gpu), _dev(v, gpu), base_position=0, seq=1)
    kc, ks = oracle.quantize_rows(k.transpose(1, 0, 2))
    vc, vs = oracle.quantize_rows(v.transpose(1, 0, 2))
    q = randn_f16(rng, (t, hq, d))
    gate = rng.standard_normal((t, hq, d)).astype(np.float32)
    out, gated = m.suffix_attention(cache, _dev(q, gpu), prefix, seq=1, gate=_dev(gate, gpu),
                                    out=torch.empty((t, hq, d), device=gpu))
    torch.cuda.synchronize()
    expect = oracle.suffix_attention_q8(q.astype(np.float32), kc, ks, vc, vs, prefix, hq, 1 / math.sqrt(d))
    assert_attention_close(out.cpu().numpy(), expect, "seq 1")
    assert_attention_close(gated.cpu().numpy(), expect / (1 + np.exp(-gate)), "seq 1 gated")


# (hq, hk, d, prefix, t): tokens packed per decode row set = largest divisor of t with
# t_pack * (hq / hk) <= 16: 32q/8kv t=4 -> 4, t=6 -> 3 (two row sets), t=2 -> 2;
# 24q/4kv t=2 -> 2, t=4 -> 2; 16q/16kv t=10 -> 10; 24q/4kv t=5 -> 1.
@pytest.mark.parametrize("hq,hk,d,prefix,t", [(32, 8, 128, 3000, 4), (32, 8, 128, 700, 6), (32, 8, 128, 4100, 2),
                                              (24, 4, 256, 2000, 2), (24, 4, 256, 1234, 4), (16, 16, 128, 999, 10),
                                              (24, 4, 256, 640, 5)])
def test_suffix_short_packed_tokens(gpu, hq, hk, d, prefix, t):
    """Short suffixes pack several tokens into one decode row set (one context stream
    serves them all); each packed column masks the keys past its own token."""
    import miinfer_amd as m
    rng = np.random.default_rng(prefix + t)
    cap = ((prefix + t + 63) // 64) * 64
    cache, ref = _setup(gpu, rng, hq, hk, d, prefix, t, cap)
    q = randn_f16(rng, (t, hq, d))
    gate = rng.standard_normal((t, hq, d)).astype(np.float32)
    out, gated = m.suffix_attention(cache, _dev(q, gpu), prefix, gate=_dev(gate, gpu),
                                    out=torch.empty((t, hq, d), device=gpu))
    torch.cuda.synchronize()
    expect = oracle.suffix_attention_q8(q.astype(np.float32), *ref, prefix, hq, 1 / math.sqrt(d))
    assert_attention_close(out.cpu().numpy(), expect, "packed")
    assert_attention_close(gated.cpu().numpy(), expect / (1 + np.exp(-gate)), "packed gated")


# fp32 queries: 16q/4kv/D256 and 32q/8kv/D128 with 2 tokens per row set (8 columns)
# take the paired-column variant (hi parts in columns 0..7, lo parts in 8..15);
# 32q/8kv/D128 t=4 (16 columns) the second fragment set.
@pytest.mark.parametrize("hq,hk,d,prefix,t", [(16, 4, 256, 1500, 2), (16, 4, 256, 900, 4), (32, 8, 128, 2000, 4),
                                              (32, 8, 128, 2100, 2)])
def test_suffix_short_packed_tokens_fp32_query(gpu, hq, hk, d, prefix, t):
    import miinfer_amd as m
    rng = np.random.default_rng(prefix + 7 * t)
    cap = ((prefix + t + 63) // 64) * 64
    cache, ref = _setup(gpu, rng, hq, hk, d, prefix, t, cap)
    q = rng.standard_normal((t, hq, d)).astype(np.float32)
    out, _ = m.suffix_attention(cache, _dev(q, gpu), prefix, out=torch.empty((t, hq, d), device=gpu))
    torch.cuda.synchronize()
    expect = oracle.suffix_attention_q8(q, *ref, prefix, hq, 1 / math.sqrt(d))
    assert_attention_close(out.cpu().numpy(), expect, "packed fp32 query")


@pytest.mark.parametrize("split", [True, False])
def test_suffix_64k_prefix_sampled_tokens(gpu, split):
    """A 64-token suffix over a 65536-token prefix (the prefix length of the reference's
    published suffix runs), 24q/4kv/D256, on the MFMA path; sampled tokens."""
    import miinfer_amd as m
    hq, hk, d, prefix, t = 24, 4, 256, 65536, 64
    rng = np.random.default_rng(65)
    cache, ref = _setup(gpu, rng, hq, hk, d, prefix, t, prefix + t)
    q = randn_f16(rng, (t, hq, d))
    out, _ = m.suffix_attention(cache, _dev(q, gpu), prefix, split=split)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    for tok in (0, 31, 63):
        expect = oracle.attention_q8(q[tok].astype(np.float32), *ref, prefix + tok + 1, hq, 1 / math.sqrt(d))
        assert_attention_close(out[tok], expect, f"token {tok}")


@pytest.mark.parametrize("fused,exact", [(False, False), (True, False), (False, True)])
def test_suffix_chunked_prefill_current_tiles(gpu, fused, exact):
    """Chunked prefill with one workspace and MIIKV_SUFFIX_TILES_CURRENT: each chunk
    expands only its own steps (chunk sizes aligned, unaligned and short, the short
    ones running as decodes while keeping the tiles current), and every chunk's output
    equals a fresh call's over the same cache bit for bit, and the oracle.  With
    `exact`, odd chunks run with MIIKV_SUFFIX_EXACT (as decodes: chunked prefill keeps
    the plain tile layout) and must still leave the tiles current for the MFMA chunks
    after them; a fresh exact call of a long chunk runs the exact-product MFMA kernel
    instead, so those two are compared within the attention tolerance, each against the
    oracle."""
    import miinfer_amd as m
    rng = np.random.default_rng(77 + fused + 2 * exact)
    hq, hk, d, cap = 24, 4, 256, 1024
    chunks = [64, 64, 3, 100, 64, 5, 250, 1, 96]
    total = sum(chunks)
    k = randn_f16(rng, (total, hk, d))
    v = randn_f16(rng, (total, hk, d))
    kc, ks = oracle.quantize_rows(k.transpose(1, 0, 2))
    vc, vs = oracle.quantize_rows(v.transpose(1, 0, 2))
    cache = m.KvCache.contiguous(hk, d, cap)
    fresh = m.KvCache.contiguous(hk, d, cap)
    ws = torch.empty(max(m.suffix_workspace_bytes(cache, hq, t, exact=exact) for t in set(chunks)),
                     dtype=torch.uint8, device=gpu)
    base = 0
    for i, t in enumerate(chunks):
        ex = exact and i % 2 == 1
        q = randn_f16(rng, (t, hq, d))
        kn, vn = _dev(k[base:base + t], gpu), _dev(v[base:base + t], gpu)
        fresh.append(kn, vn, base_position=base)
        if fused:
            got, _ = m.suffix_attention(cache, _dev(q, gpu), base, k_new=kn, v_new=vn, workspace=ws,
                                        tiles_current=True)
        else:
            cache.append(kn, vn, base_position=base)
            got, _ = m.suffix_attention(cache, _dev(q, gpu), base, workspace=ws, tiles_current=True, exact=ex)
        ref, _ = m.suffix_attention(fresh, _dev(q, gpu), base, exact=ex)
        torch.cuda.synchronize()
        if not ex:
            assert torch.equal(got, ref), (base, t, (got - ref).abs().max().item())
        expect = oracle.suffix_attention_q8(q.astype(np.float32), kc[:, :base + t], ks[:, :base + t],
                                            vc[:, :base + t], vs[:, :base + t], base, hq, 1 / math.sqrt(d))
        assert_attention_close(got.cpu().numpy(), expect, f"chunk at {base}")
        assert_attention_close(ref.cpu().numpy(), expect, f"fresh chunk at {base}")
        base += t


def test_suffix_chunked_prefill_current_tiles_graph(gpu):
    """The reference's pipeline shape: one captured suffix step (paged cache, positions
    from a device prefill state, current tiles) replayed for successive 64-token chunks,
    the last one shorter on the device; every replay checked against the oracle."""
    import miinfer_amd as m
    rng = np.random.default_rng(5)
    hq, hk, d, pt, t = 24, 4, 256, 256, 64
    npages = 4
    table = _dev(rng.permutation(npages + 3)[:npages].astype(np.int32).reshape(1, npages), gpu)
    cache = m.KvCache.paged_cache(hk, d, npages + 3, table, page_tokens=pt)
    total = 5 * t
    k = randn_f16(rng, (total, hk, d))
    v = randn_f16(rng, (total, hk, d))
    kc, ks = oracle.quantize_rows(k.transpose(1, 0, 2))
    vc, vs = oracle.quantize_rows(v.transpose(1, 0, 2))
    k_in = torch.zeros((t, hk, d), dtype=torch.float16, device=gpu)
    v_in = torch.zeros_like(k_in)
    q_in = torch.zeros((t, hq, d), dtype=torch.float16, device=gpu)
    out = torch.zeros((t, hq, d), dtype=torch.float32, device=gpu)
    ps = m.make_prefill_state(0, t, device=gpu)
    ws = torch.empty(m.suffix_workspace_bytes(cache, hq, t), dtype=torch.uint8, device=gpu)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.graph(g, stream=s):
        m.suffix_attention(cache, q_in, 0, prefill_state=ps, out=out, workspace=ws, k_new=k_in, v_new=v_in,
                           tiles_current=True)
    torch.cuda.synchronize()
    base = 0
    for n in (t, t, t, t, 37):
        q = randn_f16(rng, (t, hq, d))
        k_in.copy_(_dev(np.pad(k[base:base + n], ((0, t - n), (0, 0), (0, 0))), gpu))
        v_in.copy_(_dev(np.pad(v[base:base + n], ((0, t - n), (0, 0), (0, 0))), gpu))
        q_in.copy_(_dev(q, gpu))
        ps[0] = base
        ps[1] = n
        ps[2] = base + n
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        expect = oracle.suffix_attention_q8(q[:n].astype(np.float32), kc[:, :base + n], ks[:, :base + n],
                                            vc[:, :base + n], vs[:, :base + n], base, hq, 1 / math.sqrt(d))
        assert_attention_close(out[:n].cpu().numpy(), expect, f"replay at {base}")
        base += n


def test_suffix_mfma_path_rounds_fp32_query_to_fp16(gpu):
    """The MFMA path's query operand is fp16: an fp32 query gives exactly the result of
    the same query rounded to fp16 (a documented contract: the lo parts would need a
    second fragment set, 64 more registers per wave than two waves per SIMD leave).
    Short suffixes on the decode route keep the lo parts (they differ)."""
    import miinfer_amd as m
    hq, hk, d, prefix = 24, 4, 256, 1500
    for t, mfma in ((96, True), (4, False)):
        rng = np.random.default_rng(t)
        cache, ref = _setup(gpu, rng, hq, hk, d, prefix, t, ((prefix + t + 63) // 64) * 64)
        q32 = rng.standard_normal((t, hq, d)).astype(np.float32)
        o32, _ = m.suffix_attention(cache, _dev(q32, gpu), prefix, out=torch.empty((t, hq, d), device=gpu))
        o16, _ = m.suffix_attention(cache, _dev(q32.astype(np.float16), gpu), prefix,
                                    out=torch.empty((t, hq, d), device=gpu))
        torch.cuda.synchronize()
        o32, o16 = o32.cpu().numpy(), o16.cpu().numpy()
        assert np.array_equal(o32, o16) == mfma, t
        assert_attention_close(o32, oracle.suffix_attention_q8(q32, *ref, prefix, hq, 1 / math.sqrt(d)), "fp32 q")


@pytest.mark.parametrize("f32", [True, False])
def test_suffix_mfma_accuracy_contract(gpu, f32):
    """The MFMA route's stated accuracy (include/miikv.h, miikv_suffix_attn): its operands
    are fp16 (the query rounded once, each tile element code * scale rounded once), which
    keeps outputs within the attention tolerance (max-abs 2e-3, relative 1e-2) for logits
    of standard deviation up to 2, and within max-abs 1.5e-2 and relative 2e-3 at standard
    deviation 6; at that sharpness MIIKV_SUFFIX_EXACT is the route within the tolerance
    (test_suffix_exact_route).  Measured here with queries x1 and x3 at scale 2/sqrt(D)."""
    import miinfer_amd as m
    from tests.helpers import attention_errors
    hq, hk, d, prefix, t = 24, 4, 256, 3000, 256
    rng = np.random.default_rng(91 + f32)
    cache, ref = _setup(gpu, rng, hq, hk, d, prefix, t, ((prefix + t + 63) // 64) * 64)
    scale = 2 / math.sqrt(d)
    base = rng.standard_normal((t, hq, d))
    for mult, atol, rtol in ((1.0, 2e-3, 1e-2), (3.0, 1.5e-2, 2e-3)):
        q = (base * mult).astype(np.float32 if f32 else np.float16)
        out, _ = m.suffix_attention(cache, _dev(q, gpu), prefix, scale, out=torch.empty((t, hq, d), device=gpu))
        torch.cuda.synchronize()
        expect = oracle.suffix_attention_q8(q.astype(np.float32), *ref, prefix, hq, scale)
        logits_sd = float(np.std(q[:, :6].astype(np.float32).reshape(-1, d) @
                                 (ref[0][0, :512].astype(np.float32) *
                                  np.repeat(ref[1][0, :512].view(np.float16).astype(np.float32), 32, axis=1)).T) * scale)
        max_abs, rel = attention_errors(out.cpu().numpy(), expect)
        assert max_abs <= atol and rel <= rtol, (mult, logits_sd, max_abs, rel)
        assert abs(logits_sd - 2 * mult) < 0.3 * mult, logits_sd


# (t, q fp32, fused store + gate, device prefill state)
@pytest.mark.parametrize("t,f32,fused,dev_state", [(96, True, False, False), (512, True, False, False),
                                                   (100, True, True, False), (70, False, False, True),
                                                   (7, True, False, False)])
def test_suffix_exact_route(gpu, t, f32, fused, dev_state):
    """MIIKV_SUFFIX_EXACT runs every token as a decode: the fp32 query's low half and
    the block scales in fp32 keep sharp attention (queries x3, scale x2, logits of
    standard deviation ~6) within the attention tolerance, where the MFMA path's fp16
    query and tiles do not; with the fused store, a gate and a device prefill state."""
    import miinfer_amd as m
    hq, hk, d, prefix = 24, 4, 256, 1500
    rng = np.random.default_rng(t + 3 * fused)
    cap = ((prefix + t + 255) // 256) * 256
    k = randn_f16(rng, (prefix + t, hk, d))
    v = randn_f16(rng, (prefix + t, hk, d))
    kc, ks = oracle.quantize_rows(k.transpose(1, 0, 2))
    vc, vs = oracle.quantize_rows(v.transpose(1, 0, 2))
    cache = m.KvCache.contiguous(hk, d, cap)
    cache.append(_dev(k[:prefix], gpu), _dev(v[:prefix], gpu), base_position=0)
    kn, vn = _dev(k[prefix:], gpu), _dev(v[prefix:], gpu)
    if not fused:
        cache.append(kn, vn, base_position=prefix)
    q = (rng.standard_normal((t, hq, d)) * 3).astype(np.float32 if f32 else np.float16)
    gate = rng.standard_normal((t, hq, d)).astype(np.float32)
    scale = 2 / math.sqrt(d)
    ps = m.make_prefill_state(prefix, t, cap, device=gpu) if dev_state else None
    kw = dict(k_new=kn, v_new=vn) if fused else {}
    out, gated = m.suffix_attention(cache, _dev(q, gpu), prefix, scale, prefill_state=ps, gate=_dev(gate, gpu),
                                    out=torch.empty((t, hq, d), device=gpu), exact=True, **kw)
    torch.cuda.synchronize()
    expect = oracle.suffix_attention_q8(q.astype(np.float32), kc, ks, vc, vs, prefix, hq, scale)
    assert_attention_close(out.cpu().numpy(), expect, "exact")
    assert_attention_close(gated.cpu().numpy(), expect / (1 + np.exp(-gate)), "exact gated")
    if fused:  # the rows were stored with the append rule
        got_kc, got_ks, _, _ = cache.export_canonical(0, prefix, t)
        torch.cuda.synchronize()
        assert np.array_equal(got_kc.cpu().numpy(), kc[:, prefix:])
        assert np.array_equal(got_ks.cpu().numpy().view(np.uint16), ks[:, prefix:])


@pytest.mark.parametrize("hq,hk,d,paged", [(32, 8, 128, True), (24, 4, 256, True), (8, 2, 128, False)])
def test_suffix_exact_mfma_kernel_shapes(gpu, hq, hk, d, paged):
    """Long suffixes with MIIKV_SUFFIX_EXACT run the exact-product MFMA kernel (key codes
    exact, block scales in fp32, the query's lo half in the spare columns): sharp
    attention (logits of s.d. ~6) within the tolerance on paged and contiguous caches,
    head_dim 128 and 256, with a gate, split and single-split workspaces."""
    import miinfer_amd as m
    rng = np.random.default_rng(hq + d + paged)
    prefix, t, pt = 1800, 200, 256
    n = prefix + t
    k = randn_f16(rng, (n, hk, d))
    v = randn_f16(rng, (n, hk, d))
    kc, ks = oracle.quantize_rows(k.transpose(1, 0, 2))
    vc, vs = oracle.quantize_rows(v.transpose(1, 0, 2))
    if paged:
        npages = (n + pt - 1) // pt
        table = _dev(rng.permutation(npages + 2)[:npages].astype(np.int32).reshape(1, npages), gpu)
        cache = m.KvCache.paged_cache(hk, d, npages + 2, table, page_tokens=pt)
    else:
        cache = m.KvCache.contiguous(hk, d, ((n + 63) // 64) * 64)
    cache.append(_dev(k, gpu), _dev(v, gpu))
    q = (rng.standard_normal((t, hq, d)) * 3).astype(np.float32)
    gate = rng.standard_normal((t, hq, d)).astype(np.float32)
    scale = 2 / math.sqrt(d)
    expect = oracle.suffix_attention_q8(q, kc, ks, vc, vs, prefix, hq, scale)
    for ws in (None, "tiles"):
        kw = {}
        if ws == "tiles":  # just the exact tiles: one split
            kw["workspace"] = torch.empty(hk * ((n + 31) // 32) * (64 * d + 64 * (d // 32)) * 2, dtype=torch.uint8,
                                          device=gpu)
        out, gated = m.suffix_attention(cache, _dev(q, gpu), prefix, scale, gate=_dev(gate, gpu),
                                        out=torch.empty((t, hq, d), device=gpu), exact=True, **kw)
        torch.cuda.synchronize()
        assert_attention_close(out.cpu().numpy(), expect, f"exact {ws}")
        assert_attention_close(gated.cpu().numpy(), expect / (1 + np.exp(-gate)), f"exact gated {ws}")


def test_suffix_exact_config4_full_size(gpu):
    """Config 4 as bench.py times the exact route: miikv_suffix_append_attn_ex with
    MIIKV_SUFFIX_EXACT stores 512 rows over an 8192-token prefix (24q/4kv/D256) and
    attends with an fp32 query at logits of s.d. ~6 (queries x3, scale x2); two tokens of
    every 32-token block of the suffix, token 511 among them, against the oracle, and the
    stored rows bit-exact."""
    import miinfer_amd as m
    hq, hk, d, prefix, t = 24, 4, 256, 8192, 512
    rng = np.random.default_rng(45)
    cap = prefix + t
    k = randn_f16(rng, (cap, hk, d))
    v = randn_f16(rng, (cap, hk, d))
    cache = m.KvCache.contiguous(hk, d, cap)
    cache.append(_dev(k[:prefix], gpu), _dev(v[:prefix], gpu), base_position=0)
    q = (rng.standard_normal((t, hq, d)) * 3).astype(np.float32)
    scale = 2 / math.sqrt(d)
    out, _ = m.suffix_attention(cache, _dev(q, gpu), prefix, scale, k_new=_dev(k[prefix:], gpu),
                                v_new=_dev(v[prefix:], gpu), exact=True)
    torch.cuda.synchronize()
    kc, ks = oracle.quantize_rows(k.transpose(1, 0, 2))
    vc, vs = oracle.quantize_rows(v.transpose(1, 0, 2))
    got_kc, got_ks, got_vc, got_vs = cache.export_canonical(0, prefix, t)
    torch.cuda.synchronize()
    assert np.array_equal(got_kc.cpu().numpy(), kc[:, prefix:])
    assert np.array_equal(got_vc.cpu().numpy(), vc[:, prefix:])
    out = out.cpu().numpy()
    for tok in sorted({x for b in range(0, t, 32) for x in (b, b + 17)} | {t - 1}):
        expect = oracle.attention_q8(q[tok], kc, ks, vc, vs, prefix + tok + 1, hq, scale)
        assert_attention_close(out[tok], expect, f"exact token {tok}")


def test_suffix_exact_route_errors(gpu):
    import miinfer_amd as m
    from miinfer_amd import _lib
    cache = m.KvCache.contiguous(1, 128, 1024)
    cache.append(_dev(np.zeros((600, 1, 128), np.float16), gpu), _dev(np.zeros((600, 1, 128), np.float16), gpu))
    q = torch.zeros((64, 32, 128), device=gpu)  # 32 query heads per kv head: no decode layout
    with pytest.raises(_lib.MiikvError) as err:
        m.suffix_attention(cache, q, 536, exact=True, workspace=torch.empty(1 << 26, dtype=torch.uint8, device=gpu))
    assert err.value.status == _lib.MIIKV_EUNSUPPORTED
    c4 = m.KvCache.contiguous(4, 256, 1024)
    c4.append(_dev(np.zeros((600, 4, 256), np.float16), gpu), _dev(np.zeros((600, 4, 256), np.float16), gpu))
    # 512 tokens over 88: a workspace of just the context's fp16 tiles runs the MFMA
    # path (one split) but cannot hold the exact route's decode records
    q4 = torch.zeros((512, 24, 256), device=gpu)
    small = torch.empty(4 * ((600 + 31) // 32) * 2 * 256 * 32 * 2, dtype=torch.uint8, device=gpu)
    m.suffix_attention(c4, q4, 88, workspace=small)
    with pytest.raises(_lib.MiikvError) as err:  # never falls back to the MFMA path
        m.suffix_attention(c4, q4, 88, exact=True, workspace=small)
    assert err.value.status == _lib.MIIKV_EWORKSPACE


@pytest.mark.parametrize("seed", range(10))
def test_suffix_random(gpu, seed):
    """Seeded random suffixes: token count (both sides of the decode-route rule),
    prefix, head layout, fused store, MIIKV_SUFFIX_EXACT, query dtype and gate; every
    output against the oracle."""
    import miinfer_amd as m
    rng = np.random.default_rng(2000 + seed)
    hq, hk, d = [(24, 4, 256), (32, 8, 128), (16, 16, 128), (8, 2, 256), (6, 1, 128)][int(rng.integers(0, 5))]
    t = int(rng.choice([1, 2, 3, 5, 8, 16, 33, 64, 65, 130, 300]))
    prefix = int(rng.integers(0, 3000))
    fused = bool(rng.integers(0, 2))
    exact = bool(rng.integers(0, 2))
    f32 = bool(rng.integers(0, 2))
    cap = ((prefix + t + 63) // 64) * 64
    k = randn_f16(rng, (prefix + t, hk, d))
    v = randn_f16(rng, (prefix + t, hk, d))
    kc, ks = oracle.quantize_rows(k.transpose(1, 0, 2))
    vc, vs = oracle.quantize_rows(v.transpose(1, 0, 2))
    cache = m.KvCache.contiguous(hk, d, cap)
    if prefix:
        cache.append(_dev(k[:prefix], gpu), _dev(v[:prefix], gpu), base_position=0)
    kn, vn = _dev(k[prefix:], gpu), _dev(v[prefix:], gpu)
    if not fused:
        cache.append(kn, vn, base_position=prefix)
    q = rng.standard_normal((t, hq, d)).astype(np.float32) if f32 else randn_f16(rng, (t, hq, d))
    gate = rng.standard_normal((t, hq, d)).astype(np.float32) if rng.integers(0, 2) else None
    kw = dict(k_new=kn, v_new=vn) if fused else {}
    out, gated = m.suffix_attention(cache, _dev(q, gpu), prefix, gate=None if gate is None else _dev(gate, gpu),
                                    out=torch.empty((t, hq, d), device=gpu), exact=exact, **kw)
    torch.cuda.synchronize()
    what = f"seed {seed}: {hq}q/{hk}kv/D{d} T={t} P={prefix} fused={fused} exact={exact} f32={f32}"
    expect = oracle.suffix_attention_q8(q.astype(np.float32), kc, ks, vc, vs, prefix, hq, 1 / math.sqrt(d))
    assert_attention_close(out.cpu().numpy(), expect, what)
    if gate is not None:
        assert_attention_close(gated.cpu().numpy(), expect / (1 + np.exp(-gate)), what + " gated")
