"""Prefix-state reuse primitives: page copies, segment copies and state clones are
byte-identical to their sources (GPU)."""
import numpy as np
import pytest
import torch

from tests.helpers import randn_f16

pytestmark = pytest.mark.gpu


def test_copy_pages_byte_identical(gpu):
    import miinfer_amd as m
    rng = np.random.default_rng(1)
    hk, d, pt, npages = 4, 256, 256, 10
    table = torch.arange(npages, dtype=torch.int32, device=gpu).reshape(1, npages)
    cache = m.KvCache.paged_cache(hk, d, npages, table, page_tokens=pt)
    for t in (cache.k_codes, cache.v_codes, cache.k_scales, cache.v_scales):
        t.copy_(torch.from_numpy(rng.integers(-100, 100, t.numel()).astype(
            t.cpu().numpy().dtype)).to(gpu))
    before = [t.clone() for t in (cache.k_codes, cache.v_codes, cache.k_scales, cache.v_scales)]
    src = torch.tensor([0, 3, 7], dtype=torch.int32, device=gpu)
    dst = torch.tensor([9, 1, 2], dtype=torch.int32, device=gpu)
    cache.copy_pages(src, dst)
    torch.cuda.synchronize()
    for b, a in zip(before, (cache.k_codes, cache.v_codes, cache.k_scales, cache.v_scales)):
        per = b.numel() // npages
        bv, av = b.view(npages, per), a.view(npages, per)
        for s_, d_ in ((0, 9), (3, 1), (7, 2)):
            assert torch.equal(av[d_], bv[s_])
        for p in (0, 3, 4, 5, 6, 7, 8):  # untouched pages
            assert torch.equal(av[p], bv[p])


def test_clone_state_byte_identical(gpu):
    import miinfer_amd as m
    nbytes = 16 * 128 * 128 * 4 + 8192 * 3 * 4  # one GDN layer of the fork config
    src = torch.randint(-2**31, 2**31 - 1, (nbytes // 4,), dtype=torch.int32, device=gpu)
    dsts = [torch.zeros_like(src) for _ in range(8)]
    m.clone_state(dsts, src)
    for d in dsts:
        assert torch.equal(d, src)


def test_copy_segments_aligned_and_ragged(gpu):
    import miinfer_amd as m
    rng = np.random.default_rng(3)
    sizes = [1 << 20, 4096, 77, 16, 1, 100_003]
    srcs = [torch.from_numpy(rng.integers(0, 255, s, dtype=np.uint8)).to(gpu) for s in sizes]
    dsts = [torch.zeros(s + 3, dtype=torch.uint8, device=gpu) for s in sizes]
    segs = []
    for i, (s, d) in enumerate(zip(srcs, dsts)):
        off = 0 if i < 3 else 1  # some unaligned destinations
        segs.append((d.data_ptr() + off, s.data_ptr(), s.numel()))
    m.copy_segments(segs)
    for i, (s, d) in enumerate(zip(srcs, dsts)):
        off = 0 if i < 3 else 1
        assert torch.equal(d[off:off + s.numel()], s)
        assert not d[:off].any() and not d[off + s.numel():].any()


def test_registry_fork_restore_and_decode(gpu):
    """Two prefixes saved from one session into the registry (the session keeps
    appending after the first save: the shared partial page is copied on write, so the
    first entry's keys stay intact), the session released, then sessions forked from
    each entry: longest-prefix lookup, recurrent state restored byte for byte, and
    decode attention over the forked rows against the oracle."""
    import math

    import miinfer_amd as m
    import oracle
    from miinfer_amd import reuse
    from tests.helpers import assert_attention_close, randn_f16
    rng = np.random.default_rng(99)
    hq, hk, d, pt, stride = 24, 4, 256, 256, 8
    pool = reuse.PagePool(40)
    reg = reuse.PrefixRegistry(pool, pt, 4, "m", "q")
    table = np.full((3, stride), -1, np.int32)
    cache = m.KvCache.paged_cache(hk, d, 40, torch.from_numpy(table.clip(0)).to(gpu), page_tokens=pt)
    k = randn_f16(rng, (1500, hk, d))
    v = randn_f16(rng, (1500, hk, d))
    toks = np.arange(1500, dtype=np.uint32) * 7 + 3
    st = reuse.RecurrentStates(4, 1000, 96, device=gpu)
    # session 1: 700 tokens, save A, then 800 more (prepare_append un-shares the
    # partial page A holds), save B
    row = table[0]
    for pos in range(0, 700):
        if pos % pt == 0:
            pool.prepare_append(row, pos, pt)
    cache.set_block_table(torch.from_numpy(table.clip(0)).to(gpu))
    cache.append(torch.from_numpy(k[:700]).to(gpu), torch.from_numpy(v[:700]).to(gpu), base_position=0, seq=0)
    st.buf.copy_(torch.randn(st.buf.numel(), device=gpu))
    ea = reg.save(toks[:700], row, st)
    state_a = st.buf.clone()
    copies = []
    for pos in range(700, 1500):
        if pos % pt == 0 or pos == 700:
            copies += pool.prepare_append(row, pos, pt)
    assert len(copies) == 1  # the partial page shared with entry A
    reuse.run_page_copies(cache, copies)
    cache.set_block_table(torch.from_numpy(table.clip(0)).to(gpu))
    cache.append(torch.from_numpy(k[700:]).to(gpu), torch.from_numpy(v[700:]).to(gpu), base_position=700, seq=0)
    st.buf.add_(1.0)
    eb = reg.save(toks, row, st)
    state_b = st.buf.clone()
    pool.release(row, 1500, pt)
    table[0] = -1
    # forks: B for a prompt extending B, A for a prompt that diverges after A
    res, e1, n1 = reg.lookup(np.concatenate([toks, [1, 2]]))
    assert (res, e1, n1) == (reuse.MatchResult.EXACT_MATCH, eb, 1500)
    res, e2, n2 = reg.lookup(np.concatenate([toks[:700], [5]]))
    assert (res, e2, n2) == (reuse.MatchResult.EXACT_MATCH, ea, 700)
    s1 = reuse.RecurrentStates(4, 1000, 96, device=gpu)
    s2 = reuse.RecurrentStates(4, 1000, 96, device=gpu)
    table[1], c1 = reg.fork(e1, stride, s1)
    table[2], c2 = reg.fork(e2, stride, s2)
    reuse.run_page_copies(cache, c1 + c2)
    torch.cuda.synchronize()
    assert torch.equal(s1.buf.view(torch.int32), state_b.view(torch.int32)) and s1.position == 1500
    assert torch.equal(s2.buf.view(torch.int32), state_a.view(torch.int32)) and s2.position == 700
    cache.set_block_table(torch.from_numpy(table[1:].clip(0)).to(gpu))
    q = randn_f16(rng, (2, hq, d))
    out, _ = m.decode_attention(cache, torch.from_numpy(q).to(gpu),
                                lengths=torch.tensor([1500, 700], dtype=torch.int32, device=gpu),
                                max_context=stride * pt)
    out = out.cpu().numpy()
    kc, ks = oracle.quantize_rows(k.transpose(1, 0, 2))
    vc, vs = oracle.quantize_rows(v.transpose(1, 0, 2))
    for j, n in enumerate((1500, 700)):
        expect = oracle.attention_q8(q[j].astype(np.float32), kc, ks, vc, vs, n, hq, 1 / math.sqrt(d))
        assert_attention_close(out[j], expect, f"fork of the {n}-token entry")
