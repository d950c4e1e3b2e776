"""Forked sessions over a shared paged prefix (GPU): copy-on-write of the last partial
page, byte-identical sharing, divergent appends that leave the parent untouched, and
recurrent-state clone / checkpoint / restore — all byte-exact."""
import math

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import assert_attention_close, randn_f16

pytestmark = pytest.mark.gpu


def _dev(a, gpu):
    return torch.from_numpy(np.ascontiguousarray(a)).to(gpu)


def _export(cache, seq, n):
    return [t.cpu().numpy() for t in cache.export_canonical(seq, 0, n)]


@pytest.mark.parametrize("prefix", [1000, 1024])
def test_fork_cow_and_divergent_appends(gpu, prefix):
    import miinfer_amd as m
    from miinfer_amd import reuse
    rng = np.random.default_rng(prefix)
    hq, hk, d, pt, nchild, extra = 24, 4, 256, 256, 3, 50
    npool = 40
    stride = (prefix + extra + pt - 1) // pt + 1
    pool = reuse.PagePool(npool)
    table = np.full((1 + nchild, stride), 0, np.int32)
    pages = (prefix + pt - 1) // pt
    table[0, :pages] = [pool.alloc() for _ in range(pages)]
    cache = m.KvCache.paged_cache(hk, d, npool, _dev(table, gpu), page_tokens=pt)
    kp = randn_f16(rng, (prefix, hk, d))
    vp = randn_f16(rng, (prefix, hk, d))
    cache.append(_dev(kp, gpu), _dev(vp, gpu), base_position=0, seq=0)
    parent_before = _export(cache, 0, prefix)

    copies = []
    for c in range(1, 1 + nchild):
        child, cp = pool.fork(table[0], prefix, pt)
        table[c] = child
        copies += cp
    reuse.run_page_copies(cache, copies)
    # children append `extra` divergent tokens each: make the receiving pages writable
    kids = {}
    for c in range(1, 1 + nchild):
        row = table[c].copy()
        cps = []
        for pos in range(prefix, prefix + extra):
            if pos % pt == 0 or pos == prefix:
                cps += pool.prepare_append(row, pos, pt)
        table[c] = row
        reuse.run_page_copies(cache, cps)
        kids[c] = (randn_f16(rng, (extra, hk, d)), randn_f16(rng, (extra, hk, d)))
    cache.set_block_table(_dev(table, gpu))
    for c, (k, v) in kids.items():
        cache.append(_dev(k, gpu), _dev(v, gpu), base_position=prefix, seq=c)
    torch.cuda.synchronize()

    # the parent is untouched and every child sees the parent's prefix byte for byte
    parent_after = _export(cache, 0, prefix)
    for a, b in zip(parent_before, parent_after):
        assert np.array_equal(a, b)
    for c in kids:
        got = _export(cache, c, prefix)
        for a, b in zip(parent_before, got):
            assert np.array_equal(a, b)
    # shared full pages are physically the same; the partial page was copied
    full = prefix // pt
    assert all((table[1:, :full] == table[0, :full]).ravel())
    if prefix % pt:
        assert len(set(table[:, full])) == 1 + nchild
    # each child attends over prefix + its own suffix
    q = randn_f16(rng, (1 + nchild, hq, d))
    lens = np.array([prefix] + [prefix + extra] * nchild, np.int32)
    out, _ = m.decode_attention(cache, _dev(q, gpu), lengths=_dev(lens, gpu),
                                max_context=stride * pt)
    out = out.cpu().numpy()
    for c in range(1 + nchild):
        k = kp if c == 0 else np.concatenate([kp, kids[c][0]])
        v = vp if c == 0 else np.concatenate([vp, kids[c][1]])
        kc, ks = oracle.quantize_rows(k.transpose(1, 0, 2))
        vc, vs = oracle.quantize_rows(v.transpose(1, 0, 2))
        expect = oracle.attention_q8(q[c].astype(np.float32), kc, ks, vc, vs, int(lens[c]), hq,
                                     1 / math.sqrt(d))
        assert_attention_close(out[c], expect, f"session {c}")


def test_recurrent_state_clone_checkpoint_restore(gpu):
    from miinfer_amd import reuse
    layers, state, conv = 48, 16 * 128 * 128, 8192 * 3  # the fork config's GDN geometry
    src = reuse.RecurrentStates(layers, state, conv, device=gpu)
    src.buf.copy_(torch.randn(src.buf.numel(), device=gpu))
    src.position = 32768
    kids = [reuse.RecurrentStates(layers, state, conv, device=gpu) for _ in range(4)]
    reuse.clone_states(src, kids)
    for k in kids:
        assert torch.equal(k.buf.view(torch.int32), src.buf.view(torch.int32))
        assert k.position == 32768
    ctx = reuse.PrefixContext("m", "q")
    ctx.save(np.arange(100, dtype=np.uint32), src)
    saved = src.buf.clone()
    src.buf.add_(1.0)
    src.position = 5
    ctx.restore(src)
    assert torch.equal(src.buf.view(torch.int32), saved.view(torch.int32))
    assert src.position == 100
