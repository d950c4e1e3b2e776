"""Config 5 at full shape (GPU): 64 sessions forked from a 32768-token prefix (last
page full) and a 32668-token prefix (last page partial) of a hybrid model with 16
attention layers (4 kv heads x D256 q8_0, 256-token pages) and 48 GDN layers (fp32
state 16x128x128 + conv 8192x3).  Checks, all on the device where the data is large:
every child's block table shares the parent's full pages, the copy-on-write copies of
the partial page equal the parent's page byte for byte, every cloned recurrent state
equals the parent's, divergent appends leave the parent untouched, and decode
attention of forked children matches the oracle."""
import math

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import assert_attention_close, randn_f16

pytestmark = pytest.mark.gpu

HQ, HKV, D, PT, LAYERS, FORKS = 24, 4, 256, 256, 16, 64
GDN_LAYERS, STATE, CONV = 48, 16 * 128 * 128, 8192 * 3


def _dev(a, gpu):
    return torch.from_numpy(np.ascontiguousarray(a)).to(gpu)


def _planes(cache, npool):
    return [t.view(torch.uint8).view(npool, -1) for t in
            (cache.k_codes, cache.k_scales, cache.v_codes, cache.v_scales)]


@pytest.mark.parametrize("prefix", [32768, 32768 - 100])
def test_fork_config5_full_shape(gpu, prefix):
    import miinfer_amd as m
    from miinfer_amd import reuse
    print(f"config 5: prefix={prefix} forks={FORKS} layers={LAYERS}+{GDN_LAYERS}", flush=True)
    rng = np.random.default_rng(prefix)
    pages = (prefix + PT - 1) // PT
    npool = pages + 2 * FORKS + 1
    stride = pages + 1
    caches, pools, rows = [], [], []
    gen = torch.Generator(device=gpu)
    gen.manual_seed(prefix)
    for li in range(LAYERS):
        pool = reuse.PagePool(npool)
        row = np.full(stride, -1, np.int32)
        row[:pages] = [pool.alloc() for _ in range(pages)]
        cache = m.KvCache.paged_cache(HKV, D, npool, _dev(row[None].clip(0), gpu), page_tokens=PT)
        if li == 0:  # layer 0 holds real keys and values for the attention check
            kp = randn_f16(rng, (prefix, HKV, D))
            vp = randn_f16(rng, (prefix, HKV, D))
            cache.append(_dev(kp, gpu), _dev(vp, gpu), base_position=0, seq=0)
        else:  # the others: arbitrary bytes (the checks are byte identity)
            for t in _planes(cache, npool):
                t.copy_(torch.randint(0, 256, t.shape, dtype=torch.uint8, device=gpu, generator=gen))
        caches.append(cache)
        pools.append(pool)
        rows.append(row)
    parent = reuse.RecurrentStates(GDN_LAYERS, STATE, CONV, device=gpu)
    parent.buf.copy_(torch.randn(parent.buf.numel(), device=gpu, generator=gen))
    parent.position = prefix
    before = [[p.clone() for p in _planes(c, npool)] for c in caches[:2]]

    # fork: block tables share every full page, the partial page is copied (CoW)
    kids_rows = []
    for li in range(LAYERS):
        child_rows, copies = pools[li].fork_many(rows[li], prefix, PT, FORKS)
        kids_rows.append(child_rows)
        full = prefix // PT
        assert (child_rows[:, :full] == rows[li][:full]).all()
        if prefix % PT:
            assert len(copies) == FORKS
            assert all(s == rows[li][full] for s, _ in copies)
            assert len({d for _, d in copies} | {rows[li][full]}) == FORKS + 1
            assert (child_rows[:, full] == [d for _, d in copies]).all()
        else:
            assert copies == []
        reuse.run_page_copies(caches[li], copies)
    kids = [reuse.RecurrentStates(GDN_LAYERS, STATE, CONV, device=gpu) for _ in range(FORKS)]
    reuse.clone_states(parent, kids)
    torch.cuda.synchronize()

    # byte identity on the device: copied pages and cloned states
    if prefix % PT:
        full = prefix // PT
        for li in range(LAYERS):
            planes = _planes(caches[li], npool)
            dst = torch.from_numpy(kids_rows[li][:, full].astype(np.int64)).to(gpu)
            for t in planes:
                assert torch.equal(t[dst], t[rows[li][full]].expand(FORKS, -1)), f"layer {li}"
    pv = parent.buf.view(torch.int32)
    for i, k in enumerate(kids):
        assert torch.equal(k.buf.view(torch.int32), pv), f"state clone {i}"
        assert k.position == prefix

    # divergent appends by four children of layer 0 (page-boundary or partial-page
    # position), then attention of those children against the oracle
    chosen = [0, 17, 40, 63]
    table = np.full((1 + len(chosen), stride), 0, np.int32)
    table[0] = rows[0].clip(0)
    new_k, new_v = {}, {}
    for j, c in enumerate(chosen):
        row = kids_rows[0][c].copy()
        cps = pools[0].prepare_append(row, prefix, PT)
        reuse.run_page_copies(caches[0], cps)
        table[1 + j] = row.clip(0)
        new_k[c] = randn_f16(rng, (1, HKV, D))
        new_v[c] = randn_f16(rng, (1, HKV, D))
    caches[0].set_block_table(_dev(table, gpu))
    for j, c in enumerate(chosen):
        caches[0].append(_dev(new_k[c], gpu), _dev(new_v[c], gpu), base_position=prefix, seq=1 + j)
    torch.cuda.synchronize()
    # the parent's pages are untouched (layer 0 took the appends, layer 1 only forks)
    for li, b in enumerate(before):
        par = torch.from_numpy(rows[li][:pages].astype(np.int64)).to(gpu)
        for t, t0 in zip(_planes(caches[li], npool), b):
            assert torch.equal(t[par], t0[par]), f"parent pages of layer {li}"
    q = randn_f16(rng, (1 + len(chosen), HQ, D))
    lens = np.array([prefix] + [prefix + 1] * len(chosen), np.int32)
    out, _ = m.decode_attention(caches[0], _dev(q, gpu), lengths=_dev(lens, gpu),
                                max_context=stride * PT)
    out = out.cpu().numpy()
    kc0, ks0 = oracle.quantize_rows(kp.transpose(1, 0, 2))
    vc0, vs0 = oracle.quantize_rows(vp.transpose(1, 0, 2))
    expect = oracle.attention_q8(q[0].astype(np.float32), kc0, ks0, vc0, vs0, prefix, HQ, 1 / math.sqrt(D))
    assert_attention_close(out[0], expect, "parent")
    for j, c in enumerate(chosen):
        kc1, ks1 = oracle.quantize_rows(new_k[c].transpose(1, 0, 2))
        vc1, vs1 = oracle.quantize_rows(new_v[c].transpose(1, 0, 2))
        expect = oracle.attention_q8(q[1 + j].astype(np.float32), np.concatenate([kc0, kc1], 1),
                                     np.concatenate([ks0, ks1], 1), np.concatenate([vc0, vc1], 1),
                                     np.concatenate([vs0, vs1], 1), prefix + 1, HQ, 1 / math.sqrt(D))
        assert_attention_close(out[1 + j], expect, f"child {c}")
