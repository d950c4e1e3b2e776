"""miikv_decode_append_attn_noalloc (GPU): the same bytes and results as
miikv_decode_append_attn with a caller workspace, on two calls in a row (the
second smaller), for a single sequence and a paged batch; and the size limit."""
import ctypes
import math

import numpy as np
import pytest
import torch

from tests.helpers import randn_f16

pytestmark = pytest.mark.gpu


def _dev(a, gpu):
    return torch.from_numpy(np.ascontiguousarray(a)).to(gpu)


def _run(cache, kn, vn, q, lens, max_ctx, noalloc, gpu, gate=None, sync=True):
    import miinfer_amd as m
    from miinfer_amd import _lib
    L = _lib.lib()
    P = ctypes.c_void_p
    batch, hq, d = q.shape
    out = torch.full((batch, hq, d), float("nan"), device=gpu)
    gated = torch.full((batch, hq, d), float("nan"), device=gpu) if gate is not None else None
    q81 = torch.zeros(batch * hq * d // 32 * 36, dtype=torch.uint8, device=gpu) if gate is not None else None
    s = P(torch.cuda.current_stream().cuda_stream)
    args = (cache.view, P(kn.data_ptr()), P(vn.data_ptr()), P(q.data_ptr()), _lib.DTYPE_F16, hq,
            ctypes.c_float(1 / math.sqrt(d)), batch, P(lens.data_ptr()), None, max_ctx, P(out.data_ptr()),
            P(gate.data_ptr()) if gate is not None else None,
            P(gated.data_ptr()) if gated is not None else None,
            P(q81.data_ptr()) if q81 is not None else None)
    if noalloc:
        st = L.miikv_decode_append_attn_noalloc(*args, s)
    else:
        ws = m.DecodeWorkspace(cache, hq, batch, max_ctx)
        st = L.miikv_decode_append_attn(*args, P(ws.buf.data_ptr()), ws.bytes, s)
    assert st == 0, st
    if sync:
        torch.cuda.synchronize()
    return out, gated, q81


def _contiguous_case(gpu, rng, hq, hk, d, length, cap):
    import miinfer_amd as m
    k = randn_f16(rng, (length, hk, d))
    v = randn_f16(rng, (length, hk, d))
    caches = []
    for _ in range(2):
        c = m.KvCache.contiguous(hk, d, cap)
        if length > 1:
            c.append(_dev(k[:-1], gpu), _dev(v[:-1], gpu))
        caches.append(c)
    q = _dev(randn_f16(rng, (1, hq, d)), gpu)
    lens = torch.tensor([length], dtype=torch.int32, device=gpu)
    return caches, _dev(k[-1:], gpu), _dev(v[-1:], gpu), q, lens


def test_noalloc_matches_workspace_entry_point(gpu):
    rng = np.random.default_rng(5)
    gate = None
    for length, cap in ((32768, 32768), (3000, 4096)):  # second call smaller
        caches, kn, vn, q, lens = _contiguous_case(gpu, rng, 32, 8, 128, length, cap)
        gate = _dev(rng.standard_normal((1, 32, 128)).astype(np.float32), gpu)
        a = _run(caches[0], kn, vn, q, lens, cap, False, gpu, gate)
        b = _run(caches[1], kn, vn, q, lens, cap, True, gpu, gate)
        for x, y in zip(a, b):
            assert torch.equal(x, y), f"L={length}"
        ea, eb = caches[0].export_canonical(0, 0, length), caches[1].export_canonical(0, 0, length)
        for x, y in zip(ea, eb):
            assert torch.equal(x, y)


def test_noalloc_paged_batch(gpu):
    import miinfer_amd as m
    rng = np.random.default_rng(6)
    hq, hk, d, pt = 24, 4, 256, 256
    for lens_l in ([300, 5000, 20000, 1], [700, 256]):  # second call smaller
        pages = [(n + pt - 1) // pt for n in lens_l]
        stride, total = max(pages), sum(pages)
        perm = rng.permutation(total).astype(np.int32)
        table = np.zeros((len(lens_l), stride), np.int32)
        o = 0
        for s_, p_ in enumerate(pages):
            table[s_, :p_] = perm[o:o + p_]
            o += p_
        caches = [m.KvCache.paged_cache(hk, d, total, _dev(table, gpu), page_tokens=pt) for _ in range(2)]
        kn = _dev(randn_f16(rng, (len(lens_l), hk, d)), gpu)
        vn = _dev(randn_f16(rng, (len(lens_l), hk, d)), gpu)
        for s_, n in enumerate(lens_l):
            if n > 1:
                k = _dev(randn_f16(rng, (n - 1, hk, d)), gpu)
                v = _dev(randn_f16(rng, (n - 1, hk, d)), gpu)
                for c in caches:
                    c.append(k, v, base_position=0, seq=s_)
        q = _dev(randn_f16(rng, (len(lens_l), hq, d)), gpu)
        lens = _dev(np.array(lens_l, np.int32), gpu)
        a = _run(caches[0], kn, vn, q, lens, stride * pt, False, gpu)
        b = _run(caches[1], kn, vn, q, lens, stride * pt, True, gpu)
        assert torch.equal(a[0], b[0]), f"lens={lens_l}"
        # the fused append wrote the same bytes into each sequence's pages
        for s_, n in enumerate(lens_l):
            ea, eb = caches[0].export_canonical(s_, 0, n), caches[1].export_canonical(s_, 0, n)
            for x, y in zip(ea, eb):
                assert torch.equal(x, y), f"lens={lens_l} seq={s_}"


def test_noalloc_rejects_geometry_beyond_scratch(gpu):
    import miinfer_amd as m
    from miinfer_amd import _lib
    L = _lib.lib()
    hq, hk, d, pt, batch = 24, 4, 256, 256, 64
    table = torch.zeros((batch, 512), dtype=torch.int32, device=gpu)
    cache = m.KvCache.paged_cache(hk, d, 1, table, page_tokens=pt)
    assert L.miikv_decode_workspace_bytes(cache.view, hq, batch, 512 * pt) > L.miikv_decode_scratch_max_bytes()
    q = torch.zeros((batch, hq, d), dtype=torch.float16, device=gpu)
    kn = torch.zeros((batch, hk, d), dtype=torch.float16, device=gpu)
    lens = torch.ones(batch, dtype=torch.int32, device=gpu)
    out = torch.empty((batch, hq, d), device=gpu)
    P = ctypes.c_void_p
    st = L.miikv_decode_append_attn_noalloc(cache.view, P(kn.data_ptr()), P(kn.data_ptr()), P(q.data_ptr()),
                                            _lib.DTYPE_F16, hq, ctypes.c_float(0.0625), batch,
                                            P(lens.data_ptr()), None, 512 * pt, P(out.data_ptr()), None, None,
                                            None, None)
    assert st == _lib.MIIKV_EWORKSPACE


def test_noalloc_calls_on_two_streams_are_ordered(gpu):
    """Two calls on two streams, enqueued back to back without a host sync: the
    second waits for the first's kernels (they share the scratch array), so both
    match the workspace entry point."""
    rng = np.random.default_rng(17)
    big = _contiguous_case(gpu, rng, 32, 8, 128, 32768, 32768)
    small = _contiguous_case(gpu, rng, 32, 8, 128, 2000, 4096)
    want_big = _run(big[0][0], *big[1:], 32768, False, gpu)
    want_small = _run(small[0][0], *small[1:], 4096, False, gpu)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    for _ in range(3):
        with torch.cuda.stream(s1):
            got_big = _run(big[0][1], *big[1:], 32768, True, gpu, sync=False)
        with torch.cuda.stream(s2):
            got_small = _run(small[0][1], *small[1:], 4096, True, gpu, sync=False)
        torch.cuda.synchronize()
        assert torch.equal(got_big[0], want_big[0])
        assert torch.equal(got_small[0], want_small[0])
