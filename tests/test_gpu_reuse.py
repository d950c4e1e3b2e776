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
