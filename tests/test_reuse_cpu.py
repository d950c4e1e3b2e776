"""Prefix-reuse host policy in libmiikv (no GPU): page pool, copy-on-write fork
planning, and ReusableContext's fingerprint / match precedence."""
import numpy as np
import pytest

import oracle


def _m():
    import torch  # noqa: F401

    from miinfer_amd import reuse
    return reuse


def _prompt(count, seed):
    # the synthetic prompt generator of bench/prefix_state_reuse_bench.cpp:60-68
    out, val = [], seed
    for _ in range(count):
        val = (val * 1664525 + 1013904223) % (2**32) % 151643
        out.append(val + 1)
    return np.array(out, np.uint32)


def test_reusable_context_six_cases():
    """The six validation cases of bench/prefix_state_reuse_bench.cpp:71-112."""
    r = _m()
    ctx = r.PrefixContext("Qwen3.8-27B", "Q4_K_M")
    prefix = _prompt(512, 100)
    ctx.save(prefix)
    exact = np.append(prefix, 1234).astype(np.uint32)
    M = r.MatchResult
    assert ctx.check_match(exact, "Qwen3.8-27B", "Q4_K_M") == M.EXACT_MATCH
    assert ctx.check_match(exact, "Qwen3.8-32B", "Q4_K_M") == M.MODEL_MISMATCH
    assert ctx.check_match(exact, "Qwen3.8-27B", "Q8_0") == M.QUANTIZATION_MISMATCH
    corrupt = exact.copy()
    corrupt[50] ^= 0x5555
    assert ctx.check_match(corrupt, "Qwen3.8-27B", "Q4_K_M") == M.PREFIX_MISMATCH
    assert ctx.check_match(_prompt(256, 100), "Qwen3.8-27B", "Q4_K_M") == M.PROMPT_SHORTER_THAN_PREFIX
    ctx.clear()
    assert ctx.check_match(exact, "Qwen3.8-27B", "Q4_K_M") == M.EMPTY_CACHE


def test_match_precedence_and_fingerprint():
    r = _m()
    M = r.MatchResult
    ctx = r.PrefixContext("m", "q")
    assert ctx.check_match([1, 2], "m", "q") == M.EMPTY_CACHE
    ctx.save([7, 8, 9])
    assert ctx.prefix_length == 3
    assert ctx.token_hash == oracle.token_hash([7, 8, 9]) == r.token_hash([7, 8, 9])
    # Version is checked before model; model before quantization; both before length.
    ctx._set_layout_version(1)
    assert ctx.check_match([1], "x", "y") == M.VERSION_MISMATCH
    ctx._set_layout_version(20260925)
    assert ctx.check_match([1], "x", "y") == M.MODEL_MISMATCH
    assert ctx.check_match([1], "m", "y") == M.QUANTIZATION_MISMATCH
    assert ctx.check_match([1], "m", "q") == M.PROMPT_SHORTER_THAN_PREFIX
    assert ctx.check_match([7, 8, 9], "m", "q") == M.EXACT_MATCH
    ctx.save([])  # an empty save clears (reusable_context.cpp:142-145)
    assert ctx.check_match([7, 8, 9], "m", "q") == M.EMPTY_CACHE


def test_token_hash_published_vectors():
    r = _m()
    assert r.token_hash([]) == 0xCBF29CE484222325
    assert r.token_hash([ord("a")]) == 0xAF63DC4C8601EC8C
    assert r.token_hash([ord(c) for c in "foobar"]) == 0x85944171F73967E8
    rng = np.random.default_rng(0)
    t = rng.integers(0, 2**32, 1000, dtype=np.uint64).astype(np.uint32)
    assert r.token_hash(t) == oracle.token_hash(t)


@pytest.mark.parametrize("length", [1000, 1024])  # partial last page, full last page
def test_pool_fork_and_copy_on_write(length):
    r = _m()
    pt = 256
    pool = r.PagePool(32)
    pages = (length + pt - 1) // pt
    parent = np.array([pool.alloc() for _ in range(pages)] + [-1] * 4, np.int32)
    child, copies = pool.fork(parent, length, pt)
    full = length // pt
    for i in range(full):
        assert child[i] == parent[i] and pool.refcount(parent[i]) == 2
    if length % pt:
        assert len(copies) == 1 and copies[0][0] == parent[pages - 1]
        assert child[pages - 1] == copies[0][1] != parent[pages - 1]
        assert pool.refcount(parent[pages - 1]) == 1 and pool.refcount(child[pages - 1]) == 1
    else:
        assert copies == []
    # the child appends: a partial page it owns needs no copy; a page boundary allocates
    before = pool.free_pages
    c = child.copy()
    assert pool.prepare_append(c, length, pt) == []
    assert pool.free_pages == before - (1 if length % pt == 0 else 0)
    # a second fork of the child shares the child's partial page only via copy
    grand, copies2 = pool.fork(c, length + 1, pt)
    assert len(copies2) == 1
    # releasing everything returns every page to the pool
    pool.release(grand, length + 1, pt)
    pool.release(c, length + 1, pt)
    pool.release(parent, length, pt)
    assert pool.free_pages == 32


def test_pool_shared_partial_page_copies_on_write():
    r = _m()
    pt = 256
    pool = r.PagePool(8)
    row = np.array([pool.alloc(), -1], np.int32)
    other = row.copy()
    assert r.PagePool.__dict__  # keep linters calm
    # share the partial page explicitly (as an engine that shares without forking would)
    from miinfer_amd._lib import lib
    assert lib().miikv_pool_ref(pool._h, int(row[0])) == 0
    copies = pool.prepare_append(other, 100, pt)
    assert len(copies) == 1 and copies[0][0] == row[0] and other[0] == copies[0][1]
    assert pool.refcount(row[0]) == 1 and pool.refcount(other[0]) == 1


def test_pool_exhaustion_and_bad_pages():
    r = _m()
    pool = r.PagePool(2)
    a, b = pool.alloc(), pool.alloc()
    with pytest.raises(MemoryError):
        pool.alloc()
    from miinfer_amd import MiikvError
    with pytest.raises(MiikvError):  # fork of a partial page needs a free page
        pool.fork(np.array([a], np.int32), 10, 256)
    assert pool.refcount(a) == 1  # a failed fork changes nothing
    with pytest.raises(MiikvError):
        pool.release(np.array([7], np.int32), 10, 256)
    pool.release(np.array([a, b], np.int32), 300, 256)
    assert pool.free_pages == 2


def test_fork_many_matches_repeated_fork():
    """One batched call plans the same rows, reference counts and copies as n single forks."""
    from miinfer_amd.reuse import PagePool
    pt, length, n = 256, 256 * 3 + 10, 5
    a, b = PagePool(40), PagePool(40)
    ra = np.array([a.alloc() for _ in range(4)], np.int32)
    rb = np.array([b.alloc() for _ in range(4)], np.int32)
    rows, copies = a.fork_many(ra, length, pt, n)
    single = [b.fork(rb, length, pt) for _ in range(n)]
    assert np.array_equal(rows, np.stack([r for r, _ in single]))
    assert copies == [c for _, cs in single for c in cs]
    assert [a.refcount(p) for p in range(40)] == [b.refcount(p) for p in range(40)]
    with pytest.raises(MemoryError):
        PagePool(5).fork_many(np.array([0, 1, 2, 3], np.int32), length, pt, 3)
    # whole pages only: no copies, every page shared n + 1 ways
    c = PagePool(8)
    rc = np.array([c.alloc() for _ in range(3)], np.int32)
    rows, copies = c.fork_many(rc, 3 * pt, pt, 6)
    assert copies == [] and np.array_equal(rows, np.tile(rc, (6, 1)))
    assert [c.refcount(int(p)) for p in rc] == [7, 7, 7] and c.free_pages == 5


def test_fork_many_exhaustion_keeps_the_completed_forks():
    """Partial-page forks need one fresh page each: with 2 free pages, 2 of 5 forks
    complete (rows, copies, reference counts as 2 single forks) and the call fails."""
    from miinfer_amd.reuse import PagePool
    from miinfer_amd import lib
    import ctypes
    pt, length = 256, 256 * 2 + 7
    a, b = PagePool(5), PagePool(5)
    ra = np.array([a.alloc() for _ in range(3)], np.int32)
    rb = np.array([b.alloc() for _ in range(3)], np.int32)
    rows = np.full((5, 3), -1, np.int32)
    src, dst = np.zeros(5, np.int32), np.zeros(5, np.int32)
    nc, done = ctypes.c_uint32(0), ctypes.c_uint32(0)
    p32 = lambda x: x.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))
    st = lib().miikv_pool_fork_n(a._h, p32(ra), length, pt, 5, p32(rows), 3, p32(src), p32(dst),
                                 ctypes.byref(nc), ctypes.byref(done))
    assert st != 0 and done.value == 2 and nc.value == 2
    single = [b.fork(rb, length, pt) for _ in range(2)]
    assert np.array_equal(rows[:2], np.stack([r for r, _ in single]))
    assert list(zip(src[:2].tolist(), dst[:2].tolist())) == [c for _, cs in single for c in cs]
    assert np.all(rows[2:] == -1)
    assert [a.refcount(p) for p in range(5)] == [b.refcount(p) for p in range(5)]
    assert a.free_pages == b.free_pages == 0


def test_pool_fork_rejects_short_rows():
    from miinfer_amd import MiikvError
    from miinfer_amd import reuse
    pool = reuse.PagePool(16)
    row = np.array([pool.alloc() for _ in range(2)], np.int32)
    with pytest.raises(MiikvError):  # 3 pages needed, the row holds 2
        pool.fork(row, 600, 256)
    assert pool.free_pages == 14


def test_pool_prepare_append_twice_at_a_boundary_keeps_one_page():
    from miinfer_amd import reuse
    pool = reuse.PagePool(8)
    row = np.full(4, -1, np.int32)
    row[0] = pool.alloc()
    assert pool.prepare_append(row, 256, 256) == []
    page = int(row[1])
    free = pool.free_pages
    assert pool.prepare_append(row, 256, 256) == []  # again: the page it holds stays
    assert int(row[1]) == page and pool.free_pages == free and pool.refcount(page) == 1
    # a shared page at the boundary is copied, not leaked
    child, _ = pool.fork(row, 512, 256)
    assert pool.refcount(page) == 2
    cps = pool.prepare_append(child, 256, 256)
    assert cps == [(page, int(child[1]))] and pool.refcount(page) == 1


def _session(pool, n, pt=256):
    row = np.full(-(-n // pt) + 2, -1, np.int32)
    for i in range(-(-n // pt)):
        row[i] = pool.alloc()
    return row


def test_registry_longest_prefix_and_precedence():
    from miinfer_amd import reuse
    M = reuse.MatchResult
    pool = reuse.PagePool(64)
    reg = reuse.PrefixRegistry(pool, 256, 8, "m", "q")
    assert reg.lookup(np.arange(10))[0] == M.EMPTY_CACHE
    a = np.arange(300, dtype=np.uint32)
    b = np.arange(800, dtype=np.uint32)          # extends a
    c = np.arange(1000, 1600, dtype=np.uint32)   # unrelated
    ea = reg.save(a, _session(pool, 300))
    eb = reg.save(b, _session(pool, 800))
    ec = reg.save(c, _session(pool, 600))
    assert len(reg) == 3
    # longest matching prefix wins; strict needs a token left to run
    assert reg.lookup(np.arange(900))[:3] == (M.EXACT_MATCH, eb, 800)
    assert reg.lookup(np.arange(500))[:3] == (M.EXACT_MATCH, ea, 300)
    assert reg.lookup(np.arange(800))[:3] == (M.EXACT_MATCH, ea, 300)
    assert reg.lookup(np.arange(800), strict=False)[:3] == (M.EXACT_MATCH, eb, 800)
    assert reg.lookup(np.concatenate([c, [7]]))[:2] == (M.EXACT_MATCH, ec)
    # no match: the most recently used entry's verdict, in check_match's precedence
    assert reg.lookup(np.arange(5, 900))[0] == M.PREFIX_MISMATCH
    assert reg.lookup(np.arange(900), model_id="other")[0] == M.MODEL_MISMATCH
    assert reg.lookup(np.arange(900), quantization="Q8")[0] == M.QUANTIZATION_MISMATCH
    reg._set_layout_version(ea, 1)
    reg._set_layout_version(eb, 1)
    reg._set_layout_version(ec, 1)
    assert reg.lookup(np.arange(900))[0] == M.VERSION_MISMATCH
    # same tokens again: the existing entry, no duplicate
    assert reg.save(a, _session(pool, 300)) == ea and len(reg) == 3
    info = reg.info(eb)
    assert info["length"] == 800 and info["hash"] == reuse.token_hash(b) and info["pages"].size == 4


def test_registry_refcounts_fork_and_release():
    from miinfer_amd import reuse
    pool = reuse.PagePool(32)
    reg = reuse.PrefixRegistry(pool, 256, 4)
    row = _session(pool, 600)                    # 3 pages, the last partial
    e = reg.save(np.arange(600), row)
    pages = row[:3].copy()
    assert all(pool.refcount(int(p)) == 2 for p in pages)
    pool.release(row, 600, 256)                  # the session ends; the entry keeps them
    assert all(pool.refcount(int(p)) == 1 for p in pages)
    child, copies = reg.fork(e, 5)
    assert (child[:2] == pages[:2]).all() and child[2] not in pages
    assert copies == [(int(pages[2]), int(child[2]))]
    assert pool.refcount(int(pages[0])) == 2 and pool.refcount(int(pages[2])) == 1
    free = pool.free_pages
    reg.release(e)
    assert len(reg) == 0
    assert pool.refcount(int(pages[0])) == 1 and pool.refcount(int(pages[2])) == 0
    assert pool.free_pages == free + 1
    pool.release(child, 600, 256)
    assert pool.free_pages == 32


def test_registry_lru_eviction():
    from miinfer_amd import reuse
    pool = reuse.PagePool(32)
    reg = reuse.PrefixRegistry(pool, 256, 2)
    rows = {}
    ids = {}
    for name, base in (("a", 0), ("b", 10000)):
        rows[name] = _session(pool, 512)
        ids[name] = reg.save(np.arange(base, base + 512), rows[name])
        pool.release(rows[name], 512, 256)
    child, _ = reg.fork(ids["a"], 4)               # a is now the most recent
    pool.release(child, 512, 256)
    rows["c"] = _session(pool, 256)
    ids["c"] = reg.save(np.arange(20000, 20256), rows["c"])  # full: b is evicted
    pool.release(rows["c"], 256, 256)
    assert len(reg) == 2
    assert reg.lookup(np.arange(10000, 10600))[0] != reuse.MatchResult.EXACT_MATCH
    assert reg.lookup(np.arange(0, 600))[1] == ids["a"]
    before = pool.free_pages
    evicted = reg.evict_until_free(before + 1)     # a (least recent) holds 2 pages alone
    assert evicted == [ids["a"]] and pool.free_pages == before + 2


def test_pool_release_clears_the_row_so_a_reused_row_cannot_write_a_foreign_page():
    """A released row's entries become -1: reusing it allocates fresh pages instead of
    handing back a page id that the pool has since given to another sequence."""
    from miinfer_amd import reuse
    pt = 256
    pool = reuse.PagePool(4)
    row = np.full(2, -1, np.int32)
    assert pool.prepare_append(row, 0, pt) == []
    old = int(row[0])
    pool.release(row, 10, pt)
    assert np.all(row == -1) and pool.refcount(old) == 0
    other = np.full(2, -1, np.int32)
    assert pool.prepare_append(other, 0, pt) == []
    assert int(other[0]) == old  # the freed page now belongs to `other`
    assert pool.prepare_append(row, 0, pt) == []  # the stale row gets a page of its own
    assert int(row[0]) != old and pool.refcount(old) == 1 and pool.refcount(int(row[0])) == 1


def test_fork_many_exhaustion_leaves_the_pool_unchanged():
    """The Python wrapper gives back the forks completed before the pool ran out."""
    from miinfer_amd.reuse import PagePool
    pt, length = 256, 256 * 2 + 7
    pool = PagePool(5)
    row = np.array([pool.alloc() for _ in range(3)], np.int32)
    free, refs = pool.free_pages, [pool.refcount(p) for p in range(5)]
    with pytest.raises(MemoryError):
        pool.fork_many(row, length, pt, 5)
    assert pool.free_pages == free and [pool.refcount(p) for p in range(5)] == refs
