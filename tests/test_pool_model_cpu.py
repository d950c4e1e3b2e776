"""Page pool against a model (CPU): random sequences of session creation, appends
(new pages and copy-on-write of shared ones), forks and releases, with the pool
often exhausted.  After every operation each page's reference count must equal the
number of live session rows that name it, and the free count the pages nobody names;
a failed operation changes nothing."""
import numpy as np
import pytest

PT = 16      # tokens per page
CAP = 12     # pages per row


def _named(sessions):
    counts = {}
    for row, length in sessions:
        for p in row[:-(-length // PT)]:
            counts[int(p)] = counts.get(int(p), 0) + 1
    return counts


def _check(pool, sessions, npages):
    counts = _named(sessions)
    assert all(pool.refcount(p) == counts.get(p, 0) for p in range(npages))
    assert pool.free_pages == npages - len(counts)


def _append(pool, row, length, n):
    """Append n tokens (prepare_append per position); returns the new length."""
    from miinfer_amd import MiikvError
    for _ in range(n):
        if length >= CAP * PT:
            break
        try:
            copies = pool.prepare_append(row, length, PT)
        except MiikvError:
            break  # pool exhausted: the row is unchanged
        for src, dst in copies:
            assert src != dst and row[length // PT] == dst
        length += 1
    return length


@pytest.mark.parametrize("seed", range(8))
def test_pool_matches_model(seed):
    from miinfer_amd.reuse import PagePool
    rng = np.random.default_rng(seed)
    npages = int(rng.integers(8, 40))
    pool = PagePool(npages)
    sessions = []  # (row, length)
    for _ in range(300):
        op = rng.integers(0, 4)
        if op == 0 or not sessions:  # a new session with a few tokens
            row = np.full(CAP, -1, np.int32)
            length = _append(pool, row, 0, int(rng.integers(1, 3 * PT)))
            if length:
                sessions.append((row, length))
        elif op == 1:  # append to a session
            i = int(rng.integers(len(sessions)))
            row, length = sessions[i]
            sessions[i] = (row, _append(pool, row, length, int(rng.integers(1, 2 * PT))))
        elif op == 2:  # fork a session
            row, length = sessions[int(rng.integers(len(sessions)))]
            before = [pool.refcount(p) for p in range(npages)], pool.free_pages
            try:
                child, copies = pool.fork(row, length, PT)
            except Exception:
                assert ([pool.refcount(p) for p in range(npages)], pool.free_pages) == before
            else:
                full = length // PT
                assert np.array_equal(child[:full], row[:full])
                if length % PT:
                    assert copies == [(int(row[full]), int(child[full]))]
                sessions.append((child, length))
        else:  # release a session
            row, length = sessions.pop(int(rng.integers(len(sessions))))
            pool.release(row, length, PT)
        _check(pool, sessions, npages)
    for row, length in sessions:
        pool.release(row, length, PT)
    assert pool.free_pages == npages


@pytest.mark.parametrize("seed", range(6))
def test_registry_and_pool_match_model(seed):
    """Sessions and saved prefixes share one pool: random saves (a repeated token
    sequence refreshes its entry), lookups (the longest saved prefix of the prompt
    that leaves a prompt token to run wins), forks from entries, releases, LRU
    evictions and session ends.  Each page's
    count must equal the session rows plus the registry entries naming it."""
    from miinfer_amd.reuse import MatchResult, PagePool, PrefixRegistry
    rng = np.random.default_rng(100 + seed)
    npages = int(rng.integers(16, 48))
    pool = PagePool(npages)
    reg = PrefixRegistry(pool, page_tokens=PT, max_entries=int(rng.integers(2, 6)))
    sessions = []  # (row, length, tokens)
    entries = {}   # id -> tokens

    def check():
        counts = _named([(r, n) for r, n, _ in sessions])
        assert len(reg) == len(entries)
        for eid in entries:
            info = reg.info(eid)
            assert info["length"] == len(entries[eid])
            for p in info["pages"]:
                counts[int(p)] = counts.get(int(p), 0) + 1
        assert all(pool.refcount(p) == counts.get(p, 0) for p in range(npages))
        assert pool.free_pages == npages - len(counts)

    vocab = 3  # few token values, so prompts share prefixes often
    for _ in range(250):
        op = rng.integers(0, 6)
        if op == 0 or not sessions:
            row = np.full(CAP, -1, np.int32)
            length = _append(pool, row, 0, int(rng.integers(1, 3 * PT)))
            if length:
                sessions.append((row, length, list(rng.integers(0, vocab, length))))
        elif op == 1:  # save a session's tokens (or a prefix of them)
            row, length, toks = sessions[int(rng.integers(len(sessions)))]
            n = int(rng.integers(1, length + 1))
            known = [e for e, t in entries.items() if t == toks[:n]]
            eid = reg.save(toks[:n], row)
            if known:
                assert eid == known[0]
            # a full registry evicted its least recently used entries first
            live = {e for e in entries if e == eid or _alive(reg, e)}
            for e in set(entries) - live:
                entries.pop(e)
            entries[eid] = toks[:n]
        elif op == 2 and entries:  # lookup a prompt
            row, length, toks = sessions[int(rng.integers(len(sessions)))]
            prompt = toks + list(rng.integers(0, vocab, int(rng.integers(0, 4))))
            r, eid, n = reg.lookup(prompt)
            # strict lookup: the prefix leaves at least one prompt token to run
            cands = [len(t) for t in entries.values() if len(t) < len(prompt) and t == prompt[:len(t)]]
            if cands:
                assert r == MatchResult.EXACT_MATCH and n == max(cands) and entries[eid] == prompt[:n]
            else:
                assert r != MatchResult.EXACT_MATCH
        elif op == 3 and entries:  # fork a session from an entry
            eid = list(entries)[int(rng.integers(len(entries)))]
            try:
                child, copies = reg.fork(eid, CAP)
            except Exception:
                pass  # pool exhausted: nothing changed (checked below)
            else:
                sessions.append((child, len(entries[eid]), list(entries[eid])))
        elif op == 4 and entries:  # release an entry, or evict the least recently used
            if rng.integers(2):
                eid = list(entries)[int(rng.integers(len(entries)))]
                reg.release(eid)
                entries.pop(eid)
            else:
                entries.pop(reg.evict_lru())
        elif op == 5:  # a session ends
            row, length, _ = sessions.pop(int(rng.integers(len(sessions))))
            pool.release(row, length, PT)
        check()
    while len(reg):
        entries.pop(reg.evict_lru())
    for row, length, _ in sessions:
        pool.release(row, length, PT)
    assert pool.free_pages == npages


def _alive(reg, eid):
    from miinfer_amd import MiikvError
    try:
        reg.info(eid)
        return True
    except MiikvError:
        return False
