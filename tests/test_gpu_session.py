"""Persistent session round trip on the GPU: save the first P tokens of several
attention layers (contiguous and paged) and the GDN state, load into fresh
storage, and compare byte for byte (persistent_session.cpp:34-258)."""
import os

import numpy as np
import pytest
import torch

from tests.helpers import randn_f16

pytestmark = pytest.mark.gpu


def _dev(a, gpu):
    return torch.from_numpy(np.ascontiguousarray(a)).to(gpu)


def _export(cache, seq, n):
    out = cache.export_canonical(seq, 0, n)
    torch.cuda.synchronize()
    return [t.cpu().numpy().tobytes() for t in out]


def _paged(m, gpu, rng, hk, d, pages, pt=256):
    table = _dev(rng.permutation(pages).astype(np.int32).reshape(1, pages), gpu)
    return m.KvCache.paged_cache(hk, d, pages, table, page_tokens=pt)


def test_session_round_trip_bytes(gpu, tmp_path):
    import miinfer_amd as m
    from miinfer_amd import session
    from miinfer_amd.reuse import RecurrentStates
    rng = np.random.default_rng(5)
    hk, d, P = 4, 256, 700
    src = [m.KvCache.contiguous(hk, d, 1024), _paged(m, gpu, rng, hk, d, 4), m.KvCache.contiguous(hk, d, 768)]
    for c in src:
        c.append(_dev(randn_f16(rng, (P + 20, hk, d)), gpu), _dev(randn_f16(rng, (P + 20, hk, d)), gpu))
    states = RecurrentStates(3, 16 * 128, 96, device=gpu)
    states.buf.copy_(torch.randn(states.buf.numel(), device=gpu))
    tokens = rng.integers(0, 150000, P).astype(np.uint32)
    path = str(tmp_path / session.session_filename(m.reuse.token_hash(tokens), P))
    session.save_session(path, "Qwen3.8-27B", "Q4_K_M", tokens, src, states)

    h, toks = session.inspect_session(path, with_tokens=True)
    layer_bytes = 2 * P * hk * (d + 2 * d // 32)
    assert (h.prefix_length, h.gqa_layers, h.gdn_layers, h.kv_quant_mode) == (P, 3, 3, 4)
    assert h.kv_bytes == 3 * layer_bytes and h.gdn_state_bytes == 3 * (16 * 128 + 96) * 4
    assert os.path.getsize(path) == 157 + 4 * P + h.gdn_state_bytes + h.kv_bytes
    assert np.array_equal(toks, tokens)

    dst = [m.KvCache.contiguous(hk, d, 1024), m.KvCache.contiguous(hk, d, 1024), _paged(m, gpu, rng, hk, d, 3)]
    fresh = RecurrentStates(3, 16 * 128, 96, device=gpu)
    got = session.load_session(path, "Qwen3.8-27B", "Q4_K_M", dst, fresh)
    assert got is not None and np.array_equal(got, tokens) and fresh.position == P
    for a, b in zip(src, dst):
        assert _export(a, 0, P) == _export(b, 0, P)
    torch.cuda.synchronize()
    assert torch.equal(fresh.buf, states.buf)
    # a truncated copy or another model's request is rejected and writes nothing
    with open(path, "rb") as f:
        data = f.read()
    bad = str(tmp_path / "bad.miinfer")
    with open(bad, "wb") as f:
        f.write(data[:-100])
    other = RecurrentStates(3, 16 * 128, 96, device=gpu)
    assert session.load_session(bad, "Qwen3.8-27B", "Q4_K_M", dst, other) is None
    assert session.load_session(path, "Qwen3.8-27B", "Q8_0", dst, other) is None
    torch.cuda.synchronize()
    assert not other.buf.any()
    assert session.find_session(str(tmp_path), "Qwen3.8-27B", "Q4_K_M",
                                np.concatenate([tokens, [1, 2, 3]])) == (path, P)
