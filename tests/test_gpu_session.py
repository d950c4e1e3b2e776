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
    return [None if t is None else t.cpu().numpy().tobytes() for t in out]


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


@pytest.mark.parametrize("mode", [0, 1, 2, 3])  # FP16_FP16, Q8_FP16, FP16_Q8, Q8_Q8
def test_session_every_quant_mode(gpu, tmp_path, mode):
    """A session of a cache in any KvCacheQuantMode (the reference writes the model's mode,
    persistent_session.cpp:54): the header carries the mode's file value, the KV bytes are
    the raw layout of kv_cache.cpp:227-297 built here from the input rows (fp16 rows as
    given, q8 planes as the oracle quantises them), and loading restores every byte; a
    cache of another mode is refused."""
    import miinfer_amd as m
    import oracle
    from miinfer_amd import _lib, session
    rng = np.random.default_rng(60 + mode)
    hk, d, P = 4, 128, 300
    k_f16, v_f16 = mode in (0, 2), mode in (0, 1)
    k = randn_f16(rng, (P, hk, d))
    v = randn_f16(rng, (P, hk, d))
    src = [m.KvCache.contiguous(hk, d, 384, quant_mode=mode),
           m.KvCache.paged_cache(hk, d, 2, _dev(np.array([[1, 0]], np.int32), gpu), page_tokens=256,
                                 quant_mode=mode)]
    for c in src:
        c.append(_dev(k, gpu), _dev(v, gpu))
    tokens = rng.integers(0, 150000, P).astype(np.uint32)
    path = str(tmp_path / "s.miinfer")
    session.save_session(path, "m", "q", tokens, src)
    h, _ = session.inspect_session(path)
    want_mode = {0: session.KV_FP16_FP16, 1: session.KV_Q8_0_32_FP16, 2: session.KV_FP16_Q8_0_32,
                 3: session.KV_Q8_0_32}[mode]
    assert h.kv_quant_mode == want_mode == _lib.lib().miikv_session_kv_mode(mode)

    def part(rows, f16):
        if f16:
            return [rows[:, hd].tobytes() for hd in range(hk)]
        codes, scales = oracle.quantize_rows(rows.transpose(1, 0, 2))
        return [codes[hd].tobytes() + scales[hd].tobytes() for hd in range(hk)]
    layer = b"".join(part(k, k_f16) + part(v, v_f16))
    with open(path, "rb") as f:
        data = f.read()
    kv = data[157 + 4 * P:]
    assert h.kv_bytes == 2 * len(layer) and kv == layer + layer

    dst = [m.KvCache.contiguous(hk, d, 512, quant_mode=mode),
           m.KvCache.paged_cache(hk, d, 3, _dev(np.array([[2, 0]], np.int32), gpu), page_tokens=256,
                                 quant_mode=mode)]
    assert session.load_session(path, "m", "q", dst) is not None
    for a, b in zip(src, dst):
        assert _export(a, 0, P) == _export(b, 0, P)
    other = [m.KvCache.contiguous(hk, d, 512, quant_mode=(mode + 1) % 4) for _ in range(2)]
    assert session.load_session(path, "m", "q", other) is None
