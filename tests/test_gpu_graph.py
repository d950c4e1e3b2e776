"""Graph replay with device-side positions (model.cpp:1136-1227): a captured
decode step (append at decode_state->position, attention over position + 1
keys, state advance) and a captured suffix step (append + suffix attention at
prefill_state->base_position) replayed with new inputs; every replay is checked
against the oracle, with eager work and synchronisations between replays."""
import math

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import assert_attention_close, randn_f16

pytestmark = pytest.mark.gpu


def _dev(a, gpu):
    return torch.from_numpy(np.ascontiguousarray(a)).to(gpu)


@pytest.mark.parametrize("fused", [False, True])
def test_decode_step_graph_replays(gpu, fused):
    """fused: the captured step is miikv_decode_append_attn (store + attention in one
    launch pair) instead of an append followed by attention."""
    import miinfer_amd as m
    rng = np.random.default_rng(41)
    hq, hk, d, cap, p0, steps = 32, 8, 128, 1024, 500, 8
    cache = m.KvCache.contiguous(hk, d, cap)
    k_all = randn_f16(rng, (p0 + steps, hk, d))
    v_all = randn_f16(rng, (p0 + steps, hk, d))
    cache.append(_dev(k_all[:p0], gpu), _dev(v_all[:p0], gpu))
    k_in = torch.zeros((1, hk, d), dtype=torch.float16, device=gpu)
    v_in = torch.zeros_like(k_in)
    q_in = torch.zeros((1, hq, d), dtype=torch.float16, device=gpu)
    out = torch.zeros((1, hq, d), dtype=torch.float32, device=gpu)
    ds = m.make_decode_state(p0, device=gpu, max_generated=6)
    tokens_out = torch.zeros(16, dtype=torch.int32, device=gpu)
    ws = m.DecodeWorkspace(cache, hq, 1, cap)
    torch.cuda.synchronize()

    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.graph(g, stream=s):
        if fused:
            m.decode_attention(cache, q_in, decode_state=ds, max_context=cap, out=out, workspace=ws,
                               k_new=k_in, v_new=v_in)
        else:
            cache.append(k_in, v_in, decode_state=ds)
            m.decode_attention(cache, q_in, decode_state=ds, max_context=cap, out=out, workspace=ws)
        m.advance_decode_state(ds, tokens_out, stop_tokens=(151643, 151645))
    torch.cuda.synchronize()

    kc, ks = oracle.quantize_rows(k_all.transpose(1, 0, 2))
    vc, vs = oracle.quantize_rows(v_all.transpose(1, 0, 2))
    toks = [11, 22, 33, 151645, 44, 55, 66, 77]
    for i in range(steps):
        q = randn_f16(rng, (1, hq, d))
        k_in.copy_(_dev(k_all[p0 + i:p0 + i + 1], gpu))
        v_in.copy_(_dev(v_all[p0 + i:p0 + i + 1], gpu))
        q_in.copy_(_dev(q, gpu))
        ds[0] = toks[i]
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        length = p0 + i + 1
        expect = oracle.attention_q8(q[0].astype(np.float32), kc[:, :length], ks[:, :length],
                                     vc[:, :length], vs[:, :length], length, hq, 1 / math.sqrt(d))
        assert_attention_close(out.cpu().numpy()[0], expect, f"replay {i}")
        st = ds.cpu().numpy()
        assert st[1] == length and st[2] == i + 1
        # stop: the stop token at step 3, and the generation limit (6) from step 5 on
        assert st[3] == (1 if i >= 3 else 0)
    assert list(tokens_out.cpu().numpy()[:steps]) == toks


@pytest.mark.parametrize("t", [64, 4])  # the MFMA path; a batch of decodes
@pytest.mark.parametrize("fused", [False, True])
def test_suffix_step_graph_replays(gpu, fused, t):
    """fused: the captured step is miikv_suffix_append_attn."""
    import miinfer_amd as m
    rng = np.random.default_rng(42)
    hq, hk, d, cap = 24, 4, 256, 2048
    cache = m.KvCache.contiguous(hk, d, cap)
    total = 3 * t + 700
    k_all = randn_f16(rng, (total, hk, d))
    v_all = randn_f16(rng, (total, hk, d))
    cache.append(_dev(k_all[:700], gpu), _dev(v_all[:700], gpu))
    k_in = torch.zeros((t, hk, d), dtype=torch.float16, device=gpu)
    v_in = torch.zeros_like(k_in)
    q_in = torch.zeros((t, hq, d), dtype=torch.float16, device=gpu)
    out = torch.zeros((t, hq, d), dtype=torch.float32, device=gpu)
    ps = m.make_prefill_state(700, t, device=gpu)
    ws = torch.empty(m.suffix_workspace_bytes(cache, hq, t), dtype=torch.uint8, device=gpu)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.graph(g, stream=s):
        if fused:
            m.suffix_attention(cache, q_in, 0, prefill_state=ps, out=out, workspace=ws, k_new=k_in, v_new=v_in)
        else:
            cache.append(k_in, v_in, prefill_state=ps)
            m.suffix_attention(cache, q_in, 0, prefill_state=ps, out=out, workspace=ws)
    torch.cuda.synchronize()
    kc, ks = oracle.quantize_rows(k_all.transpose(1, 0, 2))
    vc, vs = oracle.quantize_rows(v_all.transpose(1, 0, 2))
    for i in range(3):
        base = 700 + i * t
        q = randn_f16(rng, (t, hq, d))
        k_in.copy_(_dev(k_all[base:base + t], gpu))
        v_in.copy_(_dev(v_all[base:base + t], gpu))
        q_in.copy_(_dev(q, gpu))
        ps[0] = base
        ps[1] = t
        ps[2] = base + t
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        expect = oracle.suffix_attention_q8(q.astype(np.float32), kc[:, :base + t], ks[:, :base + t],
                                            vc[:, :base + t], vs[:, :base + t], base, hq, 1 / math.sqrt(d))
        assert_attention_close(out.cpu().numpy(), expect, f"suffix replay {i}")
