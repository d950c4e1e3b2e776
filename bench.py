"""Decode attention over a 32k-token q8_0 KV cache on one MI355X.

Workload (the headline benchmark's config 2 at its largest context): Qwen3-8B-shaped GQA layer,
32 query heads, 8 KV heads, head_dim 128, batch 1, context 32768.  One step =
one layer-token: quantize-append one fp16 K/V row per KV head into the q8_0
cache (at position 32767), then single-token attention over the 32768 cached
tokens.  Steps rotate over several independent layer caches so the working set
(8 x 71.3 MB) exceeds the 256 MB Infinity Cache and every step streams its
cache from HBM.  Inputs are seeded N(0,1) fp16, resident in HBM before timing.

Prints one JSON line.  `value` is algorithmic GB/s of the whole step (append +
attention): per step 2176 B/token x 32768 tokens of K/V codes and scales, plus
the append (8 KiB fp16 in, 2176 B out) and q/out (8 KiB + 16 KiB).  The
`roofline` object covers the dominant kernel (decode attention) alone.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HQ, HKV, D = 32, 8, 128
PEAK_HBM_GBS = 8000.0


def kv_bytes_per_token(hkv=HKV, d=D) -> int:
    # K and V: codes (d bytes) + scales (2 bytes per 32-value block), per kv head
    return 2 * hkv * (d + 2 * (d // 32))


def decode_bytes(ctx, hq=HQ, hkv=HKV, d=D) -> int:
    return ctx * kv_bytes_per_token(hkv, d) + hq * d * 2 + hq * d * 4


def append_bytes(hkv=HKV, d=D) -> int:
    return 2 * hkv * d * 2 + kv_bytes_per_token(hkv, d)


def _cpu_case(ctx, seed, threads, warmup, reps):
    import numpy as np

    import oracle
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((HKV, ctx, D)).astype(np.float32).astype(np.float16)
    v = rng.standard_normal((HKV, ctx, D)).astype(np.float32).astype(np.float16)
    q = rng.standard_normal((HQ, D)).astype(np.float32).astype(np.float16).astype(np.float32)
    kc, ks = oracle.quantize_rows(k)
    vc, vs = oracle.quantize_rows(v)
    return oracle.time_attention_q8(q, kc, ks, vc, vs, ctx, HQ, 1 / math.sqrt(D), threads=threads,
                                    warmup=warmup, reps=reps)


def cpu_baseline() -> dict:
    """Config 1 of the headline benchmark on the host CPU: the oracle's C restatement of the reference
    CPU attention path (fp32 loop over a dequantised cache, double-denominator softmax),
    32q/8kv/D128, one fp16 query, context 4096; plus the GPU headline's context (32768)."""
    nproc = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    threads = max(1, min(nproc, HQ))  # the port splits query heads over threads
    t1 = _cpu_case(4096, 1, 1, 3, 20)
    tn = _cpu_case(4096, 1, threads, 3, 20)
    t32 = _cpu_case(32768, 1, threads, 2, 10)
    b = decode_bytes(4096)
    return {
        "value": round(b / tn / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
        "host_cores_nproc": nproc,
        "us_per_layer_token": round(tn * 1e6, 1),
        "single_thread": {"value": round(b / t1 / 1e9, 3), "us_per_layer_token": round(t1 * 1e6, 1)},
        "context_32768": {"value": round(decode_bytes(32768) / t32 / 1e9, 3),
                          "us_per_layer_token": round(t32 * 1e6, 1), "cores": threads},
        "sample": f"config 1: 32q/8kv/D128 q8_0 decode, one query token, context 4096, attention "
                  f"only: median of 20 calls after 3 warm-ups on {threads} threads (query heads "
                  f"split; {nproc} cores available) and on 1 thread; context 32768 median of 10 "
                  "after 2; the cache is dequantised to fp32 once, outside timing, as the reference "
                  "CPU path holds it",
    }


def _time_graph(fn, nsteps, warmup, inner=1):
    """Capture `fn(stream)` `inner` times in one graph, replay; returns (us per call of fn,
    replays).  Short calls use inner > 1 so the host's replay cost stays hidden."""
    import torch
    stream = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for _ in range(inner):
            fn(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            g.replay()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(nsteps):
            g.replay()
        e1.record(stream)
    e1.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (nsteps * inner), nsteps


def bench_c3(dev, args) -> int:
    """Config 3: batched paged decode, 24q/4kv/D256, 16 sequences with context lengths
    uniform in [1024, 65536] (seeded), 256-token pages behind a random permutation
    block table; each step appends one row per sequence, then attends."""
    import ctypes

    import numpy as np
    import torch

    import miinfer_amd as m
    from miinfer_amd import _lib
    hq, hkv, d, pt, batch = 24, 4, 256, 256, 16
    rng = np.random.default_rng(3)
    lens = rng.integers(1024, 65536 + 1, size=batch)
    pages = [(int(n) + pt) // pt for n in lens]  # room for the appended row
    stride = max(pages)
    perm = rng.permutation(sum(pages)).astype(np.int32)
    table = np.zeros((batch, stride), np.int32)
    o = 0
    for b, p in enumerate(pages):
        table[b, :p] = perm[o:o + p]
        o += p
    tab = torch.from_numpy(table).to(dev)
    cache = m.KvCache.paged_cache(hkv, d, sum(pages), tab, page_tokens=pt, device=dev)
    torch.manual_seed(0)
    for b, n in enumerate(lens):
        for t0 in range(0, int(n), 8192):
            c = min(8192, int(n) - t0)
            cache.append(torch.randn((c, hkv, d), device=dev).half(),
                         torch.randn((c, hkv, d), device=dev).half(), base_position=t0, seq=b)
    q = torch.randn((batch, hq, d), device=dev).half()
    kn = torch.randn((batch, hkv, d), device=dev).half()
    vn = torch.randn((batch, hkv, d), device=dev).half()
    pos = torch.from_numpy(lens.astype(np.int32) - 1).to(dev)   # overwrite the last row
    lengths = torch.from_numpy(lens.astype(np.int32)).to(dev)
    max_ctx = stride * pt
    out = torch.empty((batch, hq, d), device=dev)
    ws = m.DecodeWorkspace(cache, hq, batch, max_ctx)
    L = _lib.lib()
    P = ctypes.c_void_p

    def step(s):
        # one launch pair: the new rows are stored and scored by the combine kernel
        st = L.miikv_decode_append_attn(cache.view, P(kn.data_ptr()), P(vn.data_ptr()), P(q.data_ptr()),
                                        _lib.DTYPE_F16, hq, ctypes.c_float(1 / math.sqrt(d)), batch,
                                        P(lengths.data_ptr()), None, max_ctx, P(out.data_ptr()), None,
                                        None, None, P(ws.buf.data_ptr()), ws.bytes, P(s.cuda_stream))
        assert st == 0, st

    def dec(s, qq=q, dt=_lib.DTYPE_F16):
        st = L.miikv_decode_attn(cache.view, P(qq.data_ptr()), dt, hq,
                                 ctypes.c_float(1 / math.sqrt(d)), batch, P(lengths.data_ptr()),
                                 None, max_ctx, P(out.data_ptr()), None, None, P(ws.buf.data_ptr()),
                                 ws.bytes, P(s.cuda_stream))
        assert st == 0, st
    q32 = q.float()
    torch.cuda.synchronize()
    # 8 calls per graph replay (back to back, as a model's layers run), so the host's
    # replay cost stays out of the per-call time
    nrep = max(4, args.steps // 80)
    _time_graph(step, nrep, 3, inner=8)  # bring the clocks up before the first timed variant
    us, n = _time_graph(step, nrep, 3, inner=8)
    us_dec, _ = _time_graph(dec, nrep, 3, inner=8)
    us_dec32, _ = _time_graph(lambda s: dec(s, q32, _lib.DTYPE_F32), nrep, 3, inner=8)
    tokens = int(lens.sum())
    dbytes = tokens * kv_bytes_per_token(hkv, d) + batch * hq * d * 6
    print(json.dumps({
        "metric": "paged batched decode-attn q8_0 KV GB/s (config 3)", "unit": "GB/s",
        "value": round((dbytes + batch * append_bytes(hkv, d)) / (us * 1e-6) / 1e9, 1),
        "us_per_step": round(us, 2), "steps": n, "n_gpus": 1,
        "config": {"workload": "config 3: 16 seqs, 24q/4kv/D256, 256-token pages, random table",
                   "context_tokens_total": tokens, "max_context": int(lens.max())},
        "roofline": {"bound": "hbm", "kernel": "miikv_decode_attn (split + combine)",
                     "achieved": round(dbytes / (us_dec * 1e-6) / 1e9, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(dbytes / (us_dec * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
                     "algorithmic_bytes_per_launch": dbytes, "avg_launch_us": round(us_dec, 2)},
        "step": "miikv_decode_append_attn (store the 16 new rows + attend)",
        "decode_fp32_query": {"avg_launch_us": round(us_dec32, 2),
                              "GBs": round((dbytes + batch * hq * d * 2) / (us_dec32 * 1e-6) / 1e9, 1)},
    }), flush=True)
    return 0


# The reference's published Q8 suffix ladder (S = 512, 16 GQA layers, 24q/4kv/D256,
# q8 K and V; MI50, experiments/EXP-V2-0019-quantized-kv-cache.md:53-55), ms per 16 layers.
REFERENCE_SUFFIX_LADDER_MI50_MS = {4096: 662.96, 32768: 4971.17, 65536: 10506.89}


def suffix_ladder(dev) -> dict:
    """The reference's suffix ladder workload on this GPU: a 512-token suffix attending
    over P cached tokens plus itself, 16 layers (16 distinct caches, one graph replay
    runs each once), attention only (the suffix rows are already stored).  Reported
    beside the reference's MI50 figures: other hardware, not a like-for-like baseline."""
    import ctypes

    import torch

    import miinfer_amd as m
    from miinfer_amd import _lib
    hq, hkv, d, t, layers = 24, 4, 256, 512, 16
    L = _lib.lib()
    P = ctypes.c_void_p
    res = {}
    for prefix, ref_ms in REFERENCE_SUFFIX_LADDER_MI50_MS.items():
        torch.manual_seed(prefix)
        caches = []
        for _ in range(layers):
            c = m.KvCache.contiguous(hkv, d, prefix + t, device=dev)
            for t0 in range(0, prefix + t, 8192):
                n = min(8192, prefix + t - t0)
                c.append(torch.randn((n, hkv, d), device=dev).half(), torch.randn((n, hkv, d), device=dev).half(),
                         base_position=t0)
            caches.append(c)
        q = torch.randn((t, hq, d), device=dev).half()
        out = torch.empty((t, hq, d), device=dev)
        ws_bytes = m.suffix_workspace_bytes(caches[0], hq, t)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)

        def attn(i, s):
            assert L.miikv_suffix_attn(caches[i % layers].view, P(q.data_ptr()), _lib.DTYPE_F16, hq,
                                       ctypes.c_float(1 / math.sqrt(d)), t, prefix, 0, None, P(out.data_ptr()),
                                       None, None, P(ws.data_ptr()), ws_bytes, P(s.cuda_stream)) == 0
        med, p10, p90 = _graph_median(attn, layers, replays=10, warm=2)
        res[str(prefix)] = {"ms_16_layers": round(med * layers / 1e3, 3), "p10_ms": round(p10 * layers / 1e3, 3),
                            "p90_ms": round(p90 * layers / 1e3, 3), "reference_mi50_ms": ref_ms,
                            "ratio": round(ref_ms / (med * layers / 1e3), 1)}
        del caches, ws
        torch.cuda.empty_cache()
    res["note"] = ("S=512 suffix over P cached tokens, 24q/4kv/D256 q8_0, 16 layers (distinct caches), attention "
                   "only; reference: MI50, EXP-V2-0019-quantized-kv-cache.md:53-55 (other hardware)")
    return res


def chunked_prefill(dev, prefix: int = 65536, t: int = 512, layers: int = 4) -> dict:
    """The last 512-token chunk of a chunked prefill at `prefix` cached tokens (24q/4kv/
    D256, q8_0), per layer (`layers` rotated caches, each with its own workspace):
    a fresh call expands the whole context into fp16 tiles, a call with
    MIIKV_SUFFIX_TILES_CURRENT only its own steps (the earlier chunks, run the same way
    while the caches were filled, left theirs in the workspace)."""
    import ctypes

    import torch

    import miinfer_amd as m
    from miinfer_amd import _lib
    hq, hkv, d = 24, 4, 256
    L = _lib.lib()
    P = ctypes.c_void_p
    torch.manual_seed(11)
    caches, wss = [], []
    q = torch.randn((t, hq, d), device=dev).half()
    out = torch.empty((t, hq, d), device=dev)
    for _ in range(layers):
        c = m.KvCache.contiguous(hkv, d, prefix + t, device=dev)
        ws = torch.empty(m.suffix_workspace_bytes(c, hq, t), dtype=torch.uint8, device=dev)
        for base in range(0, prefix + t, t):  # the prefill, chunk by chunk, tiles kept current
            c.append(torch.randn((t, hkv, d), device=dev).half(), torch.randn((t, hkv, d), device=dev).half(),
                     base_position=base)
            assert L.miikv_suffix_attn_ex(c.view, None, None, P(q.data_ptr()), _lib.DTYPE_F16, hq,
                                          ctypes.c_float(1 / math.sqrt(d)), t, base, 0, None,
                                          _lib.SUFFIX_TILES_CURRENT, P(out.data_ptr()), None, None,
                                          P(ws.data_ptr()), ws.numel(), None) == 0
        caches.append(c)
        wss.append(ws)
    torch.cuda.synchronize()
    res = {}
    for name, flags in (("fresh_us", 0), ("current_tiles_us", _lib.SUFFIX_TILES_CURRENT)):
        def step(i, s, flags=flags):
            assert L.miikv_suffix_attn_ex(caches[i % layers].view, None, None, P(q.data_ptr()), _lib.DTYPE_F16,
                                          hq, ctypes.c_float(1 / math.sqrt(d)), t, prefix, 0, None, flags,
                                          P(out.data_ptr()), None, None, P(wss[i % layers].data_ptr()),
                                          wss[i % layers].numel(), P(s.cuda_stream)) == 0
        med, p10, p90 = _graph_median(step, layers, replays=10, warm=2)
        res[name] = round(med, 1)
    res["note"] = (f"the chunk of {t} tokens at P = {prefix}, 24q/4kv/D256 q8_0, per layer over {layers} rotated "
                   "caches and workspaces; fresh: miikv_suffix_attn (expands every key), current_tiles: "
                   "miikv_suffix_attn_ex with MIIKV_SUFFIX_TILES_CURRENT (expands the chunk's own steps)")
    del caches, wss
    torch.cuda.empty_cache()
    return res


def bench_c4(dev, args) -> int:
    """Config 4: 512-token suffix (24q/4kv/D256) over an 8192-token q8_0 prefix: append the
    512 new K/V rows, then causal suffix attention.  MFMA roofline over the visible pairs."""
    import ctypes

    import torch

    import miinfer_amd as m
    from miinfer_amd import _lib
    hq, hkv, d, prefix, t = 24, 4, 256, 8192, 512
    cache = m.KvCache.contiguous(hkv, d, prefix + t, device=dev)
    torch.manual_seed(0)
    kp = torch.randn((prefix, hkv, d), device=dev).half()
    vp = torch.randn((prefix, hkv, d), device=dev).half()
    cache.append(kp, vp)
    q = torch.randn((t, hq, d), device=dev).half()
    kn = torch.randn((t, hkv, d), device=dev).half()
    vn = torch.randn((t, hkv, d), device=dev).half()
    out = torch.empty((t, hq, d), device=dev)
    L = _lib.lib()
    P = ctypes.c_void_p
    ws_bytes = m.suffix_workspace_bytes(cache, hq, t)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)

    def append(s):
        assert L.miikv_append_f16(cache.view, P(kn.data_ptr()), P(vn.data_ptr()), t, prefix, 0,
                                  None, None, P(s.cuda_stream)) == 0

    def attn(s):
        assert L.miikv_suffix_attn(cache.view, P(q.data_ptr()), _lib.DTYPE_F16, hq,
                                   ctypes.c_float(1 / math.sqrt(d)), t, prefix, 0, None,
                                   P(out.data_ptr()), None, None, P(ws.data_ptr()), ws_bytes,
                                   P(s.cuda_stream)) == 0

    def step_unfused(s):
        append(s)
        attn(s)

    def step(s):  # the 512 new rows are quantised and stored by the expand pass of the attention
        assert L.miikv_suffix_append_attn(cache.view, P(kn.data_ptr()), P(vn.data_ptr()), P(q.data_ptr()),
                                          _lib.DTYPE_F16, hq, ctypes.c_float(1 / math.sqrt(d)), t, prefix, 0,
                                          None, P(out.data_ptr()), None, None, P(ws.data_ptr()), ws_bytes,
                                          P(s.cuda_stream)) == 0
    torch.cuda.synchronize()
    nrep = max(10, args.steps // 20)
    # 8 calls per graph replay (back to back, as a model's layers run), so the host's
    # replay cost stays out of the per-call time
    _time_graph(step, 20, 3, inner=8)  # bring the clocks up before the first timed variant
    # three interleaved rounds, median per variant (the order of variants otherwise
    # shows as ~2 us of clock drift)
    rounds = {"step": [], "unfused": [], "attn": []}
    for _ in range(3):
        for name, fn in (("step", step), ("unfused", step_unfused), ("attn", attn)):
            rounds[name].append(_time_graph(fn, max(4, nrep // 24), 3, inner=8)[0])
    us_step, us_unfused, us_attn = (sorted(rounds[k])[1] for k in ("step", "unfused", "attn"))
    us_app, _ = _time_graph(append, nrep, 5, inner=20)

    def bulk(s):  # the whole prefix again (prefill-sized append)
        assert L.miikv_append_f16(cache.view, P(kp.data_ptr()), P(vp.data_ptr()), prefix, 0, 0,
                                  None, None, P(s.cuda_stream)) == 0
    us_bulk, _ = _time_graph(bulk, nrep, 5, inner=20)

    # Short suffixes over the same prefix (speculative-verify sizes), through the same
    # entry point: they run as a batch of decodes, several tokens per context pass.
    short, short32 = {}, {}
    for ts in (1, 2, 4, 8):
        ws_s = torch.empty(m.suffix_workspace_bytes(cache, hq, ts), dtype=torch.uint8, device=dev)
        outs = out[:ts]
        for dt, qs, res in ((_lib.DTYPE_F16, q[:ts].contiguous(), short),
                            (_lib.DTYPE_F32, q[:ts].float().contiguous(), short32)):
            def attn_short(s, ts=ts, ws_s=ws_s, qs=qs, outs=outs, dt=dt):
                assert L.miikv_suffix_attn(cache.view, P(qs.data_ptr()), dt, hq,
                                           ctypes.c_float(1 / math.sqrt(d)), ts, prefix, 0, None,
                                           P(outs.data_ptr()), None, None, P(ws_s.data_ptr()),
                                           ws_s.numel(), P(s.cuda_stream)) == 0
            res[f"T{ts}_us"] = round(sorted(_time_graph(attn_short, max(4, nrep // 24), 3, inner=8)[0]
                                            for _ in range(3))[1], 2)
    # The reference's own call arguments (attention_layer.cpp:297-343): fp32 q_rope,
    # gate and gated output, on the MFMA path.
    q32 = q.float()
    gate = torch.randn((t, hq, d), device=dev)
    gated = torch.empty((t, hq, d), device=dev)

    def attn_ref(s):
        assert L.miikv_suffix_attn(cache.view, P(q32.data_ptr()), _lib.DTYPE_F32, hq,
                                   ctypes.c_float(1 / math.sqrt(d)), t, prefix, 0, None,
                                   None, P(gate.data_ptr()), P(gated.data_ptr()), P(ws.data_ptr()), ws_bytes,
                                   P(s.cuda_stream)) == 0
    us_ref = sorted(_time_graph(attn_ref, max(4, nrep // 24), 3, inner=8)[0] for _ in range(3))[1]
    # The exact route (MIIKV_SUFFIX_EXACT, fp32 query): every token as a decode.
    ws_x = torch.empty(m.suffix_workspace_bytes(cache, hq, t, exact=True), dtype=torch.uint8, device=dev)

    def attn_exact(s):
        assert L.miikv_suffix_attn_ex(cache.view, None, None, P(q32.data_ptr()), _lib.DTYPE_F32, hq,
                                      ctypes.c_float(1 / math.sqrt(d)), t, prefix, 0, None, _lib.SUFFIX_EXACT,
                                      P(out.data_ptr()), None, None, P(ws_x.data_ptr()), ws_x.numel(),
                                      P(s.cuda_stream)) == 0
    us_exact = sorted(_time_graph(attn_exact, max(4, nrep // 48), 3, inner=4)[0] for _ in range(3))[1]
    del ws_x
    ladder = suffix_ladder(dev) if not getattr(args, "no_sweep", False) else None
    chunked = chunked_prefill(dev) if not getattr(args, "no_sweep", False) else None
    pairs = sum(prefix + i + 1 for i in range(t))
    flops = 4 * hq * d * pairs
    print(json.dumps({
        "metric": "suffix attention over q8_0 prefix TFLOP/s (config 4)", "unit": "TFLOP/s",
        "value": round(flops / (us_step * 1e-6) / 1e12, 2), "us_per_step": round(us_step, 2),
        "n_gpus": 1,
        "config": {"workload": "config 4: 512-token suffix over 8192-token prefix, 24q/4kv/D256"},
        "roofline": {"bound": "mfma", "kernel": "miikv_suffix_attn = expand_kernel<256> + suffix_kernel<256> + suffix_combine_kernel<256>",
                     "achieved": round(flops / (us_attn * 1e-6) / 1e12, 2), "peak": 2500.0,
                     "unit": "TFLOP/s", "frac": round(flops / (us_attn * 1e-6) / 1e12 / 2500.0, 4),
                     "algorithmic_flops_per_launch": flops, "avg_launch_us": round(us_attn, 2)},
        "step": "miikv_suffix_append_attn (store the 512 new rows + attend, one pass)",
        "us_per_step_append_then_attend": round(us_unfused, 2),
        "split_workspace_bytes": ws_bytes,
        "append": {"us": round(us_app, 2), "rows": t * hkv,
                   "GBs": round(t * append_bytes(hkv, d) / (us_app * 1e-6) / 1e9, 1)},
        "append_bulk": {"us": round(us_bulk, 2), "tokens": prefix,
                        "GBs": round(prefix * append_bytes(hkv, d) / (us_bulk * 1e-6) / 1e9, 1)},
        "short_suffix": dict(short, note="miikv_suffix_attn with T tokens over the same 8192-token prefix "
                                         "(a batch of decodes, 2 tokens per context pass)"),
        "short_suffix_f32_query": dict(short32, note="the same with an fp32 query (its low half kept)"),
        "reference_signature": {"us": round(us_ref, 2), "TFLOPs": round(flops / (us_ref * 1e-6) / 1e12, 2),
                                "note": "miikv_suffix_attn with an fp32 query, gate and gated output (the "
                                        "reference's arguments), MFMA path"},
        "exact_route": {"us": round(us_exact, 2), "TFLOPs": round(flops / (us_exact * 1e-6) / 1e12, 2),
                        "note": "miikv_suffix_attn_ex with MIIKV_SUFFIX_EXACT and an fp32 query: the exact-product "
                                "MFMA kernels (key codes exact with the block scales in fp32, the query's low half in "
                                "the spare MFMA columns)"},
        "reference_ladder": ladder,
        "chunked_prefill": chunked,
    }), flush=True)
    return 0


def bench_c5(dev, args) -> int:
    """Config 5: 64 sessions forked from a shared 32768-token prefix of a hybrid model:
    16 attention layers (4 kv heads x D256 q8_0, 256-token pages) and 48 GDN layers
    (fp32 state 16x128x128 + conv 8192x3).  Each fork shares the prefix pages (block
    table + reference counts), copies the last partial page (copy-on-write), and clones
    the full recurrent state.  Timed: the device work of all 64 forks."""
    import numpy as np
    import torch

    import miinfer_amd as m
    from miinfer_amd import reuse
    hkv, d, pt, layers_attn, forks = 4, 256, 256, 16, 64
    state, conv, layers_gdn = 16 * 128 * 128, 8192 * 3, 48
    results = {}
    for prefix in (32768, 32768 - 100):
        pages = (prefix + pt - 1) // pt
        npool = pages + forks + 1
        caches, pools, tables = [], [], []
        for _ in range(layers_attn):
            pool = reuse.PagePool(npool)
            row = np.array([pool.alloc() for _ in range(pages)], np.int32)
            cache = m.KvCache.paged_cache(hkv, d, npool, torch.from_numpy(row[None]).to(dev),
                                          page_tokens=pt, device=dev)
            for t in (cache.k_codes, cache.v_codes):
                t.copy_(torch.randint(-128, 128, t.shape, dtype=torch.int8, device=dev))
            for t in (cache.k_scales, cache.v_scales):
                t.copy_(torch.randint(0, 2**15, t.shape, dtype=torch.int16, device=dev))
            caches.append(cache)
            pools.append(pool)
            tables.append(row)
        parent = reuse.RecurrentStates(layers_gdn, state, conv, device=dev)
        parent.buf.copy_(torch.randn(parent.buf.numel(), device=dev))
        kids = [reuse.RecurrentStates(layers_gdn, state, conv, device=dev) for _ in range(forks)]
        # host planning: 64 forks per attention layer
        t0 = time.perf_counter()
        copies = []
        for li in range(layers_attn):
            _, cl = pools[li].fork_many(tables[li], prefix, pt, forks)
            copies.append(cl)
        host_s = time.perf_counter() - t0
        src = [torch.tensor([c[0] for c in cl], dtype=torch.int32, device=dev) for cl in copies]
        dst = [torch.tensor([c[1] for c in cl], dtype=torch.int32, device=dev) for cl in copies]
        ptrs = torch.tensor([k.buf.data_ptr() for k in kids], dtype=torch.int64, device=dev)
        import ctypes

        from miinfer_amd import _lib
        L = _lib.lib()

        def device_work(s):
            for li in range(layers_attn):
                if len(copies[li]):
                    assert L.miikv_copy_pages(caches[li].view, ctypes.c_void_p(src[li].data_ptr()),
                                              ctypes.c_void_p(dst[li].data_ptr()), len(copies[li]),
                                              ctypes.c_void_p(s.cuda_stream)) == 0
            assert L.miikv_clone_state(ctypes.c_void_p(ptrs.data_ptr()),
                                       ctypes.c_void_p(parent.buf.data_ptr()), parent.nbytes, forks,
                                       ctypes.c_void_p(s.cuda_stream)) == 0
        torch.cuda.synchronize()
        us, n = _time_graph(device_work, max(5, args.steps // 200), 3)
        # byte-exact spot checks of the timed work
        assert torch.equal(kids[-1].buf.view(torch.int32), parent.buf.view(torch.int32))
        if copies[0]:
            s0, d0 = copies[0][-1]
            per = caches[0].k_codes.numel() // npool
            assert torch.equal(caches[0].k_codes.view(npool, per)[d0], caches[0].k_codes.view(npool, per)[s0])
        page_bytes = 2 * hkv * pt * (d + d // 16)
        cow = sum(len(c) for c in copies) * page_bytes * 2
        clone = parent.nbytes * (1 + forks)
        results[str(prefix)] = {
            "us": round(us, 1), "GBs": round((cow + clone) / (us * 1e-6) / 1e9, 1),
            "cow_pages": sum(len(c) for c in copies), "cow_bytes_rw": cow, "clone_bytes_rw": clone,
            "host_planning_us": round(host_s * 1e6, 1)}
        del caches, kids, parent
        torch.cuda.empty_cache()
    main_r = results[str(32768 - 100)]
    print(json.dumps({
        "metric": "fork 64 sessions: CoW pages + recurrent-state clone, GB/s (config 5)",
        "unit": "GB/s", "value": main_r["GBs"], "n_gpus": 1,
        "config": {"workload": "config 5: 64 forks, 16 attn layers (4kv x D256 q8_0, 256-token "
                               "pages) + 48 GDN layers (16x128x128 + 8192x3 fp32)"},
        "by_prefix_tokens": results,
        "roofline": {"bound": "hbm", "kernel": "copy_pages_kernel + clone_state_kernel",
                     "achieved": main_r["GBs"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(main_r["GBs"] / PEAK_HBM_GBS, 4)},
    }), flush=True)
    return 0


def calibrate_copy(dev) -> int:
    """A plain 256 MiB device-to-device copy through miikv_copy_segments: its
    FETCH_SIZE / WRITE_SIZE under rocprofv3 --pmc give the counter scale factor."""
    import torch

    import miinfer_amd as m
    n = 256 << 20
    src = torch.ones(n, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(5):
        m.copy_segments([(dst.data_ptr(), src.data_ptr(), n)], device=dev)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "copy_segments_kernel", "bytes_read": n, "bytes_written": n}))
    return 0


def stream_read_ceiling(dev, span_bytes: int, spans: int = 8, reps: int = 20) -> dict:
    """Cold single-pass read of `span_bytes` (rotating over `spans` buffers so the
    256 MB Infinity Cache does not serve it), timed like the decode step: back-to-back
    launches captured in one graph.  The practical per-launch ceiling of a kernel
    streaming the same bytes on this device."""
    import ctypes

    import torch

    from miinfer_amd import _lib
    blocks = 2048
    span = span_bytes // (16 * blocks) * (16 * blocks)
    buf = torch.ones(span * spans, dtype=torch.uint8, device=dev)
    sink = torch.empty(blocks, dtype=torch.int32, device=dev)
    lib = _lib.lib()
    counter = [0]

    def read(s):
        i = counter[0] % spans
        counter[0] += 1
        st = lib.miikv_stream_read(ctypes.c_void_p(buf.data_ptr() + i * span), span,
                                   ctypes.c_void_p(sink.data_ptr()), blocks, ctypes.c_void_p(s.cuda_stream))
        if st:
            raise RuntimeError(f"stream probe failed: {st}")
    us, _ = _time_graph(read, reps, 3, inner=8 * spans)
    del buf
    return {"bytes": span, "us_per_launch": round(us, 2), "GBs": round(span / (us * 1e-6) / 1e9, 1),
            "note": "miikv_stream_read, 2048x256 threads, 16 B nontemporal loads, cold (rotating "
                    f"{spans} spans), {8 * spans} back-to-back launches per graph replay"}


def _graph_median(fn, steps_per_graph: int, replays: int = 30, warm: int = 5):
    """Capture fn(i, stream) for i < steps_per_graph into one graph; per-replay HIP
    events; returns (median, p10, p90) us per step."""
    import torch
    stream = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for i in range(steps_per_graph):
            fn(i, torch.cuda.current_stream())
    times = []
    with torch.cuda.stream(stream):
        for _ in range(warm):
            g.replay()
        for _ in range(replays):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            g.replay()
            e1.record(stream)
            e1.synchronize()
            times.append(e0.elapsed_time(e1) * 1e3 / steps_per_graph)
    times.sort()
    return times[len(times) // 2], times[len(times) // 10], times[(9 * len(times)) // 10]


def decode_variants(dev, ctx: int = 32768, nl: int = 8) -> dict:
    """More config 2 lines at 32k, same rotation and protocol as the headline:
    * reference_signature: the drop-in call sequence of the reference's decode step
      (attention_layer.cpp:599-632): miikv_append_f32 with the fused K RMSNorm + RoPE
      prologue on fp32 rows at the decode-state position, then miikv_decode_attn_q8_1 with
      an fp32 query, gate, gated output and the Q8_1 epilogue;
    * reference_signature_fused: the same arguments through miikv_decode_append_attn_f32
      (one launch pair);
    * fp16_control: attention over an FP16_FP16 cache (the reference's production default,
      qwen3_primitives.hip:2198-2293), attention only, 2x the KV bytes of q8_0."""
    import ctypes

    import torch

    import miinfer_amd as m
    from miinfer_amd import _lib
    L = _lib.lib()
    P = ctypes.c_void_p
    torch.manual_seed(5)
    out = {}
    # reference-signature step over q8_0 caches
    caches = []
    for _ in range(nl):
        c = m.KvCache.contiguous(HKV, D, ctx, device=dev)
        for t0 in range(0, ctx, 8192):
            n = min(8192, ctx - t0)
            c.append(torch.randn((n, HKV, D), device=dev).half(), torch.randn((n, HKV, D), device=dev).half(),
                     base_position=t0)
        caches.append(c)
    q32 = torch.randn((1, HQ, D), device=dev)
    gate = torch.randn((1, HQ, D), device=dev)
    gated = torch.empty((1, HQ, D), device=dev)
    q81 = torch.empty(HQ * D // 32 * 36, dtype=torch.uint8, device=dev)
    k32 = torch.randn((1, HKV, D), device=dev)
    v32 = torch.randn((1, HKV, D), device=dev)
    w = torch.rand(D, device=dev) + 0.5
    ds = m.make_decode_state(ctx - 1, device=dev)
    ws = m.DecodeWorkspace(caches[0], HQ, 1, ctx)

    def ref_step(i, s):
        c = caches[i % nl]
        assert L.miikv_append_f32(c.view, P(k32.data_ptr()), P(v32.data_ptr()), P(w.data_ptr()), 1, 0, 0,
                                  ctypes.c_float(1.0e6), ctypes.c_float(1e-6), None, P(ds.data_ptr()),
                                  P(s.cuda_stream)) == 0
        assert L.miikv_decode_attn_q8_1(c.view, P(q32.data_ptr()), _lib.DTYPE_F32, HQ,
                                        ctypes.c_float(1 / math.sqrt(D)), 1, None, P(ds.data_ptr()), ctx, None,
                                        P(gate.data_ptr()), P(gated.data_ptr()), P(q81.data_ptr()),
                                        P(ws.buf.data_ptr()), ws.bytes, P(s.cuda_stream)) == 0
    med, p10, p90 = _graph_median(ref_step, 8 * nl)
    nbytes = decode_bytes(ctx) + 2 * HKV * D * 4 + kv_bytes_per_token() + HQ * D * 4 * 2
    out["reference_signature"] = {
        "calls": "miikv_append_f32 (K RMSNorm + RoPE prologue, fp32 rows, decode state) + "
                 "miikv_decode_attn_q8_1 (fp32 query, gate, gated output, Q8_1 blocks)",
        "us_median": round(med, 3), "us_p10": round(p10, 3), "us_p90": round(p90, 3),
        "GBs_median": round(nbytes / (med * 1e-6) / 1e9, 1)}

    def ref_fused(i, s):
        c = caches[i % nl]
        assert L.miikv_decode_append_attn_f32(c.view, P(k32.data_ptr()), P(v32.data_ptr()), P(w.data_ptr()),
                                              ctypes.c_float(1.0e6), ctypes.c_float(1e-6), P(q32.data_ptr()),
                                              _lib.DTYPE_F32, HQ, ctypes.c_float(1 / math.sqrt(D)), 1, None,
                                              P(ds.data_ptr()), ctx, None, P(gate.data_ptr()), P(gated.data_ptr()),
                                              P(q81.data_ptr()), P(ws.buf.data_ptr()), ws.bytes,
                                              P(s.cuda_stream)) == 0
    med, p10, p90 = _graph_median(ref_fused, 8 * nl)
    out["reference_signature_fused"] = {
        "calls": "miikv_decode_append_attn_f32 (the same arguments in one launch pair)",
        "us_median": round(med, 3), "us_p10": round(p10, 3), "us_p90": round(p90, 3),
        "GBs_median": round(nbytes / (med * 1e-6) / 1e9, 1)}
    del caches
    torch.cuda.empty_cache()
    # fp16 control
    caches = []
    for _ in range(nl):
        c = m.KvCache.contiguous(HKV, D, ctx, device=dev, quant_mode=_lib.KV_FP16_FP16)
        for t0 in range(0, ctx, 8192):
            n = min(8192, ctx - t0)
            c.append(torch.randn((n, HKV, D), device=dev).half(), torch.randn((n, HKV, D), device=dev).half(),
                     base_position=t0)
        caches.append(c)
    q = torch.randn((1, HQ, D), device=dev).half()
    o = torch.empty((1, HQ, D), device=dev)
    lens = torch.tensor([ctx], dtype=torch.int32, device=dev)
    ws = m.DecodeWorkspace(caches[0], HQ, 1, ctx)

    def f16_step(i, s):
        assert L.miikv_decode_attn(caches[i % nl].view, P(q.data_ptr()), _lib.DTYPE_F16, HQ,
                                   ctypes.c_float(1 / math.sqrt(D)), 1, P(lens.data_ptr()), None, ctx,
                                   P(o.data_ptr()), None, None, P(ws.buf.data_ptr()), ws.bytes,
                                   P(s.cuda_stream)) == 0
    med, p10, p90 = _graph_median(f16_step, 8 * nl)
    fbytes = ctx * 2 * HKV * D * 2 + HQ * D * 6
    out["fp16_control"] = {
        "kv_mode": "FP16_FP16", "us_median": round(med, 3), "us_p10": round(p10, 3), "us_p90": round(p90, 3),
        "GBs_median": round(fbytes / (med * 1e-6) / 1e9, 1), "kv_bytes_per_launch": fbytes}
    del caches
    torch.cuda.empty_cache()
    out["reference_decode_ladder"] = reference_decode_ladder(dev)
    return out


# The reference's published split-K decode attention (fp16 K/V, one layer, 24q/4kv/D256;
# MI50, experiments/EXP-0203-wave64-barrier-free-splitk-attention.md:42-46), ms.
REFERENCE_DECODE_FP16_MI50_MS = {4096: 0.393, 16384: 0.762, 32768: 1.032, 65536: 1.893}


def reference_decode_ladder(dev, nl: int = 8) -> dict:
    """Decode attention at the reference's decode-ladder shape (24q/4kv/D256, batch 1,
    one query token) and contexts, fp16 K/V (its kernel's format) and q8_0, cold (nl
    rotated layer caches), attention only; beside the reference's MI50 figures (other
    hardware, not a like-for-like baseline)."""
    import ctypes

    import torch

    import miinfer_amd as m
    from miinfer_amd import _lib
    hq, hkv, d = 24, 4, 256
    L = _lib.lib()
    P = ctypes.c_void_p
    res = {}
    for ctx, ref_ms in REFERENCE_DECODE_FP16_MI50_MS.items():
        row = {"reference_mi50_fp16_ms": ref_ms}
        for name, mode in (("fp16", _lib.KV_FP16_FP16), ("q8_0", _lib.KV_Q8_Q8)):
            torch.manual_seed(ctx)
            caches = []
            for _ in range(nl):
                c = m.KvCache.contiguous(hkv, d, ctx, device=dev, quant_mode=mode)
                for t0 in range(0, ctx, 8192):
                    n = min(8192, ctx - t0)
                    c.append(torch.randn((n, hkv, d), device=dev).half(), torch.randn((n, hkv, d), device=dev).half(),
                             base_position=t0)
                caches.append(c)
            q = torch.randn((1, hq, d), device=dev).half()
            o = torch.empty((1, hq, d), device=dev)
            lens = torch.tensor([ctx], dtype=torch.int32, device=dev)
            ws = m.DecodeWorkspace(caches[0], hq, 1, ctx)

            def step(i, s, caches=caches, q=q, o=o, lens=lens, ws=ws):
                assert L.miikv_decode_attn(caches[i % nl].view, P(q.data_ptr()), _lib.DTYPE_F16, hq,
                                           ctypes.c_float(1 / math.sqrt(d)), 1, P(lens.data_ptr()), None, ctx,
                                           P(o.data_ptr()), None, None, P(ws.buf.data_ptr()), ws.bytes,
                                           P(s.cuda_stream)) == 0
            med, p10, p90 = _graph_median(step, 4 * nl, replays=20, warm=3)
            kv_bytes = ctx * 2 * hkv * (2 * d if mode == _lib.KV_FP16_FP16 else d + 2 * (d // 32))
            row[name + "_us"] = round(med, 2)
            row[name + "_GBs"] = round(kv_bytes / (med * 1e-6) / 1e9, 1)
            del caches, ws
            torch.cuda.empty_cache()
        res[str(ctx)] = row
    res["note"] = ("decode attention, 24q/4kv/D256, batch 1, cold over rotated layer caches; reference: fp16 "
                   "K/V on MI50, EXP-0203-wave64-barrier-free-splitk-attention.md:42-46 (other hardware)")
    return res


def decode_at(dev, ctx: int, nl: int, replays: int = 30) -> dict:
    """Fused append + decode (config 2 shape) at context `ctx` over `nl` rotated layer
    caches: per-replay HIP-event times (one replay = 8 rounds over the layers) give the
    median and p10/p90 per layer-token."""
    import ctypes

    import torch

    import miinfer_amd as m
    from miinfer_amd import _lib
    torch.manual_seed(ctx)
    caches = []
    for _ in range(nl):
        c = m.KvCache.contiguous(HKV, D, ctx, device=dev)
        for t0 in range(0, ctx, 8192):
            n = min(8192, ctx - t0)
            c.append(torch.randn((n, HKV, D), device=dev).half(), torch.randn((n, HKV, D), device=dev).half(),
                     base_position=t0)
        caches.append(c)
    q = torch.randn((1, HQ, D), device=dev).half()
    kn = torch.randn((1, HKV, D), device=dev).half()
    vn = torch.randn((1, HKV, D), device=dev).half()
    out = torch.empty((1, HQ, D), device=dev)
    lens = torch.tensor([ctx], dtype=torch.int32, device=dev)
    ws = m.DecodeWorkspace(caches[0], HQ, 1, ctx)
    L = _lib.lib()
    P = ctypes.c_void_p
    stream = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for i in range(8 * nl):
            st = L.miikv_decode_append_attn(caches[i % nl].view, P(kn.data_ptr()), P(vn.data_ptr()),
                                            P(q.data_ptr()), _lib.DTYPE_F16, HQ, ctypes.c_float(1 / math.sqrt(D)),
                                            1, P(lens.data_ptr()), None, ctx, P(out.data_ptr()), None, None,
                                            None, P(ws.buf.data_ptr()), ws.bytes,
                                            P(torch.cuda.current_stream().cuda_stream))
            assert st == 0, st
    times = []
    with torch.cuda.stream(stream):
        for _ in range(5):
            g.replay()
        for _ in range(replays):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            g.replay()
            e1.record(stream)
            e1.synchronize()
            times.append(e0.elapsed_time(e1) * 1e3 / (8 * nl))
    times.sort()
    med = times[len(times) // 2]
    nbytes = decode_bytes(ctx) + append_bytes()
    del caches
    return {"context": ctx, "layers_rotated": nl, "working_set_mb": round(nl * ctx * kv_bytes_per_token() / 1e6, 1),
            "us_median": round(med, 3), "us_p10": round(times[len(times) // 10], 3),
            "us_p90": round(times[(9 * len(times)) // 10], 3),
            "GBs_median": round(nbytes / (med * 1e-6) / 1e9, 1)}


def traffic_from_profile():
    """HBM bytes per decode launch measured with rocprofv3 --pmc (FETCH_SIZE +
    WRITE_SIZE, scaled by the copy calibration), from the committed summary."""
    path = os.path.join(ROOT, "profiles", "decode_attn_c2_32k_pmc.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":", 1)[1]))
    return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=6400)
    ap.add_argument("--warmup", type=int, default=640)
    ap.add_argument("--context", type=int, default=32768)
    ap.add_argument("--layers", type=int, default=8)
    ap.add_argument("--repeats", type=int, default=10,
                    help="timed blocks of --steps steps each (median and p10/p90 over them)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--no-sweep", action="store_true",
                    help="config 2 at 32k only (skip the 4k/16k and hot-cache lines)")
    ap.add_argument("--workload", default="c2", choices=["c2", "c3", "c4", "c5"],
                    help="c2 (default, the headline metric); c3 paged batched decode; c4 suffix "
                         "attention (these print their own JSON line, not the headline)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run only a 256 MiB device copy (known bytes) to calibrate PMC counters")
    args = ap.parse_args()
    if args.steps < 1:
        ap.error("--steps must be at least 1")
    if args.repeats < 1:
        ap.error("--repeats must be at least 1")
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this path runs on a single MI355X "
              "(it would shard by kv head or by sequence with no exchange; only one GPU's share runs here)", file=sys.stderr)
        return 2

    import torch

    import miinfer_amd as m
    from miinfer_amd import _lib

    dev = torch.device("cuda:0")
    if args.calibrate_copy:
        return calibrate_copy(dev)
    if args.workload == "c3":
        return bench_c3(dev, args)
    if args.workload == "c4":
        return bench_c4(dev, args)
    if args.workload == "c5":
        return bench_c5(dev, args)
    ctx, nl = args.context, args.layers
    torch.manual_seed(0)
    caches = []
    for _ in range(nl):
        c = m.KvCache.contiguous(HKV, D, ctx, device=dev)
        for t0 in range(0, ctx, 4096):
            n = min(4096, ctx - t0)
            k = torch.randn((n, HKV, D), device=dev).half()
            v = torch.randn((n, HKV, D), device=dev).half()
            c.append(k, v, base_position=t0)
        caches.append(c)
    q = [torch.randn((1, HQ, D), device=dev).half() for _ in range(nl)]
    knew = [torch.randn((1, HKV, D), device=dev).half() for _ in range(nl)]
    vnew = [torch.randn((1, HKV, D), device=dev).half() for _ in range(nl)]
    outs = [torch.empty((1, HQ, D), device=dev) for _ in range(nl)]
    lens = torch.tensor([ctx], dtype=torch.int32, device=dev)
    ws = m.DecodeWorkspace(caches[0], HQ, 1, ctx)
    torch.cuda.synchronize()

    L = _lib.lib()
    scale = 1.0 / math.sqrt(D)
    import ctypes

    def step(i, stream):
        c = caches[i % nl]
        s = ctypes.c_void_p(stream.cuda_stream)
        # one fused launch pair: store the new K/V row at ctx-1, attend over ctx keys
        st = L.miikv_decode_append_attn(c.view, ctypes.c_void_p(knew[i % nl].data_ptr()),
                                        ctypes.c_void_p(vnew[i % nl].data_ptr()),
                                        ctypes.c_void_p(q[i % nl].data_ptr()), _lib.DTYPE_F16, HQ,
                                        ctypes.c_float(scale), 1, ctypes.c_void_p(lens.data_ptr()),
                                        None, ctx, ctypes.c_void_p(outs[i % nl].data_ptr()), None,
                                        None, None, ctypes.c_void_p(ws.buf.data_ptr()), ws.bytes, s)
        if st:
            raise RuntimeError(f"launch failed: {st}")

    def decode_only(i, stream):
        c = caches[i % nl]
        st = L.miikv_decode_attn(c.view, ctypes.c_void_p(q[i % nl].data_ptr()), _lib.DTYPE_F16,
                                 HQ, ctypes.c_float(scale), 1, ctypes.c_void_p(lens.data_ptr()),
                                 None, ctx, ctypes.c_void_p(outs[i % nl].data_ptr()), None, None,
                                 ctypes.c_void_p(ws.buf.data_ptr()), ws.bytes,
                                 ctypes.c_void_p(stream.cuda_stream))
        if st:
            raise RuntimeError(f"launch failed: {st}")

    stream = torch.cuda.Stream()
    graph_steps = nl * 8  # one full graph = 8 rounds over the layer caches

    def make_graph(fn, n):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for i in range(n):
                fn(i, torch.cuda.current_stream())
        return g

    use_graph = not args.no_graph
    full, rem = divmod(args.steps, graph_steps)
    graphs = {}
    if use_graph:
        try:
            for kind, fn in (("step", step), ("decode", decode_only)):
                graphs[kind] = make_graph(fn, graph_steps)
                if rem:
                    graphs[kind + "_rem"] = make_graph(fn, rem)
        except Exception as e:  # pragma: no cover - reported, then eager launches
            print(f"graph capture failed ({e}); timing eager launches", file=sys.stderr)
            use_graph = False

    def run(kind, nsteps, timed=True):
        """Run exactly nsteps steps of `kind` on `stream`: full graph replays, then one
        replay of the remainder graph.  Returns (total ms, per-replay us per step of the
        full replays, or of the remainder when there is none)."""
        nfull, nrem = divmod(nsteps, graph_steps)
        marks = []
        with torch.cuda.stream(stream):
            ev = torch.cuda.Event(enable_timing=True)
            ev.record(stream)
            marks.append(ev)
            if use_graph:
                for _ in range(nfull):
                    graphs[kind].replay()
                    ev = torch.cuda.Event(enable_timing=True)
                    ev.record(stream)
                    marks.append(ev)
                if nrem:
                    (graphs[kind + "_rem"] if nrem == rem else make_graph(
                        step if kind == "step" else decode_only, nrem)).replay()
                    ev = torch.cuda.Event(enable_timing=True)
                    ev.record(stream)
                    marks.append(ev)
            else:
                fn = step if kind == "step" else decode_only
                for i in range(nsteps):
                    fn(i, stream)
                ev = torch.cuda.Event(enable_timing=True)
                ev.record(stream)
                marks.append(ev)
        marks[-1].synchronize()
        total = marks[0].elapsed_time(marks[-1])
        if not timed:
            return total, []
        if use_graph and nfull:
            per = [marks[i].elapsed_time(marks[i + 1]) * 1e3 / graph_steps for i in range(nfull)]
        else:
            per = [total * 1e3 / nsteps]
        return total, per

    def stats(per):
        per = sorted(per)
        return statistics.median(per), per[len(per) // 10], per[(9 * len(per)) // 10]

    # At least --warmup steps, in whole replays and no fewer than five (clocks and the
    # graphs' first-replay upload settle), and one replay of each remainder graph.
    warm = max(-(-max(args.warmup, 1) // graph_steps), 5) * graph_steps
    for kind in ("step", "decode"):
        run(kind, warm, timed=False)
        if rem:
            run(kind, rem, timed=False)
    # The timed block is exactly --steps steps; it is repeated `repeats` times so that
    # the headline is a median with a real spread (per block: total time / steps).
    repeats = args.repeats
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    blocks = [run("step", args.steps, timed=False)[0] for _ in range(repeats)]
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_start
    blocks_dec = [run("decode", args.steps, timed=False)[0] for _ in range(repeats)]
    per = [b * 1e3 / args.steps for b in blocks]
    per_dec = [b * 1e3 / args.steps for b in blocks_dec]
    ms = statistics.median(blocks)

    us_step, us_p10, us_p90 = stats(per)
    us_dec, us_dec_p10, us_dec_p90 = stats(per_dec)
    step_bytes = decode_bytes(ctx) + append_bytes()
    value = step_bytes / (us_step * 1e-6) / 1e9
    dec_gbs = decode_bytes(ctx) / (us_dec * 1e-6) / 1e9

    # correctness spot check of the timed path (cheap): the output is finite
    assert bool(torch.isfinite(outs[0]).all())

    line = {
        "metric": "decode-attn q8_0 KV GB/s (% HBM peak) + us/layer/token at 32k ctx",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us_step / 1e3, 6),
        "us_per_layer_token": round(us_step, 3),
        "us_per_layer_token_p10": round(us_p10, 3),
        "us_per_layer_token_p90": round(us_p90, 3),
        "timing": {"steps_requested": args.steps, "steps_per_block": args.steps, "repeats": repeats,
                   "block_ms_median": round(ms, 4), "block_ms_all": [round(b, 4) for b in blocks],
                   "samples": len(per),
                   "protocol": f"a timed block is exactly --steps steps (graph replays of {graph_steps} "
                               f"steps, 8 rounds over {nl} rotated layer caches, plus one replay of the "
                               "remainder), HIP events around the block; the block runs --repeats times "
                               "after the warmup; value and us_per_layer_token are the median over the "
                               "blocks of block time / steps, p10/p90 beside them"},
        "pct_hbm_peak": round(100 * value / PEAK_HBM_GBS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 KV codes (q8_0) x fp16 query, fp32 accumulate",
        "data": "synthetic N(0,1) fp16 K/V/q from seed, resident in HBM",
        "config": {"workload": "config 2: GQA decode 32q/8kv/D128, batch 1, ctx 32768, q8_0-32 KV, "
                               "append 1 row per kv head then attend (fused in one launch pair)",
                   "context": ctx, "layers_rotated": nl, "graph": use_graph,
                   "wall_s_timed": round(wall, 3)},
        "roofline": {"bound": "hbm",
                     "kernel": "miikv_decode_append_attn = decode_kernel<128,false,true> + combine_kernel<128>",
                     "achieved": round(value, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(value / PEAK_HBM_GBS, 4), "traffic": traffic_from_profile(),
                     "algorithmic_bytes_per_launch": step_bytes,
                     "avg_launch_us": round(us_step, 3)},
        "decode_only": {"kernel": "miikv_decode_attn = decode_kernel<128,false,false> + combine_kernel<128>",
                        "avg_launch_us": round(us_dec, 3), "p10_us": round(us_dec_p10, 3),
                        "p90_us": round(us_dec_p90, 3), "GBs": round(dec_gbs, 1),
                        "algorithmic_bytes_per_launch": decode_bytes(ctx)},
    }
    line["roofline"]["stream_read_ceiling"] = stream_read_ceiling(dev, decode_bytes(ctx))
    if not args.no_sweep:
        del caches, graphs
        caches = graphs = None
        torch.cuda.empty_cache()
        line.update(decode_variants(dev, ctx, nl))
    # The other contexts of config 2, cold (enough rotated layers to exceed the 256 MB
    # Infinity Cache) and hot (one layer, MALL-resident), with per-replay spread.
    if not args.no_sweep:
        line["contexts"] = {
            "cold": [decode_at(dev, c, max(8, -(-300_000_000 // (c * kv_bytes_per_token())))) for c in (4096, 16384, 32768)],
            "hot": [decode_at(dev, c, 1) for c in (4096, 16384, 32768)],
        }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
