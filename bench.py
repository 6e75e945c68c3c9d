#!/usr/bin/env python3
"""Benchmark of the MI355X attention hot path (one GPU).

    python bench.py [--steps K] [--warmup W] [--no-cpu] [--no-extra]

Headline ("config 2"): one step = 48 sequential
decode-attention calls, one per layer, each over 4,096 cached positions of a
fp32 KV cache (GQA 32/4, head_dim 128), through the C ABI with device
pointers. The step is captured once into a HIP graph and replayed, the way a
serving loop runs its per-token layer sequence; inputs are resident in HBM
before timing starts. `value` is the unique K+V+q+out bytes of all 48 calls
per second of wall time (GB/s). The eager (one host call per layer) step time
is reported beside it.

`roofline` is for the dominant kernel (the decode tile kernel): algorithmic
bytes per launch over its average duration, given two ways. `trace` is the
rocprofv3 kernel-trace average recorded in the committed summary of this
same command (profiles/decode_tile_ctx4096_f32.md: the kernel's execution
window); `events` is this run's own, timed live over eager steps with HIP
events that the kernel launch itself fills on the launch stream
(RV_TUNE_KERNEL_TIMING, hipExtLaunchKernelGGL), which also hold the launch's
dispatch latency. `frac_source` names the one `frac` uses (the trace when
the summary records it). `traffic` is the HBM bytes per launch from the same
summary's counter passes.

`roofline.whole_call` is the same bytes over the whole call's time per layer
(tile kernel + split-merge kernel, from the graph replay).

`extra` carries the other configurations: prefill TFLOP/s of configs 3 and 4
in the three arithmetic modes, the long-context f16 decode of config 5 (the
library's own split plan and BASELINE's 8 / 16 / 32 splits per kv head), the
fused decode step of config 1, the decode context ladder (f16 cache, 64 ..
32,768 positions, a 1-layer and a 48-layer arm, as benches/kernels.rs:168,
:691-738), the widening legs (projections, batched projections, router,
attention block), and each config's CPU baseline. `cpu_baseline` is the C
restatement of the reference's CPU decode path (oracle/, AVX2+F16C, kv-head
fan-out over 4 threads) on a bounded sample of config 2; the prefill
baselines time the whole 512-row chunk over the box's cores (at most 16).

Prints exactly one JSON line on stdout; progress goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0  # dense fp16/bf16
DECODE_PROFILE = os.path.join(ROOT, "profiles", "decode_tile_ctx4096_f32.md")
CONFIG5_PROFILE = os.path.join(ROOT, "profiles", "decode_tile_ctx32768_f16.md")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def decode_bytes(positions: int, elem_bytes: int) -> int:
    """Algorithmic bytes of one decode call: the layer's K and V head slices
    read once, q read, out written (benches/kernels.rs:245-270 convention)."""
    return 2 * positions * 512 * elem_bytes + 2 * 4096 * 4


def prefill_flops(rows: int, start: int) -> int:
    """4 * d * causal pairs * heads, pairs = rows*start + rows*(rows+1)/2."""
    pairs = rows * start + rows * (rows + 1) // 2
    return 4 * 128 * pairs * 32


def timed(torch, fn, iters: int) -> float:
    """Wall seconds of `iters` calls, synchronised on both sides."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(iters):
        fn()
    torch.cuda.synchronize()
    return time.perf_counter() - t0


def kernel_avg(torch, kv, fn, iters: int, lead_cycles: int = 0):
    """Average dominant-kernel duration (s) over `iters` eager calls of fn,
    from the library's HIP events on the launch stream.

    With lead_cycles, each call is queued behind a bounded spin of that many
    GPU clock cycles (torch.cuda._sleep: no memory traffic, not timed), so the
    host gets ahead of the GPU and the timed kernels run back to back as in a
    graph replay; without it, a host that submits more slowly than the GPU
    drains leaves the GPU idle between launches and the event spans grow by
    ~3 us (seen on some boxes, with unchanged kernel execution windows in the
    trace)."""
    kv.set_tuning(7, 1)
    kv.kernel_time()  # reset
    for _ in range(iters):
        if lead_cycles:
            torch.cuda._sleep(lead_cycles)
        fn()
    ms, n = kv.kernel_time()
    kv.set_tuning(7, 0)
    return (ms / 1e3 / n) if n else None, n


def profile_value(path: str, key: str):
    """A `key: value` figure recorded in a committed rocprofv3 summary."""
    try:
        with open(path) as f:
            m = re.search(key + r":\s*([0-9.]+)", f.read())
        return float(m.group(1)) if m else None
    except OSError:
        return None


def traffic_from_profile(path: str):
    """HBM bytes per launch recorded in a committed counter summary."""
    return profile_value(path, "traffic_bytes_per_launch")


def bench_config2(torch, rv, synth, steps, warmup):
    log("config 2: building 48-layer fp32 cache at ctx 4096 ...")
    kv = rv.KvCache(48, 4, 128, 4096, "f32")
    for layer in range(48):
        K, V = synth.cached_kv(2, layer, 4096)
        kv.append_rows(layer, K, V)
    del K, V
    q = torch.stack([torch.from_numpy(synth.normal(synth.seed(2, synth.T_Q, l), synth.Q_DIM)) for l in range(48)]).cuda()
    out = torch.zeros_like(q)
    qs = [q[l] for l in range(48)]
    outs = [out[l] for l in range(48)]
    scale = float(synth.SCALE)

    def step():
        for l in range(48):
            rv.decode_attention(qs[l], kv, l, scale, None, outs[l])

    for _ in range(warmup):
        step()
    eager = timed(torch, step, steps) / steps
    ref = out.clone()

    # The same step captured once and replayed.
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for _ in range(warmup):
        graph.replay()
    per_step = timed(torch, graph.replay, steps) / steps
    # The replay must rewrite every output: start it from NaN.
    out.fill_(float("nan"))
    graph.replay()
    torch.cuda.synchronize()
    graph_ok = bool(torch.equal(out, ref))

    byts = decode_bytes(4096, 4)
    # ~1 ms of GPU spin ahead of each 48-layer step, longer than the host
    # needs to queue the step.
    k_avg, k_n = kernel_avg(torch, kv, step, max(1, min(steps, 50)), lead_cycles=2_000_000)
    return {
        "kv": kv, "graph": graph, "graph_matches_eager": graph_ok,
        "ms_per_step": per_step * 1e3,
        "value_gbs": 48 * byts / per_step / 1e9,
        "us_per_layer": per_step / 48 * 1e6,
        "eager_us_per_layer": eager / 48 * 1e6,
        "eager_gbs": 48 * byts / eager / 1e9,
        "kernel_us": k_avg * 1e6 if k_avg else None,
        "whole_call_gbs": byts / (per_step / 48) / 1e9,
        "kernel_launches_timed": k_n,
        "achieved_gbs": byts / k_avg / 1e9 if k_avg else None,
        "bytes_per_launch": byts,
    }


def bench_prefill(torch, rv, synth, cfg, mode, iters=20, tune=None):
    c = synth.CONFIGS[cfg]
    start, rows = c.context, c.rows
    q, k, v = synth.new_rows(cfg, rows)
    wq, wk = synth.norm_weight(cfg, synth.T_QN), synth.norm_weight(cfg, synth.T_KN)
    dq, dk, dv = (torch.from_numpy(a).cuda() for a in (q, k, v))
    dwq, dwk = torch.from_numpy(wq).cuda(), torch.from_numpy(wk).cuda()
    out = torch.zeros_like(dq)
    kv = rv.KvCache(1, 4, 128, start + rows, "f32")
    for knob, value in (tune or {}).items():
        kv.set_tuning(knob, value)
    if start:
        K, V = synth.cached_kv(cfg, 0, start)
        kv.append_rows(0, K, V)

    def once():
        kv.truncate(start)
        rv.prefill_chunk(kv, 0, dq, dk, dv, dwq, dwk, synth.EPS, synth.THETA, start, synth.SCALE, out, mode=mode)

    for _ in range(3):
        once()
    wall = timed(torch, once, iters) / iters
    k_avg, _ = kernel_avg(torch, kv, once, iters, lead_cycles=400_000)
    flops = prefill_flops(rows, start)
    return {"mode": mode, "us_per_call": round(wall * 1e6, 2), "us_attention_kernel": round(k_avg * 1e6, 2),
            "tflops_call": round(flops / wall / 1e12, 2), "tflops_kernel": round(flops / k_avg / 1e12, 2),
            "mfma_frac_kernel": round(flops / k_avg / 1e12 / MFMA_F16_PEAK_TFLOPS, 4), "flops": flops}


def bench_config1(torch, rv, synth, iters=50):
    """Config 1: the fused decode step (q/k RMSNorm + RoPE, append, attention)
    at position 512 after 512 cached rows, fp32 KV; the cache truncated back
    to 512 between calls. Bytes: the K and V head slices of 513 positions
    read once, q and out."""
    start = 512
    kv = rv.KvCache(1, 4, 128, start + 1, "f32")
    K, V = synth.cached_kv(1, 0, start)
    kv.append_rows(0, K, V)
    q, k, v = (torch.from_numpy(a[0].copy()).cuda() for a in synth.new_rows(1, 1))
    wq, wk = (torch.from_numpy(synth.norm_weight(1, t)).cuda() for t in (synth.T_QN, synth.T_KN))
    out = torch.zeros_like(q)

    def once():
        kv.truncate(start)
        rv.decode_step(kv, 0, q, k, v, wq, wk, synth.EPS, synth.THETA, start, synth.SCALE, out)

    for _ in range(3):
        once()
    wall = timed(torch, once, iters) / iters
    k_avg, _ = kernel_avg(torch, kv, once, iters, lead_cycles=400_000)
    nbytes = 2 * (start + 1) * 512 * 4 + 2 * 4096 * 4

    # The same step from a token graph: 32 device-position steps per replay
    # (contexts 513 .. 544, each followed by its position advance), the
    # position reset to 512 before each replay; no host work per step.
    n_graph = 32
    kvg = rv.KvCache(1, 4, 128, start + 64, "f32")
    kvg.append_rows(0, K, V)
    pos = torch.tensor([start], dtype=torch.int32, device="cuda")

    def steps():
        for _ in range(n_graph):
            rv.decode_step_dev(kvg, 0, q, k, v, wq, wk, synth.EPS, synth.THETA, pos, start + 63, synth.SCALE, out)
            rv.position_advance(kvg, pos, 1)

    steps()  # eagerly: builds the (cos, sin) table
    pos.fill_(start)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        steps()

    def replay():
        pos.fill_(start)
        graph.replay()

    replay()
    per_step = timed(torch, replay, iters) / (iters * n_graph)
    del graph
    return {"us_per_call": round(wall * 1e6, 2), "us_attention_kernel": round(k_avg * 1e6, 2),
            "gbs_kernel": round(nbytes / k_avg / 1e9, 1), "hbm_frac_kernel": round(nbytes / k_avg / 1e9 / HBM_PEAK_GBS, 4),
            "bytes_per_call": nbytes,
            "token_graph": {"us_per_step": round(per_step * 1e6, 2), "steps_per_replay": n_graph,
                            "contexts": [start + 1, start + n_graph],
                            "note": "decode_step_dev + position_advance per step, position reset per replay"}}


def bench_config5(torch, rv, synth, iters=50, n_caches=5, split_lens=(0, 1024, 2048, 4096)):
    """ctx 32,768 f16 KV, rotating 5 distinct caches (335 MB) past the 256 MB
    MALL. One result per split length: 0 is the library's own plan (256
    positions per split at this length: 128 splits per kv head); 1024 / 2048
    / 4096 pin RV_TUNE_DECODE_SPLIT_LEN to BASELINE config 5's 32 / 16 / 8
    splits per kv head."""
    n = 32768
    caches = []
    for i in range(n_caches):
        K, V = synth.cached_kv(5, i, n)
        kv = rv.KvCache(1, 4, 128, n, "f16")
        kv.append_rows(0, K, V)
        caches.append(kv)
    q = torch.from_numpy(synth.rope_f64(synth.normal(synth.seed(5, synth.T_Q), synth.Q_DIM), 128, n,
                                        synth.THETA)).cuda()
    out = torch.zeros_like(q)
    scale = float(synth.SCALE)
    byts = decode_bytes(n, 2)

    def once():
        for kv in caches:
            rv.decode_attention(q, kv, 0, scale, None, out)

    res = {}
    for split_len in split_lens:
        for kv in caches:
            kv.set_tuning(rv.RV_TUNE_DECODE_SPLIT_LEN, split_len)
        for _ in range(3):
            once()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            once()
        graph.replay()
        per = timed(torch, graph.replay, iters) / (iters * n_caches)
        del graph
        tot, cnt = 0.0, 0
        for kv in caches:
            kv.set_tuning(rv.RV_TUNE_KERNEL_TIMING, 1)
            kv.kernel_time()
        for _ in range(iters):
            torch.cuda._sleep(400_000)  # the host queues the five calls ahead of the GPU
            once()
        for kv in caches:
            ms, c = kv.kernel_time()
            kv.set_tuning(rv.RV_TUNE_KERNEL_TIMING, 0)
            tot += ms
            cnt += c
        k_avg = tot / 1e3 / cnt
        sl = split_len or 256
        res["default" if split_len == 0 else f"splits_{n // sl}"] = {
            "split_len": sl, "splits_per_kv_head": -(-n // sl),
            "us_per_call": round(per * 1e6, 3), "gbs_call": round(byts / per / 1e9, 1),
            "frac_call": round(byts / per / 1e9 / HBM_PEAK_GBS, 4),
            "us_tile_kernel": round(k_avg * 1e6, 3), "gbs_tile_kernel": round(byts / k_avg / 1e9, 1),
            "hbm_frac_tile_kernel": round(byts / k_avg / 1e9 / HBM_PEAK_GBS, 4), "bytes_per_call": byts}
    for kv in caches:
        kv.set_tuning(rv.RV_TUNE_DECODE_SPLIT_LEN, 0)
    # The same graph shape over ONE cache (67 MB, which the 256 MB MALL can
    # hold between calls): how much faster a MALL-resident cache streams
    # than the five rotating ones the figures above use.
    def one_cache():
        for _ in range(n_caches):
            rv.decode_attention(q, caches[0], 0, scale, None, out)

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        one_cache()
    graph.replay()
    per1 = timed(torch, graph.replay, iters) / (iters * n_caches)
    del graph
    res["default"]["us_per_call_one_cache_mall"] = round(per1 * 1e6, 3)
    return res


def bench_ladder(torch, rv, synth, ctxs=(64, 128, 256, 512, 1024, 2048, 4096, 8192, 16384, 32768)):
    """Decode attention against context length, as the reference's ladder
    (benches/kernels.rs:168-214, :691-738): f16 cache (the reference's
    format), GQA 32/4, d 128, the cache grown in place through the rungs.
    Arm A: one layer, timed unit = one call, 48 calls on that layer per
    replayed graph (its planes, up to 64 MiB, stay cache-resident). Arm B: 48
    layers, one token's 48 calls per graph (up to 3 GiB of planes, streamed
    from HBM). ns/pos = ns per call / context; the linearity ratio is
    max(ns/pos) / min(ns/pos) over the rungs, as the reference prints it;
    `fit` is the least-squares line us_per_call = floor + slope * context,
    the GPU's fixed per-call cost and its per-position cost."""
    cap = max(ctxs)
    rng = np.random.default_rng(0x1ADD)
    scale = float(synth.SCALE)
    res = {}
    for arm, layers in (("arm_a", 1), ("arm_b", 48)):
        kv = rv.KvCache(layers, 4, 128, cap, "f16")
        q = torch.from_numpy(rng.standard_normal((layers, synth.Q_DIM)).astype(np.float32)).cuda()
        out = torch.zeros_like(q)
        qs, outs = [q[l] for l in range(layers)], [out[l] for l in range(layers)]
        have, rows = 0, []
        for ctx in ctxs:
            blk = rng.standard_normal((ctx - have, 512)).astype(np.float32)
            for layer in range(layers):
                kv.append_rows(layer, blk, blk[::-1].copy())
            have = ctx

            def step():
                for i in range(48):
                    layer = i % layers
                    rv.decode_attention(qs[layer], kv, layer, scale, None, outs[layer])

            for _ in range(3):
                step()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                step()
            graph.replay()
            iters = max(5, 100 * 1024 // max(ctx, 1024))
            per = timed(torch, graph.replay, iters) / iters / 48
            del graph
            byts = decode_bytes(ctx, 2)
            rows.append({"context": ctx, "us_per_call": round(per * 1e6, 3),
                         "ms_per_token_48_layers": round(per * 48 * 1e3, 4),
                         "ns_per_position": round(per * 1e9 / ctx, 4), "gbs": round(byts / per / 1e9, 1)})
        del kv
        res[arm] = rows
        nsp = [r["ns_per_position"] for r in rows]
        res[f"linearity_{arm}"] = round(max(nsp) / min(nsp), 3)
        slope, floor = np.polyfit([r["context"] for r in rows], [r["us_per_call"] for r in rows], 1)
        res[f"fit_{arm}"] = {"floor_us": round(float(floor), 3), "ns_per_position": round(float(slope) * 1e3, 4)}
    return res


PROJ_SHAPES = {"hidden": 2048, "q_dim": 4096, "kv_dim": 512}
PROJ_FORMATS = {"q": 1, "k": 4, "v": 3, "o": 2}  # Q4_K q, Q8_0 k, Q6_K v, Q5_K o (the audited model's)


def synth_weight_rows(rng, fmt: int, rows: int, in_dim: int) -> np.ndarray:
    """Random packed rows of `fmt` (every quant byte uniform, f16 scales in
    [1e-3, 5e-2)): synthetic weights of the real geometry."""
    bb = {1: 144, 2: 176, 3: 210, 4: 34}[fmt]
    nb = in_dim // (32 if fmt == 4 else 256)
    w = rng.integers(0, 256, size=(rows, nb, bb), dtype=np.uint8)
    offs = {1: (0, 2), 2: (0, 2), 3: (208,), 4: (0,)}[fmt]
    for off in offs:
        bits = rng.uniform(1e-3, 5e-2, size=(rows, nb)).astype(np.float16).view(np.uint16)
        w[:, :, off] = bits & 0xFF
        w[:, :, off + 1] = bits >> 8
    return w.reshape(rows, nb * bb)


def bench_projections(torch, rv, iters=100, n_sets=24):
    """The attention projections of one decode layer (model/forward.rs:2574-2646):
    rv_attn_in_proj (quantize both ways, q/k/v GEMVs) and rv_attn_out_proj,
    over n_sets distinct layers' weights (300 MB, past the 256 MB MALL), graph
    replayed; per-layer time and the rate of the weight bytes streamed."""
    from ramvamp_amd import projections as P
    H, Q, KV = PROJ_SHAPES["hidden"], PROJ_SHAPES["q_dim"], PROJ_SHAPES["kv_dim"]
    F = PROJ_FORMATS
    rng = np.random.default_rng(0x9E0)
    sets = []
    for _ in range(n_sets):
        sets.append({k: torch.from_numpy(synth_weight_rows(rng, F[k], rows, ind).ravel()).cuda()
                     for k, rows, ind in (("q", Q, H), ("k", KV, H), ("v", KV, H), ("o", H, Q))})
    wbytes = sum(t.numel() for t in sets[0].values())
    x = torch.from_numpy(rng.standard_normal(H).astype(np.float32)).cuda()
    a = torch.from_numpy(rng.standard_normal(Q).astype(np.float32)).cuda()
    q, k, v = (torch.empty(n, device="cuda") for n in (Q, KV, KV))
    o = torch.empty(H, device="cuda")
    s_in = torch.empty(P.attn_in_proj_scratch_bytes(H), dtype=torch.uint8, device="cuda")
    s_out = torch.empty(P.attn_out_proj_scratch_bytes(Q), dtype=torch.uint8, device="cuda")

    def once():
        for w in sets:
            P.attn_in_proj(x, F["q"], w["q"], q, w["k"], k, F["v"], w["v"], v, s_in)
            P.attn_out_proj(a, F["o"], w["o"], o, s_out)

    for _ in range(3):
        once()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        once()
    graph.replay()
    per = timed(torch, graph.replay, iters) / (iters * n_sets)
    return {"us_per_layer": round(per * 1e6, 3), "weight_bytes_per_layer": wbytes,
            "gbs": round(wbytes / per / 1e9, 1), "hbm_frac": round(wbytes / per / 1e9 / HBM_PEAK_GBS, 4),
            "formats": "q Q4_K 4096x2048, k Q8_0 512x2048, v Q6_K 512x2048, o Q5_K 2048x4096",
            "launches_per_layer": 2, "distinct_layers": n_sets}


def bench_prefill_projections(torch, rv, iters=20, n_rows=512, n_sets=24):
    """A 512-row prefill chunk's attention projections per layer
    (prefill.rs:1985-2053, :2113-2154): rv_attn_in_proj_rows (both
    quantizations, batched q/k/v on int8 MFMA, row-major outputs) and
    rv_attn_out_proj_rows (quantization, batched o, residual add), over
    n_sets distinct layers' weights, graph replayed."""
    from ramvamp_amd import projections as P
    H, Q, KV = PROJ_SHAPES["hidden"], PROJ_SHAPES["q_dim"], PROJ_SHAPES["kv_dim"]
    F = PROJ_FORMATS
    rng = np.random.default_rng(0x9E1)
    sets = []
    for _ in range(n_sets):
        sets.append({k: torch.from_numpy(synth_weight_rows(rng, F[k], rows, ind).ravel()).cuda()
                     for k, rows, ind in (("q", Q, H), ("k", KV, H), ("v", KV, H), ("o", H, Q))})
    wbytes = sum(t.numel() for t in sets[0].values())
    x = torch.from_numpy(rng.standard_normal((n_rows, H)).astype(np.float32)).cuda()
    attn = torch.from_numpy(rng.standard_normal((n_rows, Q)).astype(np.float32)).cuda()
    res = torch.zeros(n_rows, H, device="cuda")
    q, k, v = (torch.empty(n_rows, m, device="cuda") for m in (Q, KV, KV))
    lib = rv._lib.load()
    s_in = torch.empty(int(lib.rv_attn_in_proj_rows_scratch_bytes(n_rows, H)), dtype=torch.uint8, device="cuda")
    s_out = torch.empty(int(lib.rv_attn_out_proj_rows_scratch_bytes(n_rows, Q)), dtype=torch.uint8, device="cuda")

    def once():
        for w in sets:
            P.attn_in_proj_rows(x, F["q"], w["q"], q, w["k"], k, F["v"], w["v"], v, s_in)
            P.attn_out_proj_rows(attn, F["o"], w["o"], res, s_out)

    for _ in range(2):
        once()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        once()
    graph.replay()
    per = timed(torch, graph.replay, iters) / (iters * n_sets)
    ops = 2 * n_rows * (H * (Q + 2 * KV) + Q * H)  # int8 multiply-adds of the exact dots, x2
    return {"us_per_layer": round(per * 1e6, 3), "rows": n_rows, "int8_tops": round(ops / per / 1e12, 2),
            "weight_bytes_per_layer": wbytes, "weight_gbs": round(wbytes / per / 1e9, 1),
            "launches_per_layer": 7, "distinct_layers": n_sets}


def bench_attn_block_prefill(torch, rv, synth, mode="f16", iters=20):
    """One layer's attention block for a 512-row prefill chunk at config 4
    (3449 cached rows, fp32 KV): rv_attn_block_prefill (row RMSNorm, batched
    q/k/v, QK norm + RoPE + append + causal attention in `mode`, batched o +
    residual add), back to back (the cache truncated to 3449 between calls)."""
    from ramvamp_amd import block as B
    H, Q, KV = PROJ_SHAPES["hidden"], PROJ_SHAPES["q_dim"], PROJ_SHAPES["kv_dim"]
    F = PROJ_FORMATS
    c = synth.CONFIGS[4]
    start, rows = c.context, c.rows
    rng = np.random.default_rng(0xB10D)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    w = B.AttnBlockWeights(d((1 + 0.02 * rng.standard_normal(H)).astype(np.float32)), F["q"],
                           d(synth_weight_rows(rng, F["q"], Q, H)), d(synth_weight_rows(rng, F["k"], KV, H)), F["v"],
                           d(synth_weight_rows(rng, F["v"], KV, H)), d(synth.norm_weight(4, synth.T_QN)),
                           d(synth.norm_weight(4, synth.T_KN)), F["o"], d(synth_weight_rows(rng, F["o"], H, Q)))
    kv = rv.KvCache(1, 4, 128, start + rows, "f32")
    K, V = synth.cached_kv(4, 0, start)
    kv.append_rows(0, K, V)
    residual = d(rng.standard_normal((rows, H)).astype(np.float32))
    scratch = torch.empty(B.prefill_scratch_bytes(rows, H, Q, KV), dtype=torch.uint8, device="cuda")

    def once():
        kv.truncate(start)
        B.attn_block_prefill(kv, 0, residual, Q, w, synth.EPS, synth.THETA, start, float(synth.SCALE), mode=mode,
                             scratch=scratch)

    for _ in range(3):
        once()
    per = timed(torch, once, iters) / iters
    return {"mode": mode, "rows": rows, "start": start, "us_per_layer": round(per * 1e6, 2),
            "us_per_token": round(per * 1e6 / rows, 4)}


def bench_router(torch, rv, iters=50, n_experts=128, hidden=2048, top_k=8):
    """The router decision (forward.rs:2658-2705) for one decode row, a
    512-row prefill chunk and 1024 rows, 128 experts over a 2048-wide row,
    top 8 with renormalization, host-timed back to back."""
    from ramvamp_amd import router as R
    rng = np.random.default_rng(0x40)
    w = torch.from_numpy((rng.standard_normal((n_experts, hidden)) * 0.03).astype(np.float32)).cuda()
    out = {}
    for rows in (1, 512, 1024):
        x = torch.from_numpy(rng.standard_normal((rows, hidden)).astype(np.float32)).cuda()
        ex = torch.empty(rows, top_k, dtype=torch.int32, device="cuda")
        wt = torch.empty(rows, top_k, device="cuda")
        fn = lambda: R.router_topk(x, w, top_k, True, ex, wt)
        for _ in range(3):
            fn()
        out[f"us_{rows}_rows"] = round(timed(torch, fn, iters) / iters * 1e6, 2)
    return out


def bench_attn_block(torch, rv, synth, iters=20, n_layers=48, n_sets=24):
    """One token's attention blocks over config 2's 48 layers (ctx 4096, fp32
    KV): rv_attn_block_decode per layer (model/forward.rs:2570-2650: RMSNorm,
    q/k/v projections, QK norm + RoPE, append, attention, output projection,
    residual add), n_sets distinct layers' weights, one captured graph per
    token replayed (each replay re-appends the token at the captured cursor
    and attends 4096 + 3 positions)."""
    from ramvamp_amd import block as B
    H, Q, KV = PROJ_SHAPES["hidden"], PROJ_SHAPES["q_dim"], PROJ_SHAPES["kv_dim"]
    F = PROJ_FORMATS
    rng = np.random.default_rng(0xB10C)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    sets = []
    for _ in range(n_sets):
        sets.append(B.AttnBlockWeights(
            d((1 + 0.02 * rng.standard_normal(H)).astype(np.float32)), F["q"], d(synth_weight_rows(rng, F["q"], Q, H)),
            d(synth_weight_rows(rng, F["k"], KV, H)), F["v"], d(synth_weight_rows(rng, F["v"], KV, H)),
            d(synth.norm_weight(2, synth.T_QN)), d(synth.norm_weight(2, synth.T_KN)), F["o"],
            d(synth_weight_rows(rng, F["o"], H, Q))))
    kv = rv.KvCache(n_layers, 4, 128, 4096 + 64, "f32")
    for layer in range(n_layers):
        K, V = synth.cached_kv(2, layer, 4096)
        kv.append_rows(layer, K, V)
    residual = d(rng.standard_normal(H).astype(np.float32))
    scratch = torch.empty(B.scratch_bytes(H, Q, KV), dtype=torch.uint8, device="cuda")
    scale = float(synth.SCALE)

    def token():
        for layer in range(n_layers):
            B.attn_block_decode(kv, layer, residual, Q, sets[layer % n_sets], synth.EPS, synth.THETA,
                                kv.len(layer), scale, scratch=scratch)

    for _ in range(2):
        token()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        token()
    graph.replay()
    per = timed(torch, graph.replay, iters) / (iters * n_layers)
    del graph
    wbytes = sum(t.numel() for t in (sets[0].wq, sets[0].wk, sets[0].wv, sets[0].wo))
    kv_bytes = 2 * 4099 * 512 * 4

    # The token graph: the same blocks with the position in device memory,
    # captured once and replayed for successive tokens (context 4096 + 1 ..
    # 4096 + 2 + iters), every replay a new token.
    kv.truncate(4096)
    pos = torch.tensor([4096], dtype=torch.int32, device="cuda")
    max_pos = kv.capacity() - 1

    def token_dev():
        for layer in range(n_layers):
            B.attn_block_decode_dev(kv, layer, residual, Q, sets[layer % n_sets], synth.EPS, synth.THETA, pos,
                                    max_pos, scale, scratch)
        rv.position_advance(kv, pos, 1)

    token_dev()  # eagerly: builds the (cos, sin) table
    tg = torch.cuda.CUDAGraph()
    with torch.cuda.graph(tg):
        token_dev()
    tg.replay()
    per_dev = timed(torch, tg.replay, iters) / (iters * n_layers)
    n_written = int(pos.item()) - 4096
    for layer in range(n_layers):
        kv.commit(layer, n_written)
    del tg
    return {"us_per_layer": round(per * 1e6, 3), "ms_per_token_48_layers": round(per * n_layers * 1e3, 3),
            "bytes_per_layer": wbytes + kv_bytes, "gbs": round((wbytes + kv_bytes) / per / 1e9, 1),
            "launches_per_layer": 4, "distinct_weight_sets": n_sets, "context": 4099,
            "token_graph": {"us_per_layer": round(per_dev * 1e6, 3),
                            "ms_per_token_48_layers": round(per_dev * n_layers * 1e3, 3),
                            "tokens": n_written, "context_range": [4097, 4096 + n_written],
                            "planned_positions": max_pos + 1,
                            "note": "one graph replayed per token; position read from device memory"}}


def bench_floors(torch, iters=50):
    """The limits the decode and prefill kernels are judged against, measured
    on this box with the probe launches of include/ramvamp_floors.h, each in
    a 48-launch graph (as config 2 replays its layers): an empty launch; a
    plain streaming read of one config-2 call's bytes (16.8 MB, 48 distinct
    buffers: 807 MB, past the 256 MB MALL) and of one config-5 call's (67.1
    MB, 5 rotating buffers: 336 MB) at several workgroup counts; and the
    issue rate of the MFMA forms (independent chains, 1 and 4 waves per
    SIMD) and the VALU work one 32x32x16 MFMA hides, timed with events
    around one long launch."""
    from ctypes import byref, c_void_p

    from ramvamp_amd import _lib as L

    lib = L.load()
    err = L.RvError()

    def ok(rc):
        if rc:
            raise RuntimeError(f"floor probe failed: {rc} {err.what}")

    def stream():
        return c_void_p(torch.cuda.current_stream().cuda_stream)

    def graph_us(fn, n_launch=48):
        fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        for _ in range(5):
            g.replay()
        t = timed(torch, g.replay, iters)
        del g
        return t / iters / n_launch * 1e6

    res = {}
    res["empty_launch_us_in_graph"] = round(graph_us(lambda: [ok(lib.rv_floor_empty(stream(), byref(err)))
                                                              for _ in range(48)]), 3)
    sink = torch.zeros(1 << 16, device="cuda")
    for name, nbytes, n_buf, grids in (("decode_ctx4096_f32", decode_bytes(4096, 4), 48, (256, 512, 1024, 2048)),
                                       ("decode_ctx32768_f16", decode_bytes(32768, 2), 5, (512, 1024, 2048, 4096))):
        nb = (nbytes + 15) // 16 * 16
        bufs = [torch.ones(nb // 4, device="cuda") for _ in range(n_buf)]
        row = {"bytes": nbytes, "buffers": n_buf}
        for n_wg in grids:
            def fn(n_wg=n_wg):
                for i in range(48):
                    ok(lib.rv_floor_stream_read(c_void_p(bufs[i % n_buf].data_ptr()), nb, n_wg,
                                                c_void_p(sink.data_ptr()), stream(), byref(err)))
            us = graph_us(fn)
            row[f"us_{n_wg}_wg"] = round(us, 3)
        best = min(v for k, v in row.items() if k.startswith("us_"))
        row["best_us"] = best
        row["best_gbs"] = round(nbytes / best / 1e3, 1)
        row["best_frac"] = round(nbytes / best / 1e3 / HBM_PEAK_GBS, 4)
        res[f"stream_read_{name}"] = row
        del bufs
    flops = {L.RV_FLOOR_MFMA_F16_16X16X32: ("f16_16x16x32", 16384, 4000),
             L.RV_FLOOR_MFMA_F16_32X32X16: ("f16_32x32x16", 32768, 2000),
             L.RV_FLOOR_MFMA_F32_16X16X4: ("f32_16x16x4", 2048, 4000)}
    for form, (name, f, it) in flops.items():
        row = {}
        for waves_per_simd in (1, 2, 4):
            n_wg = 256 * waves_per_simd
            for _ in range(2):  # warm-up
                ok(lib.rv_floor_mfma(form, 4, it, n_wg, c_void_p(sink.data_ptr()), stream(), byref(err)))
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            ok(lib.rv_floor_mfma(form, 4, it, n_wg, c_void_p(sink.data_ptr()), stream(), byref(err)))
            e1.record()
            torch.cuda.synchronize()
            s_ = e0.elapsed_time(e1) / 1e3
            tf = n_wg * 4 * it * 4 * f / s_ / 1e12
            row[f"tflops_{waves_per_simd}_waves_per_simd"] = round(tf, 1)
            row[f"ns_per_mfma_per_simd_{waves_per_simd}_waves"] = round(s_ / (waves_per_simd * it * 4) * 1e9, 2)
        res[f"mfma_{name}"] = row
    # How much VALU work one v_mfma_f32_32x32x16_f16 hides on its SIMD: ns per
    # MFMA per SIMD with k independent VALU instructions after each, at two
    # waves per SIMD (the prefill kernel's occupancy).
    row = {}
    for kind, kname, ks in ((L.RV_FLOOR_VALU_FMA, "fma", (0, 2, 4, 8)), (L.RV_FLOOR_VALU_EXP, "exp", (2, 4, 8))):
        for k in ks:
            n_wg, it = 512, 1000
            for _ in range(2):  # warm-up
                ok(lib.rv_floor_mfma_valu(kind, k, it, n_wg, c_void_p(sink.data_ptr()), stream(), byref(err)))
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            ok(lib.rv_floor_mfma_valu(kind, k, it, n_wg, c_void_p(sink.data_ptr()), stream(), byref(err)))
            e1.record()
            torch.cuda.synchronize()
            s_ = e0.elapsed_time(e1) / 1e3
            row[f"ns_per_mfma_{kname}_{k}"] = round(s_ / (2 * it * 4) * 1e9, 2)
    res["mfma_32x32x16_valu_overlap_2_waves"] = row
    return res


def cpu_baseline(synth, budget_s=12.0, n_layers=48, sample_layers=8):
    """The oracle (C restatement of ramvamp's AVX2+F16C decode path with its
    kv-head fan-out over min(4, cores) threads, forward.rs:1914-2063) on the
    same config-2 inputs (the first layers' seeded K/V, regenerated), timed on
    this host for a bounded sample of layers."""
    import oracle

    threads = max(1, min(4, os.cpu_count() or 1))
    caches = []
    for layer in range(sample_layers):
        K, V = synth.cached_kv(2, layer, 4096)
        ref = oracle.KvCache(1, 4, 128, 4096, oracle.RV_ELEM_F32)
        ref.append_rows(0, K, V)
        caches.append(ref)
    qs = [synth.normal(synth.seed(2, synth.T_Q, l), synth.Q_DIM) for l in range(len(caches))]
    times = []
    t_end = time.perf_counter() + budget_s
    calls = 0
    while time.perf_counter() < t_end or calls < len(caches):
        i = calls % len(caches)
        t0 = time.perf_counter()
        caches[i].pool_decode_attention(qs[i], 0, float(synth.SCALE), threads)
        times.append(time.perf_counter() - t0)
        calls += 1
    per_layer = float(np.median(times))
    return {
        "value": round(decode_bytes(4096, 4) / per_layer / 1e9, 3), "unit": "GB/s", "cores": threads,
        "kind": "port", "us_per_layer": round(per_layer * 1e6, 1),
        "sample": f"{calls} decode calls (ctx 4096, fp32 KV) over {len(caches)} of the {n_layers} config-2 layers, "
                  f"median per call; oracle AVX2+F16C body, kv-head fan-out over {threads} threads",
    }


def cpu_configs(synth, threads, prefill_threads):
    """The oracle (the reference's CPU path restated) on configs 1, 3, 4 and
    5, on this host: decode with its kv-head fan-out over `threads` (the
    reference's ceiling of 4 shards), prefill with the cost-balanced row split
    over `prefill_threads` (the host's cores, capped at a GPU's CPU share), the
    whole 512-row chunk timed (nothing extrapolated)."""
    import oracle
    res = {}
    # Config 1: the fused decode step after 512 cached rows.
    ref = oracle.KvCache(1, 4, 128, 513, oracle.RV_ELEM_F32)
    K, V = synth.cached_kv(1, 0, 512)
    ref.append_rows(0, K, V)
    q, k, v = (a[0] for a in synth.new_rows(1, 1))
    wq, wk = synth.norm_weight(1, synth.T_QN), synth.norm_weight(1, synth.T_KN)
    times = []
    for i in range(21):  # the first call warms up (not timed)
        ref.truncate(512)
        t0 = time.perf_counter()
        ref.decode_step(0, q, k, v, wq, wk, synth.EPS, synth.THETA, 512, synth.SCALE, threads=threads)
        if i:
            times.append(time.perf_counter() - t0)
    res["config1"] = {"us_per_call": round(float(np.median(times)) * 1e6, 1), "cores": threads, "kind": "port",
                      "sample": "20 decode steps, median"}
    # Configs 3 and 4: the whole chunk, median of 3 after a warm-up.
    for cfg in (3, 4):
        c = synth.CONFIGS[cfg]
        start = c.context
        ref = oracle.KvCache(1, 4, 128, start + c.rows, oracle.RV_ELEM_F32)
        if start:
            K, V = synth.cached_kv(cfg, 0, start)
            ref.append_rows(0, K, V)
        q, k, v = synth.new_rows(cfg, c.rows)
        wq, wk = synth.norm_weight(cfg, synth.T_QN), synth.norm_weight(cfg, synth.T_KN)
        times = []
        for i in range(4):
            ref.truncate(start)
            t0 = time.perf_counter()
            ref.prefill_chunk(0, q, k, v, wq, wk, synth.EPS, synth.THETA, start, synth.SCALE,
                              threads=prefill_threads)
            if i:
                times.append(time.perf_counter() - t0)
        per = float(np.median(times))
        flops = prefill_flops(c.rows, start)
        res[f"config{cfg}"] = {"us_per_call": round(per * 1e6, 1), "tflops": round(flops / per / 1e12, 5),
                               "cores": prefill_threads, "kind": "port",
                               "sample": f"the whole {c.rows}-row chunk, 3 timed calls after a warm-up, median; "
                                         f"row split over {prefill_threads} threads"}
    # Config 5: decode over 32768 f16 positions.
    ref = oracle.KvCache(1, 4, 128, 32768, oracle.RV_ELEM_F16)
    K, V = synth.cached_kv(5, 0, 32768)
    ref.append_rows(0, K, V)
    q5 = synth.normal(synth.seed(5, synth.T_Q), synth.Q_DIM)
    ref.pool_decode_attention(q5, 0, float(synth.SCALE), threads)  # warm-up
    times = []
    for _ in range(5):
        t0 = time.perf_counter()
        ref.pool_decode_attention(q5, 0, float(synth.SCALE), threads)
        times.append(time.perf_counter() - t0)
    per = float(np.median(times))
    res["config5"] = {"us_per_call": round(per * 1e6, 1), "gbs": round(67141632 / per / 1e9, 3), "cores": threads,
                      "kind": "port", "sample": "5 decode calls, median"}
    return res


def cpu_projections(budget_s=4.0):
    """The oracle's scalar projections (quantize both ways, the q/k/v GEMVs,
    quantize, the o GEMV; kernels/quants/dot.rs, one thread) at the bench
    shapes, timed on this host for a bounded number of layers."""
    import oracle
    H, Q, KV = PROJ_SHAPES["hidden"], PROJ_SHAPES["q_dim"], PROJ_SHAPES["kv_dim"]
    F = PROJ_FORMATS
    rng = np.random.default_rng(0x9E0)
    w = {k: synth_weight_rows(rng, F[k], rows, ind) for k, rows, ind in (("q", Q, H), ("k", KV, H), ("v", KV, H),
                                                                          ("o", H, Q))}
    wbytes = sum(a.size for a in w.values())
    x = rng.standard_normal(H).astype(np.float32)
    a = rng.standard_normal(Q).astype(np.float32)
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 2:
        t0 = time.perf_counter()
        ak, a0 = oracle.quantize_row_q8_k(x), oracle.quantize_row_q8_0(x)
        oracle.gemv(F["q"], w["q"], H, Q, ak)
        oracle.gemv(F["k"], w["k"], H, KV, a0)
        oracle.gemv(F["v"], w["v"], H, KV, ak)
        oracle.gemv(F["o"], w["o"], Q, H, oracle.quantize_row_q8_k(a))
        times.append(time.perf_counter() - t0)
    per = float(np.median(times))
    return {"value": round(wbytes / per / 1e9, 3), "unit": "GB/s of weights", "cores": 1, "kind": "port",
            "us_per_layer": round(per * 1e6, 1),
            "sample": f"{len(times)} layers' projections (one weight set), median; oracle scalar dots, one thread"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--prefill-case", action="append", default=[], metavar="CFG:MODE",
                    help="with --prefill-only: run only these cases (e.g. 4:f16), repeatable")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only run the prefill legs (configs 3 and 4, every mode), log them and exit (for profiling)")
    ap.add_argument("--projections-only", action="store_true",
                    help="only run the attention-projection leg, log it and exit (for profiling)")
    ap.add_argument("--prefill-proj-only", action="store_true",
                    help="only run the prefill-chunk projection leg (512 rows), log it and exit (for profiling)")
    ap.add_argument("--block-only", action="store_true",
                    help="only run the attention-block leg (48 layers, ctx 4096), log it and exit (for profiling)")
    ap.add_argument("--router-only", action="store_true",
                    help="only run the router leg (1, 512 and 1024 rows), log it and exit (for profiling)")
    ap.add_argument("--config1-only", action="store_true",
                    help="only config 1 (the fused decode step, eager and token graph), for profiling")
    ap.add_argument("--config5-only", action="store_true",
                    help="only run the config 5 leg (ctx 32768, f16, every split shape), log it and exit (for profiling)")
    ap.add_argument("--floors", action="store_true",
                    help="only measure the floors (empty launch, streaming reads, MFMA issue rates), log them and exit")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run ten 64 MiB device-to-device copies (the reference kernel that scales the "
                         "FETCH_SIZE / WRITE_SIZE counters to bytes) and exit")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (one layer's attention would "
              "shard by kv head, one GPU per head group, with no exchange); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    import ramvamp_amd as rv
    from ramvamp_amd import synth

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.copy_calibration:
        a = torch.ones(16 << 20, device="cuda")  # 64 MiB of f32
        b = torch.empty_like(a)
        for _ in range(10):
            b.copy_(a)
        torch.cuda.synchronize()
        log("copied 10 x 64 MiB")
        return
    if args.floors:
        log(json.dumps(bench_floors(torch), indent=1))
        return
    if args.projections_only:
        rp = bench_projections(torch, rv)
        log(f"projections: {rp['us_per_layer']:.2f} us/layer, {rp['gbs']:.0f} GB/s of weights")
        return
    if args.prefill_proj_only:
        rpp = bench_prefill_projections(torch, rv)
        log(f"prefill projections: {rpp['us_per_layer']:.2f} us/layer for {rpp['rows']} rows, "
            f"{rpp['int8_tops']:.1f} int8 TOP/s")
        return
    if args.router_only:
        rr = bench_router(torch, rv)
        log(f"router: {rr['us_1_rows']:.1f} us for 1 row, {rr['us_512_rows']:.1f} us for 512 rows, "
            f"{rr['us_1024_rows']:.1f} us for 1024 rows")
        return
    if args.block_only:
        rb = bench_attn_block(torch, rv, synth)
        log(f"attention block: {rb['us_per_layer']:.2f} us/layer, {rb['ms_per_token_48_layers']:.3f} ms per token; "
            f"token graph {rb['token_graph']['us_per_layer']:.2f} us/layer over {rb['token_graph']['tokens']} tokens")
        for mode in ("f16", "exact"):
            rbp = bench_attn_block_prefill(torch, rv, synth, mode)
            log(f"attention block prefill {mode}: {rbp['us_per_layer']:.1f} us/layer for {rbp['rows']} rows")
        return
    if args.config1_only:
        r1 = bench_config1(torch, rv, synth)
        log(f"config 1: {r1['us_per_call']:.2f} us/call, kernel {r1['us_attention_kernel']:.2f} us, "
            f"token graph {r1['token_graph']['us_per_step']:.2f} us/step")
        return
    if args.config5_only:
        r5 = bench_config5(torch, rv, synth)
        for name, r in r5.items():
            log(f"config 5 {name} ({r['splits_per_kv_head']} splits/kv head): {r['us_per_call']:.2f} us/call, "
                f"tile kernel {r['us_tile_kernel']:.2f} us")
        log(f"config 5 default over one MALL-resident cache: {r5['default']['us_per_call_one_cache_mall']:.2f} us/call")
        return
    if args.prefill_only:
        cases = [(int(c.split(":")[0]), c.split(":")[1]) for c in args.prefill_case] or \
            [(3, "f16"), (3, "bf16"), (3, "exact"), (4, "f16"), (4, "bf16"), (4, "exact")]
        for cfg, mode in cases:
            r = bench_prefill(torch, rv, synth, cfg, mode)
            log(f"config {cfg} {mode}: {r['us_per_call']:.1f} us/call, kernel {r['us_attention_kernel']:.1f} us, "
                f"{r['tflops_kernel']:.1f} TFLOP/s")
        return
    r2 = bench_config2(torch, rv, synth, args.steps, args.warmup)
    log(f"config 2: {r2['us_per_layer']:.2f} us/layer (graph), {r2['eager_us_per_layer']:.2f} us/layer (eager), "
        f"kernel {r2['kernel_us']:.2f} us, {r2['value_gbs']:.0f} GB/s")
    extra = {"config2_eager": {"us_per_layer": round(r2["eager_us_per_layer"], 3),
                               "gbs": round(r2["eager_gbs"], 1)},
             "config2_graph_matches_eager": r2["graph_matches_eager"]}
    if not args.no_extra:
        extra["floors"] = bench_floors(torch)
        log("floors: " + json.dumps(extra["floors"]))
        for cfg, mode in ((3, "f16"), (3, "bf16"), (3, "exact"), (4, "f16"), (4, "bf16"), (4, "exact")):
            r = bench_prefill(torch, rv, synth, cfg, mode)
            extra[f"config{cfg}_prefill_{mode}"] = r
            log(f"config {cfg} {mode}: {r['us_per_call']:.1f} us/call, kernel {r['us_attention_kernel']:.1f} us, "
                f"{r['tflops_kernel']:.1f} TFLOP/s")
        r1 = bench_config1(torch, rv, synth)
        extra["config1_decode_step_ctx512"] = r1
        log(f"config 1: {r1['us_per_call']:.2f} us/call, kernel {r1['us_attention_kernel']:.2f} us, "
            f"token graph {r1['token_graph']['us_per_step']:.2f} us/step")
        r5 = bench_config5(torch, rv, synth)
        c5_trace = profile_value(CONFIG5_PROFILE, "trace_us_per_launch")
        if c5_trace:
            d5 = r5["default"]
            d5["us_tile_kernel_trace"] = c5_trace
            d5["hbm_frac_tile_kernel_trace"] = round(d5["bytes_per_call"] / (c5_trace * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
            d5["trace_profile"] = os.path.relpath(CONFIG5_PROFILE, ROOT)
        extra["config5_decode_f16_ctx32768"] = r5
        for name, r in r5.items():
            log(f"config 5 {name} ({r['splits_per_kv_head']} splits/kv head): {r['us_per_call']:.2f} us/call, "
                f"tile kernel {r['us_tile_kernel']:.2f} us, {r['gbs_call']:.0f} GB/s per call")
        rl = bench_ladder(torch, rv, synth)
        extra["decode_ladder_f16"] = rl
        for arm in ("arm_a", "arm_b"):
            log(f"ladder {arm}: " + ", ".join(f"{r['context']}:{r['us_per_call']:.2f}us" for r in rl[arm]) +
                f"; linearity {rl['linearity_' + arm]}; fit {rl['fit_' + arm]}")
        rp = bench_projections(torch, rv)
        extra["projections_decode_layer"] = rp
        log(f"projections: {rp['us_per_layer']:.2f} us/layer, {rp['gbs']:.0f} GB/s of weights")
        rpp = bench_prefill_projections(torch, rv)
        extra["prefill_projections_512_rows"] = rpp
        log(f"prefill projections: {rpp['us_per_layer']:.2f} us/layer for {rpp['rows']} rows, "
            f"{rpp['int8_tops']:.1f} int8 TOP/s")
        rb = bench_attn_block(torch, rv, synth)
        extra["attn_block_decode_layer"] = rb
        log(f"attention block: {rb['us_per_layer']:.2f} us/layer, {rb['ms_per_token_48_layers']:.3f} ms per token; "
            f"token graph {rb['token_graph']['us_per_layer']:.2f} us/layer over {rb['token_graph']['tokens']} tokens")
        rr = bench_router(torch, rv)
        extra["router_128x2048_top8"] = rr
        log(f"router: {rr['us_1_rows']:.1f} us for 1 row, {rr['us_512_rows']:.1f} us for 512 rows, "
            f"{rr['us_1024_rows']:.1f} us for 1024 rows")
        for mode in ("f16", "exact"):
            rbp = bench_attn_block_prefill(torch, rv, synth, mode)
            extra[f"attn_block_prefill_config4_{mode}"] = rbp
            log(f"attention block prefill {mode}: {rbp['us_per_layer']:.1f} us/layer for {rbp['rows']} rows")
    cpu = None
    if not args.no_cpu:
        log("cpu baseline ...")
        cpu = cpu_baseline(synth)
        if "projections_decode_layer" in extra:
            extra["projections_decode_layer"]["cpu_baseline"] = cpu_projections()
            threads = max(1, min(4, os.cpu_count() or 1))
            prefill_threads = max(1, min(16, os.cpu_count() or 1))  # a GPU box's CPU share is 16 cores
            for name, r in cpu_configs(synth, threads, prefill_threads).items():
                for key in extra:
                    if key.startswith(name + "_"):
                        extra[key]["cpu_baseline"] = r
    traffic = traffic_from_profile(DECODE_PROFILE)
    # Two figures for the tile kernel's launch duration: the committed
    # rocprofv3 kernel-trace average of this same command (the kernel's
    # execution window), and this run's HIP events around each launch
    # (which also hold the launch's dispatch latency, ~0.5-1 us longer).
    # frac uses the trace figure when the profile records one.
    trace_us = profile_value(DECODE_PROFILE, "trace_us_per_launch")
    byts = r2["bytes_per_launch"]
    ev = {"us_per_launch": round(r2["kernel_us"], 3), "achieved": round(r2["achieved_gbs"], 1),
          "frac": round(r2["achieved_gbs"] / HBM_PEAK_GBS, 4), "launches_timed": r2["kernel_launches_timed"]}
    if trace_us:
        tr_gbs = byts / (trace_us * 1e-6) / 1e9
        tr = {"us_per_launch": trace_us, "achieved": round(tr_gbs, 1), "frac": round(tr_gbs / HBM_PEAK_GBS, 4),
              "profile": os.path.relpath(DECODE_PROFILE, ROOT)}
        head, source = tr, "trace"
    else:
        tr, head, source = None, ev, "events"
    roofline = {"bound": "hbm", "achieved": head["achieved"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": head["frac"], "frac_source": source, "traffic": traffic,
                "kernel": "decode_tile_kernel<float, 4, 1>", "us_per_launch": head["us_per_launch"],
                "bytes_per_launch": byts, "trace": tr, "events": ev,
                "events_over_trace": round(r2["kernel_us"] / trace_us, 3) if trace_us and r2["kernel_us"] else None,
                "whole_call": {"kernels": "decode_tile_kernel + decode_merge_kernel",
                               "achieved": round(r2["whole_call_gbs"], 1),
                               "frac": round(r2["whole_call_gbs"] / HBM_PEAK_GBS, 4),
                               "us_per_call": round(r2["us_per_layer"], 3)}}
    line = {
        "metric": "decode attn µs/layer + HBM GB/s at ctx 4096; prefill attn TFLOP/s (512 tok)",
        "value": round(r2["value_gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r2["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,1) K/V/q, ramvamp_amd/synth.py)",
        "config": {"workload": "config 2: 48 sequential decode-attention layers, ctx 4096, fp32 KV, GQA 32/4, d 128, "
                               "graph-replayed step",
                   "layers": 48, "context": 4096, "n_q_heads": 32, "n_kv_heads": 4, "head_dim": 128,
                   "kv_elem": "f32", "parallelism": "single GPU"},
        "us_per_layer": round(r2["us_per_layer"], 3),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
