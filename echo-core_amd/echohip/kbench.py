"""Kernel-level measurements of the decode hot path on one GPU.

Each HBM-bound case cycles through >= 512 MB of distinct buffers (the 256 MB
Infinity Cache would otherwise hold the working set) and times every launch
with its own pair of HIP events on the launch stream; the reported duration is
the mean over launches.  Algorithmic bytes / FLOPs per launch follow the
workload definitions (weights + activations + outputs actually required).
"""
from __future__ import annotations

import math

import numpy as np
import torch

from . import lib as L
from . import synth

HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3
ROTATE_BYTES = 512 << 20


def _events_mean_us(launch, n_copies, iters, replays=5):
    """Mean GPU time per launch: `iters` launches over the rotation are captured
    in one HIP graph (so host submission never gaps the GPU), the graph is
    replayed between two HIP events on the launch stream, and the elapsed time is
    divided by the launch count.  Returns (mean, best-replay mean) in us."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(n_copies):  # warm every copy once, outside the capture
            launch(i, side.cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        st = torch.cuda.current_stream().cuda_stream
        for i in range(iters):
            launch(i % n_copies, st)
    g.replay()
    torch.cuda.synchronize()
    t = []
    for _ in range(replays):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        g.replay()
        b.record()
        torch.cuda.synchronize()
        t.append(a.elapsed_time(b) * 1e3 / iters)
    del g
    return float(np.mean(t)), float(np.min(t))


def matvec_case(hip, fmt, N, K, M=1, iters=200, seed=0, pieces=1, nsplit=1):
    """Decode matvec y = W x over a rotation of weight copies; `pieces` int8
    pieces per activation element, nsplit > 1: the split-K form (partial sums)."""
    st = torch.cuda.current_stream().cuda_stream
    if fmt == L.Q8_0:
        wbytes = N * K // 32 * 34
        Wd = torch.empty(wbytes, dtype=torch.uint8, device="cuda")
        hip.fill_random(1, Wd, N * K // 32, seed, 0.02, stream=st)  # same bytes as synth.q8_0_blocks
    else:
        wbytes = N * K // 256 * 144
        Wd = torch.from_numpy(synth.q4_K_blocks(seed, N, K)).cuda()
    tb = hip.tiled_bytes(fmt, N, K)
    n_copies = max(2, math.ceil(ROTATE_BYTES / tb) + 1)
    tiled = torch.empty((n_copies, tb), dtype=torch.uint8, device="cuda")
    hip.repack(fmt, Wd, tiled[0], N, K, stream=st)
    for i in range(1, n_copies):
        tiled[i].copy_(tiled[0])
    del Wd
    x = torch.from_numpy(synth.activations(seed + 1, M * K)).cuda()
    act = torch.empty(hip.act_bytes(fmt, M, K, pieces=pieces), dtype=torch.uint8, device="cuda")
    hip.quantize_act(fmt, x, act, M, K, stream=st, pieces=pieces)
    y = torch.empty(nsplit * M * N, dtype=torch.float32, device="cuda")

    def launch(i, stream):
        if nsplit > 1:
            hip.matvec_split(fmt, tiled[i], act, y, M, N, K, nsplit, stream=stream, pieces=pieces)
        else:
            hip.matvec(fmt, tiled[i], act, y, M, N, K, stream=stream, pieces=pieces)

    mean_us, med_us = _events_mean_us(launch, n_copies, iters)
    x_bytes = M * (pieces * K + K // 32 * 4 * (2 if fmt == L.Q4_K else 1))
    alg = wbytes + x_bytes + M * N * 4
    gbs = alg / (mean_us * 1e-6) / 1e9
    del tiled
    torch.cuda.empty_cache()
    return {"kernel": "k_mv_q8_0" if fmt == L.Q8_0 else "k_mv_q4_K", "M": M, "N": N, "K": K, "pieces": pieces,
            "bytes": alg, "us": round(mean_us, 3), "us_best": round(med_us, 3), "GBs": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4), "copies": n_copies}


def gguf_f32_case(hip, fmt, N, K, iters=200, seed=0):
    """The reference-signature matvec path (ec_matvec_gguf_f32: GGUF bytes read in
    place, fp32 activations, y += W x) over a rotation of weight copies, device
    pointers.  Algorithmic bytes: weights + fp32 x + y read and written."""
    st = torch.cuda.current_stream().cuda_stream
    if fmt == L.Q8_0:
        wbytes = N * K // 32 * 34
        W0 = torch.empty(wbytes, dtype=torch.uint8, device="cuda")
        hip.fill_random(1, W0, N * K // 32, seed, 0.02, stream=st)
    else:
        wbytes = N * K // 256 * 144
        W0 = torch.from_numpy(synth.q4_K_blocks(seed, N, K).reshape(-1)).cuda()
    n_copies = max(2, math.ceil(ROTATE_BYTES / wbytes) + 1)
    Ws = torch.empty((n_copies, wbytes), dtype=torch.uint8, device="cuda")
    for i in range(n_copies):
        Ws[i].copy_(W0)
    del W0
    x = torch.from_numpy(synth.activations(seed + 1, K)).cuda()
    y = torch.zeros(N, dtype=torch.float32, device="cuda")

    def launch(i, stream):
        hip.matvec_gguf_f32(fmt, Ws[i], x, y, N, K, stream=stream)

    mean_us, best_us = _events_mean_us(launch, n_copies, iters)
    alg = wbytes + K * 4 + 2 * N * 4
    gbs = alg / (mean_us * 1e-6) / 1e9
    del Ws
    torch.cuda.empty_cache()
    return {"kernel": "k_gguf_q8_0_f32" if fmt == L.Q8_0 else "k_gguf_q4_K_f32", "M": 1, "N": N, "K": K,
            "bytes": alg, "us": round(mean_us, 3), "us_best": round(best_us, 3), "GBs": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4), "copies": n_copies}


def stream_read_sweep(hip, nbytes, iters=100):
    """Fastest single launch of a plain non-temporal 16-byte read of `nbytes`
    over launch shapes (256 .. 8192 workgroups of 256 / 512 / 1024 threads, 1 ..
    8 loads in flight per thread), each timed over a >= 512 MB rotation: the
    achievable ceiling for one kernel that must read that many bytes."""
    n_copies = max(2, math.ceil(ROTATE_BYTES / nbytes) + 1)
    buf = torch.empty((n_copies, nbytes), dtype=torch.uint8, device="cuda")
    buf.fill_(1)
    out = torch.zeros(8192, dtype=torch.int32, device="cuda")
    best = None
    for threads in (256, 512, 1024):
        for unroll in (1, 2, 4, 8):
            for blocks in (256, 512, 1024, 2048, 4096, 8192):
                if blocks * threads * unroll * 16 > 4 * nbytes:  # most threads would have nothing to load
                    continue

                def launch(i, stream, b=blocks, t=threads, u=unroll):
                    hip.stream_read_shape(buf[i], nbytes, out, b, t, u, stream=stream)

                us, _ = _events_mean_us(launch, n_copies, iters, replays=3)
                if best is None or us < best["us"]:
                    best = {"blocks": blocks, "threads": threads, "unroll": unroll, "us": round(us, 3)}
    del buf
    torch.cuda.empty_cache()
    gbs = nbytes / (best["us"] * 1e-6) / 1e9
    return {"kernel": "k_stream_read_u", "bytes": nbytes, **best, "GBs": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4), "copies": n_copies}


def stream_read_case(hip, nbytes, iters=100, blocks=4096):
    """Plain streaming read over a >= 512 MB rotation: the achievable-HBM reference."""
    n_copies = max(2, math.ceil(ROTATE_BYTES / nbytes) + 1)
    buf = torch.empty((n_copies, nbytes), dtype=torch.uint8, device="cuda")
    buf.fill_(1)
    out = torch.zeros(blocks, dtype=torch.int32, device="cuda")

    def launch(i, stream):
        hip.stream_read(buf[i], nbytes, out, blocks, stream=stream)

    mean_us, best_us = _events_mean_us(launch, n_copies, iters)
    gbs = nbytes / (mean_us * 1e-6) / 1e9
    del buf
    torch.cuda.empty_cache()
    return {"kernel": "k_stream_read", "bytes": nbytes, "us": round(mean_us, 3), "GBs": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4), "copies": n_copies}


def attention_case(hip, ctxs, n_heads=16, n_kv=4, hd=256, iters=100, seed=0):
    """Decode attention over n_seq = len(ctxs) sequences, each with its own context length
    (a ragged batch); the cache is sized to the longest one."""
    ctxs = [int(c) for c in np.atleast_1d(ctxs)]
    n_seq, max_ctx = len(ctxs), max(ctxs)
    kv = max_ctx * n_kv * hd
    per = n_seq * (2 * kv + 2 * max_ctx * n_kv * 4)
    n_copies = max(2, math.ceil(ROTATE_BYTES / per) + 1)
    keys = torch.randint(-127, 128, (n_copies, n_seq * kv), dtype=torch.int8, device="cuda")
    vals = torch.randint(-127, 128, (n_copies, n_seq * kv), dtype=torch.int8, device="cuda")
    ks = torch.rand((n_copies, n_seq * max_ctx * n_kv), device="cuda") * 0.02 + 0.01
    vs = torch.rand((n_copies, n_seq * max_ctx * n_kv), device="cuda") * 0.02 + 0.01
    q = torch.from_numpy(synth.activations(seed, n_seq * n_heads * hd)).cuda()
    out = torch.empty(n_seq * n_heads * hd, dtype=torch.float32, device="cuda")
    cl = torch.tensor(ctxs, dtype=torch.int32, device="cuda")
    ws = torch.empty(hip.attn_ws_bytes(n_seq, n_heads, hd, max_ctx), dtype=torch.uint8, device="cuda")

    def launch(i, stream):
        hip.attn_decode(q, keys[i], vals[i], ks[i], vs[i], out, cl, n_seq, kv, n_heads, n_kv, hd, max_ctx, ws,
                        stream=stream)

    mean_us, med_us = _events_mean_us(launch, n_copies, iters)
    # bytes the path must read: K and V rows plus their scales for every live position, q, out
    alg = sum(ctxs) * n_kv * (2 * hd + 8) + 2 * n_seq * n_heads * hd * 4
    gbs = alg / (mean_us * 1e-6) / 1e9
    return {"kernel": "k_attn_mfma+k_attn_merge", "ctxs": ctxs if n_seq <= 8 else f"{n_seq} seqs",
            "bytes": alg, "us": round(mean_us, 3), "GBs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
            "copies": n_copies}


def deltanet_case(hip, T=1024, n_v=32, d=128, iters=5, seed=0, chunked=False):
    """The 1024-token, 32-head gated delta-net workload: the token loop
    (k_deltanet) or the chunked scan (k_dn_chunk_prep + k_dn_chunk_scan, both
    launches timed); flops counted as the token loop's 7*d*d per token and head."""
    st = torch.cuda.current_stream().cuda_stream
    g = torch.Generator(device="cuda").manual_seed(seed)
    state0 = torch.randn((n_v, d, d), generator=g, device="cuda") * 0.02
    q = torch.nn.functional.normalize(torch.randn((T, n_v, d), generator=g, device="cuda"), dim=-1)
    k = torch.nn.functional.normalize(torch.randn((T, n_v, d), generator=g, device="cuda"), dim=-1)
    v = torch.randn((T, n_v, d), generator=g, device="cuda")
    dec = torch.sigmoid(torch.randn((T, n_v), generator=g, device="cuda") * 0.5 + 2)
    bet = torch.sigmoid(torch.randn((T, n_v), generator=g, device="cuda"))
    out = torch.empty((T, n_v, d), device="cuda")
    state = state0.clone()
    ws = torch.empty(hip.deltanet_chunked_ws_bytes(T, 1, n_v), dtype=torch.uint8, device="cuda") if chunked else None

    # time only the recurrence: events around the delta-net launch
    evs = []
    for i in range(iters + 1):
        state.copy_(state0)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        if chunked:
            hip.deltanet_chunked(state, q, k, v, dec, bet, out, T, 1, n_v, n_v, d, d, ws, stream=st)
        else:
            hip.deltanet(state, q, k, v, dec, bet, out, T, 1, n_v, n_v, d, d, stream=st)
        b.record()
        evs.append((a, b))
    torch.cuda.synchronize()
    us = float(np.mean([a.elapsed_time(b) for a, b in evs[1:]]) * 1e3)
    flops = 7 * n_v * d * d * T
    tf = flops / (us * 1e-6) / 1e12
    name = "k_dn_chunk_prep+k_dn_chunk_scan" if chunked else "k_deltanet"
    return {"kernel": name, "T": T, "flops": flops, "us": round(us, 2), "us_per_token": round(us / T, 4),
            "TFLOPs": round(tf, 2), "frac": round(tf / FP32_PEAK_TFLOPS, 4)}


INT8_PEAK_TOPS = 5000.0


def attn_prefill_case(hip, T=512, pos0=3584, n_heads=16, n_kv=4, iters=10, seed=0):
    """Causal attention of a T-token prompt chunk at positions pos0 .. pos0+T-1
    (ec_attn_prefill) over an int8 cache; int8 TOP/s counts the MFMA work
    (QK^T and softmax . V, three int8 pieces of q and of p each:
    2 * 2 * 3 * 256 ops per query row and visible position)."""
    hd, max_ctx = 256, pos0 + T
    g = torch.Generator(device="cuda").manual_seed(seed)
    keys = torch.randint(-127, 128, (max_ctx * n_kv * hd,), generator=g, device="cuda", dtype=torch.int32).to(torch.int8)
    vals = torch.randint(-127, 128, (max_ctx * n_kv * hd,), generator=g, device="cuda", dtype=torch.int32).to(torch.int8)
    ks = torch.rand(max_ctx * n_kv, generator=g, device="cuda") * 0.02
    vs = torch.rand(max_ctx * n_kv, generator=g, device="cuda") * 0.02
    q = torch.randn(T, n_heads * hd, generator=g, device="cuda")
    out = torch.empty_like(q)
    ws = torch.empty(max(hip.attn_prefill_ws_bytes(T, n_heads, max_ctx), 16), dtype=torch.uint8, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    hip.attn_prefill(q, keys, vals, ks, vs, out, T, pos0, n_heads, n_kv, hd, max_ctx, ws=ws, stream=st)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(iters):
        hip.attn_prefill(q, keys, vals, ks, vs, out, T, pos0, n_heads, n_kv, hd, max_ctx, ws=ws, stream=st)
    b.record()
    torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1e3 / iters
    visible = T * pos0 + T * (T + 1) / 2  # (query, position) pairs
    ops = 2 * 2 * 3 * hd * n_heads * visible
    tops = ops / (us * 1e-6) / 1e12
    return {"kernel": "k_attn_prefill", "T": T, "pos0": pos0, "us": round(us, 2), "TOPs": round(tops, 1),
            "frac": round(tops / INT8_PEAK_TOPS, 4)}


def gemm_case(hip, fmt, N, K, M=512, iters=20, seed=0):
    """Prefill GEMM (M tokens x N rows x K) on int8 MFMA over a >= 512 MB weight
    rotation; reports int8 TOP/s (2*M*N*K ops) and the fraction of the dense
    int8 MFMA peak."""
    st = torch.cuda.current_stream().cuda_stream
    if fmt == L.Q8_0:
        Wd = torch.empty(N * K // 32 * 34, dtype=torch.uint8, device="cuda")
        hip.fill_random(1, Wd, N * K // 32, seed, 0.02, stream=st)
    else:
        Wd = torch.from_numpy(synth.q4_K_blocks(seed, N, K)).cuda()
    tb = hip.tiled_bytes(fmt, N, K)
    n_copies = max(2, math.ceil(ROTATE_BYTES / tb) + 1)
    tiled = torch.empty((n_copies, tb), dtype=torch.uint8, device="cuda")
    hip.repack(fmt, Wd, tiled[0], N, K, stream=st)
    for i in range(1, n_copies):
        tiled[i].copy_(tiled[0])
    del Wd
    x = torch.from_numpy(synth.activations(seed + 1, M * K)).cuda()
    act = torch.empty(hip.gemm_act_bytes(fmt, M, K), dtype=torch.uint8, device="cuda")
    hip.gemm_quantize_act(fmt, x, act, M, K, stream=st)
    y = torch.empty(M * N, dtype=torch.float32, device="cuda")

    def launch(i, stream):
        hip.gemm(fmt, tiled[i], act, y, M, N, K, stream=stream)

    mean_us, best_us = _events_mean_us(launch, n_copies, iters)
    ops = 2.0 * M * N * K
    tops = ops / (mean_us * 1e-6) / 1e12
    del tiled
    torch.cuda.empty_cache()
    return {"kernel": "k_gemm_q8_0" if fmt == L.Q8_0 else "k_gemm_q4_K", "M": M, "N": N, "K": K,
            "us": round(mean_us, 2), "TOPs": round(tops, 1), "frac": round(tops / INT8_PEAK_TOPS, 4)}


def run_all(hip, quick=False):
    res = {}
    res["q8_0_9216x2560_m1"] = matvec_case(hip, L.Q8_0, 9216, 2560)
    res["q4_K_9216x2560_m1"] = matvec_case(hip, L.Q4_K, 9216, 2560)
    res["q4_K_2560x9216_m1"] = matvec_case(hip, L.Q4_K, 2560, 9216)
    res["q8_0_9216x2560_m8"] = matvec_case(hip, L.Q8_0, 9216, 2560, M=8)
    res["q8_0_151936x2560_m8"] = matvec_case(hip, L.Q8_0, 151936, 2560, M=8, iters=20)
    for ctx in (512, 4096, 32768):
        res[f"attn_ctx{ctx}"] = attention_case(hip, [ctx])
    # a decode batch like the hybrid decoder's: 8 ragged prompts of U[128, 4096] plus 128 generated tokens
    ctxs = (synth.randint(synth.stream_seed(5, 0), 8, 128, 4096) + 128).tolist()
    res["attn_batch8"] = attention_case(hip, ctxs)
    res["deltanet_1024"] = deltanet_case(hip)
    for fmt, tag in ((L.Q4_K, "q4_K"), (L.Q8_0, "q8_0")):
        res[f"gemm_{tag}_512x9216x2560"] = gemm_case(hip, fmt, 9216, 2560)
        res[f"gemm_{tag}_512x2560x9216"] = gemm_case(hip, fmt, 2560, 9216)
    return res


# ---------------------------------------------------------------- PMC traffic
# Matvec shapes of one decode step of the 4B-class hybrid decoder at batch 8
# (M = 8 token rows, two activation pieces): (name, N output rows, K, launches
# per step, K splits), the splits being the engine's defaults for two pieces
# (host/engine.cpp: delta-net input 1, gate/up 4, attention input 4, the
# projections that add into the residual 3; a split writes one partial output).
DECODE_STEP_MATVECS = [("delta_in", 12352, 2560, 24, 1), ("delta_out", 2560, 4096, 24, 3),
                       ("attn_in", 6144, 2560, 8, 4), ("attn_out", 2560, 4096, 8, 3),
                       ("ffn_gate_up", 18432, 2560, 32, 4), ("ffn_down", 2560, 9216, 32, 3),
                       ("lm_head", 151936, 2560, 1, 1)]
PMC_LAUNCHES = 3
CALIB_BYTES = 256 << 20


def pmc_workload(hip, M=8, pieces=2):
    """Launch sequence for rocprofv3 counter collection: every decode-step
    matvec shape PMC_LAUNCHES times (eager, each launch on a different weight
    copy of a >= 512 MB rotation; the decode step's two-piece activations),
    then the calibration kernels of known traffic: k_stream_read of
    CALIB_BYTES twice (reads) and a CALIB_BYTES fill twice (writes)."""
    st = torch.cuda.current_stream().cuda_stream
    for name, N, K, _, ns in DECODE_STEP_MATVECS:
        tb = hip.tiled_bytes(L.Q8_0, N, K)
        n_copies = max(PMC_LAUNCHES, math.ceil(ROTATE_BYTES / tb) + 1)
        Wd = torch.empty(N * K // 32 * 34, dtype=torch.uint8, device="cuda")
        hip.fill_random(1, Wd, N * K // 32, 0, 0.02, stream=st)
        tiled = torch.empty((n_copies, tb), dtype=torch.uint8, device="cuda")
        hip.repack(L.Q8_0, Wd, tiled[0], N, K, stream=st)
        for i in range(1, n_copies):
            tiled[i].copy_(tiled[0])
        del Wd
        x = torch.from_numpy(synth.activations(1, M * K)).cuda()
        act = torch.empty(hip.act_bytes(L.Q8_0, M, K, pieces=pieces), dtype=torch.uint8, device="cuda")
        hip.quantize_act(L.Q8_0, x, act, M, K, stream=st, pieces=pieces)
        y = torch.empty(ns * M * N, dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        for i in range(PMC_LAUNCHES):
            hip.matvec_split(L.Q8_0, tiled[(i * 7919) % n_copies], act, y, M, N, K, ns, stream=st, pieces=pieces)
            torch.cuda.synchronize()
        del tiled
        torch.cuda.empty_cache()
    bufs = [torch.full((CALIB_BYTES,), 1, dtype=torch.uint8, device="cuda") for _ in range(3)]
    out = torch.zeros(4096, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    for i in range(2):
        hip.stream_read(bufs[i], CALIB_BYTES, out, 4096, stream=st)
        torch.cuda.synchronize()
    for i in range(2):
        bufs[2 - i].fill_(2)
        torch.cuda.synchronize()


def pmc_summary(csv_path, counter):
    """Per-dispatch counter values of a pmc_workload run (rocprofv3
    counter_collection.csv), assigned to the launches in order: mean KiB per
    launch of every matvec shape and of the two calibration kernels."""
    import csv
    rows = [r for r in csv.DictReader(open(csv_path)) if r.get("Counter_Name") == counter]
    rows.sort(key=lambda r: int(r["Dispatch_Id"]))
    mv = [float(r["Counter_Value"]) for r in rows if "k_mv_q8_0" in r["Kernel_Name"]]
    rd = [float(r["Counter_Value"]) for r in rows if "k_stream_read" in r["Kernel_Name"]]
    fl = [float(r["Counter_Value"]) for r in rows if "FillFunctor<unsigned char>" in r["Kernel_Name"]][-2:]
    assert len(mv) == PMC_LAUNCHES * len(DECODE_STEP_MATVECS), len(mv)
    res = {"counter": counter, "shapes": {}}
    for j, (name, N, K, per_step, ns) in enumerate(DECODE_STEP_MATVECS):
        v = mv[j * PMC_LAUNCHES:(j + 1) * PMC_LAUNCHES]
        res["shapes"][name] = {"N": N, "K": K, "per_step": per_step, "splits": ns, "KiB": [round(x, 1) for x in v]}
    res["calib_read_KiB"] = [round(x, 1) for x in rd]
    res["calib_fill_KiB"] = [round(x, 1) for x in fl]
    res["calib_bytes"] = CALIB_BYTES
    return res


def pmc_cases(hip, which):
    """Eager launches for counter collection: `attn_prefill` runs the causal
    chunk attention of 512 tokens at position 3584 (16 heads, 4 KV heads),
    `matvec` runs the decode matvec
    at M = 1 (Q8_0 9216 x 2560, Q4_K 9216 x 2560 and 2560 x 9216), `attention` runs the decode
    attention at 512 / 4096 / 32768 positions (16 query heads, 4 KV heads,
    head_dim 256, one sequence), `gemm` the M = 512 prefill GEMMs (Q8_0 and
    Q4_K, 9216 x 2560 and 2560 x 9216), `deltanet` the 1024-token 32-head
    recurrence (token loop, chunked scan) and the batch-8 fused decode update,
    PMC_LAUNCHES times each on different
    buffer copies of a >= 512 MB rotation; then the calibration kernels of
    pmc_workload (a 256 MiB read, a 256 MiB fill).  `gguf` runs the fp32 Q4_K
    matvec over GGUF bytes (ec_matvec_gguf_f32) at 9216 x 2560 and 2560 x 9216, then the Q8_0 one."""
    st = torch.cuda.current_stream().cuda_stream
    if which == "attention":
        for ctx in (512, 4096, 32768):
            n_kv, hd, n_heads = 4, 256, 16
            kv = ctx * n_kv * hd
            per = 2 * kv + 2 * ctx * n_kv * 4
            n_copies = max(PMC_LAUNCHES, math.ceil(ROTATE_BYTES / per) + 1)
            keys = torch.randint(-127, 128, (n_copies, kv), dtype=torch.int8, device="cuda")
            vals = torch.randint(-127, 128, (n_copies, kv), dtype=torch.int8, device="cuda")
            ks = torch.rand((n_copies, ctx * n_kv), device="cuda") * 0.02 + 0.01
            vs = torch.rand((n_copies, ctx * n_kv), device="cuda") * 0.02 + 0.01
            q = torch.from_numpy(synth.activations(0, n_heads * hd)).cuda()
            out = torch.empty(n_heads * hd, dtype=torch.float32, device="cuda")
            cl = torch.tensor([ctx], dtype=torch.int32, device="cuda")
            ws = torch.empty(hip.attn_ws_bytes(1, n_heads, hd, ctx), dtype=torch.uint8, device="cuda")
            torch.cuda.synchronize()
            for i in range(PMC_LAUNCHES):
                c = (i * 7919) % n_copies
                hip.attn_decode(q, keys[c], vals[c], ks[c], vs[c], out, cl, 1, kv, n_heads, n_kv, hd, ctx, ws, stream=st)
                torch.cuda.synchronize()
            del keys, vals, ks, vs
            torch.cuda.empty_cache()
    elif which == "attn_prefill":
        T, pos0, n_heads, n_kv, hd = 512, 3584, 16, 4, 256
        max_ctx = pos0 + T
        g = torch.Generator(device="cuda").manual_seed(0)
        keys = torch.randint(-127, 128, (max_ctx * n_kv * hd,), generator=g, device="cuda", dtype=torch.int32).to(torch.int8)
        vals = torch.randint(-127, 128, (max_ctx * n_kv * hd,), generator=g, device="cuda", dtype=torch.int32).to(torch.int8)
        ks = torch.rand(max_ctx * n_kv, generator=g, device="cuda") * 0.02
        vs = torch.rand(max_ctx * n_kv, generator=g, device="cuda") * 0.02
        q = torch.randn(T, n_heads * hd, generator=g, device="cuda")
        out = torch.empty_like(q)
        ws = torch.empty(max(hip.attn_prefill_ws_bytes(T, n_heads, max_ctx), 16), dtype=torch.uint8, device="cuda")
        torch.cuda.synchronize()
        for _ in range(PMC_LAUNCHES):
            hip.attn_prefill(q, keys, vals, ks, vs, out, T, pos0, n_heads, n_kv, hd, max_ctx, ws=ws, stream=st)
            torch.cuda.synchronize()
        del keys, vals, ks, vs, q, out
        torch.cuda.empty_cache()
    elif which == "pieces":
        # the decode step's gate/up projection (18432 x 2560, 3 K-splits) at M = 8 with one, then two
        # activation pieces
        N, K, M, ns = 18432, 2560, 8, 3
        Wd = torch.empty(N * K // 32 * 34, dtype=torch.uint8, device="cuda")
        hip.fill_random(1, Wd, N * K // 32, 0, 0.02, stream=st)
        tb = hip.tiled_bytes(L.Q8_0, N, K)
        n_copies = max(PMC_LAUNCHES, math.ceil(ROTATE_BYTES / tb) + 1)
        tiled = torch.empty((n_copies, tb), dtype=torch.uint8, device="cuda")
        hip.repack(L.Q8_0, Wd, tiled[0], N, K, stream=st)
        for i in range(1, n_copies):
            tiled[i].copy_(tiled[0])
        x = torch.from_numpy(synth.activations(1, M * K)).cuda()
        y = torch.empty(ns * M * N, dtype=torch.float32, device="cuda")
        for pieces in (1, 2):
            act = torch.empty(hip.act_bytes(L.Q8_0, M, K, pieces=pieces), dtype=torch.uint8, device="cuda")
            hip.quantize_act(L.Q8_0, x, act, M, K, stream=st, pieces=pieces)
            torch.cuda.synchronize()
            for i in range(PMC_LAUNCHES):
                hip.matvec_split(L.Q8_0, tiled[(i * 7919) % n_copies], act, y, M, N, K, ns, stream=st, pieces=pieces)
                torch.cuda.synchronize()
        del tiled
        torch.cuda.empty_cache()
    elif which == "matvec":
        for fmt, N, K in ((L.Q8_0, 9216, 2560), (L.Q4_K, 9216, 2560), (L.Q4_K, 2560, 9216)):
            if fmt == L.Q8_0:
                Wd = torch.empty(N * K // 32 * 34, dtype=torch.uint8, device="cuda")
                hip.fill_random(1, Wd, N * K // 32, 0, 0.02, stream=st)
            else:
                Wd = torch.from_numpy(synth.q4_K_blocks(0, N, K).reshape(-1)).cuda()
            tb = hip.tiled_bytes(fmt, N, K)
            n_copies = max(PMC_LAUNCHES, math.ceil(ROTATE_BYTES / tb) + 1)
            tiled = torch.empty((n_copies, tb), dtype=torch.uint8, device="cuda")
            hip.repack(fmt, Wd, tiled[0], N, K, stream=st)
            for i in range(1, n_copies):
                tiled[i].copy_(tiled[0])
            x = torch.from_numpy(synth.activations(1, K)).cuda()
            act = torch.empty(hip.act_bytes(fmt, 1, K), dtype=torch.uint8, device="cuda")
            hip.quantize_act(fmt, x, act, 1, K, stream=st)
            y = torch.empty(N, dtype=torch.float32, device="cuda")
            torch.cuda.synchronize()
            for i in range(PMC_LAUNCHES):
                hip.matvec(fmt, tiled[(i * 7919) % n_copies], act, y, 1, N, K, stream=st)
                torch.cuda.synchronize()
            del Wd, tiled, x, act, y
            torch.cuda.empty_cache()
    elif which == "gguf":
        # the reference-signature fp32 matvec (GGUF bytes in place), Q4_K then Q8_0, each at 9216 x 2560
        # then 2560 x 9216
        for fmt in (L.Q4_K, L.Q8_0):
            for N, K in ((9216, 2560), (2560, 9216)):
                if fmt == L.Q4_K:
                    wbytes = N * K // 256 * 144
                    W0 = torch.from_numpy(synth.q4_K_blocks(0, N, K).reshape(-1)).cuda()
                else:
                    wbytes = N * K // 32 * 34
                    W0 = torch.empty(wbytes, dtype=torch.uint8, device="cuda")
                    hip.fill_random(1, W0, N * K // 32, 0, 0.02, stream=st)
                n_copies = max(PMC_LAUNCHES, math.ceil(ROTATE_BYTES / wbytes) + 1)
                Ws = torch.empty((n_copies, wbytes), dtype=torch.uint8, device="cuda")
                for i in range(n_copies):
                    Ws[i].copy_(W0)
                del W0
                x = torch.from_numpy(synth.activations(1, K)).cuda()
                y = torch.zeros(N, dtype=torch.float32, device="cuda")
                torch.cuda.synchronize()
                for i in range(PMC_LAUNCHES):
                    hip.matvec_gguf_f32(fmt, Ws[(i * 7919) % n_copies], x, y, N, K, stream=st)
                    torch.cuda.synchronize()
                del Ws, x, y
                torch.cuda.empty_cache()
    elif which == "gemm":
        for fmt in (L.Q8_0, L.Q4_K):
            for N, K in ((9216, 2560), (2560, 9216)):
                M = 512
                if fmt == L.Q8_0:
                    Wd = torch.empty(N * K // 32 * 34, dtype=torch.uint8, device="cuda")
                    hip.fill_random(1, Wd, N * K // 32, 0, 0.02, stream=st)
                else:
                    Wd = torch.from_numpy(synth.q4_K_blocks(0, N, K).reshape(-1)).cuda()
                tiled = torch.empty(hip.tiled_bytes(fmt, N, K), dtype=torch.uint8, device="cuda")
                hip.repack(fmt, Wd, tiled, N, K, stream=st)
                x = torch.from_numpy(synth.activations(1, M * K)).cuda()
                act = torch.empty(hip.gemm_act_bytes(fmt, M, K), dtype=torch.uint8, device="cuda")
                hip.gemm_quantize_act(fmt, x, act, M, K, stream=st)
                y = torch.empty(M * N, dtype=torch.float32, device="cuda")
                torch.cuda.synchronize()
                for _ in range(PMC_LAUNCHES):
                    hip.gemm(fmt, tiled, act, y, M, N, K, stream=st)
                    torch.cuda.synchronize()
                del Wd, tiled, x, act, y
                torch.cuda.empty_cache()
    elif which == "deltanet":
        # the 1024-token, 32-head recurrence (token loop, then chunked scan) and
        # the decode step's fused delta-net update at batch 8 (4B shapes: 32
        # value heads, 16 key heads, conv kernel 4)
        T, n_v, d = 1024, 32, 128
        g = torch.Generator(device="cuda").manual_seed(0)
        state = torch.randn((n_v, d, d), generator=g, device="cuda") * 0.02
        q = torch.nn.functional.normalize(torch.randn((T, n_v, d), generator=g, device="cuda"), dim=-1)
        k = torch.nn.functional.normalize(torch.randn((T, n_v, d), generator=g, device="cuda"), dim=-1)
        v = torch.randn((T, n_v, d), generator=g, device="cuda")
        dec = torch.sigmoid(torch.randn((T, n_v), generator=g, device="cuda") * 0.5 + 2)
        bet = torch.sigmoid(torch.randn((T, n_v), generator=g, device="cuda"))
        out = torch.empty((T, n_v, d), device="cuda")
        ws = torch.empty(hip.deltanet_chunked_ws_bytes(T, 1, n_v), dtype=torch.uint8, device="cuda")
        torch.cuda.synchronize()
        for _ in range(PMC_LAUNCHES):
            hip.deltanet(state, q, k, v, dec, bet, out, T, 1, n_v, n_v, d, d, stream=st)
            torch.cuda.synchronize()
        for _ in range(PMC_LAUNCHES):
            hip.deltanet_chunked(state, q, k, v, dec, bet, out, T, 1, n_v, n_v, d, d, ws, stream=st)
            torch.cuda.synchronize()
        del q, k, v, dec, bet, out, ws
        B, n_k, kern = 8, 16, 4
        conv_dim = 2 * n_k * d + n_v * d
        Nin = conv_dim + n_v * d + 2 * n_v
        proj = torch.randn((B, Nin), generator=g, device="cuda")
        conv_state = torch.randn((B, kern, conv_dim), generator=g, device="cuda") * 0.1
        conv_w = torch.randn((kern, conv_dim), generator=g, device="cuda") * 0.3
        a_log = torch.randn(n_v, generator=g, device="cuda") * 0.1
        dt_bias = torch.randn(n_v, generator=g, device="cuda") * 0.1
        norm_w = 1 + 0.1 * torch.randn(d, generator=g, device="cuda")
        states = torch.randn((3, B, n_v, d, d), generator=g, device="cuda") * 0.02
        act = torch.empty(hip.act_bytes(L.Q8_0, B, n_v * d), dtype=torch.uint8, device="cuda")
        pos = torch.arange(100, 100 + B, dtype=torch.int32, device="cuda")
        torch.cuda.synchronize()
        for i in range(PMC_LAUNCHES):
            hip.delta_step(proj, Nin, conv_state, conv_w, a_log, dt_bias, norm_w, states[i % 3], act, pos, B, n_k,
                           n_v, kern, stream=st)
            torch.cuda.synchronize()
        del states
        torch.cuda.empty_cache()
    else:
        raise ValueError(which)
    bufs = [torch.full((CALIB_BYTES,), 1, dtype=torch.uint8, device="cuda") for _ in range(3)]
    out = torch.zeros(4096, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    for i in range(2):
        hip.stream_read(bufs[i], CALIB_BYTES, out, 4096, stream=st)
        torch.cuda.synchronize()
    for i in range(2):
        bufs[2 - i].fill_(2)
        torch.cuda.synchronize()


def pmc_kernel_means(csv_path, counters):
    """Mean value per dispatch of each counter, per kernel name, from a
    rocprofv3 counter_collection.csv (several counters of one pass)."""
    import csv
    acc = {}
    for r in csv.DictReader(open(csv_path)):
        if r.get("Counter_Name") not in counters:
            continue
        k = r["Kernel_Name"].replace("(anonymous namespace)::", "").split("(")[0]
        d = acc.setdefault(k, {}).setdefault(r["Counter_Name"], [])
        d.append(float(r["Counter_Value"]))
    return {k: {c: round(sum(v) / len(v), 1) for c, v in cs.items()} | {"dispatches": len(next(iter(cs.values())))}
            for k, cs in acc.items()}


if __name__ == "__main__":
    import json
    import sys
    if len(sys.argv) > 1 and sys.argv[1] == "--pmc-workload":
        pmc_workload(L.load())
        print("pmc workload done", flush=True)
    elif len(sys.argv) > 2 and sys.argv[1] == "--pmc-cases":
        pmc_cases(L.load(), sys.argv[2])
        print("pmc cases done", flush=True)
    elif len(sys.argv) > 3 and sys.argv[1] == "--pmc-means":
        print(json.dumps(pmc_kernel_means(sys.argv[2], sys.argv[3].split(",")), indent=1))
    elif len(sys.argv) > 3 and sys.argv[1] == "--pmc-summary":
        print(json.dumps(pmc_summary(sys.argv[2], sys.argv[3])))
    elif len(sys.argv) > 1 and sys.argv[1] == "--ceiling":
        hip = L.load()
        for nbytes in (13271040, 25067520, 50135040, 436 << 20):
            print(json.dumps(stream_read_sweep(hip, nbytes)), flush=True)
    else:
        hip = L.load()
        r = run_all(hip)
        for k, v in r.items():
            print(k, json.dumps(v), flush=True)
