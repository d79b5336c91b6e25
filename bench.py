#!/usr/bin/env python3
"""Decode throughput of the synthetic 4B-class hybrid Q8_0 decoder on one MI355X.

Workload: 32 blocks (24 gated-delta-net + 8 full-attention, GQA 16q/4kv,
head_dim 256, INT8 KV), hidden 2560, FFN 9216 SwiGLU, vocab 151936, all
matrices Q8_0 with seeded random weights generated on the device.  A ragged
batch of 8 sequences with prompt lengths drawn uniformly from [128, 4096]
(uniform random token ids) is prefilled (chunked prefill, 512-token chunks of
int8-MFMA GEMMs; timed separately and reported as config.prefill_tok_s, not
part of `value`), then W warm-up and K timed greedy decode steps run as
HIP-graph replays.  --prefill loop feeds the prompts token by token through
the decode graph instead.

value = 8 * K / (time of the K steps): decode tokens per second.
roofline: the Q8_0 matvec (the dominant kernel) — algorithmic bytes of the
129 matvec launches of one decode step / their GPU time (the step's matvecs
replayed alone in a HIP graph between HIP events), vs 8 TB/s; traffic = HBM
bytes per launch from rocprofv3 FETCH_SIZE / WRITE_SIZE
(profiles/matvec_q8_0_traffic.txt).
cpu_baseline: the oracle's AVX2 restatement of the reference decoder
(fp32 activations, OpenMP over matvec rows) on this host's cores with the same
weights, the reference's token-at-a-time loop (engine.zig:843-854): decode
steps of the same batch of 8 at the same contexts (each step = 8 sequence
tokens in turn) and one 512-token prompt chunk as a token loop; all-core
sample: 16 decode steps and the 512-token chunk; 1-thread sample: one decode
step and 16 prompt tokens (the rates are per token, so the extrapolation to
the full workload is linear; stated in the line).
"""
from __future__ import annotations

import argparse
import dataclasses
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT / "echo-core_amd", ROOT / "oracle"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

HBM_PEAK_GBS = 8000.0


def log(msg):
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


def step_traffic_bytes(cfg, eng_weight_bytes, ctx_sum, batch):
    """Algorithmic HBM bytes of one decode step: weights once, delta-net state
    read+written, conv state read+written, KV (int8 K+V + scales) read."""
    n_delta = sum(1 for l in range(cfg.n_layers) if not cfg.is_attn(l))
    n_attn = cfg.n_layers - n_delta
    state = n_delta * batch * cfg.ssm_heads * 128 * 128 * 4 * 2
    conv = n_delta * batch * cfg.conv_kernel * cfg.conv_dim * 4 * 2
    kv = n_attn * ctx_sum * (2 * cfg.n_kv * cfg.head_dim + 2 * cfg.n_kv * 4)
    return eng_weight_bytes + state + conv + kv


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo), or 'unknown'."""
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(eng, cfg, lens, threads, decode_steps=16, prefill_tokens=512):
    """The reference decoder's CPU rate on the engine's own weights (host copy):
    the oracle's AVX2 decoder, fp32 activations, one token at a time
    (engine.zig:843-854).  Decode: the benchmark's batch of sequences at its
    contexts (lens; cache and state contents do not change the work), each
    step one token of every sequence in turn; prefill: a fresh sequence's
    prompt tokens one by one from position 0.  `threads` threads, then 1
    thread on a 1-step / 16-token sample.  Returns {threads: (decode tok/s,
    prefill tok/s, seconds)}."""
    from oracle import Baseline, Decoder

    m = eng.export_model()
    bl = Baseline()
    B = len(lens)
    dcfg = dataclasses.replace(cfg, max_batch=B, max_ctx=max(lens) + decode_steps + 2)
    pcfg = dataclasses.replace(cfg, max_batch=1, max_ctx=prefill_tokens + 2)
    res = {}
    for nthr, nsteps, ntok in ((threads, decode_steps, prefill_tokens), (1, 1, 16)):
        bl.threads(nthr)
        dec = Decoder(bl, dcfg, m, n_seq=B, quant_act=False)
        for s in range(B):
            dec.seqs[s].pos = int(lens[s])
        dec.token(0, 1)  # warm-up (page-in), then back to the sequence's context
        dec.seqs[0].pos = int(lens[0])
        t0 = time.perf_counter()
        for step in range(nsteps):
            for s in range(B):
                dec.token(s, 1000 + 17 * step + 3 * s)
        td = time.perf_counter() - t0
        del dec
        pre = Decoder(bl, pcfg, m, n_seq=1, quant_act=False)
        t0 = time.perf_counter()
        for i in range(ntok):
            pre.token(0, 2000 + 13 * i)
        tp = time.perf_counter() - t0
        del pre
        res[nthr] = (nsteps * B / td, ntok / tp, td + tp)
        log(f"cpu baseline: {nthr} thread(s): {nsteps} batch-{B} decode steps in {td:.2f} s "
            f"({res[nthr][0]:.3f} tok/s), {ntok} prompt tokens in {tp:.2f} s ({res[nthr][1]:.3f} tok/s)")
    return res


def cpu_kernel_baselines(threads):
    """The matvec, attention and delta-net workloads on the host CPU: the
    oracle's AVX2 row kernels (reference structure, fp32 activations) and its
    attention / delta-net restatements, OpenMP over rows / heads, on 1 thread
    and on `threads`; one warm-up, then the best of 5 (the delta-net: 64 of
    the 1024 tokens, per-token time reported)."""
    import ctypes as C

    import numpy as np

    from echohip import synth
    from oracle import Baseline

    bl = Baseline()
    L = bl.lib
    res = {}

    def best(fn, reps=5):
        fn()
        t = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            t.append(time.perf_counter() - t0)
        return min(t)

    p = lambda a: a.ctypes.data  # noqa: E731
    for fmt, N, K in ((6, 9216, 2560), (10, 9216, 2560), (10, 2560, 9216)):
        W = synth.q8_0_blocks(0, N, K) if fmt == 6 else synth.q4_K_blocks(0, N, K)
        x = synth.activations(1, K)
        y = np.zeros(N, np.float32)
        fn = L.ob_matvec_q8_0_avx2 if fmt == 6 else L.ob_matvec_q4_K_avx2
        name = f"{'q8_0' if fmt == 6 else 'q4_K'}_{N}x{K}"
        row = {}
        for nthr in (1, threads):
            bl.threads(nthr)
            s = best(lambda: fn(p(W), p(x), p(y), N, K))
            row[f"us_{nthr}t"] = round(s * 1e6, 1)
            row[f"GBs_{nthr}t"] = round(W.nbytes / s / 1e9, 2)
        res[name] = row
    n_heads, n_kv, hd = 16, 4, 256
    for ctx in (512, 4096, 32768):
        keys = synth.randint(3, ctx * n_kv * hd, -127, 127).astype(np.int8)
        vals = synth.randint(4, ctx * n_kv * hd, -127, 127).astype(np.int8)
        ks = (0.01 + 0.02 * synth.uniform01(5, ctx * n_kv)).astype(np.float32)
        vs = (0.01 + 0.02 * synth.uniform01(6, ctx * n_kv)).astype(np.float32)
        q = synth.activations(7, n_heads * hd)
        out = np.zeros(n_heads * hd, np.float32)
        row = {}
        for nthr in (1, threads):
            bl.threads(nthr)
            s = best(lambda: L.oc_attn_decode_int8(p(q), p(keys), p(vals), p(ks), p(vs), p(out), n_heads, n_kv, hd,
                                                   ctx))
            row[f"us_{nthr}t"] = round(s * 1e6, 1)
            row[f"GBs_{nthr}t"] = round((2080 * ctx + 32768) / s / 1e9, 2)
        res[f"attn_ctx{ctx}"] = row
    n_v, d, T = 32, 128, 64
    rng = np.random.default_rng(0)
    S0 = (rng.standard_normal((n_v, d, d)) * 0.02).astype(np.float32)
    qk = rng.standard_normal((2, T, n_v, d)).astype(np.float32)
    qk /= np.linalg.norm(qk, axis=-1, keepdims=True)
    v = rng.standard_normal((T, n_v, d)).astype(np.float32)
    dec = (1 / (1 + np.exp(-rng.normal(2, 0.5, (T, n_v))))).astype(np.float32)
    bet = (1 / (1 + np.exp(-rng.normal(0, 1, (T, n_v))))).astype(np.float32)
    o = np.zeros(n_v * d, np.float32)
    row = {}
    for nthr in (1, threads):
        bl.threads(nthr)
        S = S0.copy()

        def run():
            for t in range(T):
                L.oc_deltanet_step(p(S), p(qk[0, t]), p(qk[1, t]), p(v[t]), p(dec[t]), p(bet[t]), p(o), n_v, n_v, d, d)
        s = best(run) / T
        row[f"us_per_token_{nthr}t"] = round(s * 1e6, 1)
        row[f"GFLOPs_{nthr}t"] = round(7 * n_v * d * d / s / 1e9, 2)
    res["deltanet_32h"] = row
    return res


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=240, help="timed decode steps")
    ap.add_argument("--warmup", type=int, default=16, help="untimed decode steps before timing")
    ap.add_argument("--batch", type=int, default=8)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--max-prompt", type=int, default=4096, help="upper bound of the prompt-length draw")
    ap.add_argument("--cpu-steps", type=int, default=16,
                    help="all-core CPU baseline: batch-8 decode steps (the 1-thread leg runs one)")
    ap.add_argument("--cpu-prefill", type=int, default=512,
                    help="all-core CPU baseline: prompt tokens of the token-loop prefill (1 thread: 16)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-kernels", action="store_true")
    ap.add_argument("--no-graph", action="store_true",
                    help="launch every step's kernels directly instead of replaying the captured HIP graph "
                         "(rocprofv3 counter collection does not follow graph launches)")
    ap.add_argument("--prefill", choices=("chunked", "loop"), default="chunked",
                    help="chunked: ec_engine_prefill per sequence; loop: token by token through the decode graph")
    ap.add_argument("--act-pieces", type=int, choices=(1, 2), default=2,
                    help="int8 pieces per decode-matvec activation element (2: within ~2e-5 of the reference's "
                         "fp32-activation matvec; 1: the reference quantizer alone, ~5e-3)")
    ap.add_argument("--copy-calibration-mb", type=int, default=0,
                    help="after the run, one device-to-device copy of this many MiB (a kernel of known "
                         "traffic, for calibrating rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1:
        sys.exit("bench.py measures one GPU: this build has no multi-GPU path (run with --gpus 1)")

    import numpy as np
    import torch

    from echohip import kbench, synth
    from echohip.engine import Engine, EngineConfig
    from echohip.lib import load

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    B, K, W = args.batch, args.steps, args.warmup
    lens = synth.randint(synth.stream_seed(args.seed, 1000), B, 128, args.max_prompt).astype(np.int64)
    max_ctx = int(lens.max()) + W + K + 8
    cfg = EngineConfig(max_batch=B, max_ctx=max_ctx)
    log(f"engine: {cfg}")
    t0 = time.perf_counter()
    eng = Engine(cfg)
    eng.set_act_pieces(args.act_pieces)
    eng.init_random(seed=args.seed)
    eng.reset()
    log(f"weights generated and repacked in {time.perf_counter() - t0:.1f} s ({eng.weight_bytes() / 1e9:.3f} GB)")
    prompts = [synth.randint(synth.stream_seed(args.seed, 2000 + s), int(lens[s]), 0, cfg.vocab - 1).astype(np.int32)
               for s in range(B)]

    # ---- prefill (not part of `value`); a one-token prefill of four sequences
    # first allocates the engine's prefill lanes, then the state is reset
    if args.prefill == "chunked":
        eng.prefill_batch([(s, prompts[s][:1], 0) for s in range(min(4, B))])
        eng.reset()
    t0 = time.perf_counter()
    T = int(lens.max())
    if args.prefill == "chunked":  # all prompts, two passes of two sequences' chunks in flight
        eng.prefill_batch([(s, prompts[s], 0) for s in range(B)])
        eng.sync()
    else:  # token loop through the decode graph, ragged
        for t in range(T):
            tok = np.array([prompts[s][t] if t < lens[s] else 0 for s in range(B)], np.int32)
            pos = np.array([t if t < lens[s] else -1 for s in range(B)], np.int32)
            eng.set_inputs(tok, pos)
            eng.step(graph=not args.no_graph)
            if t % 512 == 0:
                eng.sync()
                log(f"prefill step {t}/{T}")
        eng.sync()
    prefill_s = time.perf_counter() - t0
    gen, last_pos = eng.tokens()  # gen[s]: greedy token after sequence s's last prompt token
    if args.prefill == "chunked":
        assert np.array_equal(last_pos, lens)
    pos = lens.astype(np.int32)  # next position of every sequence
    prefill_tps = int(lens.sum()) / prefill_s
    log(f"prefill ({args.prefill}) {int(lens.sum())} tokens in {prefill_s:.2f} s -> {prefill_tps:.0f} tok/s; "
        f"prompts {lens.tolist()}")

    # ---- decode: warm-up then timed graph replays
    eng.set_inputs(gen, pos)
    ext = torch.cuda.ExternalStream(eng.stream)
    for _ in range(W):
        eng.step(graph=not args.no_graph)
    eng.sync()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    w0 = time.perf_counter()
    e0.record(ext)
    for _ in range(K):
        eng.step(graph=not args.no_graph)
    e1.record(ext)
    eng.sync()
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    ms = e0.elapsed_time(e1)
    ms_per_step = ms / K
    value = B * K / (ms * 1e-3)
    gen2, pos2 = eng.tokens()
    assert np.array_equal(pos2, pos + W + K)
    log(f"decode: {K} steps in {ms:.1f} ms (wall {wall * 1e3:.1f} ms) -> {value:.1f} tok/s; last tokens {gen2.tolist()}")

    # ---- roofline of the dominant kernel (Q8_0 matvec): the step's matvecs
    # alone, captured in a graph and replayed between HIP events on the engine stream
    n_mv, mv_bytes, mv_us = eng.profile_matvecs(reps=20)
    mv_gbs = mv_bytes / (mv_us * 1e-6) / 1e9
    traffic = None
    tf = ROOT / "profiles" / "matvec_q8_0_traffic.txt"
    if tf.exists():  # HBM bytes of one step's matvecs measured with rocprofv3 PMC counters (see that file)
        for ln in tf.read_text().splitlines():
            if ln.startswith("hbm_bytes_per_step_matvecs:"):
                traffic = round(int(ln.split(":")[1]) / n_mv)
    ctx_sum = int((pos2).sum())
    step_bytes = step_traffic_bytes(cfg, eng.weight_bytes(), ctx_sum, B)
    log(f"matvec: {n_mv} launches/step, {mv_bytes / 1e9:.3f} GB in {mv_us:.1f} us -> {mv_gbs:.0f} GB/s; "
        f"step: {step_bytes / 1e9:.3f} GB in {ms_per_step:.3f} ms -> {step_bytes / ms_per_step / 1e6:.0f} GB/s")

    kernels = None
    if not args.no_kernels:
        hip = load()
        kernels = {}
        for name, fn in (("q8_0_9216x2560", lambda: kbench.matvec_case(hip, 6, 9216, 2560)),
                         ("q4_K_9216x2560", lambda: kbench.matvec_case(hip, 10, 9216, 2560)),
                         ("q4_K_2560x9216", lambda: kbench.matvec_case(hip, 10, 2560, 9216)),
                         ("gguf_f32_q8_0_9216x2560", lambda: kbench.gguf_f32_case(hip, 6, 9216, 2560)),
                         ("gguf_f32_q4_K_9216x2560", lambda: kbench.gguf_f32_case(hip, 10, 9216, 2560)),
                         ("gguf_f32_q4_K_2560x9216", lambda: kbench.gguf_f32_case(hip, 10, 2560, 9216)),
                         ("attn_ctx512", lambda: kbench.attention_case(hip, 512)),
                         ("attn_ctx4096", lambda: kbench.attention_case(hip, 4096)),
                         ("attn_ctx32768", lambda: kbench.attention_case(hip, 32768)),
                         ("attn_prefill_512tok_at_3584", lambda: kbench.attn_prefill_case(hip)),
                         ("deltanet_1024tok", lambda: kbench.deltanet_case(hip)),
                         ("deltanet_1024tok_chunked", lambda: kbench.deltanet_case(hip, chunked=True))):
            r = fn()
            kernels[name] = {k: r[k] for k in ("us", "GBs", "TFLOPs", "TOPs", "frac") if k in r}
            log(f"kernel {name}: {kernels[name]}")

    cpu = None
    if not args.no_cpu:
        # the host share of one GPU: OMP_NUM_THREADS (16 on this pool's one-GPU boxes), else every core
        threads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
        res = cpu_baseline(eng, cfg, lens.tolist(), threads, args.cpu_steps, args.cpu_prefill)
        log("cpu baseline: kernel workloads")
        cpu_kernels = cpu_kernel_baselines(threads)
        log(f"cpu kernels: {cpu_kernels}")
        d_all, p_all, s_all = res[threads]
        d_one, p_one, s_one = res[1]
        full_tokens = B * (W + K)
        cpu = {"value": round(d_all, 4), "unit": "tok/s", "cores": threads, "kind": "port",
               "sample": f"the reference's token-at-a-time loop (oracle AVX2 decoder, fp32 activations, OpenMP over "
                         f"matvec rows, {threads} threads = the host share of one GPU, OMP_NUM_THREADS) on the same "
                         f"4B-class weights: {args.cpu_steps} decode steps of the same batch of {B} at the same "
                         f"contexts ({min(lens.tolist())}..{max(lens.tolist())}), i.e. {args.cpu_steps * B} tokens, "
                         f"{d_all:.3f} tok/s, and one {args.cpu_prefill}-token prompt chunk fed token by token, "
                         f"{p_all:.3f} tok/s ({s_all:.1f} s); 1 thread on 1 decode step ({B} tokens) and "
                         f"{16} prompt tokens: {d_one:.4f} / {p_one:.4f} tok/s ({s_one:.1f} s).  Extrapolated "
                         f"linearly (per-token rates): this run's {W + K} decode steps ({full_tokens} tokens) take "
                         f"{full_tokens / d_all:.0f} s on {threads} threads and {full_tokens / d_one:.0f} s on "
                         f"1 thread; its {int(lens.sum())} prompt tokens {int(lens.sum()) / p_all:.0f} s and "
                         f"{int(lens.sum()) / p_one:.0f} s.  Host CPU: {cpu_model()}, {os.cpu_count()} hardware "
                         f"threads visible",
               "decode_tok_s_1t": round(d_one, 4), "prefill_tok_s": round(p_all, 4),
               "prefill_tok_s_1t": round(p_one, 4), "kernels": cpu_kernels}

    line = {
        "metric": "decode tok/s (4B-class Q8_0, 1 GPU); matvec HBM GB/s as % of peak",
        "value": round(value, 2), "unit": "tok/s", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8", "data": "synthetic (seeded random Q8_0 weights generated on device, uniform random prompts)",
        "config": {"workload": "hybrid 4B-class Q8_0 decoder: 24 delta-net + 8 attention blocks, hidden 2560, "
                               "ffn 9216, vocab 151936; ragged batch of 8, greedy decode",
                   "global_batch": B, "prompt_lens": lens.tolist(), "decode_steps": W + K,
                   "act_pieces": args.act_pieces,
                   "prefill": ("chunked (512-token chunks per sequence; two sequences' chunks per int8-MFMA GEMM, two such passes in flight)" if args.prefill == "chunked"
                               else "token loop through the decode graph"),
                   "prefill_tok_s": round(prefill_tps, 1),
                   "step_hbm_bytes": int(step_bytes),
                   "step_hbm_frac": round(step_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
        "roofline": {"bound": "hbm", "achieved": round(mv_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(mv_gbs / HBM_PEAK_GBS, 4), "traffic": traffic, "kernel": "k_mv_q8_0 (M=8)",
                     "bytes_per_launch": int(round(mv_bytes / n_mv)), "avg_launch_us": round(mv_us / n_mv, 3),
                     "bytes_per_step": int(mv_bytes), "launches_per_step": n_mv},
        "cpu_baseline": cpu,
        "kernels": kernels,
    }
    print(json.dumps(line), flush=True)
    eng.close()
    if args.copy_calibration_mb:
        n = args.copy_calibration_mb << 20
        src = torch.empty(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        src.fill_(1)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy calibration: {n} bytes read + {n} bytes written")
    return 0


if __name__ == "__main__":
    sys.exit(main())
