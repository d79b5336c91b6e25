"""Small hybrid-decoder fixtures shared by the decoder tests: seeded weights,
upload into the GPU engine, and the oracle's token-by-token decoder
(oracle.c oc_decoder_token) on the same weights."""
from __future__ import annotations

import numpy as np

from echohip import synth
from echohip.engine import (F16, F32, Q4_K, Q8_0, EngineConfig, T_A_LOG, T_ATTN_NORM, T_CONV_W, T_DT_BIAS, T_EMBED,
                            T_FFN_NORM, T_FINAL_NORM, T_K_NORM, T_LM_HEAD, T_Q_NORM, T_SSM_NORM, T_W_DOWN, T_W_GATE,
                            T_W_IN, T_W_OUT, T_W_UP)
from oracle import Decoder as OracleDecoder  # noqa: F401  (the oracle's decoder binding)


def small_config(max_batch=3, max_ctx=64):
    return EngineConfig(vocab=1000, hidden=256, ffn=512, n_layers=4, n_heads=4, n_kv=2, head_dim=256, ssm_inner=512,
                        ssm_heads=4, conv_kernel=4, attn_interval=4, max_batch=max_batch, max_ctx=max_ctx)


def _f16vec(seed, n, mean, std):
    """fp32 values that are exactly representable in fp16 (the reference keeps norms as fp16)."""
    return (mean + std * synth.normal(seed, n)).astype(np.float16).astype(np.float32)


# Q4_K blocks of make_model: d, dmin ~ |N|*Q4K_D_STD, sub-scales and mins
# U{0..63}, nibbles U{0..15} -- weights d*sc*q - dmin*m of RMS ~0.02
Q4K_D_STD = 1e-4


def make_model(cfg: EngineConfig, seed=0, w_std=0.02 / 73.0, fmts=None):
    """Weights with weight std ~0.02 (d ~ |N|*w_std, qs ~ U{-127..127}).

    fmts: {(layer, name): format} for matrices stored as Q4_K (name w_in,
    w_out, w_gate, w_up, w_down; layer -1 for lm_head) and an F16 / F32
    embedding ((-1, "embed")); every other matrix Q8_0.  The random streams do
    not depend on fmts."""
    fmts = dict(fmts or {})
    s = iter(range(10_000))
    sd = lambda: synth.stream_seed(seed, next(s))  # noqa: E731
    H, F = cfg.hidden, cfg.ffn

    def mat(l, name, N, K):
        seed_ = sd()
        if fmts.get((l, name), Q8_0) == Q4_K:
            return synth.q4_K_blocks(seed_, N, K, Q4K_D_STD)
        return synth.q8_0_blocks(seed_, N, K, w_std)

    emb_seed = sd()
    emb_fmt = fmts.get((-1, "embed"), Q8_0)
    if emb_fmt == Q8_0:
        emb = synth.q8_0_blocks(emb_seed, cfg.vocab, H, w_std)
    else:
        emb = (0.02 * synth.normal(emb_seed, cfg.vocab * H)).astype(np.float16 if emb_fmt == F16 else np.float32)
    m = {"embed": emb, "final_norm": _f16vec(sd(), H, 1.0, 0.1), "lm_head": mat(-1, "lm_head", cfg.vocab, H),
         "layers": []}
    if fmts:
        m["fmt"] = fmts
    for l in range(cfg.n_layers):
        attn = cfg.is_attn(l)
        nin = cfg.nin_attn if attn else cfg.nin_delta
        kout = cfg.n_heads * cfg.head_dim if attn else cfg.ssm_inner
        y = {"attn": attn, "w_in": mat(l, "w_in", nin, H), "w_out": mat(l, "w_out", H, kout),
             "w_gate": mat(l, "w_gate", F, H), "w_up": mat(l, "w_up", F, H), "w_down": mat(l, "w_down", H, F),
             "attn_norm": _f16vec(sd(), H, 1.0, 0.1), "ffn_norm": _f16vec(sd(), H, 1.0, 0.1)}
        if attn:
            y["q_norm"] = _f16vec(sd(), cfg.head_dim, 1.0, 0.1)
            y["k_norm"] = _f16vec(sd(), cfg.head_dim, 1.0, 0.1)
        else:
            y["conv_w"] = _f16vec(sd(), cfg.conv_kernel * cfg.conv_dim, 0.0, 0.5)
            y["a_log"] = np.log(1.0 + 15.0 * synth.uniform01(sd(), cfg.ssm_heads)).astype(np.float32)
            y["dt_bias"] = _f16vec(sd(), cfg.ssm_heads, 0.0, 0.1)
            y["ssm_norm"] = _f16vec(sd(), 128, 1.0, 0.1)
        m["layers"].append(y)
    return m


# A mixed-format small model (small_config: delta-net blocks 0-2, attention
# block 3): each Q4_K input path of the decode step is taken at least once --
# RMSNorm rows (w_in, gate/up, lm_head), the delta step's fp32 output (block 1
# and 2 w_out), attention's output (block 3 w_out) and SwiGLU rows (w_down) --
# next to Q8_0 matrices, with an F16 embedding.
MIXED_FMTS = {(0, "w_in"): Q4_K, (0, "w_down"): Q4_K, (1, "w_out"): Q4_K, (1, "w_gate"): Q4_K, (1, "w_up"): Q4_K,
              (2, "w_in"): Q4_K, (2, "w_out"): Q4_K, (3, "w_in"): Q4_K, (3, "w_out"): Q4_K, (3, "w_gate"): Q4_K,
              (3, "w_up"): Q4_K, (3, "w_down"): Q4_K, (-1, "lm_head"): Q4_K, (-1, "embed"): F16}


def upload(eng, m):
    ids = {"w_in": T_W_IN, "w_out": T_W_OUT, "w_gate": T_W_GATE, "w_up": T_W_UP, "w_down": T_W_DOWN,
           "lm_head": T_LM_HEAD, "embed": T_EMBED}
    for (l, name), fmt in m.get("fmt", {}).items():
        eng.set_format(max(l, 0), ids[name], fmt)
    eng.set_tensor(0, T_EMBED, m["embed"])
    eng.set_tensor(0, T_FINAL_NORM, m["final_norm"])
    eng.set_tensor(0, T_LM_HEAD, m["lm_head"])
    ids = {"w_in": T_W_IN, "w_out": T_W_OUT, "w_gate": T_W_GATE, "w_up": T_W_UP, "w_down": T_W_DOWN,
           "attn_norm": T_ATTN_NORM, "ffn_norm": T_FFN_NORM, "q_norm": T_Q_NORM, "k_norm": T_K_NORM,
           "conv_w": T_CONV_W, "a_log": T_A_LOG, "dt_bias": T_DT_BIAS, "ssm_norm": T_SSM_NORM}
    for l, y in enumerate(m["layers"]):
        for k, t in ids.items():
            if k in y:
                eng.set_tensor(l, t, y[k])

