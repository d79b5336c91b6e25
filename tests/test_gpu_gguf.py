"""GGUF -> device loader (ec_engine_load_gguf) on the small hybrid model.

The test model (decoder_util.make_model) is written as a GGUF file with the
reference's tensor names and shapes (blk.N.attn_qkv / attn_gate / ssm_alpha /
ssm_beta / ssm_out / ssm_conv1d / ssm_a / ssm_dt.bias / ssm_norm for delta-net
blocks, attn_q / attn_k / attn_v / attn_output / attn_q_norm / attn_k_norm for
attention blocks, ffn_*, attn_norm, post_attention_norm, token_embd,
output_norm, output), loaded through the file, and compared with the same
model uploaded tensor by tensor: every tensor read back must be
byte-identical, and a few decode steps must give bit-identical logits.
"""
import dataclasses

import numpy as np
import pytest

import gguf_writer as gw
from decoder_util import make_model, small_config, upload

pytestmark = pytest.mark.gpu

Q8, F32 = 6, 0


def _rows(b, K, r0, r1):
    rb = K // 32 * 34
    return b.reshape(-1)[r0 * rb:r1 * rb]


def model_gguf(cfg, m, path, tied=False):
    from test_gguf import hybrid_metadata
    H, F = cfg.hidden, cfg.ffn
    T = [("token_embd.weight", Q8, [H, cfg.vocab], m["embed"]), ("output_norm.weight", F32, [H], m["final_norm"])]
    if not tied:
        T.append(("output.weight", Q8, [H, cfg.vocab], m["lm_head"]))
    for l, y in enumerate(m["layers"]):
        b = f"blk.{l}."
        T += [(b + "attn_norm.weight", F32, [H], y["attn_norm"]), (b + "post_attention_norm.weight", F32, [H],
                                                                     y["ffn_norm"]),
              (b + "ffn_gate.weight", Q8, [H, F], y["w_gate"]), (b + "ffn_up.weight", Q8, [H, F], y["w_up"]),
              (b + "ffn_down.weight", Q8, [F, H], y["w_down"])]
        if y["attn"]:
            q, kv = cfg.n_heads * cfg.head_dim, cfg.n_kv * cfg.head_dim
            T += [(b + "attn_q.weight", Q8, [H, q], _rows(y["w_in"], H, 0, q)),
                  (b + "attn_k.weight", Q8, [H, kv], _rows(y["w_in"], H, q, q + kv)),
                  (b + "attn_v.weight", Q8, [H, kv], _rows(y["w_in"], H, q + kv, q + 2 * kv)),
                  (b + "attn_output.weight", Q8, [q, H], y["w_out"]),
                  (b + "attn_q_norm.weight", F32, [cfg.head_dim], y["q_norm"]),
                  (b + "attn_k_norm.weight", F32, [cfg.head_dim], y["k_norm"])]
        else:
            c, v, n = cfg.conv_dim, cfg.ssm_inner, cfg.ssm_heads
            T += [(b + "attn_qkv.weight", Q8, [H, c], _rows(y["w_in"], H, 0, c)),
                  (b + "attn_gate.weight", Q8, [H, v], _rows(y["w_in"], H, c, c + v)),
                  (b + "ssm_alpha.weight", Q8, [H, n], _rows(y["w_in"], H, c + v, c + v + n)),
                  (b + "ssm_beta.weight", Q8, [H, n], _rows(y["w_in"], H, c + v + n, c + v + 2 * n)),
                  (b + "ssm_out.weight", Q8, [v, H], y["w_out"]),
                  (b + "ssm_conv1d.weight", F32, [cfg.conv_kernel, c], y["conv_w"]),
                  (b + "ssm_a", F32, [n], y["a_log"]), (b + "ssm_dt.bias", F32, [n], y["dt_bias"]),
                  (b + "ssm_norm.weight", F32, [128], y["ssm_norm"])]
    T = [(name, t, shape, np.ascontiguousarray(a).view(np.uint8).reshape(-1).tobytes()) for name, t, shape, a in T]
    gw.write(path, hybrid_metadata(cfg), T)


def _decode(eng, steps=6):
    eng.reset()
    toks = np.array([5, 77, 901], np.int32)
    out = []
    for s in range(steps):
        eng.set_inputs(toks, np.array([s, s, s], np.int32))
        eng.step(graph=False)
        gen, _ = eng.tokens()
        out.append([eng.logits(i) for i in range(3)])
        toks = gen.astype(np.int32)
    return out


@pytest.mark.parametrize("tied", [False, True])
def test_gguf_load_matches_upload(tmp_path, tied):
    from echohip.engine import (T_A_LOG, T_ATTN_NORM, T_CONV_W, T_DT_BIAS, T_EMBED, T_FFN_NORM, T_FINAL_NORM, T_K_NORM,
                                T_LM_HEAD, T_Q_NORM, T_SSM_NORM, T_W_DOWN, T_W_GATE, T_W_IN, T_W_OUT, T_W_UP, Engine)
    from echohip.gguf import GGUF
    cfg = small_config(max_batch=3, max_ctx=32)
    m = make_model(cfg, seed=11)
    if tied:
        m["lm_head"] = m["embed"]
    f = tmp_path / "small.gguf"
    model_gguf(cfg, m, f, tied=tied)
    with GGUF(f) as g:
        gcfg = g.engine_config(3, 32)
        assert gcfg == cfg
        a = Engine(gcfg)
        g.load_into(a)
    b = Engine(cfg)
    upload(b, m)
    glob = [(T_EMBED, m["embed"]), (T_FINAL_NORM, m["final_norm"]), (T_LM_HEAD, m["lm_head"])]
    for t, arr in glob:
        nb = np.asarray(arr).nbytes
        assert np.array_equal(a.get_tensor(0, t, nb), b.get_tensor(0, t, nb))
    ids = {"w_in": T_W_IN, "w_out": T_W_OUT, "w_gate": T_W_GATE, "w_up": T_W_UP, "w_down": T_W_DOWN,
           "attn_norm": T_ATTN_NORM, "ffn_norm": T_FFN_NORM, "q_norm": T_Q_NORM, "k_norm": T_K_NORM,
           "conv_w": T_CONV_W, "a_log": T_A_LOG, "dt_bias": T_DT_BIAS, "ssm_norm": T_SSM_NORM}
    for l, y in enumerate(m["layers"]):
        for k, t in ids.items():
            if k in y:
                nb = np.asarray(y[k]).nbytes
                ga, gb = a.get_tensor(l, t, nb), b.get_tensor(l, t, nb)
                assert np.array_equal(ga, gb), (l, k)
                assert np.array_equal(ga, np.ascontiguousarray(y[k]).view(np.uint8).reshape(-1)), (l, k)
    la, lb = _decode(a), _decode(b)
    for sa, sb in zip(la, lb):
        for x, y in zip(sa, sb):
            assert np.array_equal(x, y)
    a.close()
    b.close()


def test_gguf_load_rejects_wrong_shapes(tmp_path):
    from echohip.engine import Engine
    from echohip.gguf import GGUF
    cfg = small_config(max_batch=1, max_ctx=16)
    m = make_model(cfg, seed=12)
    f = tmp_path / "small.gguf"
    model_gguf(cfg, m, f)
    with GGUF(f) as g:
        wrong = Engine(dataclasses.replace(cfg, ffn=1024))
        with pytest.raises(Exception, match="ffn_gate.weight"):
            g.load_into(wrong)
        wrong.close()
