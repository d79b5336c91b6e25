"""GGUF -> device loader (ec_engine_load_gguf) on the small hybrid model.

The test model (decoder_util.make_model) is written as a GGUF file with the
reference's tensor names and shapes (blk.N.attn_qkv / attn_gate / ssm_alpha /
ssm_beta / ssm_out / ssm_conv1d / ssm_a / ssm_dt.bias / ssm_norm for delta-net
blocks, attn_q / attn_k / attn_v / attn_output / attn_q_norm / attn_k_norm for
attention blocks, ffn_*, attn_norm, post_attention_norm, token_embd,
output_norm, output), loaded through the file, and compared with the same
model uploaded tensor by tensor: every tensor read back must be
byte-identical, and a few decode steps must give bit-identical logits.  The
mixed-format model stores its matrices as Q4_K or Q8_0 per tensor, its
embedding and every vector as F16 (the reference's fp16 norms,
src/inference.cpp:233-265), and is also decoded against the oracle.
"""
import dataclasses

import numpy as np
import pytest

import gguf_writer as gw
from conftest import rel_l2
from decoder_util import MIXED_FMTS, OracleDecoder, make_model, small_config, upload

pytestmark = pytest.mark.gpu

# type ids of the reference's GGMLType enum (include/gguf_reader.h:14-36),
# which are also the engine's format ids
Q8, Q4K, Q6K, F16, F32 = 6, 10, 12, 1, 0
VECTORS = ("attn_norm", "ffn_norm", "q_norm", "k_norm", "conv_w", "a_log", "dt_bias", "ssm_norm")


def _rows(b, fmt, K, r0, r1):
    from echohip.engine import gguf_row_bytes
    rb = gguf_row_bytes(fmt, K)
    return b.reshape(-1)[r0 * rb:r1 * rb]


def model_gguf(cfg, m, path, tied=False, vec_type=F32, override=None):
    """Write model m as a GGUF file; matrices in m's formats (m["fmt"]), vectors
    as vec_type (F16 holds them exactly only if they are fp16 values);
    override: {tensor name: (type, bytes)} replaces tensors as written."""
    from test_gguf import hybrid_metadata
    H, F = cfg.hidden, cfg.ffn
    fm = m.get("fmt", {})
    ft = lambda l, name: fm.get((l, name), Q8)  # noqa: E731
    vec = lambda a: np.asarray(a, np.float32).astype(np.float16) if vec_type == F16 else a  # noqa: E731
    T = [("token_embd.weight", ft(-1, "embed"), [H, cfg.vocab], m["embed"]),
         ("output_norm.weight", vec_type, [H], vec(m["final_norm"]))]
    if not tied:
        T.append(("output.weight", ft(-1, "lm_head"), [H, cfg.vocab], m["lm_head"]))
    for l, y in enumerate(m["layers"]):
        b = f"blk.{l}."
        fi = ft(l, "w_in")
        T += [(b + "attn_norm.weight", vec_type, [H], vec(y["attn_norm"])),
              (b + "post_attention_norm.weight", vec_type, [H], vec(y["ffn_norm"])),
              (b + "ffn_gate.weight", ft(l, "w_gate"), [H, F], y["w_gate"]),
              (b + "ffn_up.weight", ft(l, "w_up"), [H, F], y["w_up"]),
              (b + "ffn_down.weight", ft(l, "w_down"), [F, H], y["w_down"])]
        if y["attn"]:
            q, kv = cfg.n_heads * cfg.head_dim, cfg.n_kv * cfg.head_dim
            T += [(b + "attn_q.weight", fi, [H, q], _rows(y["w_in"], fi, H, 0, q)),
                  (b + "attn_k.weight", fi, [H, kv], _rows(y["w_in"], fi, H, q, q + kv)),
                  (b + "attn_v.weight", fi, [H, kv], _rows(y["w_in"], fi, H, q + kv, q + 2 * kv)),
                  (b + "attn_output.weight", ft(l, "w_out"), [q, H], y["w_out"]),
                  (b + "attn_q_norm.weight", vec_type, [cfg.head_dim], vec(y["q_norm"])),
                  (b + "attn_k_norm.weight", vec_type, [cfg.head_dim], vec(y["k_norm"]))]
        else:
            c, v, n = cfg.conv_dim, cfg.ssm_inner, cfg.ssm_heads
            T += [(b + "attn_qkv.weight", fi, [H, c], _rows(y["w_in"], fi, H, 0, c)),
                  (b + "attn_gate.weight", fi, [H, v], _rows(y["w_in"], fi, H, c, c + v)),
                  (b + "ssm_alpha.weight", fi, [H, n], _rows(y["w_in"], fi, H, c + v, c + v + n)),
                  (b + "ssm_beta.weight", fi, [H, n], _rows(y["w_in"], fi, H, c + v + n, c + v + 2 * n)),
                  (b + "ssm_out.weight", ft(l, "w_out"), [v, H], y["w_out"]),
                  (b + "ssm_conv1d.weight", vec_type, [cfg.conv_kernel, c], vec(y["conv_w"])),
                  (b + "ssm_a", vec_type, [n], vec(y["a_log"])), (b + "ssm_dt.bias", vec_type, [n], vec(y["dt_bias"])),
                  (b + "ssm_norm.weight", vec_type, [128], vec(y["ssm_norm"]))]
    T = [(name, t, shape, np.ascontiguousarray(a).view(np.uint8).reshape(-1).tobytes()) for name, t, shape, a in T]
    for name, (t, data) in (override or {}).items():
        i = next(i for i, x in enumerate(T) if x[0] == name)
        T[i] = (name, t, T[i][2], data)
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
    _same_tensors(a, b, m, ids)
    la, lb = _decode(a), _decode(b)
    for sa, sb in zip(la, lb):
        for x, y in zip(sa, sb):
            assert np.array_equal(x, y)
    a.close()
    b.close()


def _same_tensors(a, b, m, ids):
    for l, y in enumerate(m["layers"]):
        for k, t in ids.items():
            if k in y:
                nb = np.asarray(y[k]).nbytes
                ga, gb = a.get_tensor(l, t, nb), b.get_tensor(l, t, nb)
                assert np.array_equal(ga, gb), (l, k)
                assert np.array_equal(ga, np.ascontiguousarray(y[k]).view(np.uint8).reshape(-1)), (l, k)
                if k.startswith("w_"):
                    assert a.get_format(l, t) == b.get_format(l, t), (l, k)


def _fp16_vectors(m):
    """m with every vector rounded to fp16 values (so an F16 file holds them exactly)."""
    r = lambda a: np.asarray(a, np.float32).astype(np.float16).astype(np.float32)  # noqa: E731
    out = dict(m, final_norm=r(m["final_norm"]), layers=[])
    for y in m["layers"]:
        out["layers"].append({k: (r(v) if k in VECTORS else v) for k, v in y.items()})
    return out


def test_gguf_mixed_formats_load_matches_upload_and_oracle(tmp_path, oc):
    """Q4_K and Q8_0 matrices, F16 embedding and F16 vectors: the loaded engine
    holds the same bytes and formats as the uploaded one, decodes bit-identical
    logits, and stays within 1e-3 of the oracle decoder on the same formats
    at every step (measured <= 2.4e-4)."""
    from echohip.engine import (T_A_LOG, T_ATTN_NORM, T_CONV_W, T_DT_BIAS, T_EMBED, T_FFN_NORM, T_FINAL_NORM, T_K_NORM,
                                T_LM_HEAD, T_Q_NORM, T_SSM_NORM, T_W_DOWN, T_W_GATE, T_W_IN, T_W_OUT, T_W_UP, Engine)
    from echohip.gguf import GGUF
    cfg = small_config(max_batch=3, max_ctx=32)
    m = _fp16_vectors(make_model(cfg, seed=13, fmts=MIXED_FMTS))
    f = tmp_path / "mixed.gguf"
    model_gguf(cfg, m, f, vec_type=F16)
    with GGUF(f) as g:
        a = Engine(g.engine_config(3, 32))
        g.load_into(a)
    b = Engine(cfg)
    upload(b, m)
    for t, arr in ((T_EMBED, m["embed"]), (T_FINAL_NORM, m["final_norm"]), (T_LM_HEAD, m["lm_head"])):
        nb = np.asarray(arr).nbytes
        assert np.array_equal(a.get_tensor(0, t, nb), b.get_tensor(0, t, nb))
        assert a.get_format(0, t) == b.get_format(0, t)
    ids = {"w_in": T_W_IN, "w_out": T_W_OUT, "w_gate": T_W_GATE, "w_up": T_W_UP, "w_down": T_W_DOWN,
           "attn_norm": T_ATTN_NORM, "ffn_norm": T_FFN_NORM, "q_norm": T_Q_NORM, "k_norm": T_K_NORM,
           "conv_w": T_CONV_W, "a_log": T_A_LOG, "dt_bias": T_DT_BIAS, "ssm_norm": T_SSM_NORM}
    _same_tensors(a, b, m, ids)
    la, lb = _decode(a), _decode(b)
    for sa, sb in zip(la, lb):
        for x, y in zip(sa, sb):
            assert np.array_equal(x, y)
    # sequence 0 of _decode against the oracle decoder (5, then greedy)
    dec = OracleDecoder(oc, cfg, m, n_seq=1, quant_act=2)  # the engine's two-piece activations
    tok, errs = 5, []
    for step in range(len(la)):
        ref = dec.token(0, tok)
        errs.append(rel_l2(la[step][0], ref))
        tok = int(np.argmax(la[step][0]))
    print("GGUF mixed model vs oracle, per-step logits rel_l2", " ".join(f"{e:.1e}" for e in errs))
    assert max(errs) < 1e-3
    a.close()
    b.close()


@pytest.mark.parametrize("case", ["gate_up_formats", "fused_formats", "q6_K"])
def test_gguf_rejects_unsupported_format_mixes(tmp_path, case):
    from echohip.engine import Engine
    from echohip.gguf import GGUF
    cfg = small_config(max_batch=1, max_ctx=16)
    m = make_model(cfg, seed=14, fmts={(1, "w_gate"): Q4K, (1, "w_up"): Q4K, (0, "w_in"): Q4K})
    H, F = cfg.hidden, cfg.ffn
    ov, match = {}, None
    if case == "gate_up_formats":   # gate Q4_K, up Q8_0 in block 1
        from echohip import synth
        ov["blk.1.ffn_up.weight"] = (Q8, synth.q8_0_blocks(1, F, H).tobytes())
        match = "one format"
    elif case == "fused_formats":   # block 0: attn_gate Q8_0 beside a Q4_K attn_qkv
        from echohip import synth
        ov["blk.0.attn_gate.weight"] = (Q8, synth.q8_0_blocks(2, cfg.ssm_inner, H).tobytes())
        match = "one format"
    else:                           # a Q6_K down projection (256 elements in 210 bytes)
        ov["blk.2.ffn_down.weight"] = (Q6K, bytes(H * F // 256 * 210))
        match = "must be Q8_0 or Q4_K"
    f = tmp_path / "bad.gguf"
    model_gguf(cfg, m, f, override=ov)
    with GGUF(f) as g:
        e = Engine(g.engine_config(1, 16))
        with pytest.raises(Exception, match=match):
            g.load_into(e)
        e.close()


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
