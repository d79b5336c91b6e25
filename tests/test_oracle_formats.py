"""Pin the oracle's per-tensor storage formats (oracle.c oc_embed_row,
oc_matvec_act and the decoder's format table), the dispatch the reference's
InferenceEngine::matvec_d makes per weight (src/inference.cpp:526-545).

A Q4_K block whose eight sub-blocks all have scale 4 and min 32 with dmin = d
holds the values 4d*(q - 8), q in 0..15: exactly the Q8_0 values of d8 = 4d,
qs = q - 8.  Such a pair is built here from the GGUF byte layouts themselves
(Q4_K: byte 32j + t of a super-block holds position 64j + t in its low nibble
and 64j + 32 + t in its high nibble), so the two formats' matvecs agree up to
fp32 summation order, and a decoder with a different subset of matrices
re-encoded this way in each block computes the same logits as the Q8_0 model.  An F32 embedding holding the
dequantized Q8_0 rows (d*q is exact in fp32) gives bit-identical logits.  A
wrong format index in the decoder's table, a wrong row size for the fused
input projection's slices or an embedding read in the wrong format fails.
"""
import numpy as np
import pytest

from conftest import rel_l2
from decoder_util import OracleDecoder, make_model, small_config
from echohip import synth
from echohip.engine import F16, F32, Q4_K, Q8_0


def q4k_q8_pair(seed, N, K, d_std=1e-3):
    """(Q4_K bytes, Q8_0 bytes) of the same [N][K] matrix 4d*(q - 8)."""
    assert K % 256 == 0
    nb = K // 256
    lev = synth.randint(synth.stream_seed(seed, 0), N * K, 0, 15).reshape(N, nb, 256)
    d = (np.abs(synth.normal(synth.stream_seed(seed, 1), N * nb)) * d_std + 1e-4).astype(np.float16)
    d = d.reshape(N, nb)
    q4 = np.zeros((N, nb, 144), np.uint8)
    q4[:, :, 0:2] = d.view(np.uint8).reshape(N, nb, 2)
    q4[:, :, 2:4] = d.view(np.uint8).reshape(N, nb, 2)  # dmin = d
    q4[:, :, 4:16] = synth.pack_q4k_scales(np.full((N, nb, 8), 4), np.full((N, nb, 8), 32))
    for j in range(4):
        lo = lev[:, :, 64 * j:64 * j + 32]
        hi = lev[:, :, 64 * j + 32:64 * j + 64]
        q4[:, :, 16 + 32 * j:16 + 32 * j + 32] = (lo | (hi << 4)).astype(np.uint8)
    qs = (lev.reshape(N, K // 32, 32) - 8).astype(np.int8)
    d8 = np.repeat((4 * d.astype(np.float32)).astype(np.float16), 8, axis=1)
    return q4.reshape(N, nb * 144), synth.q8_0_from_parts(qs, d8)


def dequant_q8_0_rows(W, K):
    """fp32 rows of GGUF Q8_0 bytes (d*q is exact in fp32)."""
    b = np.asarray(W).reshape(-1, K // 32, 34)
    d = b[:, :, 0:2].copy().view(np.float16).astype(np.float32)
    q = b[:, :, 2:].view(np.int8).astype(np.float32)
    return (q * d).reshape(-1, K)


def test_reencoded_q4_K_matches_q8_0(oc):
    W4, W8 = q4k_q8_pair(1, 40, 512)
    x = synth.activations(2, 512)
    a, b = oc.matvec_q4_K(W4, x), oc.matvec_q8_0(W8, x)
    assert rel_l2(a, b) < 1e-6
    assert not np.array_equal(a, oc.matvec_q4_K(W4, np.roll(x, 32)))  # the position layout matters


def test_matvec_act_dispatch(oc):
    W4 = synth.q4_K_blocks(3, 24, 512, 1e-3)
    W8 = synth.q8_0_blocks(4, 24, 512)
    x = synth.activations(5, 512)
    assert np.array_equal(oc.matvec_act(Q4_K, W4, x, quant_act=False), oc.matvec_q4_K(W4, x))
    rq, rd, _ = oc.quantize_act_q4_K(x)
    assert np.array_equal(oc.matvec_act(Q4_K, W4, x), oc.matvec_q4_K(W4, oc.dequant_act_q4_K(rq, rd)))
    assert np.array_equal(oc.matvec_act(Q8_0, W8, x), oc.matvec_act_q8_0(W8, x))
    assert np.array_equal(oc.matvec_act(Q8_0, W8, x, quant_act=False), oc.matvec_q8_0(W8, x))


def test_embed_row_formats(oc):
    H, V = 256, 12
    E8 = synth.q8_0_blocks(6, V, H)
    E16 = (0.1 * synth.normal(7, V * H)).astype(np.float16)
    E32 = synth.normal(8, V * H).astype(np.float32)
    for t in (0, 5, V - 1):
        assert np.array_equal(oc.embed_row(Q8_0, E8, H, t), oc.embed_row_q8_0(E8, H, t))
        assert np.array_equal(oc.embed_row(Q8_0, E8, H, t), dequant_q8_0_rows(E8, H)[t])
        assert np.array_equal(oc.embed_row(F16, E16, H, t), E16[t * H:(t + 1) * H].astype(np.float32))
        assert np.array_equal(oc.embed_row(F32, E32, H, t), E32[t * H:(t + 1) * H])


def _logits(oc, cfg, m, toks, quant_act):
    dec = OracleDecoder(oc, cfg, m, n_seq=1, quant_act=quant_act)
    return [dec.token(0, t) for t in toks]


@pytest.mark.parametrize("quant_act", [False, True])
def test_decoder_f32_embedding_equals_q8_0(oc, quant_act):
    cfg = small_config(max_batch=1, max_ctx=8)
    m8 = make_model(cfg, seed=21)
    m32 = dict(m8, embed=dequant_q8_0_rows(m8["embed"], cfg.hidden).reshape(-1), fmt={(-1, "embed"): F32})
    toks = [3, 999, 0, 41]
    for a, b in zip(_logits(oc, cfg, m8, toks, quant_act), _logits(oc, cfg, m32, toks, quant_act)):
        assert np.array_equal(a, b)


# matrices stored as Q4_K per layer of the small model (three delta-net
# blocks, then attention): each layer a different subset, so that a format
# read for the wrong matrix fails
Q4_SUBSETS = [("w_in", "w_down"), ("w_out", "w_gate", "w_up"), ("w_in", "w_out"), ("w_gate", "w_up", "w_down")]


def test_decoder_reencoded_q4_K_matrices_match_q8_0(oc):
    """A subset of the small hybrid model's matrices stored both ways (fp32
    activations: the two formats then differ only in summation order)."""
    cfg = small_config(max_batch=1, max_ctx=8)
    m8 = make_model(cfg, seed=22)
    m4 = {k: v for k, v in m8.items() if k != "layers"}
    m4["layers"], fmts = [], {}
    seed = iter(range(100, 1000))
    H, F = cfg.hidden, cfg.ffn
    for l, y in enumerate(m8["layers"]):
        nin = cfg.nin_attn if y["attn"] else cfg.nin_delta
        kout = cfg.n_heads * cfg.head_dim if y["attn"] else cfg.ssm_inner
        y8, y4 = dict(y), dict(y)
        for name, N, K in (("w_in", nin, H), ("w_out", H, kout), ("w_gate", F, H), ("w_up", F, H),
                           ("w_down", H, F)):
            y4[name], y8[name] = q4k_q8_pair(next(seed), N, K)
            if name in Q4_SUBSETS[l]:
                fmts[(l, name)] = Q4_K
            else:
                y4[name] = y8[name]
        m8["layers"][l] = y8
        m4["layers"].append(y4)
    m4["lm_head"], m8["lm_head"] = q4k_q8_pair(next(seed), cfg.vocab, H)
    fmts[(-1, "lm_head")] = Q4_K
    m4["fmt"] = fmts
    toks = [3, 999, 0, 41]
    for a, b in zip(_logits(oc, cfg, m8, toks, False), _logits(oc, cfg, m4, toks, False)):
        assert rel_l2(a, b) < 1e-4
