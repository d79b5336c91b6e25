"""Pin the oracle's hybrid decoder (oc_decoder_token) on the CPU.

The decoder composes ops pinned individually in test_oracle_path.py; these
checks pin the composition: the residual wiring, the embedding/final-norm/head
path, the per-layer KV and recurrent state and the activation quantization
switch.
"""
import numpy as np

from conftest import rel_l2
from decoder_util import OracleDecoder, make_model, small_config


def _deq_rows(blocks, rows, K):
    b = blocks.reshape(rows, K // 32, 34)
    d = b[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
    q = b[:, :, 2:].view(np.int8).astype(np.float64)
    return (q * d[..., None]).reshape(rows, K)


def test_zero_blocks_reduce_to_embedding_head(oc):
    """With every block's output projection zero, each block adds nothing to
    the residual (engine.zig:421-462), so logits = head . rmsnorm(embed row)."""
    cfg = small_config()
    m = make_model(cfg, seed=3)
    for y in m["layers"]:
        y["w_out"] = np.zeros_like(y["w_out"])
        y["w_down"] = np.zeros_like(y["w_down"])
    dec = OracleDecoder(oc, cfg, m, n_seq=1, quant_act=False)
    for tok in (5, 999, 0):
        lg = dec.token(0, tok)
        x = _deq_rows(m["embed"], cfg.vocab, cfg.hidden)[tok]
        h = x / np.sqrt(np.mean(x * x) + 1e-6) * m["final_norm"]
        ref = _deq_rows(m["lm_head"], cfg.vocab, cfg.hidden) @ h
        assert rel_l2(lg, ref) < 1e-5


def test_state_carries_across_tokens(oc):
    """The second token's logits depend on the first (recurrent state, KV), and
    a fresh decoder reproduces the same sequence exactly."""
    cfg = small_config()
    m = make_model(cfg, seed=4)
    a = OracleDecoder(oc, cfg, m, n_seq=2, quant_act=True)
    l1 = a.token(0, 10)
    l2 = a.token(0, 10)
    assert rel_l2(l1, l2) > 1e-3
    l1b = a.token(1, 10)
    assert np.array_equal(l1, l1b)
    assert a.pos(0) == 2 and a.pos(1) == 1


def test_activation_quantization_is_small_perturbation(oc):
    cfg = small_config()
    m = make_model(cfg, seed=5)
    q = OracleDecoder(oc, cfg, m, n_seq=1, quant_act=True)
    f = OracleDecoder(oc, cfg, m, n_seq=1, quant_act=False)
    for tok in (1, 2, 3):
        assert rel_l2(q.token(0, tok), f.token(0, tok)) < 0.1
