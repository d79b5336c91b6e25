"""Chunked prefill checked one operation at a time against the oracle
(tests/prefill_ops.py): every launch of ec_engine_prefill_traced is
recomputed from the GPU's own inputs -- embedding rows bit-exact, fp32 rows
within 1e-5 relative L2 per token, quantized activations and KV rows equal to
the reference quantizer except at rounding boundaries.

Small model (hidden 256, 3 delta-net + 1 attention blocks): a 40-token prompt
(the token-loop delta rule), a 600-token prompt (a 512-token chunk through the
chunked delta-net scan and causal chunk attention, then 88 tokens), and a
prompt continued at position 130; the same with Q4_K matrices and an F16
embedding; and the 4B-class shapes (hidden 2560, 32 blocks) for a 150-token
prompt on a subset of matrix rows."""
import numpy as np
import pytest

from decoder_util import MIXED_FMTS, make_model, small_config, upload
from prefill_ops import PrefillChecker

pytestmark = pytest.mark.gpu


def _run(oc, eng, cfg, m, seq, tokens, pos0, rows=None):
    chk = PrefillChecker(oc, eng, cfg, m, seq, tokens, pos0, rows_per_matrix=rows, seed=seq)
    print(f"prefill seq {seq}: {len(tokens)} tokens at {pos0}", flush=True)
    eng.prefill_traced(seq, tokens, pos0, chk)
    print(chk.summary(), flush=True)
    return chk


@pytest.mark.parametrize("fmts", [None, MIXED_FMTS], ids=["q8_0", "mixed"])
def test_prefill_every_op_matches_oracle(oc, fmts):
    from echohip.engine import OP_PF_ATTN, OP_PF_DELTA, OP_PF_HEAD, Engine
    cfg = small_config(max_batch=3, max_ctx=640)
    m = make_model(cfg, seed=41, fmts=fmts)
    eng = Engine(cfg)
    upload(eng, m)
    eng.reset()
    rng = np.random.default_rng(5)
    cases = [(0, rng.integers(0, cfg.vocab, 40), 0), (1, rng.integers(0, cfg.vocab, 600), 0),
             (2, rng.integers(0, cfg.vocab, 130), 0), (2, rng.integers(0, cfg.vocab, 70), 130)]
    for seq, toks, pos0 in cases:
        chk = _run(oc, eng, cfg, m, seq, toks.astype(np.int32), pos0)
        assert chk.counts.get(OP_PF_DELTA, 0) > 0 and chk.counts.get(OP_PF_ATTN, 0) > 0
        assert chk.counts.get(OP_PF_HEAD, 0) > 0
        gen, pos = eng.tokens()
        assert pos[seq] == pos0 + len(toks)
    eng.close()


def test_prefill_4b_shapes_every_op_matches_oracle(oc):
    """The benchmark's 4B-class decoder (seeded device weights): a 150-token
    prompt, every launch checked (matrices on 256 random rows each)."""
    from echohip.engine import Engine, EngineConfig
    cfg = EngineConfig(max_batch=1, max_ctx=256)
    eng = Engine(cfg)
    eng.init_random(seed=3)
    eng.reset()
    m = eng.export_model()
    toks = np.random.default_rng(6).integers(0, cfg.vocab, 150).astype(np.int32)
    _run(oc, eng, cfg, m, 0, toks, 0, rows=256)
    eng.close()
