"""The benchmark's own scale checked against the oracle, one operation at a
time (tests/decoder_ops.py, tests/prefill_ops.py tolerances), on the 4B-class
decoder with the benchmark's weights (ec_engine_init_random seed 0):

* a 600-token prompt through the traced chunked prefill: one full 512-token
  chunk (chunked delta scan, causal chunk attention, 512-row GEMMs), then an
  88-token chunk continuing it;
* a ragged batch of 8 sequences at contexts of 300 .. 3105 positions (the
  benchmark draws 1536 .. 3105), prefilled by the engine's two-lane batch
  prefill, then two traced decode steps with every launch checked: attention
  over the whole cache of each sequence, the delta-net state of every
  sequence, the matvecs with two-piece activations (on a subset of rows).
"""
import numpy as np
import pytest

from decoder_ops import OpChecker
from prefill_ops import PrefillChecker

pytestmark = pytest.mark.gpu

ROWS = 192  # matrix rows recomputed per launch


def test_bench_scale_prefill_600_tokens(oc):
    from echohip.engine import OP_PF_ATTN, OP_PF_DELTA, OP_PF_HEAD, Engine, EngineConfig
    cfg = EngineConfig(max_batch=1, max_ctx=640)
    eng = Engine(cfg)
    eng.init_random(seed=0)
    eng.reset()
    m = eng.export_model()
    toks = np.random.default_rng(11).integers(0, cfg.vocab, 600).astype(np.int32)
    chk = PrefillChecker(oc, eng, cfg, m, 0, toks, 0, rows_per_matrix=ROWS, seed=2)
    print("prefill 600 tokens (512 + 88)", flush=True)
    eng.prefill_traced(0, toks, 0, chk)
    print(chk.summary(), flush=True)
    # every token's delta-rule output and the state after each chunk, 24 delta-net blocks
    assert chk.counts.get(OP_PF_DELTA, 0) == 24 * (512 + 1 + 88 + 1) and chk.counts.get(OP_PF_ATTN, 0) > 0
    assert chk.counts.get(OP_PF_HEAD, 0) > 0
    assert eng.tokens()[1][0] == 600
    eng.close()


def test_bench_scale_decode_batch8_ragged(oc):
    from echohip.engine import OP_ATTN, OP_DELTA_STEP, Engine, EngineConfig
    lens = [300, 3105, 1536, 2200, 700, 2900, 1800, 2600]
    cfg = EngineConfig(max_batch=8, max_ctx=max(lens) + 4)
    eng = Engine(cfg)
    eng.init_random(seed=0)
    eng.reset()
    m = eng.export_model()
    rng = np.random.default_rng(12)
    prompts = [rng.integers(0, cfg.vocab, n).astype(np.int32) for n in lens]
    print(f"prefill batch of 8: {lens}", flush=True)
    eng.prefill_batch([(s, prompts[s], 0) for s in range(8)])
    gen, pos = eng.tokens()
    assert pos.tolist() == lens
    chk = OpChecker(oc, eng, cfg, m, rows_per_matrix=ROWS, seed=3)
    tok = gen.copy()
    for step in range(2):
        print(f"decode step {step} at contexts {[n + step + 1 for n in lens]}", flush=True)
        eng.set_inputs(tok, np.array(lens, np.int32) + step)
        eng.step_traced(chk)
        tok, _ = eng.tokens()
    print(chk.summary(), flush=True)
    assert chk.counts.get(OP_ATTN, 0) == 2 * 8 * 8 * 2  # output and activation, 8 layers, 8 sequences, 2 steps
    assert chk.counts.get(OP_DELTA_STEP, 0) >= 2 * 24 * 8
    eng.close()
