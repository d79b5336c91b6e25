"""GPU hybrid decoder (echo_engine.h) vs the oracle's token-by-token decoder.

Small config (hidden 256, 4 blocks: 3 delta-net + 1 attention, vocab 1000),
three sequences entering at different steps (ragged batch), prompt tokens
first, then each sequence's own greedy tokens.  The oracle quantizes matvec
inputs exactly as the GPU path does (quant_act=1), so the two agree to fp32
rounding (~1e-7 relative L2 of the logits) except where an activation lands on
an int8 rounding boundary: the GPU's reduction order (RMSNorm, matvec sums)
differs from the oracle's sequential sums by ~1e-6 relative, which can move one
element across a .5 boundary and change it by one quantum.  At hidden 256 one
such flip at the final norm shifts the logits by ~5e-3 relative L2 and leaves
the carried state untouched (the next step agrees to ~1e-7 again).  The checks:
  - most steps agree to 1e-5 (the exact-path case);
  - every step is within 2e-2 (a few single-quantum flips at most);
  - a step that differs is followed by agreeing steps (no state divergence);
  - greedy tokens agree wherever the oracle's top-2 margin is clear.
"""
import numpy as np
import pytest

from conftest import rel_l2
from decoder_util import OracleDecoder, make_model, small_config, upload

pytestmark = pytest.mark.gpu


def _run(oc, graph):
    from echohip.engine import Engine
    cfg = small_config(max_batch=3, max_ctx=64)
    m = make_model(cfg, seed=7)
    eng = Engine(cfg)
    upload(eng, m)
    eng.reset()
    ref = OracleDecoder(oc, cfg, m, n_seq=3)
    start = [0, 2, 4]
    prompt = [[11, 523, 7, 999], [42, 0, 17], [300, 301, 302, 303, 304]]
    nxt = [None, None, None]
    got, want, toks = [], [], []
    for step in range(12):
        tok = np.zeros(3, np.int32)
        pos = np.full(3, -1, np.int32)
        for s in range(3):
            i = step - start[s]
            if i < 0:
                continue
            tok[s] = prompt[s][i] if i < len(prompt[s]) else nxt[s]
            pos[s] = i
        eng.set_inputs(tok, pos)
        eng.step(graph=graph)
        gen, gpos = eng.tokens()
        for s in range(3):
            if pos[s] < 0:
                assert gpos[s] == -1
                continue
            assert gpos[s] == pos[s] + 1
            lg = eng.logits(s)
            lr = ref.token(s, int(tok[s]))
            got.append(lg)
            want.append(lr)
            toks.append((int(gen[s]), lr))
            nxt[s] = int(gen[s])
    eng.close()
    return got, want, toks


def test_decoder_matches_oracle(oc):
    got, want, toks = _run(oc, graph=False)
    errs = np.array([rel_l2(g, w) for g, w in zip(got, want)])
    print("per-step logits rel_l2:", " ".join(f"{e:.1e}" for e in errs))
    exact = errs < 1e-5
    assert exact.mean() >= 0.75, errs
    assert errs.max() < 2e-2, errs
    # no divergence: the last quarter of the run is dominated by exact steps again
    tail = exact[-len(exact) // 4:]
    assert tail.mean() >= 0.5, errs
    checked = 0
    for g_tok, lr in toks:
        top2 = np.sort(lr)[-2:]
        if top2[1] - top2[0] > 1e-2 * max(1.0, abs(top2[1])):
            assert g_tok == int(np.argmax(lr))
            checked += 1
    assert checked > len(toks) // 2


def test_decoder_graph_replay_matches_eager(oc):
    a, _, _ = _run(oc, graph=False)
    b, _, _ = _run(oc, graph=True)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)
