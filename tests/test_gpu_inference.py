"""InferenceEngine (include/inference.h, the reference's engine interface) over the device engine.

A C++ program built with g++ against include/inference.h and
include/gguf_reader.h loads the small hybrid model from a GGUF file and feeds
a prompt token by token (the reference's calling pattern) or in one call; the
logits must equal, bit for bit, the device engine driven directly (graph
decode steps / chunked prefill), which test_gpu_decoder and test_gpu_prefill
tie to the oracle.  The all-attention model (the reference C++ engine's shape:
no delta-net blocks) is checked stepwise against the oracle decoder.
"""
import subprocess
from pathlib import Path

import numpy as np
import pytest

from conftest import rel_l2
from decoder_util import OracleDecoder, make_model, small_config, upload

pytestmark = pytest.mark.gpu
ROOT = Path(__file__).resolve().parents[1]
LIBDIR = ROOT / "echo-core_amd"


@pytest.fixture(scope="module")
def inference_use(tmp_path_factory):
    exe = tmp_path_factory.mktemp("inf") / "inference_use"
    subprocess.run(["g++", "-std=c++17", "-O1", "-I", str(ROOT / "include"),
                    str(ROOT / "tests" / "abi" / "inference_use.cpp"), "-o", str(exe), "-L", str(LIBDIR), "-lechohip",
                    "-Wl,-rpath," + str(LIBDIR), "-Wl,--allow-shlib-undefined"], check=True)
    return exe


@pytest.mark.parametrize("mode", ["loop", "once"])
def test_cpp_inference_engine_matches_device_engine(tmp_path, inference_use, mode):
    import dataclasses
    from echohip.engine import Engine
    from test_gpu_gguf import model_gguf
    cfg = small_config(max_batch=3, max_ctx=32)
    m = make_model(cfg, seed=31)
    f = tmp_path / "m.gguf"
    model_gguf(cfg, m, f)
    prompt = [7, 400, 13, 999, 250, 4, 61]
    out = tmp_path / "logits.bin"
    p = subprocess.run([str(inference_use), str(f), mode, str(out)] + [str(t) for t in prompt],
                       capture_output=True, text=True)
    assert p.returncode == 0, p.stdout + p.stderr
    assert f"seen {len(prompt)}" in p.stdout and "after_reset 0" in p.stdout
    got = np.fromfile(out, np.float32)
    e = Engine(dataclasses.replace(cfg, max_batch=1, max_ctx=64))
    upload(e, m)
    e.reset()
    if mode == "loop":
        for i, t in enumerate(prompt):
            e.set_inputs(np.array([t], np.int32), np.array([i], np.int32))
            e.step(graph=True)
    else:
        e.prefill(0, prompt, 0)
    want = e.logits(0)
    e.close()
    assert np.array_equal(got, want)


def test_attention_only_model_matches_oracle(oc):
    """attn_interval 1, no delta-net: device engine vs the oracle decoder, state-synced per step."""
    import dataclasses
    from echohip.engine import S_KEYS, S_KSCALES, S_VALS, S_VSCALES, Engine
    cfg = dataclasses.replace(small_config(max_batch=2, max_ctx=32), attn_interval=1, ssm_inner=0, ssm_heads=0)
    m = make_model(cfg, seed=33)
    eng = Engine(cfg)
    upload(eng, m)
    eng.reset()
    ref = OracleDecoder(oc, cfg, m, n_seq=2)
    kinds = {"k": S_KEYS, "v": S_VALS, "ks": S_KSCALES, "vs": S_VSCALES}
    toks = [[5, 17, 900, 3, 44, 61], [800, 2, 2, 71, 9, 333]]
    errs = []
    for step in range(6):
        tok = np.array([toks[0][step], toks[1][step]], np.int32)
        pos = np.array([step, step], np.int32)
        for s in range(2):
            ref.load_state(s, step, lambda l, kind, s=s: eng.get_state(l, kinds[kind], s))
        eng.set_inputs(tok, pos)
        eng.step(graph=False)
        for s in range(2):
            errs.append(rel_l2(eng.logits(s), ref.token(s, int(tok[s]))))
    errs = np.array(errs)
    print("per-step logits rel_l2:", " ".join(f"{x:.1e}" for x in errs))
    assert (errs < 1e-5).mean() >= 0.75, errs
    assert errs.max() < 5e-2, errs
    eng.close()
