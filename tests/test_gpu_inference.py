"""InferenceEngine (include/inference.h, the reference's engine interface) over the device engine.

A C++ program built with g++ against include/inference.h and
include/gguf_reader.h loads the small hybrid model from a GGUF file and feeds
a prompt token by token (the reference's calling pattern) or in one call; the
logits must equal, bit for bit, the device engine driven directly (graph
decode steps / chunked prefill), which test_gpu_decoder and test_gpu_prefill
tie to the oracle.  The all-attention model (the reference C++ engine's shape:
no delta-net blocks) is checked launch by launch against the oracle.
"""
import subprocess
from pathlib import Path

import numpy as np
import pytest

from decoder_util import make_model, small_config, upload

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
    """attn_interval 1, no delta-net (the reference C++ engine's shape): every launch of six decode steps checked
    against the oracle on the GPU's own inputs (tests/decoder_ops.py)."""
    import dataclasses
    from decoder_ops import OpChecker
    from echohip.engine import Engine
    cfg = dataclasses.replace(small_config(max_batch=2, max_ctx=32), attn_interval=1, ssm_inner=0, ssm_heads=0)
    m = make_model(cfg, seed=33)
    eng = Engine(cfg)
    upload(eng, m)
    eng.reset()
    chk = OpChecker(oc, eng, cfg, m)
    toks = [[5, 17, 900, 3, 44, 61], [800, 2, 2, 71, 9, 333]]
    for step in range(6):
        eng.set_inputs(np.array([toks[0][step], toks[1][step]], np.int32), np.array([step, step], np.int32))
        eng.step_traced(chk)
    print(chk.summary())
    assert chk.counts.get(6, 0) == 2 * 6 * 2 * cfg.n_layers  # output and activation of every attention launch
    eng.close()


def test_engine_at_bench_shapes_uploads_rope_frequencies():
    """The engine's set-up copies (RoPE inverse frequencies, positions) are ordered after the zeroing of its
    buffers on the engine stream, also when gigabytes of memsets are queued ahead (4B-class shapes, batch 8)."""
    from echohip.engine import B_INV_FREQ, B_POS, Engine, EngineConfig
    cfg = EngineConfig(max_batch=8, max_ctx=4608)
    eng = Engine(cfg)
    inv = eng.read_buffer(B_INV_FREQ, np.float32)
    i = np.arange(0, cfg.head_dim, 2, dtype=np.float64)
    assert np.allclose(inv, 1.0 / cfg.rope_base ** (i / cfg.head_dim), rtol=1e-6, atol=0)
    assert np.array_equal(eng.read_buffer(B_POS, np.int32), np.full(8, -1, np.int32))
    eng.close()
