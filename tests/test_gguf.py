"""GGUF v3 reader (include/gguf_reader.h C++ interface, include/echo_gguf.h C ABI).

Known answers are the reference's own reader tests
(echo-core-zig/src/gguf/reader.zig:659-905): the synthetic llama file (alignment
64, data section = the last 128 bytes, tokens, scores, head_dim = hidden/heads)
and the synthetic qwen35 file (key_length overrides head_dim; a Q8_0
[2560, 8192] tensor is 22,282,240 bytes, as the reference's tensor report of
the 4B model lists for blk.0.attn_qkv.weight).  The files are written here by
tests/gguf_writer.py in the byte layout those tests build.  Malformed files
must fail with an error, never read out of bounds.
"""
import struct
import subprocess
from pathlib import Path

import numpy as np
import pytest

import gguf_writer as gw

ROOT = Path(__file__).resolve().parents[1]
LIBDIR = ROOT / "echo-core_amd"
pytestmark = pytest.mark.skipif(not (LIBDIR / "libechohip.so").exists(), reason="libechohip.so not built")


def llama_file():
    md = [("general.alignment", gw.U32, 64), ("llama.context_length", gw.U32, 128),
          ("llama.embedding_length", gw.U32, 8), ("llama.block_count", gw.U32, 1),
          ("llama.feed_forward_length", gw.U32, 16), ("llama.attention.head_count", gw.U32, 2),
          ("llama.attention.head_count_kv", gw.U32, 1),
          ("tokenizer.ggml.tokens", gw.ARRAY, (gw.STRING, ["hello", "world"])),
          ("tokenizer.ggml.scores", gw.ARRAY, (gw.F32, [1.25, -0.5]))]
    return gw.gguf_bytes(md, [("blk.0.attn_q.weight", 1, [8, 8], b"\xab" * 128)], alignment=64)


def qwen35_file():
    md = [("general.alignment", gw.U32, 32), ("qwen35.context_length", gw.U32, 262144),
          ("qwen35.embedding_length", gw.U32, 2560), ("qwen35.block_count", gw.U32, 32),
          ("qwen35.attention.head_count", gw.U32, 16), ("qwen35.attention.head_count_kv", gw.U32, 4),
          ("qwen35.attention.key_length", gw.U32, 256), ("qwen35.ssm.group_count", gw.U32, 16),
          ("tokenizer.ggml.tokens", gw.ARRAY, (gw.STRING, ["hello", "world"]))]
    return gw.gguf_bytes(md, [("blk.0.attn_qkv.weight", 6, [2560, 8192], b"\xcd" * 22282240)])


@pytest.fixture(scope="module")
def gguf_use(tmp_path_factory):
    d = tmp_path_factory.mktemp("gguf_use")
    exe = d / "gguf_use"
    subprocess.run(["g++", "-std=c++17", "-O1", "-I", str(ROOT / "include"), str(ROOT / "tests" / "abi" / "gguf_use.cpp"),
                    "-o", str(exe), "-L", str(LIBDIR), "-lechohip", "-Wl,-rpath," + str(LIBDIR),
                    "-Wl,--allow-shlib-undefined"], check=True)

    def run(path, *args):
        p = subprocess.run([str(exe), str(path), *args], capture_output=True, text=True)
        lines = p.stdout.splitlines()
        kv = {}
        for ln in lines:
            k, _, v = ln.partition(" ")
            kv.setdefault(k, []).append(v)
        return p.returncode, kv
    return run


def test_cpp_reader_llama_known_answers(tmp_path, gguf_use):
    data = llama_file()
    f = tmp_path / "sample.gguf"
    f.write_bytes(data)
    rc, kv = gguf_use(f, "attn_q.weight")
    assert rc == 0, kv
    assert kv["alignment"] == ["64"]
    assert kv["data_offset"] == [str(len(data) - 128)]
    assert kv["max_seq_len"] == ["128"] and kv["hidden_dim"] == ["8"] and kv["num_layers"] == ["1"]
    assert kv["num_heads"] == ["2"] and kv["num_kv_heads"] == ["1"] and kv["head_dim"] == ["4"]
    assert kv["ffn_hidden_dim"] == ["16"] and kv["gated_swiglu"] == ["1"] and kv["vocab_size"] == ["2"]
    assert kv["token"] == ["0 hello", "1 world"]
    assert kv["score"] == ["1.250000", "-0.500000"]
    assert kv["tensor"] == ["blk.0.attn_q.weight type 1 size 128 offset 0 first 171 last 171"]
    assert kv["suffix"] == ["attn_q.weight found"] and kv["aligned"] == ["1"]


def test_cpp_reader_qwen35_key_length(tmp_path, gguf_use):
    f = tmp_path / "qwen35.gguf"
    f.write_bytes(qwen35_file())
    rc, kv = gguf_use(f)
    assert rc == 0, kv
    assert kv["hidden_dim"] == ["2560"] and kv["num_heads"] == ["16"] and kv["num_kv_heads"] == ["4"]
    assert kv["head_dim"] == ["256"] and kv["max_seq_len"] == ["262144"]
    assert kv["tensor"] == ["blk.0.attn_qkv.weight type 6 size 22282240 offset 0 first 205 last 205"]


def test_c_abi_reader(tmp_path):
    from echohip.gguf import GGUF
    data = llama_file()
    f = tmp_path / "sample.gguf"
    f.write_bytes(data)
    with GGUF(f) as g:
        assert g.alignment == 64 and g.data_offset == len(data) - 128 and g.arch_prefix == "llama."
        assert g.get_uint("llama.block_count") == 1 and g.get_uint("general.alignment") == 64
        assert g.tokens() == ["hello", "world"]
        assert g.names() == ["blk.0.attn_q.weight"]
        t = g.tensor("blk.0.attn_q.weight")
        assert t["type"] == 1 and t["shape"] == [8, 8] and t["bytes"] == 128
        assert np.all(t["data"] == 0xAB)
        with pytest.raises(Exception, match="not found"):
            g.tensor("blk.0.attn_k.weight")
        with pytest.raises(Exception):
            g.get_uint("llama.rope.freq_base")


def _expect_error(gguf_use, path, fragment):
    rc, kv = gguf_use(path)
    assert rc == 1 and fragment in kv["error"][0], kv
    from echohip.gguf import GGUF
    with pytest.raises(Exception, match=fragment):
        GGUF(path)


def test_malformed_files_fail_cleanly(tmp_path, gguf_use):
    good = llama_file()
    cases = {
        "magic": (b"GGUX" + good[4:], "bad magic"),
        "version": (gw.gguf_bytes([], [], version=2), "unsupported version"),
        "truncated_meta": (good[:40], "truncated"),
        "truncated_data": (good[:-64], "past the end"),
        "huge_array": (b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + gw._str("a") + struct.pack("<IIQ", gw.ARRAY, gw.U32, 2**62),
                       "array length"),
        "bad_type": (gw.gguf_bytes([], [("t", 99, [4], b"\0" * 16)]), "unknown GGML type"),
        "partial_block": (gw.gguf_bytes([], [("t", 6, [40], b"\0" * 68)]), "whole number of blocks"),
    }
    for name, (data, frag) in cases.items():
        p = tmp_path / f"{name}.gguf"
        p.write_bytes(data)
        _expect_error(gguf_use, p, frag)


def hybrid_metadata(cfg, arch="qwen35"):
    return [("general.alignment", gw.U32, 32), (f"{arch}.context_length", gw.U32, 4096),
            (f"{arch}.embedding_length", gw.U32, cfg.hidden), (f"{arch}.block_count", gw.U32, cfg.n_layers),
            (f"{arch}.feed_forward_length", gw.U32, cfg.ffn), (f"{arch}.attention.head_count", gw.U32, cfg.n_heads),
            (f"{arch}.attention.head_count_kv", gw.U32, cfg.n_kv),
            (f"{arch}.attention.key_length", gw.U32, cfg.head_dim),
            (f"{arch}.ssm.inner_size", gw.U32, cfg.ssm_inner), (f"{arch}.ssm.time_step_rank", gw.U32, cfg.ssm_heads),
            (f"{arch}.ssm.conv_kernel", gw.U32, cfg.conv_kernel), (f"{arch}.ssm.group_count", gw.U32,
                                                                    cfg.ssm_heads // 2),
            (f"{arch}.full_attention_interval", gw.U32, cfg.attn_interval),
            (f"{arch}.rope.freq_base", gw.F32, cfg.rope_base)]


def test_engine_config_from_metadata(tmp_path):
    """ec_gguf_engine_config: shape from metadata, vocab from token_embd, block types checked."""
    from echohip.engine import EngineConfig
    from echohip.gguf import GGUF
    cfg = EngineConfig(vocab=320, hidden=256, ffn=512, n_layers=4, n_heads=4, n_kv=2, head_dim=256, ssm_inner=512,
                       ssm_heads=4, conv_kernel=4, attn_interval=4, max_batch=3, max_ctx=64, rope_base=5e5)
    emb = ("token_embd.weight", 6, [cfg.hidden, cfg.vocab], b"\0" * (cfg.vocab * cfg.hidden // 32 * 34))
    ssm = [(f"blk.{l}.ssm_out.weight", 6, [cfg.ssm_inner, cfg.hidden], b"\0" * (cfg.hidden * cfg.ssm_inner // 32 * 34))
           for l in range(3)]
    f = tmp_path / "h.gguf"
    gw.write(f, hybrid_metadata(cfg), [emb] + ssm)
    with GGUF(f) as g:
        assert g.engine_config(3, 64) == cfg
    # a delta-net block where the interval says attention
    bad = ssm + [("blk.3.ssm_out.weight", 6, [cfg.ssm_inner, cfg.hidden], ssm[0][3])]
    gw.write(f, hybrid_metadata(cfg), [emb] + bad)
    with GGUF(f) as g, pytest.raises(Exception, match="block 3 should be attention"):
        g.engine_config(3, 64)
