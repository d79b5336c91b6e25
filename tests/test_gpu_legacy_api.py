"""The reference-signature C++ interface of libechohip.so (include/kernels/*.h,
include/kv_cache.h), called by its mangled names the way a program built
against the reference's headers links to it, with host (numpy) buffers --
staged through the device by the library -- and with device tensors.

Expected values are the reference's own outputs (tests/golden/*.npz, written
by tests/golden/gen_golden.py from the reference's compiled kernels) or closed
forms stated per test.  Tolerances: int8 and fp16 outputs bit-exact;
fp32 sums within 1e-5 relative (the GPU's summation order differs from the
reference's by fp32 rounding).
"""
import numpy as np
import pytest

from conftest import rel_l2
from test_gpu_kernels import dev, empty, host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lgold():
    from pathlib import Path
    return np.load(Path(__file__).resolve().parent / "golden" / "legacy_golden.npz")


@pytest.fixture(scope="module")
def lg(hip):
    from echohip.legacy import Legacy
    return Legacy()


@pytest.mark.parametrize("width", [4, 8, 12, 16, 32, 37, 256, 1024])
@pytest.mark.parametrize("on_device", [False, True])
def test_quantize_per_token_symmetric(lg, golden, width, on_device):
    import torch
    x = golden[f"quant_w{width}_x"]
    rows = x.size // width
    if on_device:
        q, s = empty(x.size, torch.int8), empty(rows, torch.float32)
        lg.quantize_per_token_symmetric(dev(x), q, s, rows, width)
        q, s = host(q), host(s)
    else:
        q, s = np.zeros(x.size, np.int8), np.zeros(rows, np.float32)
        lg.quantize_per_token_symmetric(x, q, s, rows, width)
    assert np.array_equal(q, golden[f"quant_w{width}_q"])
    assert np.array_equal(s.view(np.uint32), golden[f"quant_w{width}_s"].view(np.uint32))


def test_quantize_ties_and_zero(lg, golden):
    x = golden["quant_ties_x"]
    q, s = np.zeros(x.size, np.int8), np.zeros(1, np.float32)
    lg.quantize_per_token_symmetric(x, q, s, 1, x.size)
    assert np.array_equal(q, golden["quant_ties_q"]) and s[0] == golden["quant_ties_s"][0]
    z = np.zeros(32, np.float32)
    q, s = np.ones(32, np.int8), np.zeros(1, np.float32)
    lg.quantize_per_token_symmetric(z, q, s, 1, 32)
    assert np.array_equal(q, golden["quant_zero_q"]) and s[0] == golden["quant_zero_s"][0] == 1.0


def test_fused_dequant_dot_int8(lg, golden):
    out = np.zeros(64, np.float32)
    lg.fused_dequant_dot_int8(golden["int8dot_q"], golden["int8dot_k"], golden["int8dot_s"], out, 256, 64)
    ref = golden["int8dot_out"]
    assert np.max(np.abs(out - ref)) < 1e-5 * np.max(np.abs(ref))


@pytest.mark.parametrize("fmt,blk", [("q8_0", 32), ("q4_K", 256)])
def test_fused_dequant_dot_rows(lg, golden, fmt, blk):
    key = fmt[:2]
    W, x = golden[f"{key}_W"], golden["mv_x"]
    got = np.array([lg.fused_dequant_dot_q8_0(np.ascontiguousarray(W[r]), 512 // blk, x) if fmt == "q8_0" else
                    lg.fused_dequant_dot_q4_K(np.ascontiguousarray(W[r]), 512 // blk, x) for r in range(W.shape[0])],
                   np.float32)
    ref = golden[f"{key}_fused"]
    assert np.max(np.abs(got - ref)) < 1e-5 * np.max(np.abs(ref))


@pytest.mark.parametrize("fmt", ["q8_0", "q4_K"])
@pytest.mark.parametrize("on_device", [False, True])
def test_matvec_accumulates(lg, golden, fmt, on_device):
    key = fmt[:2]
    W, x, y0 = golden[f"{key}_W"], golden["mv_x"], golden["mv_y0"]
    if on_device:
        y = dev(y0)
        lg.matvec(fmt, dev(W), dev(x), y, W.shape[0], 512)
        y = host(y)
    else:
        y = y0.copy()
        lg.matvec(fmt, W, x, y, W.shape[0], 512)
    assert rel_l2(y, golden[f"{key}_matvec"]) < 1e-5


def test_matvec_drops_partial_block(lg, golden):
    """K = 512 + 31: the reference reads K/32 whole blocks per row (matvec.cpp:65)."""
    W, x, y0 = golden["q8_W"], golden["mv_x"], golden["mv_y0"]
    xx = np.concatenate([x, np.full(31, 1e3, np.float32)])
    y = y0.copy()
    lg.matvec("q8_0", W, xx, y, W.shape[0], 512 + 31)
    assert rel_l2(y, golden["q8_matvec"]) < 1e-5


def test_q4_K_layout_probe(lg, golden):
    """One non-zero nibble per row at every position: pins the reference's nibble order."""
    W, x = golden["q4_probe_W"], golden["q4_probe_x"]
    y = np.zeros(W.shape[0], np.float32)
    lg.matvec("q4_K", W, x, y, W.shape[0], 256)
    assert rel_l2(y, golden["q4_probe_y"]) < 1e-6


def test_dequantize_to_fp16(lg, golden):
    """Q8_0: d*q rounded to fp16 (exact closed form).  Q4_K: the fp16 weights,
    used in an fp32 matvec on the host, reproduce the reference's matvec to
    fp16 weight rounding (< 1e-3)."""
    W = golden["q8_W"]
    out = np.zeros(W.shape[0] * 512, np.uint16)
    lg.dequantize_to_fp16("q8_0", W, out, out.size)
    blk = W.reshape(-1, 34)
    ref = (blk[:, 0:2].copy().view(np.float16).astype(np.float32) * blk[:, 2:].view(np.int8)).astype(np.float16)
    assert np.array_equal(out, ref.reshape(-1).view(np.uint16))
    W4 = golden["q4_W"]
    out = np.zeros(W4.shape[0] * 512, np.uint16)
    lg.dequantize_to_fp16("q4_K", W4, out, out.size)
    Wf = out.view(np.float16).astype(np.float64).reshape(W4.shape[0], 512)
    y = golden["mv_y0"] + Wf @ golden["mv_x"].astype(np.float64)
    assert rel_l2(y, golden["q4_matvec"]) < 1e-3


def test_q2_K_dequant_matches_matvec(lg):
    """Q2_K has no reference fixture: the fp16 dequantization and the fp32
    matvec are separate kernels; W_fp16 . x must equal matvec_q2_K within fp16
    weight rounding.  Block layout as the reference reads it
    (src/kernels/matvec.cpp:158-162): fp16 d, fp16 dmin, 16 scale bytes, 64
    bytes of 2-bit weights."""
    rng = np.random.default_rng(3)
    M, K = 48, 512
    nb = K // 256
    blocks = rng.integers(0, 256, (M, nb, 84), dtype=np.uint8)
    d = (np.abs(rng.standard_normal((M, nb, 2))) * 0.01).astype(np.float16)
    blocks[:, :, 0:4] = d.view(np.uint8).reshape(M, nb, 4)
    W = np.ascontiguousarray(blocks.reshape(M, nb * 84))
    x = rng.standard_normal(K).astype(np.float32)
    y = np.zeros(M, np.float32)
    lg.matvec("q2_K", W, x, y, M, K)
    out = np.zeros(M * K, np.uint16)
    lg.dequantize_to_fp16("q2_K", W, out, out.size)
    yr = out.view(np.float16).astype(np.float64).reshape(M, K) @ x.astype(np.float64)
    assert rel_l2(y, yr) < 2e-3


@pytest.mark.parametrize("which", ["<1024,512>", "<2048,1024>", "dispatch"])
def test_matvec_fp16(lg, which):
    from echohip.legacy import ModelConfig
    rng = np.random.default_rng(4)
    M, K = 300, 1000
    W = (rng.standard_normal((M, K)) * 0.05).astype(np.float16)
    x = rng.standard_normal(K).astype(np.float32)
    y0 = rng.standard_normal(M).astype(np.float32)
    y = y0.copy()
    Wb = np.ascontiguousarray(W.view(np.uint16))
    if which == "dispatch":
        lg.matvec_dispatch(Wb, x, y, M, K, ModelConfig(hidden_dim=K))
    else:
        t = tuple(int(v) for v in which.strip("<>").split(","))
        lg.matvec_fp16_fp32(t, Wb, x, y, M, K)
    ref = y0 + W.astype(np.float64) @ x.astype(np.float64)
    assert rel_l2(y, ref) < 1e-6


def test_kv_cache_class(lg, oc):
    """KVCache::append quantizes each (token, kv_head) row like the oracle's
    append (bit-exact int8 and scales); seq_len / reset follow the reference;
    an append past max_seq_len is rejected with an error."""
    from echohip.legacy import KVCache, ModelConfig
    from echohip.lib import EchoHipError
    n_kv, hd, max_seq = 4, 256, 6
    cfg = ModelConfig(num_layers=2, num_kv_heads=n_kv, head_dim=hd, max_seq_len=max_seq, num_heads=16,
                      use_kv_quantization=True)
    kv = KVCache(lg, cfg)
    rng = np.random.default_rng(6)
    keys = np.zeros(max_seq * n_kv * hd, np.int8)
    vals = np.zeros_like(keys)
    ks = np.zeros(max_seq * n_kv, np.float32)
    vs = np.zeros_like(ks)
    for p in range(3):
        k = rng.standard_normal(n_kv * hd).astype(np.float32)
        v = rng.standard_normal(n_kv * hd).astype(np.float32)
        kv.append(0, k, v) if p % 2 == 0 else kv.append(0, dev(k), dev(v))
        oc.kv_append(k, v, keys, vals, ks, vs, p, n_kv, hd)
    kv.append(1, k, v)
    assert kv.seq_len() == 3 and kv.layer(1).seq_len == 1
    y = kv.layer(0)
    got = {n: np.zeros_like(a) for n, a in (("k", keys), ("v", vals), ("ks", ks), ("vs", vs))}
    lg.hip.copy(got["k"], y.keys_int8, keys.nbytes)
    lg.hip.copy(got["v"], y.values_int8, vals.nbytes)
    lg.hip.copy(got["ks"], y.key_scales, ks.nbytes)
    lg.hip.copy(got["vs"], y.val_scales, vs.nbytes)
    assert np.array_equal(got["k"], keys) and np.array_equal(got["v"], vals)
    assert np.array_equal(got["ks"].view(np.uint32), ks.view(np.uint32))
    assert np.array_equal(got["vs"].view(np.uint32), vs.view(np.uint32))
    for _ in range(3):
        kv.append(0, k, v)
    with pytest.raises(EchoHipError):
        kv.append(0, k, v)
    assert kv.seq_len() == max_seq
    kv.reset()
    assert kv.seq_len() == 0 and kv.layer(1).seq_len == 0
    kv.close()


def test_kv_cache_fp32_mode(lg):
    from echohip.legacy import KVCache, ModelConfig
    n_kv, hd = 2, 64
    cfg = ModelConfig(num_layers=1, num_kv_heads=n_kv, head_dim=hd, max_seq_len=4, use_kv_quantization=False)
    kv = KVCache(lg, cfg)
    k = np.arange(n_kv * hd, dtype=np.float32)
    v = -k
    kv.append(0, k, v)
    kv.append(0, v, k)
    y = kv.layer(0)
    assert not y.keys_int8 and y.keys_fp32
    got = np.zeros(2 * n_kv * hd, np.float32)
    lg.hip.copy(got, y.keys_fp32, got.nbytes)
    assert np.array_equal(got, np.concatenate([k, v]))
    kv.close()


def test_q2_K_matvec_golden(lg, lgold):
    W, x, y0 = lgold["q2_W"], lgold["q2_x"], lgold["q2_y0"]
    y = y0.copy()
    lg.matvec("q2_K", W, x, y, W.shape[0], x.size)
    assert rel_l2(y, lgold["q2_matvec"]) < 1e-5


@pytest.mark.parametrize("key,fmt", [("q8", "q8_0"), ("q4", "q4_K"), ("q2", "q2_K")])
def test_dequantize_to_fp16_golden(lg, golden, lgold, key, fmt):
    W = lgold["q2_W"] if key == "q2" else golden[f"{key}_W"]
    ref = lgold[f"deq_{key}"]
    out = np.zeros(ref.size, np.uint16)
    lg.dequantize_to_fp16(fmt, W, out, out.size)
    assert np.array_equal(out, ref)


@pytest.mark.parametrize("tk,tm", [(1024, 512), (2048, 1024)])
def test_matvec_fp16_golden(lg, lgold, tk, tm):
    W, x, y0 = lgold["f16_W"], lgold["f16_x"], lgold["f16_y0"]
    M, K = y0.size, x.size
    y = y0.copy()
    lg.matvec_fp16_fp32((tk, tm), np.ascontiguousarray(W), x, y, M, K)
    assert rel_l2(y, lgold[f"f16_matvec_{tk}_{tm}"]) < 1e-6
