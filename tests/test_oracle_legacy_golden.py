"""CPU checks of tests/golden/legacy_golden.npz (reference outputs) against
independent numpy restatements, so the fixture's layout reading is pinned:

* Q2_K (src/kernels/matvec.cpp:146-183): block = fp16 d, fp16 dmin, 16 scale
  bytes, 64 bytes of 2-bit weights; weight j of a block uses sub-block
  sb = j/8, s = sb/2, scale byte scales[s] (even sb) or scales[s+8] (odd sb,
  which reaches into the weight bytes for s >= 8, as the reference indexes),
  low nibble * d and high nibble * dmin; q = bits 2*(j%4) of byte j/4.
* fp16 dequantization: the fp32 weights of each format rounded to fp16.
* fp16 matvec: y0 + W x in float64 (the reference's fp32 sums agree to 1e-6).
"""
from pathlib import Path

import numpy as np

from conftest import rel_l2

G = np.load(Path(__file__).resolve().parent / "golden" / "legacy_golden.npz")
K0 = np.load(Path(__file__).resolve().parent / "golden" / "kernels_golden.npz")


def q2k_weights(W, K):
    M = W.shape[0]
    nb = K // 256
    b = W.reshape(M, nb, 84)
    d = b[:, :, 0:2].copy().view(np.float16).astype(np.float64)[..., 0]
    dm = b[:, :, 2:4].copy().view(np.float16).astype(np.float64)[..., 0]
    scales = b[:, :, 4:]  # 80 bytes: 16 scale bytes then the weight bytes (index s+8 may reach them)
    qs = b[:, :, 20:84]
    j = np.arange(256)
    sb = j // 8
    s = sb // 2
    sidx = np.where(sb % 2 == 0, s, s + 8)
    sc = scales[:, :, sidx]
    q = (qs[:, :, j // 4] >> (2 * (j % 4))) & 3
    w = d[..., None] * (sc & 0x0F) * q - dm[..., None] * (sc >> 4)
    return w.reshape(M, K)


def test_q2_K_matvec_fixture():
    W, x, y0 = G["q2_W"], G["q2_x"], G["q2_y0"]
    y = y0 + q2k_weights(W, x.size) @ x.astype(np.float64)
    assert rel_l2(G["q2_matvec"], y) < 1e-5


def test_q2_K_dequant_fixture():
    w = q2k_weights(G["q2_W"], 512).astype(np.float32).astype(np.float16)
    assert np.array_equal(G["deq_q2"], w.reshape(-1).view(np.uint16))


def test_q8_0_dequant_fixture():
    blk = K0["q8_W"].reshape(-1, 34)
    w = (blk[:, 0:2].copy().view(np.float16).astype(np.float32) * blk[:, 2:].view(np.int8)).astype(np.float16)
    assert np.array_equal(G["deq_q8"], w.reshape(-1).view(np.uint16))


def test_q4_K_dequant_fixture(oc):
    """fp16 weights of the reference's Q4_K dequantizer, used in an fp64 matvec,
    reproduce the reference's own Q4_K matvec within fp16 weight rounding."""
    Wf = G["deq_q4"].view(np.float16).astype(np.float64).reshape(K0["q4_W"].shape[0], 512)
    y = K0["mv_y0"] + Wf @ K0["mv_x"].astype(np.float64)
    assert rel_l2(y, K0["q4_matvec"]) < 1e-3


def test_fp16_matvec_fixture():
    W = G["f16_W"].view(np.float16).astype(np.float64).reshape(G["f16_y0"].size, G["f16_x"].size)
    y = G["f16_y0"] + W @ G["f16_x"].astype(np.float64)
    for k in ("f16_matvec_1024_512", "f16_matvec_2048_1024"):
        assert rel_l2(G[k], y) < 1e-6
