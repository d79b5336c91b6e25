"""Prefill GEMM (ec_gemm, int8 MFMA) vs exact fp64 products of the same
quantized operands.

X is quantized per 32-element block by the reference quantizer (the oracle's
oc_quantize_act_*, bit-identical to the GPU's), W decoded from its GGUF bytes
in numpy (Q4_K with the reference's nibble order and scale unpack, pinned here
against the reference's own Q4_K matvec golden vector).  Y_ref = X_deq @ W_deq^T
in float64 is then the exact value of what the GPU sums; the GPU's fp32 result
must agree within 1e-5 relative L2 (fp32 accumulation over K only; a single
wrong int8 value or a scale applied to the wrong block moves Y by ~1e-3).
Shapes include BASELINE config 2' (M = 512; 9216x2560 and 2560x9216).
"""
import numpy as np
import pytest

from conftest import rel_l2
from echohip import synth
from echohip.lib import Q4_K, Q8_0
from test_gpu_kernels import dev, empty, host

pytestmark = pytest.mark.gpu


def q8_dequant(W, K):
    b = W.reshape(W.shape[0], K // 32, 34)
    d = b[:, :, 0:2].copy().view(np.float16).astype(np.float64)
    return (d * b[:, :, 2:].view(np.int8)).reshape(W.shape[0], K)


def q4k_unpack(s):
    """get_scale_min_k4 (reference quant.cpp:222-242) over [..., 12] bytes -> sc, m [..., 8]."""
    s = s.astype(np.int64)
    sc = np.zeros(s.shape[:-1] + (8,), np.int64)
    m = np.zeros_like(sc)
    for j in range(4):
        sc[..., j] = s[..., j] & 63
        m[..., j] = s[..., j + 4] & 63
    for j in range(4, 8):
        sc[..., j] = (s[..., j + 4] & 0x0F) | ((s[..., j - 4] >> 6) << 4)
        m[..., j] = (s[..., j + 4] >> 4) | ((s[..., j] >> 6) << 4)
    return sc, m


def q4k_pos(s, i):
    return 64 * (s // 2) + 16 * (s % 2) + i if i < 16 else 64 * (s // 2) + 32 + 16 * (s % 2) + (i - 16)


def q4k_dequant(W, K):
    rows, nb = W.shape[0], K // 256
    b = W.reshape(rows, nb, 144)
    d = b[:, :, 0:2].copy().view(np.float16).astype(np.float64)[..., 0]
    dmin = b[:, :, 2:4].copy().view(np.float16).astype(np.float64)[..., 0]
    sc, m = q4k_unpack(b[:, :, 4:16])
    qs = b[:, :, 16:]
    out = np.zeros((rows, nb, 256))
    for s in range(8):
        for i in range(32):
            byte = qs[:, :, 16 * s + (i % 16)].astype(np.int64)
            q = byte & 15 if i < 16 else byte >> 4
            out[:, :, q4k_pos(s, i)] = d * sc[:, :, s] * q - dmin * m[:, :, s]
    return out.reshape(rows, K)


def test_q4k_dequant_matches_reference_matvec(golden):
    """The numpy Q4_K decoding above reproduces the reference's matvec_q4_K."""
    W = golden["q4_W"]
    y = golden["mv_y0"] + q4k_dequant(W, 512) @ golden["mv_x"].astype(np.float64)
    assert rel_l2(y, golden["q4_matvec"]) < 1e-6


def x_dequant(oc, fmt, X):
    M, K = X.shape
    out = np.zeros((M, K))
    for mrow in range(M):
        if fmt == Q8_0:
            xq, xd = oc.quantize_act_q8_0(X[mrow])
            out[mrow] = (xq.reshape(-1, 32).astype(np.float64) * xd[:, None].astype(np.float64)).reshape(K)
        else:
            xq, xd, _ = oc.quantize_act_q4_K(X[mrow])
            v = xq.reshape(-1, 32).astype(np.float64) * xd[:, None].astype(np.float64)  # [K/32][32] by sub-block
            out[mrow, _q4k_perm(K)] = v.reshape(K)
    return out


def _q4k_perm(K):
    """Position in the row of element i of sub-block sb (sub-block order -> natural order)."""
    return np.array([256 * (sb // 8) + q4k_pos(sb % 8, i) for sb in range(K // 32) for i in range(32)])


CASES = [(Q8_0, 37, 256, 512), (Q8_0, 512, 9216, 2560), (Q8_0, 512, 2560, 9216), (Q8_0, 100, 272, 384),
         (Q8_0, 19, 48, 160), (Q8_0, 70, 40, 4128),
         (Q4_K, 37, 256, 512), (Q4_K, 512, 9216, 2560), (Q4_K, 512, 2560, 9216), (Q4_K, 64, 48, 768),
         # the rows of a ragged multi-sequence prefill pass (two or more chunks)
         (Q8_0, 1024, 2560, 2560), (Q8_0, 1100, 272, 512), (Q4_K, 1030, 256, 768), (Q4_K, 2048, 96, 512)]


@pytest.mark.parametrize("fmt,M,N,K", CASES)
def test_gemm(hip, oc, fmt, M, N, K):
    import torch
    W = synth.q8_0_blocks(31, N, K) if fmt == Q8_0 else synth.q4_K_blocks(32, N, K)
    X = (synth.activations(33, M * K) * 2.0).astype(np.float32).reshape(M, K)
    tiled = empty(hip.tiled_bytes(fmt, N, K), torch.uint8)
    hip.repack(fmt, dev(W), tiled, N, K)
    act = empty(hip.gemm_act_bytes(fmt, M, K), torch.uint8)
    hip.gemm_quantize_act(fmt, dev(X), act, M, K)
    y0 = synth.activations(34, M * N).reshape(M, N)
    y = dev(y0)
    hip.gemm(fmt, tiled, act, y, M, N, K, accumulate=True)
    got = host(y)
    Wd = q8_dequant(W, K) if fmt == Q8_0 else q4k_dequant(W, K)
    ref = y0 + x_dequant(oc, fmt, X) @ Wd.T
    err = rel_l2(got - y0, ref - y0)
    print(f"fmt {fmt} M {M} N {N} K {K}: rel_l2 {err:.2e}")
    assert err < 1e-5
