"""GPU two-piece activations (ec_quantize_act_pieces and the _pieces matvec and
glue entry points) against the oracle's two-piece quantizer
(oc_quantize_act2_q8_0 / oc_quantize_act2_q4_K, pinned by
tests/test_oracle_pieces.py).

* the activation quantizer: both pieces and the scales bit-exact (Q8_0 and
  Q4_K, M = 1 .. 16 tokens, i.e. up to 32 layout rows);
* block dots: every layout row's int32 dots bit-exact with the oracle's dots of
  that piece;
* matvec: y within 1e-5 of the oracle's fp32 matvec on the dequantized
  two-piece input, and within 1e-4 of the reference's fp32-activation matvec on
  x itself (src/kernels/matvec.cpp:62-142; one piece is ~5e-3 away);
* split-K: the parts add up to the matvec;
* the glue ops that write activations: piece 0 and the scales byte-identical to
  the same op with one piece, and the two-piece value within the quantizer's
  bound (s/512 per element, plus fp32 slack) of the oracle's fp32 op.
The delta step's and attention's two-piece outputs are checked per operation in
the decoder tests (tests/decoder_ops.py).
"""
import numpy as np
import pytest

from conftest import rel_l2
from echohip import synth
from echohip.lib import Q4_K, Q8_0
from test_gpu_kernels import dev, empty, host

pytestmark = pytest.mark.gpu


def _act2(hip, fmt, X):
    import torch
    M, K = X.shape
    act = empty(hip.act_bytes(fmt, M, K, pieces=2), torch.uint8)
    hip.quantize_act(fmt, dev(X.astype(np.float32)), act, M, K, pieces=2)
    return act


def _unpack2(hip, fmt, act, M, K, pieces=2):
    import torch
    xq = empty(pieces * M * K, torch.int8)
    xd = empty(M * K // 32, torch.float32)
    hip.act_unpack(fmt, act, xq, xd, M, K, pieces=pieces)
    return host(xq).reshape(M, pieces, K), host(xd).reshape(M, K // 32)


def _oc_act2(oc, fmt, x):
    return oc.quantize_act2_q4_K(x) if fmt == Q4_K else oc.quantize_act2_q8_0(x)


def _weights(fmt, seed, N, K):
    return synth.q4_K_blocks(seed, N, K, 1e-2) if fmt == Q4_K else synth.q8_0_blocks(seed, N, K)


@pytest.mark.parametrize("fmt", [Q8_0, Q4_K], ids=["q8_0", "q4_K"])
@pytest.mark.parametrize("M,K", [(1, 512), (3, 768), (8, 2560), (16, 256), (16, 9216)])
def test_quantize_act_two_pieces_bit_exact(hip, oc, fmt, M, K):
    X = (synth.activations(100 + M, M * K).reshape(M, K) * (1.0 + synth.uniform01(7, M * K).reshape(M, K)))
    X = X.astype(np.float32)
    xq, xd = _unpack2(hip, fmt, _act2(hip, fmt, X), M, K)
    for m in range(M):
        q0, q1, d = _oc_act2(oc, fmt, X[m])
        assert np.array_equal(xq[m, 0], q0) and np.array_equal(xq[m, 1], q1), m
        assert np.array_equal(xd[m].view(np.uint32), d.view(np.uint32)), m


# (8, 9216, 2560) and (16, 4112, 512) run two 16-row tiles per wave (Q4_K: 288 / 129 workgroups); 4112 rows
# are 257 tiles, so the last workgroup's second tile is past the end (read, not stored)
CASES = [(1, 48, 512), (3, 40, 768), (8, 64, 2560), (16, 16, 256), (5, 33, 1024), (16, 64, 9216), (8, 9216, 2560),
         (16, 4112, 512)]


@pytest.mark.parametrize("fmt", [Q8_0, Q4_K], ids=["q8_0", "q4_K"])
@pytest.mark.parametrize("M,N,K", CASES)
def test_matvec_two_pieces(hip, oc, fmt, M, N, K):
    import torch
    W = _weights(fmt, 300 + K + fmt, N, K)
    X = synth.activations(400 + M, M * K).reshape(M, K).astype(np.float32)
    Wd = dev(W)
    tiled = empty(hip.tiled_bytes(fmt, N, K), torch.uint8)
    hip.repack(fmt, Wd, tiled, N, K)
    act = _act2(hip, fmt, X)
    nb = K // 32
    dots = empty(2 * M * N * nb, torch.int32)
    hip.block_dots(fmt, tiled, act, dots, M, N, K, pieces=2)
    dots = host(dots).reshape(M, 2, N, nb)
    y0 = synth.activations(5, M * N).reshape(M, N)
    y = dev(y0)
    hip.matvec(fmt, tiled, act, y, M, N, K, accumulate=True, pieces=2)
    y = host(y) - y0
    bd = oc.block_dots_q4_K if fmt == Q4_K else oc.block_dots_q8_0
    f32 = oc.matvec_q4_K if fmt == Q4_K else oc.matvec_q8_0
    deq = oc.dequant_act2_q4_K if fmt == Q4_K else oc.dequant_act2_q8_0
    worst = 0.0
    for m in range(M):
        q0, q1, d = _oc_act2(oc, fmt, X[m])
        assert np.array_equal(dots[m, 0], bd(W, q0)) and np.array_equal(dots[m, 1], bd(W, q1)), m
        assert rel_l2(y[m], f32(W, deq(q0, q1, d))) < 1e-5
        worst = max(worst, rel_l2(y[m], f32(W, X[m])))
    print(f"two-piece matvec vs the fp32-activation reference: {worst:.2e}")
    assert worst < 1e-4
    y2 = dev(np.full((M, N), 7.0, np.float32))
    hip.matvec(fmt, tiled, act, y2, M, N, K, accumulate=False, pieces=2)
    assert np.allclose(host(y2), y, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("M,N,K,ns", [(8, 40, 4096, 4), (16, 64, 9216, 3), (1, 48, 512, 2), (8, 2560, 9216, 3)])
def test_matvec_split_two_pieces(hip, M, N, K, ns):
    import torch
    W = synth.q8_0_blocks(500 + K, N, K)
    X = synth.activations(600 + M, M * K).reshape(M, K).astype(np.float32)
    tiled = empty(hip.tiled_bytes(Q8_0, N, K), torch.uint8)
    hip.repack(Q8_0, dev(W), tiled, N, K)
    act = _act2(hip, Q8_0, X)
    parts = empty(ns * M * N, torch.float32)
    hip.matvec_split(Q8_0, tiled, act, parts, M, N, K, ns, pieces=2)
    y = empty(M * N, torch.float32)
    hip.matvec(Q8_0, tiled, act, y, M, N, K, pieces=2)
    assert rel_l2(host(parts).reshape(ns, M, N).sum(axis=0), host(y).reshape(M, N)) < 1e-6


def _check_glue(hip, oc, run, M, K, ref_rows):
    """run(act, pieces) writes an activation; piece 0 and the scales of the two-piece run equal the one-piece
    run's bytes, and the two-piece value is within the quantizer's bound of the oracle's fp32 rows."""
    import torch
    a1 = empty(hip.act_bytes(Q8_0, M, K), torch.uint8)
    a2 = empty(hip.act_bytes(Q8_0, M, K, pieces=2), torch.uint8)
    run(a1, 1)
    run(a2, 2)
    q1, d1 = _unpack2(hip, Q8_0, a1, M, K, pieces=1)
    q2, d2 = _unpack2(hip, Q8_0, a2, M, K, pieces=2)
    assert np.array_equal(q2[:, 0], q1[:, 0]) and np.array_equal(d2.view(np.uint32), d1.view(np.uint32))
    for m in range(M):
        s = np.repeat(d2[m].astype(np.float64), 32)
        deq = oc.dequant_act2_q8_0(q2[m, 0], q2[m, 1], d2[m]).astype(np.float64)
        # s/512 per element (s/256 where piece 1 saturates), plus the fp32 difference of the two rows
        bound = s * np.where(q2[m, 1] == 127, 1.02 / 256, 1.02 / 512) + 3e-4 * s
        assert np.all(np.abs(deq - ref_rows[m]) <= bound), (m, np.max(np.abs(deq - ref_rows[m]) / s))
        one = oc.dequant_act_q8_0(q1[m, 0], d1[m]).astype(np.float64)
        assert 30 * rel_l2(deq, ref_rows[m]) < rel_l2(one, ref_rows[m])


@pytest.mark.parametrize("M,H", [(8, 2560), (3, 256), (16, 128), (2, 5120)])
def test_rmsnorm_quant_two_pieces(hip, oc, M, H):
    x = (3.0 * synth.normal(synth.stream_seed(11, H), M * H)).astype(np.float32).reshape(M, H)
    w = (1.0 + 0.1 * synth.normal(synth.stream_seed(12, H), H)).astype(np.float32)
    ref = np.stack([oc.rmsnorm(x[i], w) for i in range(M)])
    _check_glue(hip, oc, lambda a, p: hip.rmsnorm_quant(dev(x), dev(w), a, M, H, pieces=p), M, H, ref)


@pytest.mark.parametrize("M,H,nparts", [(8, 2560, 3), (8, 2560, 6), (2, 5120, 2), (16, 384, 1)])
def test_add_rmsnorm_quant_two_pieces(hip, oc, M, H, nparts):
    """Both kernels of ec_glue_add_rmsnorm_quant: one workgroup per row (up to 4 parts, rows up to 4096) and
    row-parallel blocks; the residual written to x_out is the same with either piece count."""
    import torch
    x = (2.0 * synth.normal(synth.stream_seed(13, H), M * H)).astype(np.float32).reshape(M, H)
    parts = (0.5 * synth.normal(synth.stream_seed(14, H), nparts * M * H)).astype(np.float32).reshape(nparts, M, H)
    w = (1.0 + 0.1 * synth.normal(synth.stream_seed(15, H), H)).astype(np.float32)
    xs = x.copy()
    for p in range(nparts):
        xs = (xs + parts[p]).astype(np.float32)
    ref = np.stack([oc.rmsnorm(xs[i], w) for i in range(M)])
    outs = []

    def run(a, p):
        xo = empty(M * H, torch.float32)
        hip.add_rmsnorm_quant(dev(x), dev(parts), nparts, xo, dev(w), a, M, H, pieces=p)
        outs.append(host(xo))
    _check_glue(hip, oc, run, M, H, ref)
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[1].reshape(M, H), xs)


@pytest.mark.parametrize("M,F,nparts", [(8, 9216, 3), (3, 512, 1)])
def test_swiglu_quant_two_pieces(hip, oc, M, F, nparts):
    gu = (2.0 * synth.normal(synth.stream_seed(16, F), nparts * M * 2 * F)).astype(np.float32)
    g = gu.reshape(nparts, M, 2 * F)
    tot = g[0].copy()
    for p in range(1, nparts):
        tot = (tot + g[p]).astype(np.float32)
    ref = np.stack([oc.swiglu(tot[i][:F], tot[i][F:]) for i in range(M)])
    _check_glue(hip, oc, lambda a, p: hip.swiglu_quant_split(dev(gu), nparts, a, M, F, pieces=p), M, F, ref)


def test_gated_norm_quant_two_pieces(hip, oc):
    M, n_v, Nin, z_off = 8, 32, 12352, 8192
    core = synth.normal(synth.stream_seed(17, 1), M * n_v * 128).astype(np.float32)
    proj = (2.0 * synth.normal(synth.stream_seed(18, 1), M * Nin)).astype(np.float32)
    w = (1.0 + 0.1 * synth.normal(synth.stream_seed(19, 1), 128)).astype(np.float32)
    pr = proj.reshape(M, Nin)
    ref = np.stack([oc.gated_rmsnorm(core.reshape(M, -1)[i], pr[i, z_off:z_off + n_v * 128], w, n_v, 128).reshape(-1)
                    for i in range(M)])
    _check_glue(hip, oc, lambda a, p: hip.gated_norm_quant(dev(core), dev(proj), Nin, z_off, dev(w), a, M, n_v,
                                                           pieces=p), M, n_v * 128, ref)
