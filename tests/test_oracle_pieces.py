"""Pin the oracle's two-piece activation quantizer (oracle.c
oc_quantize_act2_q8_0 / oc_quantize_act2_q4_K and the quant_act = 2 matvec)
with closed forms on the CPU.

Piece 0 is the reference quantizer (src/kernels/quant.cpp:18-98) per 32-block,
scale s = amax/127; piece 1 quantizes the residual r = x - s*q0 with the step
s/256: q1 = sat8(rne(r * (256/s))).  So:

  x = s*(q0 + q1/256) on that grid      ->  both pieces come back exactly and
                                            the dequantized value equals x
  s a power of two                       ->  r*256/s is exact: ties round to
                                            even, and a residual of exactly
                                            +s/2 (q1 = 128) saturates to 127
  any x                                  ->  |x - deq| <= s/512 up to fp32
                                            rounding (s/256 where q1 saturates)
  piece 0                                ->  bit for bit the one-piece quantizer

A step of s/254 instead of s/256, a missing residual, piece 1 computed from x
instead of r, or a Q4_K sub-block gathered in the wrong order fails one of
these.  The reference has no two-piece activation (its matvecs take fp32 x,
src/kernels/matvec.cpp:62-142); this is the GPU decode step's arithmetic, and
the quant_act = 2 matvec is pinned against the fp32 matvec on the dequantized x.
"""
import numpy as np

from conftest import rel_l2
from echohip import synth


def _grid_block(rng, s_exp_num, s_pow):
    """One 32-block on the two-piece grid: scale s = s_exp_num * 2^s_pow, q0 with max |q0| = 127 at a q1 = 0
    element, q1 in [-127, 127] elsewhere."""
    q0 = rng.integers(-127, 128, 32)
    q1 = rng.integers(-127, 128, 32)
    q0[5] = 127 if rng.integers(0, 2) else -127
    q1[5] = 0
    q1[np.abs(q0) == 127] = -np.sign(q0[np.abs(q0) == 127]) * np.abs(q1[np.abs(q0) == 127])  # |x| <= 127 s
    s = np.float32(s_exp_num * 2.0 ** s_pow)
    x = (s.astype(np.float64) * (q0 + q1 / 256.0)).astype(np.float32)
    assert np.array_equal(x.astype(np.float64), s * (q0 + q1 / 256.0))  # exactly representable
    return x, q0, q1, s


def test_two_piece_grid_round_trips_exactly(oc):
    rng = np.random.default_rng(7)
    blocks = [_grid_block(rng, num, p) for num, p in [(3, -7), (5, -12), (1, 0), (7, -20), (3, 4)] * 6]
    x = np.concatenate([b[0] for b in blocks])
    q0, q1, d = oc.quantize_act2_q8_0(x)
    assert np.array_equal(d, np.array([b[3] for b in blocks], np.float32))
    assert np.array_equal(q0, np.concatenate([b[1] for b in blocks]).astype(np.int8))
    assert np.array_equal(q1, np.concatenate([b[2] for b in blocks]).astype(np.int8))
    assert np.array_equal(oc.dequant_act2_q8_0(q0, q1, d), x)


def test_two_piece_ties_and_saturation(oc):
    """s = 2^-7 (amax = 127 * 2^-7): x/s and r*256/s are exact, so ties are exact halves."""
    s = 2.0 ** -7
    t = np.zeros(32)
    t[0] = 127.0                        # sets the scale
    t[1:8] = [2.5, -2.5, 3.5, 0.5 / 256, 1.5 / 256, -0.5 / 256, 2.5 / 256]
    t[8:10] = [1.0 + 3.5 / 256, -(1.0 + 3.5 / 256)]
    x = (t * s).astype(np.float32)
    q0, q1, d = oc.quantize_act2_q8_0(x)
    assert d[0] == np.float32(s)
    # piece 0 rounds half to even; a residual of +s/2 (q1 = 128) saturates to 127, -s/2 fits (-128)
    assert list(q0[1:4]) == [2, -2, 4] and list(q1[1:4]) == [127, -128, -128]
    # piece 1 rounds half to even: 0.5 -> 0, 1.5 -> 2, -0.5 -> 0, 2.5 -> 2, 3.5 -> 4
    assert list(q0[4:10]) == [0, 0, 0, 0, 1, -1] and list(q1[4:10]) == [0, 2, 0, 2, 4, -4]


def test_two_piece_error_bound_and_piece0_is_the_reference_quantizer(oc):
    for seed, scale in ((1, 1.0), (2, 1e-3), (3, 40.0)):
        x = (scale * synth.normal(seed, 4096) * (1.0 + 4.0 * synth.uniform01(seed + 10, 4096))).astype(np.float32)
        q0, q1, d = oc.quantize_act2_q8_0(x)
        r0, rd = oc.quantize_act_q8_0(x)
        assert np.array_equal(q0, r0) and np.array_equal(d, rd)
        deq = oc.dequant_act2_q8_0(q0, q1, d).astype(np.float64)
        s = np.repeat(d.astype(np.float64), 32)
        err = np.abs(deq - x)
        # a residual rounding to +128 saturates (error up to s/256); fp32 rounding of the pieces' sum adds
        # at most ~1.2% of s/512 at |x| = 127 s (the exact-grid test pins the step s/256 itself)
        sat = q1 == 127
        assert np.all(err[~sat] <= s[~sat] / 512 * 1.02)
        assert np.all(err <= s / 256 * 1.02)
        # two pieces are ~256x finer than one
        one = oc.dequant_act_q8_0(r0, rd).astype(np.float64)
        assert 100 * rel_l2(deq, x) < rel_l2(one, x)


def test_two_piece_q4_K_is_the_q8_0_split_in_sub_block_order(oc):
    K = 768
    x = (synth.normal(20, K) * (1.0 + synth.uniform01(21, K))).astype(np.float32)
    pos = np.array([oc.lib.oc_q4k_pos(s, i) for s in range(8) for i in range(32)], np.int64)
    perm = (256 * np.arange(K // 256)[:, None] + pos[None, :]).reshape(-1)
    q0, q1, d = oc.quantize_act2_q4_K(x)
    e0, e1, ed = oc.quantize_act2_q8_0(x[perm])
    assert np.array_equal(q0, e0) and np.array_equal(q1, e1) and np.array_equal(d, ed)
    r0, rd, _ = oc.quantize_act_q4_K(x)
    assert np.array_equal(q0, r0) and np.array_equal(d, rd)
    deq = oc.dequant_act2_q4_K(q0, q1, d)
    assert np.array_equal(deq[perm], oc.dequant_act2_q8_0(e0, e1, ed))  # back in original positions
    s_at = np.empty(K)
    s_at[perm] = np.repeat(d.astype(np.float64), 32)  # each element's sub-block scale, original positions
    assert np.all(np.abs(deq.astype(np.float64) - x) <= s_at / 256 * 1.02)


def test_quant_act_2_matvec_is_the_fp32_matvec_of_the_two_piece_input(oc):
    N, K = 48, 512
    Wq8 = synth.q8_0_blocks(30, N, K)
    Wq4 = synth.q4_K_blocks(31, N, K, 1e-2)
    x = synth.normal(32, K).astype(np.float32)
    q0, q1, d = oc.quantize_act2_q8_0(x)
    ref8 = oc.matvec_q8_0(Wq8, oc.dequant_act2_q8_0(q0, q1, d))
    assert np.array_equal(oc.matvec_act(6, Wq8, x, 2), ref8)
    p0, p1, pd = oc.quantize_act2_q4_K(x)
    ref4 = oc.matvec_q4_K(Wq4, oc.dequant_act2_q4_K(p0, p1, pd))
    assert np.array_equal(oc.matvec_act(10, Wq4, x, 2), ref4)
    # against the reference's fp32 activations: two pieces ~2e-5, one piece ~5e-3
    for fmt, W, f32 in ((6, Wq8, oc.matvec_q8_0), (10, Wq4, oc.matvec_q4_K)):
        exact = f32(W, x)
        e2, e1 = rel_l2(oc.matvec_act(fmt, W, x, 2), exact), rel_l2(oc.matvec_act(fmt, W, x, 1), exact)
        assert e2 < 1e-4 and e1 > 30 * e2, (fmt, e1, e2)
