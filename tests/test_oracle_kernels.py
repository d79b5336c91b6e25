"""Pin the C oracle's kernel restatements (CPU only).

Checks against: the reference's own known-answer tests
(src/kernels/quant.cpp:403-654, echo-core-zig/src/kernels/matvec.zig:289-352),
golden vectors written by the compiled reference (tests/golden/gen_golden.py),
exhaustive codecs, fp64 brute force and exact integer closed forms.
"""
import numpy as np
import pytest

from conftest import rel_l2
from echohip import synth


# ------------------------------------------------------------------ fp16
def test_fp16_decode_exhaustive(oc):
    h = np.arange(65536, dtype=np.uint32)
    ref = h.astype(np.uint16).view(np.float16).astype(np.float32)
    got = np.array([oc.lib.oc_fp16_to_fp32(int(v)) for v in h], np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.all(np.isnan(got[~finite]) == np.isnan(ref[~finite]))


def test_fp16_encode_rne(oc):
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0,
        rng.standard_normal(5000).astype(np.float32) * 1e-5,  # subnormal halves
        np.array([65504, 65519.99, 65520, 1e9, 2 ** -24, 2 ** -25, 1.5 * 2 ** -25, 0.0, -0.0], np.float32),
        # exact ties between adjacent halves
        (np.arange(1024, 2048, dtype=np.float32) + 0.5) / 1024.0,
    ])
    ref = x.astype(np.float16).view(np.uint16)
    got = np.array([oc.lib.oc_fp32_to_fp16(float(v)) for v in x], np.uint16)
    assert np.array_equal(got, ref)


# ------------------------------------------------------------------- RNG
def test_splitmix64_known_answer(oc):
    # splitmix64 from state 0: published first outputs
    want = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    assert [oc.lib.oc_splitmix64_at(0, i) for i in range(3)] == want
    assert [int(v) for v in synth.splitmix64(0, 3)] == want
    s = 0x1234ABCD
    assert [oc.lib.oc_splitmix64_at(s, i) for i in range(100, 105)] == [int(v) for v in synth.splitmix64(s, 5, 100)]


# ------------------------------------------------------------- quantizer
def test_quant_reference_test1(oc):
    # src/kernels/quant.cpp:403-432
    q, s = oc.quantize(np.array([1, 2, 3, 4], np.float32), 4)
    assert abs(s[0] - 4.0 / 127.0) < 1e-6
    assert q.tolist() == [[32, 64, 95, 127]]
    assert np.max(np.abs(q[0] * s[0] - np.array([1, 2, 3, 4]))) < s[0] * 0.5 + 1e-6


@pytest.mark.parametrize("width", [4, 8, 12, 16, 32, 37, 256, 1024])
def test_quant_golden(oc, golden, width):
    q, s = oc.quantize(golden[f"quant_w{width}_x"], width)
    assert np.array_equal(q.ravel(), golden[f"quant_w{width}_q"])
    assert np.array_equal(s.view(np.uint32), golden[f"quant_w{width}_s"].view(np.uint32))


def test_quant_ties_and_zero(oc, golden):
    x = golden["quant_ties_x"]
    q, s = oc.quantize(x, x.size)
    assert np.array_equal(q.ravel(), golden["quant_ties_q"])
    # body (first 8) rounds half-to-even, tail rounds half away from zero
    assert q.ravel()[1:4].tolist() == [2, 4, 0]
    assert q.ravel()[8:11].tolist() == [3, 4, 1]
    q, s = oc.quantize(np.zeros(32, np.float32), 32)
    assert s[0] == 1.0 and not q.any()
    assert np.array_equal(q.ravel(), golden["quant_zero_q"])


# ------------------------------------------------------------- int8 dot
def test_int8_dot_golden(oc, golden):
    dim, seq = 256, 64
    out = np.zeros(seq, np.float32)
    oc.lib.oc_fused_dequant_dot_int8(golden["int8dot_q"], golden["int8dot_k"], golden["int8dot_s"], out, dim, seq)
    ref = golden["int8dot_out"]
    assert np.max(np.abs(out - ref)) < 1e-4 * max(1.0, float(np.max(np.abs(ref))))


def test_int8_dot_reference_test2(oc):
    # src/kernels/quant.cpp:434-486: fused == explicit dequant dot within 1e-4
    q = np.array([1, 2, 3, 4], np.float32)
    keys = np.array([1, 0, -1, 0.5, 0, 1, 0, 0, 2, 2, 2, 2], np.float32)
    kq, ks = oc.quantize(keys, 4)
    out = np.zeros(3, np.float32)
    oc.lib.oc_fused_dequant_dot_int8(q, kq.ravel(), ks, out, 4, 3)
    exp = (kq.astype(np.float64) * ks[:, None]) @ q
    assert np.max(np.abs(out - exp)) < 1e-4


# ------------------------------------------------------------------ Q8_0
def test_q8_0_reference_test4(oc):
    # src/kernels/quant.cpp:523-555
    qs = np.stack([np.arange(32) - 16, np.arange(32) - 16]).astype(np.int8)[None]
    d = np.array([[0.5, 1.0]], np.float16)
    W = synth.q8_0_from_parts(qs, d)
    x = (((np.arange(64) % 7) + 1) * 0.1).astype(np.float32)
    exp = sum(float(d[0, b]) * float(qs[0, b, i]) * float(x[b * 32 + i]) for b in range(2) for i in range(32))
    y = oc.matvec_q8_0(W, x)
    assert abs(y[0] - exp) < 1e-2
    assert abs(oc.lib.oc_dot_q8_0_f64(W.ravel(), 2, x) - exp) < 1e-4


def test_q8_0_golden(oc, golden):
    W, x, y0 = golden["q8_W"], golden["mv_x"], golden["mv_y0"]
    y = oc.matvec_q8_0(W, x, y0)
    assert rel_l2(y, golden["q8_matvec"]) < 1e-6
    assert rel_l2(y - y0, golden["q8_fused"]) < 1e-5
    f64 = np.array([oc.lib.oc_dot_q8_0_f64(np.ascontiguousarray(W[m]), W.shape[1] // 34, x)
                    for m in range(W.shape[0])])
    assert rel_l2(golden["q8_fused"], f64) < 1e-6


def test_q8_0_block_dots_closed_form(oc):
    M, K = 24, 256
    W = synth.q8_0_blocks(5, M, K)
    xq = synth.randint(6, K, -127, 127).astype(np.int8)
    got = oc.block_dots_q8_0(W, xq)
    qs = W.reshape(M, K // 32, 34)[:, :, 2:].view(np.int8).astype(np.int64)
    exp = np.einsum("mbj,bj->mb", qs, xq.astype(np.int64).reshape(K // 32, 32))
    assert np.array_equal(got, exp)


def test_q8_0_act_quant_matches_quantizer(oc):
    x = synth.activations(3, 512)
    xq, xd = oc.quantize_act_q8_0(x)
    q2, s2 = oc.quantize(x, 32)
    assert np.array_equal(xq, q2.ravel()) and np.array_equal(xd, s2)
    assert np.array_equal(oc.dequant_act_q8_0(xq, xd), (q2 * s2[:, None]).ravel().astype(np.float32))


# ------------------------------------------------------------------ Q4_K
def _q4k_fixture_block():
    """The Q4_K block of src/kernels/quant.cpp:567-591 (= matvec.zig:290-306)."""
    b = np.zeros(144, np.uint8)
    b[0:2] = np.frombuffer(np.float16(63.0).tobytes(), np.uint8)
    b[2:4] = np.frombuffer(np.float16(63.0).tobytes(), np.uint8)
    sc = b[4:16]
    for j in range(4):
        sc[j] = j + 1
        sc[j + 4] = j
    for j in range(4):
        sc[j] |= 1 << 6
    sc[8], sc[9], sc[10], sc[11] = 0x12, 0x23, 0x34, 0x45
    b[16:] = 0x55
    return b[None, :]


def test_q4_K_reference_test5(oc):
    W = _q4k_fixture_block()
    x = (((np.arange(256) % 11) + 1) * 0.01).astype(np.float32)
    y = oc.matvec_q4_K(W, x)
    # observed value of the reference's own test program (fused = 51276.957031)
    assert abs(y[0] - 51276.96) < 1e-2
    assert abs(oc.lib.oc_dot_q4_K_f64(W.ravel(), 1, x) - 51276.96) < 1e-2


def test_q4_K_golden(oc, golden):
    W, x, y0 = golden["q4_W"], golden["mv_x"], golden["mv_y0"]
    y = oc.matvec_q4_K(W, x, y0)
    assert rel_l2(y, golden["q4_matvec"]) < 1e-6
    assert rel_l2(y - y0, golden["q4_fused"]) < 1e-5
    f64 = np.array([oc.lib.oc_dot_q4_K_f64(np.ascontiguousarray(W[m]), W.shape[1] // 144, x)
                    for m in range(W.shape[0])])
    assert rel_l2(golden["q4_fused"], f64) < 1e-6


def test_q4_K_nibble_layout_probe(oc, golden):
    """One non-zero nibble per position: the reference output names the x index."""
    W, x, yref = golden["q4_probe_W"], golden["q4_probe_x"], golden["q4_probe_y"]
    for p in range(256):
        y = oc.matvec_q4_K(W[p:p + 1], x)
        assert y[0] == yref[p]
        byte, hi = divmod(p, 2)
        s, i = divmod(byte, 16)
        # sub-block s owns qs bytes [16s,16s+16); low nibble -> i, high -> 16+i
        assert int(yref[p]) - 1 == oc.lib.oc_q4k_pos(s, i + 16 * hi)


def test_q4_K_scale_pack_roundtrip(oc):
    sc = np.repeat(np.arange(64), 64)
    mn = np.tile(np.arange(64), 64)
    for j in range(8):
        s8 = np.zeros((4096, 8), np.int64)
        m8 = np.zeros((4096, 8), np.int64)
        s8[:, j], m8[:, j] = sc, mn
        s8[:, (j + 3) % 8] = 63 - sc  # neighbours share bits: make them busy
        packed = synth.pack_q4k_scales(s8, m8)
        import ctypes
        for r in range(0, 4096, 97):
            a, b = ctypes.c_uint8(), ctypes.c_uint8()
            oc.lib.oc_q4k_scale_min.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
            row = np.ascontiguousarray(packed[r])
            oc.lib.oc_q4k_scale_min(row.ctypes.data, j, ctypes.byref(a), ctypes.byref(b))
            assert (a.value, b.value) == (s8[r, j], m8[r, j])


def test_q4_K_act_quant_grouping(oc):
    K = 512
    x = synth.activations(21, K)
    xq, xd, xs = oc.quantize_act_q4_K(x)
    # each sub-block's 32 values are the reference quantizer applied to the gathered positions
    pos = np.array([[oc.lib.oc_q4k_pos(s, i) for i in range(32)] for s in range(8)])
    gathered = np.concatenate([x[256 * b + pos].reshape(-1) for b in range(K // 256)])
    q2, s2 = oc.quantize(gathered, 32)
    assert np.array_equal(xq, q2.ravel()) and np.array_equal(xd, s2)
    assert np.array_equal(xs, q2.astype(np.int32).sum(1))
    xdeq = oc.dequant_act_q4_K(xq, xd)
    assert rel_l2(xdeq, x) < 1e-2  # the dequantized vector approximates x in natural order


def test_q4_K_block_dots_closed_form(oc):
    M, K = 16, 512
    W = synth.q4_K_blocks(31, M, K)
    xq = synth.randint(32, K, -127, 127).astype(np.int8)
    got = oc.block_dots_q4_K(W, xq)
    qs = W.reshape(M, K // 256, 144)[:, :, 16:].reshape(M, K // 256, 8, 16).astype(np.int64)
    nib = np.concatenate([qs & 15, qs >> 4], axis=3)  # [M, nb, 8, 32] in sub-block order
    exp = np.einsum("mbsi,bsi->mbs", nib, xq.astype(np.int64).reshape(K // 256, 8, 32)).reshape(M, K // 32)
    assert np.array_equal(got, exp)


def test_q4_K_integer_form_equals_reference(oc):
    """y from block dots: sum dx*(d*sc*isum - dmin*m*xsum) == matvec_q4_K(W, x_deq)."""
    M, K = 32, 512
    W = synth.q4_K_blocks(41, M, K)
    x = synth.activations(42, K)
    xq, xd, xs = oc.quantize_act_q4_K(x)
    isum = oc.block_dots_q4_K(W, xq).astype(np.float64)
    blk = W.reshape(M, K // 256, 144)
    d = blk[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
    dm = blk[:, :, 2:4].copy().view(np.float16)[..., 0].astype(np.float64)
    sc = np.zeros((M, K // 256, 8))
    mn = np.zeros((M, K // 256, 8))
    import ctypes
    oc.lib.oc_q4k_scale_min.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    for m in range(M):
        for b in range(K // 256):
            row = np.ascontiguousarray(blk[m, b, 4:16])
            for j in range(8):
                a, c = ctypes.c_uint8(), ctypes.c_uint8()
                oc.lib.oc_q4k_scale_min(row.ctypes.data, j, ctypes.byref(a), ctypes.byref(c))
                sc[m, b, j], mn[m, b, j] = a.value, c.value
    dx = xd.reshape(K // 256, 8).astype(np.float64)
    xsum = xs.reshape(K // 256, 8).astype(np.float64)
    y_int = np.sum(dx[None] * (d[..., None] * sc * isum.reshape(M, K // 256, 8) - dm[..., None] * mn * xsum[None]),
                   axis=(1, 2))
    y_ref = oc.matvec_q4_K(W, oc.dequant_act_q4_K(xq, xd))
    assert rel_l2(y_ref, y_int) < 1e-5


def test_two_piece_activation_quantizer(oc):
    """oc_quantize_act2_q8_0: piece 0 is the reference quantizer; piece 1 quantizes the residual with scale/256, so
    |x - (q0*s + q1*s/256)| <= s/512 wherever q1 did not saturate, and exactly representable inputs come back
    exactly."""
    import ctypes as C
    f32 = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
    i8 = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
    oc.lib.oc_quantize_act2_q8_0.argtypes = [f32, i8, i8, f32, C.c_uint32]
    oc.lib.oc_dequant_act2_q8_0.argtypes = [i8, i8, f32, f32, C.c_uint32]
    K = 4096
    x = synth.activations(17, K) * 3
    q0, q1 = np.zeros(K, np.int8), np.zeros(K, np.int8)
    xd, xr = np.zeros(K // 32, np.float32), np.zeros(K, np.float32)
    oc.lib.oc_quantize_act2_q8_0(x, q0, q1, xd, K)
    oc.lib.oc_dequant_act2_q8_0(q0, q1, xd, xr, K)
    rq, rs = oc.quantize_act_q8_0(x)
    assert np.array_equal(q0, rq) and np.array_equal(xd, rs)
    s = np.repeat(xd.astype(np.float64), 32)
    ok = np.abs(q1) < 127
    assert ok.mean() > 0.98
    fp32_sum = 2.0 ** -22 * np.abs(x.astype(np.float64))  # the fp32 rounding of q0*s + q1*s/256 itself
    assert np.all((np.abs(x.astype(np.float64) - xr) <= s / 512 + fp32_sum)[ok])
    # values on the two-piece grid (q0*s + q1*s/256 with |q1| < 128) are reproduced exactly
    s0 = np.float32(0.5)
    g = np.zeros(32, np.float32)
    g[0] = 127 * s0  # sets the block scale to exactly 0.5
    g[1:] = (np.arange(1, 32) - 16) * s0 + (np.arange(1, 32) % 7 - 3) * (s0 / 256)
    oc.lib.oc_quantize_act2_q8_0(g, q0[:32].copy(), q1[:32].copy(), xd[:1].copy(), 32)
    a0, a1, ad, ar = np.zeros(32, np.int8), np.zeros(32, np.int8), np.zeros(1, np.float32), np.zeros(32, np.float32)
    oc.lib.oc_quantize_act2_q8_0(g, a0, a1, ad, 32)
    oc.lib.oc_dequant_act2_q8_0(a0, a1, ad, ar, 32)
    assert ad[0] == s0 and np.array_equal(ar, g)
