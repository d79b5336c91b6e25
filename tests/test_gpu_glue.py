"""GPU parity of the decode-step glue ops (glue.hip, deltanet.hip k_delta_step).

The glue ops produce Q8_0 activations, so they are compared after
quantization: scales within 1e-5 relative of the oracle's, and int8 values
equal except where a value sits on a rounding boundary, which moves it by
exactly one quantum.  The reference sums a norm's squares sequentially in
fp32 (engine.zig:787), whose rounding error grows like sqrt(n) ulp (~1e-6
relative at n = 2560); the GPU's tree reduction is closer to the exact sum,
so the two differ by that much.
"""
import numpy as np
import pytest

from conftest import rel_l2
from echohip import synth
from echohip.lib import Q8_0
from test_gpu_kernels import dev, empty, host

pytestmark = pytest.mark.gpu


def _unpack(hip, act, M, K):
    import torch
    xq = empty(M * K, torch.int8)
    xd = empty(M * K // 32, torch.float32)
    hip.act_unpack(Q8_0, act, xq, xd, M, K)
    return host(xq).reshape(M, K), host(xd).reshape(M, K // 32)


def _check_q8(xq, xd, xq_r, xd_r):
    assert np.max(np.abs(xd - xd_r) / np.maximum(np.abs(xd_r), 1e-30)) < 1e-5
    diff = np.abs(xq.astype(np.int32) - xq_r.astype(np.int32))
    assert diff.max() <= 1
    assert (diff != 0).mean() < 1e-3, (diff != 0).sum()


@pytest.mark.parametrize("M,H", [(8, 2560), (3, 256), (1, 384), (16, 128), (2, 5120)])
def test_rmsnorm_quant(hip, oc, M, H):
    import torch
    x = (3.0 * synth.normal(synth.stream_seed(1, H), M * H)).astype(np.float32).reshape(M, H)
    w = (1.0 + 0.1 * synth.normal(synth.stream_seed(2, H), H)).astype(np.float32)
    act = empty(hip.act_bytes(Q8_0, M, H), torch.uint8)
    hip.rmsnorm_quant(dev(x), dev(w), act, M, H)
    xq, xd = _unpack(hip, act, M, H)
    for i in range(M):
        y = np.zeros(H, np.float32)
        oc.lib.oc_rmsnorm(x[i], w, y, H)
        xq_r, xd_r = oc.quantize_act_q8_0(y)
        _check_q8(xq[i], xd[i], xq_r, xd_r)


@pytest.mark.parametrize("use_norms", [True, False])
def test_qk_rope_append_matches_oracle(hip, oc, use_norms):
    """ec_glue_qk_rope_append (fp32 q output): head RMSNorm + RoPE of q and k
    (engine.zig head norms / rope, oracle oc_head_rmsnorm + oc_rope) within
    fp32 rounding (sincosf vs libm, norm summation order); V rows appended bit
    for bit as the oracle's per-token quantizer; K rows within one quantum;
    ctx = pos + 1, and nothing appended for pos < 0 or pos >= max_ctx."""
    import torch
    n_heads, n_kv, HD, max_ctx = 8, 2, 256, 40
    pos = np.array([0, 17, 39, -1, 40], np.int32)
    n_seq = pos.size
    Nin = (n_heads + 2 * n_kv) * HD
    seq_stride = max_ctx * n_kv * HD
    rng = np.random.default_rng(3)
    proj = (2 * rng.standard_normal((n_seq, Nin))).astype(np.float32)
    qn = (1 + 0.1 * rng.standard_normal(HD)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(HD)).astype(np.float32)
    inv = np.zeros(HD // 2, np.float32)
    oc.lib.oc_rope_inv_freq(inv, HD, 10000.0)
    keys = empty(n_seq * seq_stride, torch.int8)
    vals = empty(n_seq * seq_stride, torch.int8)
    ks = empty(n_seq * max_ctx * n_kv, torch.float32)
    vs = empty(n_seq * max_ctx * n_kv, torch.float32)
    ctx = dev(np.full(n_seq, 9, np.int32))
    q_out = empty(n_seq * n_heads * HD, torch.float32)
    hip.qk_rope_append(dev(proj), Nin, dev(qn), dev(kn), use_norms, use_norms, dev(inv), dev(pos), q_out, None, None,
                       keys, vals, ks, vs, ctx, n_seq, seq_stride, max_ctx, n_heads, n_kv, HD)
    assert host(ctx).tolist() == [1, 18, 40, 0, 0]
    qo = host(q_out).reshape(n_seq, n_heads * HD)
    kh = host(keys).reshape(n_seq, max_ctx, n_kv * HD)
    vh = host(vals).reshape(n_seq, max_ctx, n_kv * HD)
    ksh = host(ks).reshape(n_seq, max_ctx, n_kv)
    vsh = host(vs).reshape(n_seq, max_ctx, n_kv)
    for s, p in enumerate(pos.tolist()):
        if p < 0 or p >= max_ctx:
            assert not kh[s].any() and not vh[s].any() and not ksh[s].any()
            continue
        q = proj[s, :n_heads * HD].copy()
        k = proj[s, n_heads * HD:(n_heads + n_kv) * HD].copy()
        v = proj[s, (n_heads + n_kv) * HD:].copy()
        if use_norms:
            oc.lib.oc_head_rmsnorm(q, qn, n_heads, HD)
            oc.lib.oc_head_rmsnorm(k, kn, n_kv, HD)
        oc.lib.oc_rope(q, n_heads, HD, p, inv)
        oc.lib.oc_rope(k, n_kv, HD, p, inv)
        assert rel_l2(qo[s], q) < 2e-6, (s, rel_l2(qo[s], q))
        kr = np.zeros(max_ctx * n_kv * HD, np.int8)
        vr = np.zeros(max_ctx * n_kv * HD, np.int8)
        ksr = np.zeros(max_ctx * n_kv, np.float32)
        vsr = np.zeros(max_ctx * n_kv, np.float32)
        oc.kv_append(k, v, kr, vr, ksr, vsr, p, n_kv, HD)
        kr, vr = kr.reshape(max_ctx, -1), vr.reshape(max_ctx, -1)
        ksr, vsr = ksr.reshape(max_ctx, -1), vsr.reshape(max_ctx, -1)
        assert np.array_equal(vh[s, p], vr[p]) and np.array_equal(vsh[s, p].view(np.uint32), vsr[p].view(np.uint32))
        assert np.abs(kh[s, p].astype(np.int32) - kr[p].astype(np.int32)).max() <= 1
        assert np.max(np.abs(ksh[s, p] - ksr[p]) / ksr[p]) < 1e-5
        others = [t for t in range(max_ctx) if t != p]
        assert not kh[s, others].any() and not vh[s, others].any()


@pytest.mark.parametrize("ns", [2, 3, 8])
def test_rope_append_split_equals_summed_input(hip, ns):
    """ec_glue_qk_rope_append_split over ns partial projections == the one-part
    entry on the parts added in order in fp32, bit for bit (packed q, K/V rows,
    scales, ctx), including an inactive sequence."""
    import torch
    n_heads, n_kv, HD, max_ctx = 16, 4, 256, 24
    pos = np.array([3, -1, 23, 0], np.int32)
    n_seq = pos.size
    Nin = (n_heads + 2 * n_kv) * HD
    seq_stride = max_ctx * n_kv * HD
    rng = np.random.default_rng(12 + ns)
    parts = rng.standard_normal((ns, n_seq, Nin)).astype(np.float32)
    total = parts[0].copy()
    for q in range(1, ns):
        total = total + parts[q]
    qn = dev((1 + 0.1 * rng.standard_normal(HD)).astype(np.float32))
    kn = dev((1 + 0.1 * rng.standard_normal(HD)).astype(np.float32))
    inv = dev((1.0 / 10000.0 ** (np.arange(HD // 2) * 2.0 / HD)).astype(np.float32))
    out = []
    for split in (True, False):
        keys = empty(n_seq * seq_stride, torch.int8)
        vals = empty(n_seq * seq_stride, torch.int8)
        ks = empty(n_seq * max_ctx * n_kv, torch.float32)
        vs = empty(n_seq * max_ctx * n_kv, torch.float32)
        ctx = empty(n_seq, torch.int32)
        qa = empty(hip.attn_qa_bytes(n_seq, n_heads), torch.uint8)
        qs = empty(n_seq * n_heads * 3, torch.float32)
        if split:
            hip.qk_rope_append_split(dev(parts), ns, Nin, qn, kn, 1, 1, inv, dev(pos), None, qa, qs, keys, vals, ks, vs,
                                     ctx, n_seq, seq_stride, max_ctx, n_heads, n_kv, HD)
        else:
            hip.qk_rope_append(dev(total), Nin, qn, kn, 1, 1, inv, dev(pos), None, qa, qs, keys, vals, ks, vs, ctx,
                               n_seq, seq_stride, max_ctx, n_heads, n_kv, HD)
        out.append([host(t).view(np.uint8) for t in (keys, vals, ks, vs, ctx, qa, qs)])
    for a, b in zip(*out):
        assert np.array_equal(a, b)


@pytest.mark.parametrize("ns", [2, 5])
def test_split_inputs_equal_summed_inputs(hip, ns):
    """ec_delta_step_split / ec_glue_swiglu_quant_split over ns partial sums ==
    the one-part entry on the parts added in order in fp32, bit for bit."""
    import torch
    n_seq, n_k, n_v, kern = 3, 2, 4, 4
    key_dim, value_dim = 128 * n_k, 128 * n_v
    conv_dim = 2 * key_dim + value_dim
    Nin = conv_dim + value_dim + 2 * n_v
    rng = np.random.default_rng(9)
    conv_w = dev((0.5 * rng.standard_normal(kern * conv_dim)).astype(np.float32))
    a_log = dev(np.log(1 + 15 * rng.random(n_v)).astype(np.float32))
    dt_bias = dev((0.1 * rng.standard_normal(n_v)).astype(np.float32))
    norm_w = dev((1 + 0.1 * rng.standard_normal(128)).astype(np.float32))
    S0 = (0.02 * rng.standard_normal(n_seq * n_v * 128 * 128)).astype(np.float32)
    ring0 = (0.3 * rng.standard_normal(n_seq * kern * conv_dim)).astype(np.float32)
    parts = rng.standard_normal((ns, n_seq, Nin)).astype(np.float32)
    total = parts[0].copy()
    for q in range(1, ns):
        total = total + parts[q]
    pos = dev(np.array([5, -1, 2], np.int32))
    out = []
    for split in (True, False):
        st, ring = dev(S0), dev(ring0)
        act = empty(hip.act_bytes(Q8_0, n_seq, value_dim), torch.uint8)
        if split:
            hip.delta_step_split(dev(parts), ns, Nin, ring, conv_w, a_log, dt_bias, norm_w, st, act, pos, n_seq, n_k,
                                 n_v, kern)
        else:
            hip.delta_step(dev(total), Nin, ring, conv_w, a_log, dt_bias, norm_w, st, act, pos, n_seq, n_k, n_v, kern)
        out.append([host(st).view(np.uint32), host(ring).view(np.uint32), host(act)])
    for a, b in zip(*out):
        assert np.array_equal(a, b)
    M, F = 5, 384
    gu = rng.standard_normal((ns, M, 2 * F)).astype(np.float32)
    gsum = gu[0].copy()
    for q in range(1, ns):
        gsum = gsum + gu[q]
    a1 = empty(hip.act_bytes(Q8_0, M, F), torch.uint8)
    a2 = empty(hip.act_bytes(Q8_0, M, F), torch.uint8)
    hip.swiglu_quant_split(dev(gu), ns, a1, M, F)
    hip.swiglu_quant(dev(gsum), a2, M, F)
    assert np.array_equal(host(a1), host(a2))


@pytest.mark.parametrize("M,H,ns", [(8, 2560, 6), (8, 2560, 4), (3, 256, 1), (16, 128, 8), (2, 5120, 3)])
def test_add_rmsnorm_quant(hip, oc, M, H, ns):
    """x_out = ((x + p0) + p1) + ... in fp32 (exact order), then RMSNorm + quantize of x_out."""
    import torch
    x = (3.0 * synth.normal(synth.stream_seed(4, H), M * H)).astype(np.float32).reshape(M, H)
    parts = synth.normal(synth.stream_seed(5, ns), ns * M * H).astype(np.float32).reshape(ns, M, H)
    w = (1.0 + 0.1 * synth.normal(synth.stream_seed(2, H), H)).astype(np.float32)
    act = empty(hip.act_bytes(Q8_0, M, H), torch.uint8)
    x_out = empty(M * H, torch.float32)
    hip.add_rmsnorm_quant(dev(x), dev(parts), ns, x_out, dev(w), act, M, H)
    want = x.copy()
    for p in range(ns):
        want = want + parts[p]
    assert np.array_equal(host(x_out).reshape(M, H).view(np.uint32), want.view(np.uint32))
    xq, xd = _unpack(hip, act, M, H)
    for i in range(M):
        y = np.zeros(H, np.float32)
        oc.lib.oc_rmsnorm(want[i], w, y, H)
        xq_r, xd_r = oc.quantize_act_q8_0(y)
        _check_q8(xq[i], xd[i], xq_r, xd_r)


def test_add_rmsnorm_quant_rejects_in_place(hip):
    import torch
    from echohip.lib import EchoHipError
    x = dev(np.ones((2, 128), np.float32))
    act = empty(hip.act_bytes(Q8_0, 2, 128), torch.uint8)
    with pytest.raises(EchoHipError):
        hip.add_rmsnorm_quant(x, dev(np.ones((1, 2, 128), np.float32)), 1, x, dev(np.ones(128, np.float32)), act, 2,
                              128)


@pytest.mark.parametrize("M,F", [(8, 9216), (2, 512), (5, 384)])
def test_swiglu_quant(hip, oc, M, F):
    import torch
    gu = (2.0 * synth.normal(synth.stream_seed(3, F), M * 2 * F)).astype(np.float32).reshape(M, 2 * F)
    act = empty(hip.act_bytes(Q8_0, M, F), torch.uint8)
    hip.swiglu_quant(dev(gu), act, M, F)
    xq, xd = _unpack(hip, act, M, F)
    silu = np.vectorize(oc.lib.oc_silu, otypes=[np.float32])
    for i in range(M):
        y = (silu(gu[i, :F]) * gu[i, F:]).astype(np.float32)
        xq_r, xd_r = oc.quantize_act_q8_0(y)
        _check_q8(xq[i], xd[i], xq_r, xd_r)


def test_delta_step_matches_unfused_ops(hip, oc):
    """ec_delta_step == ec_glue_conv_gates -> ec_deltanet -> ec_glue_gated_norm_quant
    over a ragged 4-step schedule (one sequence joins late, one idles)."""
    import torch
    n_seq, n_k, n_v, kern = 3, 2, 4, 4
    key_dim, value_dim = 128 * n_k, 128 * n_v
    conv_dim = 2 * key_dim + value_dim
    Nin = conv_dim + value_dim + 2 * n_v
    rng = np.random.default_rng(5)
    conv_w = dev((0.5 * rng.standard_normal(kern * conv_dim)).astype(np.float32))
    a_log = dev(np.log(1 + 15 * rng.random(n_v)).astype(np.float32))
    dt_bias = dev((0.1 * rng.standard_normal(n_v)).astype(np.float32))
    norm_w = dev((1 + 0.1 * rng.standard_normal(128)).astype(np.float32))
    S0 = (0.02 * rng.standard_normal(n_seq * n_v * 128 * 128)).astype(np.float32)
    stA, stB = dev(S0), dev(S0)
    cA = empty(n_seq * kern * conv_dim, torch.float32)
    cB = empty(n_seq * kern * conv_dim, torch.float32)
    q = empty(n_seq * key_dim, torch.float32)
    k = empty(n_seq * key_dim, torch.float32)
    v = empty(n_seq * value_dim, torch.float32)
    dec = empty(n_seq * n_v, torch.float32)
    bet = empty(n_seq * n_v, torch.float32)
    core = empty(n_seq * value_dim, torch.float32)
    actA = empty(hip.act_bytes(Q8_0, n_seq, value_dim), torch.uint8)
    actB = empty(hip.act_bytes(Q8_0, n_seq, value_dim), torch.uint8)
    sched = [[0, -1, 0], [1, -1, 1], [2, 0, -1], [3, 1, 2]]
    for step, p in enumerate(sched):
        proj = dev(rng.standard_normal(n_seq * Nin).astype(np.float32))
        pos = dev(np.array(p, np.int32))
        hip.conv_gates(proj, Nin, cA, conv_w, a_log, dt_bias, q, k, v, dec, bet, pos, n_seq, n_k, n_v, kern)
        hip.deltanet(stA, q, k, v, dec, bet, core, 1, n_seq, n_v, n_k, 128, 128, seq_pos=pos)
        hip.gated_norm_quant(core, proj, Nin, conv_dim, norm_w, actA, n_seq, n_v)
        hip.delta_step(proj, Nin, cB, conv_w, a_log, dt_bias, norm_w, stB, actB, pos, n_seq, n_k, n_v, kern)
        assert np.array_equal(host(cA), host(cB)), step
        assert rel_l2(host(stB), host(stA)) < 1e-6, step
        xqA, xdA = _unpack(hip, actA, n_seq, value_dim)
        xqB, xdB = _unpack(hip, actB, n_seq, value_dim)
        for s in range(n_seq):
            if p[s] >= 0:
                _check_q8(xqB[s], xdB[s], xqA[s], xdA[s])


def _argmax_ref(row):
    """First index of the maximum over the non-NaN entries above -inf (the
    reference's strictly-greater scan, engine.zig:860-867); 0 when there is none."""
    best, bi = -np.inf, 0
    ok = ~np.isnan(row) & (row > -np.inf)
    if ok.any():
        best = row[ok].max()
        bi = int(np.flatnonzero(ok & (row == best))[0])
    return bi


@pytest.mark.parametrize("slices", [0, 16, 7, 64])
@pytest.mark.parametrize("vocab", [151936, 151935, 1000, 7, 70001])
def test_argmax_advance_edge_cases(hip, vocab, slices):
    """ec_glue_argmax_advance_bounded (slices = 0) and the two-launch
    ec_glue_argmax_advance_sliced on rows with ties at the maximum (first index
    wins, also across float4 groups, threads and slices), NaNs, -inf, an
    all-NaN and an all -inf row (token 0), -0.0 against +0.0, unaligned rows
    (vocab % 4 != 0), more slices than 4-entry groups (vocab 7: empty slices),
    an inactive sequence (pos < 0: nothing written) and the max_pos bound (a
    sequence whose next position would reach it becomes inactive)."""
    import torch
    rng = np.random.default_rng(vocab)
    rows = []
    r = rng.standard_normal(vocab).astype(np.float32)
    rows.append(r)                                         # plain
    r = rng.standard_normal(vocab).astype(np.float32)
    idx = sorted(rng.choice(vocab, size=min(5, vocab), replace=False))
    r[idx] = 9.0
    rows.append(r)                                         # ties: first of 5
    r = rng.standard_normal(vocab).astype(np.float32)
    r[rng.choice(vocab, size=max(1, vocab // 7), replace=False)] = np.nan
    rows.append(r)                                         # NaNs
    rows.append(np.full(vocab, np.nan, np.float32))        # all NaN
    rows.append(np.full(vocab, -np.inf, np.float32))       # all -inf
    r = np.full(vocab, -1.0, np.float32)
    r[vocab - 1] = 0.0
    r[vocab // 2] = -0.0
    rows.append(r)                                         # -0.0 first, then +0.0: equal, first wins
    r = rng.standard_normal(vocab).astype(np.float32)
    r[0] = np.inf
    r[vocab - 1] = np.inf
    rows.append(r)                                         # +inf twice
    r = rng.standard_normal(vocab).astype(np.float32)
    rows.append(r)                                         # inactive sequence
    n = len(rows)
    logits = torch.from_numpy(np.stack(rows)).cuda()
    max_pos = 100
    pos0 = np.array([5, 6, 7, 8, 9, 10, max_pos - 1, -1], np.int32)
    gen = torch.full((n,), -7, dtype=torch.int32, device="cuda")
    nxt = torch.full((n,), -7, dtype=torch.int32, device="cuda")
    pos = torch.from_numpy(pos0.copy()).cuda()
    ws = torch.empty(max(1, hip.argmax_ws_bytes(n, slices)), dtype=torch.uint8, device="cuda")
    for rep in range(2):  # a second call on the advanced positions
        before = pos.cpu().numpy().copy()
        hip.argmax_advance(logits, vocab, gen, nxt, pos, n, max_pos, slices=slices, ws=ws)
        torch.cuda.synchronize()
        g, q, p = gen.cpu().numpy(), nxt.cpu().numpy(), pos.cpu().numpy()
        for s in range(n):
            if before[s] < 0:
                assert g[s] == (-7 if rep == 0 else g[s]) and p[s] == before[s], s
                continue
            want = _argmax_ref(rows[s])
            assert g[s] == want and q[s] == want, (vocab, s, g[s], want)
            assert p[s] == (before[s] + 1 if before[s] + 1 < max_pos else -1), (s, p[s])
