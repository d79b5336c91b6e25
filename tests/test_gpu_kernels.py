"""GPU parity: libechohip.so kernels vs the oracle on identical seeded inputs.

Integer work (quantizer, block dots, KV int8) must be bit-exact; fp32 outputs
must be within 1e-3 relative L2 of the oracle (the reference's kernels on the
same quantized activations).
"""
import numpy as np
import pytest

from conftest import rel_l2
from echohip import synth
from echohip.lib import Q8_0

pytestmark = pytest.mark.gpu

TOL = 1e-3


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def empty(n, dtype):
    import torch
    return torch.zeros(n, dtype=dtype, device="cuda")


# ------------------------------------------------------------------ quantizer
@pytest.mark.parametrize("width", [4, 8, 12, 16, 32, 37, 256, 1024])
def test_quantize_rows_bit_exact(hip, oc, golden, width):
    import torch
    x = golden[f"quant_w{width}_x"]
    rows = x.size // width
    q = empty(x.size, torch.int8)
    s = empty(rows, torch.float32)
    hip.quantize_rows(dev(x), q, s, rows, width)
    assert np.array_equal(host(q), golden[f"quant_w{width}_q"])
    assert np.array_equal(host(s).view(np.uint32), golden[f"quant_w{width}_s"].view(np.uint32))


def test_quantize_rows_ties_zero(hip, golden):
    import torch
    x = golden["quant_ties_x"]
    q = empty(x.size, torch.int8)
    s = empty(1, torch.float32)
    hip.quantize_rows(dev(x), q, s, 1, x.size)
    assert np.array_equal(host(q), golden["quant_ties_q"])
    z = np.zeros(32, np.float32)
    q = empty(32, torch.int8)
    hip.quantize_rows(dev(z), q, s, 1, 32)
    assert host(s)[0] == 1.0 and not host(q).any()


# --------------------------------------------------------- decode matvec core
def _prep(hip, fmt, W, X):
    """Upload GGUF weights, repack, quantize M activation rows."""
    import torch
    N = W.shape[0]
    M, K = X.shape
    Wd = dev(W)
    tiled = empty(hip.tiled_bytes(fmt, N, K), torch.uint8)
    hip.repack(fmt, Wd, tiled, N, K)
    act = empty(hip.act_bytes(fmt, M, K), torch.uint8)
    hip.quantize_act(fmt, dev(X.astype(np.float32)), act, M, K)
    return tiled, act


def _unpack(hip, fmt, act, M, K):
    import torch
    xq = empty(M * K, torch.int8)
    xd = empty(M * K // 32, torch.float32)
    hip.act_unpack(fmt, act, xq, xd, M, K)
    return host(xq).reshape(M, K), host(xd).reshape(M, K // 32)


# (16, 64, 9216): 72 chunks per tile at 16 tokens, where a workgroup's LDS
# (waves x staged activation) must be capped below 160 KB.
CASES = [(1, 48, 512), (3, 40, 384), (8, 64, 2560), (16, 16, 256), (5, 33, 1024), (16, 64, 9216), (1, 40, 384),
         (1, 16, 9216), (1, 24, 160)]


@pytest.mark.parametrize("M,N,K", CASES)
def test_q8_0_act_and_block_dots_bit_exact(hip, oc, M, N, K):
    import torch
    W = synth.q8_0_blocks(1000 + K, N, K)
    X = synth.activations(2000 + M, M * K).reshape(M, K)
    tiled, act = _prep(hip, 6, W, X)
    xq, xd = _unpack(hip, 6, act, M, K)
    dots = empty(M * N * (K // 32), torch.int32)
    hip.block_dots(6, tiled, act, dots, M, N, K)
    dots = host(dots).reshape(M, N, K // 32)
    for m in range(M):
        rq, rd = oc.quantize_act_q8_0(X[m])
        assert np.array_equal(xq[m], rq)
        assert np.array_equal(xd[m].view(np.uint32), rd.view(np.uint32))
        assert np.array_equal(dots[m], oc.block_dots_q8_0(W, rq))


@pytest.mark.parametrize("M,N,K", CASES)
def test_q8_0_matvec(hip, oc, M, N, K):
    import torch
    W = synth.q8_0_blocks(3000 + K, N, K)
    X = synth.activations(4000 + M, M * K).reshape(M, K)
    tiled, act = _prep(hip, 6, W, X)
    y0 = synth.activations(5, M * N).reshape(M, N)
    y = dev(y0)
    hip.matvec(6, tiled, act, y, M, N, K, accumulate=True)
    y = host(y)
    for m in range(M):
        rq, rd = oc.quantize_act_q8_0(X[m])
        ref = oc.matvec_q8_0(W, oc.dequant_act_q8_0(rq, rd), y0[m])
        assert rel_l2(y[m], ref) < TOL
        assert rel_l2(y[m] - y0[m], ref - y0[m]) < 1e-5
    # overwrite mode
    y2 = dev(np.full((M, N), 7.0, np.float32))
    hip.matvec(6, tiled, act, y2, M, N, K, accumulate=False)
    assert np.allclose(host(y2), y - y0, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("M,N,K,ns", [(8, 40, 4096, 4), (8, 64, 9216, 6), (3, 33, 992, 8), (1, 48, 512, 1),
                                      (16, 16, 384, 3), (5, 20, 2560, 20)])
def test_q8_0_matvec_split(hip, oc, M, N, K, ns):
    """parts[sp] = the matvec over 128-element chunks [sp*nG/ns, (sp+1)*nG/ns) of K."""
    import torch
    W = synth.q8_0_blocks(6000 + K, N, K)
    X = synth.activations(7000 + M, M * K).reshape(M, K)
    tiled, act = _prep(hip, 6, W, X)
    parts = dev(np.full((ns, M, N), 3.0, np.float32))
    hip.matvec_split(6, tiled, act, parts, M, N, K, ns)
    parts = host(parts).reshape(ns, M, N)
    nG = -(-K // 128)
    Wb = W.reshape(N, K // 32, 34)
    for m in range(M):
        rq, rd = oc.quantize_act_q8_0(X[m])
        xdq = oc.dequant_act_q8_0(rq, rd)
        for sp in range(ns):
            b0, b1 = 4 * (sp * nG // ns), min(K // 32, 4 * ((sp + 1) * nG // ns))
            ref = oc.matvec_q8_0(np.ascontiguousarray(Wb[:, b0:b1]).reshape(N, -1), xdq[32 * b0:32 * b1])
            assert rel_l2(parts[sp, m], ref) < 1e-5, (m, sp)
    y = empty(M * N, torch.float32)
    hip.matvec(6, tiled, act, y, M, N, K)
    assert rel_l2(parts.sum(0), host(y).reshape(M, N)) < 1e-6


def test_q8_0_matvec_split_rejects_bad_arguments(hip):
    import torch
    from echohip.lib import EchoHipError
    W = synth.q8_0_blocks(1, 16, 256)
    tiled, act = _prep(hip, 6, W, synth.activations(2, 256).reshape(1, 256))
    parts = empty(4 * 16, torch.float32)
    with pytest.raises(EchoHipError):
        hip.matvec_split(6, tiled, act, parts, 1, 16, 256, 3)  # 2 chunks of 128
    with pytest.raises(EchoHipError):
        hip.matvec_split(6, tiled, act, parts, 1, 16, 256, 0)
    with pytest.raises(EchoHipError):
        hip.matvec_split(10, tiled, act, parts, 1, 16, 256, 1)  # Q4_K


@pytest.mark.parametrize("M,N,K", [(1, 48, 512), (3, 40, 768), (8, 64, 2560), (16, 16, 256)])
def test_q4_K_act_and_block_dots_bit_exact(hip, oc, M, N, K):
    import torch
    W = synth.q4_K_blocks(5000 + K, N, K)
    X = synth.activations(6000 + M, M * K).reshape(M, K)
    tiled, act = _prep(hip, 10, W, X)
    xq, xd = _unpack(hip, 10, act, M, K)
    dots = empty(M * N * (K // 32), torch.int32)
    hip.block_dots(10, tiled, act, dots, M, N, K)
    dots = host(dots).reshape(M, N, K // 32)
    for m in range(M):
        rq, rd, _ = oc.quantize_act_q4_K(X[m])
        assert np.array_equal(xq[m], rq)
        assert np.array_equal(xd[m].view(np.uint32), rd.view(np.uint32))
        assert np.array_equal(dots[m], oc.block_dots_q4_K(W, rq))


@pytest.mark.parametrize("M,N,K", [(1, 48, 512), (3, 40, 768), (8, 64, 2560), (16, 16, 256), (1, 40, 768),
                                   (1, 16, 9216), (1, 48, 256), (16, 4112, 512)])
def test_q4_K_matvec(hip, oc, M, N, K):
    """M = 1 takes the direct-load MFMA kernel (one wave per tile at K = 256: the direct store; 12 waves at
    9216; a ragged last tile at N = 40); M > 1 the LDS-staged MFMA kernel, at 16 x 4112 x 512 with two tiles
    per wave (129 workgroups, the last one's second tile past the end: read, not stored)."""
    W = synth.q4_K_blocks(7000 + K, N, K)
    X = synth.activations(8000 + M, M * K).reshape(M, K)
    tiled, act = _prep(hip, 10, W, X)
    y0 = synth.activations(9, M * N).reshape(M, N)
    y = dev(y0)
    hip.matvec(10, tiled, act, y, M, N, K, accumulate=True)
    y = host(y)
    for m in range(M):
        rq, rd, _ = oc.quantize_act_q4_K(X[m])
        ref = oc.matvec_q4_K(W, oc.dequant_act_q4_K(rq, rd), y0[m])
        assert rel_l2(y[m] - y0[m], ref - y0[m]) < TOL


# ------------------------------------------------- full benchmark shapes (M=1)
@pytest.mark.parametrize("fmt,N,K", [(6, 9216, 2560), (10, 9216, 2560), (10, 2560, 9216)])
def test_full_shape_matvec(hip, oc, fmt, N, K):
    """The measured shapes: every int32 block dot bit-exact, y within 1e-3."""
    import torch
    W = synth.q8_0_blocks(0, N, K) if fmt == 6 else synth.q4_K_blocks(0, N, K)
    x = synth.activations(1, K)
    tiled, act = _prep(hip, fmt, W, x[None])
    dots = empty(N * (K // 32), torch.int32)
    hip.block_dots(fmt, tiled, act, dots, 1, N, K)
    y = empty(N, torch.float32)
    hip.matvec(fmt, tiled, act, y, 1, N, K)
    dots, y = host(dots).reshape(N, K // 32), host(y)
    if fmt == 6:
        rq, rd = oc.quantize_act_q8_0(x)
        assert np.array_equal(dots, oc.block_dots_q8_0(W, rq))
        ref = oc.matvec_q8_0(W, oc.dequant_act_q8_0(rq, rd))
    else:
        rq, rd, _ = oc.quantize_act_q4_K(x)
        assert np.array_equal(dots, oc.block_dots_q4_K(W, rq))
        ref = oc.matvec_q4_K(W, oc.dequant_act_q4_K(rq, rd))
    assert rel_l2(y, ref) < TOL


# ------------------------------------------------ reference-semantics fp32 path
def test_gguf_f32_matvec_golden(hip, golden):
    x, y0 = golden["mv_x"], golden["mv_y0"]
    for fmt, key in ((6, "q8"), (10, "q4")):
        W = golden[f"{key}_W"]
        y = dev(y0)
        hip.matvec_gguf_f32(fmt, dev(W), dev(x), y, W.shape[0], x.size)
        assert rel_l2(host(y), golden[f"{key}_matvec"]) < 1e-5


def test_dequant_dot_int8_golden(hip, golden):
    import torch
    out = empty(64, torch.float32)
    hip.dequant_dot_int8(dev(golden["int8dot_q"]), dev(golden["int8dot_k"]), dev(golden["int8dot_s"]), out, 256, 64)
    ref = golden["int8dot_out"]
    assert np.max(np.abs(host(out) - ref)) < 1e-4 * max(1.0, float(np.max(np.abs(ref))))


def test_dequantize_to_fp16(hip, golden):
    import torch
    W = golden["q8_W"]
    out = empty(W.shape[0] * 512, torch.float16)
    hip.dequantize_to_fp16(6, dev(W), out, W.shape[0] * 512)
    blk = W.reshape(-1, 34)
    ref = (blk[:, 0:2].copy().view(np.float16).astype(np.float32) * blk[:, 2:].view(np.int8)).astype(np.float16)
    assert np.array_equal(host(out).view(np.uint16), ref.reshape(-1).view(np.uint16))


# ------------------------------------------------------------ KV + attention
def _kv_case(oc, n_seq, ctxs, max_ctx, n_kv, hd, seed):
    keys = np.zeros((n_seq, max_ctx * n_kv * hd), np.int8)
    vals = np.zeros_like(keys)
    ks = np.zeros((n_seq, max_ctx * n_kv), np.float32)
    vs = np.zeros_like(ks)
    kf, vf = [], []
    for s in range(n_seq):
        k = synth.activations(seed + 2 * s, ctxs[s] * n_kv * hd).reshape(ctxs[s], n_kv * hd)
        v = synth.activations(seed + 2 * s + 1, ctxs[s] * n_kv * hd).reshape(ctxs[s], n_kv * hd)
        for p in range(ctxs[s]):
            oc.kv_append(k[p], v[p], keys[s], vals[s], ks[s], vs[s], p, n_kv, hd)
        kf.append(k)
        vf.append(v)
    return keys, vals, ks, vs, kf, vf


def test_kv_append_bit_exact(hip, oc):
    import torch
    n_seq, max_ctx, n_kv, hd = 3, 8, 4, 256
    keys_r, vals_r, ks_r, vs_r, kf, vf = _kv_case(oc, n_seq, [5, 8, 2], max_ctx, n_kv, hd, 11)
    keys = empty(n_seq * max_ctx * n_kv * hd, torch.int8)
    vals = empty(n_seq * max_ctx * n_kv * hd, torch.int8)
    ks = empty(n_seq * max_ctx * n_kv, torch.float32)
    vs = empty(n_seq * max_ctx * n_kv, torch.float32)
    for p in range(max_ctx):
        pos = np.array([p if p < c else -1 for c in (5, 8, 2)], np.int32)
        k = np.stack([kf[s][min(p, len(kf[s]) - 1)] for s in range(n_seq)])
        v = np.stack([vf[s][min(p, len(vf[s]) - 1)] for s in range(n_seq)])
        hip.kv_append(dev(k), dev(v), keys, vals, ks, vs, dev(pos), n_seq, max_ctx * n_kv * hd, n_kv, hd)
    assert np.array_equal(host(keys).reshape(n_seq, -1), keys_r)
    assert np.array_equal(host(vals).reshape(n_seq, -1), vals_r)
    assert np.array_equal(host(ks).reshape(n_seq, -1).view(np.uint32), ks_r.view(np.uint32))
    assert np.array_equal(host(vs).reshape(n_seq, -1).view(np.uint32), vs_r.view(np.uint32))


@pytest.mark.parametrize("ctxs,max_ctx,n_heads,n_kv,hd", [
    ([1], 1, 16, 4, 256), ([7], 7, 16, 4, 256), ([512], 512, 16, 4, 256), ([4096], 4096, 16, 4, 256),
    ([300, 1, 0, 777], 800, 16, 4, 256), ([65, 130], 200, 4, 4, 256), ([129, 64], 192, 8, 4, 256),
    ([333], 400, 32, 4, 256), ([200, 0], 256, 8, 2, 128),
    # 66 chunks of 64 x 4 kv heads x 8 sequences >= 2048 workgroups: 128-position chunks
    ([4200, 1, 0, 129, 128, 127, 4000, 2050], 4200, 16, 4, 256),
    # more than 16 sequences: q packed by a separate pass, not by each workgroup
    ([5 + 37 * i for i in range(20)], 720, 16, 4, 256),
    # one long sequence: 516 chunks of 64 x 4 kv heads >= 2048 workgroups, so
    # 128-position chunks, and the merge in four 64-dim slices (16 pairs)
    ([33000], 33000, 16, 4, 256)])
def test_attention_decode(hip, oc, ctxs, max_ctx, n_heads, n_kv, hd):
    """16/4 heads and 4/4, 8/4 run the int8-MFMA kernel; 32/4 and head_dim 128 the VALU kernel."""
    import torch
    n_seq = len(ctxs)
    keys, vals, ks, vs, _, _ = _kv_case(oc, n_seq, ctxs, max_ctx, n_kv, hd, 50)
    q = synth.activations(77, n_seq * n_heads * hd).reshape(n_seq, n_heads * hd)
    out = empty(n_seq * n_heads * hd, torch.float32)
    ws = empty(hip.attn_ws_bytes(n_seq, n_heads, hd, max_ctx), torch.uint8)
    hip.attn_decode(dev(q), dev(keys), dev(vals), dev(ks), dev(vs), out, dev(np.array(ctxs, np.int32)), n_seq,
                    max_ctx * n_kv * hd, n_heads, n_kv, hd, max_ctx, ws)
    out = host(out).reshape(n_seq, n_heads, hd)
    for s in range(n_seq):
        if ctxs[s] == 0:
            assert not out[s].any()
            continue
        ref = oc.attn_decode(q[s], keys[s], vals[s], ks[s], vs[s], n_heads, n_kv, hd, ctxs[s])
        err = rel_l2(out[s], ref)
        print(f"seq {s} ctx {ctxs[s]}: rel_l2 {err:.2e}")
        assert err < TOL


@pytest.mark.parametrize("T,pos0,n_heads,n_kv", [(64, 0, 16, 4), (100, 333, 16, 4), (1, 0, 16, 4), (37, 5, 8, 4),
                                                  (20, 64, 4, 4), (512, 3584, 16, 4), (24, 16000, 16, 4),
                                                  (128, 3968, 16, 4)])
def test_attention_prefill(hip, oc, T, pos0, n_heads, n_kv):
    """Causal chunk attention (ec_attn_prefill): query t at position pos0 + t
    against the oracle's decode attention over pos0 + t + 1 positions, every
    token within 1e-5 (partial key blocks, partial query groups, GQA 4:1, 2:1
    and 1:1, a 512-token chunk at 3584, 24 tokens after 16000 positions),
    with the walk cut into merged segments (workspace) and in one pass."""
    import torch
    hd, max_ctx = 256, pos0 + T + 3
    ctx = pos0 + T
    keys, vals, ks, vs, _, _ = _kv_case(oc, 1, [ctx], max_ctx, n_kv, hd, 90 + T)
    q = synth.activations(91 + pos0, T * n_heads * hd).reshape(T, n_heads * hd)
    nws = hip.attn_prefill_ws_bytes(T, n_heads, max_ctx)
    ws = empty(max(nws, 16), torch.uint8)
    outs = {}
    for tag, w in (("segments", ws), ("one pass", None)):
        out = dev(np.full(T * n_heads * hd, 7.0, np.float32))
        hip.attn_prefill(dev(q), dev(keys[0]), dev(vals[0]), dev(ks[0]), dev(vs[0]), out, T, pos0, n_heads, n_kv, hd,
                         max_ctx, ws=w)
        outs[tag] = host(out).reshape(T, n_heads * hd)
    for tag, out in outs.items():
        worst = 0.0
        for t in range(T):
            ref = oc.attn_decode(q[t], keys[0], vals[0], ks[0], vs[0], n_heads, n_kv, hd, pos0 + t + 1)
            e = rel_l2(out[t], ref)
            worst = max(worst, e)
            assert e < 1e-5, (tag, t, e)
        print(f"T {T} pos0 {pos0} ({tag}, workspace {nws} B): worst per-token rel_l2 {worst:.2e}")


def _pack_q_pieces(q, n_heads, n_kv):
    """q [n_seq][n_heads*256] -> the three-piece int8 A-operand layout of
    ec_attn_decode_packed: per (seq, kv head) [3G rows][4 k-groups][64 bytes],
    row p*G+g = piece p of head kvh + n_kv*g; byte 8m+e of k-group g' is dim
    16g' + 64(m//2) + 8(m%2) + e.  Scales s0 = max|q|/127, s_{p+1} = s_p/254."""
    n_seq, G = q.shape[0], n_heads // n_kv
    qa = np.zeros((n_seq, n_kv, 3 * G, 4, 64), np.int8)
    qs = np.zeros((n_seq, n_kv, 3 * G), np.float32)
    d = np.arange(256)
    gq, at = (d % 64) // 16, (2 * (d // 64) + (d % 16) // 8) * 8 + d % 8
    for s in range(n_seq):
        for head in range(n_heads):
            kvh, g = head % n_kv, head // n_kv
            r = q[s, head * 256:(head + 1) * 256].astype(np.float64)
            step = np.abs(r).max() / 127.0 or 1.0
            for pc in range(3):
                qi = np.clip(np.rint(r / step), -127, 127)
                qa[s, kvh, pc * G + g, gq, at] = qi
                qs[s, kvh, pc * G + g] = step
                r = r - qi * step
                step /= 254.0
    return qa.reshape(-1), qs.reshape(-1)


@pytest.mark.parametrize("ctxs,n_heads,n_kv", [([300, 1, 0, 777], 16, 4), ([65, 200, 64], 8, 4)])
def test_attention_decode_packed_fused_act(hip, oc, ctxs, n_heads, n_kv):
    """Pre-packed q, and the merged output quantized straight into the Q8_0
    activation layout: the activation must equal ec_quantize_act of the output."""
    import torch
    hd, max_ctx, n_seq = 256, 800, len(ctxs)
    keys, vals, ks, vs, _, _ = _kv_case(oc, n_seq, ctxs, max_ctx, n_kv, hd, 51)
    q = synth.activations(78, n_seq * n_heads * hd).reshape(n_seq, n_heads * hd)
    qa, qs = _pack_q_pieces(q, n_heads, n_kv)
    assert qa.size == hip.attn_qa_bytes(n_seq, n_heads)
    out = empty(n_seq * n_heads * hd, torch.float32)
    K = n_heads * hd
    act = empty(hip.act_bytes(Q8_0, n_seq, K), torch.uint8)
    ws = empty(hip.attn_ws_bytes(n_seq, n_heads, hd, max_ctx), torch.uint8)
    hip.attn_decode_packed(dev(qa), dev(qs), dev(keys), dev(vals), dev(ks), dev(vs), out, act,
                           dev(np.array(ctxs, np.int32)), n_seq, max_ctx * n_kv * hd, n_heads, n_kv, max_ctx, ws)
    act2 = empty(hip.act_bytes(Q8_0, n_seq, K), torch.uint8)
    hip.quantize_act(Q8_0, out, act2, n_seq, K)
    assert np.array_equal(host(act), host(act2))
    out = host(out).reshape(n_seq, n_heads, hd)
    for s in range(n_seq):
        if ctxs[s] == 0:
            assert not out[s].any()
            continue
        ref = oc.attn_decode(q[s], keys[s], vals[s], ks[s], vs[s], n_heads, n_kv, hd, ctxs[s])
        assert rel_l2(out[s], ref) < 1e-5


# ------------------------------------------------------------------- delta-net
@pytest.mark.parametrize("T,n_seq,n_v,n_k", [(1, 1, 32, 32), (16, 2, 32, 16), (64, 1, 4, 4)])
def test_deltanet(hip, oc, T, n_seq, n_v, n_k):
    d = 128
    rng = np.random.default_rng(T + n_v)
    S0 = (rng.standard_normal((n_seq, n_v, d, d)) * 0.02).astype(np.float32)  # reference layout [k][v]
    q = rng.standard_normal((T, n_seq, n_k, d)).astype(np.float32)
    k = rng.standard_normal((T, n_seq, n_k, d)).astype(np.float32)
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((T, n_seq, n_v, d)).astype(np.float32)
    dec = synth.sigmoid(rng.normal(2, 0.5, (T, n_seq, n_v))).astype(np.float32)
    bet = synth.sigmoid(rng.normal(0, 1, (T, n_seq, n_v))).astype(np.float32)
    state = dev(np.ascontiguousarray(S0.transpose(0, 1, 3, 2)))  # device layout [v][k]
    import torch
    out = empty(T * n_seq * n_v * d, torch.float32)
    hip.deltanet(state, dev(q), dev(k), dev(v), dev(dec), dev(bet), out, T, n_seq, n_v, n_k, d, d)
    out = host(out).reshape(T, n_seq, n_v, d)
    S = host(state).reshape(n_seq, n_v, d, d).transpose(0, 1, 3, 2)
    Sr = S0.copy()
    ref_o = np.zeros_like(out)
    for t in range(T):
        for s in range(n_seq):
            ref_o[t, s] = oc.deltanet_step(Sr[s], q[t, s], k[t, s], v[t, s], dec[t, s], bet[t, s], n_v, n_k, d, d)
    assert rel_l2(out, ref_o) < TOL
    assert rel_l2(S, Sr) < TOL


def test_deltanet_1024_tokens_32_heads(hip, oc):
    """The 1024-token delta-net workload at full size: 32 heads, d_k = d_v = 128, S0 ~ N(0, 0.02^2), q and k
    L2-normalised N(0,1), v ~ N(0,1), decay = sigmoid(N(2, 0.5)), beta = sigmoid(N(0, 1)); all 1024 tokens in one
    launch with the state on chip, against 1024 sequential oracle steps: every token's output and the final
    state within 1e-3 relative L2 (fp32 rounding differences accumulate through the recurrence)."""
    import torch
    T, n_v, d = 1024, 32, 128
    rng = np.random.default_rng(1024)
    S0 = (rng.standard_normal((n_v, d, d)) * 0.02).astype(np.float32)  # reference layout [k][v]
    q = rng.standard_normal((T, n_v, d)).astype(np.float32)
    k = rng.standard_normal((T, n_v, d)).astype(np.float32)
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((T, n_v, d)).astype(np.float32)
    dec = synth.sigmoid(rng.normal(2, 0.5, (T, n_v))).astype(np.float32)
    bet = synth.sigmoid(rng.normal(0, 1, (T, n_v))).astype(np.float32)
    state = dev(np.ascontiguousarray(S0.transpose(0, 2, 1)))  # device layout [v][k]
    out = empty(T * n_v * d, torch.float32)
    hip.deltanet(state, dev(q), dev(k), dev(v), dev(dec), dev(bet), out, T, 1, n_v, n_v, d, d)
    out = host(out).reshape(T, n_v, d)
    S = host(state).reshape(n_v, d, d).transpose(0, 2, 1)
    Sr = S0.copy()
    worst = 0.0
    for t in range(T):
        ref = oc.deltanet_step(Sr, q[t], k[t], v[t], dec[t], bet[t], n_v, n_v, d, d)
        e = rel_l2(out[t], ref)
        worst = max(worst, e)
        assert e < 1e-3, (t, e)
    es = rel_l2(S, Sr)
    print(f"1024 tokens: worst per-token output rel_l2 {worst:.2e}, final state rel_l2 {es:.2e}")
    assert es < 1e-3


def _dn_inputs(T, n_seq, n_v, n_k, seed, d=128):
    rng = np.random.default_rng(seed)
    S0 = (rng.standard_normal((n_seq, n_v, d, d)) * 0.02).astype(np.float32)  # reference layout [k][v]
    q = rng.standard_normal((T, n_seq, n_k, d)).astype(np.float32)
    k = rng.standard_normal((T, n_seq, n_k, d)).astype(np.float32)
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((T, n_seq, n_v, d)).astype(np.float32)
    dec = synth.sigmoid(rng.normal(2, 0.5, (T, n_seq, n_v))).astype(np.float32)
    bet = synth.sigmoid(rng.normal(0, 1, (T, n_seq, n_v))).astype(np.float32)
    return S0, q, k, v, dec, bet


@pytest.mark.parametrize("T,n_seq,n_v,n_k,zero_decay", [(1, 1, 4, 4, False), (64, 1, 4, 4, False),
                                                        (200, 2, 4, 2, False), (130, 3, 2, 1, True)])
def test_deltanet_chunked(hip, oc, T, n_seq, n_v, n_k, zero_decay):
    """Chunked scan (64-token chunks, a partial last chunk, GQA head sharing,
    several sequences, the last one skipped by seq_pos) against the oracle's
    token loop; zero_decay: a few tokens with decay exactly 0 (the state is
    reset there)."""
    import torch
    d = 128
    S0, q, k, v, dec, bet = _dn_inputs(T, n_seq, n_v, n_k, 7 * T + n_v)
    if zero_decay:
        dec[[0, 63, 64, 100]] = 0.0
    state = dev(np.ascontiguousarray(S0.transpose(0, 1, 3, 2)))  # device layout [v][k]
    out = dev(np.full(T * n_seq * n_v * d, 7.0, np.float32))
    ws = empty(hip.deltanet_chunked_ws_bytes(T, n_seq, n_v), torch.uint8)
    seq_pos = np.zeros(n_seq, np.int32)
    if n_seq > 2:
        seq_pos[-1] = -1
    hip.deltanet_chunked(state, dev(q), dev(k), dev(v), dev(dec), dev(bet), out, T, n_seq, n_v, n_k, d, d, ws,
                         seq_pos=dev(seq_pos))
    out = host(out).reshape(T, n_seq, n_v, d)
    S = host(state).reshape(n_seq, n_v, d, d).transpose(0, 1, 3, 2)
    for s in range(n_seq):
        if seq_pos[s] < 0:
            assert np.array_equal(S[s], S0[s]) and np.all(out[:, s] == 7.0)
            continue
        Sr = S0[s].copy()
        for t in range(T):
            ref = oc.deltanet_step(Sr, q[t, s], k[t, s], v[t, s], dec[t, s], bet[t, s], n_v, n_k, d, d)
            assert rel_l2(out[t, s], ref) < TOL, (s, t, rel_l2(out[t, s], ref))
        assert rel_l2(S[s], Sr) < TOL


def test_deltanet_chunked_1024_tokens_32_heads(hip, oc):
    """The 1024-token, 32-head workload through the chunked scan: every token's
    output and the final state within 1e-3 of 1024 sequential oracle steps, and
    within 1e-4 of the GPU token loop (ec_deltanet)."""
    import torch
    T, n_v, d = 1024, 32, 128
    S0, q, k, v, dec, bet = _dn_inputs(T, 1, n_v, n_v, 1024)
    S0 = S0[0]
    st_c = dev(np.ascontiguousarray(S0.transpose(0, 2, 1)))
    st_t = dev(np.ascontiguousarray(S0.transpose(0, 2, 1)))
    out_c = empty(T * n_v * d, torch.float32)
    out_t = empty(T * n_v * d, torch.float32)
    ws = empty(hip.deltanet_chunked_ws_bytes(T, 1, n_v), torch.uint8)
    args = (dev(q), dev(k), dev(v), dev(dec), dev(bet))
    hip.deltanet_chunked(st_c, *args, out_c, T, 1, n_v, n_v, d, d, ws)
    hip.deltanet(st_t, *args, out_t, T, 1, n_v, n_v, d, d)
    oc_, ot = host(out_c).reshape(T, n_v, d), host(out_t).reshape(T, n_v, d)
    S = host(st_c).reshape(n_v, d, d).transpose(0, 2, 1)
    assert rel_l2(oc_, ot) < 1e-4 and rel_l2(host(st_c), host(st_t)) < 1e-4
    Sr = S0.copy()
    worst = 0.0
    for t in range(T):
        ref = oc.deltanet_step(Sr, q[t, 0], k[t, 0], v[t, 0], dec[t, 0], bet[t, 0], n_v, n_v, d, d)
        e = rel_l2(oc_[t], ref)
        worst = max(worst, e)
        assert e < 1e-3, (t, e)
    es = rel_l2(S, Sr)
    print(f"chunked 1024 tokens: worst per-token output rel_l2 {worst:.2e}, final state rel_l2 {es:.2e}")
    assert es < 1e-3


@pytest.mark.parametrize("fmt,N,K", [(6, 9216, 2560), (6, 2560, 9216), (6, 1000, 4096), (6, 77, 96), (6, 2563, 9216),
                                     (6, 1030, 13312), (6, 333, 512), (6, 500, 1088), (6, 130, 320), (6, 700, 11008),
                                     (6, 300, 16384), (6, 16401, 1024),
                                     (10, 9216, 2560), (10, 2560, 9216), (10, 333, 512), (10, 1001, 4096),
                                     (10, 2563, 9216), (10, 1030, 13312), (10, 700, 11008), (10, 130, 16640)])
def test_gguf_f32_matvec_full_shapes(hip, oc, fmt, N, K):
    """The reference-signature path (GGUF bytes in place, fp32 activations, y += W x) at the matvec workloads'
    full shapes, ragged row counts and a K whose rows are not 16-byte aligned (K = 96: per-row kernel), against
    the oracle's reference-order matvec: within 1e-5 relative L2 (fp32 summation order only).
    Q4_K: every rows-per-thread variant (1 row: 9216 x 2560, 2560 x 9216, 2563 x 9216 with a last tile of 3 of
    4 rows; 2 rows: 1030 x 13312, whose 832 threads exceed the 4-row variant's bound; 4 rows: 333 x 512,
    700 x 11008, 1001 x 4096 with a last tile of 9 of 16 rows) and workgroups padded to whole waves (11008:
    688 threads of 704; 16640: 520 of 576).
    Q8_0 (block pairs, K % 64 == 0): four threads per pair column, raised to fill a wave for narrow rows
    (333 x 512: 8, 130 x 320: 16 with 8 threads per row in the row sums); one row per thread, two at
    16401 x 1024 (one row would mean 4101 workgroups; last tile 1 of 8 rows); workgroups padded to whole waves
    (9216 x 2560: 160 threads of 192, 500 x 1088 -- 17 pairs -- 68 of 128, 700 x 11008: 688 of 704); ragged
    last tiles (2563 x 9216: 3 of 4 rows, 1030 x 13312: 2 of 4, 333 x 512: 5 of 8, 130 x 320: 2 of 16);
    300 x 16384 stages 66 KB of x (above 64 KB of LDS)."""
    W = synth.q8_0_blocks(fmt + N, N, K) if fmt == 6 else synth.q4_K_blocks(fmt + N, N, K)
    x = synth.activations(N + 1, K)
    y0 = synth.activations(N + 2, N)
    y = dev(y0)
    hip.matvec_gguf_f32(fmt, dev(W), dev(x), y, N, K)
    ref = (oc.matvec_q8_0 if fmt == 6 else oc.matvec_q4_K)(W, x, y0)
    assert rel_l2(host(y), ref) < 1e-5
