"""Chunked prefill (ec_engine_prefill and its glue) against the token-by-token path.

* ec_glue_conv_gates_chunk over T tokens == T single-token ec_glue_conv_gates
  steps, bit for bit (q, k, v, decay, beta and the ring left behind), for
  chunks longer and shorter than the conv kernel and starting at position 0.
* The fp32 row ops equal their formulas (engine.zig:783-792, core/math.zig:35-37,
  qwen_linear.zig:252-257) to fp32 rounding.
* A prefilled sequence matches the same prompt fed through the decode graph
  one token per step, both engines with one-piece activations (the prefill
  GEMMs' arithmetic; the decode step's default second piece would add its own
  difference).  This is a consistency check of two GPU paths; parity
  with the oracle is established per operation for both
  (tests/test_gpu_prefill_ops.py, tests/test_gpu_decoder.py, 1e-5 per op).
  The two paths differ only in fp32 summation order (int8-MFMA GEMM vs
  matvec epilogues), so a prompt agrees to fp32 rounding unless an activation
  lands on an int8 rounding boundary in one path: it then moves by one
  quantum and the recurrent state carries the difference until it decays.
  Measured on MI355X: prompts of 1, 3, 7 and 25 tokens (and 7, 40 mixed)
  agree within 2e-7; 40..1100-token prompts over four seeds differ by
  7e-3..1.2e-2 in the logits and at most 6.9e-3 in the fp32 states.  States
  and logits are held to PATH_TOL = 2e-2 (KV caches dequantized), the first
  KV position within one quantum; prompts of 1, 3, 7, 25, 40 and 600 tokens
  (two 512-token chunks), followed by decode steps on both engines.
"""
import numpy as np
import pytest

from conftest import rel_l2
from decoder_util import MIXED_FMTS, make_model, small_config, upload
from echohip import synth
from test_gpu_kernels import dev, empty, host

pytestmark = pytest.mark.gpu

PATH_TOL = 2e-2  # prefill vs token loop, one-quantum flips carried (measured <= 1.2e-2)


@pytest.mark.parametrize("T,p0,zero_ring,kern", [(7, 5, False, 4), (2, 9, False, 4), (6, 0, True, 4),
                                                  (3, 1, True, 4), (1, 12, False, 4), (20, 3, False, 4),
                                                  (17, 0, True, 4), (20, 5, False, 3), (9, 6, False, 5)])
def test_conv_gates_chunk_equals_single_steps(hip, T, p0, zero_ring, kern):
    """Four taps take the register-window kernel, other tap counts the
    one-token-per-iteration kernel; both bit-identical to single steps."""
    import torch
    n_k, n_v = 2, 4
    Nin = 2 * n_k * 128 + 2 * n_v * 128 + 2 * n_v
    conv_dim = 2 * n_k * 128 + n_v * 128
    proj = synth.normal(synth.stream_seed(1, T), T * Nin).astype(np.float32).reshape(T, Nin)
    ring0 = np.zeros((kern, conv_dim), np.float32) if zero_ring else \
        synth.normal(synth.stream_seed(2, p0), kern * conv_dim).astype(np.float32).reshape(kern, conv_dim)
    conv_w = (0.5 * synth.normal(synth.stream_seed(3, 0), kern * conv_dim)).astype(np.float32)
    a_log = np.log(1 + 15 * synth.uniform01(synth.stream_seed(4, 0), n_v)).astype(np.float32)
    dt_bias = (0.1 * synth.normal(synth.stream_seed(5, 0), n_v)).astype(np.float32)
    outs = lambda: [empty(T * n_k * 128, torch.float32), empty(T * n_k * 128, torch.float32),  # noqa: E731
                    empty(T * n_v * 128, torch.float32), empty(T * n_v, torch.float32), empty(T * n_v, torch.float32)]
    ring_c = dev(ring0)
    qc, kc, vc, dc, bc = outs()
    hip.conv_gates_chunk(dev(proj), Nin, ring_c, dev(conv_w), dev(a_log), dev(dt_bias), qc, kc, vc, dc, bc, T, p0,
                         n_k, n_v, kern)
    ring_s = dev(ring0)
    qs, ks, vs, ds, bs = outs()
    cw, al, dtb = dev(conv_w), dev(a_log), dev(dt_bias)
    for t in range(T):
        pos = dev(np.array([p0 + t], np.int32))
        hip.conv_gates(dev(proj[t]), Nin, ring_s, cw, al, dtb, qs[t * n_k * 128:], ks[t * n_k * 128:],
                       vs[t * n_v * 128:], ds[t * n_v:], bs[t * n_v:], pos, 1, n_k, n_v, kern)
    for a, b in [(qc, qs), (kc, ks), (vc, vs), (dc, ds), (bc, bs), (ring_c, ring_s)]:
        assert np.array_equal(host(a).view(np.uint32), host(b).view(np.uint32))


@pytest.mark.parametrize("H", [640, 642, 4100])  # float4 path; scalar path (H % 4, H > 4096)
def test_row_ops(hip, oc, H):
    import torch
    M, F, n_v = 5, 384, 3
    x = (3 * synth.normal(synth.stream_seed(6, 0), M * H)).astype(np.float32).reshape(M, H)
    w = (1 + 0.1 * synth.normal(synth.stream_seed(7, 0), H)).astype(np.float32)
    y = empty(M * H, torch.float32)
    hip.rmsnorm_rows(dev(x), dev(w), y, M, H)
    for i in range(M):
        r = np.zeros(H, np.float32)
        oc.lib.oc_rmsnorm(x[i], w, r, H)
        assert rel_l2(host(y).reshape(M, H)[i], r) < 1e-6
    gu = (2 * synth.normal(synth.stream_seed(8, 0), M * 2 * F)).astype(np.float32).reshape(M, 2 * F)
    y = empty(M * F, torch.float32)
    hip.swiglu_rows(dev(gu), y, M, F)
    g = gu[:, :F].astype(np.float64)
    ref = g / (1 + np.exp(-g)) * gu[:, F:]
    assert rel_l2(host(y).reshape(M, F), ref) < 1e-6
    Nin = 1000
    core = synth.normal(synth.stream_seed(9, 0), M * n_v * 128).astype(np.float32).reshape(M, n_v, 128)
    proj = synth.normal(synth.stream_seed(10, 0), M * Nin).astype(np.float32).reshape(M, Nin)
    nw = (1 + 0.1 * synth.normal(synth.stream_seed(11, 0), 128)).astype(np.float32)
    y = empty(M * n_v * 128, torch.float32)
    z_off = 200
    hip.gated_norm_rows(dev(core), dev(proj), Nin, z_off, dev(nw), y, M, n_v)
    c64 = core.astype(np.float64)
    inv = 1 / np.sqrt((c64 ** 2).mean(-1, keepdims=True) + 1e-6)
    z = proj[:, z_off:z_off + n_v * 128].reshape(M, n_v, 128).astype(np.float64)
    ref = c64 * inv * nw * (z / (1 + np.exp(-z)))
    assert rel_l2(host(y).reshape(M, n_v, 128), ref) < 1e-6


@pytest.mark.parametrize("M,H,F,n_v", [(5, 640, 384, 3), (37, 2560, 9216, 32), (16, 4000, 160, 1)])
def test_row_ops_gemm_act(hip, M, H, F, n_v):
    """The _gemm_act row ops write byte for byte what the fp32 row op followed
    by ec_gemm_quantize_act writes: block bytes, scales, padding tokens (M not
    a multiple of 16) and padding blocks (H = 4000, F = 160: K not a multiple
    of 128)."""
    import torch
    from echohip.lib import Q8_0

    def both(K, fp32_op, fused_op):
        nbytes = hip.gemm_act_bytes(Q8_0, M, K)
        y = empty(M * K, torch.float32)
        ref = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
        got = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
        fp32_op(y)
        hip.gemm_quantize_act(Q8_0, y, ref, M, K)
        fused_op(got)
        r, g = host(ref), host(got)
        assert np.array_equal(r, g), f"K {K}: {np.count_nonzero(r != g)} bytes differ"

    x = (3 * synth.normal(synth.stream_seed(16, 0), M * H)).astype(np.float32).reshape(M, H)
    w = (1 + 0.1 * synth.normal(synth.stream_seed(17, 0), H)).astype(np.float32)
    xd, wd = dev(x), dev(w)
    both(H, lambda y: hip.rmsnorm_rows(xd, wd, y, M, H), lambda a: hip.rmsnorm_rows_gemm_act(xd, wd, a, M, H))
    gu = dev((2 * synth.normal(synth.stream_seed(18, 0), M * 2 * F)).astype(np.float32))
    both(F, lambda y: hip.swiglu_rows(gu, y, M, F), lambda a: hip.swiglu_rows_gemm_act(gu, a, M, F))
    Nin, z_off = n_v * 128 + 300, 200
    core = dev(synth.normal(synth.stream_seed(19, 0), M * n_v * 128).astype(np.float32))
    proj = dev(synth.normal(synth.stream_seed(20, 0), M * Nin).astype(np.float32))
    nw = dev((1 + 0.1 * synth.normal(synth.stream_seed(21, 0), 128)).astype(np.float32))
    both(n_v * 128, lambda y: hip.gated_norm_rows(core, proj, Nin, z_off, nw, y, M, n_v),
         lambda a: hip.gated_norm_rows_gemm_act(core, proj, Nin, z_off, nw, a, M, n_v))


def _states(eng, cfg, seq):
    from echohip.engine import S_CONV, S_KEYS, S_KSCALES, S_SSM, S_VALS, S_VSCALES
    out = {}
    for l in range(cfg.n_layers):
        kinds = [S_KEYS, S_VALS, S_KSCALES, S_VSCALES] if cfg.is_attn(l) else [S_CONV, S_SSM]
        for k in kinds:
            out[(l, k)] = eng.get_state(l, k, seq)
    return out


def _compare_states(a, b, cfg):
    """fp32 states within PATH_TOL; KV caches compared dequantized (int8 x
    row scale) within PATH_TOL, and the first position's rows (before any carried
    difference) within one quantum."""
    from echohip.engine import S_KEYS, S_KSCALES, S_VALS, S_VSCALES
    scale_of = {S_KEYS: S_KSCALES, S_VALS: S_VSCALES}
    for key, x in a.items():
        y = b[key]
        if key[1] in scale_of:
            sk = (key[0], scale_of[key[1]])
            xa = x.reshape(cfg.max_ctx, cfg.n_kv, cfg.head_dim).astype(np.float64)
            xb = y.reshape(cfg.max_ctx, cfg.n_kv, cfg.head_dim).astype(np.float64)
            da = xa * a[sk].reshape(cfg.max_ctx, cfg.n_kv, 1)
            db = xb * b[sk].reshape(cfg.max_ctx, cfg.n_kv, 1)
            assert rel_l2(da, db) < PATH_TOL, (key, rel_l2(da, db))
            assert np.abs(xa[0] - xb[0]).max() <= 1, key
        else:
            assert rel_l2(x, y) < PATH_TOL, (key, rel_l2(x, y))


@pytest.mark.parametrize("lens,fmts", [((40, 7, 1), None), ((600, 3, 25), None), ((40, 7, 1), MIXED_FMTS)],
                         ids=["short", "long", "mixed"])
def test_prefill_matches_token_loop(lens, fmts):
    from echohip.engine import Engine
    cfg = small_config(max_batch=3, max_ctx=640)
    m = make_model(cfg, seed=21, fmts=fmts)
    rng = np.random.default_rng(3)
    prompts = [rng.integers(0, cfg.vocab, n).astype(np.int32) for n in lens]
    a, b = Engine(cfg), Engine(cfg)
    upload(a, m)
    upload(b, m)
    a.set_act_pieces(1)
    b.set_act_pieces(1)
    a.reset()
    b.reset()
    for s, p in enumerate(prompts):
        a.prefill(s, p, 0)
    last_b = {}
    for t in range(max(lens)):
        tok = np.array([p[t] if t < len(p) else 0 for p in prompts], np.int32)
        pos = np.array([t if t < len(p) else -1 for p in prompts], np.int32)
        b.set_inputs(tok, pos)
        b.step(graph=True)
        for s, n in enumerate(lens):
            if t == n - 1:  # later steps overwrite an inactive sequence's logits row
                last_b[s] = b.logits(s)
    ga, pa = a.tokens()
    gb, _ = b.tokens()  # b's finished prompts are inactive (position -1) after their last step
    assert pa.tolist() == list(lens)
    pb = np.array(lens, np.int32)
    for s in range(3):
        _compare_states(_states(a, cfg, s), _states(b, cfg, s), cfg)
        la, lb = a.logits(s), last_b[s]
        print(f"prompt {lens[s]}: logits rel_l2 {rel_l2(la, lb):.1e}")
        assert rel_l2(la, lb) < (1e-5 if lens[s] == 1 else PATH_TOL), (s, rel_l2(la, lb))
        top2 = np.sort(lb)[-2:]
        if top2[1] - top2[0] > 1e-2 * max(1.0, abs(top2[1])):
            assert ga[s] == gb[s]
    # continue decoding on both from the same tokens
    for step in range(4):
        a.set_inputs(gb, pb + step)
        b.set_inputs(gb, pb + step)
        a.step(graph=True)
        b.step(graph=True)
        for s in range(3):
            assert rel_l2(a.logits(s), b.logits(s)) < PATH_TOL
        gb, _ = b.tokens()
    a.close()
    b.close()


@pytest.mark.parametrize("fmts", [None, MIXED_FMTS], ids=["q8_0", "mixed"])
def test_prefill_batch_equals_one_by_one(fmts):
    """ec_engine_prefill_batch (two sequences' chunks per pass, two passes on two streams) == ec_engine_prefill per
    sequence, bit for bit: logits, greedy tokens, positions, every state;
    ragged lengths across chunk boundaries, a nonzero start position; Q8_0
    weights and a mix of Q8_0 / Q4_K matrices (Q4_K GEMMs over the pass's rows)."""
    from echohip.engine import Engine
    cfg = small_config(max_batch=4, max_ctx=700)
    m = make_model(cfg, seed=25, fmts=fmts)
    rng = np.random.default_rng(4)
    lens = [600, 7, 513, 40]
    prompts = [rng.integers(0, cfg.vocab, n).astype(np.int32) for n in lens]
    a, b = Engine(cfg), Engine(cfg)
    upload(a, m)
    upload(b, m)
    a.reset()
    b.reset()
    a.prefill(3, prompts[3][:10], 0)
    b.prefill(3, prompts[3][:10], 0)
    for s in range(3):
        a.prefill(s, prompts[s], 0)
    a.prefill(3, prompts[3][10:], 10)
    b.prefill_batch([(s, prompts[s], 0) for s in range(3)] + [(3, prompts[3][10:], 10)])
    ga, pa = a.tokens()
    gb, pb = b.tokens()
    assert ga.tolist() == gb.tolist() and pa.tolist() == pb.tolist() == [600, 7, 513, 40]
    for s in range(4):
        assert np.array_equal(a.logits(s).view(np.uint32), b.logits(s).view(np.uint32))
        sa, sb = _states(a, cfg, s), _states(b, cfg, s)
        for key in sa:
            assert np.array_equal(sa[key].view(np.uint8), sb[key].view(np.uint8)), (s, key)
    a.close()
    b.close()


def test_prefill_batch_rejects_bad_arguments():
    from echohip.engine import Engine
    from echohip.lib import EchoHipError
    cfg = small_config(max_batch=2, max_ctx=16)
    e = Engine(cfg)
    upload(e, make_model(cfg, seed=1))
    e.reset()
    with pytest.raises(EchoHipError):
        e.prefill_batch([(0, [1, 2], 0), (0, [3], 2)])  # the same sequence twice
    with pytest.raises(EchoHipError):
        e.prefill_batch([(0, [1, 2], 0), (1, list(range(20)), 0)])  # past max_ctx
    e.close()


def test_prefill_rejects_bad_arguments():
    from echohip.engine import Engine
    from echohip.lib import EchoHipError
    cfg = small_config(max_batch=2, max_ctx=16)
    e = Engine(cfg)
    upload(e, make_model(cfg, seed=1))
    e.reset()
    with pytest.raises(EchoHipError):
        e.prefill(2, [1, 2], 0)           # seq >= max_batch
    with pytest.raises(EchoHipError):
        e.prefill(0, list(range(10)), 8)  # past max_ctx
    with pytest.raises(EchoHipError):
        e.prefill(0, [cfg.vocab], 0)      # token id
    e.close()


@pytest.mark.parametrize("fmts", [None, MIXED_FMTS], ids=["q8_0", "mixed"])
def test_prefill_one_token_is_the_decode_step(fmts):
    """A one-token prompt: the GEMM path and the decode graph agree to fp32
    rounding (both with one-piece activations, the GEMMs' arithmetic).  A Q4_K
    product is the difference of two terms (d*sc*isum and dmin*m*xsum, each
    larger than the result) that the GEMM and the matvec round in different
    groupings, so the mixed model's bound is 1e-4."""
    from echohip.engine import Engine
    cfg = small_config(max_batch=2, max_ctx=16)
    m = make_model(cfg, seed=23, fmts=fmts)
    a, b = Engine(cfg), Engine(cfg)
    upload(a, m)
    upload(b, m)
    a.set_act_pieces(1)
    b.set_act_pieces(1)
    a.reset()
    b.reset()
    a.prefill(1, [417], 0)
    b.set_inputs(np.array([0, 417], np.int32), np.array([-1, 0], np.int32))
    b.step(graph=False)
    assert rel_l2(a.logits(1), b.logits(1)) < (1e-6 if fmts is None else 1e-4)
    assert a.tokens()[0][1] == b.tokens()[0][1]
    a.close()
    b.close()


_ARRANGEMENT_SCRIPT = r"""
import sys
sys.path[:0] = [{tests!r}, {pkg!r}]
from test_gpu_prefill import _batch_digest
print("digest", _batch_digest(), flush=True)
"""


def _batch_digest():
    """One ragged prefill_batch (5 sequences, 1 .. 1100 tokens, one starting at
    position 10) on a small hybrid model; a digest of every sequence's greedy
    token, position, logits and states."""
    import hashlib
    from echohip.engine import Engine
    cfg = small_config(max_batch=5, max_ctx=1200)
    m = make_model(cfg, seed=31)
    rng = np.random.default_rng(8)
    lens = [1100, 1, 530, 64, 200]
    prompts = [rng.integers(0, cfg.vocab, n).astype(np.int32) for n in lens]
    e = Engine(cfg)
    upload(e, m)
    e.reset()
    e.prefill(4, prompts[4][:10], 0)
    e.prefill_batch([(s, prompts[s], 0) for s in range(4)] + [(4, prompts[4][10:], 10)])
    h = hashlib.sha256()
    g, p = e.tokens()
    h.update(g.tobytes())
    h.update(p.tobytes())
    for s in range(5):
        h.update(e.logits(s).tobytes())
        for key, v in sorted(_states(e, cfg, s).items()):
            h.update(v.tobytes())
    e.close()
    return h.hexdigest()


def test_prefill_batch_arrangements_bit_identical():
    """The ragged multi-sequence prefill gives the same bits however the
    sequences are arranged: lanes x sequences per pass of 1 x 1, 1 x 3, 3 x 2
    and 2 x 4 (EC_PREFILL_LANES / EC_PREFILL_GROUP are read once per process,
    so each arrangement runs in a child process, one after another) equal the
    default arrangement run here -- row ops and GEMMs give each row the result
    it gets alone, whatever rows share the launch."""
    import os
    import subprocess
    import sys
    from pathlib import Path
    here = Path(__file__).resolve().parent
    ref = _batch_digest()
    script = _ARRANGEMENT_SCRIPT.format(tests=str(here), pkg=str(here.parent / "echo-core_amd"))
    for lanes, group in ((1, 1), (1, 3), (3, 2), (2, 4)):
        env = dict(os.environ, EC_PREFILL_LANES=str(lanes), EC_PREFILL_GROUP=str(group))
        print(f"arrangement lanes={lanes} group={group}", flush=True)
        r = subprocess.run([sys.executable, "-c", script], env=env, capture_output=True, text=True, timeout=150)
        assert r.returncode == 0, r.stderr[-2000:]
        got = [ln.split()[1] for ln in r.stdout.splitlines() if ln.startswith("digest ")]
        assert got == [ref], (lanes, group, got, ref)
