"""Pin the oracle's delta-net gates, gated RMSNorm and the three blocks the
decoder composes (oracle.c oc_deltanet_gates, oc_gated_rmsnorm,
oc_deltanet_block, oc_attention_block, oc_ffn_block, oc_decoder_token) with
closed forms on the CPU.

The gated delta-net has no test in the reference (qwen_linear.forward,
echo-core-zig/src/kernels/qwen_linear.zig:103-271) and no Zig toolchain is
available to produce vectors, so these cases are chosen from the mathematics
of qwen_linear.zig:215-219 (gates) and :252-257 (gated norm) so that a dropped
softplus, a dropped SiLU(z), a swapped gate/up, a wrong slice of the fused
projection (the alpha/beta rows, and the q / k order, which only a non-zero
initial state with q != k can show: from S0 = 0 the first token is symmetric
in q and k) or a transposed state fails:

  softplus(0) = ln 2          ->  alpha + dt_bias = 0 gives decay 2^-exp(A_log)
  softplus(x > 20) = x        ->  decay = exp(-exp(A_log) * x)
  sigmoid(0) = 1/2            ->  beta = 0.5
  sigmoid(-63.5) ~ 3e-28      ->  beta ~ 0: o = decay * S0^T q / sqrt(128)
  z = 0                       ->  SiLU(z) = 0, so the gated norm is 0
  constant core c             ->  w * c / sqrt(c^2 + 1e-6) * SiLU(z)

The attention block (engine.zig:520-621) is pinned at position 1, where the
softmax runs over two keys: equal scores give the mean of the two cached V
rows (the block attends over pos + 1 positions, itself included), and an
fp64 brute force over the oracle's own cache pins the q / k head RMSNorm
(applied only when its weight is not all zero, :548-553) and RoPE.

The block tests use Q8_0 matrices whose rows are unit vectors (d = 1.0 and a
single qs = 1), so every projection is an exact copy of its input slice and
the block output has a closed form.
"""
import numpy as np
import pytest

from conftest import rel_l2
from decoder_util import OracleDecoder
from echohip import synth
from echohip.engine import EngineConfig


def silu(x):
    x = np.asarray(x, np.float64)
    return x / (1.0 + np.exp(-x))


def q8_0_from_int(Q, d=1.0):
    """GGUF Q8_0 rows from an integer matrix Q [rows, K] (|Q| <= 127), one fp16 scale d per block."""
    Q = np.asarray(Q, np.int64)
    rows, K = Q.shape
    out = np.zeros((rows, K // 32, 34), np.uint8)
    out[:, :, 0:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    out[:, :, 2:] = Q.reshape(rows, K // 32, 32).astype(np.int8).view(np.uint8)
    return out.reshape(rows, K // 32 * 34)


def select(rows, K, cols, scale=1):
    """Rows that copy input element cols[r] (times the integer `scale`)."""
    Q = np.zeros((rows, K), np.int64)
    Q[np.arange(rows), cols] = scale
    return Q


# ------------------------------------------------------------------- gates
def test_gates_closed_forms(oc):
    a_log = np.array([0.3, -0.5, 0.0, 1.2, np.log(0.01)], np.float32)
    zero = np.zeros(5, np.float32)
    dec, bet = oc.deltanet_gates(zero, zero, a_log, zero)
    # softplus(0) = ln 2, so decay = exp(-exp(A) ln 2) = 2^-exp(A); sigmoid(0) = 1/2
    assert np.allclose(dec, 2.0 ** -np.exp(a_log.astype(np.float64)), rtol=2e-6, atol=0)
    assert np.array_equal(bet, np.full(5, 0.5, np.float32))
    # alpha + dt_bias > 20 takes softplus(x) = x: decay = exp(-exp(A) x); split between alpha and dt_bias
    alpha = np.array([20.5, 5.0, 30.0, 21.0, 15.0], np.float32)
    dt = np.array([0.0, 20.0, -5.0, 0.0, 10.0], np.float32)
    dec, _ = oc.deltanet_gates(alpha, zero, a_log, dt)
    x = (alpha + dt).astype(np.float64)
    assert np.allclose(dec, np.exp(-np.exp(a_log.astype(np.float64)) * x), rtol=2e-6, atol=1e-30)
    # strongly negative alpha: softplus -> 0, decay -> 1 (not > 1)
    dec, _ = oc.deltanet_gates(np.full(5, -40.0, np.float32), zero, a_log, zero)
    assert np.all(dec <= 1.0) and np.allclose(dec, 1.0, atol=1e-12)
    # beta = sigmoid(b): ln 3 -> 3/4, -ln 3 -> 1/4
    _, bet = oc.deltanet_gates(zero, np.array([np.log(3), -np.log(3), 0, 0, 0], np.float32), a_log, zero)
    assert np.allclose(bet[:2], [0.75, 0.25], rtol=1e-6)


# -------------------------------------------------------------- gated norm
def test_gated_rmsnorm_closed_forms(oc):
    n_v, d_v = 3, 128
    w = (1.0 + 0.1 * synth.normal(1, d_v)).astype(np.float32)
    z = (2.0 * synth.normal(2, n_v * d_v)).astype(np.float32)
    core = synth.normal(3, n_v * d_v).astype(np.float32)
    # z = 0: SiLU(0) = 0 -> the output is exactly zero whatever the core
    assert np.array_equal(oc.gated_rmsnorm(core, np.zeros_like(z), w, n_v, d_v), np.zeros((n_v, d_v), np.float32))
    # constant core c per head: mean(c^2) = c^2 -> w * c / sqrt(c^2 + 1e-6) * SiLU(z)
    c = np.array([0.7, -3.0, 1e-3], np.float32)
    cc = np.repeat(c, d_v)
    got = oc.gated_rmsnorm(cc, z, w, n_v, d_v)
    c64 = c.astype(np.float64)[:, None]
    ref = w[None, :] * c64 / np.sqrt(c64 ** 2 + 1e-6) * silu(z).reshape(n_v, d_v)
    assert rel_l2(got, ref) < 2e-6
    # the norm is per head: scaling one head's core leaves the output unchanged (eps aside)
    scaled = core.reshape(n_v, d_v).copy()
    scaled[1] *= 8.0
    a = oc.gated_rmsnorm(core, z, w, n_v, d_v)
    b = oc.gated_rmsnorm(scaled, z, w, n_v, d_v)
    assert rel_l2(a, b) < 1e-6


# ------------------------------------------------------------------ blocks
def _delta_cfg():
    # hidden 256, value_dim 256 = 2 heads of 128, key_dim 128 = 1 q/k head, conv_dim 512
    return EngineConfig(vocab=64, hidden=256, ffn=256, n_layers=1, n_heads=1, n_kv=1, head_dim=256, ssm_inner=256,
                        ssm_heads=2, conv_kernel=4, attn_interval=0, max_batch=1, max_ctx=8)


def _delta_model(cfg, w_qkv_rows, w_z_rows, w_ab=None, a_log=(0.3, -0.5), dt_bias=(0.0, 0.0), conv_last=1.0):
    H, C = cfg.hidden, cfg.conv_dim
    n_v = cfg.ssm_heads
    conv = np.zeros((cfg.conv_kernel, C), np.float32)
    conv[cfg.conv_kernel - 1] = conv_last  # slot 0 (the newest input) meets tap row kernel-1 (qwen_linear.zig:197)
    w_in = np.concatenate([q8_0_from_int(w_qkv_rows), q8_0_from_int(w_z_rows),
                           q8_0_from_int(np.zeros((2 * n_v, H)) if w_ab is None else w_ab)])
    y = {"attn": False, "w_in": w_in, "w_out": q8_0_from_int(select(H, cfg.ssm_inner, np.arange(H))),
         "w_gate": q8_0_from_int(np.zeros((cfg.ffn, H))), "w_up": q8_0_from_int(np.zeros((cfg.ffn, H))),
         "w_down": q8_0_from_int(np.zeros((H, cfg.ffn))), "attn_norm": np.ones(H, np.float32),
         "ffn_norm": np.ones(H, np.float32), "conv_w": conv.reshape(-1),
         "a_log": np.array(a_log, np.float32), "dt_bias": np.array(dt_bias, np.float32),
         "ssm_norm": (1.0 + 0.1 * synth.normal(11, 128)).astype(np.float32)}
    return {"embed": q8_0_from_int(np.zeros((cfg.vocab, H))), "final_norm": np.ones(H, np.float32),
            "lm_head": q8_0_from_int(np.zeros((cfg.vocab, H))), "layers": [y]}


def test_deltanet_block_first_token_closed_form(oc):
    """S0 = 0, q = k: S1 = k (x) beta*v, o = (q.k) beta v / sqrt(128), then the gated norm and an identity output."""
    cfg = _delta_cfg()
    H = cfg.hidden
    # q rows and k rows both copy x[0:128]; v rows copy x[0:256]; z rows copy x[0:256]
    qkv = np.concatenate([select(128, H, np.arange(128)), select(128, H, np.arange(128)), select(256, H, np.arange(256))])
    m = _delta_model(cfg, qkv, select(256, H, np.arange(256)))
    x = synth.normal(21, H).astype(np.float32)
    for quant_act in (False, True):
        dec = OracleDecoder(oc, cfg, m, n_seq=1, quant_act=quant_act)
        out = dec.deltanet_block(0, 0, x)
        xin = x.astype(np.float64)
        if quant_act:  # the projections see the Q8_0-quantized input
            xq, xd = oc.quantize_act_q8_0(x)
            xin = oc.dequant_act_q8_0(xq, xd).astype(np.float64)
        u = silu(xin[:128])
        k = u / np.sqrt(np.sum(u * u) + 1e-6)
        v = silu(xin).reshape(2, 128)
        o = (k @ k) * 0.5 * v / np.sqrt(128.0)  # beta = sigmoid(0) = 1/2
        g = o / np.sqrt(np.mean(o * o, axis=1, keepdims=True) + 1e-6) * m["layers"][0]["ssm_norm"] * \
            silu(xin).reshape(2, 128)
        ref = g.reshape(-1)
        if quant_act:  # the gated-norm output is quantized before the identity output projection
            gq, gd = oc.quantize_act_q8_0(ref.astype(np.float32))
            ref = oc.dequant_act_q8_0(gq, gd)
            assert rel_l2(out, ref) < 1e-3
        else:
            assert rel_l2(out, ref) < 2e-6
        # the state is k (x) delta with delta = beta v (reference layout S[k][v] per head)
        S = dec.states[0]["ssm"][0].reshape(2, 128, 128)
        Sref = np.einsum("k,hv->hkv", k, 0.5 * v)
        assert rel_l2(S, Sref) < (1e-3 if quant_act else 2e-6)


def test_deltanet_block_zero_z_gives_zero_output(oc):
    cfg = _delta_cfg()
    H = cfg.hidden
    qkv = np.concatenate([select(128, H, np.arange(128)), select(128, H, np.arange(128, 256)),
                          select(256, H, np.arange(256))])
    m = _delta_model(cfg, qkv, np.zeros((256, H)))
    dec = OracleDecoder(oc, cfg, m, n_seq=1, quant_act=False)
    for t in range(3):
        out = dec.deltanet_block(0, 0, synth.normal(30 + t, H).astype(np.float32))
        assert np.array_equal(out, np.zeros(H, np.float32))
    assert np.abs(dec.states[0]["ssm"][0]).max() > 0.0  # the state did advance


@pytest.mark.parametrize("dt_bias", [0.0, 25.0])
def test_deltanet_block_decay_of_state(oc, dt_bias):
    """Zero q|k|v projections (conv of zeros, L2 norm of zero = 0): one token scales the state by decay exactly."""
    cfg = _delta_cfg()
    H = cfg.hidden
    a_log = (0.3, np.log(0.01))
    m = _delta_model(cfg, np.zeros((512, H)), select(256, H, np.arange(256)), a_log=a_log, dt_bias=(dt_bias, dt_bias))
    dec = OracleDecoder(oc, cfg, m, n_seq=1, quant_act=False)
    S0 = (0.02 * synth.normal(40, 2 * 128 * 128)).astype(np.float32)
    np.copyto(dec.states[0]["ssm"][0], S0)
    out = dec.deltanet_block(0, 0, synth.normal(41, H).astype(np.float32))
    assert np.array_equal(out, np.zeros(H, np.float32))  # o = S^T 0 = 0
    sp = np.log(2.0) if dt_bias == 0 else dt_bias  # softplus(0) = ln 2; softplus(25) = 25
    decay = np.exp(-np.exp(np.array(a_log)) * sp)
    S1 = dec.states[0]["ssm"][0].reshape(2, -1).astype(np.float64)
    assert np.allclose(S1, S0.reshape(2, -1) * decay[:, None], rtol=3e-6, atol=0)


def test_deltanet_block_gates_come_from_alpha_beta_rows(oc):
    """The last 2*n_v rows of the fused projection are alpha then beta: a beta row reading x[0] = ln 3 gives
    beta = 3/4 (delta = 3/4 v), an alpha row with alpha = 0 leaves decay = 2^-exp(A)."""
    cfg = _delta_cfg()
    H = cfg.hidden
    qkv = np.concatenate([select(128, H, np.arange(128)), select(128, H, np.arange(128)), select(256, H, np.arange(256))])
    ab = np.zeros((4, H), np.int64)
    ab[2, 0] = 1  # beta logit of head 0 = x[0]
    ab[3, 0] = 1  # beta logit of head 1 = x[0]
    m = _delta_model(cfg, qkv, select(256, H, np.arange(256)), w_ab=ab)
    x = synth.normal(50, H).astype(np.float32)
    x[0] = np.float32(np.log(3.0))
    dec = OracleDecoder(oc, cfg, m, n_seq=1, quant_act=False)
    dec.deltanet_block(0, 0, x)
    u = silu(x[:128].astype(np.float64))
    k = u / np.sqrt(np.sum(u * u) + 1e-6)
    v = silu(x.astype(np.float64)).reshape(2, 128)
    S = dec.states[0]["ssm"][0].reshape(2, 128, 128)
    assert rel_l2(S, np.einsum("k,hv->hkv", k, 0.75 * v)) < 2e-6


def test_attention_block_first_position_returns_dequantized_v(oc):
    """At position 0 the softmax is over one key, so head h outputs V[0, h % n_kv] dequantized; an identity output
    projection returns it (engine.zig:556-619, modulo GQA mapping)."""
    cfg = EngineConfig(vocab=64, hidden=1024, ffn=256, n_layers=1, n_heads=4, n_kv=2, head_dim=256, ssm_inner=0,
                       ssm_heads=0, conv_kernel=4, attn_interval=1, max_batch=1, max_ctx=8)
    H, hd = cfg.hidden, cfg.head_dim
    q_dim, kv_dim = cfg.n_heads * hd, cfg.n_kv * hd
    # q|k rows copy x[0:1024] and x[0:512]; v rows copy 2 * x[512:1024]
    w_in = np.concatenate([select(q_dim, H, np.arange(q_dim)), select(kv_dim, H, np.arange(kv_dim)),
                           select(kv_dim, H, np.arange(512, 1024), scale=2)])
    y = {"attn": True, "w_in": q8_0_from_int(w_in), "w_out": q8_0_from_int(select(H, q_dim, np.arange(H))),
         "w_gate": q8_0_from_int(np.zeros((cfg.ffn, H))), "w_up": q8_0_from_int(np.zeros((cfg.ffn, H))),
         "w_down": q8_0_from_int(np.zeros((H, cfg.ffn))), "attn_norm": np.ones(H, np.float32),
         "ffn_norm": np.ones(H, np.float32), "q_norm": np.zeros(hd, np.float32), "k_norm": np.zeros(hd, np.float32)}
    m = {"embed": q8_0_from_int(np.zeros((cfg.vocab, H))), "final_norm": np.ones(H, np.float32),
         "lm_head": q8_0_from_int(np.zeros((cfg.vocab, H))), "layers": [y]}
    dec = OracleDecoder(oc, cfg, m, n_seq=1, quant_act=False)
    x = synth.normal(60, H).astype(np.float32)
    out = dec.attention_block(0, 0, x, 0)
    vq, vs = oc.quantize(2.0 * x[512:1024], hd)  # per (token, kv head) scale
    vdeq = vq.astype(np.float64) * vs[:, None]
    ref = np.stack([vdeq[h % cfg.n_kv] for h in range(cfg.n_heads)]).reshape(-1)
    assert rel_l2(out, ref) < 1e-6


def test_ffn_block_closed_form(oc):
    """gate = identity, up = 2 x identity, down = identity: out = silu(x) * 2x (SiLU on the gate, not the up)."""
    cfg = EngineConfig(vocab=64, hidden=256, ffn=256, n_layers=1, n_heads=1, n_kv=1, head_dim=256, ssm_inner=0,
                       ssm_heads=0, conv_kernel=4, attn_interval=1, max_batch=1, max_ctx=8)
    H = cfg.hidden
    eye = select(H, H, np.arange(H))
    y = {"attn": True, "w_in": q8_0_from_int(np.zeros((cfg.nin_attn, H))), "w_out": q8_0_from_int(np.zeros((H, 256))),
         "w_gate": q8_0_from_int(eye), "w_up": q8_0_from_int(2 * eye), "w_down": q8_0_from_int(eye),
         "attn_norm": np.ones(H, np.float32), "ffn_norm": np.ones(H, np.float32),
         "q_norm": np.zeros(256, np.float32), "k_norm": np.zeros(256, np.float32)}
    m = {"embed": q8_0_from_int(np.zeros((cfg.vocab, H))), "final_norm": np.ones(H, np.float32),
         "lm_head": q8_0_from_int(np.zeros((cfg.vocab, H))), "layers": [y]}
    dec = OracleDecoder(oc, cfg, m, n_seq=1, quant_act=False)
    x = (2.0 * synth.normal(70, H)).astype(np.float32)
    out = dec.ffn_block(0, x)
    assert rel_l2(out, silu(x) * 2.0 * x) < 2e-6


def test_decoder_token_composes_the_blocks(oc):
    """oc_decoder_token = embed, then per block x += block(rmsnorm(x)), x += ffn(rmsnorm(x)), then the head
    (engine.zig:360-463), with the blocks above; both activation modes."""
    from decoder_util import make_model, small_config
    cfg = small_config(max_batch=1, max_ctx=16)
    m = make_model(cfg, seed=12)
    H = cfg.hidden

    def deq_row(blocks, K, r):
        b = blocks.reshape(-1, K // 32, 34)[r]
        d = b[:, 0:2].copy().view(np.float16)[:, 0].astype(np.float32)
        return (b[:, 2:].view(np.int8).astype(np.float32) * d[:, None]).reshape(-1)

    def rms(x, w):
        out = np.zeros(H, np.float32)
        oc.lib.oc_rmsnorm(np.ascontiguousarray(x, np.float32), np.ascontiguousarray(w, np.float32), out, H)
        return out

    for quant_act in (False, True):
        full = OracleDecoder(oc, cfg, m, n_seq=1, quant_act=quant_act)
        parts = OracleDecoder(oc, cfg, m, n_seq=1, quant_act=quant_act)
        for pos, tok in enumerate((7, 500, 3)):
            lg = full.token(0, tok)
            x = deq_row(m["embed"], H, tok)
            for l, y in enumerate(m["layers"]):
                h = rms(x, y["attn_norm"])
                b = parts.attention_block(0, l, h, pos) if cfg.is_attn(l) else parts.deltanet_block(0, l, h)
                x = (x + b).astype(np.float32)
                x = (x + parts.ffn_block(l, rms(x, y["ffn_norm"]))).astype(np.float32)
            ref = oc.matvec_act_q8_0(m["lm_head"], rms(x, m["final_norm"]), quant_act)
            assert np.array_equal(lg, ref)


# ------------------------------------------------------- head RMSNorm (q, k)
def test_head_rmsnorm_closed_forms(oc):
    """oc_head_rmsnorm (engine.zig:507-518): each head of head_dim values is RMS-normalised on its own and scaled
    by the same per-dimension weight."""
    n_h, hd = 3, 256
    w = (1.0 + 0.1 * synth.normal(80, hd)).astype(np.float32)
    # a constant head c: mean(c^2) = c^2 -> w * c / sqrt(c^2 + 1e-6)
    c = np.array([0.5, -3.0, 1e-3], np.float32)
    got = oc.head_rmsnorm(np.repeat(c, hd), w, n_h, hd).reshape(n_h, hd)
    c64 = c.astype(np.float64)[:, None]
    assert rel_l2(got, w[None, :] * c64 / np.sqrt(c64 ** 2 + 1e-6)) < 2e-6
    # per head: scaling head 1 by 8 changes no head's output (eps aside); head h uses w, not w shifted by h
    x = (3.0 * synth.normal(81, n_h * hd)).astype(np.float32)
    a = oc.head_rmsnorm(x, w, n_h, hd).reshape(n_h, hd)
    x2 = x.reshape(n_h, hd).copy()
    x2[1] *= 8.0
    b = oc.head_rmsnorm(x2, w, n_h, hd).reshape(n_h, hd)
    assert rel_l2(a, b) < 1e-6
    xh = x.reshape(n_h, hd).astype(np.float64)
    ref = w[None, :] * xh / np.sqrt(np.mean(xh * xh, axis=1, keepdims=True) + 1e-6)
    assert rel_l2(a, ref) < 2e-6


def _attn_cfg():
    # q_dim 1024 (4 heads), kv_dim 512 (2 kv heads), hidden 2048 so q, k and v read disjoint input slices
    return EngineConfig(vocab=64, hidden=2048, ffn=256, n_layers=1, n_heads=4, n_kv=2, head_dim=256, ssm_inner=0,
                        ssm_heads=0, conv_kernel=4, attn_interval=1, max_batch=1, max_ctx=8)


def _attn_model(cfg, q_norm, k_norm, zero_k=False):
    """q rows copy x[0:1024], k rows x[1024:1536] (zero rows if zero_k), v rows x[1536:2048]; the output projection
    copies the attention output into out[0:1024]."""
    H, hd = cfg.hidden, cfg.head_dim
    q_dim, kv_dim = cfg.n_heads * hd, cfg.n_kv * hd
    k_rows = np.zeros((kv_dim, H), np.int64) if zero_k else select(kv_dim, H, np.arange(1024, 1536))
    w_in = np.concatenate([select(q_dim, H, np.arange(q_dim)), k_rows, select(kv_dim, H, np.arange(1536, 2048))])
    w_out = np.zeros((H, q_dim), np.int64)
    w_out[np.arange(q_dim), np.arange(q_dim)] = 1
    y = {"attn": True, "w_in": q8_0_from_int(w_in), "w_out": q8_0_from_int(w_out),
         "w_gate": q8_0_from_int(np.zeros((cfg.ffn, H))), "w_up": q8_0_from_int(np.zeros((cfg.ffn, H))),
         "w_down": q8_0_from_int(np.zeros((H, cfg.ffn))), "attn_norm": np.ones(H, np.float32),
         "ffn_norm": np.ones(H, np.float32), "q_norm": np.asarray(q_norm, np.float32),
         "k_norm": np.asarray(k_norm, np.float32)}
    return {"embed": q8_0_from_int(np.zeros((cfg.vocab, H))), "final_norm": np.ones(H, np.float32),
            "lm_head": q8_0_from_int(np.zeros((cfg.vocab, H))), "layers": [y]}


def test_attention_block_attends_over_itself_at_position_1(oc):
    """k = 0 makes every score 0, so at position 1 the softmax weights the two cached V rows 1/2 each: the output
    is their mean -- the block appends the token before attending and covers pos + 1 positions
    (engine.zig:556-567)."""
    cfg = _attn_cfg()
    hd = cfg.head_dim
    m = _attn_model(cfg, np.zeros(hd), np.zeros(hd), zero_k=True)
    dec = OracleDecoder(oc, cfg, m, n_seq=1, quant_act=False)
    xs = [synth.normal(90 + p, cfg.hidden).astype(np.float32) for p in range(2)]
    for pos, x in enumerate(xs):
        out = dec.attention_block(0, 0, x, pos)
    vdeq = []
    for x in xs:  # V row of each position, per (token, kv head) scale
        vq, vs = oc.quantize(x[1536:2048], hd)
        vdeq.append(vq.astype(np.float64) * vs[:, None])
    mean = 0.5 * (vdeq[0] + vdeq[1])
    ref = np.stack([mean[h % cfg.n_kv] for h in range(cfg.n_heads)]).reshape(-1)
    assert rel_l2(out[:1024], ref) < 1e-6
    assert np.array_equal(out[1024:], np.zeros(1024, np.float32))


def _rope64(heads, pos, base=10000.0):
    """GPT-J RoPE of adjacent pairs (d, d+1) at angle pos * base^(-d/head_dim), in fp64."""
    hd = heads.shape[-1]
    ang = pos * base ** (-np.arange(0, hd, 2, dtype=np.float64) / hd)
    c, s = np.cos(ang), np.sin(ang)
    a, b = heads[..., 0::2], heads[..., 1::2]
    out = np.empty_like(heads)
    out[..., 0::2] = a * c - b * s
    out[..., 1::2] = a * s + b * c
    return out


@pytest.mark.parametrize("normed", [True, False], ids=["head_norm", "zero_norm_weight"])
def test_attention_block_head_norm_rope_at_position_1(oc, normed):
    """fp64 brute force of the block at position 1 over the oracle's own cache.  q and k are 3 x N(0,1), so the
    head RMSNorm (x / rms(x) * w, rms ~ 3) visibly rescales them; an all-zero norm weight means no norm
    (engine.zig:548-553), not a zero vector.  The cached keys are checked as int8 of RoPE(norm(k)) per
    (token, kv head), and the output as softmax over both positions of q . k / 16 times the cached V."""
    cfg = _attn_cfg()
    hd, n_h, n_kv = cfg.head_dim, cfg.n_heads, cfg.n_kv
    qn = (1.0 + 0.2 * synth.normal(95, hd)).astype(np.float32) if normed else np.zeros(hd, np.float32)
    kn = (1.0 + 0.2 * synth.normal(96, hd)).astype(np.float32) if normed else np.zeros(hd, np.float32)
    dec = OracleDecoder(oc, cfg, _attn_model(cfg, qn, kn), n_seq=1, quant_act=False)
    xs = []
    for pos in range(2):
        x = synth.normal(97 + pos, cfg.hidden).astype(np.float32)
        x[:1536] *= 3.0
        xs.append(x)
        out = dec.attention_block(0, 0, x, pos)

    def prep(v, w, n, pos):
        h = v.reshape(n, hd).astype(np.float64)
        if normed:
            h = w[None, :] * h / np.sqrt(np.mean(h * h, axis=1, keepdims=True) + 1e-6)
        return _rope64(h, pos)

    st = dec.states[0]
    keys = st["k"][0].reshape(cfg.max_ctx, n_kv, hd)[:2].astype(np.float64)
    vals = st["v"][0].reshape(cfg.max_ctx, n_kv, hd)[:2].astype(np.float64)
    ks = st["ks"][0].reshape(cfg.max_ctx, n_kv)[:2]
    vs = st["vs"][0].reshape(cfg.max_ctx, n_kv)[:2]
    for p, x in enumerate(xs):
        kref = prep(x[1024:1536], kn, n_kv, p)
        kq, kscale = oc.quantize(kref.astype(np.float32).reshape(-1), hd)
        assert np.allclose(ks[p], kscale, rtol=1e-6)
        assert np.mean(kq.reshape(n_kv, hd) != keys[p]) <= 0.01  # int8 of the same values up to rounding ties
        assert np.abs(kq.reshape(n_kv, hd) - keys[p]).max() <= 1
    kdeq = keys * ks[:, :, None]
    vdeq = vals * vs[:, :, None]
    q = prep(xs[1][:1024], qn, n_h, 1)
    ref = np.zeros((n_h, hd))
    for h in range(n_h):
        s = kdeq[:, h % n_kv, :] @ q[h] / np.sqrt(hd)
        a = np.exp(s - s.max())
        a /= a.sum()
        ref[h] = a @ vdeq[:, h % n_kv, :]
    assert rel_l2(out[:1024], ref.reshape(-1)) < 1e-5
    # the two scores differ enough that a change of q's scale would move the output
    s_spread = [np.ptp(kdeq[:, h % n_kv, :] @ q[h]) / np.sqrt(hd) for h in range(n_h)]
    assert max(s_spread) > 0.5


def test_deltanet_block_q_k_slices_with_nonzero_state(oc):
    """q rows copy x[0:128] and k rows x[128:256], S0 != 0 and beta ~ 0 (a beta row reading 127 * x[255] with
    x[255] = -0.5): the state only decays, S1 = decay S0, and o = decay S0^T q_hat / sqrt(128) before the gated
    norm (qwen_linear.zig:209-211, 221-249).  Swapping the q and k slices gives S0^T k_hat instead."""
    cfg = _delta_cfg()
    H = cfg.hidden
    qkv = np.concatenate([select(128, H, np.arange(128)), select(128, H, np.arange(128, 256)),
                          select(256, H, np.arange(256))])
    ab = np.zeros((4, H), np.int64)
    ab[2, 255] = 127  # beta logits of both heads = 127 * x[255]
    ab[3, 255] = 127
    a_log = (0.3, -0.5)
    m = _delta_model(cfg, qkv, select(256, H, np.arange(256)), w_ab=ab, a_log=a_log)
    dec = OracleDecoder(oc, cfg, m, n_seq=1, quant_act=False)
    S0 = (0.02 * synth.normal(100, 2 * 128 * 128)).astype(np.float32)
    np.copyto(dec.states[0]["ssm"][0], S0)
    x = synth.normal(101, H).astype(np.float32)
    x[255] = -0.5
    out = dec.deltanet_block(0, 0, x)
    xin = x.astype(np.float64)
    conv = silu(xin)  # zero conv history, newest tap weight 1: conv output = SiLU(projection)
    q = conv[:128] / np.sqrt(np.sum(conv[:128] ** 2) + 1e-6)
    k = conv[128:256] / np.sqrt(np.sum(conv[128:256] ** 2) + 1e-6)
    decay = 2.0 ** -np.exp(np.array(a_log))  # alpha = 0: softplus(0) = ln 2
    S = S0.reshape(2, 128, 128).astype(np.float64)  # [head][k][v]
    o = decay[:, None] * np.einsum("hkv,k->hv", S, q) / np.sqrt(128.0)
    g = o / np.sqrt(np.mean(o * o, axis=1, keepdims=True) + 1e-6) * m["layers"][0]["ssm_norm"] * silu(xin).reshape(2, 128)
    assert rel_l2(out, g.reshape(-1)) < 1e-5
    S1 = dec.states[0]["ssm"][0].reshape(2, 128, 128)
    assert rel_l2(S1, decay[:, None, None] * S) < 1e-6
    # the q / k order matters here: S0^T k_hat is far from S0^T q_hat
    o_k = decay[:, None] * np.einsum("hkv,k->hv", S, k) / np.sqrt(128.0)
    assert rel_l2(o_k, o) > 0.5
