"""Pin the oracle's attention, KV append, delta-net and decoder-glue
restatements (CPU only) with closed forms, invariants and fp64 brute force.

No reference test exercises the INT8 engine attention or the delta-net
(qwen_linear.forward has no test and no Zig toolchain is available), so these
are pinned by mathematics; each case is chosen so that a plausible slip (wrong
kv-head mapping, a missing decay, a transposed state, a dropped beta) fails.
"""
import numpy as np
import pytest

from conftest import rel_l2
from echohip import synth


# ------------------------------------------------------------ KV + attention
def _kv(oc, ctx, n_kv, hd, seed, k=None, v=None):
    keys = np.zeros(ctx * n_kv * hd, np.int8)
    vals = np.zeros(ctx * n_kv * hd, np.int8)
    ks = np.zeros(ctx * n_kv, np.float32)
    vs = np.zeros(ctx * n_kv, np.float32)
    kf = synth.activations(seed, ctx * n_kv * hd).reshape(ctx, -1) if k is None else k
    vf = synth.activations(seed + 1, ctx * n_kv * hd).reshape(ctx, -1) if v is None else v
    for p in range(ctx):
        oc.kv_append(kf[p], vf[p], keys, vals, ks, vs, p, n_kv, hd)
    return keys, vals, ks, vs


def test_kv_append_per_head_scale(oc):
    n_kv, hd = 4, 256
    k = synth.activations(1, n_kv * hd) * np.repeat(np.array([1, 10, 100, 1000], np.float32), hd)
    keys, vals, ks, vs = _kv(oc, 1, n_kv, hd, 0, k=k[None], v=k[None])
    for h in range(n_kv):
        amax = np.max(np.abs(k[h * hd:(h + 1) * hd]))
        assert ks[h] == np.float32(amax) / np.float32(127.0)
        q, s = oc.quantize(k[h * hd:(h + 1) * hd], hd)
        assert np.array_equal(keys[h * hd:(h + 1) * hd], q.ravel())


def _attn_f64(q, keys, vals, ks, vs, n_heads, n_kv, hd, ctx):
    K = keys.reshape(ctx, n_kv, hd).astype(np.float64) * ks.reshape(ctx, n_kv, 1)
    V = vals.reshape(ctx, n_kv, hd).astype(np.float64) * vs.reshape(ctx, n_kv, 1)
    out = np.zeros((n_heads, hd))
    for h in range(n_heads):
        s = K[:, h % n_kv] @ q[h].astype(np.float64) / np.sqrt(hd)
        a = np.exp(s - s.max())
        a /= a.sum()
        out[h] = a @ V[:, h % n_kv]
    return out


@pytest.mark.parametrize("ctx", [1, 7, 64])
def test_attention_brute_force(oc, ctx):
    n_heads, n_kv, hd = 16, 4, 256
    keys, vals, ks, vs = _kv(oc, ctx, n_kv, hd, 10 + ctx)
    q = synth.activations(99, n_heads * hd).reshape(n_heads, hd)
    got = oc.attn_decode(q, keys, vals, ks, vs, n_heads, n_kv, hd, ctx)
    assert rel_l2(got, _attn_f64(q, keys, vals, ks, vs, n_heads, n_kv, hd, ctx)) < 1e-5


def test_attention_identical_keys_give_mean_of_values(oc):
    n_heads, n_kv, hd, ctx = 8, 2, 64, 20
    k = np.tile(synth.activations(5, n_kv * hd), (ctx, 1))
    keys, vals, ks, vs = _kv(oc, ctx, n_kv, hd, 6, k=k)
    q = synth.activations(7, n_heads * hd).reshape(n_heads, hd)
    got = oc.attn_decode(q, keys, vals, ks, vs, n_heads, n_kv, hd, ctx)
    V = vals.reshape(ctx, n_kv, hd).astype(np.float64) * vs.reshape(ctx, n_kv, 1)
    for h in range(n_heads):
        assert np.allclose(got[h], V[:, h % n_kv].mean(0), atol=1e-5)


def test_attention_gqa_modulo_and_dominant_key(oc):
    """kv head = h % n_kv (src/inference.cpp:335, engine.zig:572): with one key
    aligned to q and the rest orthogonal-ish small, head h returns V[p*, h % n_kv]."""
    n_heads, n_kv, hd, ctx = 8, 4, 64, 16
    rng = np.random.default_rng(3)
    k = rng.standard_normal((ctx, n_kv * hd)).astype(np.float32) * 0.01
    q = np.zeros((n_heads, hd), np.float32)
    star = {h: (3 * h + 1) % ctx for h in range(n_kv)}
    for kvh in range(n_kv):
        dirv = np.zeros(hd, np.float32)
        dirv[kvh * 7] = 1.0
        k[star[kvh], kvh * hd:(kvh + 1) * hd] = dirv * 40.0
    for h in range(n_heads):
        q[h, (h % n_kv) * 7] = 40.0
    v = (np.arange(ctx * n_kv * hd, dtype=np.float32).reshape(ctx, n_kv * hd) % 97) - 48
    keys, vals, ks, vs = _kv(oc, ctx, n_kv, hd, 0, k=k, v=v)
    got = oc.attn_decode(q, keys, vals, ks, vs, n_heads, n_kv, hd, ctx)
    V = vals.reshape(ctx, n_kv, hd).astype(np.float64) * vs.reshape(ctx, n_kv, 1)
    for h in range(n_heads):
        kvh = h % n_kv
        assert np.allclose(got[h], V[star[kvh], kvh], atol=1e-3)


# ------------------------------------------------------------------ delta-net
def _dn_f64(state, q, k, v, decay, beta, n_v, n_k, dk, dv):
    S = state.astype(np.float64).reshape(n_v, dk, dv)
    out = np.zeros((n_v, dv))
    rep = n_v // n_k
    for h in range(n_v):
        kh = k[h // rep].astype(np.float64)
        qh = q[h // rep].astype(np.float64) / np.sqrt(dk)
        S[h] *= decay[h]
        delta = (v[h] - S[h].T @ kh) * beta[h]
        S[h] += np.outer(kh, delta)
        out[h] = S[h].T @ qh
    return S, out


def _unit(x):
    return x / np.linalg.norm(x, axis=-1, keepdims=True)


def test_deltanet_one_step_from_zero(oc):
    """decay=1, beta=1, S0=0, unit k: S = k (x) v and o = (q.k/sqrt(d)) v."""
    n_v = n_k = 2
    dk = dv = 16
    rng = np.random.default_rng(1)
    q = _unit(rng.standard_normal((n_k, dk))).astype(np.float32)
    k = _unit(rng.standard_normal((n_k, dk))).astype(np.float32)
    v = rng.standard_normal((n_v, dv)).astype(np.float32)
    S = np.zeros((n_v, dk, dv), np.float32)
    out = oc.deltanet_step(S, q, k, v, np.ones(n_v, np.float32), np.ones(n_v, np.float32), n_v, n_k, dk, dv)
    for h in range(n_v):
        assert np.allclose(S[h], np.outer(k[h], v[h]), atol=1e-6)
        assert np.allclose(out[h], (q[h] @ k[h]) / 4.0 * v[h], atol=1e-6)


def test_deltanet_beta_zero_is_pure_decay(oc):
    n_v = n_k = 2
    dk = dv = 8
    S0 = synth.activations(3, n_v * dk * dv).reshape(n_v, dk, dv)
    S = S0.copy()
    dec = np.array([0.9, 0.5], np.float32)
    rng = np.random.default_rng(2)
    for t in range(5):
        q = _unit(rng.standard_normal((n_k, dk))).astype(np.float32)
        k = _unit(rng.standard_normal((n_k, dk))).astype(np.float32)
        v = rng.standard_normal((n_v, dv)).astype(np.float32)
        oc.deltanet_step(S, q, k, v, dec, np.zeros(n_v, np.float32), n_v, n_k, dk, dv)
    for h in range(n_v):
        assert np.allclose(S[h], S0[h] * float(dec[h]) ** 5, rtol=1e-5, atol=1e-7)


def test_deltanet_orthonormal_retrieval(oc):
    """decay=1, beta=1, orthonormal keys: after writing (k_i, v_i), S^T k_i = v_i."""
    n_v = n_k = 1
    dk = dv = 16
    Q, _ = np.linalg.qr(np.random.default_rng(4).standard_normal((dk, dk)))
    keys = Q.T.astype(np.float32)
    vals = np.random.default_rng(5).standard_normal((6, dv)).astype(np.float32)
    S = np.zeros((1, dk, dv), np.float32)
    for i in range(6):
        oc.deltanet_step(S, keys[i:i + 1], keys[i:i + 1], vals[i:i + 1], np.ones(1, np.float32),
                         np.ones(1, np.float32), n_v, n_k, dk, dv)
    for i in range(6):
        assert np.allclose(S[0].T @ keys[i], vals[i], atol=1e-5)


def test_deltanet_column_permutation_and_brute_force(oc):
    n_v, n_k, dk, dv = 4, 2, 8, 8  # repeat factor 2 (q/k head = h // 2)
    rng = np.random.default_rng(6)
    S = (rng.standard_normal((n_v, dk, dv)) * 0.02).astype(np.float32)
    S_perm = S[:, :, ::-1].copy()
    Sf = S.astype(np.float64)
    for t in range(64):
        q = _unit(rng.standard_normal((n_k, dk))).astype(np.float32)
        k = _unit(rng.standard_normal((n_k, dk))).astype(np.float32)
        v = rng.standard_normal((n_v, dv)).astype(np.float32)
        dec = synth.sigmoid(rng.normal(2, 0.5, n_v)).astype(np.float32)
        bet = synth.sigmoid(rng.normal(0, 1, n_v)).astype(np.float32)
        o = oc.deltanet_step(S, q, k, v, dec, bet, n_v, n_k, dk, dv)
        op = oc.deltanet_step(S_perm, q, k, v[:, ::-1].copy(), dec, bet, n_v, n_k, dk, dv)
        Sf, of = _dn_f64(Sf, q, k, v, dec, bet, n_v, n_k, dk, dv)
        assert np.allclose(op, o[:, ::-1], atol=1e-6)
        assert rel_l2(o, of) < 1e-5
    assert rel_l2(S, Sf) < 1e-5


# ------------------------------------------------------------------------ glue
def test_rmsnorm_and_heads(oc):
    x = synth.activations(1, 256) * 3
    w = synth.activations(2, 256)
    out = np.zeros(256, np.float32)
    oc.lib.oc_rmsnorm(x, w, out, 256)
    ref = x / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6) * w
    assert rel_l2(out, ref) < 1e-6


def test_rope_rotation(oc):
    hd, nh = 256, 4
    inv = np.zeros(hd // 2, np.float32)
    oc.lib.oc_rope_inv_freq(inv, hd, 10000.0)
    assert np.allclose(inv, 1.0 / 10000.0 ** (np.arange(0, hd, 2) / hd), rtol=1e-6)
    x = synth.activations(3, nh * hd)
    for pos in (0, 1, 17, 4095):
        y = x.copy()
        oc.lib.oc_rope(y, nh, hd, pos, inv)
        if pos == 0:
            assert np.array_equal(y, x)
        pairs_x = x.reshape(-1, 2).astype(np.float64)
        pairs_y = y.reshape(-1, 2).astype(np.float64)
        assert np.allclose(np.hypot(*pairs_y.T), np.hypot(*pairs_x.T), rtol=1e-5)
        ang = (np.float32(pos) * np.tile(inv, nh)).astype(np.float64)
        ref = np.stack([pairs_x[:, 0] * np.cos(ang) - pairs_x[:, 1] * np.sin(ang),
                        pairs_x[:, 0] * np.sin(ang) + pairs_x[:, 1] * np.cos(ang)], 1)
        assert rel_l2(pairs_y, ref) < 1e-5


def test_conv_step_tap_major(oc):
    C, Kc = 8, 4
    st = np.zeros(Kc * C, np.float32)
    w = synth.activations(5, Kc * C)
    xs = [synth.activations(10 + t, C) for t in range(6)]
    for t, x in enumerate(xs):
        out = np.zeros(C, np.float32)
        oc.lib.oc_conv_step(st, x, w, out, C, Kc)
        # slot s holds x_{t-s}; weight row (Kc-1-s) pairs with it (qwen_linear.zig:193-201)
        acc = np.zeros(C)
        for s in range(Kc):
            if t - s >= 0:
                acc += xs[t - s].astype(np.float64) * w.reshape(Kc, C)[Kc - 1 - s]
        assert np.allclose(out, acc / (1 + np.exp(-acc)), atol=1e-5)


def test_softplus_l2norm(oc):
    for x in (-30.0, -1.0, 0.0, 0.5, 19.9, 20.0, 20.1, 50.0):
        ref = x if x > 20 else np.log1p(np.exp(x))
        assert abs(oc.lib.oc_softplus(x) - ref) <= 1e-6 * max(1.0, abs(ref))
    x = synth.activations(7, 4 * 128)
    y = x.copy()
    oc.lib.oc_l2norm_heads(y, 4, 128)
    n = np.linalg.norm(x.reshape(4, 128).astype(np.float64), axis=1, keepdims=True)
    assert rel_l2(y, x.reshape(4, 128) / np.sqrt(n ** 2 + 1e-6)) < 1e-6
