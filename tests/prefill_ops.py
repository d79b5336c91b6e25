"""Per-operation parity of chunked prefill against the oracle.

ec_engine_prefill_traced runs one sequence's prefill (chunks of up to 512
tokens, in order) and calls back around every launch; each operation is then
recomputed by the oracle (oracle.c) from the GPU's own inputs, row by row (one
row per token of the chunk), with the tolerances of tests/decoder_ops.py:

  embedding rows             bit-exact
  RMSNorm / gated-norm rows  fp32, relative L2 <= FP_TOL per token; when the
  and SwiGLU rows            op writes the next Q8_0 GEMM's activation itself,
                             that activation against the reference quantizer
                             of the oracle's row (as decoder_ops checks
                             quantized outputs: boundary flips only)
  GEMMs                      the reference quantizer applied to the GPU's fp32
                             input row (Q8_0 per 32 elements, Q4_K per
                             sub-block), or the GPU's own activation where the
                             producing op wrote it, then the oracle's matvec on
                             that activation (+ the residual row for the
                             output projections): relative L2 <= FP_TOL per
                             token
  conv + gates               q, k (L2-normalized), v, decay, beta per token
                             within FP_TOL, the conv ring's new slots bit-exact
  delta rule                 the oracle's token loop from the GPU's state:
                             every token's output and the final state within
                             FP_TOL; chunks of CHUNKED_DELTA_MIN tokens or
                             more run the chunked scan (decay ratios and a
                             triangular solve per 64 tokens: another fp32
                             rounding order than the token loop), bounded by
                             CHUNKED_DELTA_TOL (worst seen 3.1e-5 at 130
                             tokens, 1.9e-5 at the 4B shapes)
  RoPE + KV append           q rows within FP_TOL, KV rows and scales as in
                             decoder_ops (boundary flips only)
  causal attention           the oracle's decode attention of each token over
                             its positions 0 .. p+t, within FP_TOL
  head                       the last token's activation (the engine's pieces)
                             against the reference quantizer of the oracle's
                             final norm (boundary flips only), logits from
                             that activation within FP_TOL
"""
from __future__ import annotations

import numpy as np

from decoder_ops import FP_TOL, QUANT_SLACK, OpChecker, rel_l2
from echohip import engine as E

CHUNK = 512               # ec_engine::kPrefillChunk
CHUNKED_DELTA_MIN = 128   # engine.cpp kChunkedDeltaMin
CHUNKED_DELTA_TOL = 1e-4

_MV_OF = {E.OP_PF_GEMM_IN: E.OP_MV_IN, E.OP_PF_GEMM_OUT: E.OP_MV_OUT, E.OP_PF_GEMM_GU: E.OP_MV_GU,
          E.OP_PF_GEMM_DOWN: E.OP_MV_DOWN}


class PrefillChecker(OpChecker):
    def __init__(self, oc, eng, cfg, m, seq, tokens, pos0, rows_per_matrix=None, seed=0):
        super().__init__(oc, eng, cfg, m, rows_per_matrix, seed)
        self.seq, self.tokens, self.pos0 = seq, np.asarray(tokens, np.int32), pos0
        self.done = 0          # tokens of the chunks before the current one
        self.T = self.p = 0    # current chunk: tokens, first position
        self.started = False
        self.norms = {}        # layer -> NORM events seen in the current chunk

    # ------------------------------------------------------------ helpers
    def _rows(self, which, width, T=None):
        T = self.T if T is None else T
        return self.eng.read_buffer(which, np.float32, 0, T * width).reshape(T, width)

    def _fp_rows(self, op, got, ref, what):
        for t in range(got.shape[0]):
            self._fp(op, got[t], ref[t], f"{what} token {t}")

    def _rows_out(self, op, ev, width, ref, where):
        """A row op's output: fp32 rows, or the Q8_0 GEMM activation it wrote."""
        if ev.x_out == E.B_PF_ACT:
            xq, xd = self.eng.read_gemm_act(E.B_PF_ACT, self.T, width)
            for t in range(self.T):
                self._quant(op, xq[t], xd[t], ref[t], f"{where} token {t} activation")
        else:
            self._fp_rows(op, self._rows(E.B_PF_N, width), ref, where)

    def _sub(self, n):
        """Row subset of an n-row matrix (all rows unless rows_per_matrix)."""
        return OpChecker._rows(self, n)

    # ------------------------------------------------------------ callback
    def _before(self, ev):
        eng, c, op, L = self.eng, self.cfg, ev.op, ev.layer
        b = self.before = {}
        if op == E.OP_PF_EMBED:
            if self.started:
                self.done += self.T
            self.started = True
            self.T = min(CHUNK, self.tokens.size - self.done)
            self.p = self.pos0 + self.done
            self.norms = {}
        elif op == E.OP_PF_NORM:
            b["x"] = self._rows(E.B_PF_X, self.H)
        elif op in _MV_OF:
            W, K, fmt = self._matrix(_MV_OF[op], L)
            if ev.x_in == E.B_PF_ACT:
                b["xq"], b["xd"] = eng.read_gemm_act(E.B_PF_ACT, self.T, K)
            else:
                b["x"] = self._rows(ev.x_in, K)
            if op in (E.OP_PF_GEMM_OUT, E.OP_PF_GEMM_DOWN):
                b["res"] = self._rows(E.B_PF_X, self.H)
        elif op == E.OP_PF_CONV:
            b["proj"] = self._rows(E.B_PF_PROJ, c.nin_delta)
            b["conv"] = eng.get_state(L, E.S_CONV, self.seq)
        elif op == E.OP_PF_DELTA:
            kd = c.key_dim
            b["q"], b["k"] = self._rows(E.B_PF_Q, kd), self._rows(E.B_PF_K, kd)
            b["v"] = self._rows(E.B_PF_V, self.V)
            b["dec"], b["beta"] = self._rows(E.B_PF_DEC, c.ssm_heads), self._rows(E.B_PF_BETA, c.ssm_heads)
            b["ssm"] = eng.get_state(L, E.S_SSM, self.seq)
        elif op == E.OP_PF_GATED_NORM:
            b["core"] = self._rows(E.B_PF_CORE, self.V)
            b["proj"] = self._rows(E.B_PF_PROJ, c.nin_delta)
        elif op == E.OP_PF_ROPE_APPEND:
            b["proj"] = self._rows(E.B_PF_PROJ, c.nin_attn)
        elif op == E.OP_PF_ATTN:
            b["q"] = self._rows(E.B_PF_N, self.q_dim)
            b["kv"] = [eng.get_state(L, w, self.seq) for w in (E.S_KEYS, E.S_VALS, E.S_KSCALES, E.S_VSCALES)]
        elif op == E.OP_PF_SWIGLU:
            b["gu"] = self._rows(E.B_PF_GU, 2 * self.F)
        elif op == E.OP_PF_HEAD:
            b["x"] = self._rows(E.B_PF_X, self.H)[self.T - 1]

    def _after(self, ev):
        eng, oc, c, op, L, b = self.eng, self.oc, self.cfg, ev.op, ev.layer, self.before
        T, where = self.T, f"prefill op {op} layer {L} chunk at {self.p}"
        if op == E.OP_PF_EMBED:
            x = self._rows(E.B_PF_X, self.H)
            fmt = self._fmt(-1, "embed")
            toks = self.tokens[self.done:self.done + T]
            for t in range(T):
                assert np.array_equal(x[t], oc.embed_row(fmt, self.m["embed"], self.H, toks[t])), f"{where} token {t}"
            self._note(op)
        elif op == E.OP_PF_NORM:
            n = self.norms.get(L, 0)
            self.norms[L] = n + 1
            w = self.m["layers"][L]["ffn_norm" if n % 2 else "attn_norm"]
            self._rows_out(op, ev, self.H, np.stack([oc.rmsnorm(b["x"][t], w) for t in range(T)]), where)
        elif op in _MV_OF:
            W, K, fmt = self._matrix(_MV_OF[op], L)
            N = W.shape[0]
            got = self._rows(ev.x_out, N)
            rows = self._sub(N)
            Wr = np.ascontiguousarray(W[rows])
            for t in range(T):
                if "xq" in b:
                    ref = oc.matvec_q8_0(Wr, oc.dequant_act_q8_0(b["xq"][t], b["xd"][t]))
                elif fmt == E.Q4_K:
                    xq, xd, _ = oc.quantize_act_q4_K(b["x"][t])
                    ref = oc.matvec_q4_K(Wr, oc.dequant_act_q4_K(xq, xd))
                else:
                    xq, xd = oc.quantize_act_q8_0(b["x"][t])
                    ref = oc.matvec_q8_0(Wr, oc.dequant_act_q8_0(xq, xd))
                if "res" in b:
                    ref = (b["res"][t][rows] + ref).astype(np.float32)
                self._fp(op, got[t][rows], ref, f"{where} token {t}")
        elif op == E.OP_PF_CONV:
            self._check_conv(L, b, where)
        elif op == E.OP_PF_DELTA:
            self._check_delta_chunk(L, b, where)
        elif op == E.OP_PF_GATED_NORM:
            y = self.m["layers"][L]
            z0 = c.conv_dim
            ref = np.stack([oc.gated_rmsnorm(b["core"][t], b["proj"][t][z0:z0 + self.V], y["ssm_norm"],
                                             c.ssm_heads, 128).reshape(-1) for t in range(T)])
            self._rows_out(op, ev, self.V, ref, where)
        elif op == E.OP_PF_ROPE_APPEND:
            self._check_rope_chunk(L, b, where)
        elif op == E.OP_PF_ATTN:
            got = self._rows(E.B_PF_ATTN, self.q_dim)
            keys, vals, ks, vs = b["kv"]
            for t in range(T):
                ctx = self.p + t + 1
                ref = oc.attn_decode(b["q"][t], keys[:ctx * self.kv_dim], vals[:ctx * self.kv_dim],
                                     ks[:ctx * c.n_kv], vs[:ctx * c.n_kv], c.n_heads, c.n_kv, c.head_dim,
                                     ctx).reshape(-1)
                self._fp(op, got[t], ref, f"{where} token {t}")
        elif op == E.OP_PF_SWIGLU:
            F = self.F
            self._rows_out(op, ev, F, np.stack([oc.swiglu(g[:F], g[F:]) for g in b["gu"]]), where)
        elif op == E.OP_PF_HEAD:
            W, K, fmt = self._matrix(E.OP_LM_HEAD, -1)
            xq, xd = eng.read_act(E.B_PF_ACT1, self.H, M=1, fmt=fmt)
            self._quant(op, xq[0], xd[0], oc.rmsnorm(b["x"], self.m["final_norm"]), f"{where} head activation", fmt)
            rows = self._sub(W.shape[0])
            Wr = np.ascontiguousarray(W[rows])
            x = self._dequant(xq[0], xd[0], fmt)
            ref = oc.matvec_q4_K(Wr, x) if fmt == E.Q4_K else oc.matvec_q8_0(Wr, x)
            logits = eng.read_buffer(E.B_LOGITS, np.float32, self.seq * c.vocab, c.vocab)
            self._fp(op, logits[rows], ref, f"{where} logits")

    def _check_conv(self, L, b, where):
        eng, oc, c, y = self.eng, self.oc, self.cfg, self.m["layers"][L]
        n_v, kd, kern, C_ = c.ssm_heads, c.key_dim, c.conv_kernel, c.conv_dim
        n_k = kd // 128
        V = self.V
        T, p = self.T, self.p
        q, k = self._rows(E.B_PF_Q, kd), self._rows(E.B_PF_K, kd)
        v = self._rows(E.B_PF_V, V)
        dec, bet = self._rows(E.B_PF_DEC, n_v), self._rows(E.B_PF_BETA, n_v)
        ring = b["conv"].reshape(kern, C_)
        st = np.zeros((kern, C_), np.float32)  # newest first, before the chunk's first token
        for i in range(kern):
            if p - 1 - i >= 0:
                st[i] = ring[(p - 1 - i) % kern]
        for t in range(T):
            pr = b["proj"][t]
            conv = oc.conv_step(st, pr[:C_], y["conv_w"], C_, kern)  # advances st
            self._fp(E.OP_PF_CONV, q[t], oc.l2norm_heads(conv[:kd], n_k, 128).reshape(-1), f"{where} token {t} q")
            self._fp(E.OP_PF_CONV, k[t], oc.l2norm_heads(conv[kd:2 * kd], n_k, 128).reshape(-1),
                     f"{where} token {t} k")
            self._fp(E.OP_PF_CONV, v[t], conv[2 * kd:], f"{where} token {t} v")
            a0 = C_ + V
            dref, bref = oc.deltanet_gates(pr[a0:a0 + n_v], pr[a0 + n_v:a0 + 2 * n_v], y["a_log"], y["dt_bias"])
            self._fp(E.OP_PF_CONV, dec[t], dref, f"{where} token {t} decay")
            self._fp(E.OP_PF_CONV, bet[t], bref, f"{where} token {t} beta")
        ring_after = eng.get_state(L, E.S_CONV, self.seq).reshape(kern, C_)
        for t in range(max(0, T - kern), T):
            assert np.array_equal(ring_after[(p + t) % kern], b["proj"][t][:C_]), f"{where}: conv ring slot {t}"

    def _check_delta_chunk(self, L, b, where):
        eng, oc, c = self.eng, self.oc, self.cfg
        n_v, n_k = c.ssm_heads, c.key_dim // 128
        got = self._rows(E.B_PF_CORE, self.V)
        tol = CHUNKED_DELTA_TOL if self.T >= CHUNKED_DELTA_MIN else FP_TOL
        S = np.ascontiguousarray(b["ssm"].reshape(n_v, 128, 128).transpose(0, 2, 1))  # reference [k][v]

        def cmp(g, r, what):
            err = rel_l2(g, r)
            self._note(E.OP_PF_DELTA, err)
            assert err <= tol, f"{what}: rel_l2 {err:.3e} > {tol}"
        for t in range(self.T):
            ref = oc.deltanet_step(S, b["q"][t], b["k"][t], b["v"][t], b["dec"][t], b["beta"][t], n_v, n_k, 128, 128)
            cmp(got[t], ref, f"{where} token {t}")
        S_gpu = eng.get_state(L, E.S_SSM, self.seq).reshape(n_v, 128, 128).transpose(0, 2, 1)
        cmp(S_gpu, S, f"{where} recurrent state")

    def _check_rope_chunk(self, L, b, where):
        eng, oc, c, y = self.eng, self.oc, self.cfg, self.m["layers"][L]
        hd = c.head_dim
        qrows = self._rows(E.B_PF_N, self.q_dim)
        keys = eng.get_state(L, E.S_KEYS, self.seq)
        vals = eng.get_state(L, E.S_VALS, self.seq)
        kss = eng.get_state(L, E.S_KSCALES, self.seq)
        vss = eng.get_state(L, E.S_VSCALES, self.seq)
        for t in range(self.T):
            pos = self.p + t
            pr = b["proj"][t]
            q, k, v = pr[:self.q_dim], pr[self.q_dim:self.q_dim + self.kv_dim], pr[self.q_dim + self.kv_dim:]
            if np.any(y["q_norm"] != 0):
                q = oc.head_rmsnorm(q, y["q_norm"], c.n_heads, hd)
            if np.any(y["k_norm"] != 0):
                k = oc.head_rmsnorm(k, y["k_norm"], c.n_kv, hd)
            q = oc.rope(q, c.n_heads, hd, pos, c.rope_base)
            k = oc.rope(k, c.n_kv, hd, pos, c.rope_base)
            self._fp(E.OP_PF_ROPE_APPEND, qrows[t], q.reshape(-1), f"{where} token {t} q")
            for cache, scs, src in ((keys, kss, k), (vals, vss, v)):
                row = cache[pos * self.kv_dim:(pos + 1) * self.kv_dim].reshape(c.n_kv, hd)
                sc = scs[pos * c.n_kv:(pos + 1) * c.n_kv]
                rq, rs = oc.quantize(src, hd)
                assert np.allclose(sc, rs, rtol=1e-5, atol=0), f"{where} token {t}: KV scales"
                diff = row.astype(np.int32) - rq.astype(np.int32)
                tt = src.reshape(c.n_kv, hd).astype(np.float64) / rs[:, None]
                near = np.abs(np.abs(tt - np.floor(tt)) - 0.5) < QUANT_SLACK
                assert not ((diff != 0) & ~near).any() and np.abs(diff).max() <= 1, f"{where} token {t}: KV row"
                self.flips[0] += int((diff != 0).sum())
                self.flips[1] += diff.size


__all__ = ["PrefillChecker", "rel_l2"]
