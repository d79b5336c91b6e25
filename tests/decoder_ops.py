"""Per-operation parity of the GPU decode step against the oracle.

The engine's decode step is run with ec_engine_step_traced: around every
launch the stream is drained and the checker reads the operation's inputs
(before) and outputs (after) from the engine's buffers.  Each operation is then
recomputed by the oracle (oracle.c) from the GPU's own inputs, so every
comparison measures that one operation:

  integer and copy work  bit-exact (embedding rows, the residual + partial-sum
                         adds, the conv ring write, KV scales' rows, greedy token)
  fp32 outputs           relative L2 <= FP_TOL per sequence (matvec sums, the
                         delta-rule state, attention output, packed q)
  int8 activations       the reference quantizer applied to the oracle's fp32
                         value: block scales within FP32_SCALE_TOL (of the
                         vector's largest scale), every int8 equal except an
                         element whose x/scale lies within the scale difference
                         or QUANT_SLACK of a rounding boundary (there the two
                         fp32 values may round to neighbours), such flips at
                         most MAX_FLIP_FRACTION of the elements.  With two
                         pieces (the engine's default) piece 0 is held to that,
                         and the two-piece value s*(q0 + q1/256): per element
                         within two piece-1 steps of the oracle's two-piece
                         quantizer of its fp32 value (each side errs by at most
                         s/512) plus QUANT_SLACK of the vector's largest scale
                         (fp32 differences of the two producers scale with the
                         vector, not with a block whose values are small), and
                         over the vector within TWO_PIECE_TOL relative L2 of
                         the oracle's fp32 value.  Piece 1 resolves the input
                         256x finer than piece 0, so fp32 differences between
                         the producers flip it far more often (reported).

A quantization launch of the GPU's own fp32 rows (QUANT_ACT) is compared bit
for bit with the reference quantizer.  Matrices stored as Q4_K read a Q4_K
activation (per 32-element sub-block, in the quantizer's sub-block order) and
are checked against the oracle's Q4_K matvec; their producers write fp32 rows
(NORM_ROWS, the delta step's fp32 output, SwiGLU rows), checked within FP_TOL.

Matrices are compared on a subset of rows when `rows_per_matrix` is set (the
4B-shape run); every row otherwise.
"""
from __future__ import annotations

import numpy as np

from echohip import engine as E

FP_TOL = 1e-5          # fp32 outputs vs the oracle on the same inputs
MAX_FLIP_FRACTION = 0.01  # boundary flips allowed over all int8 elements compared
FP32_SCALE_TOL = 1e-4  # block scale difference, relative to the vector's largest block scale
QUANT_SLACK = 2e-3     # |x/scale - (k + 1/2)| below which an int8 may differ by one
TWO_PIECE_TOL = 6e-5   # two-piece activation vs the oracle's fp32 value: FP_TOL + the pieces' own ~3e-5


def rel_l2(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))


class OpChecker:
    def __init__(self, oc, eng, cfg, m, rows_per_matrix=None, seed=0):
        self.fmts = m.get("fmt", {})
        self.oc, self.eng, self.cfg, self.m = oc, eng, cfg, m
        self.B = cfg.max_batch
        self.H, self.F = cfg.hidden, cfg.ffn
        self.q_dim, self.kv_dim = cfg.n_heads * cfg.head_dim, cfg.n_kv * cfg.head_dim
        self.V = cfg.ssm_inner
        self.rng = np.random.default_rng(seed)
        self.rows_per_matrix = rows_per_matrix
        self.before = {}
        self.counts = {}     # op -> number of (op, sequence) comparisons made
        self.worst = {}      # op -> worst fp32 relative error seen
        self.flips = [0, 0]  # int8 elements that differ by one at a boundary, elements compared
        self.flips2 = [0, 0]  # two-piece values (256 q0 + q1) that differ, elements compared

    # ------------------------------------------------------------- helpers
    def _note(self, op, err=None):
        self.counts[op] = self.counts.get(op, 0) + 1
        if err is not None:
            self.worst[op] = max(self.worst.get(op, 0.0), err)

    def _fp(self, op, got, ref, what):
        err = rel_l2(got, ref)
        self._note(op, err)
        assert err <= FP_TOL, f"{what}: rel_l2 {err:.3e} > {FP_TOL}"

    def _fmt(self, layer, name):
        return self.fmts.get((layer, name), E.Q8_0)

    def _sub_order(self, K):
        """Index into a K vector of each element of a Q4_K activation (sub-block order)."""
        if getattr(self, "_perm_k", None) != K:
            pos = np.array([self.oc.lib.oc_q4k_pos(s, i) for s in range(8) for i in range(32)], np.int64)
            self._perm = (256 * np.arange(K // 256)[:, None] + pos[None, :]).reshape(-1)
            self._perm_k = K
        return self._perm

    def _width(self, which):
        """Elements per row of an fp32 step buffer or an activation buffer."""
        return {E.B_ACT_H: self.H, E.B_ACT4_H: self.H, E.B_HN: self.H, E.B_ACT_V: self.V, E.B_ACT4_V: self.V,
                E.B_CORE: self.V, E.B_ACT_F: self.F, E.B_ACT4_F: self.F, E.B_FF: self.F, E.B_ACT_Q: self.q_dim,
                E.B_ACT4_Q: self.q_dim, E.B_ATTN_OUT: self.q_dim}[which]

    def _rows_f32(self, which):
        K = self._width(which)
        return self.eng.read_buffer(which, np.float32, 0, self.B * K).reshape(self.B, K)

    def _dequant(self, xq, xd, fmt):
        """fp32 value of a GPU activation row: xq [K] or [1][K] (one piece) or [2][K] (two pieces)."""
        xq = np.asarray(xq)
        oc = self.oc
        if xq.ndim == 2 and xq.shape[0] == 2:
            return oc.dequant_act2_q4_K(xq[0], xq[1], xd) if fmt == E.Q4_K else oc.dequant_act2_q8_0(xq[0], xq[1], xd)
        q = xq.reshape(-1)
        return oc.dequant_act_q4_K(q, xd) if fmt == E.Q4_K else oc.dequant_act_q8_0(q, xd)

    def _quant(self, op, xq, xd, ref, what, fmt=E.Q8_0):
        """GPU int8 block activation (xq, xd) against the reference quantizer of the oracle's fp32 `ref`.

        The GPU quantizes its own fp32 value g (bit-exact reference quantizer,
        pinned by the kernel tests); g differs from the oracle's `ref` by fp32
        rounding.  So: each block scale within FP32_SCALE_TOL of the oracle's
        (a block of elements much smaller than the vector's norm carries a
        larger relative error: the bound is relative to the vector's largest
        scale), and every int8 equal to the oracle's except where x/scale is
        within the scale difference or QUANT_SLACK of a rounding boundary
        (there the neighbour is allowed), such flips at most
        MAX_FLIP_FRACTION of all elements compared.  The dequantized vectors'
        relative L2 is reported (one flip moves a block by one quantum).
        xq [P][K] with P = 2: piece 0 as above, then the two-piece values."""
        ref = np.ascontiguousarray(ref, np.float32)
        xq = np.asarray(xq)
        xq1 = xq[1] if xq.ndim == 2 and xq.shape[0] == 2 else None
        xq = xq.reshape(-1) if xq.ndim == 1 else xq[0]
        if xq1 is not None:
            r2 = self.oc.quantize_act2_q4_K(ref) if fmt == E.Q4_K else self.oc.quantize_act2_q8_0(ref)
        if fmt == E.Q4_K:
            rq, rd, _ = self.oc.quantize_act_q4_K(ref)
            ref = ref[self._sub_order(ref.size)]
        else:
            rq, rd = self.oc.quantize_act_q8_0(ref)
        xd64, rd64 = xd.astype(np.float64), rd.astype(np.float64)
        sdev = np.abs(xd64 - rd64) / max(rd64.max(initial=0.0), 1e-30)
        self.scale_dev = max(getattr(self, "scale_dev", 0.0), float(sdev.max(initial=0.0)))
        assert sdev.max(initial=0.0) <= FP32_SCALE_TOL, f"{what}: block scale off by {sdev.max():.2e} of the largest"
        diff = xq.astype(np.int32) - rq.astype(np.int32)
        t = ref.astype(np.float64) / np.repeat(rd64, 32)
        slack = QUANT_SLACK + 127.0 * np.repeat(np.abs(xd64 - rd64) / np.maximum(rd64, 1e-30), 32)
        near = np.abs(np.abs(t - np.floor(t)) - 0.5) < slack
        bad = (diff != 0) & ~near
        assert not bad.any(), f"{what}: {int(bad.sum())} int8 values differ away from a rounding boundary"
        assert np.abs(diff).max(initial=0) <= 1, f"{what}: int8 values differ by more than one"
        deq = xq.astype(np.float64) * np.repeat(xd64, 32)
        rdeq = rq.astype(np.float64) * np.repeat(rd64, 32)
        self.act_dev = max(getattr(self, "act_dev", 0.0), rel_l2(deq, rdeq))  # reported: a flip moves one quantum
        self.flips[0] += int((diff != 0).sum())
        self.flips[1] += diff.size
        assert self.flips[0] <= MAX_FLIP_FRACTION * self.flips[1], f"{what}: too many boundary flips {self.flips}"
        if xq1 is not None:
            s_g, s_r = np.repeat(xd64, 32), np.repeat(rd64, 32)
            t_g = 256.0 * xq.astype(np.float64) + xq1
            t_r = 256.0 * r2[0].astype(np.float64) + r2[1]
            dev = np.abs(t_g * s_g - t_r * s_r) / 256.0
            smax = max(rd64.max(initial=0.0), 1e-30)
            tol = s_r * (2.04 / 256.0) + QUANT_SLACK * smax + 128.0 * np.abs(s_g - s_r)
            assert np.all(dev <= tol), f"{what}: two-piece value off by {np.max(dev) / smax:.2e} of the largest scale"
            err = rel_l2(t_g * s_g / 256.0, ref)
            assert err <= TWO_PIECE_TOL, f"{what}: two-piece activation rel_l2 {err:.2e} from the oracle's fp32 value"
            self.flips2[0] += int((t_g != t_r).sum())
            self.flips2[1] += t_g.size
            self.act2_dev = max(getattr(self, "act2_dev", 0.0), err)
        self._note(op)

    def _active(self):
        return [s for s in range(self.B) if self.before["pos"][s] >= 0]

    def _parts(self, which, nparts, width):
        a = self.eng.read_buffer(which, np.float32, 0, max(nparts, 1) * self.B * width)
        return a.reshape(max(nparts, 1), self.B, width)

    @staticmethod
    def _sum_parts(p):
        acc = p[0].copy()
        for i in range(1, p.shape[0]):
            acc = (acc + p[i]).astype(np.float32)
        return acc

    def _rows(self, n):
        if self.rows_per_matrix is None or self.rows_per_matrix >= n:
            return np.arange(n)
        return np.sort(self.rng.choice(n, self.rows_per_matrix, replace=False))

    def _matrix(self, op, layer):
        """(GGUF rows [N][row bytes], K, format) of the op's matrix."""
        y = self.m["layers"][layer] if layer >= 0 else None

        def rows(w, K, name):
            fmt = self._fmt(layer, name)
            return np.asarray(w).reshape(-1, E.gguf_row_bytes(fmt, K)), K, fmt
        if op == E.OP_MV_IN:
            return rows(y["w_in"], self.H, "w_in")
        if op == E.OP_MV_OUT:
            return rows(y["w_out"], self.q_dim if y["attn"] else self.V, "w_out")
        if op == E.OP_MV_GU:
            return rows(np.concatenate([np.asarray(y["w_gate"]).reshape(-1), np.asarray(y["w_up"]).reshape(-1)]),
                        self.H, "w_gate")
        if op == E.OP_MV_DOWN:
            return rows(y["w_down"], self.F, "w_down")
        return rows(self.m["lm_head"], self.H, "lm_head")

    def _decode_q(self, qa, qsc, s):
        """q [n_heads][head_dim] from the three-piece int8 layout (csrc/layout.hpp)."""
        c = self.cfg
        G, P = c.n_heads // c.n_kv, 3
        d = np.arange(c.head_dim)
        gq, at = (d % 64) // 16, (2 * (d // 64) + (d % 16) // 8) * 8 + d % 8
        q = np.zeros((c.n_heads, c.head_dim), np.float64)
        for kvh in range(c.n_kv):
            base = (s * c.n_kv + kvh) * (P * G) * 4 * 64
            for g in range(G):
                for pc in range(P):
                    row = pc * G + g
                    piece = qa[base + (row * 4 + gq) * 64 + at].astype(np.float64)
                    q[kvh + c.n_kv * g] += piece * qsc[(s * c.n_kv + kvh) * P * G + row]
        return q

    # ------------------------------------------------------------ callback
    def __call__(self, ev):
        if ev.phase == 0:
            self._before(ev)
        else:
            self._after(ev)

    def _before(self, ev):
        eng, c, op, L = self.eng, self.cfg, ev.op, ev.layer
        b = self.before = {"pos": eng.read_buffer(E.B_POS, np.int32)}
        if op == E.OP_EMBED:
            b["tok"] = eng.read_buffer(E.B_TOK, np.int32)
        elif op == E.OP_NORM:
            b["x"] = eng.read_buffer(ev.x_in, np.float32, 0, self.B * self.H).reshape(self.B, self.H)
            if ev.nparts:
                b["parts"] = self._parts(E.B_PARTS, ev.nparts, self.H)
        elif op in (E.OP_MV_IN, E.OP_MV_OUT, E.OP_MV_GU, E.OP_MV_DOWN, E.OP_LM_HEAD):
            b["xq"], b["xd"] = eng.read_act(ev.x_in, self._width(ev.x_in))
        elif op in (E.OP_NORM_ROWS, E.OP_QUANT_ACT):
            b["rows"] = self._rows_f32(ev.x_in) if op == E.OP_QUANT_ACT else \
                eng.read_buffer(ev.x_in, np.float32, 0, self.B * self.H).reshape(self.B, self.H)
        elif op == E.OP_DELTA_STEP:
            b["proj"] = self._parts(E.B_PROJ, ev.nparts, c.nin_delta)
            b["conv"] = {s: eng.get_state(L, E.S_CONV, s) for s in self._active()}
            b["ssm"] = {s: eng.get_state(L, E.S_SSM, s) for s in self._active()}
        elif op == E.OP_ROPE_APPEND:
            b["proj"] = self._parts(E.B_PROJ, ev.nparts, c.nin_attn)
        elif op == E.OP_ATTN:
            b["qa"] = eng.read_buffer(E.B_Q_PACKED, np.int8)
            b["qsc"] = eng.read_buffer(E.B_Q_SCALES, np.float32)
            b["ctx"] = eng.read_buffer(E.B_CTX, np.int32)
            b["kv"] = {s: [eng.get_state(L, w, s) for w in (E.S_KEYS, E.S_VALS, E.S_KSCALES, E.S_VSCALES)]
                       for s in self._active()}
        elif op == E.OP_SWIGLU:
            b["gu"] = self._parts(E.B_GU, ev.nparts, 2 * self.F)
        elif op == E.OP_ARGMAX:
            b["logits"] = eng.read_buffer(E.B_LOGITS, np.float32).reshape(self.B, c.vocab)

    def _after(self, ev):
        eng, oc, c, op, L, b = self.eng, self.oc, self.cfg, ev.op, ev.layer, self.before
        act = self._active()
        where = f"op {op} layer {L}"
        if op == E.OP_EMBED:
            x = eng.read_buffer(E.B_X, np.float32, 0, self.B * self.H).reshape(self.B, self.H)
            fmt = self._fmt(-1, "embed")
            for s in act:
                assert np.array_equal(x[s], oc.embed_row(fmt, self.m["embed"], self.H, b["tok"][s])), where
                self._note(op)
        elif op == E.OP_NORM:
            w = self.m["final_norm"] if L < 0 else \
                self.m["layers"][L]["ffn_norm" if self._norm_is_ffn(L) else "attn_norm"]
            self.norm_w = w
            xo = eng.read_buffer(ev.x_out, np.float32, 0, self.B * self.H).reshape(self.B, self.H)
            xq, xd = eng.read_act(E.B_ACT_H, self.H)
            xin = b["x"]
            if ev.nparts:
                xin = self._sum_parts(np.concatenate([b["x"][None], b["parts"]]))
            for s in act:
                assert np.array_equal(xo[s], xin[s]), f"{where}: residual + partial sums not bit-exact"
                self._quant(op, xq[s], xd[s], oc.rmsnorm(xin[s], w), f"{where} seq {s}")
        elif op == E.OP_NORM_ROWS:
            hn = self._rows_f32(ev.x_out)
            for s in act:
                self._fp(op, hn[s], oc.rmsnorm(b["rows"][s], self.norm_w), f"{where} seq {s}")
        elif op == E.OP_QUANT_ACT:
            K = self._width(ev.x_out)
            xq, xd = eng.read_act(ev.x_out, K)
            q4 = ev.x_out in E.ACT4_BUFFERS
            for s in act:
                if xq.shape[1] == 2:
                    rq0, rq1, rd = (oc.quantize_act2_q4_K if q4 else oc.quantize_act2_q8_0)(b["rows"][s])
                    ok = np.array_equal(xq[s][0], rq0) and np.array_equal(xq[s][1], rq1)
                else:
                    rq, rd = (oc.quantize_act_q4_K(b["rows"][s])[:2] if q4 else oc.quantize_act_q8_0(b["rows"][s]))
                    ok = np.array_equal(xq[s][0], rq)
                assert ok and np.array_equal(xd[s], rd), \
                    f"{where} seq {s}: quantized activation of the GPU's rows not bit-exact"
                self._note(op)
        elif op in (E.OP_MV_IN, E.OP_MV_OUT, E.OP_MV_GU, E.OP_MV_DOWN, E.OP_LM_HEAD):
            W, K, fmt = self._matrix(op, L)
            assert (ev.x_in in E.ACT4_BUFFERS) == (fmt == E.Q4_K), f"{where}: activation format"
            N = W.shape[0]
            if op == E.OP_LM_HEAD:
                y = eng.read_buffer(E.B_LOGITS, np.float32).reshape(self.B, N)
            else:
                buf = {E.OP_MV_IN: E.B_PROJ, E.OP_MV_GU: E.B_GU}.get(op, E.B_PARTS)
                y = self._sum_parts(self._parts(buf, ev.nparts, N))
            rows = self._rows(N)
            Wr = np.ascontiguousarray(W[rows])
            for s in act:
                x = self._dequant(b["xq"][s], b["xd"][s], fmt)
                ref = oc.matvec_q4_K(Wr, x) if fmt == E.Q4_K else oc.matvec_q8_0(Wr, x)
                self._fp(op, y[s][rows], ref, f"{where} seq {s}")
        elif op == E.OP_DELTA_STEP:
            self._check_delta(L, act, b, where, ev.x_out)
        elif op == E.OP_ROPE_APPEND:
            self._check_rope(L, act, b, where)
        elif op == E.OP_ATTN:
            out = eng.read_buffer(E.B_ATTN_OUT, np.float32, 0, self.B * self.q_dim).reshape(self.B, self.q_dim)
            xq, xd = eng.read_act(E.B_ACT_Q, self.q_dim) if ev.x_out == E.B_ACT_Q else (None, None)
            for s in act:
                q = self._decode_q(b["qa"], b["qsc"], s).astype(np.float32)
                keys, vals, ks, vs = b["kv"][s]
                ctx = int(b["ctx"][s])
                assert ctx == b["pos"][s] + 1, where
                ref = oc.attn_decode(q, keys[:ctx * self.kv_dim], vals[:ctx * self.kv_dim], ks[:ctx * c.n_kv],
                                     vs[:ctx * c.n_kv], c.n_heads, c.n_kv, c.head_dim, ctx).reshape(-1)
                self._fp(op, out[s], ref, f"{where} seq {s} attention")
                if xq is not None:
                    self._quant(op, xq[s], xd[s], ref, f"{where} seq {s} attention activation")
        elif op == E.OP_SWIGLU:
            gu = self._sum_parts(b["gu"])
            if ev.x_out == E.B_FF:
                ff = self._rows_f32(E.B_FF)
                for s in act:
                    self._fp(op, ff[s], oc.swiglu(gu[s][:self.F], gu[s][self.F:]), f"{where} seq {s} rows")
            else:
                xq, xd = eng.read_act(E.B_ACT_F, self.F)
                for s in act:
                    self._quant(op, xq[s], xd[s], oc.swiglu(gu[s][:self.F], gu[s][self.F:]), f"{where} seq {s}")
        elif op == E.OP_ARGMAX:
            gen = eng.read_buffer(E.B_GEN, np.int32)
            pos = eng.read_buffer(E.B_POS, np.int32)
            for s in act:
                lg = b["logits"][s]
                assert gen[s] == int(np.flatnonzero(lg == lg.max())[0]), where
                p1 = b["pos"][s] + 1
                assert pos[s] == (p1 if p1 < c.max_ctx else -1), where
                self._note(op)

    def _norm_is_ffn(self, L):
        # the first NORM of a block reads attn_norm, the second ffn_norm
        key = ("norm", L)
        n = self.counts.get(key, 0)
        self.counts[key] = n + 1
        return n % 2 == 1

    def _check_delta(self, L, act, b, where, x_out):
        eng, oc, c, y = self.eng, self.oc, self.cfg, self.m["layers"][L]
        n_v, kd = c.ssm_heads, c.key_dim
        n_k, C_, kern = kd // 128, c.conv_dim, c.conv_kernel
        proj = self._sum_parts(b["proj"])
        fp_out = x_out == E.B_CORE
        if fp_out:
            core_f = self._rows_f32(E.B_CORE)
        else:
            xq, xd = eng.read_act(E.B_ACT_V, self.V)
        for s in act:
            p = int(b["pos"][s])
            pr = proj[s]
            a, z = pr[:C_], pr[C_:C_ + self.V]
            alpha, beta_l = pr[C_ + self.V:C_ + self.V + n_v], pr[C_ + self.V + n_v:C_ + self.V + 2 * n_v]
            ring = b["conv"][s].reshape(kern, C_)
            st = np.zeros((kern, C_), np.float32)  # newest first, before this token
            for t in range(kern):
                if p - 1 - t >= 0:
                    st[t] = ring[(p - 1 - t) % kern]
            conv = oc.conv_step(st, a, y["conv_w"], C_, kern)
            qn = oc.l2norm_heads(conv[:kd], n_k, 128)
            kn = oc.l2norm_heads(conv[kd:2 * kd], n_k, 128)
            v = conv[2 * kd:]
            dec, bet = oc.deltanet_gates(alpha, beta_l, y["a_log"], y["dt_bias"])
            S = np.ascontiguousarray(b["ssm"][s].reshape(n_v, 128, 128).transpose(0, 2, 1))
            core = oc.deltanet_step(S, qn, kn, v, dec, bet, n_v, n_k, 128, 128)
            g = oc.gated_rmsnorm(core, z, y["ssm_norm"], n_v, 128).reshape(-1)
            if fp_out:
                self._fp(E.OP_DELTA_STEP, core_f[s], g, f"{where} seq {s} gated-norm rows")
            else:
                self._quant(E.OP_DELTA_STEP, xq[s], xd[s], g, f"{where} seq {s} gated-norm activation")
            S_gpu = eng.get_state(L, E.S_SSM, s).reshape(n_v, 128, 128).transpose(0, 2, 1)
            self._fp(E.OP_DELTA_STEP, S_gpu, S, f"{where} seq {s} recurrent state")
            ring_after = eng.get_state(L, E.S_CONV, s).reshape(kern, C_)
            assert np.array_equal(ring_after[p % kern], a), f"{where} seq {s}: conv ring slot"

    def _check_rope(self, L, act, b, where):
        eng, oc, c, y = self.eng, self.oc, self.cfg, self.m["layers"][L]
        proj = self._sum_parts(b["proj"])
        qa = eng.read_buffer(E.B_Q_PACKED, np.int8)
        qsc = eng.read_buffer(E.B_Q_SCALES, np.float32)
        ctx = eng.read_buffer(E.B_CTX, np.int32)
        hd = c.head_dim
        for s in act:
            p = int(b["pos"][s])
            pr = proj[s]
            q, k, v = pr[:self.q_dim], pr[self.q_dim:self.q_dim + self.kv_dim], pr[self.q_dim + self.kv_dim:]
            if np.any(y["q_norm"] != 0):
                q = oc.head_rmsnorm(q, y["q_norm"], c.n_heads, hd)
            if np.any(y["k_norm"] != 0):
                k = oc.head_rmsnorm(k, y["k_norm"], c.n_kv, hd)
            q = oc.rope(q, c.n_heads, hd, p, c.rope_base)
            k = oc.rope(k, c.n_kv, hd, p, c.rope_base)
            self._fp(E.OP_ROPE_APPEND, self._decode_q(qa, qsc, s).reshape(-1), q, f"{where} seq {s} packed q")
            assert ctx[s] == p + 1, f"{where} seq {s}: ctx"
            for which, ws, src in ((E.S_KEYS, E.S_KSCALES, k), (E.S_VALS, E.S_VSCALES, v)):
                row = eng.get_state(L, which, s)[p * self.kv_dim:(p + 1) * self.kv_dim].reshape(c.n_kv, hd)
                sc = eng.get_state(L, ws, s)[p * c.n_kv:(p + 1) * c.n_kv]
                rq, rs = oc.quantize(src, hd)  # one scale per (token, kv head)
                assert np.allclose(sc, rs, rtol=1e-5, atol=0), f"{where} seq {s}: KV scales"
                diff = row.astype(np.int32) - rq.astype(np.int32)
                t = src.reshape(c.n_kv, hd).astype(np.float64) / rs[:, None]
                near = np.abs(np.abs(t - np.floor(t)) - 0.5) < QUANT_SLACK
                assert not ((diff != 0) & ~near).any() and np.abs(diff).max() <= 1, f"{where} seq {s}: KV row"
                self.flips[0] += int((diff != 0).sum())
                self.flips[1] += diff.size

    def summary(self):
        ops = {v: k for k, v in vars(E).items() if k.startswith("OP_")}
        parts = [f"{ops.get(k, k)}:{n}" for k, n in self.counts.items() if not isinstance(k, tuple)]
        worst = " ".join(f"{ops.get(k, k)}={v:.1e}" for k, v in self.worst.items())
        return (f"checks {' '.join(parts)}; worst fp32 rel_l2 {worst}; int8 flips {self.flips[0]}/{self.flips[1]}; "
                f"two-piece value flips {self.flips2[0]}/{self.flips2[1]}; "
                f"worst block-scale deviation {getattr(self, 'scale_dev', 0.0):.1e}, "
                f"dequantized activation rel_l2 {getattr(self, 'act_dev', 0.0):.1e} "
                f"(two-piece, vs the oracle's fp32 value: {getattr(self, 'act2_dev', 0.0):.1e})")
