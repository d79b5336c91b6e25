"""ctypes binding of the device-resident hybrid decoder (include/echo_engine.h)."""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, fields

import numpy as np

from .lib import EchoHipError, load

T_EMBED, T_FINAL_NORM, T_LM_HEAD = 0, 1, 2
T_ATTN_NORM, T_FFN_NORM, T_W_IN, T_W_OUT, T_W_GATE, T_W_UP, T_W_DOWN = 10, 11, 12, 13, 14, 15, 16
T_CONV_W, T_A_LOG, T_DT_BIAS, T_SSM_NORM, T_Q_NORM, T_K_NORM = 17, 18, 19, 20, 21, 22
S_CONV, S_SSM, S_KEYS, S_VALS, S_KSCALES, S_VSCALES = 0, 1, 2, 3, 4, 5
# tensor formats (echo_hip.h ec_wfmt)
F32, F16, Q8_0, Q4_K = 0, 1, 6, 10
MATRICES = (T_W_IN, T_W_OUT, T_W_GATE, T_W_UP, T_W_DOWN)
# step trace operations and step buffers (echo_engine.h EC_OP_* / EC_B_*)
(OP_EMBED, OP_NORM, OP_MV_IN, OP_DELTA_STEP, OP_MV_OUT, OP_ROPE_APPEND, OP_ATTN, OP_QUANT_ACT, OP_MV_GU, OP_SWIGLU,
 OP_MV_DOWN, OP_LM_HEAD, OP_ARGMAX, OP_NORM_ROWS) = range(14)
(B_X, B_X2, B_PARTS, B_PROJ, B_GU, B_ACT_H, B_ACT_V, B_ACT_F, B_ACT_Q, B_ATTN_OUT, B_Q_PACKED, B_Q_SCALES, B_QBUF,
 B_LOGITS, B_TOK, B_POS, B_GEN, B_CTX, B_INV_FREQ, B_HN, B_CORE, B_FF, B_ACT4_H, B_ACT4_V, B_ACT4_Q,
 B_ACT4_F) = range(26)
ACT4_BUFFERS = (B_ACT4_H, B_ACT4_V, B_ACT4_Q, B_ACT4_F)
# chunked prefill trace operations and lane-0 chunk buffers
(OP_PF_EMBED, OP_PF_NORM, OP_PF_GEMM_IN, OP_PF_CONV, OP_PF_DELTA, OP_PF_GATED_NORM, OP_PF_GEMM_OUT,
 OP_PF_ROPE_APPEND, OP_PF_ATTN, OP_PF_GEMM_GU, OP_PF_SWIGLU, OP_PF_GEMM_DOWN, OP_PF_HEAD) = range(20, 33)
(B_PF_X, B_PF_N, B_PF_PROJ, B_PF_Q, B_PF_K, B_PF_V, B_PF_DEC, B_PF_BETA, B_PF_CORE, B_PF_GU, B_PF_ATTN, B_PF_TOK,
 B_PF_ACT1, B_PF_ACT) = range(30, 44)


def gguf_row_bytes(fmt: int, K: int) -> int:
    """Bytes of one GGUF row of K elements."""
    return {Q8_0: K // 32 * 34, Q4_K: K // 256 * 144, F16: 2 * K, F32: 4 * K}[fmt]


class TraceEvent(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("op", "layer", "phase", "nparts", "x_in", "x_out")]


_TRACE_FN = C.CFUNCTYPE(None, C.c_void_p, C.POINTER(TraceEvent))


@dataclass
class EngineConfig:
    vocab: int = 151936
    hidden: int = 2560
    ffn: int = 9216
    n_layers: int = 32
    n_heads: int = 16
    n_kv: int = 4
    head_dim: int = 256
    ssm_inner: int = 4096
    ssm_heads: int = 32
    conv_kernel: int = 4
    attn_interval: int = 4
    max_batch: int = 8
    max_ctx: int = 4608
    rope_base: float = 10000.0

    def is_attn(self, layer: int) -> bool:
        return self.attn_interval != 0 and (layer + 1) % self.attn_interval == 0

    @property
    def key_dim(self):
        return self.ssm_inner // 2

    @property
    def conv_dim(self):
        return 2 * self.key_dim + self.ssm_inner

    @property
    def nin_delta(self):
        return self.conv_dim + self.ssm_inner + 2 * self.ssm_heads

    @property
    def nin_attn(self):
        return (self.n_heads + 2 * self.n_kv) * self.head_dim


class _Cfg(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("vocab", "hidden", "ffn", "n_layers", "n_heads", "n_kv", "head_dim",
                                          "ssm_inner", "ssm_heads", "conv_kernel", "attn_interval", "max_batch",
                                          "max_ctx")] + [("rope_base", C.c_float)]


class Engine:
    def __init__(self, cfg: EngineConfig):
        self.cfg = cfg
        self.hip = load()
        L = self.L = self.hip.L
        vp, u32, i32 = C.c_void_p, C.c_uint32, C.c_int
        L.ec_engine_create.argtypes = [C.POINTER(_Cfg), C.POINTER(vp)]
        L.ec_engine_destroy.argtypes = [vp]
        L.ec_engine_destroy.restype = None
        L.ec_engine_set_tensor.argtypes = [vp, i32, i32, vp, C.c_size_t]
        L.ec_engine_init_random.argtypes = [vp, C.c_uint64, C.c_float]
        L.ec_engine_get_tensor.argtypes = [vp, i32, i32, vp, C.c_size_t]
        L.ec_engine_get_state.argtypes = [vp, i32, i32, u32, vp, C.c_size_t]
        L.ec_engine_reset.argtypes = [vp]
        L.ec_engine_set_inputs.argtypes = [vp, vp, vp, u32]
        L.ec_engine_step.argtypes = [vp, i32]
        L.ec_engine_prefill.argtypes = [vp, u32, vp, u32, i32]
        L.ec_engine_prefill_batch.argtypes = [vp, u32, vp, vp, vp, vp]
        L.ec_engine_sync.argtypes = [vp]
        L.ec_engine_get_tokens.argtypes = [vp, vp, vp]
        L.ec_engine_get_logits.argtypes = [vp, vp, u32]
        L.ec_engine_stream.argtypes = [vp]
        L.ec_engine_stream.restype = vp
        L.ec_engine_weight_bytes.argtypes = [vp]
        L.ec_engine_weight_bytes.restype = C.c_size_t
        L.ec_engine_profile_matvecs.argtypes = [vp, u32, C.POINTER(u32), C.POINTER(C.c_double),
                                                C.POINTER(C.c_double)]
        L.ec_engine_step_traced.argtypes = [vp, _TRACE_FN, vp]
        L.ec_engine_prefill_traced.argtypes = [vp, u32, vp, u32, i32, _TRACE_FN, vp]
        L.ec_engine_buffer.argtypes = [vp, i32, C.POINTER(vp), C.POINTER(C.c_size_t)]
        L.ec_engine_set_format.argtypes = [vp, i32, i32, i32]
        L.ec_engine_set_act_pieces.argtypes = [vp, C.c_uint32]
        L.ec_engine_get_act_pieces.argtypes = [vp]
        L.ec_engine_get_format.argtypes = [vp, i32, i32]
        c = _Cfg(**{f.name: getattr(cfg, f.name) for f in fields(cfg)})
        h = vp()
        self._check(L.ec_engine_create(C.byref(c), C.byref(h)), "ec_engine_create")
        self.h = h

    def _check(self, rc, name):
        if rc != 0:
            raise EchoHipError(f"{name} failed ({rc}): {self.L.ec_last_error().decode()}")

    def close(self):
        if getattr(self, "h", None):
            self.L.ec_engine_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    # ---- weights
    def set_act_pieces(self, pieces: int):
        """int8 pieces per decode-matvec activation element (ec_engine_set_act_pieces): 2 (default) or 1."""
        self._check(self.L.ec_engine_set_act_pieces(self.h, pieces), "set_act_pieces")

    @property
    def act_pieces(self) -> int:
        return self.L.ec_engine_get_act_pieces(self.h)

    def set_format(self, layer: int, tensor: int, fmt: int):
        """Storage format of a matrix (Q8_0 / Q4_K) or of the embedding (Q8_0 / F16 / F32)."""
        self._check(self.L.ec_engine_set_format(self.h, layer, tensor, fmt), "set_format")

    def get_format(self, layer: int, tensor: int) -> int:
        return self.L.ec_engine_get_format(self.h, layer, tensor)

    def set_tensor(self, layer: int, tensor: int, arr: np.ndarray):
        a = np.ascontiguousarray(arr)
        self._check(self.L.ec_engine_set_tensor(self.h, layer, tensor, a.ctypes.data, a.nbytes), "set_tensor")

    def get_tensor(self, layer: int, tensor: int, nbytes: int, dtype=np.uint8) -> np.ndarray:
        out = np.empty(nbytes, np.uint8)
        self._check(self.L.ec_engine_get_tensor(self.h, layer, tensor, out.ctypes.data, nbytes), "get_tensor")
        return out.view(dtype)

    def get_state(self, layer: int, which: int, seq: int) -> np.ndarray:
        """One sequence's state (echo_engine.h ec_engine_get_state) as a flat array."""
        c = self.cfg
        conv_dim = c.conv_dim
        n, dt = {S_CONV: (c.conv_kernel * conv_dim, np.float32), S_SSM: (c.ssm_heads * 128 * 128, np.float32),
                 S_KEYS: (c.max_ctx * c.n_kv * c.head_dim, np.int8), S_VALS: (c.max_ctx * c.n_kv * c.head_dim, np.int8),
                 S_KSCALES: (c.max_ctx * c.n_kv, np.float32), S_VSCALES: (c.max_ctx * c.n_kv, np.float32)}[which]
        out = np.empty(n, dt)
        self._check(self.L.ec_engine_get_state(self.h, layer, which, seq, out.ctypes.data, out.nbytes), "get_state")
        return out

    def export_model(self) -> dict:
        """Copy the weights back to the host in the oracle decoder's weight
        dict: GGUF matrices of their storage format (w_in = the fused
        input-projection rows; the formats under "fmt" when not all Q8_0),
        fp32 vectors."""
        cfg = self.cfg
        H, F = cfg.hidden, cfg.ffn
        f32 = lambda n: (n * 4, np.float32)  # noqa: E731
        fmts = {}

        def mat(l, t, name, rows, K):
            fmt = self.get_format(l, t)
            if fmt != Q8_0:
                fmts[(l, name)] = fmt
            return self.get_tensor(l, t, rows * gguf_row_bytes(fmt, K))
        emb_fmt = self.get_format(0, T_EMBED)
        if emb_fmt != Q8_0:
            fmts[(-1, "embed")] = emb_fmt
        emb = self.get_tensor(0, T_EMBED, cfg.vocab * gguf_row_bytes(emb_fmt, H))
        if emb_fmt in (F16, F32):
            emb = emb.view(np.float16 if emb_fmt == F16 else np.float32)
        m = {"embed": emb, "final_norm": self.get_tensor(0, T_FINAL_NORM, *f32(H)),
             "lm_head": mat(-1, T_LM_HEAD, "lm_head", cfg.vocab, H), "layers": []}
        for l in range(cfg.n_layers):
            attn = cfg.is_attn(l)
            nin = cfg.nin_attn if attn else cfg.nin_delta
            kout = cfg.n_heads * cfg.head_dim if attn else cfg.ssm_inner
            y = {"attn": attn, "w_in": mat(l, T_W_IN, "w_in", nin, H), "w_out": mat(l, T_W_OUT, "w_out", H, kout),
                 "w_gate": mat(l, T_W_GATE, "w_gate", F, H), "w_up": mat(l, T_W_UP, "w_up", F, H),
                 "w_down": mat(l, T_W_DOWN, "w_down", H, F),
                 "attn_norm": self.get_tensor(l, T_ATTN_NORM, *f32(H)),
                 "ffn_norm": self.get_tensor(l, T_FFN_NORM, *f32(H))}
            if attn:
                y["q_norm"] = self.get_tensor(l, T_Q_NORM, *f32(cfg.head_dim))
                y["k_norm"] = self.get_tensor(l, T_K_NORM, *f32(cfg.head_dim))
            else:
                y["conv_w"] = self.get_tensor(l, T_CONV_W, *f32(cfg.conv_kernel * cfg.conv_dim))
                y["a_log"] = self.get_tensor(l, T_A_LOG, *f32(cfg.ssm_heads))
                y["dt_bias"] = self.get_tensor(l, T_DT_BIAS, *f32(cfg.ssm_heads))
                y["ssm_norm"] = self.get_tensor(l, T_SSM_NORM, *f32(128))
            m["layers"].append(y)
        if fmts:
            m["fmt"] = fmts
        return m

    def init_random(self, seed: int = 0, w_scale: float = 0.02 / 73.0):
        self._check(self.L.ec_engine_init_random(self.h, seed, w_scale), "init_random")

    # ---- running
    def reset(self):
        self._check(self.L.ec_engine_reset(self.h), "reset")

    def set_inputs(self, tok, pos):
        t = np.ascontiguousarray(tok, np.int32)
        p = np.ascontiguousarray(pos, np.int32)
        assert t.size == p.size
        self._check(self.L.ec_engine_set_inputs(self.h, t.ctypes.data, p.ctypes.data, t.size), "set_inputs")

    def prefill(self, seq: int, tokens, pos0: int):
        """Chunked prefill of one sequence (ec_engine_prefill): tokens at positions pos0 .. pos0+n-1."""
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        self._check(self.L.ec_engine_prefill(self.h, seq, t.ctypes.data, t.size, pos0), "prefill")

    def prefill_batch(self, jobs):
        """ec_engine_prefill_batch: jobs = [(seq, tokens, pos0), ...], distinct sequences."""
        toks = [np.ascontiguousarray(t, dtype=np.int32) for _, t, _ in jobs]
        seqs = np.array([j[0] for j in jobs], np.uint32)
        lens = np.array([t.size for t in toks], np.uint32)
        pos0 = np.array([j[2] for j in jobs], np.int32)
        ptrs = (C.c_void_p * len(toks))(*[t.ctypes.data for t in toks])
        self._check(self.L.ec_engine_prefill_batch(self.h, len(toks), seqs.ctypes.data, C.cast(ptrs, C.c_void_p),
                                                   lens.ctypes.data, pos0.ctypes.data), "prefill_batch")

    def step(self, graph: bool = True):
        self._check(self.L.ec_engine_step(self.h, int(graph)), "step")

    def sync(self):
        self._check(self.L.ec_engine_sync(self.h), "sync")

    def tokens(self):
        B = self.cfg.max_batch
        gen = np.zeros(B, np.int32)
        pos = np.zeros(B, np.int32)
        self._check(self.L.ec_engine_get_tokens(self.h, gen.ctypes.data, pos.ctypes.data), "get_tokens")
        return gen, pos

    def logits(self, seq: int):
        out = np.zeros(self.cfg.vocab, np.float32)
        self._check(self.L.ec_engine_get_logits(self.h, out.ctypes.data, seq), "get_logits")
        return out

    def step_traced(self, fn):
        """One decode step launched eagerly with fn(event) called before (phase
        0) and after (phase 1) every launch, the stream drained each time
        (ec_engine_step_traced); fn reads buffers with read_buffer / get_state."""
        err = []

        def cb(_user, ev):
            if err:
                return
            try:
                e = ev.contents
                fn(TraceEvent(e.op, e.layer, e.phase, e.nparts, e.x_in, e.x_out))
            except BaseException as x:  # noqa: BLE001 (re-raised after the step)
                err.append(x)
        c_cb = _TRACE_FN(cb)
        rc = self.L.ec_engine_step_traced(self.h, c_cb, None)
        if err:
            raise err[0]
        self._check(rc, "step_traced")

    def prefill_traced(self, seq: int, tokens, pos0: int, fn):
        """ec_engine_prefill of one sequence with fn(event) called before and
        after every launch (ec_engine_prefill_traced)."""
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        err = []

        def cb(_user, ev):
            if err:
                return
            try:
                e = ev.contents
                fn(TraceEvent(e.op, e.layer, e.phase, e.nparts, e.x_in, e.x_out))
            except BaseException as x:  # noqa: BLE001 (re-raised after the prefill)
                err.append(x)
        c_cb = _TRACE_FN(cb)
        rc = self.L.ec_engine_prefill_traced(self.h, seq, t.ctypes.data, t.size, pos0, c_cb, None)
        if err:
            raise err[0]
        self._check(rc, "prefill_traced")

    def buffer(self, which: int):
        """(device address, bytes) of a step buffer (ec_engine_buffer)."""
        p, n = C.c_void_p(), C.c_size_t()
        self._check(self.L.ec_engine_buffer(self.h, which, C.byref(p), C.byref(n)), "buffer")
        return p.value or 0, n.value

    def read_buffer(self, which: int, dtype=np.float32, offset: int = 0, count: int | None = None) -> np.ndarray:
        """Copy (part of) a step buffer to the host: `count` elements of dtype from element `offset`."""
        p, n = self.buffer(which)
        isz = np.dtype(dtype).itemsize
        count = n // isz - offset if count is None else count
        assert 0 <= offset and offset + count <= n // isz, (which, offset, count, n)
        out = np.empty(count, dtype)
        if count:
            self.hip.copy(out, p + offset * isz, out.nbytes)
        return out

    def read_gemm_act(self, which: int, M: int, K: int):
        """A prefill GEMM activation (ec_gemm_quantize_act's Q8_0 layout for M
        tokens of K elements) as (xq int8 [M][K], xd fp32 [M][K/32])."""
        p, n = self.buffer(which)
        Mp, Kp = -(-M // 16) * 16, -(-K // 128) * 128
        nch, nbp = Kp // 128, Kp // 32
        xq_bytes = Mp // 16 * nch * 2048
        xd_off = -(-xq_bytes // 256) * 256
        assert xd_off + Mp * nbp * 4 <= n, (which, M, K, n)
        raw = np.empty(xd_off + Mp * nbp * 4, np.uint8)
        self.hip.copy(raw, p, raw.nbytes)
        # chunk (token tile T, 4-block group G) = [block pair][operand lane = r + 16*(8-group)][block of the pair][8 B]
        q = raw[:xq_bytes].view(np.int8).reshape(Mp // 16, nch, 2, 4, 16, 2, 8)
        xq = q.transpose(0, 4, 1, 2, 5, 3, 6).reshape(Mp, Kp)[:M, :K]
        xd = raw[xd_off:].view(np.float32).reshape(Mp, nbp)[:M, :K // 32]
        return np.ascontiguousarray(xq), np.ascontiguousarray(xd)

    def read_act(self, which: int, K: int, M: int | None = None, fmt: int | None = None, pieces: int | None = None):
        """An activation buffer (ec_quantize_act_pieces layout, M = max_batch;
        Q4_K for the B_ACT4_* buffers, Q8_0 otherwise; pieces = the engine's)
        as (xq int8 [B][pieces][K], xd fp32 [B][K/32]); Q4_K values in the
        quantizer's sub-block order."""
        import torch
        p, n = self.buffer(which)
        assert n, f"step buffer {which} is not allocated"
        B = self.cfg.max_batch if M is None else M
        P = self.act_pieces if pieces is None else pieces
        xq = torch.empty(P * B * K, dtype=torch.int8, device="cuda")
        xd = torch.empty(B * (K // 32), dtype=torch.float32, device="cuda")
        if fmt is None:
            fmt = Q4_K if which in ACT4_BUFFERS else Q8_0
        self.hip.act_unpack(fmt, p, xq, xd, B, K, pieces=P)
        torch.cuda.synchronize()
        return xq.cpu().numpy().reshape(B, P, K), xd.cpu().numpy().reshape(B, K // 32)

    @property
    def stream(self) -> int:
        return self.L.ec_engine_stream(self.h)

    def weight_bytes(self) -> int:
        return self.L.ec_engine_weight_bytes(self.h)

    def profile_matvecs(self, reps: int = 20):
        """(launches per step, algorithmic bytes per step, GPU us per step) of the
        step's matvecs replayed alone in a HIP graph (ec_engine_profile_matvecs)."""
        n, by, us = C.c_uint32(), C.c_double(), C.c_double()
        self._check(self.L.ec_engine_profile_matvecs(self.h, reps, C.byref(n), C.byref(by), C.byref(us)),
                    "profile_matvecs")
        return n.value, by.value, us.value
