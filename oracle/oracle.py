"""ctypes view of the C oracle (liboracle.so) and of the compiled reference
kernels (_ref/libref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by the smoke check and by the
cpu_baseline leg of bench.py, never by the product library.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_u32 = C.c_uint32


def _load(name: str) -> C.CDLL:
    path = HERE / name
    if not path.exists():
        raise FileNotFoundError(f"{path} is not built (run `make -C {HERE}`)")
    return C.CDLL(str(path))


class Oracle:
    """Scalar C restatement (liboracle.so)."""

    def __init__(self, libname: str = "liboracle.so"):
        L = self.lib = _load(libname)
        L.oc_fp16_to_fp32.argtypes = [C.c_uint16]
        L.oc_fp16_to_fp32.restype = C.c_float
        L.oc_fp32_to_fp16.argtypes = [C.c_float]
        L.oc_fp32_to_fp16.restype = C.c_uint16
        L.oc_splitmix64_at.argtypes = [C.c_uint64, C.c_uint64]
        L.oc_splitmix64_at.restype = C.c_uint64
        L.oc_quantize_per_token_symmetric.argtypes = [_f32p, _i8p, _f32p, _u32, _u32]
        L.oc_fused_dequant_dot_int8.argtypes = [_f32p, _i8p, _f32p, _f32p, _u32, _u32]
        L.oc_dot_q8_0_f64.argtypes = [_u8p, _u32, _f32p]
        L.oc_dot_q8_0_f64.restype = C.c_double
        L.oc_dot_q4_K_f64.argtypes = [_u8p, _u32, _f32p]
        L.oc_dot_q4_K_f64.restype = C.c_double
        for fn in (L.oc_matvec_q8_0, L.oc_matvec_q4_K):
            fn.argtypes = [_u8p, _f32p, _f32p, _u32, _u32]
        L.oc_q4k_pos.argtypes = [_u32, _u32]
        L.oc_q4k_pos.restype = _u32
        L.oc_quantize_act_q8_0.argtypes = [_f32p, _i8p, _f32p, _u32]
        L.oc_quantize_act_q4_K.argtypes = [_f32p, _i8p, _f32p, _i32p, _u32]
        L.oc_dequant_act_q8_0.argtypes = [_i8p, _f32p, _f32p, _u32]
        L.oc_quantize_act2_q8_0.argtypes = [_f32p, _i8p, _i8p, _f32p, _u32]
        L.oc_dequant_act2_q8_0.argtypes = [_i8p, _i8p, _f32p, _f32p, _u32]
        L.oc_quantize_act2_q4_K.argtypes = [_f32p, _i8p, _i8p, _f32p, _u32]
        L.oc_dequant_act2_q4_K.argtypes = [_i8p, _i8p, _f32p, _f32p, _u32]
        L.oc_dequant_act_q4_K.argtypes = [_i8p, _f32p, _f32p, _u32]
        L.oc_block_dots_q8_0.argtypes = [_u8p, _i8p, _i32p, _u32, _u32]
        L.oc_block_dots_q4_K.argtypes = [_u8p, _i8p, _i32p, _u32, _u32]
        L.oc_kv_append.argtypes = [_f32p, _f32p, _i8p, _i8p, _f32p, _f32p, _u32, _u32, _u32]
        L.oc_attn_decode_int8.argtypes = [_f32p, _i8p, _i8p, _f32p, _f32p, _f32p, _u32, _u32, _u32, _u32]
        L.oc_deltanet_step.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _u32, _u32, _u32, _u32]
        L.oc_rmsnorm.argtypes = [_f32p, _f32p, _f32p, _u32]
        L.oc_head_rmsnorm.argtypes = [_f32p, _f32p, _u32, _u32]
        L.oc_rope_inv_freq.argtypes = [_f32p, _u32, C.c_float]
        L.oc_rope.argtypes = [_f32p, _u32, _u32, _u32, _f32p]
        L.oc_silu.argtypes = [C.c_float]
        L.oc_silu.restype = C.c_float
        L.oc_softplus.argtypes = [C.c_float]
        L.oc_softplus.restype = C.c_float
        L.oc_l2norm_heads.argtypes = [_f32p, _u32, _u32]
        L.oc_conv_step.argtypes = [_f32p, _f32p, _f32p, _f32p, _u32, _u32]
        L.oc_argmax.argtypes = [_f32p, _u32]
        L.oc_argmax.restype = _u32
        L.oc_embed_row_q8_0.argtypes = [_u8p, _u32, _u32, _f32p]
        L.oc_deltanet_gates.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _u32]
        L.oc_gated_rmsnorm.argtypes = [_f32p, _f32p, _f32p, _u32, _u32]
        L.oc_matvec_act_q8_0.argtypes = [_u8p, _f32p, _f32p, _u32, _u32, C.c_int]
        L.oc_matvec_act.argtypes = [C.c_int, _u8p, _f32p, _f32p, _u32, _u32, C.c_int]
        L.oc_embed_row.argtypes = [C.c_int, C.c_void_p, _u32, _u32, _f32p]
        L.oc_swiglu.argtypes = [_f32p, _f32p, _f32p, _u32]

    def swiglu(self, gate, up):
        g = np.ascontiguousarray(gate, np.float32).reshape(-1)
        out = np.zeros(g.size, np.float32)
        self.lib.oc_swiglu(g, np.ascontiguousarray(up, np.float32).reshape(-1), out, g.size)
        return out

    def rmsnorm(self, x, w):
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        out = np.zeros(x.size, np.float32)
        self.lib.oc_rmsnorm(x, np.ascontiguousarray(w, np.float32).reshape(-1), out, x.size)
        return out

    def embed_row_q8_0(self, embed, H, tok):
        out = np.zeros(H, np.float32)
        self.lib.oc_embed_row_q8_0(np.ascontiguousarray(embed).reshape(-1), H, int(tok), out)
        return out

    def embed_row(self, fmt, embed, H, tok):
        """Row `tok` of an embedding table of format fmt (6 Q8_0 blocks, 1 F16, 0 F32 rows)."""
        e = np.ascontiguousarray(embed).reshape(-1)
        out = np.zeros(H, np.float32)
        self.lib.oc_embed_row(int(fmt), e.ctypes.data, H, int(tok), out)
        return out

    def matvec_act(self, fmt, W, x, quant_act=True):
        """y = W x for a GGUF matrix of format fmt (6 Q8_0, 10 Q4_K), x quantized first when quant_act."""
        M = W.shape[0]
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        y = np.zeros(M, np.float32)
        self.lib.oc_matvec_act(int(fmt), np.ascontiguousarray(W).reshape(-1), x, y, M, x.size, int(quant_act))
        return y

    def conv_step(self, state, x, w, C_, kernel):
        """Advances state ([kernel][C] newest first) in place; returns silu(conv)."""
        out = np.zeros(C_, np.float32)
        self.lib.oc_conv_step(state.reshape(-1), np.ascontiguousarray(x, np.float32).reshape(-1),
                              np.ascontiguousarray(w, np.float32).reshape(-1), out, C_, kernel)
        return out

    def l2norm_heads(self, x, n_heads, head_dim):
        y = np.array(x, np.float32).reshape(-1)
        self.lib.oc_l2norm_heads(y, n_heads, head_dim)
        return y

    def head_rmsnorm(self, x, w, n_heads, head_dim):
        y = np.array(x, np.float32).reshape(-1)
        self.lib.oc_head_rmsnorm(y, np.ascontiguousarray(w, np.float32), n_heads, head_dim)
        return y

    def rope(self, x, n_heads, head_dim, pos, base=10000.0):
        inv = np.zeros(head_dim // 2, np.float32)
        self.lib.oc_rope_inv_freq(inv, head_dim, base)
        y = np.array(x, np.float32).reshape(-1)
        self.lib.oc_rope(y, n_heads, head_dim, pos, inv)
        return y

    def deltanet_gates(self, alpha, beta_logit, a_log, dt_bias):
        """(decay, beta) per value head (qwen_linear.zig:215-219)."""
        f = lambda a: np.ascontiguousarray(a, np.float32).reshape(-1)  # noqa: E731
        alpha, beta_logit, a_log, dt_bias = f(alpha), f(beta_logit), f(a_log), f(dt_bias)
        n = alpha.size
        dec, bet = np.zeros(n, np.float32), np.zeros(n, np.float32)
        self.lib.oc_deltanet_gates(alpha, beta_logit, a_log, dt_bias, dec, bet, n)
        return dec, bet

    def gated_rmsnorm(self, core, z, w, n_v, d_v):
        """core * rsqrt(mean(core^2) + 1e-6) * w * silu(z) per head (qwen_linear.zig:244-257)."""
        out = np.array(core, np.float32).reshape(-1)
        self.lib.oc_gated_rmsnorm(out, np.ascontiguousarray(z, np.float32).reshape(-1),
                                  np.ascontiguousarray(w, np.float32).reshape(-1), n_v, d_v)
        return out.reshape(n_v, d_v)

    def matvec_act_q8_0(self, W, x, quant_act=True):
        M = W.shape[0]
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        y = np.zeros(M, np.float32)
        self.lib.oc_matvec_act_q8_0(np.ascontiguousarray(W).reshape(-1), x, y, M, x.size, int(quant_act))
        return y

    # -- wrappers returning numpy arrays
    def quantize(self, x: np.ndarray, width: int):
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        rows = x.size // width
        q = np.zeros(rows * width, np.int8)
        s = np.zeros(rows, np.float32)
        self.lib.oc_quantize_per_token_symmetric(x, q, s, rows, width)
        return q.reshape(rows, width), s

    def matvec_q8_0(self, W: np.ndarray, x: np.ndarray, y0: np.ndarray | None = None):
        M = W.shape[0]
        K = x.size
        y = np.zeros(M, np.float32) if y0 is None else np.array(y0, np.float32)
        self.lib.oc_matvec_q8_0(np.ascontiguousarray(W).reshape(-1), np.ascontiguousarray(x, np.float32), y, M, K)
        return y

    def matvec_q4_K(self, W: np.ndarray, x: np.ndarray, y0: np.ndarray | None = None):
        M = W.shape[0]
        K = x.size
        y = np.zeros(M, np.float32) if y0 is None else np.array(y0, np.float32)
        self.lib.oc_matvec_q4_K(np.ascontiguousarray(W).reshape(-1), np.ascontiguousarray(x, np.float32), y, M, K)
        return y

    def quantize_act_q8_0(self, x: np.ndarray):
        K = x.size
        xq = np.zeros(K, np.int8)
        xd = np.zeros(K // 32, np.float32)
        self.lib.oc_quantize_act_q8_0(np.ascontiguousarray(x, np.float32), xq, xd, K)
        return xq, xd

    def quantize_act_q4_K(self, x: np.ndarray):
        K = x.size
        xq = np.zeros(K, np.int8)
        xd = np.zeros(K // 32, np.float32)
        xs = np.zeros(K // 32, np.int32)
        self.lib.oc_quantize_act_q4_K(np.ascontiguousarray(x, np.float32), xq, xd, xs, K)
        return xq, xd, xs

    def quantize_act2_q8_0(self, x: np.ndarray):
        """Two int8 pieces per 32-block (oc_quantize_act2_q8_0): (q0, q1, scales)."""
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        q0, q1 = np.zeros(x.size, np.int8), np.zeros(x.size, np.int8)
        d = np.zeros(x.size // 32, np.float32)
        self.lib.oc_quantize_act2_q8_0(x, q0, q1, d, x.size)
        return q0, q1, d

    def dequant_act2_q8_0(self, q0, q1, xd):
        q0, q1 = np.ascontiguousarray(q0, np.int8).reshape(-1), np.ascontiguousarray(q1, np.int8).reshape(-1)
        out = np.zeros(q0.size, np.float32)
        self.lib.oc_dequant_act2_q8_0(q0, q1, np.ascontiguousarray(xd, np.float32).reshape(-1), out, q0.size)
        return out

    def quantize_act2_q4_K(self, x: np.ndarray):
        """Two pieces per Q4_K sub-block (oc_quantize_act2_q4_K), values in sub-block order: (q0, q1, scales)."""
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        q0, q1 = np.zeros(x.size, np.int8), np.zeros(x.size, np.int8)
        d = np.zeros(x.size // 32, np.float32)
        self.lib.oc_quantize_act2_q4_K(x, q0, q1, d, x.size)
        return q0, q1, d

    def dequant_act2_q4_K(self, q0, q1, xd):
        q0, q1 = np.ascontiguousarray(q0, np.int8).reshape(-1), np.ascontiguousarray(q1, np.int8).reshape(-1)
        out = np.zeros(q0.size, np.float32)
        self.lib.oc_dequant_act2_q4_K(q0, q1, np.ascontiguousarray(xd, np.float32).reshape(-1), out, q0.size)
        return out

    def dequant_act_q8_0(self, xq, xd):
        out = np.zeros(xq.size, np.float32)
        self.lib.oc_dequant_act_q8_0(np.ascontiguousarray(xq), np.ascontiguousarray(xd), out, xq.size)
        return out

    def dequant_act_q4_K(self, xq, xd):
        out = np.zeros(xq.size, np.float32)
        self.lib.oc_dequant_act_q4_K(np.ascontiguousarray(xq), np.ascontiguousarray(xd), out, xq.size)
        return out

    def block_dots_q8_0(self, W, xq):
        M = W.shape[0]
        K = xq.size
        out = np.zeros(M * (K // 32), np.int32)
        self.lib.oc_block_dots_q8_0(np.ascontiguousarray(W).reshape(-1), np.ascontiguousarray(xq), out, M, K)
        return out.reshape(M, K // 32)

    def block_dots_q4_K(self, W, xq):
        M = W.shape[0]
        K = xq.size
        out = np.zeros(M * (K // 32), np.int32)
        self.lib.oc_block_dots_q4_K(np.ascontiguousarray(W).reshape(-1), np.ascontiguousarray(xq), out, M, K)
        return out.reshape(M, K // 32)

    def kv_append(self, k, v, keys, vals, ks, vs, pos, n_kv, head_dim):
        self.lib.oc_kv_append(np.ascontiguousarray(k, np.float32), np.ascontiguousarray(v, np.float32),
                              keys, vals, ks, vs, pos, n_kv, head_dim)

    def attn_decode(self, q, keys, vals, ks, vs, n_heads, n_kv, head_dim, ctx):
        out = np.zeros(n_heads * head_dim, np.float32)
        self.lib.oc_attn_decode_int8(np.ascontiguousarray(q, np.float32).reshape(-1),
                                     np.ascontiguousarray(keys).reshape(-1), np.ascontiguousarray(vals).reshape(-1),
                                     np.ascontiguousarray(ks, np.float32).reshape(-1),
                                     np.ascontiguousarray(vs, np.float32).reshape(-1), out, n_heads, n_kv, head_dim,
                                     ctx)
        return out.reshape(n_heads, head_dim)

    def deltanet_step(self, state, q, k, v, decay, beta, n_v, n_k, d_k, d_v):
        """Advances ``state`` ([n_v, d_k, d_v] float32, reference layout) in place."""
        out = np.zeros(n_v * d_v, np.float32)
        self.lib.oc_deltanet_step(state.reshape(-1), np.ascontiguousarray(q, np.float32).reshape(-1),
                                  np.ascontiguousarray(k, np.float32).reshape(-1),
                                  np.ascontiguousarray(v, np.float32).reshape(-1),
                                  np.ascontiguousarray(decay, np.float32), np.ascontiguousarray(beta, np.float32),
                                  out, n_v, n_k, d_k, d_v)
        return out.reshape(n_v, d_v)


class Reference:
    """The reference's own kernels, compiled from its sources into _ref/libref.so
    (oracle/Makefile `ref`).  C++ linkage, so symbols are looked up mangled."""

    SYMS = {
        "quantize_per_token_symmetric": "_Z28quantize_per_token_symmetricPKfPaPfjj",
        "fused_dequant_dot_int8": "_Z22fused_dequant_dot_int8PKfPKaS0_Pfjj",
        "fused_dequant_dot_q8_0": "_Z22fused_dequant_dot_q8_0PK10block_q8_0jPKf",
        "fused_dequant_dot_q4_K": "_Z22fused_dequant_dot_q4_KPK10block_q4_KjPKf",
        "matvec_q8_0": "_Z11matvec_q8_0PKvPKfPfjj",
        "matvec_q4_K": "_Z11matvec_q4_KPKvPKfPfjj",
        "matvec_q2_K": "_Z11matvec_q2_KPKvPKfPfjj",
        "dequantize_q8_0_to_fp16": "_Z23dequantize_q8_0_to_fp16PKvPtm",
        "dequantize_q4_K_to_fp16": "_Z23dequantize_q4_K_to_fp16PKvPtm",
        "dequantize_q2_K_to_fp16": "_Z23dequantize_q2_K_to_fp16PKvPtm",
        "matvec_fp16_fp32<1024,512>": "_Z16matvec_fp16_fp32ILj1024ELj512EEvPKtPKfPfjj",
        "matvec_fp16_fp32<2048,1024>": "_Z16matvec_fp16_fp32ILj2048ELj1024EEvPKtPKfPfjj",
    }

    def __init__(self):
        L = self.lib = _load("_ref/libref.so")
        f = self.fn = {k: getattr(L, v) for k, v in self.SYMS.items()}
        f["quantize_per_token_symmetric"].argtypes = [_f32p, _i8p, _f32p, _u32, _u32]
        f["fused_dequant_dot_int8"].argtypes = [_f32p, _i8p, _f32p, _f32p, _u32, _u32]
        f["fused_dequant_dot_q8_0"].argtypes = [_u8p, _u32, _f32p]
        f["fused_dequant_dot_q8_0"].restype = C.c_float
        f["fused_dequant_dot_q4_K"].argtypes = [_u8p, _u32, _f32p]
        f["fused_dequant_dot_q4_K"].restype = C.c_float
        f["matvec_q8_0"].argtypes = [_u8p, _f32p, _f32p, _u32, _u32]
        f["matvec_q4_K"].argtypes = [_u8p, _f32p, _f32p, _u32, _u32]
        f["matvec_q2_K"].argtypes = [_u8p, _f32p, _f32p, _u32, _u32]
        for k in ("q8_0", "q4_K", "q2_K"):
            f[f"dequantize_{k}_to_fp16"].argtypes = [C.c_void_p, C.c_void_p, C.c_size_t]
        for k in ("matvec_fp16_fp32<1024,512>", "matvec_fp16_fp32<2048,1024>"):
            f[k].argtypes = [C.c_void_p, _f32p, _f32p, _u32, _u32]

    @staticmethod
    def available() -> bool:
        return (HERE / "_ref" / "libref.so").exists()


class Baseline:
    """AVX2 + OpenMP CPU baseline (liboracle_avx2.so)."""

    def __init__(self):
        L = self.lib = _load("liboracle_avx2.so")
        L.ob_matvec_q8_0_avx2.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, _u32, _u32]
        L.ob_matvec_q4_K_avx2.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, _u32, _u32]
        L.ob_set_threads.argtypes = [C.c_int]
        L.ob_max_threads.restype = C.c_int
        L.oc_attn_decode_int8.argtypes = [C.c_void_p] * 6 + [_u32] * 4
        L.oc_deltanet_step.argtypes = [C.c_void_p] * 7 + [_u32] * 4

    def threads(self, n: int):
        self.lib.ob_set_threads(int(n))


# ---------------------------------------------------------------- decoder
class _OcCfg(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("hidden", "ffn", "n_layers", "vocab", "n_heads", "n_kv", "head_dim",
                                          "ssm_inner", "ssm_heads", "conv_kernel", "attn_interval", "max_ctx")] + \
               [("rope_base", C.c_float)]


_PP = C.POINTER(C.c_void_p)


class _OcW(C.Structure):
    _fields_ = [(n, _PP) for n in ("w_qkv", "w_z", "w_ab", "w_out", "w_gate", "w_up", "w_down", "attn_norm",
                                   "ffn_norm", "conv_w", "a_log", "dt_bias", "ssm_norm", "q_norm", "k_norm")] + \
               [("embed", C.c_void_p), ("final_norm", C.c_void_p), ("lm_head", C.c_void_p), ("fmt", C.c_void_p)]


class _OcSeq(C.Structure):
    _fields_ = [(n, _PP) for n in ("conv_state", "ssm_state", "keys", "vals", "kscales", "vscales")] + \
               [("pos", C.c_uint32)]


class Decoder:
    """n_seq independent sequences decoded token by token by oc_decoder_token
    (oracle.c).  `cfg` is an echohip.engine.EngineConfig-like object and `m`
    the weight dict of tests/decoder_util.make_model (GGUF matrices, Q8_0
    unless m["fmt"] maps (layer, name) to another format -- layer -1 for
    "lm_head" and "embed" -- fp32 vectors, the fused w_in rows of the engine)."""

    def __init__(self, oc, cfg: EngineConfig, m, n_seq, quant_act=True):
        self.oc, self.cfg, self.quant_act = oc, cfg, int(quant_act)
        L = cfg.n_layers
        self.keep = []
        c = self.c = _OcCfg(hidden=cfg.hidden, ffn=cfg.ffn, n_layers=L, vocab=cfg.vocab, n_heads=cfg.n_heads,
                            n_kv=cfg.n_kv, head_dim=cfg.head_dim, ssm_inner=cfg.ssm_inner, ssm_heads=cfg.ssm_heads,
                            conv_kernel=cfg.conv_kernel, attn_interval=cfg.attn_interval, max_ctx=cfg.max_ctx,
                            rope_base=cfg.rope_base)

        def arr(ptrs):
            a = (C.c_void_p * L)(*ptrs)
            self.keep.append(a)
            return C.cast(a, _PP)

        def p(x):
            if x is None:
                return None
            x = np.ascontiguousarray(x)
            self.keep.append(x)
            return x.ctypes.data

        H = cfg.hidden
        fm = m.get("fmt", {})
        lay = m["layers"]
        fmt = np.full(4 * L + 2, 6, np.int32)
        for l in range(L):
            fmt[4 * l:4 * l + 4] = [fm.get((l, n), 6) for n in ("w_in", "w_out", "w_gate", "w_down")]
            assert fm.get((l, "w_up"), 6) == fmt[4 * l + 2], "gate and up share one format"
        fmt[4 * L] = fm.get((-1, "lm_head"), 6)
        fmt[4 * L + 1] = fm.get((-1, "embed"), 6)
        w = {k: [] for k, _ in _OcW._fields_[:15]}
        for l, y in enumerate(lay):
            rowb = H // 32 * 34 if fmt[4 * l] == 6 else H // 256 * 144
            w["w_qkv"].append(p(y["w_in"]))
            base = y["w_in"].reshape(-1)
            if y["attn"]:
                w["w_z"].append(None)
                w["w_ab"].append(None)
            else:
                w["w_z"].append(p(base[cfg.conv_dim * rowb:]))
                w["w_ab"].append(p(base[(cfg.conv_dim + cfg.ssm_inner) * rowb:]))
            for k in ("w_out", "w_gate", "w_up", "w_down", "attn_norm", "ffn_norm", "conv_w", "a_log", "dt_bias",
                      "ssm_norm", "q_norm", "k_norm"):
                w[k].append(p(y.get(k)))
        self.w = _OcW(**{k: arr(v) for k, v in w.items()}, embed=p(m["embed"]), final_norm=p(m["final_norm"]),
                      lm_head=p(m["lm_head"]), fmt=p(fmt) if fm else None)
        self.seqs, self.states = [], []
        kvd = cfg.n_kv * cfg.head_dim
        for _ in range(n_seq):
            st = {"conv": [], "ssm": [], "k": [], "v": [], "ks": [], "vs": []}
            for l in range(L):
                if cfg.is_attn(l):
                    st["conv"].append(None)
                    st["ssm"].append(None)
                    st["k"].append(np.zeros(cfg.max_ctx * kvd, np.int8))
                    st["v"].append(np.zeros(cfg.max_ctx * kvd, np.int8))
                    st["ks"].append(np.zeros(cfg.max_ctx * cfg.n_kv, np.float32))
                    st["vs"].append(np.zeros(cfg.max_ctx * cfg.n_kv, np.float32))
                else:
                    st["conv"].append(np.zeros(cfg.conv_kernel * cfg.conv_dim, np.float32))
                    st["ssm"].append(np.zeros(cfg.ssm_heads * 128 * 128, np.float32))
                    for k in ("k", "v", "ks", "vs"):
                        st[k].append(None)
            self.keep.append(st)
            self.states.append(st)
            s = _OcSeq(conv_state=arr([p(x) for x in st["conv"]]), ssm_state=arr([p(x) for x in st["ssm"]]),
                       keys=arr([p(x) for x in st["k"]]), vals=arr([p(x) for x in st["v"]]),
                       kscales=arr([p(x) for x in st["ks"]]), vscales=arr([p(x) for x in st["vs"]]), pos=0)
            self.seqs.append(s)
        oc.lib.oc_decoder_token.argtypes = [C.POINTER(_OcCfg), C.POINTER(_OcW), C.POINTER(_OcSeq), C.c_uint32,
                                            C.c_void_p, C.c_int]
        oc.lib.oc_deltanet_block.argtypes = [C.POINTER(_OcCfg), C.POINTER(_OcW), _u32, _f32p, _f32p, _f32p, _f32p,
                                             C.c_int]
        oc.lib.oc_attention_block.argtypes = [C.POINTER(_OcCfg), C.POINTER(_OcW), _u32, _i8p, _i8p, _f32p, _f32p,
                                              _u32, _f32p, _f32p, C.c_int]
        oc.lib.oc_ffn_block.argtypes = [C.POINTER(_OcCfg), C.POINTER(_OcW), _u32, _f32p, _f32p, C.c_int]

    def token(self, seq: int, tok: int):
        logits = np.zeros(self.cfg.vocab, np.float32)
        self.oc.lib.oc_decoder_token(C.byref(self.c), C.byref(self.w), C.byref(self.seqs[seq]), tok,
                                     logits.ctypes.data, self.quant_act)
        return logits

    def pos(self, seq: int) -> int:
        return self.seqs[seq].pos

    # -- the blocks oc_decoder_token composes, on one sequence's state
    def deltanet_block(self, seq: int, layer: int, x):
        """qwen_linear.forward of `layer` on the normed input x; advances the
        sequence's conv and recurrent state of that layer."""
        st = self.states[seq]
        out = np.zeros(self.cfg.hidden, np.float32)
        self.oc.lib.oc_deltanet_block(C.byref(self.c), C.byref(self.w), layer, st["conv"][layer], st["ssm"][layer],
                                      np.ascontiguousarray(x, np.float32), out, self.quant_act)
        return out

    def attention_block(self, seq: int, layer: int, x, pos: int):
        st = self.states[seq]
        out = np.zeros(self.cfg.hidden, np.float32)
        self.oc.lib.oc_attention_block(C.byref(self.c), C.byref(self.w), layer, st["k"][layer], st["v"][layer],
                                       st["ks"][layer], st["vs"][layer], pos, np.ascontiguousarray(x, np.float32), out,
                                       self.quant_act)
        return out

    def ffn_block(self, layer: int, x):
        out = np.zeros(self.cfg.hidden, np.float32)
        self.oc.lib.oc_ffn_block(C.byref(self.c), C.byref(self.w), layer, np.ascontiguousarray(x, np.float32), out,
                                 self.quant_act)
        return out

    def load_state(self, seq: int, pos: int, get):
        """Overwrite sequence `seq`'s state with another decoder's, at position
        `pos` (tokens processed).  get(layer, kind) returns that decoder's state
        in the oracle's layout: kind "conv" fp32 [kernel][C] newest first, "ssm"
        fp32 [heads][k][v], "k"/"v" int8 [max_ctx][n_kv][head_dim], "ks"/"vs" fp32."""
        st = self.states[seq]
        for l in range(self.cfg.n_layers):
            for kind in (("k", "v", "ks", "vs") if self.cfg.is_attn(l) else ("conv", "ssm")):
                np.copyto(st[kind][l], get(l, kind).reshape(st[kind][l].shape))
        self.seqs[seq].pos = pos
