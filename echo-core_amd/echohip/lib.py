"""ctypes binding of libechohip.so's C ABI (include/echo_hip.h).

Arguments that are device buffers accept torch tensors (their data_ptr is
passed) or raw integer addresses.  Every call checks the returned ec_status and
raises EchoHipError with the library's message.  There is no fallback: if the
library is missing the import fails loudly.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

PKG = Path(__file__).resolve().parents[1]
LIBPATH = PKG / "libechohip.so"

Q8_0 = 6
Q4_K = 10
Q2_K = 8
F16 = 1

_vp = C.c_void_p
_u32 = C.c_uint32
_u64 = C.c_uint64
_sz = C.c_size_t

_SIGS = {
    "ec_device_init": [C.c_int],
    "ec_copy": [_vp, _vp, _sz],
    "ec_quantize_rows": [_vp, _vp, _vp, _u32, _u32, _vp],
    "ec_repack": [C.c_int, _vp, _vp, _u32, _u32, _vp],
    "ec_quantize_act": [C.c_int, _vp, _vp, _u32, _u32, _vp],
    "ec_act_unpack": [C.c_int, _vp, _vp, _vp, _u32, _u32, _vp],
    "ec_matvec": [C.c_int, _vp, _vp, _vp, _u32, _u32, _u32, _u32, C.c_int, _vp],
    "ec_block_dots": [C.c_int, _vp, _vp, _vp, _u32, _u32, _u32, _vp],
    "ec_matvec_split": [C.c_int, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _vp],
    "ec_matvec_gguf_f32": [C.c_int, _vp, _vp, _vp, _u32, _u32, _vp],
    "ec_dequant_dot_int8": [_vp, _vp, _vp, _vp, _u32, _u32, _vp],
    "ec_dequantize_to_fp16": [C.c_int, _vp, _vp, _sz, _vp],
    "ec_kv_append": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u64, _u32, _u32, _vp],
    "ec_attn_decode": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u64, _u32, _u32, _u32, _u32, _vp, _vp],
    "ec_attn_decode_noalloc": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u64, _u32, _u32, _u32, _u32, _vp],
    "ec_attn_decode_packed": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u64, _u32, _u32, _u32, _vp, _vp],
    "ec_glue_qk_rope_append": [_vp, _u32, _vp, _vp, C.c_int, C.c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                               _vp, _u32, _u64, _u32, _u32, _u32, _u32, _vp],
    "ec_glue_qk_rope_append_split": [_vp, _u32, _u32, _vp, _vp, C.c_int, C.c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                     _vp, _vp, _vp, _u32, _u64, _u32, _u32, _u32, _u32, _vp],
    "ec_deltanet": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _vp, _vp],
    "ec_attn_prefill": [_vp, _vp, _vp, _vp, _vp, _vp, _u32, C.c_int32, _u32, _u32, _u32, _u32, _vp, _vp],
    "ec_deltanet_chunked": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _vp, _vp, _vp],
    "ec_fill_random": [C.c_int, _vp, _u64, _u64, C.c_float, _u32, _vp],
    "ec_gemm_quantize_act": [C.c_int, _vp, _vp, _u32, _u32, _vp],
    "ec_gemm": [C.c_int, _vp, _vp, _vp, _u32, _u32, _u32, _u32, C.c_int, _vp],
    "ec_delta_step": [_vp, _u32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _vp],
    "ec_glue_conv_gates": [_vp, _u32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32,
                           _vp],
    "ec_glue_gated_norm_quant": [_vp, _vp, _u32, _u32, _vp, _vp, _u32, _u32, _vp],
    "ec_glue_rmsnorm_quant": [_vp, _vp, _vp, _u32, _u32, _vp],
    "ec_glue_add_rmsnorm_quant": [_vp, _vp, _u32, _vp, _vp, _vp, _u32, _u32, _vp],
    "ec_glue_swiglu_quant": [_vp, _vp, _u32, _u32, _vp],
    "ec_glue_swiglu_quant_split": [_vp, _u32, _vp, _u32, _u32, _vp],
    "ec_delta_step_split": [_vp, _u32, _u32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _vp],
    "ec_glue_conv_gates_chunk": [_vp, _u32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32,
                                 _vp],
    "ec_glue_rmsnorm_rows": [_vp, _vp, _vp, _u32, _u32, _vp],
    "ec_glue_swiglu_rows": [_vp, _vp, _u32, _u32, _vp],
    "ec_glue_gated_norm_rows": [_vp, _vp, _u32, _u32, _vp, _vp, _u32, _u32, _vp],
    "ec_glue_rmsnorm_rows_gemm_act": [_vp, _vp, _vp, _u32, _u32, _vp],
    "ec_glue_swiglu_rows_gemm_act": [_vp, _vp, _u32, _u32, _vp],
    "ec_glue_gated_norm_rows_gemm_act": [_vp, _vp, _u32, _u32, _vp, _vp, _u32, _u32, _vp],
    "ec_stream_read": [_vp, _sz, _vp, _u32, _vp],
    # two-piece activation variants (the trailing _u32 before the stream is the piece count)
    "ec_quantize_act_pieces": [C.c_int, _vp, _vp, _u32, _u32, _u32, _vp],
    "ec_act_unpack_pieces": [C.c_int, _u32, _vp, _vp, _vp, _u32, _u32, _vp],
    "ec_matvec_pieces": [C.c_int, _u32, _vp, _vp, _vp, _u32, _u32, _u32, _u32, C.c_int, _vp],
    "ec_matvec_split_pieces": [C.c_int, _u32, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _vp],
    "ec_block_dots_pieces": [C.c_int, _u32, _vp, _vp, _vp, _u32, _u32, _u32, _vp],
    "ec_glue_rmsnorm_quant_pieces": [_vp, _vp, _vp, _u32, _u32, _u32, _vp],
    "ec_glue_argmax_advance_bounded": [_vp, _u32, _vp, _vp, _vp, _u32, _u32, _vp],
    "ec_glue_argmax_advance_sliced": [_vp, _u32, _vp, _vp, _vp, _u32, _u32, _u32, _vp, _vp],
    "ec_glue_add_rmsnorm_quant_pieces": [_vp, _vp, _u32, _vp, _vp, _vp, _u32, _u32, _u32, _vp],
    "ec_glue_swiglu_quant_split_pieces": [_vp, _u32, _vp, _u32, _u32, _u32, _vp],
    "ec_glue_gated_norm_quant_pieces": [_vp, _vp, _u32, _u32, _vp, _vp, _u32, _u32, _u32, _vp],
    "ec_delta_step_out_pieces": [_vp, _u32, _u32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32,
                                 _u32, _u32, _vp],
    "ec_attn_decode_packed_pieces": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u64, _u32, _u32, _u32, _u32,
                                     _vp, _vp],
    "ec_stream_read_shape": [_vp, _sz, _vp, _u32, _u32, _u32, _vp],
}
_SIZE_FNS = {
    "ec_tiled_bytes": [C.c_int, _u32, _u32],
    "ec_act_bytes": [C.c_int, _u32, _u32],
    "ec_act_bytes_pieces": [C.c_int, _u32, _u32, _u32],
    "ec_attn_ws_bytes": [_u32, _u32, _u32, _u32],
    "ec_attn_qa_bytes": [_u32, _u32],
    "ec_gemm_act_bytes": [C.c_int, _u32, _u32],
    "ec_attn_noalloc_max_bytes": [],
    "ec_deltanet_chunked_ws_bytes": [_u32, _u32, _u32],
    "ec_attn_prefill_ws_bytes": [_u32, _u32, _u32],
    "ec_glue_argmax_ws_bytes": [_u32, _u32],
}


def _hptr(x):
    """Address of a numpy array, torch tensor or raw integer address."""
    if x is None or isinstance(x, int):
        return x
    if hasattr(x, "ctypes"):
        return x.ctypes.data
    return x.data_ptr()


class EchoHipError(RuntimeError):
    pass


def _ptr(x):
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return x.data_ptr()


class Lib:
    def __init__(self, path: Path = LIBPATH):
        # torch ships its own HIP runtime (same soname, different DT_NEEDED
        # name).  Loading torch first makes libechohip bind to that runtime, so
        # one process never holds two HIP runtimes.
        import torch  # noqa: F401
        if not path.exists():
            raise FileNotFoundError(f"{path} is not built: run __graft_entry__.build() (make -C echo-core_amd)")
        self.path = path
        L = self.L = C.CDLL(str(path))
        for name, args in _SIGS.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = C.c_int
        for name, args in _SIZE_FNS.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = _sz
        L.ec_last_error.restype = C.c_char_p

    def _call(self, name, *args):
        rc = getattr(self.L, name)(*args)
        if rc != 0:
            raise EchoHipError(f"{name} failed ({rc}): {self.L.ec_last_error().decode()}")

    @staticmethod
    def _stream(stream):
        if stream is None:
            import torch
            return torch.cuda.current_stream().cuda_stream
        return stream

    # ---- sizes
    def tiled_bytes(self, fmt, N, K):
        return self.L.ec_tiled_bytes(fmt, N, K)

    def act_bytes(self, fmt, M, K, pieces=1):
        return self.L.ec_act_bytes_pieces(fmt, M, K, pieces)

    def attn_ws_bytes(self, n_seq, n_heads, head_dim, max_ctx):
        return self.L.ec_attn_ws_bytes(n_seq, n_heads, head_dim, max_ctx)

    # ---- entry points
    def device_init(self, dev=0):
        self._call("ec_device_init", dev)

    def quantize_rows(self, x, q, scales, rows, width, stream=None):
        self._call("ec_quantize_rows", _ptr(x), _ptr(q), _ptr(scales), rows, width, self._stream(stream))

    def repack(self, fmt, gguf, tiled, N, K, stream=None):
        self._call("ec_repack", fmt, _ptr(gguf), _ptr(tiled), N, K, self._stream(stream))

    def quantize_act(self, fmt, x, act, M, K, stream=None, pieces=1):
        """ec_quantize_act (pieces 1) or its two-piece form ec_quantize_act_pieces."""
        if pieces == 1:
            self._call("ec_quantize_act", fmt, _ptr(x), _ptr(act), M, K, self._stream(stream))
        else:
            self._call("ec_quantize_act_pieces", fmt, _ptr(x), _ptr(act), M, K, pieces, self._stream(stream))

    def act_unpack(self, fmt, act, xq, xd, M, K, stream=None, pieces=1):
        """xq [pieces*M][K] (row 2i + p: token i, piece p), xd [M][K/32]."""
        self._call("ec_act_unpack_pieces", fmt, pieces, _ptr(act), _ptr(xq), _ptr(xd), M, K, self._stream(stream))

    def matvec(self, fmt, tiled, act, y, M, N, K, ldy=None, accumulate=False, stream=None, pieces=1):
        if pieces == 1:
            self._call("ec_matvec", fmt, _ptr(tiled), _ptr(act), _ptr(y), M, N, K, N if ldy is None else ldy,
                       int(bool(accumulate)), self._stream(stream))
        else:
            self._call("ec_matvec_pieces", fmt, pieces, _ptr(tiled), _ptr(act), _ptr(y), M, N, K,
                       N if ldy is None else ldy, int(bool(accumulate)), self._stream(stream))

    def matvec_split(self, fmt, tiled, act, parts, M, N, K, nsplit, stream=None, pieces=1):
        if pieces == 1:
            self._call("ec_matvec_split", fmt, _ptr(tiled), _ptr(act), _ptr(parts), M, N, K, nsplit,
                       self._stream(stream))
        else:
            self._call("ec_matvec_split_pieces", fmt, pieces, _ptr(tiled), _ptr(act), _ptr(parts), M, N, K, nsplit,
                       self._stream(stream))

    def block_dots(self, fmt, tiled, act, out, M, N, K, stream=None, pieces=1):
        """int32 block dots; with two pieces out is [2M][N][K/32] (row 2i + p = token i, piece p)."""
        if pieces == 1:
            self._call("ec_block_dots", fmt, _ptr(tiled), _ptr(act), _ptr(out), M, N, K, self._stream(stream))
        else:
            self._call("ec_block_dots_pieces", fmt, pieces, _ptr(tiled), _ptr(act), _ptr(out), M, N, K,
                       self._stream(stream))

    def matvec_gguf_f32(self, fmt, gguf, x, y, M, K, stream=None):
        self._call("ec_matvec_gguf_f32", fmt, _ptr(gguf), _ptr(x), _ptr(y), M, K, self._stream(stream))

    def dequant_dot_int8(self, q, keys, scales, scores, dim, seq, stream=None):
        self._call("ec_dequant_dot_int8", _ptr(q), _ptr(keys), _ptr(scales), _ptr(scores), dim, seq,
                   self._stream(stream))

    def dequantize_to_fp16(self, fmt, src, dst, n, stream=None):
        self._call("ec_dequantize_to_fp16", fmt, _ptr(src), _ptr(dst), n, self._stream(stream))

    def kv_append(self, k, v, keys, vals, ks, vs, pos, n_seq, seq_stride, n_kv, head_dim, stream=None):
        self._call("ec_kv_append", _ptr(k), _ptr(v), _ptr(keys), _ptr(vals), _ptr(ks), _ptr(vs), _ptr(pos), n_seq,
                   seq_stride, n_kv, head_dim, self._stream(stream))

    def attn_decode(self, q, keys, vals, ks, vs, out, ctx, n_seq, seq_stride, n_heads, n_kv, head_dim, max_ctx, ws,
                    stream=None):
        self._call("ec_attn_decode", _ptr(q), _ptr(keys), _ptr(vals), _ptr(ks), _ptr(vs), _ptr(out), _ptr(ctx),
                   n_seq, seq_stride, n_heads, n_kv, head_dim, max_ctx, _ptr(ws), self._stream(stream))

    def attn_decode_noalloc(self, q, keys, vals, ks, vs, out, ctx, n_seq, seq_stride, n_heads, n_kv, head_dim,
                            max_ctx, stream=None):
        """ec_attn_decode with the library's fixed per-GPU scratch instead of a workspace (no allocation)."""
        self._call("ec_attn_decode_noalloc", _ptr(q), _ptr(keys), _ptr(vals), _ptr(ks), _ptr(vs), _ptr(out),
                   _ptr(ctx), n_seq, seq_stride, n_heads, n_kv, head_dim, max_ctx, self._stream(stream))

    def attn_noalloc_max_bytes(self):
        return self.L.ec_attn_noalloc_max_bytes()

    def attn_decode_packed(self, q_packed, q_scales, keys, vals, ks, vs, out, act_q8, ctx, n_seq, seq_stride, n_heads,
                           n_kv, max_ctx, ws, stream=None, pieces=1):
        self._call("ec_attn_decode_packed_pieces", _ptr(q_packed), _ptr(q_scales), _ptr(keys), _ptr(vals), _ptr(ks),
                   _ptr(vs), _ptr(out), _ptr(act_q8), _ptr(ctx), n_seq, seq_stride, n_heads, n_kv, max_ctx, pieces,
                   _ptr(ws), self._stream(stream))

    def qk_rope_append(self, proj, Nin, q_norm, k_norm, use_qn, use_kn, inv_freq, pos, q_out, q_packed, q_scales, keys,
                       vals, ks, vs, ctx, n_seq, seq_stride, max_ctx, n_heads, n_kv, head_dim, stream=None):
        self._call("ec_glue_qk_rope_append", _ptr(proj), Nin, _ptr(q_norm), _ptr(k_norm), int(use_qn), int(use_kn),
                   _ptr(inv_freq), _ptr(pos), _ptr(q_out), _ptr(q_packed), _ptr(q_scales), _ptr(keys), _ptr(vals),
                   _ptr(ks), _ptr(vs), _ptr(ctx), n_seq, seq_stride, max_ctx, n_heads, n_kv, head_dim,
                   self._stream(stream))

    def qk_rope_append_split(self, proj, nparts, Nin, q_norm, k_norm, use_qn, use_kn, inv_freq, pos, q_out, q_packed,
                             q_scales, keys, vals, ks, vs, ctx, n_seq, seq_stride, max_ctx, n_heads, n_kv, head_dim,
                             stream=None):
        self._call("ec_glue_qk_rope_append_split", _ptr(proj), nparts, Nin, _ptr(q_norm), _ptr(k_norm), int(use_qn),
                   int(use_kn), _ptr(inv_freq), _ptr(pos), _ptr(q_out), _ptr(q_packed), _ptr(q_scales), _ptr(keys),
                   _ptr(vals), _ptr(ks), _ptr(vs), _ptr(ctx), n_seq, seq_stride, max_ctx, n_heads, n_kv, head_dim,
                   self._stream(stream))

    def attn_qa_bytes(self, n_seq, n_heads):
        return self.L.ec_attn_qa_bytes(n_seq, n_heads)

    def delta_step(self, proj, Nin, conv_state, conv_w, a_log, dt_bias, norm_w, state, act, pos, n_seq, n_k, n_v,
                   kern, stream=None):
        self._call("ec_delta_step", _ptr(proj), Nin, _ptr(conv_state), _ptr(conv_w), _ptr(a_log), _ptr(dt_bias),
                   _ptr(norm_w), _ptr(state), _ptr(act), _ptr(pos), n_seq, n_k, n_v, kern, self._stream(stream))

    def delta_step_split(self, proj, nparts, Nin, conv_state, conv_w, a_log, dt_bias, norm_w, state, act, pos, n_seq,
                         n_k, n_v, kern, stream=None):
        self._call("ec_delta_step_split", _ptr(proj), nparts, Nin, _ptr(conv_state), _ptr(conv_w), _ptr(a_log),
                   _ptr(dt_bias), _ptr(norm_w), _ptr(state), _ptr(act), _ptr(pos), n_seq, n_k, n_v, kern,
                   self._stream(stream))

    def conv_gates(self, proj, Nin, conv_state, conv_w, a_log, dt_bias, q, k, v, dec, beta, pos, n_seq, n_k, n_v,
                   kern, stream=None):
        self._call("ec_glue_conv_gates", _ptr(proj), Nin, _ptr(conv_state), _ptr(conv_w), _ptr(a_log),
                   _ptr(dt_bias), _ptr(q), _ptr(k), _ptr(v), _ptr(dec), _ptr(beta), _ptr(pos), n_seq, n_k, n_v, kern,
                   self._stream(stream))

    def gated_norm_quant(self, core, proj, Nin, z_off, norm_w, act, M, n_v, stream=None, pieces=1):
        self._call("ec_glue_gated_norm_quant_pieces", _ptr(core), _ptr(proj), Nin, z_off, _ptr(norm_w), _ptr(act), M,
                   n_v, pieces, self._stream(stream))

    def delta_step_out(self, proj, nparts, Nin, conv_state, conv_w, a_log, dt_bias, norm_w, state, act, out, pos,
                       n_seq, n_k, n_v, kern, stream=None, pieces=1):
        self._call("ec_delta_step_out_pieces", _ptr(proj), nparts, Nin, _ptr(conv_state), _ptr(conv_w), _ptr(a_log),
                   _ptr(dt_bias), _ptr(norm_w), _ptr(state), _ptr(act), _ptr(out), _ptr(pos), n_seq, n_k, n_v, kern,
                   pieces, self._stream(stream))

    def conv_gates_chunk(self, proj, Nin, ring, conv_w, a_log, dt_bias, q, k, v, dec, beta, T, p0, n_k, n_v, kern,
                         stream=None):
        self._call("ec_glue_conv_gates_chunk", _ptr(proj), Nin, _ptr(ring), _ptr(conv_w), _ptr(a_log), _ptr(dt_bias),
                   _ptr(q), _ptr(k), _ptr(v), _ptr(dec), _ptr(beta), T, p0, n_k, n_v, kern, self._stream(stream))

    def rmsnorm_rows(self, x, w, y, M, H, stream=None):
        self._call("ec_glue_rmsnorm_rows", _ptr(x), _ptr(w), _ptr(y), M, H, self._stream(stream))

    def swiglu_rows(self, gu, y, M, F, stream=None):
        self._call("ec_glue_swiglu_rows", _ptr(gu), _ptr(y), M, F, self._stream(stream))

    def gated_norm_rows(self, core, proj, Nin, z_off, norm_w, y, M, n_v, stream=None):
        self._call("ec_glue_gated_norm_rows", _ptr(core), _ptr(proj), Nin, z_off, _ptr(norm_w), _ptr(y), M, n_v,
                   self._stream(stream))

    def rmsnorm_rows_gemm_act(self, x, w, act, M, H, stream=None):
        self._call("ec_glue_rmsnorm_rows_gemm_act", _ptr(x), _ptr(w), _ptr(act), M, H, self._stream(stream))

    def swiglu_rows_gemm_act(self, gu, act, M, F, stream=None):
        self._call("ec_glue_swiglu_rows_gemm_act", _ptr(gu), _ptr(act), M, F, self._stream(stream))

    def gated_norm_rows_gemm_act(self, core, proj, Nin, z_off, norm_w, act, M, n_v, stream=None):
        self._call("ec_glue_gated_norm_rows_gemm_act", _ptr(core), _ptr(proj), Nin, z_off, _ptr(norm_w), _ptr(act), M,
                   n_v, self._stream(stream))

    def argmax_advance(self, logits, vocab, gen, nxt, pos, n_seq, max_pos=0, stream=None, slices=0, ws=None):
        if slices:
            self._call("ec_glue_argmax_advance_sliced", _ptr(logits), vocab, _ptr(gen), _ptr(nxt), _ptr(pos), n_seq,
                       max_pos, slices, _ptr(ws), self._stream(stream))
        else:
            self._call("ec_glue_argmax_advance_bounded", _ptr(logits), vocab, _ptr(gen), _ptr(nxt), _ptr(pos), n_seq,
                       max_pos, self._stream(stream))

    def argmax_ws_bytes(self, n_seq, slices):
        return self.L.ec_glue_argmax_ws_bytes(n_seq, slices)

    def rmsnorm_quant(self, x, w, act, M, H, stream=None, pieces=1):
        if pieces == 1:
            self._call("ec_glue_rmsnorm_quant", _ptr(x), _ptr(w), _ptr(act), M, H, self._stream(stream))
        else:
            self._call("ec_glue_rmsnorm_quant_pieces", _ptr(x), _ptr(w), _ptr(act), M, H, pieces, self._stream(stream))

    def add_rmsnorm_quant(self, x, parts, nparts, x_out, w, act, M, H, stream=None, pieces=1):
        if pieces == 1:
            self._call("ec_glue_add_rmsnorm_quant", _ptr(x), _ptr(parts), nparts, _ptr(x_out), _ptr(w), _ptr(act), M,
                       H, self._stream(stream))
        else:
            self._call("ec_glue_add_rmsnorm_quant_pieces", _ptr(x), _ptr(parts), nparts, _ptr(x_out), _ptr(w),
                       _ptr(act), M, H, pieces, self._stream(stream))

    def swiglu_quant(self, gu, act, M, F, stream=None):
        self._call("ec_glue_swiglu_quant", _ptr(gu), _ptr(act), M, F, self._stream(stream))

    def swiglu_quant_split(self, gu, nparts, act, M, F, stream=None, pieces=1):
        if pieces == 1:
            self._call("ec_glue_swiglu_quant_split", _ptr(gu), nparts, _ptr(act), M, F, self._stream(stream))
        else:
            self._call("ec_glue_swiglu_quant_split_pieces", _ptr(gu), nparts, _ptr(act), M, F, pieces,
                       self._stream(stream))

    def gemm_act_bytes(self, fmt, M, K):
        return self.L.ec_gemm_act_bytes(fmt, M, K)

    def gemm_quantize_act(self, fmt, x, act, M, K, stream=None):
        self._call("ec_gemm_quantize_act", fmt, _ptr(x), _ptr(act), M, K, self._stream(stream))

    def gemm(self, fmt, tiled, act, y, M, N, K, ldy=None, accumulate=False, stream=None):
        self._call("ec_gemm", fmt, _ptr(tiled), _ptr(act), _ptr(y), M, N, K, N if ldy is None else ldy,
                   int(bool(accumulate)), self._stream(stream))

    def copy(self, dst, src, nbytes):
        """Synchronous copy between host (numpy) and device buffers / raw addresses."""
        self._call("ec_copy", _hptr(dst), _hptr(src), nbytes)

    def deltanet(self, state, q, k, v, decay, beta, out, T, n_seq, n_v, n_k, d_k, d_v, seq_pos=None, stream=None):
        self._call("ec_deltanet", _ptr(state), _ptr(q), _ptr(k), _ptr(v), _ptr(decay), _ptr(beta), _ptr(out), T,
                   n_seq, n_v, n_k, d_k, d_v, _ptr(seq_pos), self._stream(stream))

    def attn_prefill_ws_bytes(self, T, n_heads, max_ctx):
        return self.L.ec_attn_prefill_ws_bytes(T, n_heads, max_ctx)

    def attn_prefill(self, q, keys, vals, ks, vs, out, T, pos0, n_heads, n_kv, head_dim, max_ctx, ws=None,
                     stream=None):
        self._call("ec_attn_prefill", _ptr(q), _ptr(keys), _ptr(vals), _ptr(ks), _ptr(vs), _ptr(out), T, pos0,
                   n_heads, n_kv, head_dim, max_ctx, _ptr(ws), self._stream(stream))

    def deltanet_chunked_ws_bytes(self, T, n_seq, n_v):
        return self.L.ec_deltanet_chunked_ws_bytes(T, n_seq, n_v)

    def deltanet_chunked(self, state, q, k, v, decay, beta, out, T, n_seq, n_v, n_k, d_k, d_v, ws, seq_pos=None,
                         stream=None):
        self._call("ec_deltanet_chunked", _ptr(state), _ptr(q), _ptr(k), _ptr(v), _ptr(decay), _ptr(beta), _ptr(out),
                   T, n_seq, n_v, n_k, d_k, d_v, _ptr(seq_pos), _ptr(ws), self._stream(stream))

    def stream_read_shape(self, src, nbytes, out, blocks, threads, unroll, stream=None):
        self._call("ec_stream_read_shape", _ptr(src), nbytes, _ptr(out), blocks, threads, unroll, self._stream(stream))

    def stream_read(self, src, nbytes, out, blocks, stream=None):
        self._call("ec_stream_read", _ptr(src), nbytes, _ptr(out), blocks, self._stream(stream))

    def fill_random(self, kind, dst, n, seed, scale=1.0, K=0, stream=None):
        self._call("ec_fill_random", kind, _ptr(dst), n, seed, scale, K, self._stream(stream))


_LIB = None


def load() -> Lib:
    global _LIB
    if _LIB is None:
        _LIB = Lib()
    return _LIB
