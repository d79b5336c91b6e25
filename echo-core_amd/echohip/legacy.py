"""ctypes binding of the reference-signature C++ interface exported by
libechohip.so (include/kernels/quant.h, include/kernels/matvec.h,
include/kv_cache.h; implemented in host/legacy.cpp).

The symbols have C++ linkage, so they are looked up by their Itanium-mangled
names, exactly the names a program built against the reference's headers
links to.  Arrays may be numpy arrays (host memory, staged through the device
by the library) or torch CUDA tensors (used in place).  Like the reference,
the functions return nothing (or a float); failures are read back from
ec_last_error() and raised here as EchoHipError.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from .lib import EchoHipError, load

SYMS = {
    "quantize_per_token_symmetric": "_Z28quantize_per_token_symmetricPKfPaPfjj",
    "fused_dequant_dot_int8": "_Z22fused_dequant_dot_int8PKfPKaS0_Pfjj",
    "fused_dequant_dot_q8_0": "_Z22fused_dequant_dot_q8_0PK10block_q8_0jPKf",
    "fused_dequant_dot_q4_K": "_Z22fused_dequant_dot_q4_KPK10block_q4_KjPKf",
    "dequantize_q8_0_to_fp16": "_Z23dequantize_q8_0_to_fp16PKvPtm",
    "dequantize_q4_K_to_fp16": "_Z23dequantize_q4_K_to_fp16PKvPtm",
    "dequantize_q2_K_to_fp16": "_Z23dequantize_q2_K_to_fp16PKvPtm",
    "matvec_fp16_fp32<1024,512>": "_Z16matvec_fp16_fp32ILj1024ELj512EEvPKtPKfPfjj",
    "matvec_fp16_fp32<2048,1024>": "_Z16matvec_fp16_fp32ILj2048ELj1024EEvPKtPKfPfjj",
    "matvec_dispatch": "_Z15matvec_dispatchPKtPKfPfjjRK11ModelConfig",
    "matvec_q8_0": "_Z11matvec_q8_0PKvPKfPfjj",
    "matvec_q4_K": "_Z11matvec_q4_KPKvPKfPfjj",
    "matvec_q2_K": "_Z11matvec_q2_KPKvPKfPfjj",
    "KVCache::KVCache": "_ZN7KVCacheC1ERK11ModelConfig",
    "KVCache::~KVCache": "_ZN7KVCacheD1Ev",
    "KVCache::layer": "_ZN7KVCache5layerEj",
    "KVCache::append": "_ZN7KVCache6appendEjPKfS1_",
    "KVCache::seq_len": "_ZNK7KVCache7seq_lenEv",
    "KVCache::reset": "_ZN7KVCache5resetEv",
}


class ModelConfig(C.Structure):
    """include/config.h ModelConfig (enum class members are ints)."""
    _fields_ = [(n, C.c_uint32) for n in ("vocab_size", "hidden_dim", "num_heads", "num_kv_heads", "head_dim",
                                          "num_layers", "ffn_hidden_dim", "max_seq_len")] + \
               [("ffn_type", C.c_int), ("norm_type", C.c_int), ("pos_encoding", C.c_int),
                ("use_kv_quantization", C.c_bool)]


class KVCacheLayer(C.Structure):
    _fields_ = [("keys_int8", C.c_void_p), ("values_int8", C.c_void_p), ("key_scales", C.c_void_p),
                ("val_scales", C.c_void_p), ("keys_fp32", C.c_void_p), ("values_fp32", C.c_void_p),
                ("seq_len", C.c_uint32)]


def _p(x):
    if x is None:
        return None
    if isinstance(x, int):
        return x
    if isinstance(x, np.ndarray):
        assert x.flags.c_contiguous
        return x.ctypes.data
    return x.data_ptr()


class Legacy:
    def __init__(self):
        self.hip = load()
        L = self.L = self.hip.L
        self.f = {}
        vp, u32 = C.c_void_p, C.c_uint32
        sig = {
            "quantize_per_token_symmetric": ([vp, vp, vp, u32, u32], None),
            "fused_dequant_dot_int8": ([vp, vp, vp, vp, u32, u32], None),
            "fused_dequant_dot_q8_0": ([vp, u32, vp], C.c_float),
            "fused_dequant_dot_q4_K": ([vp, u32, vp], C.c_float),
            "dequantize_q8_0_to_fp16": ([vp, vp, C.c_size_t], None),
            "dequantize_q4_K_to_fp16": ([vp, vp, C.c_size_t], None),
            "dequantize_q2_K_to_fp16": ([vp, vp, C.c_size_t], None),
            "matvec_fp16_fp32<1024,512>": ([vp, vp, vp, u32, u32], None),
            "matvec_fp16_fp32<2048,1024>": ([vp, vp, vp, u32, u32], None),
            "matvec_dispatch": ([vp, vp, vp, u32, u32, C.POINTER(ModelConfig)], None),
            "matvec_q8_0": ([vp, vp, vp, u32, u32], None),
            "matvec_q4_K": ([vp, vp, vp, u32, u32], None),
            "matvec_q2_K": ([vp, vp, vp, u32, u32], None),
            "KVCache::KVCache": ([vp, C.POINTER(ModelConfig)], None),
            "KVCache::~KVCache": ([vp], None),
            "KVCache::layer": ([vp, u32], C.POINTER(KVCacheLayer)),
            "KVCache::append": ([vp, u32, vp, vp], None),
            "KVCache::seq_len": ([vp], u32),
            "KVCache::reset": ([vp], None),
        }
        for name, (args, res) in sig.items():
            fn = getattr(L, SYMS[name])
            fn.argtypes = args
            fn.restype = res
            self.f[name] = fn

    def _call(self, name, *args):
        L = self.L
        L.ec_last_error.restype = C.c_char_p
        before = L.ec_last_error()
        r = self.f[name](*args)
        after = L.ec_last_error()
        if after and after != before:
            raise EchoHipError(f"{name}: {after.decode()}")
        return r

    def clear_error(self):
        self.hip.L.ec_clear_error()

    # -- kernels/quant.h
    def quantize_per_token_symmetric(self, x, q, scales, num_tokens, num_elements):
        self.clear_error()
        self._call("quantize_per_token_symmetric", _p(x), _p(q), _p(scales), num_tokens, num_elements)

    def fused_dequant_dot_int8(self, query, keys, scales, scores, dim, seq_len):
        self.clear_error()
        self._call("fused_dequant_dot_int8", _p(query), _p(keys), _p(scales), _p(scores), dim, seq_len)

    def fused_dequant_dot_q8_0(self, blocks, n_blocks, query) -> float:
        self.clear_error()
        return self._call("fused_dequant_dot_q8_0", _p(blocks), n_blocks, _p(query))

    def fused_dequant_dot_q4_K(self, blocks, n_blocks, query) -> float:
        self.clear_error()
        return self._call("fused_dequant_dot_q4_K", _p(blocks), n_blocks, _p(query))

    def dequantize_to_fp16(self, fmt: str, src, dst, n_weights):
        self.clear_error()
        self._call(f"dequantize_{fmt}_to_fp16", _p(src), _p(dst), n_weights)

    # -- kernels/matvec.h (all accumulate into y)
    def matvec(self, fmt: str, W, x, y, M, K):
        self.clear_error()
        self._call(f"matvec_{fmt}", _p(W), _p(x), _p(y), M, K)

    def matvec_fp16_fp32(self, tiles: tuple, W, x, y, M, K):
        self.clear_error()
        self._call(f"matvec_fp16_fp32<{tiles[0]},{tiles[1]}>", _p(W), _p(x), _p(y), M, K)

    def matvec_dispatch(self, W, x, y, M, K, cfg: ModelConfig):
        self.clear_error()
        self._call("matvec_dispatch", _p(W), _p(x), _p(y), M, K, C.byref(cfg))


class KVCache:
    """The reference's KVCache class, constructed in a ctypes buffer."""

    def __init__(self, legacy: Legacy, cfg: ModelConfig):
        self.lg, self.cfg = legacy, cfg
        self._obj = (C.c_uint8 * 256)()  # >= sizeof(KVCache) (64 on x86-64), 64-byte aligned below
        base = C.addressof(self._obj)
        self.this = (base + 63) & ~63
        legacy.clear_error()
        legacy._call("KVCache::KVCache", self.this, C.byref(cfg))
        self.alive = True

    def layer(self, idx: int) -> KVCacheLayer:
        return self.lg._call("KVCache::layer", self.this, idx).contents

    def append(self, layer_idx: int, k, v):
        self.lg.clear_error()
        self.lg._call("KVCache::append", self.this, layer_idx, _p(k), _p(v))

    def seq_len(self) -> int:
        return self.lg._call("KVCache::seq_len", self.this)

    def reset(self):
        self.lg._call("KVCache::reset", self.this)

    def close(self):
        if self.alive:
            self.lg.f["KVCache::~KVCache"](self.this)
            self.alive = False

    def __del__(self):
        self.close()
