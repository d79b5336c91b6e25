"""ctypes binding of the GGUF v3 reader and loader (include/echo_gguf.h)."""
from __future__ import annotations

import ctypes as C
from dataclasses import fields

import numpy as np

from .engine import EngineConfig, _Cfg
from .lib import EchoHipError, load

F32, F16, Q4_K, Q8_0 = 0, 1, 10, 6


class _Tensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("type", C.c_uint32), ("n_dims", C.c_uint32), ("shape", C.c_uint64 * 4),
                ("offset", C.c_uint64), ("bytes", C.c_uint64), ("data", C.c_void_p)]


def _bind(L):
    vp, u64 = C.c_void_p, C.c_uint64
    L.ec_gguf_open.argtypes = [C.c_char_p, C.POINTER(vp)]
    L.ec_gguf_close.argtypes = [vp]
    L.ec_gguf_close.restype = None
    L.ec_gguf_tensor_count.argtypes = [vp]
    L.ec_gguf_tensor_count.restype = u64
    L.ec_gguf_tensor_at.argtypes = [vp, u64, C.POINTER(_Tensor)]
    L.ec_gguf_find_tensor.argtypes = [vp, C.c_char_p, C.POINTER(_Tensor)]
    L.ec_gguf_get_uint.argtypes = [vp, C.c_char_p, C.POINTER(u64)]
    L.ec_gguf_get_float.argtypes = [vp, C.c_char_p, C.POINTER(C.c_double)]
    L.ec_gguf_get_string.argtypes = [vp, C.c_char_p, C.POINTER(C.c_char_p)]
    L.ec_gguf_token_count.argtypes = [vp]
    L.ec_gguf_token_count.restype = u64
    L.ec_gguf_token.argtypes = [vp, u64]
    L.ec_gguf_token.restype = C.c_char_p
    L.ec_gguf_alignment.argtypes = [vp]
    L.ec_gguf_alignment.restype = C.c_uint32
    L.ec_gguf_data_offset.argtypes = [vp]
    L.ec_gguf_data_offset.restype = u64
    L.ec_gguf_arch_prefix.argtypes = [vp]
    L.ec_gguf_arch_prefix.restype = C.c_char_p
    L.ec_gguf_engine_config.argtypes = [vp, C.c_uint32, C.c_uint32, C.POINTER(_Cfg)]
    L.ec_engine_load_gguf.argtypes = [vp, vp]


class GGUF:
    """A mapped GGUF v3 file.  Tensor data are copies (numpy uint8) of the mapped bytes."""

    def __init__(self, path):
        self.L = load().L
        _bind(self.L)
        h = C.c_void_p()
        self._check(self.L.ec_gguf_open(str(path).encode(), C.byref(h)), "ec_gguf_open")
        self.h = h

    def _check(self, rc, name):
        if rc != 0:
            raise EchoHipError(f"{name} failed ({rc}): {self.L.ec_last_error().decode()}")

    def close(self):
        if getattr(self, "h", None):
            self.L.ec_gguf_close(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    @staticmethod
    def _info(t: _Tensor, with_data):
        d = {"name": t.name.decode(), "type": t.type, "shape": list(t.shape[:t.n_dims]), "offset": t.offset,
             "bytes": t.bytes}
        if with_data:
            d["data"] = np.ctypeslib.as_array((C.c_uint8 * t.bytes).from_address(t.data)).copy() if t.bytes else \
                np.zeros(0, np.uint8)
        return d

    def names(self):
        out = []
        for i in range(self.L.ec_gguf_tensor_count(self.h)):
            t = _Tensor()
            self._check(self.L.ec_gguf_tensor_at(self.h, i, C.byref(t)), "ec_gguf_tensor_at")
            out.append(t.name.decode())
        return out

    def tensor(self, name, data=True):
        t = _Tensor()
        self._check(self.L.ec_gguf_find_tensor(self.h, name.encode(), C.byref(t)), "ec_gguf_find_tensor")
        return self._info(t, data)

    def get_uint(self, key):
        v = C.c_uint64()
        self._check(self.L.ec_gguf_get_uint(self.h, key.encode(), C.byref(v)), "ec_gguf_get_uint")
        return v.value

    def get_float(self, key):
        v = C.c_double()
        self._check(self.L.ec_gguf_get_float(self.h, key.encode(), C.byref(v)), "ec_gguf_get_float")
        return v.value

    def get_string(self, key):
        v = C.c_char_p()
        self._check(self.L.ec_gguf_get_string(self.h, key.encode(), C.byref(v)), "ec_gguf_get_string")
        return v.value.decode()

    def tokens(self):
        return [self.L.ec_gguf_token(self.h, i).decode() for i in range(self.L.ec_gguf_token_count(self.h))]

    @property
    def alignment(self):
        return self.L.ec_gguf_alignment(self.h)

    @property
    def data_offset(self):
        return self.L.ec_gguf_data_offset(self.h)

    @property
    def arch_prefix(self):
        return self.L.ec_gguf_arch_prefix(self.h).decode()

    def engine_config(self, max_batch, max_ctx) -> EngineConfig:
        c = _Cfg()
        self._check(self.L.ec_gguf_engine_config(self.h, max_batch, max_ctx, C.byref(c)), "ec_gguf_engine_config")
        return EngineConfig(**{f.name: getattr(c, f.name) for f in fields(EngineConfig)})

    def load_into(self, eng):
        """Upload the decoder's tensors into an Engine (ec_engine_load_gguf)."""
        self._check(self.L.ec_engine_load_gguf(eng.h, self.h), "ec_engine_load_gguf")
