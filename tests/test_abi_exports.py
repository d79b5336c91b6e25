"""The drop-in library exports what the headers in include/ declare.

* C ABI (echo_hip.h, echo_engine.h, echo_gguf.h): every `ec_*` function declared there is
  found by the dynamic loader in libechohip.so (loaded with ctypes; no GPU call
  is made).
* Reference-signature C++ interface (include/kernels/*.h, include/kv_cache.h):
  a translation unit that calls every declared function is compiled with g++
  against the headers, and every mangled symbol it needs is defined by
  libechohip.so -- the link contract of a program built against the
  reference's headers.
* include/types.h half-precision helpers: decode is exact for all 65536
  halves and encode rounds to nearest even (checked against numpy).
"""
import ctypes as C
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
INC = ROOT / "include"
LIB = ROOT / "echo-core_amd" / "libechohip.so"

pytestmark = pytest.mark.skipif(not LIB.exists(), reason="libechohip.so not built")


def _declared_c_functions():
    names = set()
    for h in ("echo_hip.h", "echo_engine.h", "echo_gguf.h"):
        text = (INC / h).read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"^[A-Za-z_][\w\s\*]*?\b(ec_\w+)\s*\(", text, flags=re.M))
    return sorted(names)


def test_c_abi_symbols_exported():
    names = _declared_c_functions()
    assert len(names) > 30, names
    lib = C.CDLL(str(LIB))
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def _defined_symbols():
    out = subprocess.run(["nm", "-D", "--defined-only", str(LIB)], check=True, capture_output=True, text=True)
    return {line.split()[-1] for line in out.stdout.splitlines() if line.strip()}


@pytest.mark.parametrize("src", ["abi_use.cpp", "gguf_use.cpp", "inference_use.cpp"])
def test_reference_signature_symbols_exported(tmp_path, src):
    obj = tmp_path / "use.o"
    subprocess.run(["g++", "-std=c++17", "-c", "-I", str(INC), str(ROOT / "tests" / "abi" / src), "-o",
                    str(obj)], check=True)
    out = subprocess.run(["nm", "-u", str(obj)], check=True, capture_output=True, text=True)
    needed = {line.split()[-1] for line in out.stdout.splitlines() if line.strip()}
    # C library and C++ standard library symbols are not ours
    needed = {s for s in needed if s.startswith("_Z") and not s.startswith(("_ZSt", "_ZNSt", "_ZNKSt", "_ZTISt",
                                                                           "_ZTVN10__cxxabiv", "_ZNSo", "_ZNKSo",
                                                                           "_ZNSa", "_ZNKSa"))}
    # the C++ runtime's own symbols (operator new/delete, unwinder) are not ours
    needed = {s for s in needed if not s.startswith(("_Znw", "_Zdl", "__cxa", "_Unwind", "__gxx", "__stack_chk"))}
    assert len(needed) >= (20 if src == "abi_use.cpp" else 3), needed
    missing = sorted(needed - _defined_symbols())
    assert not missing, missing


def test_types_h_half_conversions(tmp_path):
    src = tmp_path / "half.cpp"
    src.write_text(r'''
#include <cstdio>
#include "types.h"
int main() {
    for (unsigned h = 0; h < 65536; ++h) {
        float f = fp16_to_fp32((fp16_t)h);
        unsigned u; std::memcpy(&u, &f, 4); std::printf("%08x\n", u);
    }
    unsigned x;
    while (std::scanf("%x", &x) == 1) {
        float f; std::memcpy(&f, &x, 4); std::printf("%04x\n", fp32_to_fp16(f));
    }
}
''')
    exe = tmp_path / "half"
    subprocess.run(["g++", "-std=c++17", "-O1", "-I", str(INC), str(src), "-o", str(exe)], check=True)
    rng = np.random.default_rng(0)
    probes = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 6.1035156e-05, 5.9604645e-08,
                  2.9802322e-08, 2.9802326e-08, 8.9406967e-08, np.inf, -np.inf], np.float32),
        (np.arange(-4096, 4096, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -20),
    ]).astype(np.float32)
    inp = "\n".join(f"{v:08x}" for v in probes.view(np.uint32)) + "\n"
    out = subprocess.run([str(exe)], input=inp, check=True, capture_output=True, text=True).stdout.split()
    dec = np.array([int(s, 16) for s in out[:65536]], np.uint32).view(np.float32)
    ref = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(dec), nan)
    assert np.array_equal(dec[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    enc = np.array([int(s, 16) for s in out[65536:]], np.uint32).astype(np.uint16)
    want = probes.astype(np.float16).view(np.uint16)
    assert np.array_equal(enc, want), np.flatnonzero(enc != want)[:10]


def test_argument_checks_before_any_gpu_call():
    """Entry points refuse bad arguments on the host, before any HIP call (no GPU needed): a GEMM activation
    source that is not 16-byte aligned (the quantizer reads 16-byte pieces), and null pointers for the greedy
    pick in both its original and its bounded form."""
    lib = C.CDLL(str(LIB))
    lib.ec_last_error.restype = C.c_char_p
    vp = C.c_void_p
    lib.ec_gemm_quantize_act.argtypes = [C.c_int, vp, vp, C.c_uint32, C.c_uint32, vp]
    assert lib.ec_gemm_quantize_act(6, 0x10004, 0x20000, 4, 256, None) == 1
    assert b"16-byte aligned" in lib.ec_last_error()
    lib.ec_glue_argmax_advance.argtypes = [vp, C.c_uint32, vp, vp, vp, C.c_uint32, vp]
    assert lib.ec_glue_argmax_advance(None, 100, None, None, None, 1, None) == 1
    lib.ec_glue_argmax_advance_bounded.argtypes = [vp, C.c_uint32, vp, vp, vp, C.c_uint32, C.c_uint32, vp]
    assert lib.ec_glue_argmax_advance_bounded(None, 100, None, None, None, 1, 64, None) == 1
