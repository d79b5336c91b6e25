"""Seeded synthetic inputs shared by the GPU path, the tests and the CPU baseline.

Portable RNG: element ``i`` of stream ``s`` is the ``(i+1)``-th output of
splitmix64 started at ``stream_seed(seed, s)``; uniforms take the top 24 bits,
normals use Box-Muller in float64.  Every consumer (CPU baseline, GPU upload,
golden fixtures) builds its inputs from these functions, so identical seeds give
identical bytes on any host.

Block formats are GGUF's (the reference's ``block_q8_0`` / ``block_q4_K``,
include/kernels/quant.h:31-34 and :46-51): 34-byte Q8_0 blocks (fp16 ``d`` then
32 int8) and 144-byte Q4_K super-blocks (fp16 ``d``, fp16 ``dmin``, 12 packed
6-bit scale/min bytes, 128 nibble bytes).
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)

Q8_0_BLOCK_BYTES = 34
Q4_K_BLOCK_BYTES = 144


def splitmix64(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """Elements offset..offset+n-1 of the splitmix64 stream started at ``seed``."""
    with np.errstate(over="ignore"):
        i = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + i * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def stream_seed(seed: int, stream: int) -> int:
    return int(splitmix64(seed, 1, offset=stream)[0])


def uniform01(seed: int, n: int) -> np.ndarray:
    """float64 uniforms on [0, 1) with 24-bit resolution."""
    return (splitmix64(seed, n) >> np.uint64(40)).astype(np.float64) * (1.0 / (1 << 24))


def normal(seed: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    """Box-Muller normals (float64): sqrt(-2 ln(1-u1)) * cos(2 pi u2)."""
    u = uniform01(seed, 2 * n)
    u1 = 1.0 - u[0::2]
    u2 = u[1::2]
    return mean + std * np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)


def randint(seed: int, n: int, lo: int, hi: int) -> np.ndarray:
    """Integers uniform on [lo, hi] (inclusive), int64."""
    r = splitmix64(seed, n) % np.uint64(hi - lo + 1)
    return r.astype(np.int64) + lo


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


# ----------------------------------------------------------------- Q8_0 blocks
def q8_0_blocks(seed: int, rows: int, K: int, d_std: float = 0.02) -> np.ndarray:
    """GGUF Q8_0 bytes [rows, K/32*34]: qs ~ U{-127..127}, d = fp16(|N(0,1)| * d_std)."""
    assert K % 32 == 0
    nb = K // 32
    qs = randint(stream_seed(seed, 0), rows * K, -127, 127).astype(np.int8).reshape(rows, nb, 32)
    d = (np.abs(normal(stream_seed(seed, 1), rows * nb)) * d_std).astype(np.float16).reshape(rows, nb)
    out = np.empty((rows, nb, Q8_0_BLOCK_BYTES), dtype=np.uint8)
    out[:, :, 0:2] = d.view(np.uint8).reshape(rows, nb, 2)
    out[:, :, 2:] = qs.view(np.uint8)
    return out.reshape(rows, nb * Q8_0_BLOCK_BYTES)


def q8_0_from_parts(qs: np.ndarray, d: np.ndarray) -> np.ndarray:
    """Assemble GGUF Q8_0 bytes from int8 qs [rows, nb, 32] and fp16 d [rows, nb]."""
    rows, nb, _ = qs.shape
    out = np.empty((rows, nb, Q8_0_BLOCK_BYTES), dtype=np.uint8)
    out[:, :, 0:2] = np.ascontiguousarray(d.astype(np.float16)).view(np.uint8).reshape(rows, nb, 2)
    out[:, :, 2:] = qs.astype(np.int8).view(np.uint8)
    return out.reshape(rows, nb * Q8_0_BLOCK_BYTES)


# ----------------------------------------------------------------- Q4_K blocks
def pack_q4k_scales(sc: np.ndarray, m: np.ndarray) -> np.ndarray:
    """Pack 8 six-bit scales and mins per super-block into 12 bytes, the inverse
    of get_scale_min_k4 (src/kernels/quant.cpp:222-242).  sc, m: [..., 8]."""
    sc = sc.astype(np.uint8)
    m = m.astype(np.uint8)
    q = np.zeros(sc.shape[:-1] + (12,), dtype=np.uint8)
    for j in range(4):
        q[..., j] = sc[..., j] & 63
        q[..., j + 4] = m[..., j] & 63
    for j in range(4, 8):
        q[..., j + 4] = (sc[..., j] & 0x0F) | ((m[..., j] & 0x0F) << 4)
        q[..., j - 4] |= (sc[..., j] >> 4) << 6
        q[..., j] |= (m[..., j] >> 4) << 6
    return q


def q4_K_blocks(seed: int, rows: int, K: int, d_std: float = 0.01) -> np.ndarray:
    """GGUF Q4_K bytes [rows, K/256*144]: d, dmin = fp16(|N(0,1)|*d_std);
    sub-scales and mins ~ U{0..63}; nibbles ~ U{0..15}."""
    assert K % 256 == 0
    nb = K // 256
    n = rows * nb
    d = (np.abs(normal(stream_seed(seed, 0), n)) * d_std).astype(np.float16)
    dmin = (np.abs(normal(stream_seed(seed, 1), n)) * d_std).astype(np.float16)
    sc = randint(stream_seed(seed, 2), n * 8, 0, 63).reshape(n, 8)
    mn = randint(stream_seed(seed, 3), n * 8, 0, 63).reshape(n, 8)
    nib = randint(stream_seed(seed, 4), n * 256, 0, 15).astype(np.uint8).reshape(n, 128, 2)
    out = np.empty((n, Q4_K_BLOCK_BYTES), dtype=np.uint8)
    out[:, 0:2] = d.view(np.uint8).reshape(n, 2)
    out[:, 2:4] = dmin.view(np.uint8).reshape(n, 2)
    out[:, 4:16] = pack_q4k_scales(sc, mn)
    out[:, 16:] = nib[:, :, 0] | (nib[:, :, 1] << 4)
    return out.reshape(rows, nb * Q4_K_BLOCK_BYTES)


# ------------------------------------------------------------- activations
def activations(seed: int, n: int) -> np.ndarray:
    return normal(seed, n).astype(np.float32)
