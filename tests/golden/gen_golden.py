"""Write golden vectors from the reference's own compiled kernels.

Run in a tree that holds the reference sources (``make -C oracle ref`` builds
oracle/_ref/libref.so from src/kernels/quant.cpp, src/kernels/matvec.cpp and
src/kv_cache.cpp with the reference's flags).  Inputs come from the seeded
generator in echohip.synth; outputs are whatever the reference computes.  The
result, tests/golden/kernels_golden.npz, is data only (inputs and expected
outputs) and is loaded with numpy's default allow_pickle=False.

    python tests/golden/gen_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "echo-core_amd"))
sys.path.insert(0, str(ROOT / "oracle"))

from echohip import synth  # noqa: E402
from oracle import Reference  # noqa: E402

OUT = Path(__file__).resolve().parent / "kernels_golden.npz"
LEGACY_OUT = Path(__file__).resolve().parent / "legacy_golden.npz"


def main() -> None:
    ref = Reference()
    f = ref.fn
    g: dict[str, np.ndarray] = {}

    # quantize_per_token_symmetric: several widths (body-only and body+tail rows)
    for width in (4, 8, 12, 16, 32, 37, 256, 1024):
        rows = 16
        x = synth.activations(100 + width, rows * width) * 3.0
        q = np.zeros(rows * width, np.int8)
        s = np.zeros(rows, np.float32)
        f["quantize_per_token_symmetric"](x, q, s, rows, width)
        g[f"quant_w{width}_x"] = x
        g[f"quant_w{width}_q"] = q
        g[f"quant_w{width}_s"] = s
    # rounding ties: scale = 1 (amax 127), body and tail both hold x.5 values
    ties = np.array([127.0, 2.5, 3.5, 0.5, -2.5, -3.5, -0.5, 1.5,
                     2.5, 3.5, 0.5, -2.5, -1.5, 126.5], np.float32)
    q = np.zeros(ties.size, np.int8)
    s = np.zeros(1, np.float32)
    f["quantize_per_token_symmetric"](ties, q, s, 1, ties.size)
    g["quant_ties_x"], g["quant_ties_q"], g["quant_ties_s"] = ties, q, s
    # all-zero row
    z = np.zeros(32, np.float32)
    q = np.zeros(32, np.int8)
    s = np.zeros(1, np.float32)
    f["quantize_per_token_symmetric"](z, q, s, 1, 32)
    g["quant_zero_q"], g["quant_zero_s"] = q, s

    # fused_dequant_dot_int8 over a [seq x dim] int8 matrix
    dim, seq = 256, 64
    keys_f = synth.activations(7, seq * dim)
    kq = np.zeros(seq * dim, np.int8)
    ks = np.zeros(seq, np.float32)
    f["quantize_per_token_symmetric"](keys_f, kq, ks, seq, dim)
    qv = synth.activations(8, dim)
    sc = np.zeros(seq, np.float32)
    f["fused_dequant_dot_int8"](qv, kq, ks, sc, dim, seq)
    g.update(int8dot_q=qv, int8dot_k=kq, int8dot_s=ks, int8dot_out=sc)

    # Q8_0 / Q4_K row dots and matvecs (accumulate into a nonzero y)
    M, K = 64, 512
    W8 = synth.q8_0_blocks(11, M, K)
    W4 = synth.q4_K_blocks(12, M, K)
    x = synth.activations(13, K)
    y0 = synth.activations(14, M)
    g.update(q8_W=W8, q4_W=W4, mv_x=x, mv_y0=y0)
    g["q8_fused"] = np.array([f["fused_dequant_dot_q8_0"](np.ascontiguousarray(W8[m]), K // 32, x)
                              for m in range(M)], np.float32)
    g["q4_fused"] = np.array([f["fused_dequant_dot_q4_K"](np.ascontiguousarray(W4[m]), K // 256, x)
                              for m in range(M)], np.float32)
    y = y0.copy()
    f["matvec_q8_0"](W8.reshape(-1), x, y, M, K)
    g["q8_matvec"] = y
    y = y0.copy()
    f["matvec_q4_K"](W4.reshape(-1), x, y, M, K)
    g["q4_matvec"] = y
    # single non-zero nibble per position: reveals the reference's nibble->position map
    probe = np.zeros((256, 144), np.uint8)
    probe[:, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)  # d = 1
    probe[:, 4:16] = synth.pack_q4k_scales(np.ones((256, 8)), np.zeros((256, 8)))
    for pos in range(256):
        byte, hi = divmod(pos, 2)
        probe[pos, 16 + byte] = (1 << 4) if hi else 1
    xr = np.arange(1, 257, dtype=np.float32)
    g["q4_probe_W"] = probe
    g["q4_probe_x"] = xr
    g["q4_probe_y"] = np.array([f["fused_dequant_dot_q4_K"](np.ascontiguousarray(probe[p]), 1, xr)
                                for p in range(256)], np.float32)

    np.savez_compressed(OUT, **g)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(g)} arrays)")
    legacy(f)


def legacy(f) -> None:
    """Q2_K matvec, the three fp16 dequantizers and the fp16 matvec templates."""
    g: dict[str, np.ndarray] = {}
    # Q2_K blocks as the reference reads them (src/kernels/matvec.cpp:158-162):
    # fp16 d, fp16 dmin, 16 scale bytes, 64 bytes of 2-bit weights; 84 B / 256 weights
    M, K = 48, 512
    nb = K // 256
    raw = (synth.splitmix64(synth.stream_seed(21, 0), M * nb * 84) & np.uint64(0xFF)).astype(np.uint8)
    blocks = raw.reshape(M, nb, 84)
    d = (np.abs(synth.normal(synth.stream_seed(21, 1), M * nb * 2)) * 0.01).astype(np.float16)
    blocks[:, :, 0:4] = d.view(np.uint8).reshape(M, nb, 4)
    W2 = np.ascontiguousarray(blocks.reshape(M, nb * 84))
    x = synth.activations(22, K)
    y0 = synth.activations(23, M)
    y = y0.copy()
    f["matvec_q2_K"](W2.reshape(-1), x, y, M, K)
    g.update(q2_W=W2, q2_x=x, q2_y0=y0, q2_matvec=y)
    gold = np.load(OUT)
    for key, W, n in (("q8", gold["q8_W"], gold["q8_W"].shape[0] * 512),
                      ("q4", gold["q4_W"], gold["q4_W"].shape[0] * 512), ("q2", W2, M * K)):
        out = np.zeros(n, np.uint16)
        src = np.ascontiguousarray(W)
        name = {"q8": "q8_0", "q4": "q4_K", "q2": "q2_K"}[key]
        f[f"dequantize_{name}_to_fp16"](src.ctypes.data, out.ctypes.data, n)
        g[f"deq_{key}"] = out
    # fp16 matvec templates (y += W x, W row-major fp16 [M][K])
    Mf, Kf = 160, 1000
    Wf = (synth.normal(synth.stream_seed(24, 0), Mf * Kf) * 0.05).astype(np.float16)
    xf = synth.activations(25, Kf)
    yf0 = synth.activations(26, Mf)
    g.update(f16_W=Wf.view(np.uint16), f16_x=xf, f16_y0=yf0)
    for tk, tm in ((1024, 512), (2048, 1024)):
        y = yf0.copy()
        f[f"matvec_fp16_fp32<{tk},{tm}>"](Wf.view(np.uint16).ctypes.data, xf, y, Mf, Kf)
        g[f"f16_matvec_{tk}_{tm}"] = y
    np.savez_compressed(LEGACY_OUT, **g)
    print(f"wrote {LEGACY_OUT} ({LEGACY_OUT.stat().st_size} bytes, {len(g)} arrays)")


if __name__ == "__main__":
    main()
