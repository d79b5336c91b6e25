// gemm_act.hpp — the prefill GEMM's Q8_0 activation layout ("XT") and the
// device code that quantizes into it, shared by the quantize pass (gemm.hip)
// and the row kernels that write their output straight into it (glue.hip).
//
// Tokens in tiles of 16, K padded to Kp (a multiple of 128: Q8_0 chunks of 4
// blocks, 256 for Q4_K super-blocks):
//   Q8_0: chunk (token tile T, group G of 4 blocks) = 2048 B at (T*nch+G)*2048,
//         lane l's 16 B at 16l (blocks 0,1) and 1024+16l (blocks 2,3), 8 B per
//         block = x[16T + l%16][128G + 32j + 8(l/16) .. +8] (the MFMA A operand);
//   xd  fp32 [Mp][Kp/32] block scales (0 for padding tokens; padding blocks
//         of real tokens hold zero bytes and scale 1, as the quantizer gives
//         for an all-zero block).
// The quantization is the reference's (src/kernels/quant.cpp:18-98): scale =
// amax/127, bytes rne(x * (1/scale)) -- every block is whole 8-chunks.
#pragma once
#include "common.hpp"
#include "layout.hpp"

namespace ec {

struct XtLayout {
    uint32_t Mp, Kp, nch;  // padded tokens, padded K, chunks per token tile
    size_t xq_bytes, xd_off, dxs_off, total;
};

__host__ __device__ inline XtLayout xt_layout(int fmt, uint32_t M, uint32_t K) {
    XtLayout L;
    L.Mp = round_up(M, 16);
    const bool q4 = fmt == EC_Q4_K;
    L.Kp = round_up(K, q4 ? 256u : 128u);
    L.nch = L.Kp / (q4 ? 256u : 128u);
    L.xq_bytes = (size_t)(L.Mp / 16) * L.nch * (q4 ? 4096u : 2048u);
    L.xd_off = (L.xq_bytes + 255) & ~(size_t)255;
    const size_t xd = (size_t)L.Mp * (L.Kp / 32) * sizeof(float);
    L.dxs_off = L.xd_off + ((xd + 255) & ~(size_t)255);
    L.total = L.dxs_off + (q4 ? xd : 0);
    return L;
}

#ifdef __HIPCC__
// Token m's elements 4q .. 4q+3 (block q/8), four per lane: the 8 lanes of a
// block must be 8 consecutive, 8-aligned lanes (lane % 8 == q % 8), all
// active.  v = 0 for padding.  real: m < M (else the scale is stored as 0).
__device__ __forceinline__ void xt_q8_store4(float4 v, uint32_t m, uint32_t q, bool real, uint8_t* __restrict__ xt,
                                             uint32_t nch, uint32_t nbp, size_t xd_off) {
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = fmaxf(amax, lane_xor<1>(amax));
    amax = fmaxf(amax, lane_xor<2>(amax));
    amax = fmaxf(amax, lane_xor<4>(amax));
    const float scale = q_scale(amax);
    const float inv = __fdiv_rn(1.0f, scale);
    const uint32_t w4 = (uint32_t)(uint8_t)q_body(v.x, inv) | ((uint32_t)(uint8_t)q_body(v.y, inv) << 8) |
                        ((uint32_t)(uint8_t)q_body(v.z, inv) << 16) | ((uint32_t)(uint8_t)q_body(v.w, inv) << 24);
    // elements 8g .. 8g+7 of the block (lanes 2g, 2g+1 of its group) are the
    // 8 bytes of operand lane m%16 + 16g
    const uint32_t hi = row_down<1>(w4);
    const uint32_t b = q / 8, e = q & 7;
    if ((e & 1) == 0) {
        const uint32_t G = b / 4, j = b % 4, l = m % 16 + 16 * (e / 2);
        *(uint2*)(xt + ((size_t)(m / 16) * nch + G) * 2048 + (j / 2) * 1024 + 16 * l + 8 * (j % 2)) = make_uint2(w4, hi);
    }
    if (e == 0) ((float*)(xt + xd_off))[(size_t)m * nbp + b] = real ? scale : 0.0f;
}

// Token m's element k (block k/32), one per lane: the 32 lanes of a block must
// be 32 consecutive, 32-aligned lanes (lane % 32 == k % 32), all active.
__device__ __forceinline__ void xt_q8_store1(float v, uint32_t m, uint32_t k, bool real, uint8_t* __restrict__ xt,
                                             uint32_t nch, uint32_t nbp, size_t xd_off) {
    float amax = fabsf(v);
    amax = fmaxf(amax, lane_xor<1>(amax));
    amax = fmaxf(amax, lane_xor<2>(amax));
    amax = fmaxf(amax, lane_xor<4>(amax));
    amax = fmaxf(amax, lane_xor<8>(amax));
    amax = fmaxf(amax, lane_xor<16>(amax));
    const float scale = q_scale(amax);
    const float inv = __fdiv_rn(1.0f, scale);
    const uint32_t qb = (uint8_t)q_body(v, inv);
    // 4 consecutive elements' bytes gathered at the first lane of each 4,
    // elements 8g .. 8g+7 at the first lane of each 8
    const uint32_t w4 = qb | (row_down<1>(qb) << 8) | (row_down<2>(qb) << 16) | (row_down<3>(qb) << 24);
    const uint32_t hi = row_down<4>(w4);
    const uint32_t b = k / 32, i = k % 32;
    if ((i & 7) == 0) {
        const uint32_t G = b / 4, j = b % 4, l = m % 16 + 16 * (i / 8);
        *(uint2*)(xt + ((size_t)(m / 16) * nch + G) * 2048 + (j / 2) * 1024 + 16 * l + 8 * (j % 2)) = make_uint2(w4, hi);
    }
    if (i == 0) ((float*)(xt + xd_off))[(size_t)m * nbp + b] = real ? scale : 0.0f;
}
#endif

}  // namespace ec
