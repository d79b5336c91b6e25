// layout.hpp — sizes and offsets of the tiled weight and packed activation
// buffers (the byte layouts are documented at the top of quant.hip).
#pragma once
#include <cstddef>
#include <cstdint>
#include "echo_hip.h"

namespace ec {

constexpr uint32_t kQ8TChunk = 2176;  // 16 rows x 4 blocks: 2048 B qs + 128 B fp16 d
constexpr uint32_t kQ4TChunk = 2304;  // 16 rows x 1 super-block: 2048 B qs + 256 B headers

struct ActLayout {
    size_t xq_off, xd_off, dxs_off, total;
    uint32_t Kp;
};

__host__ __device__ inline uint32_t round_up(uint32_t x, uint32_t m) { return (x + m - 1) / m * m; }

__host__ __device__ inline ActLayout act_layout(int fmt, uint32_t M, uint32_t K) {
    ActLayout a;
    a.Kp = round_up(K, fmt == EC_Q4_K ? 256u : 128u);
    a.xq_off = 0;
    size_t xq = (size_t)a.Kp * M;
    a.xd_off = (xq + 255) & ~(size_t)255;
    size_t xd = (size_t)(a.Kp / 32) * 16 * sizeof(float);
    a.dxs_off = a.xd_off + xd;
    a.total = a.dxs_off + (fmt == EC_Q4_K ? xd : 0);
    return a;
}

// ---- packed q for decode attention (head_dim 256, int8 MFMA A operand)
// q of each head is split into kQPieces int8 vectors, q ~ sum_p s_p * Q_p with
// s_0 = max|q|/127 and s_{p+1} = s_p/254.  Per (sequence, kv head) the A bytes
// are [kQPieces*G rows][4 k-groups][64]: row p*G + g holds piece p of head
// kvh + n_kv*g; within a (row, k-group g') record, byte 8m + e is dim
// 16g' + 64(m/2) + 8(m%2) + e (m < 8, e < 8).  Scales [kQPieces*G] fp32 follow
// the same row order.
constexpr uint32_t kQPieces = 3;

__host__ __device__ inline size_t qa_bytes(uint32_t n_seq, uint32_t n_heads) {
    return (size_t)n_seq * n_heads * kQPieces * 4 * 64;
}

// k-group of dim d in bits 16.., byte position inside its 64-byte record in bits 0..15
__host__ __device__ inline uint32_t qa_offset(uint32_t d) {
    const uint32_t i = d / 64, gq = (d % 64) / 16, h = (d % 16) / 8, e = d % 8;
    return (gq << 16) | ((2 * i + h) * 8 + e);
}

#ifdef __HIPCC__
// Three int8 pieces of x for a group whose max |x| is amax:
//   x ~ sum_pc piece_pc * step_pc,  step_0 = amax/127, step_{pc+1} = step_pc/254,
// piece_pc = rint(r_pc / step_pc) (clamped), r_{pc+1} = r_pc - piece_pc*step_pc
// (one rounding, fma); the divisions are products with 1/step_pc, so each
// value costs one reciprocal per group (|x - sum| <= amax * 6.2e-8).
__device__ inline void split_pieces(float x, float amax, int8_t (&pc_out)[kQPieces], float (&step_out)[kQPieces]) {
    float step = amax > 0.0f ? amax * (1.0f / 127.0f) : 1.0f;
    float inv = amax > 0.0f ? 127.0f / amax : 1.0f;
    float r = x;
#pragma unroll
    for (uint32_t pc = 0; pc < kQPieces; ++pc) {
        const float qi = fminf(fmaxf(rintf(r * inv), -127.0f), 127.0f);
        pc_out[pc] = (int8_t)qi;
        step_out[pc] = step;
        r = fmaf(-qi, step, r);
        step = step * (1.0f / 254.0f);
        inv = inv * 254.0f;
    }
}

// The kQPieces int8 pieces of dim d of query head g (of G per kv head) given
// the head's max|q|: rows pc*G + g of one kv head's packed block at `rows`
// ([kQPieces*G][4][64] bytes), piece scales at sc[pc*G + g] (written by d == 0).
__device__ inline void pack_q_pieces(float val, float amax, uint32_t d, uint32_t g, uint32_t G,
                                     uint8_t* __restrict__ rows, float* __restrict__ sc) {
    const uint32_t off = qa_offset(d), gq = off >> 16, at = off & 0xFFFF;
    int8_t pcs[kQPieces];
    float steps[kQPieces];
    split_pieces(val, amax, pcs, steps);
#pragma unroll
    for (uint32_t pc = 0; pc < kQPieces; ++pc) {
        rows[((size_t)(pc * G + g) * 4 + gq) * 64 + at] = (uint8_t)pcs[pc];
        if (d == 0) sc[pc * G + g] = steps[pc];
    }
}

// Thread d of a 256-thread group stores dim d of (sequence s, head) given the head's max|q|.
__device__ inline void store_q_pieces(float val, float amax, uint32_t d, uint32_t s, uint32_t head, uint32_t n_heads,
                                      uint32_t n_kv, uint8_t* __restrict__ qa, float* __restrict__ qsc) {
    const uint32_t G = n_heads / n_kv, kvh = head % n_kv, g = head / n_kv;
    pack_q_pieces(val, amax, d, g, G, qa + ((size_t)s * n_kv + kvh) * (kQPieces * G) * 4 * 64,
                  qsc + ((size_t)s * n_kv + kvh) * kQPieces * G);
}
#endif

}  // namespace ec
