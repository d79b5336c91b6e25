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

}  // namespace ec
