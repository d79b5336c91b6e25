// gemm.hip — prefill GEMM over block-quantized weights on int8 MFMA (gfx950).
//
// Y[m][n] (+)= sum over K of X[m][k] * W[n][k] for M tokens (prefill chunks,
// e.g. 512), with X quantized per 32-element block by the reference quantizer
// (src/kernels/quant.cpp:18-98) and W in the tiled decode layout (quant.hip).
// Every 32-block product is one exact int32 (v_mfma_i32_16x16x32_i8: A = 16
// tokens x 32 int8, B = 32 int8 x 16 weight rows); the fp32 epilogue applies
// the block scales:
//   Q8_0: Y += d_x[m,b] * d_w[n,b] * isum_b
//   Q4_K: Y += d_x[m,s] * (d*sc_s * isum_s - dmin*m_s * xsum_s)   (per sub-block s)
// which is the reference's matvec arithmetic (matvec.cpp:62-142) on the
// quantized activations, in a different summation order.
//
// Activation layout ("XT", gemm_act.hpp), tokens in tiles of 16:
//   Q8_0: chunk (token tile T, group G of 4 blocks) = 2048 B at (T*nG+G)*2048,
//         lane l's 16 B at 16l (blocks 0,1) and 1024+16l (blocks 2,3), 8 B per
//         block = x[16T + l%16][128G + 32j + 8(l/16) .. +8] (the MFMA A operand);
//   Q4_K: chunk (T, super-block b) = 4096 B, lane l's 8 B per sub-block s at
//         (s/2)*1024 + 16l + 8(s%2): the sub-block's elements 4g..4g+3 and
//         16+4g..16+4g+3 (g = l/16) in the reference's Q4_K position order
//         (so they meet the weight nibbles of the same positions);
//   xd  fp32 [Mp][Kp/32] block scales; Q4_K adds dxs = xd * sum(block int8).
//
// Tiling: a 256-thread workgroup computes 64 tokens x (32*RTW) rows; each wave
// 32 tokens (2 token tiles) x 16*RTW rows.  Per K chunk a wave loads its A and
// B operands straight from global memory (16-byte loads, the next chunk's
// loads issued before the current chunk's MFMAs), the workgroup stages the
// chunk's activation scales in LDS.  The epilogue (int32 -> fp32, scale,
// accumulate: 3 VALU ops per output element per block for Q8_0, 4 for Q4_K)
// costs more issue slots than the MFMA itself: the kernel is VALU-bound at
// roughly a third of the int8 MFMA peak by construction of 32-element scales.
#include <type_traits>

#include "gemm_act.hpp"

namespace ec {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ long gpack2(uint32_t lo, uint32_t hi) {
    return (long)(((uint64_t)hi << 32) | (uint64_t)lo);
}

// ----------------------------------------------------------- activation prep
// Q4_K with 16-byte loads: a wave takes one super-block (256 elements) of its
// token per step, lane l elements 4l .. 4l+3.  Sub-block s = 2h + j holds the
// runs 64h + 16j + (0..15) and 64h + 32 + 16j + (0..15) (the reference's
// position order), i.e. lanes 16h + 4j + (0..3) and those 8 above: the
// sub-block's amax and int8 sum take xor 1, 2, 8 over its 8 lanes, and the
// run-0 lane stores its 4 bytes with the run-1 lane's 4 (bytes 4g .. 4g+3 and
// 16+4g .. 16+4g+3 of operand lane token%16 + 16g).  The reference
// quantizer per sub-block (scale = amax/127, bytes rne(x * (1/scale)), dxs =
// scale * the sub-block's int8 sum).  grid (ceil(nch / 2), Mp / 4).
__global__ __launch_bounds__(256) void k_gemm_quantize_x4v(const float* __restrict__ x, uint8_t* __restrict__ xt,
                                                           uint32_t M, uint32_t K, uint32_t ldx, uint32_t nch,
                                                           uint32_t nbp, size_t xd_off, size_t dxs_off) {
    const uint32_t lane = threadIdx.x & 63, m = blockIdx.y * 4 + (threadIdx.x >> 6);
    const uint32_t b0 = blockIdx.x * 2, h = lane / 16, j = (lane & 7) / 4, g = lane & 3;
    const uint32_t s = 2 * h + j;
    float4 v[2];
#pragma unroll
    for (uint32_t st = 0; st < 2; ++st) {
        const uint32_t k = 256 * (b0 + st) + 4 * lane;  // K % 256 == 0
        v[st] = (m < M && k < K) ? *(const float4*)(x + (size_t)m * ldx + k) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (uint32_t st = 0; st < 2; ++st) {
        const uint32_t b = b0 + st;
        if (b >= nch) break;  // uniform over the wave
        float amax = fmaxf(fmaxf(fabsf(v[st].x), fabsf(v[st].y)), fmaxf(fabsf(v[st].z), fabsf(v[st].w)));
        amax = fmaxf(amax, lane_xor<1>(amax));
        amax = fmaxf(amax, lane_xor<2>(amax));
        amax = fmaxf(amax, lane_xor<8>(amax));
        const float scale = q_scale(amax);
        const float inv = __fdiv_rn(1.0f, scale);
        const int8_t q0 = q_body(v[st].x, inv), q1 = q_body(v[st].y, inv), q2 = q_body(v[st].z, inv),
                     q3 = q_body(v[st].w, inv);
        const uint32_t w4 = (uint32_t)(uint8_t)q0 | ((uint32_t)(uint8_t)q1 << 8) | ((uint32_t)(uint8_t)q2 << 16) |
                            ((uint32_t)(uint8_t)q3 << 24);
        const uint32_t hi = row_down<8>(w4);
        int sum = (int)q0 + (int)q1 + (int)q2 + (int)q3;
        sum += lane_xor_i<1>(sum);
        sum += lane_xor_i<2>(sum);
        sum += lane_xor_i<8>(sum);
        if ((lane & 8) == 0) {  // run-0 lanes
            const uint32_t l = m % 16 + 16 * g;
            *(uint2*)(xt + ((size_t)(m / 16) * nch + b) * 4096 + h * 1024 + 16 * l + 8 * j) = make_uint2(w4, hi);
            if (g == 0) {
                ((float*)(xt + xd_off))[(size_t)m * nbp + 8 * b + s] = m < M ? scale : 0.0f;
                ((float*)(xt + dxs_off))[(size_t)m * nbp + 8 * b + s] = scale * (float)sum;
            }
        }
    }
}

// Q8_0: each lane quantizes 4 consecutive elements (one 16-byte load), 8
// consecutive lanes a 32-element block; a wave covers 8 blocks (1 KB of its
// token's row) per step and kQxSteps steps, the workgroup's four waves four
// tokens.  grid (ceil(nbp / (8 kQxSteps)), Mp / 4).
constexpr uint32_t kQxSteps = 2;
__global__ __launch_bounds__(256) void k_gemm_quantize_x8(const float* __restrict__ x, uint8_t* __restrict__ xt,
                                                          uint32_t M, uint32_t K, uint32_t ldx, uint32_t nch,
                                                          uint32_t nbp, size_t xd_off) {
    const uint32_t lane = threadIdx.x & 63, m = blockIdx.y * 4 + (threadIdx.x >> 6);
    const uint32_t q0 = blockIdx.x * 64 * kQxSteps;  // first float4 of the wave
    float4 v[kQxSteps];
#pragma unroll
    for (uint32_t st = 0; st < kQxSteps; ++st) {
        const uint32_t k = 4 * (q0 + 64 * st + lane);  // K % 32 == 0: a block is all real or all padding
        v[st] = (m < M && k < K) ? *(const float4*)(x + (size_t)m * ldx + k) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (uint32_t st = 0; st < kQxSteps; ++st) {
        const uint32_t q = q0 + 64 * st + lane;
        if (q / 8 < nbp) xt_q8_store4(v[st], m, q, m < M, xt, nch, nbp, xd_off);  // whole 8-lane groups
    }
}

// ------------------------------------------------------------------ Q8_0
template <int RTW>
__global__ __launch_bounds__(256, 2) void k_gemm_q8_0(const uint8_t* __restrict__ W, const uint8_t* __restrict__ xt,
                                                   float* __restrict__ y, uint32_t M, uint32_t N, uint32_t n_tt,
                                                   uint32_t n_rt, uint32_t nG, uint32_t nbp, size_t xd_off,
                                                   uint32_t ldy, int accumulate) {
    constexpr int TTW = 2;
    __shared__ float dx_s[2][4][64];  // [buffer][block j of the chunk][token of the workgroup tile]
    const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 4;
    const uint32_t wt = w & 1, wr = w >> 1;
    const uint32_t tt0 = blockIdx.y * 4 + wt * TTW;
    const uint32_t rt0 = blockIdx.x * (2 * RTW) + wr * RTW;
    const float* xd = (const float*)(xt + xd_off);
    const uint32_t tok = blockIdx.y * 64 + (threadIdx.x & 63), jj = threadIdx.x >> 6;  // scale staging

    float acc[TTW][RTW][4];
#pragma unroll
    for (int t = 0; t < TTW; ++t)
#pragma unroll
        for (int r = 0; r < RTW; ++r)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[t][r][e] = 0.0f;

    u32x4 a[2][TTW][2], b[2][RTW][2];
    uint2 dw[2][RTW];
    float dxv[2];
    auto load = [&](int buf, uint32_t G) {
#pragma unroll
        for (int t = 0; t < TTW; ++t) {
            const uint32_t T = min(tt0 + t, n_tt - 1);
            const uint8_t* p = xt + ((size_t)T * nG + G) * 2048 + 16 * lane;
            a[buf][t][0] = *(const u32x4*)p;
            a[buf][t][1] = *(const u32x4*)(p + 1024);
        }
#pragma unroll
        for (int r = 0; r < RTW; ++r) {
            const uint32_t R = min(rt0 + r, n_rt - 1);
            const uint8_t* p = W + ((size_t)R * nG + G) * kQ8TChunk;
            b[buf][r][0] = *(const u32x4*)(p + 16 * lane);
            b[buf][r][1] = *(const u32x4*)(p + 1024 + 16 * lane);
            dw[buf][r] = *(const uint2*)(p + 2048 + 8 * (lane & 15));
        }
        dxv[buf] = tok < n_tt * 16 ? xd[(size_t)tok * nbp + 4 * G + jj] : 0.0f;
    };

    // register buffers are indexed by compile-time constants: the chunk loop is
    // unrolled by two (even chunks in buffer 0, odd chunks in buffer 1)
    auto step = [&](auto bufc, uint32_t G) {
        constexpr int cur = decltype(bufc)::value;
        dx_s[cur][jj][threadIdx.x & 63] = dxv[cur];
        __syncthreads();
        if (G + 1 < nG) load(cur ^ 1, G + 1);
        // blocks in pairs: both blocks' MFMAs are issued before either
        // block's epilogue, so the epilogue does not wait on the MFMA it
        // follows (9216 x 2560 / 2560 x 9216 / 18432 x 2560 at M = 512:
        // 69.9 / 83.3 / 120.8 -> 67.7 / 77.5 / 117.0 us; all four blocks
        // first: 68.4 / 79.2 / 117.6)
#pragma unroll
        for (int j0 = 0; j0 < 4; j0 += 2) {
            v4i c[2][TTW][RTW];
            float dwf[2][RTW];
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const int j = j0 + jj;
                long A[TTW], B[RTW];
#pragma unroll
                for (int t = 0; t < TTW; ++t) {
                    const u32x4 v = a[cur][t][j >> 1];
                    A[t] = (j & 1) ? gpack2(v.z, v.w) : gpack2(v.x, v.y);
                }
#pragma unroll
                for (int r = 0; r < RTW; ++r) {
                    const u32x4 v = b[cur][r][j >> 1];
                    B[r] = (j & 1) ? gpack2(v.z, v.w) : gpack2(v.x, v.y);
                    const uint32_t h = (j < 2) ? dw[cur][r].x : dw[cur][r].y;
                    dwf[jj][r] = h2f((j & 1) ? (h >> 16) : (h & 0xFFFF));
                }
#pragma unroll
                for (int t = 0; t < TTW; ++t)
#pragma unroll
                    for (int r = 0; r < RTW; ++r) {
                        const v4i z = {0, 0, 0, 0};
                        c[jj][t][r] = __builtin_amdgcn_mfma_i32_16x16x32_i8(A[t], B[r], z, 0, 0, 0);
                    }
            }
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const int j = j0 + jj;
#pragma unroll
                for (int t = 0; t < TTW; ++t) {
                    const float4 d4 = *(const float4*)&dx_s[cur][j][(wt * TTW + t) * 16 + 4 * g];
                    const float dxe[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                    for (int r = 0; r < RTW; ++r)
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            acc[t][r][e] = fmaf((float)c[jj][t][r][e], dxe[e] * dwf[jj][r], acc[t][r][e]);
                }
            }
        }
    };
    load(0, 0);
    for (uint32_t G = 0; G < nG; G += 2) {
        step(std::integral_constant<int, 0>{}, G);
        if (G + 1 < nG) step(std::integral_constant<int, 1>{}, G + 1);
    }
    // D[i][j]: token row 4g+e of the token tile, weight row lane%16 of the row tile
#pragma unroll
    for (int t = 0; t < TTW; ++t)
#pragma unroll
        for (int r = 0; r < RTW; ++r) {
            const uint32_t n = 16 * (rt0 + r) + (lane & 15);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t m = 16 * (tt0 + t) + 4 * g + e;
                if (m < M && n < N && tt0 + t < n_tt && rt0 + r < n_rt) {
                    float* dst = y + (size_t)m * ldy + n;
                    *dst = accumulate ? *dst + acc[t][r][e] : acc[t][r][e];
                }
            }
        }
}

// ------------------------------------------------------------------ Q4_K
typedef float v4f __attribute__((ext_vector_type(4)));

// The eight 6-bit (scale, min) pairs of a super-block from its 12 scale
// bytes (q[0] = bytes 0-3, ...), four per dword: sc[0] holds sub-blocks 0-3
// (byte s = scale of sub-block s), sc[1] sub-blocks 4-7, mn likewise -- the
// unpack of src/kernels/quant.cpp:222-242 on four bytes per operation.
__device__ __forceinline__ void q4k_sm4(const uint32_t (&q)[3], uint32_t (&sc)[2], uint32_t (&mn)[2]) {
    sc[0] = q[0] & 0x3F3F3F3Fu;
    mn[0] = q[1] & 0x3F3F3F3Fu;
    sc[1] = (q[2] & 0x0F0F0F0Fu) | ((q[0] >> 2) & 0x30303030u);
    mn[1] = ((q[2] >> 4) & 0x0F0F0F0Fu) | ((q[1] >> 2) & 0x30303030u);
}

// Byte n of v as a float (v_cvt_f32_ubyte<n>).
__device__ __forceinline__ float ubyte_f(uint32_t v, int n) { return (float)((v >> (8 * n)) & 0xFFu); }

// The K loop steps over half super-blocks (128 elements, 4 sub-blocks: the
// Q8_0 kernel's chunk, so the double-buffered operands fit two waves per
// SIMD).  Per step a wave unpacks its rows' headers once: d*sc of the four
// sub-blocks (the integer dots' scale) and dmin*m of the sub-block its lane
// group feeds to the min-term product.  The min term
//   Y[t][n] -= sum_s (dmin*m)[n][s] * dxs[t][s]
// is a dense fp32 product with contraction over the sub-blocks: one
// v_mfma_f32_16x16x4_f32 per (token tile, row tile) and step (A = -dxs[token]
// [4h + k], B = (dmin*m)[4h + k][row]; lane l holds A[l%16][l/16] and
// B[l/16][l%16], its D layout the int8 MFMA's) into the same accumulators,
// once per step, so the running sums stay at the result's magnitude (the min
// and scale terms, each larger than the result, cancel every 4 sub-blocks as
// in the reference's per-sub-block form), and the per-(token, row,
// sub-block) epilogue is the Q8_0 kernel's: one conversion and one FMA per
// output element.
template <int RTW>
__global__ __launch_bounds__(256, 2) void k_gemm_q4_K(const uint8_t* __restrict__ W, const uint8_t* __restrict__ xt,
                                                      float* __restrict__ y, uint32_t M, uint32_t N, uint32_t n_tt,
                                                      uint32_t n_rt, uint32_t nB, uint32_t nbp, size_t xd_off,
                                                      size_t dxs_off, uint32_t ldy, int accumulate) {
    constexpr int TTW = 2;
    __shared__ float dx_s[2][4][64], dm_s[2][4][64];  // [buffer][sub-block of the step][token]
    const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 4, row = lane & 15;
    const uint32_t wt = w & 1, wr = w >> 1;
    const uint32_t tt0 = blockIdx.y * 4 + wt * TTW;
    const uint32_t rt0 = blockIdx.x * (2 * RTW) + wr * RTW;
    const float* xd = (const float*)(xt + xd_off);
    const float* dxs = (const float*)(xt + dxs_off);
    const uint32_t tok = blockIdx.y * 64 + (threadIdx.x & 63), sq = threadIdx.x >> 6;  // stages sub-block sq
    const uint32_t nC = 2 * nB;  // half super-blocks

    v4f acc[TTW][RTW];
#pragma unroll
    for (int t = 0; t < TTW; ++t)
#pragma unroll
        for (int r = 0; r < RTW; ++r) acc[t][r] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

    u32x4 a[2][TTW][2], b[2][RTW], hd[2][RTW];
    float sv[2][2];
    auto load = [&](int buf, uint32_t C) {
        const uint32_t B = C >> 1, h = C & 1;
#pragma unroll
        for (int t = 0; t < TTW; ++t) {
            const uint32_t T = min(tt0 + t, n_tt - 1);
            const uint8_t* p = xt + ((size_t)T * nB + B) * 4096 + 2048 * h + 16 * lane;
            a[buf][t][0] = *(const u32x4*)p;
            a[buf][t][1] = *(const u32x4*)(p + 1024);
        }
#pragma unroll
        for (int r = 0; r < RTW; ++r) {
            const uint32_t R = min(rt0 + r, n_rt - 1);
            const uint8_t* p = W + ((size_t)R * nB + B) * kQ4TChunk;
            b[buf][r] = *(const u32x4*)(p + 1024 * h + 16 * lane);
            hd[buf][r] = *(const u32x4*)(p + 2048 + 16 * row);
        }
        const bool ok = tok < n_tt * 16;
        const size_t at = (size_t)(ok ? tok : 0) * nbp + 8 * B + 4 * h + sq;
        sv[buf][0] = ok ? xd[at] : 0.0f;
        sv[buf][1] = ok ? dxs[at] : 0.0f;
    };

    auto step = [&](auto bufc, uint32_t C) {
        constexpr int cur = decltype(bufc)::value;
        const uint32_t h = C & 1;
        dx_s[cur][sq][threadIdx.x & 63] = sv[cur][0];
        dm_s[cur][sq][threadIdx.x & 63] = sv[cur][1];
        __syncthreads();
        if (C + 1 < nC) load(cur ^ 1, C + 1);
        // the rows' headers: this half's four (scale, min) pairs
        float dr[RTW], bmin[RTW];
        uint32_t scr[RTW];
#pragma unroll
        for (int r = 0; r < RTW; ++r) {
            const uint32_t scb[3] = {hd[cur][r].y, hd[cur][r].z, hd[cur][r].w};
            uint32_t sc4[2], mn4[2];
            q4k_sm4(scb, sc4, mn4);
            scr[r] = h ? sc4[1] : sc4[0];
            dr[r] = h2f(hd[cur][r].x & 0xFFFF);
            bmin[r] = h2f(hd[cur][r].x >> 16) * (float)(((h ? mn4[1] : mn4[0]) >> (8 * g)) & 0xFFu);
        }
        // min term on the fp32 matrix core
#pragma unroll
        for (int t = 0; t < TTW; ++t) {
            const float am = -dm_s[cur][g][(wt * TTW + t) * 16 + row];
#pragma unroll
            for (int r = 0; r < RTW; ++r)
                acc[t][r] = __builtin_amdgcn_mfma_f32_16x16x4f32(am, bmin[r], acc[t][r], 0, 0, 0);
        }
        // sub-blocks in pairs, both MFMAs issued before either epilogue (as
        // in the Q8_0 kernel)
#pragma unroll
        for (int s0 = 0; s0 < 4; s0 += 2) {
            v4i c[2][TTW][RTW];
            float dsc[2][RTW];
#pragma unroll
            for (int ss = 0; ss < 2; ++ss) {
                const int s = s0 + ss;
                long A[TTW], Bq[RTW];
#pragma unroll
                for (int t = 0; t < TTW; ++t) {
                    const u32x4 v = a[cur][t][s >> 1];
                    A[t] = (s & 1) ? gpack2(v.z, v.w) : gpack2(v.x, v.y);
                }
#pragma unroll
                for (int r = 0; r < RTW; ++r) {
                    dsc[ss][r] = dr[r] * ubyte_f(scr[r], s);
                    const u32x4 v = b[cur][r];
                    const uint32_t q = s == 0 ? v.x : s == 1 ? v.y : s == 2 ? v.z : v.w;
                    Bq[r] = gpack2(q & 0x0F0F0F0Fu, (q >> 4) & 0x0F0F0F0Fu);
                }
#pragma unroll
                for (int t = 0; t < TTW; ++t)
#pragma unroll
                    for (int r = 0; r < RTW; ++r) {
                        const v4i z = {0, 0, 0, 0};
                        c[ss][t][r] = __builtin_amdgcn_mfma_i32_16x16x32_i8(A[t], Bq[r], z, 0, 0, 0);
                    }
            }
#pragma unroll
            for (int ss = 0; ss < 2; ++ss) {
                const int s = s0 + ss;
#pragma unroll
                for (int t = 0; t < TTW; ++t) {
                    const int tb = (wt * TTW + t) * 16 + 4 * g;
                    const float4 d4 = *(const float4*)&dx_s[cur][s][tb];
                    const float dxe[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                    for (int r = 0; r < RTW; ++r)
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            acc[t][r][e] = fmaf((float)c[ss][t][r][e], dxe[e] * dsc[ss][r], acc[t][r][e]);
                }
            }
        }
    };
    load(0, 0);
    for (uint32_t C = 0; C < nC; C += 2) {
        step(std::integral_constant<int, 0>{}, C);
        step(std::integral_constant<int, 1>{}, C + 1);  // nC is even
    }
#pragma unroll
    for (int t = 0; t < TTW; ++t)
#pragma unroll
        for (int r = 0; r < RTW; ++r) {
            const uint32_t n = 16 * (rt0 + r) + row;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t m = 16 * (tt0 + t) + 4 * g + e;
                if (m < M && n < N && tt0 + t < n_tt && rt0 + r < n_rt) {
                    float* dst = y + (size_t)m * ldy + n;
                    *dst = accumulate ? *dst + acc[t][r][e] : acc[t][r][e];
                }
            }
        }
}

}  // namespace ec

using namespace ec;

extern "C" size_t ec_gemm_act_bytes(int fmt, uint32_t M, uint32_t K) {
    if (fmt != EC_Q8_0 && fmt != EC_Q4_K) return 0;
    return xt_layout(fmt, M, K).total;
}

extern "C" int ec_gemm_quantize_act(int fmt, const float* x, void* act, uint32_t M, uint32_t K, void* stream) {
    if (M == 0) return EC_OK;
    if (!x || !act || (fmt != EC_Q8_0 && fmt != EC_Q4_K) || K == 0 || K % 32 || (fmt == EC_Q4_K && K % 256))
        return ec_set_error(EC_ERR_ARG, "ec_gemm_quantize_act: bad argument (Q8_0: K % 32 == 0, Q4_K: K % 256 == 0)");
    if ((uintptr_t)x % 16)  // the quantizers read x with 16-byte loads
        return ec_set_error(EC_ERR_ARG, "ec_gemm_quantize_act: x must be 16-byte aligned");
    const XtLayout L = xt_layout(fmt, M, K);
    const uint32_t nbp = L.Kp / 32;
    if (fmt == EC_Q8_0)
        hipLaunchKernelGGL(k_gemm_quantize_x8, dim3((nbp + 8 * kQxSteps - 1) / (8 * kQxSteps), L.Mp / 4), dim3(256), 0,
                           (hipStream_t)stream, x, (uint8_t*)act, M, K, K, L.nch, nbp, L.xd_off);
    else
        hipLaunchKernelGGL(k_gemm_quantize_x4v, dim3((L.nch + 1) / 2, L.Mp / 4), dim3(256), 0, (hipStream_t)stream,
                           x, (uint8_t*)act, M, K, K, L.nch, nbp, L.xd_off, L.dxs_off);
    EC_CHECK_LAUNCH();
    return EC_OK;
}

extern "C" int ec_gemm(int fmt, const void* tiled, const void* act, float* y, uint32_t M, uint32_t N, uint32_t K,
                       uint32_t ldy, int accumulate, void* stream) {
    if (M == 0 || N == 0) return EC_OK;
    if (!tiled || !act || !y || ldy < N || (fmt != EC_Q8_0 && fmt != EC_Q4_K) || K == 0 ||
        (fmt == EC_Q4_K && K % 256) || K % 32)
        return ec_set_error(EC_ERR_ARG, "ec_gemm: bad argument");
    const XtLayout L = xt_layout(fmt, M, K);
    const uint32_t n_tt = L.Mp / 16, n_rt = round_up(N, 16) / 16, nbp = L.Kp / 32;
    const uint32_t gy = (n_tt + 3) / 4;
    hipStream_t st = (hipStream_t)stream;
    // 64 tokens x 64 rows per workgroup (RTW = 2): with the epilogue as the
    // bottleneck, two waves per SIMD (<= 256 registers) beat larger register
    // tiles.  Q4_K takes RTW = 1 (64 x 32, three waves per SIMD) where RTW = 2
    // leaves fewer than 1024 workgroups (M = 512, 2560 x 9216: 116.7 -> 104.2
    // us; Q8_0 there 81.9 -> 84.5, so Q8_0 keeps RTW = 2).  EC_GEMM_RTW = 1 or
    // 2 forces one, for comparison.
    static const int rtw_env = [] {
        const char* v = getenv("EC_GEMM_RTW");
        return v ? atoi(v) : 0;
    }();
    const int rtw = rtw_env == 1 || rtw_env == 2       ? rtw_env
                    : fmt == EC_Q4_K && (n_rt + 3) / 4 * gy < 1024 ? 1
                                                                    : 2;
    const dim3 blk(256);
    if (fmt == EC_Q8_0) {
        if (rtw == 1)
            hipLaunchKernelGGL(k_gemm_q8_0<1>, dim3((n_rt + 1) / 2, gy), blk, 0, st, (const uint8_t*)tiled,
                               (const uint8_t*)act, y, M, N, n_tt, n_rt, L.nch, nbp, L.xd_off, ldy, accumulate);
        else
            hipLaunchKernelGGL(k_gemm_q8_0<2>, dim3((n_rt + 3) / 4, gy), blk, 0, st, (const uint8_t*)tiled,
                               (const uint8_t*)act, y, M, N, n_tt, n_rt, L.nch, nbp, L.xd_off, ldy, accumulate);
    } else {
        if (rtw == 1)
            hipLaunchKernelGGL(k_gemm_q4_K<1>, dim3((n_rt + 1) / 2, gy), blk, 0, st, (const uint8_t*)tiled,
                               (const uint8_t*)act, y, M, N, n_tt, n_rt, L.nch, nbp, L.xd_off, L.dxs_off, ldy,
                               accumulate);
        else
            hipLaunchKernelGGL(k_gemm_q4_K<2>, dim3((n_rt + 3) / 4, gy), blk, 0, st, (const uint8_t*)tiled,
                               (const uint8_t*)act, y, M, N, n_tt, n_rt, L.nch, nbp, L.xd_off, L.dxs_off, ldy,
                               accumulate);
    }
    EC_CHECK_LAUNCH();
    return EC_OK;
}
