// common.hpp — device helpers shared by the echo-hip kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <cstdint>
#include <cstddef>
#include <cstdlib>
#include <cstdio>

#include "echo_hip.h"

namespace ec {

constexpr int kWave = 64;

// Exact binary16 -> binary32 (v_cvt_f32_f16 is exact for every half).
__device__ __forceinline__ float h2f(uint16_t h) {
    return __half2float(__ushort_as_half(h));
}

// Value of lane i ^ O.  Inside a 16-lane row (O < 16) this is DPP on the
// VALU (a few cycles); across rows it is ds_bpermute (an LDS round trip).
//   O = 1, 2: quad_perm [1,0,3,2] / [2,3,0,1]
//   O = 4:    row_shl:4 into banks 0 and 2 (lane i reads i+4), row_shr:4 into
//             banks 1 and 3 (lane i reads i-4)
//   O = 8:    row_ror:8 (i+8 mod 16 == i^8)
template <int CTRL, int BANKS>
__device__ __forceinline__ int dpp_i(int old, int v) {
    return __builtin_amdgcn_update_dpp(old, v, CTRL, 0xF, BANKS, false);
}
template <int O>
__device__ __forceinline__ int lane_xor_i(int v) {
    static_assert(O == 1 || O == 2 || O == 4 || O == 8 || O == 16 || O == 32, "xor of 1 .. 32");
    if constexpr (O == 1) return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, true);
    else if constexpr (O == 2) return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, true);
    else if constexpr (O == 4) return dpp_i<0x114, 0xA>(dpp_i<0x104, 0x5>(v, v), v);
    else if constexpr (O == 8) return __builtin_amdgcn_mov_dpp(v, 0x128, 0xF, 0xF, true);
    else return __shfl_xor(v, O);
}
template <int O>
__device__ __forceinline__ float lane_xor(float v) {
    return __int_as_float(lane_xor_i<O>(__float_as_int(v)));
}
// Value of lane i + N of the same 16-lane row (DPP row_shl:N, N = 1 .. 15);
// a lane whose source lies past the row's end reads 0.
template <int N>
__device__ __forceinline__ uint32_t row_down(uint32_t v) {
    static_assert(N >= 1 && N <= 15, "shift inside a row");
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x100 + N, 0xF, 0xF, true);
}

// Sum over the 16 lanes of a DPP row; every lane of the row receives the total
// (butterfly xor 1, 2, 4, 8: each level adds the same two partial sums in
// every lane, so all lanes hold the identical total).
__device__ __forceinline__ float row16_sum(float v) {
    v += lane_xor<1>(v);
    v += lane_xor<2>(v);
    v += lane_xor<4>(v);
    v += lane_xor<8>(v);
    return v;
}

// x*x rounded on its own, never contracted into a following add: summed by a
// butterfly reduction, a contracted square would make the first level an FMA
// in one lane of each pair and a separately rounded sum in the other, so the
// lanes' totals could differ in the last bit.
__device__ __forceinline__ float sq_rn(float x) {
#pragma clang fp contract(off)
    return x * x;
}

// Butterfly over the wave, xor 32 first (the same association in every lane).
__device__ __forceinline__ float wave_sum(float v) {
    v += lane_xor<32>(v);
    v += lane_xor<16>(v);
    v += lane_xor<8>(v);
    v += lane_xor<4>(v);
    v += lane_xor<2>(v);
    v += lane_xor<1>(v);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, lane_xor<32>(v));
    v = fmaxf(v, lane_xor<16>(v));
    v = fmaxf(v, lane_xor<8>(v));
    v = fmaxf(v, lane_xor<4>(v));
    v = fmaxf(v, lane_xor<2>(v));
    v = fmaxf(v, lane_xor<1>(v));
    return v;
}

// The reference quantizer's rounding (src/kernels/quant.cpp:70-96): elements of
// whole 8-chunks use rne(x * (1/scale)) with int8 saturation; tail elements use
// round-half-away(x / scale) clamped to [-127, 127].  Divisions are IEEE.
__device__ __forceinline__ float q_scale(float amax) {
    return amax > 0.0f ? __fdiv_rn(amax, 127.0f) : 1.0f;
}
__device__ __forceinline__ int8_t q_body(float x, float inv) {
    int v = (int)rintf(__fmul_rn(x, inv));
    v = v > 127 ? 127 : (v < -128 ? -128 : v);
    return (int8_t)v;
}
__device__ __forceinline__ int8_t q_tail(float x, float scale) {
    int v = (int)roundf(__fdiv_rn(x, scale));
    v = v > 127 ? 127 : (v < -127 ? -127 : v);
    return (int8_t)v;
}

// Second int8 piece of a two-piece activation: with q0 = q_body(x, inv) at
// scale s (inv = 1/s), the residual r = fma(-q0, s, x) in steps of s/256,
// q1 = sat8(rne(r * (inv*256))).  x ~ s*q0 + (s/256)*q1 with |error| <= s/512
// unless q0 saturated.
__device__ __forceinline__ int8_t q_piece1(float x, int8_t q0, float scale, float inv) {
    const float r = fmaf(-(float)q0, scale, x);
    int v = (int)rintf(__fmul_rn(r, inv * 256.0f));
    v = v > 127 ? 127 : (v < -128 ? -128 : v);
    return (int8_t)v;
}

__device__ __forceinline__ float silu(float x) { return x / (1.0f + __expf(-x)); }

// RoPE of element d paired with its neighbour d^1 (value `other`) at angle
// ang: even d -> x cos - other sin, odd d -> other sin + x cos.  Products and
// the sum are rounded separately (never contracted into an FMA), so every
// kernel that rotates rounds the same way.
__device__ __forceinline__ float rope_rot(float x, float other, uint32_t d, float sn, float cs) {
#pragma clang fp contract(off)
    return (d & 1) ? other * sn + x * cs : x * cs - other * sn;
}
__device__ __forceinline__ float rope_pair(float x, float other, uint32_t d, float ang) {
    float sn, cs;
    sincosf(ang, &sn, &cs);
    return rope_rot(x, other, d, sn, cs);
}

// Causal depthwise conv of channel c at position p over a ring state
// [kern][conv_dim] (slot q % kern = input of position q, zeros before 0):
//   sum_k x_{p-k} * w[(kern-1-k)*conv_dim + c], x_p = xin, newest tap first.
__device__ __forceinline__ float conv_ring(const float* __restrict__ st, const float* __restrict__ w, float xin,
                                           uint32_t p, uint32_t kern, uint32_t conv_dim, uint32_t c) {
    // newest tap first, each further tap one fma: the order every conv kernel
    // (decode step, prefill chunk) uses, so their sums agree bit for bit
    float acc = __fmul_rn(xin, w[(size_t)(kern - 1) * conv_dim + c]);
    if (kern <= 4) {
        // all taps loaded before the first use (one memory round trip); a tap
        // k >= kern reads slot 0 / tap 0 and is multiplied by zero
        float sv[3], wv[3];
#pragma unroll
        for (uint32_t k = 1; k < 4; ++k) {
            const bool ok = k < kern;
            sv[k - 1] = st[(size_t)(ok ? (p + kern - k) % kern : 0) * conv_dim + c];
            const float wk = w[(size_t)(ok ? kern - 1 - k : 0) * conv_dim + c];
            wv[k - 1] = ok ? wk : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < 3; ++k) acc = fmaf(sv[k], wv[k], acc);
        return acc;
    }
    for (uint32_t k = 1; k < kern; ++k)
        acc = fmaf(st[(size_t)((p + kern - k) % kern) * conv_dim + c], w[(size_t)(kern - 1 - k) * conv_dim + c], acc);
    return acc;
}

// Four lanes' bytes (this lane's and the next three of its row) in one dword.
__device__ __forceinline__ uint32_t pack4_lanes(uint32_t b) {
    return b | (row_down<1>(b) << 8) | (row_down<2>(b) << 16) | (row_down<3>(b) << 24);
}

// Lanes 32m .. 32m+31 of a wave hold the 32 values of one Q8_0 block of
// activation row i (block sb = k/32, lane % 32 == k % 32): quantize it with the
// reference quantizer's body rule and store it in the Q8_0 activation layout
// (quant.hip: element e of block sb = 4G + j of layout row r at byte
// ((G*4 + e/8)*R + r)*32 + 8j + e%8, scale at xd[i][sb], nbp = blocks per
// row).  P = 2 pieces: M tokens occupy R = 2M layout rows, token i's piece p
// in row 2i + p (q_piece1 for p = 1); P = 1: R = M, row i.  Four lanes pack
// their bytes into one dword store.
__device__ __forceinline__ void store_act_q8_lane(float v, uint8_t* __restrict__ act, float* __restrict__ xd,
                                                  uint32_t M, uint32_t nbp, uint32_t i, uint32_t k, uint32_t P = 1) {
    float amax = fabsf(v);
    amax = fmaxf(amax, lane_xor<1>(amax));
    amax = fmaxf(amax, lane_xor<2>(amax));
    amax = fmaxf(amax, lane_xor<4>(amax));
    amax = fmaxf(amax, lane_xor<8>(amax));
    amax = fmaxf(amax, lane_xor<16>(amax));
    const float scale = q_scale(amax);
    const float inv = __fdiv_rn(1.0f, scale);
    const int8_t q0 = q_body(v, inv);
    const uint32_t w = pack4_lanes((uint8_t)q0);
    const uint32_t sb = k / 32, e = k % 32, G = sb / 4, j = sb % 4;
    uint8_t* dst = act + (((size_t)G * 4 + e / 8) * (P * M) + P * i) * 32 + 8 * j + (e % 8);
    if ((e & 3) == 0) *(uint32_t*)dst = w;
    if (P == 2) {
        const uint32_t w1 = pack4_lanes((uint8_t)q_piece1(v, q0, scale, inv));
        if ((e & 3) == 0) *(uint32_t*)(dst + 32) = w1;
    }
    if (e == 0) xd[(size_t)i * nbp + sb] = scale;
}

}  // namespace ec

// Launch-error plumbing for the C ABI: every entry point returns an ec_status.
#define EC_CHECK_LAUNCH()                                              \
    do {                                                               \
        hipError_t _e = hipGetLastError();                             \
        if (_e != hipSuccess) return ec_set_hip_error(_e, __func__);   \
    } while (0)

extern "C" int ec_set_hip_error(hipError_t e, const char* where);
extern "C" int ec_set_error(int code, const char* msg);
