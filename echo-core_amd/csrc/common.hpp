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

// Sum over the 16 lanes of a DPP row; every lane of the row receives the total.
__device__ __forceinline__ float row16_sum(float v) {
    v += __shfl_xor(v, 1);
    v += __shfl_xor(v, 2);
    v += __shfl_xor(v, 4);
    v += __shfl_xor(v, 8);
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
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

}  // namespace ec

// Launch-error plumbing for the C ABI: every entry point returns an ec_status.
#define EC_CHECK_LAUNCH()                                              \
    do {                                                               \
        hipError_t _e = hipGetLastError();                             \
        if (_e != hipSuccess) return ec_set_hip_error(_e, __func__);   \
    } while (0)

extern "C" int ec_set_hip_error(hipError_t e, const char* where);
extern "C" int ec_set_error(int code, const char* msg);
