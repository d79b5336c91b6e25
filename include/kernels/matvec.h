/* kernels/matvec.h — reference-signature matrix-vector products on MI355X.
 *
 * Same declarations as the echo-core interface include/kernels/matvec.h:1-26.
 * Every product accumulates, y[m] += W[m,:] . x, with W row-major (M rows of K
 * weights) and fp32 x, y; the caller zeroes y first.  A K that is not a
 * multiple of the block size drops the remainder, as the reference does
 * (src/kernels/matvec.cpp:65,95).  Pointers may be device, managed, pinned or
 * host memory (host buffers are staged); each call completes before it
 * returns and reports failures through ec_last_error() (echo_hip.h).
 * These run the fp32-activation kernels (no activation quantization), so
 * they agree with the reference to fp32 rounding. */
#pragma once

#include "config.h"
#include "types.h"

/* fp16 weights.  TILE_K / TILE_M tune the reference's CPU L3 tiling and do
 * not change the GPU kernel; <1024,512> and <2048,1024> are instantiated,
 * as in the reference (src/kernels/matvec.cpp:48-49). */
template <uint32_t TILE_K, uint32_t TILE_M>
void matvec_fp16_fp32(const fp16_t* W, const float* x, float* y, uint32_t M, uint32_t K);

void matvec_dispatch(const fp16_t* W, const float* x, float* y, uint32_t M, uint32_t K, const ModelConfig& config);

/* GGUF block formats read in place (34-byte Q8_0, 144-byte Q4_K, 84-byte Q2_K blocks). */
void matvec_q8_0(const void* blocks, const float* x, float* y, uint32_t M, uint32_t K);
void matvec_q4_K(const void* blocks, const float* x, float* y, uint32_t M, uint32_t K);
void matvec_q2_K(const void* blocks, const float* x, float* y, uint32_t M, uint32_t K);
