/* kernels/quant.h — reference-signature quantization entry points on MI355X.
 *
 * Same declarations as the echo-core interface include/kernels/quant.h:8-69;
 * implemented in libechohip.so (echo-core_amd/host/legacy.cpp) on the GPU.
 * Pointer arguments may be device, managed, pinned or ordinary host memory
 * (host buffers are staged through the device); every call completes before
 * it returns.  Nothing throws: a failure leaves outputs untouched and is
 * reported by ec_last_error() (echo_hip.h). */
#pragma once

#include <cstddef>
#include <cstdint>

/* Per-row symmetric int8 quantization (reference src/kernels/quant.cpp:18-98):
 * scale = max|row|/127 (1 for an all-zero row); elements of whole 8-element
 * chunks round half to even with saturation, tail elements round half away
 * from zero and clamp to +-127. */
void quantize_per_token_symmetric(const float* input, int8_t* output, float* scales, uint32_t num_tokens,
                                  uint32_t num_elements);

/* scores[p] = sum_k query[k] * key_cache[p*dim + k] * scales[p]
 * (reference src/kernels/quant.cpp:100-144). */
void fused_dequant_dot_int8(const float* query, const int8_t* key_cache, const float* scales, float* scores,
                            uint32_t dim, uint32_t seq_len);

/* GGUF Q8_0 block: fp16 scale d (little endian) + 32 int8 weights, 34 bytes. */
struct block_q8_0 {
    uint16_t d;
    int8_t qs[32];
};

/* dot(query, dequant(blocks)) over n_blocks*32 weights (reference quant.cpp:150-194). */
float fused_dequant_dot_q8_0(const block_q8_0* blocks, uint32_t n_blocks, const float* query_fp32);

/* GGUF Q4_K super-block, 256 weights in 144 bytes: fp16 d, fp16 dmin, 12 bytes
 * of packed 6-bit (scale, min) pairs, 128 bytes of nibbles (the reference's
 * nibble-to-position mapping, quant.cpp:202-207). */
struct block_q4_K {
    uint16_t d;
    uint16_t dmin;
    uint8_t scales[12];
    uint8_t qs[128];
};

/* dot(query, dequant(blocks)) over n_blocks*256 weights (reference quant.cpp:210-304). */
float fused_dequant_dot_q4_K(const block_q4_K* blocks, uint32_t n_blocks, const float* query_fp32);

/* GGUF blocks -> fp16 weights, n_weights a multiple of the block size
 * (reference quant.cpp:308-396). */
void dequantize_q8_0_to_fp16(const void* src, uint16_t* dst, size_t n_weights);
void dequantize_q4_K_to_fp16(const void* src, uint16_t* dst, size_t n_weights);
void dequantize_q2_K_to_fp16(const void* src, uint16_t* dst, size_t n_weights);
