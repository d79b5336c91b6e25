/*
 * echo_gguf.h — C ABI of the GGUF v3 reader and the GGUF -> device loader of
 * the hybrid decoder (libechohip.so).  No counterpart in the reference's C ABI:
 * it exposes to C / FFI callers what the reference's GGUFReader
 * (src/gguf_reader.cpp:275-433, echo-core-zig/src/gguf/reader.zig:263-328) and
 * its weight loader (echo-core-zig/src/ports/inference.zig:529-567,651-1032)
 * do, and the C++ interface of include/gguf_reader.h is the same reader.
 *
 * Functions return 0 or an EC_ERR_* code with the message in ec_last_error().
 */
#ifndef ECHO_GGUF_H
#define ECHO_GGUF_H
#include <stddef.h>
#include <stdint.h>

#include "echo_engine.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ec_gguf ec_gguf;

typedef struct {
    const char* name;
    uint32_t type;     /* ggml type id (GGMLType) */
    uint32_t n_dims;
    uint64_t shape[4]; /* ne0 (fastest) first; unused dims 1 */
    uint64_t offset;   /* relative to the data section */
    uint64_t bytes;
    const void* data;  /* the file's bytes, mapped read-only; valid until ec_gguf_close */
} ec_gguf_tensor;

/* Map and parse a GGUF v3 file (magic, version 3, metadata, tensor infos;
 * every tensor must lie inside the file). */
int ec_gguf_open(const char* path, ec_gguf** out);
void ec_gguf_close(ec_gguf* g);

uint64_t ec_gguf_tensor_count(const ec_gguf* g);
/* i-th tensor in file order. */
int ec_gguf_tensor_at(const ec_gguf* g, uint64_t i, ec_gguf_tensor* out);
/* Tensor by exact name (EC_ERR_ARG if absent). */
int ec_gguf_find_tensor(const ec_gguf* g, const char* name, ec_gguf_tensor* out);

/* Scalar metadata by full key: unsigned or non-negative signed integers,
 * integers or floats as double, strings (EC_ERR_ARG if absent or of another type). */
int ec_gguf_get_uint(const ec_gguf* g, const char* key, uint64_t* out);
int ec_gguf_get_float(const ec_gguf* g, const char* key, double* out);
int ec_gguf_get_string(const ec_gguf* g, const char* key, const char** out);
/* tokenizer.ggml.tokens */
uint64_t ec_gguf_token_count(const ec_gguf* g);
const char* ec_gguf_token(const ec_gguf* g, uint64_t i);

uint32_t ec_gguf_alignment(const ec_gguf* g);
uint64_t ec_gguf_data_offset(const ec_gguf* g);
/* Architecture key prefix detected from the metadata, e.g. "qwen35." */
const char* ec_gguf_arch_prefix(const ec_gguf* g);

/* Decoder shape from the metadata (<arch>.embedding_length, block_count,
 * feed_forward_length, attention.head_count[_kv], attention.key_length,
 * ssm.inner_size, ssm.time_step_rank, ssm.conv_kernel, full_attention_interval,
 * rope.freq_base) and token_embd.weight (vocab); batch and context sizes
 * are the caller's.  Checks that the file's block types (ssm_out.weight
 * present = delta-net block) follow the attention interval. */
int ec_gguf_engine_config(const ec_gguf* g, uint32_t max_batch, uint32_t max_ctx, ec_engine_cfg* out);

/* Upload every tensor of the decoder from the file (GGUF names of the
 * reference's tensor reports): token_embd, output_norm, output (or tied to
 * token_embd), per block attn_norm, post_attention_norm, ffn_gate/up/down;
 * delta-net blocks attn_qkv | attn_gate | ssm_alpha | ssm_beta (stacked into
 * the input projection), ssm_out, ssm_conv1d (bytes as stored, read tap-major
 * as qwen_linear.zig:193-201 does), ssm_a (as A_log), ssm_dt.bias, ssm_norm;
 * attention blocks attn_q | attn_k | attn_v, attn_output, attn_q_norm and
 * attn_k_norm (absent = not applied).  Matrices must be Q8_0 with the
 * engine's shapes, vectors F32. */
int ec_engine_load_gguf(ec_engine* e, const ec_gguf* g);

#ifdef __cplusplus
}
#endif
#endif
