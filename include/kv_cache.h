/* kv_cache.h — the reference's per-layer KV cache, resident in HBM.
 *
 * Same class and struct layout as the echo-core interface
 * include/kv_cache.h:7-49.  Storage is one device allocation; the pointers in
 * KVCacheLayer are device pointers (pass them to ec_attn_decode).  Appends
 * quantize one (token, kv_head) row of head_dim values per scale, the layout
 * the reference's readers index (src/inference.cpp:347,387): key_scales /
 * val_scales are [max_seq_len][num_kv_heads].  (The reference's writer,
 * src/kv_cache.cpp:101,105, scales the whole kv_dim row with one value at
 * [pos]; that disagrees with its own readers and is not reproduced.)
 * k_proj / v_proj may be host or device memory.  Overflow (seq_len ==
 * max_seq_len) records an error (ec_last_error) and appends nothing, where
 * the reference asserts.  reset() rewinds seq_len and keeps the data, as the
 * reference does (src/kv_cache.cpp:120-124). */
#pragma once

#include "config.h"
#include "kernels/quant.h"
#include "types.h"

struct alignas(64) KVCacheLayer {
    int8_t* keys_int8;    /* [max_seq_len * num_kv_heads * head_dim] */
    int8_t* values_int8;  /* [max_seq_len * num_kv_heads * head_dim] */
    float* key_scales;    /* [max_seq_len * num_kv_heads] */
    float* val_scales;    /* [max_seq_len * num_kv_heads] */
    float* keys_fp32;     /* fp32 mode (use_kv_quantization = false) */
    float* values_fp32;
    uint32_t seq_len;
};

class KVCache {
    ModelConfig config_;
    KVCacheLayer* layers_;
    uint8_t* storage_;

public:
    explicit KVCache(const ModelConfig& config);
    ~KVCache();

    KVCacheLayer& layer(uint32_t layer_idx);
    const KVCacheLayer& layer(uint32_t layer_idx) const;

    /* k_proj, v_proj: one token, [num_kv_heads * head_dim] fp32. */
    void append(uint32_t layer_idx, const float* k_proj, const float* v_proj);

    /* Layer 0's length (reference src/kv_cache.cpp:115-118). */
    uint32_t seq_len() const;

    void reset();

    KVCache(const KVCache&) = delete;
    KVCache& operator=(const KVCache&) = delete;
};
