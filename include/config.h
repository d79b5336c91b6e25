/* config.h — model configuration of the reference-signature interface.
 *
 * Same fields, order and enum values as the echo-core interface
 * include/config.h:6-26, followed by the hybrid-model fields the device
 * engine needs (defaulting to zero; code compiled against this header passes
 * it by reference across the library boundary).  The cache-tile helpers of the reference
 * (include/config.h:28-60) tune a CPU L3 tiling; they are kept so that code
 * naming them compiles, and have no effect on the GPU kernels. */
#pragma once

#include <cstddef>
#include <cstdint>

struct ModelConfig {
    uint32_t vocab_size;
    uint32_t hidden_dim;
    uint32_t num_heads;
    uint32_t num_kv_heads;
    uint32_t head_dim;
    uint32_t num_layers;
    uint32_t ffn_hidden_dim;
    uint32_t max_seq_len;

    enum class FFNType { Dense, GatedSwiGLU, GatedGeLU };
    FFNType ffn_type;

    enum class NormType { LayerNorm, RMSNorm };
    NormType norm_type;

    enum class PosEncoding { RoPE, Learned, ALiBi, None };
    PosEncoding pos_encoding;

    bool use_kv_quantization;

    // Appended for hybrid delta-net / attention models (echo-core-zig
    // src/core/config.zig:19-23); the fields above keep the reference's order.
    // All zero = every block is attention (the reference C++ engine's model).
    uint32_t ssm_inner_size = 0;           // delta-net value dim (ssm.inner_size)
    uint32_t ssm_num_heads = 0;            // delta-net value heads (ssm.time_step_rank)
    uint32_t ssm_conv_kernel = 0;          // causal conv taps (ssm.conv_kernel); 0 = 4
    uint32_t full_attention_interval = 0;  // block i is attention iff (i+1) % interval == 0
    float rope_base = 0.0f;                // RoPE base (rope.freq_base); 0 = 10000
};

template <uint64_t L3_SIZE_BYTES>
struct CacheTileConfig {
    static constexpr uint64_t L3_BUDGET = L3_SIZE_BYTES * 6 / 10;
    static constexpr uint32_t TILE_K = (L3_BUDGET >= 18ULL * 1024 * 1024) ? 2048 : 1024;
    static constexpr uint32_t TILE_M = (L3_BUDGET >= 18ULL * 1024 * 1024) ? 1024 : 512;
    static constexpr uint64_t TILE_FOOTPRINT = 2ULL * TILE_M * TILE_K + 4ULL * TILE_K + 4ULL * TILE_M;
};

using Intel13500H_Tiles = CacheTileConfig<18ULL * 1024 * 1024>;
using AMD_Ryzen3600_Tiles = CacheTileConfig<32ULL * 1024 * 1024>;
