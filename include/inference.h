// inference.h — InferenceEngine with the reference's public interface
// (echo-core include/inference.h:81-99), running on the MI355X device engine
// (echo_engine.h): weights, KV cache and recurrent state stay in HBM, the
// caller sees host token ids and host logits as before.
//
// Models: what the device engine runs — RMSNorm, RoPE, gated SwiGLU FFN, GGUF
// Q8_0 matrices, head_dim 256; every block attention (the reference C++
// engine's model, ModelConfig's hybrid fields zero) or the hybrid
// delta-net / attention stack (ModelConfig::ssm_* and full_attention_interval,
// as GGUFReader::config() fills them).  The constructor throws
// std::runtime_error for anything else.
//
// Semantics kept from the reference:
//   - forward(tokens, seq_len, logits) writes the logits of tokens[seq_len-1]
//     given the tokens before it, reading the cache for earlier positions;
//   - reset() forgets the sequence (KV cache and recurrent state zeroed);
//   - errors throw std::runtime_error.
// Differences: forward feeds every token in tokens[n_seen .. seq_len) that the
// engine has not seen since reset() (a one-token-per-call loop, as the
// reference's callers use it, feeds exactly the new token; a whole prompt in one
// call is prefilled in 512-token GEMM chunks), and seq_len <= n_seen throws;
// load_weights() of a host FP16 weight pool is not supported (throws) — load a
// Q8_0 GGUF with load_weights_from_gguf().
#pragma once

#include <cstdint>
#include <string>

#include "config.h"
#include "gguf_reader.h"
#include "types.h"

struct ec_engine;

class InferenceEngine {
public:
    explicit InferenceEngine(const ModelConfig& config);
    ~InferenceEngine();
    InferenceEngine(const InferenceEngine&) = delete;
    InferenceEngine& operator=(const InferenceEngine&) = delete;

    // Reference: copy an FP16 weight pool laid out per WeightLayout.  Not
    // supported by the device engine (throws std::runtime_error).
    void load_weights(const fp16_t* weights);

    // Upload the model's tensors from a GGUF file (reader parsed from model_path).
    void load_weights_from_gguf(const GGUFReader& reader, const std::string& model_path);

    // Logits [vocab_size] of tokens[seq_len - 1] (host memory).
    void forward(const uint32_t* tokens, uint32_t seq_len, float* logits);

    // Forget the sequence: KV cache, conv and recurrent state zeroed.
    void reset();

    const ModelConfig& config() const { return config_; }

    // Extension: tokens fed since reset().
    uint32_t tokens_seen() const { return seen_; }

private:
    ModelConfig config_;
    ec_engine* engine_ = nullptr;
    uint32_t seen_ = 0;
};
