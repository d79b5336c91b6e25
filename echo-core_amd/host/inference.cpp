// inference.cpp — the reference's InferenceEngine interface (include/inference.h)
// over the device engine: a one-sequence engine (max_batch 1) whose forward()
// feeds new tokens through the chunked prefill or one graph-replayed decode
// step and copies the last token's logits to the host.
#include <stdexcept>
#include <string>
#include <vector>

#include "echo_engine.h"
#include "echo_hip.h"
#include "gguf_reader.h"
#include "inference.h"

void ec_load_gguf_tensors(ec_engine* e, const GGUFReader& r);

namespace {
void check(int rc, const char* what) {
    if (rc != EC_OK) throw std::runtime_error(std::string("InferenceEngine: ") + what + ": " + ec_last_error());
}
}  // namespace

InferenceEngine::InferenceEngine(const ModelConfig& config) : config_(config) {
    const ModelConfig& m = config;
    if (m.ffn_type != ModelConfig::FFNType::GatedSwiGLU || m.norm_type != ModelConfig::NormType::RMSNorm ||
        m.pos_encoding != ModelConfig::PosEncoding::RoPE)
        throw std::runtime_error("InferenceEngine: the device engine runs RMSNorm + RoPE + gated SwiGLU models");
    ec_engine_cfg c{};
    c.vocab = m.vocab_size;
    c.hidden = m.hidden_dim;
    c.ffn = m.ffn_hidden_dim;
    c.n_layers = m.num_layers;
    c.n_heads = m.num_heads;
    c.n_kv = m.num_kv_heads ? m.num_kv_heads : m.num_heads;
    c.head_dim = m.head_dim;
    c.ssm_inner = m.ssm_inner_size;
    c.ssm_heads = m.ssm_num_heads;
    c.conv_kernel = m.ssm_conv_kernel ? m.ssm_conv_kernel : 4;
    c.attn_interval = m.ssm_inner_size ? m.full_attention_interval : 1;
    c.max_batch = 1;
    c.max_ctx = m.max_seq_len;
    c.rope_base = m.rope_base > 0.0f ? m.rope_base : 10000.0f;
    check(ec_engine_create(&c, &engine_), "create");
    check(ec_engine_reset(engine_), "reset");
}

InferenceEngine::~InferenceEngine() { ec_engine_destroy(engine_); }

void InferenceEngine::load_weights(const fp16_t*) {
    throw std::runtime_error(
        "InferenceEngine::load_weights: FP16 weight pools are not supported by the device engine "
        "(load a Q8_0 GGUF with load_weights_from_gguf)");
}

void InferenceEngine::load_weights_from_gguf(const GGUFReader& reader, const std::string&) {
    ec_load_gguf_tensors(engine_, reader);
    reset();
}

void InferenceEngine::forward(const uint32_t* tokens, uint32_t seq_len, float* logits) {
    if (!tokens || !logits || seq_len == 0) throw std::runtime_error("InferenceEngine::forward: bad argument");
    if (seq_len <= seen_)
        throw std::runtime_error("InferenceEngine::forward: tokens[seq_len-1] was already fed (call reset() first)");
    if (seq_len > config_.max_seq_len) throw std::runtime_error("InferenceEngine::forward: past max_seq_len");
    const uint32_t n = seq_len - seen_;
    std::vector<int32_t> t(tokens + seen_, tokens + seq_len);
    if (n == 1) {
        const int32_t pos = (int32_t)seen_;
        check(ec_engine_set_inputs(engine_, t.data(), &pos, 1), "set_inputs");
        check(ec_engine_step(engine_, 1), "step");
    } else {
        check(ec_engine_prefill(engine_, 0, t.data(), n, (int32_t)seen_), "prefill");
    }
    seen_ = seq_len;
    check(ec_engine_get_logits(engine_, logits, 0), "logits");
}

void InferenceEngine::reset() {
    check(ec_engine_reset(engine_), "reset");
    seen_ = 0;
}
