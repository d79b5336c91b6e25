// Drives include/gguf_reader.h (the reference's GGUFReader interface) on one
// file and prints what a caller would read, one "key value" per line.
#include <cstdio>
#include <string>
#include <variant>

#include "gguf_reader.h"

int main(int argc, char** argv) {
    if (argc < 2) return 2;
    try {
        GGUFReader r(argv[1]);
        const ModelConfig& c = r.config();
        std::printf("alignment %d\n", r.alignment());
        std::printf("data_offset %lld\n", (long long)r.data_offset());
        std::printf("max_seq_len %u\nhidden_dim %u\nnum_layers %u\nffn_hidden_dim %u\n", c.max_seq_len, c.hidden_dim,
                    c.num_layers, c.ffn_hidden_dim);
        std::printf("num_heads %u\nnum_kv_heads %u\nhead_dim %u\nvocab_size %u\n", c.num_heads, c.num_kv_heads,
                    c.head_dim, c.vocab_size);
        std::printf("gated_swiglu %d\n", c.ffn_type == ModelConfig::FFNType::GatedSwiGLU ? 1 : 0);
        for (size_t i = 0; i < r.tokens().size(); ++i) std::printf("token %zu %s\n", i, r.tokens()[i].c_str());
        auto sc = r.metadata().find("tokenizer.ggml.scores");
        if (sc != r.metadata().end())
            if (auto p = std::get_if<std::vector<double>>(&sc->second))
                for (double v : *p) std::printf("score %.6f\n", v);
        for (const auto& kv : r.tensors()) {
            const TensorInfo& t = kv.second;
            std::vector<uint8_t> d = r.load_tensor(kv.first);
            std::printf("tensor %s type %u size %llu offset %llu first %u last %u\n", kv.first.c_str(),
                        (unsigned)t.dtype, (unsigned long long)t.size, (unsigned long long)t.offset,
                        d.empty() ? 0u : d.front(), d.empty() ? 0u : d.back());
        }
        if (argc > 2) {
            const TensorInfo* s = r.find_tensor_by_suffix(argv[2]);
            std::printf("suffix %s %s\n", argv[2], s ? "found" : "missing");
        }
        try {
            r.assert_alignment(r.alignment());
            std::printf("aligned 1\n");
        } catch (const std::runtime_error&) {
            std::printf("aligned 0\n");
        }
    } catch (const std::runtime_error& ex) {
        std::printf("error %s\n", ex.what());
        return 1;
    }
    return 0;
}
