// Drives include/inference.h (the reference's InferenceEngine interface) on a
// GGUF file: feeds the prompt token by token ("loop") or in one call ("once"),
// writes the final logits to a file and checks the error paths.
#include <cstdio>
#include <cstdlib>
#include <stdexcept>
#include <vector>

#include "gguf_reader.h"
#include "inference.h"

int main(int argc, char** argv) {
    if (argc < 5) return 2;
    const std::string path = argv[1], mode = argv[2], out = argv[3];
    std::vector<uint32_t> toks;
    for (int i = 4; i < argc; ++i) toks.push_back((uint32_t)std::atoi(argv[i]));
    try {
        GGUFReader r(path);
        ModelConfig c = r.config();
        c.max_seq_len = 64;
        InferenceEngine e(c);
        try {
            e.load_weights(nullptr);
            std::printf("load_weights did not throw\n");
            return 1;
        } catch (const std::runtime_error&) {
        }
        e.load_weights_from_gguf(r, path);
        std::vector<float> logits(c.vocab_size);
        const uint32_t n = (uint32_t)toks.size();
        if (mode == "loop") {
            for (uint32_t i = 1; i <= n; ++i) e.forward(toks.data(), i, logits.data());
        } else {
            e.forward(toks.data(), n, logits.data());
        }
        try {
            e.forward(toks.data(), n, logits.data());
            std::printf("re-feed did not throw\n");
            return 1;
        } catch (const std::runtime_error&) {
        }
        std::printf("seen %u\n", e.tokens_seen());
        FILE* f = std::fopen(out.c_str(), "wb");
        std::fwrite(logits.data(), 4, logits.size(), f);
        std::fclose(f);
        e.reset();
        std::printf("after_reset %u\n", e.tokens_seen());
    } catch (const std::runtime_error& ex) {
        std::printf("error %s\n", ex.what());
        return 1;
    }
    return 0;
}
