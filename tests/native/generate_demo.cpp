// The reference's runtime usage (cdna3-prims/include/cdna3/runtime/session.hpp:29-31, and its
// bench_generate / validate_runtime callers) written against include/cdna3/runtime/session.hpp:
// load a model directory, greedy-generate, print the sequence. Host-only C++ (plain clang++),
// linked against libcdna4_attn.so.
//   generate_demo <model_dir> <max_seq> <max_new_tokens> <id> [<id> ...]
// prints "tokens: t0 t1 ..." (prompt followed by the generated tokens) and
// "logits0: <first 4 prefill logits>"; exit status 1 on an error.
#include <cdna3/runtime/session.hpp>
#include <cstdio>
#include <cstdlib>
#include <exception>
#include <vector>

int main(int argc, char** argv) {
    if (argc < 5) {
        std::fprintf(stderr, "usage: %s model_dir max_seq max_new_tokens id...\n", argv[0]);
        return 2;
    }
    try {
        cdna3::runtime::Session sess(argv[1], std::atoi(argv[2]));
        std::vector<int> ids;
        for (int i = 4; i < argc; ++i) ids.push_back(std::atoi(argv[i]));
        cdna3::runtime::GenerateCfg cfg;
        cfg.max_new_tokens = std::atoi(argv[3]);
        const std::vector<int> seq = sess.generate(ids, cfg);
        std::printf("tokens:");
        for (int t : seq) std::printf(" %d", t);
        std::printf("\n");
        const std::vector<float> lg = sess.prefill_logits(ids);
        std::printf("logits0: %.6f %.6f %.6f %.6f\n", lg[0], lg[1], lg[2], lg[3]);
        const cdna3::runtime::ModelConfig c = sess.config();
        std::printf("config: layers %d hidden %d heads %d/%d vocab %d\n", c.n_layers, c.hidden, c.n_heads,
                    c.n_kv_heads, c.vocab_size);
        try {   // invalid ids throw, as documented
            sess.generate({c.vocab_size}, cfg);
            std::printf("invalid id: no error\n");
            return 1;
        } catch (const std::runtime_error&) {
            std::printf("invalid id: rejected\n");
        }
    } catch (const std::exception& e) {
        std::fprintf(stderr, "error: %s\n", e.what());
        return 1;
    }
    return 0;
}
