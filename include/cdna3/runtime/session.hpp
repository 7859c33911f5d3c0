#pragma once
// cdna3/runtime/session.hpp — greedy batch-1 LLM session (gfx950), host side.
//
// Drop-in for the reference's cdna3::runtime::Session (cdna3-prims/include/cdna3/runtime/
// session.hpp:47-331), GenerateCfg (:42-45) and ModelConfig (model_loader.hpp:52-61), over
// libcdna4_attn.so:
//   cdna3::runtime::Session sess("/tmp/model", /*max_seq*/4096);
//   std::vector<int> seq = sess.generate(input_ids, {/*max_new_tokens*/256});
//   std::vector<float> logits = sess.prefill_logits(input_ids);
// The model directory is the reference exporter's format (meta.json + one fp16 .bin per tensor).
// As in the reference, the constructor throws std::runtime_error when the model cannot be loaded
// and generate returns the prompt followed by the generated tokens. Deviations: invalid token
// ids or a prompt longer than max_seq throw instead of reading or writing out of bounds.
#include <stdexcept>
#include <string>
#include <vector>
#include "../../cdna4_attn.h"
#include "model_config.hpp"

namespace cdna3 {
namespace runtime {

struct GenerateCfg {
    int max_new_tokens = 64;
    int eos_token_id = -1;   // stop once produced; -1 = run to max_new_tokens
};

class Session {
    cdna3_session* s_ = nullptr;
    int max_seq_;

    static void check(int rc, const char* what) {
        if (rc != 0) throw std::runtime_error(std::string(what) + ": " + cdna3_error_string(rc));
    }

public:
    explicit Session(const std::string& model_dir, int max_seq = 4096) : max_seq_(max_seq) {
        check(cdna3_session_create(model_dir.c_str(), max_seq, &s_), "Session");
    }
    ~Session() { cdna3_session_destroy(s_); }
    Session(const Session&) = delete;
    Session& operator=(const Session&) = delete;

    ModelConfig config() const {
        cdna3_model_cfg c;
        check(cdna3_session_config(s_, &c), "Session::config");
        return {c.n_layers, c.hidden, c.n_heads, c.n_kv_heads, c.head_dim, c.ffn_dim, c.vocab_size,
                c.rope_theta, c.qkv_bias != 0, c.layernorm != 0, c.norm_eps};
    }
    int max_seq() const { return max_seq_; }

    // Greedy generate: the prompt followed by the generated tokens (session.hpp:262-296).
    std::vector<int> generate(const std::vector<int>& input_ids, const GenerateCfg& cfg) {
        std::vector<int> out(cfg.max_new_tokens > 0 ? cfg.max_new_tokens : 1);
        int n = 0;
        check(cdna3_session_generate(s_, input_ids.data(), (int)input_ids.size(), cfg.max_new_tokens,
                                     cfg.eos_token_id, out.data(), &n, nullptr, nullptr, nullptr),
              "Session::generate");
        std::vector<int> seq = input_ids;
        seq.insert(seq.end(), out.begin(), out.begin() + n);
        return seq;
    }

    // Prefill only: logits of the last prompt token, fp16 values widened to float (session.hpp:298-317).
    std::vector<float> prefill_logits(const std::vector<int>& input_ids) {
        std::vector<float> logits(config().vocab_size);
        check(cdna3_session_prefill_logits(s_, input_ids.data(), (int)input_ids.size(), logits.data()),
              "Session::prefill_logits");
        return logits;
    }
};

}  // namespace runtime
}  // namespace cdna3
