#pragma once
// cdna3/runtime/model_config.hpp — the runtime's model configuration (gfx950 build).
//
// The reference's ModelConfig (cdna3-prims/include/cdna3/runtime/model_loader.hpp:52-61), field
// for field, followed by three fields this build adds (QKV biases present, LayerNorm instead of
// RMSNorm, the norm epsilon); aggregate initialisation of the first eight is unchanged.
namespace cdna3 {
namespace runtime {

struct ModelConfig {
    int n_layers;
    int hidden;       // hidden_size
    int n_heads;      // num_attention_heads
    int n_kv_heads;   // num_key_value_heads
    int head_dim;     // hidden / n_heads
    int ffn_dim;      // intermediate_size
    int vocab_size;
    float rope_theta;
    bool qkv_bias = false;
    bool layernorm = false;
    float norm_eps = 1e-6f;
};

}  // namespace runtime
}  // namespace cdna3
