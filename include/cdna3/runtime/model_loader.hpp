#pragma once
// cdna3/runtime/model_loader.hpp — weight loader of the runtime (gfx950 build).
//
// Same types and members as the reference's loader (cdna3-prims/include/cdna3/runtime/
// model_loader.hpp:51-193): ModelLoader(model_dir), load(), weights() returning ModelWeights with
// one LayerWeights of device pointers per layer (fp16, row-major [out][in], the exporter's layout;
// q/k/v biases null unless meta.json sets qkv_bias). The directory format is the reference
// exporter's (meta.json + one raw fp16 .bin per tensor). The loading is done by libcdna4_attn.so
// (cdna3_model_load, C ABI); the buffers live until the loader is destroyed. As in the reference,
// load() throws std::runtime_error when a file cannot be read.
#include <hip/hip_fp16.h>
#include <stdio.h>
#include <stdexcept>
#include <string>
#include <vector>
#include "../../cdna4_attn.h"
#include "model_config.hpp"

namespace cdna3 {
namespace runtime {

struct LayerWeights {
    __half* Wq = nullptr;   // [n_heads*head_dim x hidden]
    __half* Wk = nullptr;   // [n_kv_heads*head_dim x hidden]
    __half* Wv = nullptr;
    __half* Wo = nullptr;   // [hidden x n_heads*head_dim]
    __half* bq = nullptr;   // null without qkv_bias
    __half* bk = nullptr;
    __half* bv = nullptr;
    __half* Wgate = nullptr;   // [ffn_dim x hidden]
    __half* Wup = nullptr;
    __half* Wdown = nullptr;   // [hidden x ffn_dim]
    __half* norm_attn = nullptr;   // [hidden]
    __half* norm_mlp = nullptr;
};

struct ModelWeights {
    ModelConfig cfg{};
    std::vector<LayerWeights> layers;
    __half* embed_tokens = nullptr;   // [vocab_size x hidden]
    __half* lm_head = nullptr;
    __half* final_norm = nullptr;     // [hidden]
};

class ModelLoader {
    std::string dir_;
    ModelWeights w_;
    cdna3_model* m_ = nullptr;

public:
    explicit ModelLoader(const std::string& model_dir) : dir_(model_dir) {}
    ~ModelLoader() { cdna3_model_free(m_); }
    ModelLoader(const ModelLoader&) = delete;
    ModelLoader& operator=(const ModelLoader&) = delete;

    const ModelWeights& weights() const { return w_; }

    void load() {
        cdna3_model_free(m_);
        m_ = nullptr;
        int rc = cdna3_model_load(dir_.c_str(), &m_);
        if (rc != 0) throw std::runtime_error("cannot load model from " + dir_ + ": " + cdna3_error_string(rc));
        cdna3_model_cfg c;
        cdna3_model_weights v;
        rc = cdna3_model_config(m_, &c);
        if (rc == 0) rc = cdna3_model_weights_get(m_, &v);
        if (rc != 0) throw std::runtime_error(std::string("ModelLoader: ") + cdna3_error_string(rc));
        w_.cfg = ModelConfig{c.n_layers, c.hidden, c.n_heads, c.n_kv_heads, c.head_dim, c.ffn_dim, c.vocab_size,
                             c.rope_theta, c.qkv_bias != 0, c.layernorm != 0, c.norm_eps};
        auto h = [](void* p) { return (__half*)p; };
        w_.embed_tokens = h(v.embed_tokens);
        w_.lm_head = h(v.lm_head);
        w_.final_norm = h(v.final_norm);
        w_.layers.assign(v.n_layers, LayerWeights{});
        for (int i = 0; i < v.n_layers; ++i) {
            const cdna3_layer_weights& s = v.layers[i];
            LayerWeights& d = w_.layers[i];
            d.Wq = h(s.Wq); d.Wk = h(s.Wk); d.Wv = h(s.Wv); d.Wo = h(s.Wo);
            d.bq = h(s.bq); d.bk = h(s.bk); d.bv = h(s.bv);
            d.Wgate = h(s.Wgate); d.Wup = h(s.Wup); d.Wdown = h(s.Wdown);
            d.norm_attn = h(s.norm_attn); d.norm_mlp = h(s.norm_mlp);
        }
        printf("ModelLoader: loaded %d layers, hidden=%d, heads=%d/%d (GQA), ffn=%d\n", c.n_layers, c.hidden,
               c.n_heads, c.n_kv_heads, c.ffn_dim);
    }
};

}  // namespace runtime
}  // namespace cdna3
