// Test-only caller of the runtime's C++ types, written as the reference's runtime code uses them
// (cdna3-prims/include/cdna3/runtime/model_loader.hpp:130-193, kv_cache.hpp:19-52, session.hpp:
// 254-260): load a model with ModelLoader, print a checksum of every tensor as read back from the
// device, allocate a KVCache for it and check its layout. Host-only C++ (plain clang++).
// Usage: runtime_types <model_dir> <max_seq>
#include <cdna3/runtime/forward.hpp>
#include <cdna3/runtime/kv_cache.hpp>
#include <cdna3/runtime/model_loader.hpp>
#include <cdna3/runtime/session.hpp>
#include <hip/hip_runtime_api.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string>
#include <vector>

static unsigned long long checksum(const __half* d, size_t n) {
    if (!d) return 0;
    std::vector<uint16_t> h(n);
    if (hipMemcpy(h.data(), d, n * 2, hipMemcpyDeviceToHost) != hipSuccess) exit(3);
    unsigned long long s = 1469598103934665603ull;   // FNV-1a over the little-endian bytes
    for (uint16_t v : h) {
        s = (s ^ (v & 0xffu)) * 1099511628211ull;
        s = (s ^ (v >> 8)) * 1099511628211ull;
    }
    return s;
}

int main(int argc, char** argv) {
    if (argc < 3) return 2;
    const int max_seq = atoi(argv[2]);
    cdna3::runtime::ModelLoader loader(argv[1]);
    loader.load();
    const cdna3::runtime::ModelWeights& w = loader.weights();
    const cdna3::runtime::ModelConfig& c = w.cfg;
    const size_t H = c.hidden, F = c.ffn_dim, V = c.vocab_size;
    const size_t qd = (size_t)c.n_heads * c.head_dim, kvd = (size_t)c.n_kv_heads * c.head_dim;
    printf("cfg %d %d %d %d %d %d %d %g %d\n", c.n_layers, c.hidden, c.n_heads, c.n_kv_heads, c.head_dim, c.ffn_dim,
           c.vocab_size, c.rope_theta, (int)c.qkv_bias);
    printf("embed_tokens %llu\n", checksum(w.embed_tokens, V * H));
    printf("lm_head %llu\n", checksum(w.lm_head, V * H));
    printf("final_norm %llu\n", checksum(w.final_norm, H));
    for (int i = 0; i < c.n_layers; ++i) {
        const cdna3::runtime::LayerWeights& l = w.layers[i];
        const std::string p = "layer_" + std::to_string(i) + "_";
        printf("%sq_proj %llu\n", p.c_str(), checksum(l.Wq, qd * H));
        printf("%sk_proj %llu\n", p.c_str(), checksum(l.Wk, kvd * H));
        printf("%sv_proj %llu\n", p.c_str(), checksum(l.Wv, kvd * H));
        printf("%so_proj %llu\n", p.c_str(), checksum(l.Wo, H * qd));
        if (c.qkv_bias) {
            printf("%sq_bias %llu\n", p.c_str(), checksum(l.bq, qd));
            printf("%sk_bias %llu\n", p.c_str(), checksum(l.bk, kvd));
            printf("%sv_bias %llu\n", p.c_str(), checksum(l.bv, kvd));
        } else if (l.bq || l.bk || l.bv) {
            return 4;
        }
        printf("%sgate_proj %llu\n", p.c_str(), checksum(l.Wgate, F * H));
        printf("%sup_proj %llu\n", p.c_str(), checksum(l.Wup, F * H));
        printf("%sdown_proj %llu\n", p.c_str(), checksum(l.Wdown, H * F));
        printf("%snorm_attn %llu\n", p.c_str(), checksum(l.norm_attn, H));
        printf("%snorm_mlp %llu\n", p.c_str(), checksum(l.norm_mlp, H));
    }
    cdna3::runtime::KVCache kv;
    if (kv.allocate(c.n_layers, c.n_kv_heads, max_seq, c.head_dim) != hipSuccess) return 5;
    const size_t per_layer = (size_t)c.n_kv_heads * max_seq * c.head_dim;
    if (kv.K_layer(1, 5) != kv.K + per_layer + 5 * (size_t)c.head_dim) return 6;
    if (kv.V_layer(c.n_layers - 1, 0) != kv.V + per_layer * (c.n_layers - 1)) return 7;
    std::vector<uint16_t> h(per_layer * c.n_layers, 1);
    if (hipMemcpy(h.data(), kv.K, kv.bytes(), hipMemcpyDeviceToHost) != hipSuccess) return 8;
    for (uint16_t v : h)
        if (v != 0) return 9;   // allocate() zero-fills, as the reference's does
    kv.free_buffers();
    if (kv.K || kv.V) return 10;
    printf("kvcache ok\n");
    return 0;
}
