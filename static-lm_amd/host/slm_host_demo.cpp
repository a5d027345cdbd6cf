// Drives the C++ host mirror (slm_attention.hpp) the way TransformerModel
// drives its layers: one batched prefill, then single-token decode steps, on
// one layer.  Used by the GPU tests to check the C++ wrapper end to end.
//
// usage: slm_host_demo dim heads kv_heads max_seq_len theta n_prefill n_decode
//                      in.bin out.bin
//   in.bin : f32 q[(P+D)][dim], k[(P+D)][kv_dim], v[(P+D)][kv_dim]
//   out.bin: f32 out[(P+D)][dim], then int32 code of an out-of-range decode
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "slm_attention.hpp"

int main(int argc, char** argv) {
    if (argc != 10) {
        std::fprintf(stderr,
                     "usage: %s dim heads kv_heads max_seq_len theta n_prefill "
                     "n_decode in.bin out.bin\n",
                     argv[0]);
        return 2;
    }
    static_lm::TransformerConfig cfg{};
    cfg.dim = std::strtoul(argv[1], nullptr, 10);
    cfg.num_heads = std::strtoul(argv[2], nullptr, 10);
    cfg.num_kv_heads = std::strtoul(argv[3], nullptr, 10);
    cfg.max_seq_len = std::strtoul(argv[4], nullptr, 10);
    cfg.hidden_dim = cfg.dim;
    cfg.rms_eps = 1e-5f;
    const float theta = std::strtof(argv[5], nullptr);
    const size_t np = std::strtoul(argv[6], nullptr, 10);
    const size_t nd = std::strtoul(argv[7], nullptr, 10);
    const size_t rows = np + nd;
    const size_t dim = cfg.dim, kvd = cfg.kv_dim();

    std::vector<float> q(rows * dim), k(rows * kvd), v(rows * kvd),
        out(rows * dim, 0.0f);
    FILE* f = std::fopen(argv[8], "rb");
    if (!f) return 3;
    const bool ok = std::fread(q.data(), 4, q.size(), f) == q.size() &&
                    std::fread(k.data(), 4, k.size(), f) == k.size() &&
                    std::fread(v.data(), 4, v.size(), f) == v.size();
    std::fclose(f);
    if (!ok) return 4;

    int32_t err_code = 0;
    try {
        static_lm::DeviceAttention attn(cfg, 1, theta);
        if (np > 0)
            attn.forward_batch_attention(0, 0, np, q.data(), k.data(), v.data(),
                                         out.data());
        for (size_t s = 0; s < nd; ++s) {
            const size_t r = np + s;
            attn.forward_token_attention(0, r, q.data() + r * dim,
                                         k.data() + r * kvd, v.data() + r * kvd,
                                         out.data() + r * dim);
        }
        try {
            attn.forward_token_attention(0, cfg.max_seq_len, q.data(), k.data(),
                                         v.data(), out.data());
        } catch (const static_lm::AttentionError& e) {
            err_code = e.code();
        }
    } catch (const static_lm::AttentionError& e) {
        std::fprintf(stderr, "AttentionError %d: %s\n", e.code(), e.what());
        return 5;
    }

    FILE* g = std::fopen(argv[9], "wb");
    if (!g) return 6;
    std::fwrite(out.data(), 4, out.size(), g);
    std::fwrite(&err_code, 4, 1, g);
    std::fclose(g);
    return 0;
}
