// C++ host mirror of static-lm's attention interface over the slm_attn C ABI.
//
// Names, argument meaning and failure behaviour follow the reference
// (src/model/transformer.rs, src/memory/arena.rs):
//   TransformerConfig            transformer.rs:8-33
//   ArenaSlice / LayerKvCache    arena.rs:10-37, transformer.rs:323-338
//   forward_token_attention      the attention block of
//                                TransformerLayer::forward_token_with_kv,
//                                transformer.rs:413-443
//   forward_batch_attention      the attention block of forward_batch_with_kv,
//                                transformer.rs:530-593
//   causal_multi_head_attention_jit  transformer.rs:275-321, on a rotated q
//   apply_rope_cached            transformer.rs:180-194, on device rows
// The reference panics on a violated assert; this wrapper throws
// static_lm::AttentionError carrying the C ABI code and message instead.
#pragma once

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

#include "slm_attn.h"

namespace static_lm {

struct TransformerConfig {
    size_t dim;
    size_t hidden_dim;
    size_t num_heads;
    size_t num_kv_heads;
    size_t max_seq_len;
    float rms_eps;

    size_t head_dim() const { return dim / num_heads; }
    size_t kv_dim() const { return (dim / num_heads) * num_kv_heads; }
    size_t kv_mul() const { return num_heads / num_kv_heads; }
};

// Offset/length handle in f32 elements, as the reference's ArenaSlice; here
// the offsets are relative to the device KV region base.
struct ArenaSlice {
    size_t offset;
    size_t len;
    size_t end() const { return offset + len; }
    bool overlaps(const ArenaSlice& o) const {
        return offset < o.end() && o.offset < end();
    }
};

struct LayerKvCache {
    ArenaSlice k_cache;
    ArenaSlice v_cache;
};

class AttentionError : public std::runtime_error {
   public:
    AttentionError(int code, const std::string& msg)
        : std::runtime_error(msg), code_(code) {}
    int code() const { return code_; }

   private:
    int code_;
};

// Device-resident KV cache plus RoPE tables for `num_layers` layers of one
// model; the MI355X counterpart of the KV part of TransformerModel.
class DeviceAttention {
   public:
    DeviceAttention(const TransformerConfig& cfg, size_t num_layers,
                    float rope_theta = 10000.0f)
        : cfg_(cfg), num_layers_(num_layers) {
        slm_attn_config c{};
        c.dim = static_cast<int32_t>(cfg.dim);
        c.num_heads = static_cast<int32_t>(cfg.num_heads);
        c.num_kv_heads = static_cast<int32_t>(cfg.num_kv_heads);
        c.max_seq_len = static_cast<int32_t>(cfg.max_seq_len);
        c.num_layers = static_cast<int32_t>(num_layers);
        c.rope_theta = rope_theta;
        check(slm_attn_create(&c, &ctx_), nullptr);
    }
    ~DeviceAttention() { slm_attn_destroy(ctx_); }
    DeviceAttention(const DeviceAttention&) = delete;
    DeviceAttention& operator=(const DeviceAttention&) = delete;

    const TransformerConfig& config() const { return cfg_; }
    size_t num_layers() const { return num_layers_; }
    slm_attn_ctx* raw() { return ctx_; }

    // The layer's K and V slices, at the offsets LayerKvCache::allocate
    // gives them when called in layer order (transformer.rs:724-726).
    LayerKvCache kv_cache(size_t layer) const {
        const size_t k = slm_kv_offset(ctx_, (int32_t)layer, 0, 0);
        const size_t v = slm_kv_offset(ctx_, (int32_t)layer, 1, 0);
        if (k == (size_t)-1 || v == (size_t)-1)
            throw AttentionError(SLM_ERR_LAYER, "layer index out of range");
        const size_t len = cfg_.max_seq_len * cfg_.kv_dim();
        return LayerKvCache{ArenaSlice{k, len}, ArenaSlice{v, len}};
    }

    // Host buffers: q[dim], k[kv_dim], v[kv_dim] -> out[dim].
    void forward_token_attention(size_t layer, size_t pos, const float* q,
                                 const float* k, const float* v, float* out) {
        check(slm_attn_decode(ctx_, (int32_t)layer, (int32_t)pos, q, k, v, out),
              ctx_);
    }

    // Host buffers: q[batch][dim], k/v[batch][kv_dim] -> out[batch][dim].
    void forward_batch_attention(size_t layer, size_t start_pos, size_t batch,
                                 const float* q, const float* k,
                                 const float* v, float* out) {
        check(slm_attn_prefill(ctx_, (int32_t)layer, (int32_t)start_pos,
                               (int32_t)batch, q, k, v, out),
              ctx_);
    }

    // Device buffers: attention of an already rotated q over the rows
    // 0..=pos of `kv` (which must be one of this model's layer caches).
    void causal_multi_head_attention_jit(const float* q_dev,
                                         const LayerKvCache& kv, float* out_dev,
                                         size_t pos) {
        check(slm_attn_attend_dev(ctx_, layer_of(kv), (int32_t)pos, q_dev,
                                  out_dev),
              ctx_);
    }

    // Device buffer: rotate `rows` rows of `row_len` floats at positions
    // pos0.. in place.
    void apply_rope_cached(float* x_dev, size_t rows, size_t row_len,
                           size_t pos0) {
        check(slm_rope_apply_dev(ctx_, x_dev, (int32_t)rows, (int32_t)row_len,
                                 (int32_t)pos0),
              ctx_);
    }

    void write_kv(size_t layer, int which, size_t pos0, size_t rows,
                  const float* host) {
        check(slm_kv_write(ctx_, (int32_t)layer, which, (int32_t)pos0,
                           (int32_t)rows, host),
              ctx_);
    }
    void read_kv(size_t layer, int which, size_t pos0, size_t rows,
                 float* host) {
        check(slm_kv_read(ctx_, (int32_t)layer, which, (int32_t)pos0,
                          (int32_t)rows, host),
              ctx_);
    }
    void synchronize() { check(slm_attn_sync(ctx_), ctx_); }

   private:
    int32_t layer_of(const LayerKvCache& kv) const {
        for (size_t l = 0; l < num_layers_; ++l) {
            const LayerKvCache c = kv_cache(l);
            if (c.k_cache.offset == kv.k_cache.offset &&
                c.v_cache.offset == kv.v_cache.offset &&
                kv.k_cache.len == c.k_cache.len && kv.v_cache.len == c.v_cache.len)
                return (int32_t)l;
        }
        throw AttentionError(SLM_ERR_ARG,
                             "LayerKvCache is not a layer cache of this model");
    }

    static void check(int rc, const slm_attn_ctx* ctx) {
        if (rc != SLM_OK) throw AttentionError(rc, slm_attn_last_error(ctx));
    }

    TransformerConfig cfg_;
    size_t num_layers_;
    slm_attn_ctx* ctx_ = nullptr;
};

}  // namespace static_lm
