/*
 * slm_layer -- the rest of static-lm's transformer block on MI355X.
 *
 * The JIT kernels that surround the projections (FuseGraph, src/jit/graph.rs:
 * 130-193, lowered by src/jit/lower.rs:212-480) and the whole block around
 * the attention path:
 *   - rmsnorm, l2_norm: bit-identical to the JIT kernels (four lane
 *     accumulators over i < n & ~3, then (l0 + l1) + (l2 + l3), then the
 *     tail in order; IEEE division and square root; no fused multiply-add);
 *   - swiglu, residual_add: elementwise, bit-identical (the SiLU uses the
 *     JIT's polynomial exp, lower.rs:22-65 and 85-91);
 *   - slm_layer_forward_dev: forward_token_with_kv (n = 1) and
 *     forward_batch_with_kv (n > 1) on a device residual stream.
 * Conventions, error codes and streams are those of slm_attn.h; *_dev calls
 * take 16-byte-aligned device pointers and run on the context's stream.  An
 * output must not overlap an input (io_slices / io2_slices, arena.rs:154-208).
 */
#ifndef SLM_LAYER_H
#define SLM_LAYER_H

#include <stdint.h>

#include "slm_quant.h"

#ifdef __cplusplus
extern "C" {
#endif

/* FuseGraph::rmsnorm(n, eps) run by exec_with_weights (engine.rs:190-208) on
 * each of `rows` rows: out[r][i] = (x[r][i] * rms_r) * w[i],
 * rms_r = 1 / sqrt(sum_i x[r][i]^2 * (1 / n) + eps).  1 <= n <= 16384. */
int slm_rmsnorm_dev(slm_attn_ctx* ctx, const float* x, const float* w, int32_t rows,
                    int32_t n, float eps, float* out);

/* FuseGraph::l2_norm(eps) run by exec_unary (engine.rs:153-166) on each row:
 * out[r][i] = x[r][i] * (1 / sqrt(sum_i x[r][i]^2 + eps)). */
int slm_l2_norm_dev(slm_attn_ctx* ctx, const float* x, int32_t rows, int32_t n, float eps,
                    float* out);

/* FuseGraph::swiglu run by exec_binary (engine.rs:170-186):
 * out[i] = silu(gate[i]) * up[i], silu(v) = v / (1 + exp(-v)). */
int slm_swiglu_dev(slm_attn_ctx* ctx, const float* gate, const float* up, int64_t n,
                   float* out);

/* FuseGraph::residual_add run by exec_binary: out[i] = a[i] + b[i]. */
int slm_residual_add_dev(slm_attn_ctx* ctx, const float* a, const float* b, int64_t n,
                         float* out);

/* One layer's weights on the context's device (TransformerWeights,
 * transformer.rs:36-47): the two RMSNorm scale vectors [dim] are device
 * pointers; hidden_dim is w_gate's row count. */
typedef struct slm_layer_weights {
    const float* rms_att;
    const slm_q4_matrix* wq;      /* dim x dim */
    const slm_q4_matrix* wk;      /* kv_dim x dim */
    const slm_q4_matrix* wv;      /* kv_dim x dim */
    const slm_q4_matrix* wo;      /* dim x dim */
    const float* rms_ffn;
    const slm_q4_matrix* w_gate;  /* hidden_dim x dim */
    const slm_q4_matrix* w_up;    /* hidden_dim x dim */
    const slm_q4_matrix* w_down;  /* dim x hidden_dim */
} slm_layer_weights;

/* The transformer block on the residual stream x [n][dim] (in place) for
 * rows start..start+n-1 of `layer`'s KV cache: forward_token_with_kv
 * (transformer.rs:391-487) when n == 1, forward_batch_with_kv (:491-651)
 * otherwise.  RMSNorm -> Q/K/V -> RoPE + KV append -> attention -> Wo +
 * residual -> RMSNorm -> gate, up -> SwiGLU -> down + residual, with the
 * reference's arithmetic in every step (projections bit-identical to the
 * scalar dot, attention within 1e-4 / 1e-3).  rms_eps is
 * TransformerConfig::rms_eps; dim at most 16384 and hidden_dim a multiple of
 * 32 and at most 16384 (SLM_ERR_SHAPE otherwise). */
int slm_layer_forward_dev(slm_attn_ctx* ctx, int32_t layer, int32_t start, int32_t n,
                          const slm_layer_weights* w, float rms_eps, float* x);

/* ---- the whole model (TransformerModel, transformer.rs:699-957) ---- */

/* A token id outside [0, vocab_size) (transformer.rs:757-760, 813, 911). */
#define SLM_ERR_TOKEN (-11)

/* ModelWeights (transformer.rs:49-56) on the context's device: one
 * slm_layer_weights per layer of the context (a host array), the final
 * RMSNorm scale (device [dim]) and the vocab_size x dim token embedding and
 * lm_head matrices. */
typedef struct slm_model_weights {
    const slm_q4_matrix* token_embd;
    const slm_layer_weights* layers;  /* [num_layers] */
    int32_t num_layers;
    const float* output_norm;
    const slm_q4_matrix* lm_head;
} slm_model_weights;

/* TransformerModel::forward_token (transformer.rs:746-796): the embedding row
 * of `token` (dequantize_row_q4_0), every layer at `pos`, the final RMSNorm,
 * the lm_head projection into logits and the greedy argmax (sample_argmax,
 * :654-666: the first index of the maximum).  logits is a device [vocab]
 * buffer or NULL (then the context keeps them); *next_token is written on the
 * host, so the call waits for the stream. */
int slm_model_forward_token_dev(slm_attn_ctx* ctx, const slm_model_weights* w, float rms_eps,
                                int32_t token, int32_t pos, float* logits, int32_t* next_token);

/* TransformerModel::prefill_tokens (transformer.rs:800-850): the n host token
 * ids at rows start..start+n-1 through every layer as one batch, then the
 * logits and argmax of the last row. */
int slm_model_prefill_dev(slm_attn_ctx* ctx, const slm_model_weights* w, float rms_eps,
                          const int32_t* tokens, int32_t n, int32_t start, float* logits,
                          int32_t* next_token);

/* TransformerModel::generate (transformer.rs:853-899): prefill of the prompt
 * at 0, then greedy decode, writing up to max_out tokens to out_tokens (host)
 * and stopping after `eos` (eos < 0: none) or at max_seq_len.  *n_out is the
 * number written (0 for an empty prompt or max_out == 0).  The decode steps
 * are pipelined (each token is read back while the next step runs on the
 * device); when generation stops at `eos` the step already run on the EOS
 * token is discarded and the K/V rows it wrote (every layer, at the position
 * after the last returned token) are restored, so the cache holds exactly
 * what the reference's leaves: rows 0..n_prompt + *n_out - 2 written. */
int slm_model_generate_dev(slm_attn_ctx* ctx, const slm_model_weights* w, float rms_eps,
                           const int32_t* prompt, int32_t n_prompt, int32_t* out_tokens,
                           int32_t max_out, int32_t eos, int32_t* n_out);

/* TransformerModel::embed_tokens (transformer.rs:904-957): the n tokens
 * through every layer as a batch at 0, each row normed with output_norm, the
 * rows averaged (accum += row * (1/n) in order) and L2-normalized into out
 * (device [dim]). */
int slm_model_embed_dev(slm_attn_ctx* ctx, const slm_model_weights* w, float rms_eps,
                        const int32_t* tokens, int32_t n, float* out);

#ifdef __cplusplus
}
#endif

#endif /* SLM_LAYER_H */
