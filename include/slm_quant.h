/*
 * slm_quant -- the Q/K/V projections that feed the attention path, on MI355X.
 *
 * static-lm computes q, k and v with Q4_0 weights times Q8_0-quantized
 * activations (src/quant/blocks.rs, src/quant/kernels.rs), called from the
 * decode block (gemv_q4_0_arena x3, transformer.rs:413-417) and the prefill
 * block (gemm_q4_0_arena x3, transformer.rs:530-561).  These entry points run
 * the same arithmetic on the device:
 *   - outputs are bit-identical to vec_dot_q4_0_q8_0_scalar
 *     (kernels.rs:145-161; the NEON path gives the same bits) and within the
 *     reference's own 1e-5 bound of its x86 AVX2 path (kernels.rs:163-212);
 *   - activation blocks are bit-identical to quantize_row_q8_0
 *     (blocks.rs:102-123).
 * Conventions, error codes and streams are those of slm_attn.h; *_dev calls
 * take 16-byte-aligned device pointers and run on the context's stream.
 */
#ifndef SLM_QUANT_H
#define SLM_QUANT_H

#include <stdint.h>

#include "slm_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* A weight matrix whose shape does not fit the call, or a length that is not
 * a multiple of 32 (the assert_eq!s of gemm_q4_0, kernels.rs:316-332, and of
 * quantize_row_q8_0, blocks.rs:103-104). */
#define SLM_ERR_SHAPE (-10)

/* Device-resident Q4_0 weight matrix. */
typedef struct slm_q4_matrix slm_q4_matrix;

/* Uploads a row-major matrix of rows x cols weights given as rows*cols/32
 * BlockQ4_0 of 18 bytes each (f16 scale, then 16 bytes of nibbles: the
 * reference's and GGUF's layout, blocks.rs:11-19) to `device`, repacked for
 * the kernels.  cols must be a multiple of 32 and at most 16384. */
int slm_q4_matrix_create(int32_t device, const void* blocks, int32_t rows, int32_t cols,
                         slm_q4_matrix** out);
void slm_q4_matrix_destroy(slm_q4_matrix* m);
int slm_q4_matrix_shape(const slm_q4_matrix* m, int32_t* rows, int32_t* cols);

/* quantize_row_q8_0 (blocks.rs:102-123): x [n] f32 (n a multiple of 32) into
 * n/32 BlockQ8_0 of 34 bytes (f16 scale, 32 i8) at `blocks` (2-byte aligned). */
int slm_quantize_q8_0_dev(slm_attn_ctx* ctx, const float* x, int64_t n, void* blocks);

/* gemm_q4_0_arena (kernels.rs:398-415): each of the batch rows of x
 * [batch][cols] is quantized to Q8_0 and out[b*rows + r] = vec_dot(W row r,
 * q8(x row b)).  batch 0 does nothing, as in the reference.  out must not
 * overlap x (gemv_slices, arena.rs:210-229). */
int slm_gemm_q4_0_dev(slm_attn_ctx* ctx, const slm_q4_matrix* w, const float* x,
                      int32_t batch, float* out);

/* A projection followed by the residual add: out[b*rows + r] = res[b*rows + r]
 * + vec_dot(W row r, q8(x row b)), the gemv_q4_0_arena / gemm_q4_0_arena call
 * and the residual_add JIT kernel after it (graph.rs:157-164): Wo then
 * x_mid = x + xb2 (transformer.rs:445-446, batched :595-605) and w_down then
 * x = x_mid + xb (:477-486, batched :640-650).  Bit-identical to the scalar
 * dot followed by one f32 add.  res may be out itself (in-place x += W.x_in);
 * otherwise neither res nor out may overlap x, and out must not overlap res. */
int slm_gemm_q4_0_residual_dev(slm_attn_ctx* ctx, const slm_q4_matrix* w, const float* x,
                               int32_t batch, const float* res, float* out);

/* The decode attention block of forward_token_with_kv from the attention
 * RMSNorm output (transformer.rs:413-443): q = Wq.xb, k = Wk.xb, v = Wv.xb
 * (xb quantized once), then slm_attn_decode_dev at `pos`.  wq is dim x dim,
 * wk and wv kv_dim x dim. */
int slm_attn_decode_xb_dev(slm_attn_ctx* ctx, int32_t layer, int32_t pos, const float* xb,
                           const slm_q4_matrix* wq, const slm_q4_matrix* wk,
                           const slm_q4_matrix* wv, float* out);

/* slm_attn_decode_xb_dev without any device allocation, for callers that
 * cannot allocate (code under HIP graph capture, serving loops, harnesses
 * that forbid hipMalloc).  No counterpart in the reference: its GEMVs write
 * into the caller's arena.  q, k, v and the decode split partials live in a
 * file-scope device array of 1 MiB (262144 floats) that each GPU holds until
 * the process ends; a call needs dim + 2*kv_dim + n_splits*num_heads*
 * (head_dim + 2) floats of it (n_splits from slm_attn_decode_splits at pos +
 * 1) and returns SLM_ERR_SHAPE above that.  Every call on a GPU shares that
 * GPU's array and nothing in it needs clearing: calls that overlap on one
 * GPU (two streams, two contexts) race and must be ordered by the caller.
 * Not timed by slm_attn_profile.  Results are identical to
 * slm_attn_decode_xb_dev's. */
int slm_attn_decode_xb_dev_noalloc(slm_attn_ctx* ctx, int32_t layer, int32_t pos,
                                   const float* xb, const slm_q4_matrix* wq,
                                   const slm_q4_matrix* wk, const slm_q4_matrix* wv,
                                   float* out);

/* The prefill attention block of forward_batch_with_kv from n rows of the
 * attention RMSNorm output (transformer.rs:530-593): the three GEMMs, then
 * slm_attn_prefill_dev for rows start..start+n-1. */
int slm_attn_prefill_xb_dev(slm_attn_ctx* ctx, int32_t layer, int32_t start, int32_t n,
                            const float* xb, const slm_q4_matrix* wq, const slm_q4_matrix* wk,
                            const slm_q4_matrix* wv, float* out);

/* The attention half of the decode block from the attention RMSNorm output
 * to the residual stream (transformer.rs:413-446): q, k, v from xb, RoPE, KV
 * append, attention written back into xb (the reference reuses ws.xb for the
 * attention output, :432-442), then x_mid = x + Wo.xb.  wo is dim x dim.
 * x_mid may be x itself; xb must not overlap x, x_mid or the KV cache. */
int slm_attn_decode_wo_dev(slm_attn_ctx* ctx, int32_t layer, int32_t pos, float* xb,
                           const slm_q4_matrix* wq, const slm_q4_matrix* wk,
                           const slm_q4_matrix* wv, const slm_q4_matrix* wo, const float* x,
                           float* x_mid);

/* The same for a prefill batch of n rows at start (transformer.rs:530-605):
 * xb, x and x_mid are [n][dim]. */
int slm_attn_prefill_wo_dev(slm_attn_ctx* ctx, int32_t layer, int32_t start, int32_t n,
                            float* xb, const slm_q4_matrix* wq, const slm_q4_matrix* wk,
                            const slm_q4_matrix* wv, const slm_q4_matrix* wo, const float* x,
                            float* x_mid);

#ifdef __cplusplus
}
#endif

#endif /* SLM_QUANT_H */
