/*
 * CPU oracle for the static-lm attention hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * This library is the checker, never the product: only tests/, the smoke()
 * entry point and bench.py's cpu_baseline leg may load it.  The product
 * (libslm_attn.so) neither links nor calls it, and fails loudly when its
 * own HIP code is missing.
 *
 * It restates, operation for operation, the reference's single-threaded CPU
 * arithmetic (Rust, src/model/transformer.rs and src/jit/lower.rs of
 * static-lm).  Compile with -O2/-O3 -fno-fast-math -ffp-contract=off so that
 * every f32 product and sum is rounded on its own, as Rust does.
 *
 * Each function cites the reference lines it follows.  How each is pinned
 * (closed forms, brute force, the reference's own test bounds) is listed in
 * tests/test_oracle.py; every function here has at least one such check.
 */
#ifndef SLM_ORACLE_H
#define SLM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* TransformerConfig subset used by attention (transformer.rs:8-33). */
typedef struct {
    int32_t dim;
    int32_t num_heads;
    int32_t num_kv_heads;
    int32_t max_seq_len;
    int32_t num_layers;
    float rope_theta; /* 10000.0f is the reference's hard-coded literal */
} orc_config;

/* Config asserts of LayerWorkspace::allocate (transformer.rs:81-101).
 * Returns 0 when valid, else a negative code. */
int orc_validate(const orc_config* cfg);

/* RoPE tables [max_seq_len][head_dim/2] (transformer.rs:124-133). */
void orc_rope_tables(int head_dim, int max_seq_len, float theta, float* cos_out,
                     float* sin_out);

/* apply_rope_cached (transformer.rs:178-194): rotate every head slice of
 * `vec` (length len, a multiple of head_dim) in place. */
void orc_apply_rope_cached(float* vec, size_t len, const float* cos_row,
                           const float* sin_row, int head_dim);

/* apply_rope_in_place (transformer.rs:196-212), theta generalised. */
void orc_apply_rope_in_place(float* vec, size_t len, int pos, int head_dim,
                             float theta);

/* emit_exp_f32x4 (lower.rs:20-65), one lane. */
float orc_jit_exp(float x);
/* orc_jit_exp over an array (test convenience). */
void orc_jit_exp_array(const float* x, float* out, size_t n);

/* FuseGraph::softmax (graph.rs:166-179) lowered by lower_fuse_graph
 * (lower.rs:212-480); in place, like the call at transformer.rs:308-311. */
void orc_softmax_jit(float* x, size_t n);

/* Softmax block of the scalar attention (transformer.rs:238-259). */
void orc_softmax_scalar(float* x, size_t n);

/* causal_multi_head_attention_jit (transformer.rs:273-321).  k_cache and
 * v_cache are one layer's [max_seq_len][kv_dim] slices; att is scratch of
 * num_heads*max_seq_len floats; out has dim floats. */
void orc_attention_jit(const float* q, const float* k_cache,
                       const float* v_cache, float* att, float* out,
                       const orc_config* cfg, int pos);

/* causal_multi_head_attention (transformer.rs:214-271). */
void orc_attention_scalar(const float* q, const float* k_cache,
                          const float* v_cache, float* att, float* out,
                          const orc_config* cfg, int pos);

/* Offset in floats of row `pos` of K (which=0) or V (which=1) of `layer`
 * inside the contiguous KV region: LayerKvCache::allocate in layer order
 * (transformer.rs:323-338, 724-726) with AlignedArena::alloc_slice
 * (arena.rs:95-113) inserting no padding because kv_dim % 32 == 0. */
size_t orc_kv_offset(const orc_config* cfg, int layer, int which, int pos);

/* Decode attention block of forward_token_with_kv (transformer.rs:413-443):
 * K row `pos` <- rope(k), V row `pos` <- v, q rotated into q_rot, then
 * causal_multi_head_attention_jit at `pos`.  kv is the whole
 * [L][2][msl][kv_dim] region; cos/sin are the tables; att scratch. */
void orc_decode(const orc_config* cfg, float* kv, const float* cos_tab,
                const float* sin_tab, int layer, int pos, const float* q,
                const float* k, const float* v, float* q_rot, float* att,
                float* out);

/* Prefill attention block of forward_batch_with_kv (transformer.rs:530-593):
 * rows start..start+n-1 of K and V written (un-rotated, as the GEMM does),
 * then for b in order: rope(q_b), rope(K row start+b), attention at
 * start+b.  q is [n][dim]; k, v are [n][kv_dim]; out is [n][dim]. */
void orc_prefill(const orc_config* cfg, float* kv, const float* cos_tab,
                 const float* sin_tab, int layer, int start, int n,
                 const float* q, const float* k, const float* v, float* q_rot,
                 float* att, float* out);

/* Independent f64 checker: exact softmax attention in double over rotated q
 * and a cache region, no reference rounding order.  Not a restatement. */
void orc_attention_f64(const float* q, const float* k_cache,
                       const float* v_cache, double* out,
                       const orc_config* cfg, int pos);

/* ---- Quantized projections (src/quant/blocks.rs, src/quant/kernels.rs) ----
 * Blocks are the reference's byte layouts: BlockQ4_0 = u16 f16 scale + 16
 * bytes of nibbles (18 B, blocks.rs:11-19), BlockQ8_0 = u16 f16 scale + 32 i8
 * (34 B, blocks.rs:32-40), scale bytes little-endian. */
#define ORC_QK 32
#define ORC_Q4_BYTES 18
#define ORC_Q8_BYTES 34

/* half::f16::from_f32 / to_f32 (round to nearest even; exact). */
uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);

/* quantize_row_q4_0 (blocks.rs:50-82); n % 32 == 0, dst n/32 blocks. */
void orc_quantize_row_q4_0(const float* src, size_t n, uint8_t* dst);
/* dequantize_row_q4_0 (blocks.rs:85-99). */
void orc_dequantize_row_q4_0(const uint8_t* src, size_t nblocks, float* dst);
/* quantize_row_q8_0 (blocks.rs:102-123). */
void orc_quantize_row_q8_0(const float* src, size_t n, uint8_t* dst);
/* dequantize_row_q8_0 (blocks.rs:126-135). */
void orc_dequantize_row_q8_0(const uint8_t* src, size_t nblocks, float* dst);

/* vec_dot_q4_0_q8_0_scalar (kernels.rs:145-161). */
float orc_vec_dot_q4_0_q8_0_scalar(const uint8_t* w, const uint8_t* a, size_t nblocks);
/* vec_dot_q4_0_q8_0_avx2 (kernels.rs:163-212), restated lane by lane. */
float orc_vec_dot_q4_0_q8_0_avx2(const uint8_t* w, const uint8_t* a, size_t nblocks);
/* gemm_q4_0 (kernels.rs:308-394): out[b*rows + r]; avx2 picks the dot. */
void orc_gemm_q4_0(const uint8_t* w, const uint8_t* x_q8, float* out, int batch, int rows,
                   int cols, int avx2);

/* ---- JIT normalisation / activation kernels and the transformer block
 * (layer.c; graph.rs:130-193 lowered by lower.rs:212-480) ---- */
/* RMSNorm's scale 1 / sqrt(sum(x^2) * (1/n) + eps), JIT reduction order. */
float orc_jit_rmsnorm_scale(const float* x, size_t n, float eps);
/* FuseGraph::rmsnorm: out[i] = (x[i] * rms) * w[i]. */
void orc_jit_rmsnorm(const float* x, const float* w, size_t n, float eps, float* out);
/* SiLU lowering: v / (1 + exp(-v)), polynomial exp. */
float orc_jit_silu(float v);
/* FuseGraph::swiglu: out[i] = silu(gate[i]) * up[i]. */
void orc_jit_swiglu(const float* gate, const float* up, size_t n, float* out);
/* FuseGraph::residual_add: out[i] = a[i] + b[i]. */
void orc_jit_residual_add(const float* a, const float* b, size_t n, float* out);
/* FuseGraph::l2_norm: out[i] = x[i] * (1 / sqrt(sum(x^2) + eps)). */
void orc_jit_l2_norm(const float* x, size_t n, float eps, float* out);
/* The reference tests' scalar_rmsnorm (transformer.rs:978-985). */
void orc_scalar_rmsnorm(const float* x, const float* w, size_t n, float eps, float* out);

/* One layer's weights: f32 norm scales and BlockQ4_0 matrices (18-byte
 * blocks, row-major) as TransformerWeights holds them (transformer.rs:36-47). */
typedef struct {
    const float* rms_att;
    const uint8_t* wq;
    const uint8_t* wk;
    const uint8_t* wv;
    const uint8_t* wo;
    const float* rms_ffn;
    const uint8_t* w_gate;
    const uint8_t* w_up;
    const uint8_t* w_down;
} orc_layer_weights;

/* forward_batch_with_kv (transformer.rs:491-651) on x [n][dim] in place;
 * n = 1 is forward_token_with_kv (391-487).  GEMMs use the scalar dot. */
void orc_layer_forward_batch(const orc_config* cfg, int hidden_dim, float eps,
                             const orc_layer_weights* w, float* kv, const float* cos_tab,
                             const float* sin_tab, int layer, int start, int n, float* x);

#ifdef __cplusplus
}
#endif

#endif
