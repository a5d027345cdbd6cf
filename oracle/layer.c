/* CPU restatement of the JIT normalisation / activation kernels and of the
 * whole transformer block of static-lm -- TEST INFRASTRUCTURE ONLY (the
 * oracle the GPU path is checked against; never linked into the product).
 *
 * JIT kernels: FuseGraph::{swiglu, rmsnorm, residual_add, l2_norm}
 * (src/jit/graph.rs:130-193) as lower_fuse_graph emits them
 * (src/jit/lower.rs:212-480): every reduction is a 4-lane F32X4 loop over
 * i < n & ~3 (lane k takes i = k mod 4, lower.rs:244, 252-320), then
 * (l0 + l1) + (l2 + l3) (323-343), then a scalar tail in order (346-378);
 * scalar ops on the reduced value are hoisted (hoist_invariant_nodes,
 * 118-190); the store pass applies the elementwise ops lane by lane
 * (391-477).  Ops are IEEE f32 with no contraction; Recip is 1.0 / x (fdiv,
 * 81-84); SiLU is v / (1 + exp(-v)) with the polynomial exp (85-91). */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "slm_oracle.h"

/* reduce_sum of x[i] * x[i] in the lowered order. */
static float jit_sum_squares(const float* x, size_t n) {
    const size_t vl = n & ~(size_t)3;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    size_t i = 0;
    for (; i < vl; i += 4)
        for (int l = 0; l < 4; ++l) {
            const float sq = x[i + l] * x[i + l];
            acc[l] = acc[l] + sq;
        }
    float s = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    for (; i < n; ++i) {
        const float sq = x[i] * x[i];
        s = s + sq;
    }
    return s;
}

float orc_jit_rmsnorm_scale(const float* x, size_t n, float eps) {
    /* graph.rs:141-156: mean = sum * (1.0 / n), + eps, sqrt, recip */
    const float inv_n = 1.0f / (float)n;
    const float mean = jit_sum_squares(x, n) * inv_n;
    const float var = mean + eps;
    const float sd = sqrtf(var);
    return 1.0f / sd;
}

void orc_jit_rmsnorm(const float* x, const float* w, size_t n, float eps, float* out) {
    const float rms = orc_jit_rmsnorm_scale(x, n, eps);
    for (size_t i = 0; i < n; ++i) {
        const float nx = x[i] * rms;
        out[i] = nx * w[i];
    }
}

float orc_jit_silu(float v) {
    /* lower.rs:85-91 */
    const float e = orc_jit_exp(-v);
    const float den = 1.0f + e;
    return v / den;
}

void orc_jit_swiglu(const float* gate, const float* up, size_t n, float* out) {
    /* graph.rs:131-139 */
    for (size_t i = 0; i < n; ++i) out[i] = orc_jit_silu(gate[i]) * up[i];
}

void orc_jit_residual_add(const float* a, const float* b, size_t n, float* out) {
    /* graph.rs:157-164 */
    for (size_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
}

void orc_jit_l2_norm(const float* x, size_t n, float eps, float* out) {
    /* graph.rs:182-193 */
    const float var = jit_sum_squares(x, n) + eps;
    const float nrm = sqrtf(var);
    const float inv = 1.0f / nrm;
    for (size_t i = 0; i < n; ++i) out[i] = x[i] * inv;
}

void orc_scalar_rmsnorm(const float* x, const float* w, size_t n, float eps, float* out) {
    /* the reference's test helper scalar_rmsnorm (transformer.rs:978-985):
     * a sequential sum and a divide, a different rounding order */
    float ss = 0.0f;
    for (size_t i = 0; i < n; ++i) ss = ss + x[i] * x[i];
    const float rms = 1.0f / sqrtf(ss / (float)n + eps);
    for (size_t i = 0; i < n; ++i) out[i] = x[i] * rms * w[i];
}

/* gemv_q4_0_arena / gemm_q4_0_arena (kernels.rs:286-303, 398-415): quantize
 * each of the batch rows of x to Q8_0, then the scalar dot per output. */
static void gemm_f32(const uint8_t* w, const float* x, float* out, int batch, int rows,
                     int cols) {
    const size_t nb = (size_t)cols / ORC_QK;
    uint8_t* xq = (uint8_t*)calloc((size_t)batch * nb, ORC_Q8_BYTES);
    for (int b = 0; b < batch; ++b)
        orc_quantize_row_q8_0(x + (size_t)b * cols, (size_t)cols, xq + (size_t)b * nb * ORC_Q8_BYTES);
    orc_gemm_q4_0(w, xq, out, batch, rows, cols, 0);
    free(xq);
}

void orc_layer_forward_batch(const orc_config* cfg, int hidden_dim, float eps,
                             const orc_layer_weights* w, float* kv, const float* cos_tab,
                             const float* sin_tab, int layer, int start, int n, float* x) {
    /* forward_batch_with_kv (transformer.rs:491-651); n = 1 is
     * forward_token_with_kv (391-487): the same operations on one row. */
    const int dim = cfg->dim;
    const int hd = dim / cfg->num_heads;
    const int kv_dim = hd * cfg->num_kv_heads;
    const size_t nd = (size_t)n * dim, nh = (size_t)n * hidden_dim;
    float* xb = (float*)malloc(nd * sizeof(float));
    float* xb2 = (float*)malloc(nd * sizeof(float));
    float* x_mid = (float*)malloc(nd * sizeof(float));
    float* q = (float*)malloc(nd * sizeof(float));
    float* q_rot = (float*)malloc(nd * sizeof(float));
    float* k = (float*)malloc((size_t)n * kv_dim * sizeof(float));
    float* v = (float*)malloc((size_t)n * kv_dim * sizeof(float));
    float* att = (float*)malloc((size_t)cfg->num_heads * cfg->max_seq_len * sizeof(float));
    float* hb = (float*)malloc(nh * sizeof(float));
    float* hb2 = (float*)malloc(nh * sizeof(float));
    float* hb_act = (float*)malloc(nh * sizeof(float));

    for (int b = 0; b < n; ++b) /* :519-527 */
        orc_jit_rmsnorm(x + (size_t)b * dim, w->rms_att, (size_t)dim, eps, xb + (size_t)b * dim);
    gemm_f32(w->wq, xb, q, n, dim, dim); /* :530-561 */
    gemm_f32(w->wk, xb, k, n, kv_dim, dim);
    gemm_f32(w->wv, xb, v, n, kv_dim, dim);
    orc_prefill(cfg, kv, cos_tab, sin_tab, layer, start, n, q, k, v, q_rot, att, xb); /* :563-593 */
    gemm_f32(w->wo, xb, xb2, n, dim, dim);  /* :595-604 */
    orc_jit_residual_add(x, xb2, nd, x_mid); /* :605 */
    for (int b = 0; b < n; ++b) /* :607-615 */
        orc_jit_rmsnorm(x_mid + (size_t)b * dim, w->rms_ffn, (size_t)dim, eps, xb + (size_t)b * dim);
    gemm_f32(w->w_gate, xb, hb, n, hidden_dim, dim); /* :617-636 */
    gemm_f32(w->w_up, xb, hb2, n, hidden_dim, dim);
    orc_jit_swiglu(hb, hb2, nh, hb_act); /* :638 */
    gemm_f32(w->w_down, hb_act, xb, n, dim, hidden_dim); /* :640-649 */
    orc_jit_residual_add(x_mid, xb, nd, x); /* :650 */

    free(xb); free(xb2); free(x_mid); free(q); free(q_rot); free(k); free(v);
    free(att); free(hb); free(hb2); free(hb_act);
}
