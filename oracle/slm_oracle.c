/*
 * CPU oracle for the static-lm attention hot path -- TEST INFRASTRUCTURE ONLY.
 * Only tests/, smoke() and bench.py's cpu_baseline leg load this code, as the
 * checker.  See slm_oracle.h for the contract and the reference citations.
 *
 * Build: -O3 -fno-fast-math -ffp-contract=off (oracle/Makefile).  Rust never
 * contracts a*b+c into an FMA and evaluates left to right, so every product
 * and every sum below is rounded on its own, in the order written.
 */
#include "slm_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#if defined(__FP_FAST_FMAF) || defined(__FAST_MATH__)
#error "the oracle must be built without fast-math or FMA contraction"
#endif

int orc_validate(const orc_config* c) {
    /* LayerWorkspace::allocate asserts, transformer.rs:81-101 */
    if (!c) return -1;
    if (c->dim <= 0 || c->num_heads <= 0 || c->num_kv_heads <= 0) return -1;
    if (c->max_seq_len <= 0 || c->num_layers <= 0) return -1;
    if (c->dim % 32 != 0) return -1;                       /* :81 */
    if (c->dim % c->num_heads != 0) return -1;             /* :88-92 */
    if (c->num_heads % c->num_kv_heads != 0) return -1;    /* :93-97 */
    int hd = c->dim / c->num_heads;
    if (hd % 2 != 0) return -1;                            /* :100 */
    if ((hd * c->num_kv_heads) % 32 != 0) return -1;       /* :101 */
    if (!(c->rope_theta > 0.0f)) return -1;
    return 0;
}

void orc_rope_tables(int head_dim, int max_seq_len, float theta, float* cos_out,
                     float* sin_out) {
    /* transformer.rs:124-133.  freq is recomputed per (pos, j) there; it is
     * a pure function of j, so computing it per (pos, j) here changes
     * nothing. */
    const int half = head_dim / 2;
    const float head_dim_f = (float)head_dim;
    for (int pos = 0; pos < max_seq_len; ++pos) {
        const float pos_f = (float)pos;
        for (int j = 0; j < half; ++j) {
            const float expo = (float)(2 * j) / head_dim_f;
            const float freq = 1.0f / powf(theta, expo);
            const float a = pos_f * freq;
            cos_out[(size_t)pos * half + j] = cosf(a);
            sin_out[(size_t)pos * half + j] = sinf(a);
        }
    }
}

void orc_apply_rope_cached(float* vec, size_t len, const float* cos_row,
                           const float* sin_row, int head_dim) {
    /* transformer.rs:180-194: interleaved pairs (2j, 2j+1) per head. */
    const int half = head_dim / 2;
    for (size_t h0 = 0; h0 + (size_t)head_dim <= len; h0 += (size_t)head_dim) {
        float* hs = vec + h0;
        for (int j = 0; j < half; ++j) {
            const float c = cos_row[j];
            const float s = sin_row[j];
            const float v0 = hs[2 * j];
            const float v1 = hs[2 * j + 1];
            const float t0 = v0 * c;
            const float t1 = v1 * s;
            const float t2 = v0 * s;
            const float t3 = v1 * c;
            hs[2 * j] = t0 - t1;
            hs[2 * j + 1] = t2 + t3;
        }
    }
}

void orc_apply_rope_in_place(float* vec, size_t len, int pos, int head_dim,
                             float theta) {
    /* transformer.rs:196-212 with i = 2j. */
    const float pos_f = (float)pos;
    const float head_dim_f = (float)head_dim;
    for (size_t h0 = 0; h0 + (size_t)head_dim <= len; h0 += (size_t)head_dim) {
        float* hs = vec + h0;
        for (int i = 0; i < head_dim; i += 2) {
            const float freq = 1.0f / powf(theta, (float)i / head_dim_f);
            const float a = pos_f * freq;
            const float s = sinf(a), c = cosf(a);
            const float v0 = hs[i];
            const float v1 = hs[i + 1];
            const float t0 = v0 * c;
            const float t1 = v1 * s;
            const float t2 = v0 * s;
            const float t3 = v1 * c;
            hs[i] = t0 - t1;
            hs[i + 1] = t2 + t3;
        }
    }
}

/* Cranelift fmax/fmin: NaN-propagating, and -0 orders below +0. */
static inline float cl_fmax(float a, float b) {
    if (a != a || b != b) return a + b;
    if (a == b) return signbit(a) ? b : a;
    return a > b ? a : b;
}
static inline float cl_fmin(float a, float b) {
    if (a != a || b != b) return a + b;
    if (a == b) return signbit(a) ? a : b;
    return a < b ? a : b;
}

float orc_jit_exp(float x) {
    /* emit_exp_f32x4, lower.rs:22-65, one lane. */
    float xc = cl_fmax(x, -87.3f);
    xc = cl_fmin(xc, 88.3f);
    const float fx = xc * 1.44269504088896340736f; /* f32 LOG2_E */
    const float n = nearbyintf(fx);                 /* `nearest`: ties to even */
    const float n_hi = n * 0.69314575f;
    const float n_lo = n * 1.4286068e-6f;
    const float r_hi = xc - n_hi;
    const float r = r_hi - n_lo;
    const float c5 = 1.0f / 120.0f, c4 = 1.0f / 24.0f, c3 = 1.0f / 6.0f;
    float p = r * c5;
    p = p + c4;
    p = r * p;
    p = p + c3;
    p = r * p;
    p = p + 0.5f;
    p = r * p;
    p = p + 1.0f;
    p = r * p;
    const float poly = p + 1.0f;
    const int32_t ni = (int32_t)n; /* fcvt_to_sint_sat; |n| <= 127 here */
    const uint32_t bits = (uint32_t)(ni + 127) << 23;
    float pow2;
    memcpy(&pow2, &bits, sizeof pow2);
    return poly * pow2;
}

void orc_jit_exp_array(const float* x, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_jit_exp(x[i]);
}

void orc_softmax_jit(float* x, size_t n) {
    /* lower_fuse_graph on FuseGraph::softmax: three passes, each a 4-lane
     * strided vector loop over i < n & ~3 (lower.rs:244, 252-320), a
     * pairwise horizontal reduction (323-343) and a scalar tail (346-378). */
    const size_t vl = n & ~(size_t)3;

    float acc[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    size_t i = 0;
    for (; i < vl; i += 4)
        for (int l = 0; l < 4; ++l) acc[l] = cl_fmax(acc[l], x[i + l]);
    float m = cl_fmax(cl_fmax(acc[0], acc[1]), cl_fmax(acc[2], acc[3]));
    for (; i < n; ++i) m = cl_fmax(m, x[i]);

    float sacc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (i = 0; i < vl; i += 4)
        for (int l = 0; l < 4; ++l) sacc[l] = sacc[l] + orc_jit_exp(x[i + l] - m);
    float sum = (sacc[0] + sacc[1]) + (sacc[2] + sacc[3]);
    for (; i < n; ++i) sum = sum + orc_jit_exp(x[i] - m);

    const float inv = 1.0f / sum; /* recip hoisted out of the store pass */
    for (i = 0; i < n; ++i) x[i] = orc_jit_exp(x[i] - m) * inv; /* 391-477 */
}

void orc_softmax_scalar(float* x, size_t n) {
    /* transformer.rs:238-259 */
    float m = -INFINITY;
    for (size_t t = 0; t < n; ++t)
        if (x[t] > m) m = x[t];
    float sum = 0.0f;
    for (size_t t = 0; t < n; ++t) {
        const float e = expf(x[t] - m);
        x[t] = e;
        sum = sum + e;
    }
    const float inv = 1.0f / sum;
    for (size_t t = 0; t < n; ++t) x[t] = x[t] * inv;
}

static void attention_common(const float* q, const float* k_cache,
                             const float* v_cache, float* att, float* out,
                             const orc_config* cfg, int pos, int use_jit) {
    /* transformer.rs:214-321: per head h, kv head h / kv_mul (234, 295);
     * dot is a sequential f32 chain scaled after the sum (299-306);
     * softmax in place; PV accumulated over t in order from zero (313-319). */
    const int hd = cfg->dim / cfg->num_heads;
    const int kv_dim = hd * cfg->num_kv_heads;
    const int kv_mul = cfg->num_heads / cfg->num_kv_heads;
    const float scale = 1.0f / sqrtf((float)hd);
    const size_t seq_len = (size_t)pos + 1;

    for (int i = 0; i < cfg->dim; ++i) out[i] = 0.0f;

    for (int h = 0; h < cfg->num_heads; ++h) {
        const float* q_h = q + (size_t)h * hd;
        const size_t kv_off = (size_t)(h / kv_mul) * hd;
        float* att_h = att + (size_t)h * cfg->max_seq_len;
        for (size_t t = 0; t < seq_len; ++t) {
            const float* k_t = k_cache + t * kv_dim + kv_off;
            float dot = 0.0f;
            for (int i = 0; i < hd; ++i) dot = dot + q_h[i] * k_t[i];
            att_h[t] = dot * scale;
        }
        if (use_jit)
            orc_softmax_jit(att_h, seq_len);
        else
            orc_softmax_scalar(att_h, seq_len);
        float* out_h = out + (size_t)h * hd;
        for (size_t t = 0; t < seq_len; ++t) {
            const float p = att_h[t];
            const float* v_t = v_cache + t * kv_dim + kv_off;
            for (int i = 0; i < hd; ++i) out_h[i] = out_h[i] + p * v_t[i];
        }
    }
}

void orc_attention_jit(const float* q, const float* k_cache,
                       const float* v_cache, float* att, float* out,
                       const orc_config* cfg, int pos) {
    attention_common(q, k_cache, v_cache, att, out, cfg, pos, 1);
}

void orc_attention_scalar(const float* q, const float* k_cache,
                          const float* v_cache, float* att, float* out,
                          const orc_config* cfg, int pos) {
    attention_common(q, k_cache, v_cache, att, out, cfg, pos, 0);
}

size_t orc_kv_offset(const orc_config* cfg, int layer, int which, int pos) {
    const size_t kv_dim =
        (size_t)(cfg->dim / cfg->num_heads) * (size_t)cfg->num_kv_heads;
    return ((size_t)(2 * layer + which) * (size_t)cfg->max_seq_len +
            (size_t)pos) *
           kv_dim;
}

void orc_decode(const orc_config* cfg, float* kv, const float* cos_tab,
                const float* sin_tab, int layer, int pos, const float* q,
                const float* k, const float* v, float* q_rot, float* att,
                float* out) {
    const int hd = cfg->dim / cfg->num_heads;
    const int half = hd / 2;
    const int kv_dim = hd * cfg->num_kv_heads;
    float* k_row = kv + orc_kv_offset(cfg, layer, 0, pos);
    float* v_row = kv + orc_kv_offset(cfg, layer, 1, pos);
    memcpy(k_row, k, sizeof(float) * kv_dim); /* Wk GEMV output, :416 */
    memcpy(v_row, v, sizeof(float) * kv_dim); /* Wv GEMV output, :417 */
    memcpy(q_rot, q, sizeof(float) * cfg->dim);
    const float* c = cos_tab + (size_t)pos * half;
    const float* s = sin_tab + (size_t)pos * half;
    orc_apply_rope_cached(q_rot, cfg->dim, c, s, hd);  /* :419-424 */
    orc_apply_rope_cached(k_row, kv_dim, c, s, hd);    /* :425-428 */
    orc_attention_jit(q_rot, kv + orc_kv_offset(cfg, layer, 0, 0),
                      kv + orc_kv_offset(cfg, layer, 1, 0), att, out, cfg,
                      pos); /* :430-443 */
}

void orc_prefill(const orc_config* cfg, float* kv, const float* cos_tab,
                 const float* sin_tab, int layer, int start, int n,
                 const float* q, const float* k, const float* v, float* q_rot,
                 float* att, float* out) {
    const int hd = cfg->dim / cfg->num_heads;
    const int half = hd / 2;
    const int kv_dim = hd * cfg->num_kv_heads;
    /* GEMMs write rows start..start+n-1 un-rotated, :545-561 */
    for (int b = 0; b < n; ++b) {
        memcpy(kv + orc_kv_offset(cfg, layer, 0, start + b),
               k + (size_t)b * kv_dim, sizeof(float) * kv_dim);
        memcpy(kv + orc_kv_offset(cfg, layer, 1, start + b),
               v + (size_t)b * kv_dim, sizeof(float) * kv_dim);
    }
    memcpy(q_rot, q, sizeof(float) * (size_t)n * cfg->dim);
    /* per-row loop, :563-593 */
    for (int b = 0; b < n; ++b) {
        const int pos = start + b;
        const float* c = cos_tab + (size_t)pos * half;
        const float* s = sin_tab + (size_t)pos * half;
        float* qb = q_rot + (size_t)b * cfg->dim;
        orc_apply_rope_cached(qb, cfg->dim, c, s, hd);
        orc_apply_rope_cached(kv + orc_kv_offset(cfg, layer, 0, pos), kv_dim,
                              c, s, hd);
        orc_attention_jit(qb, kv + orc_kv_offset(cfg, layer, 0, 0),
                          kv + orc_kv_offset(cfg, layer, 1, 0), att,
                          out + (size_t)b * cfg->dim, cfg, pos);
    }
}

void orc_attention_f64(const float* q, const float* k_cache,
                       const float* v_cache, double* out,
                       const orc_config* cfg, int pos) {
    const int hd = cfg->dim / cfg->num_heads;
    const int kv_dim = hd * cfg->num_kv_heads;
    const int kv_mul = cfg->num_heads / cfg->num_kv_heads;
    const size_t seq_len = (size_t)pos + 1;
    const double scale = 1.0 / sqrt((double)hd);
    double* s = (double*)malloc(sizeof(double) * seq_len);
    if (!s) return;
    for (int h = 0; h < cfg->num_heads; ++h) {
        const size_t kv_off = (size_t)(h / kv_mul) * hd;
        double m = -INFINITY;
        for (size_t t = 0; t < seq_len; ++t) {
            double dot = 0.0;
            for (int i = 0; i < hd; ++i)
                dot += (double)q[(size_t)h * hd + i] *
                       (double)k_cache[t * kv_dim + kv_off + i];
            s[t] = dot * scale;
            if (s[t] > m) m = s[t];
        }
        double sum = 0.0;
        for (size_t t = 0; t < seq_len; ++t) {
            s[t] = exp(s[t] - m);
            sum += s[t];
        }
        for (int i = 0; i < hd; ++i) {
            double acc = 0.0;
            for (size_t t = 0; t < seq_len; ++t)
                acc += s[t] * (double)v_cache[t * kv_dim + kv_off + i];
            out[(size_t)h * hd + i] = acc / sum;
        }
    }
    free(s);
}
