// Host side of slm_layer.h: the JIT normalisation / activation kernels and
// the whole transformer block around the attention path.
#include "../../include/slm_layer.h"

#include <stdint.h>

#include <string>

#include "slm_host.h"

using namespace slm_host;

namespace {

// An output must not overlap an input (io_slices / io2_slices,
// arena.rs:154-208) nor the KV cache.
int check_io(slm_attn_ctx* c, const float* out, size_t out_floats,
             std::initializer_list<std::pair<const void*, size_t>> ins) {
    for (const auto& in : ins)
        if (in.first && overlaps(out, out_floats * 4, in.first, in.second * 4))
            return fail(c, SLM_ERR_ALIAS, "out must not overlap an input");
    if (overlaps(out, out_floats * 4, c->kv, c->kv_floats * 4))
        return fail(c, SLM_ERR_ALIAS, "out must not overlap the KV cache");
    return SLM_OK;
}

slm::Q8Out q8_out(slm_attn_ctx* c, int nb) {
    return slm::Q8Out{c->q8_q, c->q8_d, c->q8_s, nb, slm::q4_scale_stride(nb)};
}

int norm_common(slm_attn_ctx* c, const float* x, const float* w, int rows, int n, float eps,
                float* out) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    if (rows < 0 || n < 1 || n > slm::norm_max_n())
        return fail(c, SLM_ERR_SHAPE, "rows must be >= 0 and 1 <= n <= 16384");
    if (rows == 0) return SLM_OK;
    int rc;
    if ((rc = check_dev_ptrs(c, {x, out})) || (w && (rc = check_dev_ptrs(c, {w}))))
        return rc;
    const size_t total = (size_t)rows * n;
    if ((rc = check_io(c, out, total, {{x, total}, {w, w ? (size_t)n : 0}}))) return rc;
    if (n % 4 != 0 && rows > 1)
        return fail(c, SLM_ERR_SHAPE, "rows of n % 4 != 0 must be normalized one at a time");
    Timed t(c, SLM_K_NORM);
    hipError_t e = slm::launch_rmsnorm(x, n, w, rows, n, eps, out, n, slm::Q8Out{}, c->stream);
    t.done();
    return launch_status(c, e, "norm kernel launch");
}

int check_weights(slm_attn_ctx* c, const slm_layer_weights* w, int* hidden) {
    const slm::Shape& s = c->shape;
    if (!w) return fail(c, SLM_ERR_ARG, "weights is NULL");
    int rc;
    if ((rc = check_matrix(c, w->wq, s.dim, s.dim, "wq")) ||
        (rc = check_matrix(c, w->wk, s.kv_dim, s.dim, "wk")) ||
        (rc = check_matrix(c, w->wv, s.kv_dim, s.dim, "wv")) ||
        (rc = check_matrix(c, w->wo, s.dim, s.dim, "wo")))
        return rc;
    if (!w->w_gate) return fail(c, SLM_ERR_ARG, "w_gate is NULL");
    const int h = w->w_gate->rows;
    if (h % 32 != 0 || h > slm::q4_max_cols())
        return fail(c, SLM_ERR_SHAPE, "hidden_dim must be a multiple of 32, at most 16384");
    if ((rc = check_matrix(c, w->w_gate, h, s.dim, "w_gate")) ||
        (rc = check_matrix(c, w->w_up, h, s.dim, "w_up")) ||
        (rc = check_matrix(c, w->w_down, s.dim, h, "w_down")) ||
        (rc = check_dev_ptrs(c, {w->rms_att, w->rms_ffn})))
        return rc;
    *hidden = h;
    return SLM_OK;
}

int run(slm_attn_ctx* c, hipError_t e, const char* what) { return launch_status(c, e, what); }

}  // namespace

extern "C" {

int slm_rmsnorm_dev(slm_attn_ctx* c, const float* x, const float* w, int32_t rows, int32_t n,
                    float eps, float* out) {
    if (c && !w) return fail(c, SLM_ERR_ARG, "w is NULL");
    return norm_common(c, x, w, rows, n, eps, out);
}

int slm_l2_norm_dev(slm_attn_ctx* c, const float* x, int32_t rows, int32_t n, float eps,
                    float* out) {
    return norm_common(c, x, nullptr, rows, n, eps, out);
}

int slm_swiglu_dev(slm_attn_ctx* c, const float* gate, const float* up, int64_t n, float* out) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    if (n < 0 || n > (int64_t)INT32_MAX * 32) return fail(c, SLM_ERR_SHAPE, "bad length");
    if (n == 0) return SLM_OK;
    int rc;
    if ((rc = check_dev_ptrs(c, {gate, up, out})) ||
        (rc = check_io(c, out, (size_t)n, {{gate, (size_t)n}, {up, (size_t)n}})))
        return rc;
    Timed t(c, SLM_K_ELEM);
    hipError_t e = slm::launch_swiglu(gate, up, (long)n, 0, out, slm::Q8Out{}, c->stream);
    t.done();
    return launch_status(c, e, "swiglu kernel launch");
}

int slm_residual_add_dev(slm_attn_ctx* c, const float* a, const float* b, int64_t n, float* out) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    if (n < 0) return fail(c, SLM_ERR_SHAPE, "bad length");
    if (n == 0) return SLM_OK;
    int rc;
    if ((rc = check_dev_ptrs(c, {a, b, out})) ||
        (rc = check_io(c, out, (size_t)n, {{a, (size_t)n}, {b, (size_t)n}})))
        return rc;
    Timed t(c, SLM_K_ELEM);
    hipError_t e = slm::launch_add(a, b, (long)n, out, c->stream);
    t.done();
    return launch_status(c, e, "add kernel launch");
}

int slm_layer_forward_dev(slm_attn_ctx* c, int32_t layer, int32_t start, int32_t n,
                          const slm_layer_weights* w, float rms_eps, float* x) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    const slm::Shape& s = c->shape;
    int rc, hidden = 0;
    if ((rc = check_layer(c, layer)) || (rc = check_batch(c, start, n)) ||
        (rc = check_weights(c, w, &hidden)) || (rc = check_dev_ptrs(c, {x})))
        return rc;
    const size_t nd = (size_t)n * s.dim;
    if (overlaps(x, nd * 4, c->kv, c->kv_floats * 4))
        return fail(c, SLM_ERR_ALIAS, "x must not overlap the KV cache");
    const int nb = s.dim / 32, nbh = hidden / 32;
    const size_t per_row = (size_t)s.dim + 2 * (size_t)s.kv_dim;
    if ((rc = ensure_q8(c, (size_t)n, nbh > nb ? nbh : nb)) ||
        (rc = ensure_buffer(c, &c->qkv, &c->qkv_floats, (size_t)n * per_row,
                            "hipMalloc(qkv rows)")) ||
        (rc = ensure_buffer(c, &c->blk_att, &c->blk_att_floats, nd, "hipMalloc(block rows)")) ||
        (rc = ensure_buffer(c, &c->blk_mid, &c->blk_mid_floats, nd, "hipMalloc(block rows)")) ||
        (rc = ensure_buffer(c, &c->blk_hid, &c->blk_hid_floats, (size_t)n * 2 * hidden,
                            "hipMalloc(hidden rows)")))
        return rc;
    hipStream_t st = c->stream;
    float* q = c->qkv;
    float* k = q + nd;
    float* v = k + (size_t)n * s.kv_dim;
    float* att = c->blk_att;
    float* x_mid = c->blk_mid;
    float* hb = c->blk_hid;                      // gate rows [n][hidden]
    float* hb2 = hb + (size_t)n * hidden;        // up rows
    const bool one = n == 1;

    // attention RMSNorm straight to Q8_0 blocks (transformer.rs:411 / 519-527)
    {
        Timed t(c, SLM_K_NORM);
        hipError_t e = slm::launch_rmsnorm(x, s.dim, w->rms_att, n, s.dim, rms_eps, nullptr, 0,
                                           q8_out(c, nb), st);
        t.done();
        if ((rc = run(c, e, "rmsnorm kernel launch"))) return rc;
    }
    // q, k, v (:413-417 / 530-561)
    {
        const slm::Q4Job jobs[3] = {q4_job(w->wq, q), q4_job(w->wk, k), q4_job(w->wv, v)};
        Timed t(c, SLM_K_GEMM);
        hipError_t e = one ? slm::launch_q4_gemv_q8(jobs, 3, c->q8_q, c->q8_d, c->q8_s, nb, st)
                           : slm::launch_q4_gemm(jobs, 3, c->q8_q, c->q8_d, nb, n, st);
        t.done();
        if ((rc = run(c, e, "q4 projection kernel launch"))) return rc;
    }
    // RoPE, KV append, attention into the attention rows (:419-443 / 563-593)
    if (one) {
        if ((rc = do_decode(c, layer, start, q, k, v, att, true))) return rc;
    } else {
        if ((rc = do_append(c, layer, start, n, k, v)) ||
            (rc = do_attend(c, layer, start, n, q, att, true)))
            return rc;
    }
    // x_mid = x + Wo . att (:445-446 / 595-605)
    if ((rc = project(c, w->wo, att, n, x_mid, x))) return rc;
    // FFN RMSNorm to Q8_0 (:448-454 / 607-615)
    {
        Timed t(c, SLM_K_NORM);
        hipError_t e = slm::launch_rmsnorm(x_mid, s.dim, w->rms_ffn, n, s.dim, rms_eps, nullptr,
                                           0, q8_out(c, nb), st);
        t.done();
        if ((rc = run(c, e, "rmsnorm kernel launch"))) return rc;
    }
    // gate and up (:456-473 / 617-636)
    {
        const slm::Q4Job jobs[2] = {q4_job(w->w_gate, hb), q4_job(w->w_up, hb2)};
        Timed t(c, SLM_K_GEMM);
        hipError_t e = one ? slm::launch_q4_gemv_q8(jobs, 2, c->q8_q, c->q8_d, c->q8_s, nb, st)
                           : slm::launch_q4_gemm(jobs, 2, c->q8_q, c->q8_d, nb, n, st);
        t.done();
        if ((rc = run(c, e, "q4 projection kernel launch"))) return rc;
    }
    // SwiGLU straight to Q8_0 (:475 / 638)
    {
        Timed t(c, SLM_K_ELEM);
        hipError_t e = slm::launch_swiglu(hb, hb2, (long)n * hidden, hidden, nullptr,
                                          q8_out(c, nbh), st);
        t.done();
        if ((rc = run(c, e, "swiglu kernel launch"))) return rc;
    }
    // x = x_mid + W_down . act (:477-486 / 640-650)
    {
        const slm::Q4Job job = q4_job(w->w_down, x, x_mid);
        Timed t(c, SLM_K_GEMM);
        hipError_t e = one ? slm::launch_q4_gemv_q8(&job, 1, c->q8_q, c->q8_d, c->q8_s, nbh, st)
                           : slm::launch_q4_gemm(&job, 1, c->q8_q, c->q8_d, nbh, n, st);
        t.done();
        if ((rc = run(c, e, "q4 projection kernel launch"))) return rc;
    }
    return SLM_OK;
}

}  // extern "C"
