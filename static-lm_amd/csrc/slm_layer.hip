// Host side of slm_layer.h: the JIT normalisation / activation kernels and
// the whole transformer block around the attention path.
#include "../../include/slm_layer.h"

#include <stdint.h>

#include <string>

#include <algorithm>

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
    // the one-token projections read a whole dim-long row per workgroup
    if (s.dim > slm::q4_max_cols())
        return fail(c, SLM_ERR_SHAPE, "dim above 16384 is not compiled for the projections");
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
        (n == 1 && (rc = ensure_q8x(c, 1, nbh))) ||
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

    // attention RMSNorm (transformer.rs:411 / 519-527), then q, k, v
    // (:413-417 / 530-561): for one token the projection normalizes the row
    // itself, for a batch the norm writes Q8_0 blocks for the GEMM
    {
        const slm::Q4Job jobs[3] = {q4_job(w->wq, q), q4_job(w->wk, k), q4_job(w->wv, v)};
        if (!one) {
            Timed t(c, SLM_K_NORM);
            hipError_t e = slm::launch_rmsnorm(x, s.dim, w->rms_att, n, s.dim, rms_eps, nullptr,
                                               0, q8_out(c, nb), st);
            t.done();
            if ((rc = run(c, e, "rmsnorm kernel launch"))) return rc;
        }
        Timed t(c, SLM_K_GEMM);
        hipError_t e = one ? slm::launch_q4_gemv_norm(jobs, 3, x, w->rms_att, rms_eps, nb, st)
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
    if (one) {
        // FFN RMSNorm (:448-454), gate and up, SwiGLU (:456-475) in one
        // kernel, act straight to Q8_0 blocks in the second activation buffer
        {
            const slm::Q4Job gate = q4_job(w->w_gate, nullptr), up = q4_job(w->w_up, nullptr);
            const slm::Q8Out act{c->q8x_q, c->q8x_d, c->q8x_s, nbh, slm::q4_scale_stride(nbh)};
            Timed t(c, SLM_K_GEMM);
            hipError_t e = slm::launch_q4_gemv_norm_swiglu(gate, up, x_mid, w->rms_ffn, rms_eps,
                                                           nb, nullptr, act, st);
            t.done();
            if ((rc = run(c, e, "q4 projection kernel launch"))) return rc;
        }
        // x = x_mid + W_down . act (:477-486)
        const slm::Q4Job job = q4_job(w->w_down, x, x_mid);
        Timed t(c, SLM_K_GEMM);
        hipError_t e = slm::launch_q4_gemv_q8(&job, 1, c->q8x_q, c->q8x_d, c->q8x_s, nbh, st);
        t.done();
        return run(c, e, "q4 projection kernel launch");
    }
    // FFN RMSNorm to Q8_0 (:607-615)
    {
        Timed t(c, SLM_K_NORM);
        hipError_t e = slm::launch_rmsnorm(x_mid, s.dim, w->rms_ffn, n, s.dim, rms_eps, nullptr,
                                           0, q8_out(c, nb), st);
        t.done();
        if ((rc = run(c, e, "rmsnorm kernel launch"))) return rc;
    }
    // gate and up (:617-636)
    {
        const slm::Q4Job jobs[2] = {q4_job(w->w_gate, hb), q4_job(w->w_up, hb2)};
        Timed t(c, SLM_K_GEMM);
        hipError_t e = slm::launch_q4_gemm(jobs, 2, c->q8_q, c->q8_d, nb, n, st);
        t.done();
        if ((rc = run(c, e, "q4 projection kernel launch"))) return rc;
    }
    // SwiGLU straight to Q8_0 (:638)
    {
        Timed t(c, SLM_K_ELEM);
        hipError_t e = slm::launch_swiglu(hb, hb2, (long)n * hidden, hidden, nullptr,
                                          q8_out(c, nbh), st);
        t.done();
        if ((rc = run(c, e, "swiglu kernel launch"))) return rc;
    }
    // x = x_mid + W_down . act (:640-650)
    const slm::Q4Job job = q4_job(w->w_down, x, x_mid);
    Timed t(c, SLM_K_GEMM);
    hipError_t e = slm::launch_q4_gemm(&job, 1, c->q8_q, c->q8_d, nbh, n, st);
    t.done();
    return run(c, e, "q4 projection kernel launch");
}

}  // extern "C"

// ---- the whole model ----

namespace {

int check_model(slm_attn_ctx* c, const slm_model_weights* w, int* vocab) {
    const slm::Shape& s = c->shape;
    if (!w || !w->layers) return fail(c, SLM_ERR_ARG, "weights is NULL");
    if (w->num_layers != c->cfg.num_layers)
        return fail(c, SLM_ERR_CONFIG, "layer count mismatch");  // transformer.rs:762-766
    if (s.dim > slm::q4_max_cols())
        return fail(c, SLM_ERR_SHAPE, "dim above 16384 is not compiled for the projections");
    int rc;
    if (!w->token_embd) return fail(c, SLM_ERR_ARG, "token_embd is NULL");
    const int v = w->token_embd->rows;
    if ((rc = check_matrix(c, w->token_embd, v, s.dim, "token_embd")) ||
        (rc = check_matrix(c, w->lm_head, v, s.dim, "lm_head")) ||
        (rc = check_dev_ptrs(c, {w->output_norm})))
        return rc;
    *vocab = v;
    return SLM_OK;
}

int ensure_model(slm_attn_ctx* c, int rows, int vocab) {
    int rc;
    if ((rc = ensure_buffer(c, &c->mdl_x, &c->mdl_x_floats, (size_t)rows * c->shape.dim,
                            "hipMalloc(model rows)")) ||
        (rc = ensure_buffer(c, &c->mdl_tok, &c->mdl_tok_n, (size_t)rows, "hipMalloc(tokens)")) ||
        (rc = ensure_buffer(c, &c->mdl_logits, &c->mdl_logits_n, (size_t)vocab,
                            "hipMalloc(logits)")) ||
        (rc = ensure_buffer(c, &c->mdl_flags, &c->mdl_flags_n, 2, "hipMalloc(flags)")) ||
        (rc = ensure_buffer(c, &c->mdl_parts, &c->mdl_parts_n,
                            (size_t)(vocab + slm::q4_gemv_rows_per_part() - 1) /
                                slm::q4_gemv_rows_per_part(),
                            "hipMalloc(argmax parts)")))
        return rc;
    return SLM_OK;
}

int check_tokens(slm_attn_ctx* c, const int32_t* tokens, int n, int vocab) {
    if (!tokens) return fail(c, SLM_ERR_ARG, "tokens is NULL");
    for (int i = 0; i < n; ++i)
        if (tokens[i] < 0 || tokens[i] >= vocab)
            return fail(c, SLM_ERR_TOKEN, "token_id out of vocabulary bounds");
    return SLM_OK;
}

// Embedding rows of n host tokens into the model rows [0, n).
int embed(slm_attn_ctx* c, const slm_model_weights* w, const int32_t* tokens, int n, int vocab) {
    SLM_HIP(c, hipMemcpyAsync(c->mdl_tok, tokens, (size_t)n * sizeof(int32_t),
                              hipMemcpyHostToDevice, c->stream));
    Timed t(c, SLM_K_ELEM);
    hipError_t e = slm::launch_embed_rows(w->token_embd->qs, w->token_embd->d, c->shape.dim / 32,
                                          vocab, c->mdl_tok, n, c->mdl_x, c->mdl_flags + 1,
                                          c->stream);
    t.done();
    return launch_status(c, e, "embedding kernel launch");
}

int all_layers(slm_attn_ctx* c, const slm_model_weights* w, float eps, int start, int n) {
    for (int l = 0; l < w->num_layers; ++l) {
        const int rc = slm_layer_forward_dev(c, l, start, n, &w->layers[l], eps, c->mdl_x);
        if (rc) return rc;
    }
    return SLM_OK;
}

// Final RMSNorm of model row `row`, lm_head, argmax into mdl_flags[0].
int head_launch(slm_attn_ctx* c, const slm_model_weights* w, float eps, int row, int vocab,
                float* logits) {
    const slm::Shape& s = c->shape;
    const int nb = s.dim / 32;
    float* lg = logits ? logits : c->mdl_logits;
    int rc;
    if ((rc = ensure_q8(c, 1, nb))) return rc;
    {
        Timed t(c, SLM_K_NORM);
        hipError_t e = slm::launch_rmsnorm(c->mdl_x + (size_t)row * s.dim, s.dim, w->output_norm,
                                           1, s.dim, eps, nullptr, 0, q8_out(c, nb), c->stream);
        t.done();
        if ((rc = run(c, e, "rmsnorm kernel launch"))) return rc;
    }
    // lm_head; each workgroup also leaves the best of its rows, so the argmax
    // (sample_argmax, transformer.rs:654-666) merges thousands of parts, not
    // the whole vocabulary
    const int n_parts = (vocab + slm::q4_gemv_rows_per_part() - 1) / slm::q4_gemv_rows_per_part();
    {
        const slm::Q4Job job = q4_job(w->lm_head, lg);
        Timed t(c, SLM_K_GEMM);
        hipError_t e = slm::launch_q4_gemv_q8_argmax(job, c->q8_q, c->q8_d, c->q8_s, nb,
                                                     c->mdl_parts, c->stream);
        t.done();
        if ((rc = run(c, e, "q4 projection kernel launch"))) return rc;
    }
    {
        Timed t(c, SLM_K_ELEM);
        hipError_t e = slm::launch_argmax_parts(c->mdl_parts, n_parts, lg, c->mdl_flags, c->stream);
        t.done();
        if ((rc = run(c, e, "argmax kernel launch"))) return rc;
    }
    return SLM_OK;
}

// The same, then *next on the host.
int head(slm_attn_ctx* c, const slm_model_weights* w, float eps, int row, int vocab,
         float* logits, int32_t* next) {
    int rc;
    if ((rc = head_launch(c, w, eps, row, vocab, logits))) return rc;
    int32_t h[2] = {0, 0};
    SLM_HIP(c, hipMemcpyAsync(h, c->mdl_flags, sizeof h, hipMemcpyDeviceToHost, c->stream));
    SLM_HIP(c, hipStreamSynchronize(c->stream));
    if (h[1]) return fail(c, SLM_ERR_TOKEN, "token_id out of vocabulary bounds");
    *next = h[0];
    return SLM_OK;
}

// One decode step of generate on the device alone: the token is the previous
// step's argmax (mdl_flags[0], always in the vocabulary), the new one goes to
// mdl_flags[0] and, asynchronously, to the pinned slot tok_pin[slot], with
// tok_ev[slot] recorded after it.
int decode_step(slm_attn_ctx* c, const slm_model_weights* w, float eps, int pos, int vocab,
                int slot) {
    int rc;
    {
        Timed t(c, SLM_K_ELEM);
        hipError_t e = slm::launch_embed_rows(w->token_embd->qs, w->token_embd->d,
                                              c->shape.dim / 32, vocab, c->mdl_flags, 1,
                                              c->mdl_x, c->mdl_flags + 1, c->stream);
        t.done();
        if ((rc = launch_status(c, e, "embedding kernel launch"))) return rc;
    }
    if ((rc = all_layers(c, w, eps, pos, 1)) || (rc = head_launch(c, w, eps, 0, vocab, nullptr)))
        return rc;
    SLM_HIP(c, hipMemcpyAsync(c->tok_pin + slot, c->mdl_flags, sizeof(int32_t),
                              hipMemcpyDeviceToHost, c->stream));
    SLM_HIP(c, hipEventRecord(c->tok_ev[slot], c->stream));
    return SLM_OK;
}

int ensure_token_readback(slm_attn_ctx* c) {
    if (!c->tok_pin) SLM_HIP(c, hipHostMalloc(reinterpret_cast<void**>(&c->tok_pin),
                                              2 * sizeof(int32_t), hipHostMallocDefault));
    for (hipEvent_t& e : c->tok_ev)
        if (!e) SLM_HIP(c, hipEventCreateWithFlags(&e, hipEventDisableTiming));
    return SLM_OK;
}

// The K and V rows at `pos` of layers 0..layers-1 to (save) or from
// (restore) gen_rows: in the [layer][K|V][msl][kv_dim] region those 2 * layers
// rows are msl * kv_dim floats apart, one launch.
int gen_rows_copy(slm_attn_ctx* c, int pos, int layers, bool save) {
    Timed t(c, SLM_K_ELEM);
    hipError_t e = slm::launch_kv_rows_copy(c->shape, c->kv + (size_t)pos * c->shape.kv_dim,
                                            c->gen_rows, 2 * layers, save, c->stream);
    t.done();
    return launch_status(c, e, "K/V row copy kernel launch");
}

int model_prefill(slm_attn_ctx* c, const slm_model_weights* w, float eps, const int32_t* tokens,
                  int n, int start, float* logits, int32_t* next) {
    int rc, vocab = 0;
    if ((rc = check_model(c, w, &vocab)) || (rc = check_batch(c, start, n))) return rc;
    if (!next) return fail(c, SLM_ERR_ARG, "next_token is NULL");
    if ((rc = check_tokens(c, tokens, n, vocab)) || (rc = ensure_model(c, n, vocab))) return rc;
    if (logits && ((rc = check_dev_ptrs(c, {logits})) ||
                   (rc = check_io(c, logits, (size_t)vocab, {}))))
        return rc;
    SLM_HIP(c, hipMemsetAsync(c->mdl_flags, 0, 2 * sizeof(int32_t), c->stream));
    if ((rc = embed(c, w, tokens, n, vocab)) || (rc = all_layers(c, w, eps, start, n)))
        return rc;
    return head(c, w, eps, n - 1, vocab, logits, next);
}

}  // namespace

extern "C" {

int slm_model_forward_token_dev(slm_attn_ctx* c, const slm_model_weights* w, float rms_eps,
                                int32_t token, int32_t pos, float* logits, int32_t* next_token) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    if (c->capturing) return refuse_capture(c, "slm_model_forward_token_dev");
    int rc;
    if ((rc = check_pos(c, pos))) return rc;
    return model_prefill(c, w, rms_eps, &token, 1, pos, logits, next_token);
}

int slm_model_prefill_dev(slm_attn_ctx* c, const slm_model_weights* w, float rms_eps,
                          const int32_t* tokens, int32_t n, int32_t start, float* logits,
                          int32_t* next_token) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    if (c->capturing) return refuse_capture(c, "slm_model_prefill_dev");
    return model_prefill(c, w, rms_eps, tokens, n, start, logits, next_token);
}

int slm_model_generate_dev(slm_attn_ctx* c, const slm_model_weights* w, float rms_eps,
                           const int32_t* prompt, int32_t n_prompt, int32_t* out_tokens,
                           int32_t max_out, int32_t eos, int32_t* n_out) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    if (c->capturing) return refuse_capture(c, "slm_model_generate_dev");
    if (!n_out) return fail(c, SLM_ERR_ARG, "n_out is NULL");
    *n_out = 0;
    if (max_out <= 0 || n_prompt <= 0) return SLM_OK;  // transformer.rs:862-864
    if (!out_tokens) return fail(c, SLM_ERR_ARG, "out_tokens is NULL");
    if (n_prompt > c->cfg.max_seq_len)  // :866
        return fail(c, SLM_ERR_BATCH, "prompt longer than max_seq_len");
    int32_t next = 0;
    int rc = model_prefill(c, w, rms_eps, prompt, n_prompt, 0, nullptr, &next);
    if (rc) return rc;
    out_tokens[0] = next;
    int generated = 1;
    if (eos >= 0 && next == eos) {
        *n_out = generated;
        return SLM_OK;
    }
    // Greedy decode (:867-897), pipelined: step k's token is read on the host
    // while step k + 1 already runs, so the device never waits for the host.
    // When step k's token is EOS, step k + 1 has already run on it, which the
    // reference never does (it stops before forward_token of the EOS token):
    // that step's token is dropped, and the K/V rows it wrote at position
    // n_prompt + k + 1 are put back from the copy taken before it ran, so the
    // cache ends exactly as the reference leaves it.  (Without an EOS id no
    // step runs ahead of a stop, and no copies are made.)
    const int steps = std::min(max_out - 1, c->cfg.max_seq_len - n_prompt);
    int vocab = 0;
    if ((rc = check_model(c, w, &vocab)) || (rc = ensure_token_readback(c))) return rc;
    const bool may_stop = eos >= 0;
    if (may_stop && (rc = ensure_buffer(c, &c->gen_rows, &c->gen_rows_floats,
                                        (size_t)2 * w->num_layers * c->shape.kv_dim,
                                        "hipMalloc(generate's K/V rows)")))
        return rc;
    for (int k = 0; k <= steps; ++k) {
        // step 0 follows the prompt's token, already known not to be EOS
        if (k < steps && ((k > 0 && may_stop &&
                           (rc = gen_rows_copy(c, n_prompt + k, w->num_layers, true))) ||
                          (rc = decode_step(c, w, rms_eps, n_prompt + k, vocab, k & 1)))) {
            (void)hipStreamSynchronize(c->stream);
            *n_out = generated;
            return rc;
        }
        if (k == 0) continue;
        SLM_HIP(c, hipEventSynchronize(c->tok_ev[(k - 1) & 1]));
        next = c->tok_pin[(k - 1) & 1];
        out_tokens[generated++] = next;
        if (may_stop && next == eos) {
            if (k < steps && (rc = gen_rows_copy(c, n_prompt + k, w->num_layers, false))) {
                (void)hipStreamSynchronize(c->stream);
                *n_out = generated;
                return rc;
            }
            break;
        }
    }
    SLM_HIP(c, hipStreamSynchronize(c->stream));
    *n_out = generated;
    return SLM_OK;
}

int slm_model_embed_dev(slm_attn_ctx* c, const slm_model_weights* w, float rms_eps,
                        const int32_t* tokens, int32_t n, float* out) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    if (c->capturing) return refuse_capture(c, "slm_model_embed_dev");
    const slm::Shape& s = c->shape;
    int rc, vocab = 0;
    if ((rc = check_model(c, w, &vocab)) || (rc = check_batch(c, 0, n)) ||
        (rc = check_tokens(c, tokens, n, vocab)) || (rc = ensure_model(c, n, vocab)) ||
        (rc = check_dev_ptrs(c, {out})) || (rc = check_io(c, out, (size_t)s.dim, {})))
        return rc;
    // normed rows reuse the block's attention-row buffer (free after the layers)
    if ((rc = ensure_buffer(c, &c->blk_att, &c->blk_att_floats, (size_t)n * s.dim,
                            "hipMalloc(block rows)")))
        return rc;
    SLM_HIP(c, hipMemsetAsync(c->mdl_flags, 0, 2 * sizeof(int32_t), c->stream));
    if ((rc = embed(c, w, tokens, n, vocab)) || (rc = all_layers(c, w, rms_eps, 0, n))) return rc;
    hipError_t e;
    {
        Timed t(c, SLM_K_NORM);
        e = slm::launch_rmsnorm(c->mdl_x, s.dim, w->output_norm, n, s.dim, rms_eps, c->blk_att,
                                s.dim, slm::Q8Out{}, c->stream);
        t.done();
        if ((rc = run(c, e, "rmsnorm kernel launch"))) return rc;
    }
    // accum (the block's x_mid buffer, [dim] at least) then its L2 norm
    if ((rc = ensure_buffer(c, &c->blk_mid, &c->blk_mid_floats, (size_t)s.dim,
                            "hipMalloc(block rows)")))
        return rc;
    float* accum = c->blk_mid;
    {
        Timed t(c, SLM_K_ELEM);
        e = slm::launch_mean_pool(c->blk_att, n, s.dim, 1.0f / (float)n, accum, c->stream);
        t.done();
        if ((rc = run(c, e, "mean pool kernel launch"))) return rc;
    }
    {
        Timed t(c, SLM_K_NORM);
        e = slm::launch_rmsnorm(accum, s.dim, nullptr, 1, s.dim, rms_eps, out, s.dim,
                                slm::Q8Out{}, c->stream);
        t.done();
        if ((rc = run(c, e, "l2 norm kernel launch"))) return rc;
    }
    int32_t bad = 0;
    SLM_HIP(c, hipMemcpyAsync(&bad, c->mdl_flags + 1, sizeof bad, hipMemcpyDeviceToHost,
                              c->stream));
    SLM_HIP(c, hipStreamSynchronize(c->stream));
    if (bad) return fail(c, SLM_ERR_TOKEN, "token_id out of vocabulary bounds");
    return SLM_OK;
}

}  // extern "C"
