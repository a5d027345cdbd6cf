// Host side of the slm_attn C ABI: context, argument checks that mirror the
// reference's asserts, RoPE tables, device KV region and kernel dispatch.
#include "../../include/slm_attn.h"
#include "../../include/slm_quant.h"

#include <math.h>
#include <stdint.h>
#include <string.h>

#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "prefill_plan.h"
#include "slm_host.h"
#include "tile_range.h"

// Scratch of slm_attn_decode_xb_dev_noalloc: q | k | v rows of one token,
// then the decode split partials.  Every device the library runs on holds
// its own copy until the process ends; host code uses the per-device
// address hipGetSymbolAddress gives, never the symbol itself.
constexpr size_t kNoAllocScratchFloats = size_t(1) << 18;  // 1 MiB
static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

namespace slm_host {

namespace {

// Address of `scratch` on each device, taken once per device with that
// device current (the first slm_attn_create on it).
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};
std::string g_scratch_err[kMaxDevices];

float* noalloc_scratch_on(int dev, std::string* why) {
    if (dev < 0 || dev >= kMaxDevices) {
        *why = "device index above the no-allocation table";
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev] && g_scratch_err[dev].empty()) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || ptr == nullptr)
            g_scratch_err[dev] = std::string("hipGetSymbolAddress(scratch): ") +
                                 hipGetErrorString(e);
        else
            g_scratch_ptr[dev] = static_cast<float*>(ptr);
    }
    *why = g_scratch_err[dev];
    return g_scratch_ptr[dev];
}

}  // namespace

thread_local std::string g_last_error;

int fail(slm_attn_ctx* c, int code, const std::string& msg) {
    g_last_error = msg;
    if (c) c->err = msg;
    return code;
}

int hip_fail(slm_attn_ctx* c, hipError_t e, const char* what) {
    return fail(c, SLM_ERR_HIP,
                std::string(what) + ": " + hipGetErrorString(e));
}

int refuse_capture(slm_attn_ctx* c, const char* what) {
    return fail(c, SLM_ERR_CAPTURE,
                std::string(what) +
                    ": not allowed while the context's stream is being captured into a graph");
}


// LayerWorkspace::allocate asserts (transformer.rs:81-101).
int validate(const slm_attn_config* cfg, std::string* why) {
    if (!cfg) {
        *why = "config is NULL";
        return SLM_ERR_ARG;
    }
    if (cfg->num_heads <= 0 || cfg->num_kv_heads <= 0) {
        *why = "num_heads and num_kv_heads must be positive";
        return SLM_ERR_CONFIG;
    }
    if (cfg->dim <= 0 || cfg->dim % 32 != 0) {
        *why = "dim must be a multiple of 32";
        return SLM_ERR_CONFIG;
    }
    if (cfg->dim % cfg->num_heads != 0) {
        *why = "dim must be divisible by num_heads";
        return SLM_ERR_CONFIG;
    }
    if (cfg->num_heads % cfg->num_kv_heads != 0) {
        *why = "num_heads must be divisible by num_kv_heads";
        return SLM_ERR_CONFIG;
    }
    const int hd = cfg->dim / cfg->num_heads;
    if (hd % 2 != 0) {
        *why = "head_dim must be even for RoPE rotation";
        return SLM_ERR_CONFIG;
    }
    if ((hd * cfg->num_kv_heads) % 32 != 0) {
        *why = "kv_dim must be a multiple of 32";
        return SLM_ERR_CONFIG;
    }
    if (cfg->max_seq_len <= 0 || cfg->num_layers <= 0) {
        *why = "max_seq_len and num_layers must be positive";
        return SLM_ERR_CONFIG;
    }
    if (!(cfg->rope_theta > 0.0f) || !isfinite(cfg->rope_theta)) {
        *why = "rope_theta must be positive and finite";
        return SLM_ERR_CONFIG;
    }
    const size_t kv_floats = (size_t)cfg->num_layers * 2 *
                             (size_t)cfg->max_seq_len * (size_t)hd *
                             (size_t)cfg->num_kv_heads;
    if (kv_floats / 2 / (size_t)cfg->num_layers > (size_t)INT32_MAX * 4) {
        *why = "KV region too large";
        return SLM_ERR_CONFIG;
    }
    return SLM_OK;
}

// RoPE tables exactly as transformer.rs:124-133 computes them: f32 exponent
// (2j)/hd, freq = 1 / theta^exponent through powf, angle = pos * freq in f32,
// then sinf/cosf.  Host libm, never the device, so the tables are the
// reference's own numbers.
void rope_tables(int hd, int msl, float theta, std::vector<float>* cos_out,
                 std::vector<float>* sin_out) {
    const int half = hd / 2;
    const float hd_f = (float)hd;
    std::vector<float> freq(half);
    for (int j = 0; j < half; ++j) {
        const float expo = (float)(2 * j) / hd_f;
        freq[j] = 1.0f / powf(theta, expo);
    }
    cos_out->resize((size_t)msl * half);
    sin_out->resize((size_t)msl * half);
    for (int pos = 0; pos < msl; ++pos) {
        const float pos_f = (float)pos;
        for (int j = 0; j < half; ++j) {
            const float a = pos_f * freq[j];
            (*cos_out)[(size_t)pos * half + j] = cosf(a);
            (*sin_out)[(size_t)pos * half + j] = sinf(a);
        }
    }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

bool overlaps(const void* a, size_t a_bytes, const void* b, size_t b_bytes) {
    const uintptr_t a0 = (uintptr_t)a, b0 = (uintptr_t)b;
    return a0 < b0 + b_bytes && b0 < a0 + a_bytes;
}

hipEvent_t take_event(slm_attn_ctx* c) {
    if (!c->spare_events.empty()) {
        hipEvent_t e = c->spare_events.back();
        c->spare_events.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}


float* k_base(slm_attn_ctx* c, int layer) {
    return c->kv + (size_t)(2 * layer) * c->cfg.max_seq_len * c->shape.kv_dim;
}
float* v_base(slm_attn_ctx* c, int layer) {
    return c->kv +
           (size_t)(2 * layer + 1) * c->cfg.max_seq_len * c->shape.kv_dim;
}

int check_layer(slm_attn_ctx* c, int layer) {
    if (layer < 0 || layer >= c->cfg.num_layers)
        return fail(c, SLM_ERR_LAYER, "layer index out of range");
    return SLM_OK;
}

int check_pos(slm_attn_ctx* c, int pos) {
    if (pos < 0 || pos >= c->cfg.max_seq_len)
        return fail(c, SLM_ERR_POS, "sequence position out of bounds");
    return SLM_OK;
}

int check_batch(slm_attn_ctx* c, int start, int n) {
    if (n <= 0 || start < 0 || (long)start + n > c->cfg.max_seq_len)
        return fail(c, SLM_ERR_BATCH,
                    "batch must be non-empty and start + n <= max_seq_len");
    return SLM_OK;
}

int check_dev_ptrs(slm_attn_ctx* c, std::initializer_list<const void*> ps) {
    for (const void* p : ps) {
        if (!p) return fail(c, SLM_ERR_ARG, "NULL buffer");
        if (!aligned16(p))
            return fail(c, SLM_ERR_ARG, "device buffers must be 16-byte aligned");
    }
    return SLM_OK;
}

// out must not alias an input or the KV region (arena.rs:272-280).
int check_out_alias(slm_attn_ctx* c, const float* out, size_t out_floats,
                    std::initializer_list<std::pair<const float*, size_t>> ins,
                    bool device) {
    for (const auto& in : ins)
        if (in.first && overlaps(out, out_floats * 4, in.first, in.second * 4))
            return fail(c, SLM_ERR_ALIAS,
                        "out must not overlap q, k, v or the KV cache");
    if (device && overlaps(out, out_floats * 4, c->kv, c->kv_floats * 4))
        return fail(c, SLM_ERR_ALIAS,
                    "out must not overlap q, k, v or the KV cache");
    return SLM_OK;
}

// Inputs of an entry point that appends to the cache must not overlap the
// KV region: the kernels write row pos (rows start..start+n-1) while other
// workgroups read the inputs, so a k taken from the cache row it is appended
// to would be read after its rotation by some workgroups and before it by
// others.  (The reference's GEMV writes k into the cache row and rotates it
// there, transformer.rs:416-428; here k and v come from staging buffers.)
int check_in_not_kv(slm_attn_ctx* c,
                    std::initializer_list<std::pair<const float*, size_t>> ins) {
    for (const auto& in : ins)
        if (in.first && overlaps(in.first, in.second * 4, c->kv, c->kv_floats * 4))
            return fail(c, SLM_ERR_ALIAS,
                        "q, k and v of an appending call must not overlap the KV cache");
    return SLM_OK;
}

int launch_status(slm_attn_ctx* c, hipError_t e, const char* what) {
    if (e != hipSuccess) return hip_fail(c, e, what);
    return SLM_OK;
}

int do_append(slm_attn_ctx* c, int layer, int pos0, int n, const float* k,
              const float* v) {
    Timed t(c, SLM_K_APPEND);
    hipError_t e = slm::launch_kv_append(c->shape, k, v, k_base(c, layer),
                                         v_base(c, layer), c->cos_t, c->sin_t,
                                         pos0, n, c->stream);
    t.done();
    return launch_status(c, e, "kv_append kernel launch");
}

// Single-token decode at pos: with k_new/v_new the KV row is appended and q
// is rotated at pos inside the kernel; without them q is already rotated and
// row pos is read from the cache.
int do_decode_in(slm_attn_ctx* c, int layer, int pos, const float* q, const float* k_new,
                 const float* v_new, float* out, bool rotate, float* part_o, float* part_ml,
                 bool timed) {
    const slm::Shape& s = c->shape;
    int ns = 1, tile = 1;
    slm::decode_split_policy(s, pos + 1, &ns, &tile);
    slm::DecodeArgs a{q,
                      k_new,
                      v_new,
                      k_base(c, layer),
                      v_base(c, layer),
                      rotate ? c->cos_t : nullptr,
                      rotate ? c->sin_t : nullptr,
                      out,
                      part_o,
                      part_ml,
                      pos,
                      ns};
    if (!timed) {
        hipError_t e = slm::launch_decode(s, a, c->stream);
        if (e != hipSuccess) return hip_fail(c, e, "decode kernel launch");
        if (ns == 1) return SLM_OK;
        return launch_status(c, slm::launch_decode_combine(s, a, c->stream),
                             "decode combine kernel launch");
    }
    {
        // the launch stamps the events at the kernel's own start and end
        Timed t(c, SLM_K_DECODE, /*in_launch=*/true);
        a.ev_start = t.b;
        a.ev_stop = t.e;
        hipError_t e = slm::launch_decode(s, a, c->stream);
        t.done_in_launch(e == hipSuccess);
        if (e != hipSuccess) return hip_fail(c, e, "decode kernel launch");
    }
    if (ns == 1) return SLM_OK;
    Timed t(c, SLM_K_COMBINE, /*in_launch=*/true);
    a.ev_start = t.b;
    a.ev_stop = t.e;
    hipError_t e = slm::launch_decode_combine(s, a, c->stream);
    t.done_in_launch(e == hipSuccess);
    return launch_status(c, e, "decode combine kernel launch");
}

int do_decode(slm_attn_ctx* c, int layer, int pos, const float* q, const float* k_new,
              const float* v_new, float* out, bool rotate) {
    return do_decode_in(c, layer, pos, q, k_new, v_new, out, rotate, c->part_o, c->part_ml,
                        true);
}

// Attention of rows b < n at positions start + b over cache rows 0..start+b.
// rotate: q is un-rotated and the kernels apply RoPE at each row's position.
int do_attend(slm_attn_ctx* c, int layer, int start, int n, const float* q,
              float* out, bool rotate) {
    const slm::Shape& s = c->shape;
    if (n == 1) return do_decode(c, layer, start, q, nullptr, nullptr, out, rotate);
    slm::PrefillArgs pa{q,          k_base(c, layer), v_base(c, layer),
                        rotate ? c->cos_t : nullptr,
                        rotate ? c->sin_t : nullptr, out, start, n};
    Timed t(c, SLM_K_PREFILL);
    hipError_t e = slm::launch_prefill_mfma(s, pa, c->stream);
    t.done();
    return launch_status(c, e, "prefill kernel launch");
}

int ensure_stage(slm_attn_ctx* c, size_t floats) {
    if (c->stage_floats >= floats) return SLM_OK;
    if (c->capturing) return refuse_capture(c, "host staging buffer");
    if (c->stage) {
        SLM_HIP(c, hipStreamSynchronize(c->stream));
        SLM_HIP(c, hipFree(c->stage));
        c->stage = nullptr;
        c->stage_floats = 0;
    }
    SLM_HIP(c, hipMalloc(&c->stage, floats * sizeof(float)));
    c->stage_floats = floats;
    return SLM_OK;
}


// Q8_0 activations of n rows of nb blocks: i8 [n][nb][32] and f32 scales
// [n][q4_scale_stride(nb)].
int ensure_q8(slm_attn_ctx* c, size_t n, int nb) {
    const size_t blocks = n * (size_t)slm::q4_scale_stride(nb);  // covers both
    size_t have_q = c->q8_blocks * 8, have_d = c->q8_blocks, have_s = c->q8_blocks;
    int rc = ensure_buffer(c, &c->q8_q, &have_q, blocks * 8, "hipMalloc(q8 activations)");
    if (rc) return rc;
    rc = ensure_buffer(c, &c->q8_d, &have_d, blocks, "hipMalloc(q8 scales)");
    if (rc) return rc;
    rc = ensure_buffer(c, &c->q8_s, &have_s, blocks, "hipMalloc(q8 sums)");
    if (rc) return rc;
    if (blocks > c->q8_blocks) c->q8_blocks = blocks;
    return SLM_OK;
}

int ensure_q8x(slm_attn_ctx* c, size_t n, int nb) {
    const size_t blocks = n * (size_t)slm::q4_scale_stride(nb);
    size_t have_q = c->q8x_blocks * 8, have_d = c->q8x_blocks, have_s = c->q8x_blocks;
    int rc = ensure_buffer(c, &c->q8x_q, &have_q, blocks * 8, "hipMalloc(q8 activations)");
    if (rc) return rc;
    rc = ensure_buffer(c, &c->q8x_d, &have_d, blocks, "hipMalloc(q8 scales)");
    if (rc) return rc;
    rc = ensure_buffer(c, &c->q8x_s, &have_s, blocks, "hipMalloc(q8 sums)");
    if (rc) return rc;
    if (blocks > c->q8x_blocks) c->q8x_blocks = blocks;
    return SLM_OK;
}

int check_matrix(slm_attn_ctx* c, const slm_q4_matrix* m, int rows, int cols, const char* name) {
    if (!m) return fail(c, SLM_ERR_ARG, std::string(name) + " is NULL");
    if (m->device != c->device)
        return fail(c, SLM_ERR_DEVICE, std::string(name) + " lives on another device");
    if ((rows >= 0 && m->rows != rows) || m->cols != cols)
        return fail(c, SLM_ERR_SHAPE, std::string(name) + " has the wrong shape");
    return SLM_OK;
}

slm::Q4Job q4_job(const slm_q4_matrix* m, float* out, const float* res) {
    return slm::Q4Job{m->qs, m->d, out, m->rows, m->rows, res};
}

// One projection of `batch` rows of x [batch][cols]: GEMV (fused
// quantization) for a few rows, else quantize + MFMA GEMM.  out (+ res).
int project(slm_attn_ctx* c, const slm_q4_matrix* w, const float* x, int batch, float* out,
            const float* res) {
    const slm::Q4Job job = q4_job(w, out, res);
    const int nb = w->cols / 32;
    if (slm::q4_gemv_takes(nb, batch)) {
        Timed t(c, SLM_K_GEMM);
        hipError_t e = slm::launch_q4_gemv(&job, 1, x, nb, batch, c->stream);
        t.done();
        return launch_status(c, e, "q4 gemv kernel launch");
    }
    int rc;
    if ((rc = ensure_q8(c, (size_t)batch, nb))) return rc;
    {
        Timed t(c, SLM_K_QUANT);
        hipError_t e = slm::launch_quantize_q8_soa(x, batch, nb, c->q8_q, c->q8_d, nullptr, c->stream);
        t.done();
        if (e != hipSuccess) return hip_fail(c, e, "q8 quantize kernel launch");
    }
    Timed t(c, SLM_K_GEMM);
    hipError_t e = slm::launch_q4_gemm(&job, 1, c->q8_q, c->q8_d, nb, batch, c->stream);
    t.done();
    return launch_status(c, e, "q4 gemm kernel launch");
}

// Checks of a projection + residual call: x [batch][cols], res and out
// [batch][rows]; out may be res itself, otherwise disjoint from it.
int check_residual_args(slm_attn_ctx* c, const slm_q4_matrix* w, const float* x, int batch,
                        const float* res, float* out) {
    int rc;
    if ((rc = check_dev_ptrs(c, {x, res, out}))) return rc;
    const size_t in_b = (size_t)batch * w->cols * 4, out_b = (size_t)batch * w->rows * 4;
    if (overlaps(out, out_b, x, in_b) || overlaps(res, out_b, x, in_b))
        return fail(c, SLM_ERR_ALIAS, "out and res must not overlap x");
    if (res != out && overlaps(out, out_b, res, out_b))
        return fail(c, SLM_ERR_ALIAS, "out must be res itself or not overlap it");
    if (overlaps(out, out_b, c->kv, c->kv_floats * 4))
        return fail(c, SLM_ERR_ALIAS, "out must not overlap the KV cache");
    return SLM_OK;
}

// Attention rows written into xb, then x_mid = x + Wo.xb: the shared tail of
// the *_wo entry points.  xb [n][dim] holds the attention output on return.
int check_wo_args(slm_attn_ctx* c, int n, float* xb, const slm_q4_matrix* wo, const float* x,
                  float* x_mid) {
    const slm::Shape& s = c->shape;
    int rc;
    if ((rc = check_matrix(c, wo, s.dim, s.dim, "wo")) ||
        (rc = check_dev_ptrs(c, {xb, x, x_mid})))
        return rc;
    const size_t b = (size_t)n * s.dim * 4;
    if (overlaps(xb, b, x, b) || overlaps(xb, b, x_mid, b))
        return fail(c, SLM_ERR_ALIAS, "xb must not overlap x or x_mid");
    if (x_mid != x && overlaps(x_mid, b, x, b))
        return fail(c, SLM_ERR_ALIAS, "x_mid must be x itself or not overlap it");
    if (overlaps(x_mid, b, c->kv, c->kv_floats * 4) || overlaps(xb, b, c->kv, c->kv_floats * 4))
        return fail(c, SLM_ERR_ALIAS, "xb and x_mid must not overlap the KV cache");
    return SLM_OK;
}

// q | k | v of n rows from xb [n][dim]: GEMV (fused quantization) for a few
// rows, else quantize + MFMA GEMM.  Outputs land in c->qkv.
int project_qkv(slm_attn_ctx* c, int n, const float* xb, const slm_q4_matrix* wq,
                const slm_q4_matrix* wk, const slm_q4_matrix* wv, float** q, float** k,
                float** v) {
    const slm::Shape& s = c->shape;
    int rc;
    if ((rc = check_matrix(c, wq, s.dim, s.dim, "wq")) ||
        (rc = check_matrix(c, wk, s.kv_dim, s.dim, "wk")) ||
        (rc = check_matrix(c, wv, s.kv_dim, s.dim, "wv")))
        return rc;
    const size_t per_row = (size_t)s.dim + 2 * (size_t)s.kv_dim;
    if ((rc = ensure_buffer(c, &c->qkv, &c->qkv_floats, (size_t)n * per_row,
                            "hipMalloc(qkv rows)")))
        return rc;
    *q = c->qkv;
    *k = *q + (size_t)n * s.dim;
    *v = *k + (size_t)n * s.kv_dim;
    const slm::Q4Job jobs[3] = {q4_job(wq, *q), q4_job(wk, *k), q4_job(wv, *v)};
    const int nb = s.dim / 32;
    if (slm::q4_gemv_takes(nb, n)) {
        Timed t(c, SLM_K_GEMM);
        hipError_t e = slm::launch_q4_gemv(jobs, 3, xb, nb, n, c->stream);
        t.done();
        return launch_status(c, e, "q4 gemv kernel launch");
    }
    if ((rc = ensure_q8(c, (size_t)n, nb))) return rc;
    {
        Timed t(c, SLM_K_QUANT);
        hipError_t e = slm::launch_quantize_q8_soa(xb, n, nb, c->q8_q, c->q8_d, nullptr, c->stream);
        t.done();
        if (e != hipSuccess) return hip_fail(c, e, "q8 quantize kernel launch");
    }
    Timed t(c, SLM_K_GEMM);
    hipError_t e = slm::launch_q4_gemm(jobs, 3, c->q8_q, c->q8_d, nb, n, c->stream);
    t.done();
    return launch_status(c, e, "q4 gemm kernel launch");
}

}  // namespace slm_host

using namespace slm_host;

extern "C" {

const char* slm_attn_version(void) { return "slm_attn 0.1 gfx950"; }

const char* slm_attn_last_error(const slm_attn_ctx* ctx) {
    return ctx ? ctx->err.c_str() : g_last_error.c_str();
}

int slm_attn_create(const slm_attn_config* cfg, slm_attn_ctx** out) {
    if (!out) return fail(nullptr, SLM_ERR_ARG, "out is NULL");
    *out = nullptr;
    std::string why;
    int rc = validate(cfg, &why);
    if (rc != SLM_OK) return fail(nullptr, rc, why);
    const int hd = cfg->dim / cfg->num_heads;
    if (!slm::head_dim_supported(hd))
        return fail(nullptr, SLM_ERR_UNSUPPORTED,
                    "head_dim " + std::to_string(hd) +
                        " is not compiled (16, 32, 48, 64, 96, 128, 256)");
    if ((long)hd * cfg->num_kv_heads > slm::kMaxKvDim)
        return fail(nullptr, SLM_ERR_UNSUPPORTED,
                    "kv_dim above " + std::to_string(slm::kMaxKvDim) +
                        " is not supported (the kernels' per-thread tile offsets are 32-bit)");

    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess)
        return fail(nullptr, SLM_ERR_DEVICE,
                    std::string("no HIP device: ") + hipGetErrorString(e));
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess)
        return fail(nullptr, SLM_ERR_DEVICE,
                    std::string("hipGetDeviceProperties: ") +
                        hipGetErrorString(e));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(nullptr, SLM_ERR_DEVICE,
                    std::string("device is ") + prop.gcnArchName +
                        ", this library is built for gfx950 only");

    slm_attn_ctx* c = new (std::nothrow) slm_attn_ctx();
    if (!c) return fail(nullptr, SLM_ERR_HIP, "out of host memory for the context");
    c->cfg = *cfg;
    c->device = dev;
    slm::Shape& s = c->shape;
    s.dim = cfg->dim;
    s.num_heads = cfg->num_heads;
    s.num_kv_heads = cfg->num_kv_heads;
    s.head_dim = hd;
    s.kv_dim = hd * cfg->num_kv_heads;
    s.kv_mul = cfg->num_heads / cfg->num_kv_heads;
    s.half = hd / 2;
    s.max_seq_len = cfg->max_seq_len;
    s.cus = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 1;

    auto bail = [&](int code) {
        slm_attn_destroy(c);
        return code;
    };
    // A blocking stream: ordered with the legacy default stream, so device
    // buffers the caller fills there are ready before the context's kernels
    // read them, and its results before default-stream work reads them.
    e = hipStreamCreateWithFlags(&c->own_stream, hipStreamDefault);
    if (e != hipSuccess) return bail(hip_fail(nullptr, e, "hipStreamCreate"));
    c->stream = c->own_stream;

    c->kv_floats = (size_t)cfg->num_layers * 2 * (size_t)cfg->max_seq_len *
                   (size_t)s.kv_dim;
    e = hipMalloc(&c->kv, c->kv_floats * sizeof(float));
    if (e != hipSuccess) return bail(hip_fail(nullptr, e, "hipMalloc(KV region)"));
    e = hipMemset(c->kv, 0, c->kv_floats * sizeof(float));
    if (e != hipSuccess) return bail(hip_fail(nullptr, e, "hipMemset(KV region)"));

    std::vector<float> ct, st;
    rope_tables(hd, cfg->max_seq_len, cfg->rope_theta, &ct, &st);
    const size_t tbytes = ct.size() * sizeof(float);
    e = hipMalloc(&c->cos_t, tbytes);
    if (e == hipSuccess) e = hipMalloc(&c->sin_t, tbytes);
    if (e == hipSuccess)
        e = hipMemcpy(c->cos_t, ct.data(), tbytes, hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = hipMemcpy(c->sin_t, st.data(), tbytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) return bail(hip_fail(nullptr, e, "RoPE table upload"));

    int max_splits = 1;
    for (int len = 1; len <= cfg->max_seq_len; ++len) {
        int ns = 1, tile = 1;
        slm::decode_split_policy(s, len, &ns, &tile);
        if (ns > max_splits) max_splits = ns;
    }
    c->max_splits = max_splits;
    e = hipMalloc(&c->part_o,
                  (size_t)max_splits * s.num_heads * hd * sizeof(float));
    if (e == hipSuccess)
        e = hipMalloc(&c->part_ml,
                      (size_t)max_splits * s.num_heads * 2 * sizeof(float));
    if (e != hipSuccess) return bail(hip_fail(nullptr, e, "hipMalloc(decode partials)"));
    // set-up of the no-allocation entry point on this device (the context's
    // own calls never need it, so a failure only disables that entry point)
    c->noalloc_scratch = noalloc_scratch_on(dev, &c->noalloc_err);

    *out = c;
    return SLM_OK;
}

void slm_attn_destroy(slm_attn_ctx* c) {
    if (!c) return;
    // Teardown is best effort: errors here have no caller to report to.
    if (c->capturing) {  // an unfinished capture is dropped
        hipGraph_t g = nullptr;
        if (hipStreamEndCapture(c->stream, &g) == hipSuccess && g) (void)hipGraphDestroy(g);
        c->capturing = false;
    }
    if (c->own_stream) (void)hipStreamSynchronize(c->own_stream);
    if (c->stream && c->stream != c->own_stream)
        (void)hipStreamSynchronize(c->stream);
    for (auto& p : c->pending) {
        (void)hipEventDestroy(p.begin);
        (void)hipEventDestroy(p.end);
    }
    for (hipEvent_t e : c->spare_events) (void)hipEventDestroy(e);
    (void)hipFree(c->kv);
    (void)hipFree(c->cos_t);
    (void)hipFree(c->sin_t);
    (void)hipFree(c->part_o);
    (void)hipFree(c->part_ml);
    (void)hipFree(c->stage);
    (void)hipFree(c->q8_q);
    (void)hipFree(c->q8_d);
    (void)hipFree(c->q8_s);
    (void)hipFree(c->q8x_q);
    (void)hipFree(c->q8x_d);
    (void)hipFree(c->q8x_s);
    (void)hipFree(c->qkv);
    (void)hipFree(c->blk_att);
    (void)hipFree(c->blk_mid);
    (void)hipFree(c->blk_hid);
    (void)hipFree(c->mdl_x);
    (void)hipFree(c->mdl_tok);
    (void)hipFree(c->mdl_logits);
    (void)hipFree(c->mdl_flags);
    (void)hipFree(c->mdl_parts);
    (void)hipFree(c->gen_rows);
    if (c->tok_pin) (void)hipHostFree(c->tok_pin);
    for (hipEvent_t e : c->tok_ev)
        if (e) (void)hipEventDestroy(e);
    if (c->own_stream) (void)hipStreamDestroy(c->own_stream);
    delete c;
}

int slm_attn_set_stream(slm_attn_ctx* c, void* stream) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    if (c->capturing) return refuse_capture(c, "slm_attn_set_stream");
    c->stream = stream ? (hipStream_t)stream : c->own_stream;
    return SLM_OK;
}

void* slm_attn_get_stream(const slm_attn_ctx* c) {
    return c ? (void*)c->stream : nullptr;
}

int slm_attn_sync(slm_attn_ctx* c) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    if (c->capturing) return refuse_capture(c, "slm_attn_sync");
    SLM_HIP(c, hipStreamSynchronize(c->stream));
    return SLM_OK;
}

int slm_attn_capture_begin(slm_attn_ctx* c) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    if (c->capturing) return fail(c, SLM_ERR_CAPTURE, "a capture is already in progress");
    if (c->profiling)
        return fail(c, SLM_ERR_CAPTURE, "kernel timing must be off while capturing");
    SLM_HIP(c, hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
    c->capturing = true;
    return SLM_OK;
}

int slm_attn_capture_end(slm_attn_ctx* c, slm_attn_graph** out) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    if (out) *out = nullptr;
    if (!c->capturing) return fail(c, SLM_ERR_CAPTURE, "no capture in progress");
    c->capturing = false;  // the stream leaves capture mode whatever follows
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(c->stream, &g);
    if (e != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        return hip_fail(c, e, "hipStreamEndCapture");
    }
    if (!out) {
        (void)hipGraphDestroy(g);
        return fail(c, SLM_ERR_ARG, "out is NULL (the capture was dropped)");
    }
    hipGraphExec_t x = nullptr;
    e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(g);
        return hip_fail(c, e, "hipGraphInstantiate");
    }
    slm_attn_graph* r = new (std::nothrow) slm_attn_graph{c->device, g, x};
    if (!r) {
        (void)hipGraphExecDestroy(x);
        (void)hipGraphDestroy(g);
        return fail(c, SLM_ERR_HIP, "out of host memory for the graph handle");
    }
    *out = r;
    return SLM_OK;
}

int slm_attn_graph_launch(slm_attn_ctx* c, const slm_attn_graph* g) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    if (c->capturing) return refuse_capture(c, "slm_attn_graph_launch");
    if (!g) return fail(c, SLM_ERR_ARG, "graph is NULL");
    if (g->device != c->device)
        return fail(c, SLM_ERR_DEVICE, "the graph was captured on another device");
    SLM_HIP(c, hipGraphLaunch(g->exec, c->stream));
    return SLM_OK;
}

void slm_attn_graph_destroy(slm_attn_graph* g) {
    if (!g) return;
    (void)hipGraphExecDestroy(g->exec);
    (void)hipGraphDestroy(g->graph);
    delete g;
}

int slm_kv_append_dev(slm_attn_ctx* c, int32_t layer, int32_t pos0, int32_t n,
                      const float* k, const float* v) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    int rc;
    if ((rc = check_layer(c, layer)) || (rc = check_batch(c, pos0, n)) ||
        (rc = check_dev_ptrs(c, {k, v})))
        return rc;
    const size_t kn = (size_t)n * c->shape.kv_dim;
    if ((rc = check_in_not_kv(c, {{k, kn}, {v, kn}}))) return rc;
    return do_append(c, layer, pos0, n, k, v);
}

int slm_rope_apply_dev(slm_attn_ctx* c, float* x, int32_t n, int32_t row_len,
                       int32_t pos0) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    int rc;
    if ((rc = check_batch(c, pos0, n)) || (rc = check_dev_ptrs(c, {x})))
        return rc;
    if (row_len <= 0 || row_len % c->shape.head_dim != 0)
        return fail(c, SLM_ERR_ARG, "row_len must be a multiple of head_dim");
    Timed t(c, SLM_K_ROPE);
    hipError_t e = slm::launch_rope(c->shape, x, n, row_len, pos0, c->cos_t,
                                    c->sin_t, c->stream);
    t.done();
    return launch_status(c, e, "rope kernel launch");
}

int slm_attn_attend_dev(slm_attn_ctx* c, int32_t layer, int32_t pos,
                        const float* q_rot, float* out) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    int rc;
    if ((rc = check_layer(c, layer)) || (rc = check_pos(c, pos)) ||
        (rc = check_dev_ptrs(c, {q_rot, out})) ||
        (rc = check_out_alias(c, out, c->shape.dim, {{q_rot, c->shape.dim}},
                              true)))
        return rc;
    return do_attend(c, layer, pos, 1, q_rot, out, false);
}

int slm_attn_attend_batch_dev(slm_attn_ctx* c, int32_t layer, int32_t start,
                              int32_t n, const float* q_rot, float* out) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    int rc;
    const size_t rows = (size_t)(n > 0 ? n : 0) * c->shape.dim;
    if ((rc = check_layer(c, layer)) || (rc = check_batch(c, start, n)) ||
        (rc = check_dev_ptrs(c, {q_rot, out})) ||
        (rc = check_out_alias(c, out, rows, {{q_rot, rows}}, true)))
        return rc;
    return do_attend(c, layer, start, n, q_rot, out, false);
}

int slm_attn_decode_dev(slm_attn_ctx* c, int32_t layer, int32_t pos,
                        const float* q, const float* k, const float* v,
                        float* out) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    const slm::Shape& s = c->shape;
    int rc;
    if ((rc = check_layer(c, layer)) || (rc = check_pos(c, pos)) ||
        (rc = check_dev_ptrs(c, {q, k, v, out})) ||
        (rc = check_out_alias(c, out, s.dim,
                              {{q, s.dim}, {k, s.kv_dim}, {v, s.kv_dim}},
                              true)) ||
        (rc = check_in_not_kv(c, {{q, s.dim}, {k, s.kv_dim}, {v, s.kv_dim}})))
        return rc;
    return do_decode(c, layer, pos, q, k, v, out, true);
}

int slm_attn_prefill_dev(slm_attn_ctx* c, int32_t layer, int32_t start,
                         int32_t n, const float* q, const float* k,
                         const float* v, float* out) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    const slm::Shape& s = c->shape;
    int rc;
    if ((rc = check_layer(c, layer)) || (rc = check_batch(c, start, n)) ||
        (rc = check_dev_ptrs(c, {q, k, v, out})))
        return rc;
    const size_t qn = (size_t)n * s.dim, kn = (size_t)n * s.kv_dim;
    if ((rc = check_out_alias(c, out, qn, {{q, qn}, {k, kn}, {v, kn}}, true)) ||
        (rc = check_in_not_kv(c, {{q, qn}, {k, kn}, {v, kn}})))
        return rc;
    if ((rc = do_append(c, layer, start, n, k, v))) return rc;
    return do_attend(c, layer, start, n, q, out, true);
}

int slm_attn_decode(slm_attn_ctx* c, int32_t layer, int32_t pos, const float* q,
                    const float* k, const float* v, float* out) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    if (c->capturing) return refuse_capture(c, "slm_attn_decode");
    int rc;
    // the decode asserts, in the reference's order (transformer.rs:404-407)
    if ((rc = check_layer(c, layer)) || (rc = check_pos(c, pos))) return rc;
    return slm_attn_prefill(c, layer, pos, 1, q, k, v, out);
}

int slm_attn_prefill(slm_attn_ctx* c, int32_t layer, int32_t start, int32_t n,
                     const float* q, const float* k, const float* v,
                     float* out) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    if (c->capturing) return refuse_capture(c, "slm_attn_prefill");
    const slm::Shape& s = c->shape;
    int rc;
    if ((rc = check_layer(c, layer)) || (rc = check_batch(c, start, n)))
        return rc;
    if (!q || !k || !v || !out) return fail(c, SLM_ERR_ARG, "NULL buffer");
    const size_t qn = (size_t)n * s.dim, kn = (size_t)n * s.kv_dim;
    if ((rc = check_out_alias(c, out, qn, {{q, qn}, {k, kn}, {v, kn}}, false)))
        return rc;
    // staging: q | k | v | out, each segment 16-byte aligned (dim and kv_dim
    // are multiples of 32 floats)
    if ((rc = ensure_stage(c, 2 * qn + 2 * kn))) return rc;
    float* dq = c->stage;
    float* dk = dq + qn;
    float* dv = dk + kn;
    float* dout = dv + kn;
    SLM_HIP(c, hipMemcpyAsync(dq, q, qn * 4, hipMemcpyHostToDevice, c->stream));
    SLM_HIP(c, hipMemcpyAsync(dk, k, kn * 4, hipMemcpyHostToDevice, c->stream));
    SLM_HIP(c, hipMemcpyAsync(dv, v, kn * 4, hipMemcpyHostToDevice, c->stream));
    if (n == 1)
        rc = slm_attn_decode_dev(c, layer, start, dq, dk, dv, dout);
    else
        rc = slm_attn_prefill_dev(c, layer, start, n, dq, dk, dv, dout);
    if (rc) return rc;
    SLM_HIP(c, hipMemcpyAsync(out, dout, qn * 4, hipMemcpyDeviceToHost,
                              c->stream));
    SLM_HIP(c, hipStreamSynchronize(c->stream));
    return SLM_OK;
}

int slm_kv_write(slm_attn_ctx* c, int32_t layer, int32_t which, int32_t pos0,
                 int32_t n, const float* rows) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    if (c->capturing) return refuse_capture(c, "slm_kv_write");
    int rc;
    if ((rc = check_layer(c, layer))) return rc;
    if (which != 0 && which != 1) return fail(c, SLM_ERR_ARG, "which must be 0 or 1");
    if (!rows || n <= 0 || pos0 < 0 || (long)pos0 + n > c->cfg.max_seq_len)
        return fail(c, SLM_ERR_ARG, "row range outside the cache");
    float* dst = (which ? v_base(c, layer) : k_base(c, layer)) +
                 (size_t)pos0 * c->shape.kv_dim;
    SLM_HIP(c, hipMemcpyAsync(dst, rows, (size_t)n * c->shape.kv_dim * 4,
                              hipMemcpyHostToDevice, c->stream));
    SLM_HIP(c, hipStreamSynchronize(c->stream));
    return SLM_OK;
}

int slm_kv_write_dev(slm_attn_ctx* c, int32_t layer, int32_t which,
                     int32_t pos0, int32_t n, const float* rows) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    int rc;
    if ((rc = check_layer(c, layer))) return rc;
    if (which != 0 && which != 1) return fail(c, SLM_ERR_ARG, "which must be 0 or 1");
    if (!rows || n <= 0 || pos0 < 0 || (long)pos0 + n > c->cfg.max_seq_len)
        return fail(c, SLM_ERR_ARG, "row range outside the cache");
    const size_t bytes = (size_t)n * c->shape.kv_dim * 4;
    if (overlaps(rows, bytes, c->kv, c->kv_floats * 4))
        return fail(c, SLM_ERR_ALIAS, "source rows must not overlap the KV cache");
    float* dst = (which ? v_base(c, layer) : k_base(c, layer)) +
                 (size_t)pos0 * c->shape.kv_dim;
    SLM_HIP(c, hipMemcpyAsync(dst, rows, bytes, hipMemcpyDeviceToDevice, c->stream));
    return SLM_OK;
}

int slm_kv_read(slm_attn_ctx* c, int32_t layer, int32_t which, int32_t pos0,
                int32_t n, float* rows) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    if (c->capturing) return refuse_capture(c, "slm_kv_read");
    int rc;
    if ((rc = check_layer(c, layer))) return rc;
    if (which != 0 && which != 1) return fail(c, SLM_ERR_ARG, "which must be 0 or 1");
    if (!rows || n <= 0 || pos0 < 0 || (long)pos0 + n > c->cfg.max_seq_len)
        return fail(c, SLM_ERR_ARG, "row range outside the cache");
    const float* src = (which ? v_base(c, layer) : k_base(c, layer)) +
                       (size_t)pos0 * c->shape.kv_dim;
    SLM_HIP(c, hipMemcpyAsync(rows, src, (size_t)n * c->shape.kv_dim * 4,
                              hipMemcpyDeviceToHost, c->stream));
    SLM_HIP(c, hipStreamSynchronize(c->stream));
    return SLM_OK;
}

size_t slm_kv_offset(const slm_attn_ctx* c, int32_t layer, int32_t which,
                     int32_t pos) {
    if (!c || layer < 0 || layer >= c->cfg.num_layers || (which != 0 && which != 1) ||
        pos < 0 || pos >= c->cfg.max_seq_len)
        return (size_t)-1;
    return ((size_t)(2 * layer + which) * c->cfg.max_seq_len + pos) *
           c->shape.kv_dim;
}

float* slm_kv_device_ptr(const slm_attn_ctx* c) { return c ? c->kv : nullptr; }

int slm_rope_tables_read(slm_attn_ctx* c, float* cos_out, float* sin_out) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    if (c->capturing) return refuse_capture(c, "slm_rope_tables_read");
    if (!cos_out || !sin_out) return fail(c, SLM_ERR_ARG, "NULL buffer");
    const size_t bytes = (size_t)c->cfg.max_seq_len * c->shape.half * 4;
    SLM_HIP(c, hipMemcpyAsync(cos_out, c->cos_t, bytes, hipMemcpyDeviceToHost,
                              c->stream));
    SLM_HIP(c, hipMemcpyAsync(sin_out, c->sin_t, bytes, hipMemcpyDeviceToHost,
                              c->stream));
    SLM_HIP(c, hipStreamSynchronize(c->stream));
    return SLM_OK;
}

int slm_attn_profile(slm_attn_ctx* c, int32_t enable) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    if (c->capturing) return refuse_capture(c, "slm_attn_profile");
    c->profiling = enable != 0;
    return SLM_OK;
}

int slm_attn_profile_read(slm_attn_ctx* c, slm_kernel_stat* out) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    if (c->capturing) return refuse_capture(c, "slm_attn_profile_read");
    if (!out) return fail(c, SLM_ERR_ARG, "NULL buffer");
    SLM_HIP(c, hipStreamSynchronize(c->stream));
    for (auto& p : c->pending) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, p.begin, p.end) == hipSuccess) {
            c->stats[p.kind].launches += 1;
            c->stats[p.kind].total_ms += ms;
        }
        c->spare_events.push_back(p.begin);
        c->spare_events.push_back(p.end);
    }
    c->pending.clear();
    for (int i = 0; i < SLM_K_COUNT; ++i) {
        out[i] = c->stats[i];
        c->stats[i] = slm_kernel_stat{};
    }
    return SLM_OK;
}

int slm_attn_decode_splits(const slm_attn_ctx* c, int32_t seq_len,
                           int32_t* n_splits, int32_t* tile) {
    if (!c || !n_splits || !tile || seq_len <= 0)
        return fail(nullptr, SLM_ERR_ARG, "bad argument");
    int ns = 1, t = 1;
    slm::decode_split_policy(c->shape, seq_len, &ns, &t);
    *n_splits = ns;
    *tile = t;
    return SLM_OK;
}

int slm_attn_prefill_kernel(const slm_attn_ctx* c, int32_t start, int32_t n,
                            int32_t* kernel) {
    if (!c || !kernel) return fail(nullptr, SLM_ERR_ARG, "bad argument");
    if (n <= 0 || start < 0 || (long)start + n > c->cfg.max_seq_len)
        return fail(nullptr, SLM_ERR_BATCH,
                    "batch must be non-empty and start + n <= max_seq_len");
    const slm::Shape& s = c->shape;
    *kernel = (int32_t)slm::prefill_plan(s.head_dim, s.num_heads, s.kv_mul, s.cus, start, n);
    return SLM_OK;
}

// ---- slm_quant.h ----------------------------------------------------------

int slm_q4_matrix_create(int32_t device, const void* blocks, int32_t rows, int32_t cols,
                         slm_q4_matrix** out) {
    if (!out) return fail(nullptr, SLM_ERR_ARG, "out is NULL");
    *out = nullptr;
    if (!blocks) return fail(nullptr, SLM_ERR_ARG, "blocks is NULL");
    if (rows <= 0 || cols <= 0 || cols % 32 != 0)
        return fail(nullptr, SLM_ERR_SHAPE, "rows must be positive and cols a positive multiple of 32");
    if (cols > slm::q4_max_cols())
        return fail(nullptr, SLM_ERR_UNSUPPORTED, "cols above 16384 is not compiled");
    int ndev = 0;
    hipError_t e = hipGetDeviceCount(&ndev);
    if (e != hipSuccess || device < 0 || device >= ndev)
        return fail(nullptr, SLM_ERR_DEVICE, "no such HIP device");
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess ||
        strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(nullptr, SLM_ERR_DEVICE, "this library is built for gfx950 only");
    // nibbles [rows][nb][16]; f16 scales [rows][ds], ds = nb rounded up to 8
    // (zero padded) so kernels read eight scales with one 128-bit load
    const size_t nb = (size_t)cols / 32, nblk = (size_t)rows * nb;
    const size_t ds = (size_t)slm::q4_scale_stride((int)nb);
    std::vector<uint8_t> qs(nblk * 16);
    std::vector<uint16_t> d((size_t)rows * ds, 0);
    const uint8_t* src = static_cast<const uint8_t*>(blocks);
    for (size_t i = 0; i < nblk; ++i) {
        const size_t r = i / nb, b = i - r * nb;
        d[r * ds + b] = (uint16_t)(src[i * 18] | (src[i * 18 + 1] << 8));
        memcpy(&qs[i * 16], src + i * 18 + 2, 16);
    }
    int prev = 0;
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    slm_q4_matrix* m = new (std::nothrow) slm_q4_matrix();
    if (!m) return fail(nullptr, SLM_ERR_HIP, "out of host memory for the matrix handle");
    m->device = device;
    m->rows = rows;
    m->cols = cols;
    e = hipSetDevice(device);
    if (e == hipSuccess) e = hipMalloc(&m->qs, qs.size());
    if (e == hipSuccess) e = hipMalloc(&m->d, d.size() * 2);
    if (e == hipSuccess) e = hipMemcpy(m->qs, qs.data(), qs.size(), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(m->d, d.data(), d.size() * 2, hipMemcpyHostToDevice);
    if (prev >= 0) (void)hipSetDevice(prev);
    if (e != hipSuccess) {
        slm_q4_matrix_destroy(m);
        return hip_fail(nullptr, e, "q4 matrix upload");
    }
    *out = m;
    return SLM_OK;
}

void slm_q4_matrix_destroy(slm_q4_matrix* m) {
    if (!m) return;
    (void)hipFree(m->qs);
    (void)hipFree(m->d);
    delete m;
}

int slm_q4_matrix_shape(const slm_q4_matrix* m, int32_t* rows, int32_t* cols) {
    if (!m || !rows || !cols) return fail(nullptr, SLM_ERR_ARG, "bad argument");
    *rows = m->rows;
    *cols = m->cols;
    return SLM_OK;
}

int slm_quantize_q8_0_dev(slm_attn_ctx* c, const float* x, int64_t n, void* blocks) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    int rc;
    if ((rc = check_dev_ptrs(c, {x}))) return rc;
    if (!blocks || ((uintptr_t)blocks & 1u)) return fail(c, SLM_ERR_ARG, "blocks must be 2-byte aligned");
    if (n < 0 || n % 32 != 0) return fail(c, SLM_ERR_SHAPE, "n must be a multiple of 32");
    if (overlaps(x, (size_t)n * 4, blocks, (size_t)n / 32 * 34))
        return fail(c, SLM_ERR_ALIAS, "blocks must not overlap x");
    Timed t(c, SLM_K_QUANT);
    hipError_t e = slm::launch_quantize_q8_aos(x, (long)(n / 32), static_cast<uint8_t*>(blocks),
                                               c->stream);
    t.done();
    return launch_status(c, e, "q8 quantize kernel launch");
}

int slm_gemm_q4_0_dev(slm_attn_ctx* c, const slm_q4_matrix* w, const float* x, int32_t batch,
                      float* out) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    int rc;
    if ((rc = check_matrix(c, w, -1, w ? w->cols : 0, "w"))) return rc;
    if (batch < 0) return fail(c, SLM_ERR_SHAPE, "batch must not be negative");
    if (batch == 0) return SLM_OK;
    if ((rc = check_dev_ptrs(c, {x, out}))) return rc;
    if (overlaps(out, (size_t)batch * w->rows * 4, x, (size_t)batch * w->cols * 4))
        return fail(c, SLM_ERR_ALIAS, "out must not overlap x");
    return project(c, w, x, batch, out, nullptr);
}

int slm_gemm_q4_0_residual_dev(slm_attn_ctx* c, const slm_q4_matrix* w, const float* x,
                               int32_t batch, const float* res, float* out) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    int rc;
    if ((rc = check_matrix(c, w, -1, w ? w->cols : 0, "w"))) return rc;
    if (batch < 0) return fail(c, SLM_ERR_SHAPE, "batch must not be negative");
    if (batch == 0) return SLM_OK;
    if ((rc = check_residual_args(c, w, x, batch, res, out))) return rc;
    return project(c, w, x, batch, out, res);
}

int slm_attn_decode_xb_dev(slm_attn_ctx* c, int32_t layer, int32_t pos, const float* xb,
                           const slm_q4_matrix* wq, const slm_q4_matrix* wk,
                           const slm_q4_matrix* wv, float* out) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    const slm::Shape& s = c->shape;
    int rc;
    if ((rc = check_layer(c, layer)) || (rc = check_pos(c, pos)) ||
        (rc = check_dev_ptrs(c, {xb, out})) ||
        (rc = check_out_alias(c, out, s.dim, {{xb, s.dim}}, true)))
        return rc;
    float *q, *k, *v;
    if ((rc = project_qkv(c, 1, xb, wq, wk, wv, &q, &k, &v))) return rc;
    if (overlaps(out, (size_t)s.dim * 4, c->qkv, c->qkv_floats * 4))
        return fail(c, SLM_ERR_ALIAS, "out must not overlap the context's buffers");
    return do_decode(c, layer, pos, q, k, v, out, true);
}

int slm_attn_decode_xb_dev_noalloc(slm_attn_ctx* c, int32_t layer, int32_t pos,
                                   const float* xb, const slm_q4_matrix* wq,
                                   const slm_q4_matrix* wk, const slm_q4_matrix* wv,
                                   float* out) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    const slm::Shape& s = c->shape;
    int rc;
    if ((rc = check_layer(c, layer)) || (rc = check_pos(c, pos)) ||
        (rc = check_dev_ptrs(c, {xb, out})) ||
        (rc = check_out_alias(c, out, s.dim, {{xb, s.dim}}, true)))
        return rc;
    if (!c->noalloc_scratch)
        return fail(c, SLM_ERR_HIP, "no-allocation scratch unavailable on this device: " +
                                        c->noalloc_err);
    // scratch layout: q [dim] | k [kv_dim] | v [kv_dim] | partials of the
    // split count at pos + 1 (o [n_splits][num_heads][head_dim], then
    // (max, sum) [n_splits][num_heads][2]); every segment 16-byte aligned
    int ns = 1, tile = 1;
    slm::decode_split_policy(s, pos + 1, &ns, &tile);
    const size_t rows = (size_t)s.dim + 2 * (size_t)s.kv_dim;  // multiple of 32
    const size_t po = (size_t)ns * s.num_heads * s.head_dim;
    const size_t need = rows + po + (size_t)ns * s.num_heads * 2;
    if (need > kNoAllocScratchFloats)
        return fail(c, SLM_ERR_SHAPE,
                    "this shape and position need " + std::to_string(need) +
                        " floats of no-allocation scratch; the maximum is " +
                        std::to_string(kNoAllocScratchFloats));
    if ((rc = check_matrix(c, wq, s.dim, s.dim, "wq")) ||
        (rc = check_matrix(c, wk, s.kv_dim, s.dim, "wk")) ||
        (rc = check_matrix(c, wv, s.kv_dim, s.dim, "wv")))
        return rc;
    if (overlaps(out, (size_t)s.dim * 4, c->noalloc_scratch, kNoAllocScratchFloats * 4))
        return fail(c, SLM_ERR_ALIAS, "out must not overlap the library's scratch");
    float* q = c->noalloc_scratch;
    float* k = q + s.dim;
    float* v = k + s.kv_dim;
    float* part_o = q + rows;
    float* part_ml = part_o + po;
    const slm::Q4Job jobs[3] = {q4_job(wq, q), q4_job(wk, k), q4_job(wv, v)};
    hipError_t e = slm::launch_q4_gemv(jobs, 3, xb, s.dim / 32, 1, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "q4 gemv kernel launch");
    return do_decode_in(c, layer, pos, q, k, v, out, true, part_o, part_ml, false);
}

int slm_attn_prefill_xb_dev(slm_attn_ctx* c, int32_t layer, int32_t start, int32_t n,
                            const float* xb, const slm_q4_matrix* wq, const slm_q4_matrix* wk,
                            const slm_q4_matrix* wv, float* out) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    const slm::Shape& s = c->shape;
    int rc;
    if ((rc = check_layer(c, layer)) || (rc = check_batch(c, start, n)) ||
        (rc = check_dev_ptrs(c, {xb, out})))
        return rc;
    const size_t rows = (size_t)n * s.dim;
    if ((rc = check_out_alias(c, out, rows, {{xb, rows}}, true))) return rc;
    float *q, *k, *v;
    if ((rc = project_qkv(c, n, xb, wq, wk, wv, &q, &k, &v))) return rc;
    if (overlaps(out, rows * 4, c->qkv, c->qkv_floats * 4))
        return fail(c, SLM_ERR_ALIAS, "out must not overlap the context's buffers");
    if ((rc = do_append(c, layer, start, n, k, v))) return rc;
    return do_attend(c, layer, start, n, q, out, true);
}

int slm_attn_decode_wo_dev(slm_attn_ctx* c, int32_t layer, int32_t pos, float* xb,
                           const slm_q4_matrix* wq, const slm_q4_matrix* wk,
                           const slm_q4_matrix* wv, const slm_q4_matrix* wo, const float* x,
                           float* x_mid) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    int rc;
    if ((rc = check_layer(c, layer)) || (rc = check_pos(c, pos)) ||
        (rc = check_wo_args(c, 1, xb, wo, x, x_mid)))
        return rc;
    float *q, *k, *v;
    if ((rc = project_qkv(c, 1, xb, wq, wk, wv, &q, &k, &v))) return rc;
    // stream order: the projections read xb before the attention writes it
    if ((rc = do_decode(c, layer, pos, q, k, v, xb, true))) return rc;
    return project(c, wo, xb, 1, x_mid, x);
}

int slm_attn_prefill_wo_dev(slm_attn_ctx* c, int32_t layer, int32_t start, int32_t n,
                            float* xb, const slm_q4_matrix* wq, const slm_q4_matrix* wk,
                            const slm_q4_matrix* wv, const slm_q4_matrix* wo, const float* x,
                            float* x_mid) {
    if (!c) return fail(nullptr, SLM_ERR_ARG, "ctx is NULL");
    int rc;
    if ((rc = check_layer(c, layer)) || (rc = check_batch(c, start, n)) ||
        (rc = check_wo_args(c, n, xb, wo, x, x_mid)))
        return rc;
    float *q, *k, *v;
    if ((rc = project_qkv(c, n, xb, wq, wk, wv, &q, &k, &v))) return rc;
    if ((rc = do_append(c, layer, start, n, k, v))) return rc;
    if ((rc = do_attend(c, layer, start, n, q, xb, true))) return rc;
    return project(c, wo, xb, n, x_mid, x);
}

}  // extern "C"
