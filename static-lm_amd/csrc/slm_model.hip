// Device upload of a GGUF model (slm_gguf.h): GgufFile::model_weights
// (loader.rs:508-552) resolved by tensor name and copied to one device as
// slm_q4_matrix handles and f32 vectors, with the slm_model_weights view the
// slm_model_*_dev entry points take.
#include "../../include/slm_gguf.h"

#include <new>
#include <string>
#include <vector>

#include "slm_host.h"

using namespace slm_host;

struct slm_model {
    int device = 0;
    int vocab = 0;
    std::vector<slm_q4_matrix*> mats;  // owned
    std::vector<float*> vecs;          // owned device f32 vectors
    std::vector<slm_layer_weights> layers;
    slm_model_weights view{};
};

namespace {

// A Q4_0 tensor [dims[1..]][dims[0]] as a rows x cols matrix on the device.
int load_q4(slm_model* m, const slm_gguf* g, const std::string& name,
            const slm_q4_matrix** out) {
    slm_gguf_tensor t;
    const void* data;
    uint64_t bytes;
    int rc;
    if ((rc = slm_gguf_tensor_info(g, name.c_str(), &t)) ||
        (rc = slm_gguf_tensor_data(g, name.c_str(), SLM_GGML_Q4_0, &data, &bytes)))
        return rc;
    const uint64_t cols = t.dims[0], rows = cols ? t.n_elements / cols : 0;
    if (cols == 0 || rows == 0 || rows > INT32_MAX || cols > INT32_MAX)
        return fail(nullptr, SLM_ERR_SHAPE, name + " has an empty or oversized shape");
    slm_q4_matrix* q = nullptr;
    if ((rc = slm_q4_matrix_create(m->device, data, (int32_t)rows, (int32_t)cols, &q))) return rc;
    m->mats.push_back(q);
    *out = q;
    return SLM_OK;
}

// An f32 vector of exactly `floats` elements: the norm kernels read that
// many floats from a bare device pointer, so a shorter tensor would be read
// out of bounds (the reference asserts weights.len() == dst.len,
// engine.rs:199).
int check_f32(const slm_gguf* g, const std::string& name, uint64_t floats) {
    slm_gguf_tensor t;
    const void* data;
    uint64_t bytes;
    int rc;
    if ((rc = slm_gguf_tensor_info(g, name.c_str(), &t)) ||
        (rc = slm_gguf_tensor_data(g, name.c_str(), SLM_GGML_F32, &data, &bytes)))
        return rc;
    if (t.n_elements != floats || bytes != floats * 4)
        return fail(nullptr, SLM_ERR_SHAPE,
                    name + " holds " + std::to_string(t.n_elements) +
                        " floats, the model dimension is " + std::to_string(floats));
    return SLM_OK;
}

int check_q4(const slm_gguf* g, const std::string& name) {
    const void* data;
    uint64_t bytes;
    return slm_gguf_tensor_data(g, name.c_str(), SLM_GGML_Q4_0, &data, &bytes);
}

// Every tensor the upload reads, checked before any device work: present,
// of the right type and, for the norm vectors, dim floats long.  In the order
// model_weights and layer_weights resolve them (loader.rs:508-552), so a file
// with several faults gets the error of the first one the reference meets.
int check_model_file(const slm_gguf* g, int num_layers, uint64_t dim) {
    int rc;
    if ((rc = check_q4(g, "token_embd.weight")) ||
        (rc = check_f32(g, "output_norm.weight", dim)))
        return rc;
    slm_gguf_tensor out_info;
    if (slm_gguf_tensor_info(g, "output.weight", &out_info) == SLM_OK &&
        (rc = check_q4(g, "output.weight")))
        return rc;
    // per layer: attn_norm, attn_q, attn_k, attn_v, attn_output, ffn_norm,
    // ffn_gate, ffn_up, ffn_down (the norms f32, the rest Q4_0)
    static const struct {
        const char* name;
        bool norm;
    } tensors[] = {{"attn_norm", true}, {"attn_q", false},   {"attn_k", false},
                   {"attn_v", false},   {"attn_output", false}, {"ffn_norm", true},
                   {"ffn_gate", false}, {"ffn_up", false},   {"ffn_down", false}};
    for (int l = 0; l < num_layers; ++l) {
        const std::string p = "blk." + std::to_string(l) + ".";
        for (const auto& t : tensors) {
            const std::string name = p + t.name + ".weight";
            if ((rc = t.norm ? check_f32(g, name, dim) : check_q4(g, name))) return rc;
        }
    }
    return SLM_OK;
}

int load_f32(slm_model* m, const slm_gguf* g, const std::string& name, uint64_t floats,
             const float** out) {
    const void* data;
    uint64_t bytes;
    int rc;
    if ((rc = check_f32(g, name, floats)) ||
        (rc = slm_gguf_tensor_data(g, name.c_str(), SLM_GGML_F32, &data, &bytes)))
        return rc;
    int prev = 0;
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    float* d = nullptr;
    hipError_t e = hipSetDevice(m->device);
    if (e == hipSuccess) e = hipMalloc(&d, bytes);
    if (e == hipSuccess) m->vecs.push_back(d);
    if (e == hipSuccess) e = hipMemcpy(d, data, bytes, hipMemcpyHostToDevice);
    if (prev >= 0) (void)hipSetDevice(prev);
    if (e != hipSuccess) return hip_fail(nullptr, e, "f32 tensor upload");
    *out = d;
    return SLM_OK;
}

}  // namespace

extern "C" {

int slm_model_load_gguf(const slm_gguf* g, int32_t device, int32_t num_layers,
                        slm_model** out) {
    if (!out) return fail(nullptr, SLM_ERR_ARG, "out is NULL");
    *out = nullptr;
    if (!g) return fail(nullptr, SLM_ERR_ARG, "gguf is NULL");
    if (num_layers < 1) return fail(nullptr, SLM_ERR_CONFIG, "num_layers must be positive");
    int rc;
    slm_gguf_tensor embd;
    if ((rc = slm_gguf_tensor_info(g, "token_embd.weight", &embd))) return rc;
    if (embd.dims[1] > INT32_MAX)
        return fail(nullptr, SLM_ERR_BOUNDS, "OutOfBounds(token_embd.weight)");
    const uint64_t dim = embd.dims[0];  // the embedding width is the model dimension
    if (dim == 0 || dim % 32 != 0)
        return fail(nullptr, SLM_ERR_SHAPE, "token_embd.weight rows must be a multiple of 32 long");
    if ((rc = check_model_file(g, num_layers, dim))) return rc;
    slm_model* m = new (std::nothrow) slm_model();
    if (!m) return fail(nullptr, SLM_ERR_HIP, "out of host memory for the model handle");
    m->device = device;
    auto bail = [&](int code) {
        slm_model_destroy(m);
        return code;
    };
    m->vocab = (int)embd.dims[1];
    const slm_q4_matrix* token_embd = nullptr;
    const slm_q4_matrix* lm_head = nullptr;
    const float* output_norm = nullptr;
    if ((rc = load_q4(m, g, "token_embd.weight", &token_embd)) ||
        (rc = load_f32(m, g, "output_norm.weight", dim, &output_norm)))
        return bail(rc);
    slm_gguf_tensor out_info;
    if (slm_gguf_tensor_info(g, "output.weight", &out_info) == SLM_OK) {
        if ((rc = load_q4(m, g, "output.weight", &lm_head))) return bail(rc);
    } else {
        lm_head = token_embd;  // tied embeddings (loader.rs:535-539)
    }
    m->layers.resize((size_t)num_layers);
    for (int l = 0; l < num_layers; ++l) {  // layer_weights (loader.rs:508-521)
        const std::string p = "blk." + std::to_string(l) + ".";
        slm_layer_weights& lw = m->layers[(size_t)l];
        if ((rc = load_f32(m, g, p + "attn_norm.weight", dim, &lw.rms_att)) ||
            (rc = load_q4(m, g, p + "attn_q.weight", &lw.wq)) ||
            (rc = load_q4(m, g, p + "attn_k.weight", &lw.wk)) ||
            (rc = load_q4(m, g, p + "attn_v.weight", &lw.wv)) ||
            (rc = load_q4(m, g, p + "attn_output.weight", &lw.wo)) ||
            (rc = load_f32(m, g, p + "ffn_norm.weight", dim, &lw.rms_ffn)) ||
            (rc = load_q4(m, g, p + "ffn_gate.weight", &lw.w_gate)) ||
            (rc = load_q4(m, g, p + "ffn_up.weight", &lw.w_up)) ||
            (rc = load_q4(m, g, p + "ffn_down.weight", &lw.w_down)))
            return bail(rc);
    }
    m->view = slm_model_weights{token_embd, m->layers.data(), num_layers, output_norm, lm_head};
    *out = m;
    return SLM_OK;
}

void slm_model_destroy(slm_model* m) {
    if (!m) return;
    for (slm_q4_matrix* q : m->mats) slm_q4_matrix_destroy(q);
    for (float* v : m->vecs) (void)hipFree(v);
    delete m;
}

const slm_model_weights* slm_model_weights_view(const slm_model* m) {
    return m ? &m->view : nullptr;
}

int32_t slm_model_vocab_size(const slm_model* m) { return m ? m->vocab : 0; }

}  // extern "C"
