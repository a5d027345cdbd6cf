// Host side shared by the C-ABI translation units: the context and weight
// handles, and the argument checks and dispatch helpers every entry point
// uses (defined in slm_attn.hip).
#pragma once

#include "../../include/slm_attn.h"
#include "../../include/slm_quant.h"

#include <stdint.h>

#include <initializer_list>
#include <string>
#include <utility>
#include <vector>

#include "slm_internal.h"

// A Q4_0 weight matrix on one device: nibbles [rows][cols/32][16] and f16
// scales [rows][cols/32 rounded up to 8], repacked from 18-byte BlockQ4_0
// (blocks.rs:11-19).
struct slm_q4_matrix {
    int device = 0;
    int rows = 0;
    int cols = 0;
    uint8_t* qs = nullptr;
    uint16_t* d = nullptr;
};

struct slm_attn_ctx {
    slm_attn_config cfg{};
    slm::Shape shape{};
    int device = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    // [num_layers][2][max_seq_len][kv_dim] f32, the arena's KV slices in order
    float* kv = nullptr;
    size_t kv_floats = 0;
    // RoPE tables [max_seq_len][head_dim/2]
    float* cos_t = nullptr;
    float* sin_t = nullptr;
    // split-K partials of one decode row
    float* part_o = nullptr;
    float* part_ml = nullptr;
    int max_splits = 1;
    // this device's copy of the file-scope scratch of the no-allocation
    // entry point (nullptr when its address could not be taken)
    float* noalloc_scratch = nullptr;
    std::string noalloc_err;
    // staging for the host-pointer entry points
    float* stage = nullptr;
    size_t stage_floats = 0;
    // projections: Q8_0 activations (i8 [blocks][32], f32 scales) and the
    // q | k | v rows the GEMMs produce for the attention kernels
    uint32_t* q8_q = nullptr;
    float* q8_d = nullptr;
    int* q8_s = nullptr;  // blocks' sums of quantized values (the GEMV's input)
    size_t q8_blocks = 0;
    // a second set, for a kernel that reads one Q8_0 activation and writes
    // another (the fused gate/up + SwiGLU projection)
    uint32_t* q8x_q = nullptr;
    float* q8x_d = nullptr;
    int* q8x_s = nullptr;
    size_t q8x_blocks = 0;
    float* qkv = nullptr;
    size_t qkv_floats = 0;
    // transformer block workspace (slm_layer.h): attention rows and x_mid
    // [n][dim], gate | up rows [n][2][hidden_dim]
    float* blk_att = nullptr;
    size_t blk_att_floats = 0;
    float* blk_mid = nullptr;
    size_t blk_mid_floats = 0;
    float* blk_hid = nullptr;
    size_t blk_hid_floats = 0;
    // whole-model workspace (slm_layer.h): residual rows [msl][dim], token
    // ids [msl], logits [vocab], the argmax result and a token-range flag
    float* mdl_x = nullptr;
    size_t mdl_x_floats = 0;
    int32_t* mdl_tok = nullptr;
    size_t mdl_tok_n = 0;
    float* mdl_logits = nullptr;
    size_t mdl_logits_n = 0;
    int32_t* mdl_flags = nullptr;  // [0] argmax, [1] bad token
    size_t mdl_flags_n = 0;
    slm::ArgmaxPart* mdl_parts = nullptr;  // the lm_head workgroups' best logits
    size_t mdl_parts_n = 0;
    int32_t* tok_pin = nullptr;            // pinned [2]: generate's tokens, read back
    hipEvent_t tok_ev[2] = {nullptr, nullptr};  // one step behind the device
    // generate's copy of the K and V rows of every layer at the position a
    // step launched ahead of its previous token writes ([2 * layers][kv_dim])
    float* gen_rows = nullptr;
    size_t gen_rows_floats = 0;
    // the stream is being captured into a HIP graph (slm_attn_capture_begin)
    bool capturing = false;
    // kernel timing
    bool profiling = false;
    struct Pending {
        int kind;
        hipEvent_t begin;
        hipEvent_t end;
    };
    std::vector<Pending> pending;
    std::vector<hipEvent_t> spare_events;
    slm_kernel_stat stats[SLM_K_COUNT]{};
    std::string err;
};

// A captured sequence of launches (slm_attn_capture_end), replayed on a
// context's stream by slm_attn_graph_launch.
struct slm_attn_graph {
    int device;
    hipGraph_t graph;
    hipGraphExec_t exec;
};

namespace slm_host {

int fail(slm_attn_ctx* c, int code, const std::string& msg);
int hip_fail(slm_attn_ctx* c, hipError_t e, const char* what);
// SLM_ERR_CAPTURE for a call that cannot be recorded into a graph
int refuse_capture(slm_attn_ctx* c, const char* what);

#define SLM_HIP(c, expr)                                   \
    do {                                                   \
        hipError_t e_ = (expr);                            \
        if (e_ != hipSuccess) return hip_fail(c, e_, #expr); \
    } while (0)

bool aligned16(const void* p);
bool overlaps(const void* a, size_t a_bytes, const void* b, size_t b_bytes);
hipEvent_t take_event(slm_attn_ctx* c);

// Brackets one kernel launch with events while profiling is on.
struct Timed {
    slm_attn_ctx* c;
    int kind;
    hipEvent_t b = nullptr;
    hipEvent_t e = nullptr;
    // in_launch: the launch itself records b and e (hipExtLaunchKernelGGL
    // stamps them at the kernel's start and end, as a kernel trace does);
    // otherwise b is recorded here and e by done()
    Timed(slm_attn_ctx* ctx, int k, bool in_launch = false) : c(ctx), kind(k) {
        if (!c->profiling) return;
        b = take_event(c);
        e = take_event(c);
        if (!b || !e) {  // a launch is timed with both events or not at all
            drop();
            return;
        }
        if (in_launch) return;
        if (b && e && hipEventRecord(b, c->stream) != hipSuccess) drop();
    }
    // after a launch that recorded b and e itself
    void done_in_launch(bool launched) {
        if (!b || !e) return;
        if (!launched) {
            drop();
            return;
        }
        c->pending.push_back({kind, b, e});
        b = e = nullptr;
    }
    void done() {
        if (!b || !e) return;
        if (hipEventRecord(e, c->stream) != hipSuccess) {
            drop();
            return;
        }
        c->pending.push_back({kind, b, e});
        b = e = nullptr;
    }
    // A launch whose events could not be recorded is left out of the stats.
    void drop() {
        if (b) c->spare_events.push_back(b);
        if (e) c->spare_events.push_back(e);
        b = e = nullptr;
    }
};

// Grows a device buffer (after the stream drained its users).
template <class T>
int ensure_buffer(slm_attn_ctx* c, T** buf, size_t* have, size_t want, const char* what) {
    if (*have >= want) return SLM_OK;
    if (c->capturing) return refuse_capture(c, what);
    if (*buf) {
        SLM_HIP(c, hipStreamSynchronize(c->stream));
        SLM_HIP(c, hipFree(*buf));
        *buf = nullptr;
        *have = 0;
    }
    hipError_t e = hipMalloc(buf, want * sizeof(T));
    if (e != hipSuccess) return hip_fail(c, e, what);
    *have = want;
    return SLM_OK;
}

float* k_base(slm_attn_ctx* c, int layer);
float* v_base(slm_attn_ctx* c, int layer);
int check_layer(slm_attn_ctx* c, int layer);
int check_pos(slm_attn_ctx* c, int pos);
int check_batch(slm_attn_ctx* c, int start, int n);
int check_dev_ptrs(slm_attn_ctx* c, std::initializer_list<const void*> ps);
int launch_status(slm_attn_ctx* c, hipError_t e, const char* what);
int do_append(slm_attn_ctx* c, int layer, int pos0, int n, const float* k, const float* v);
int do_decode(slm_attn_ctx* c, int layer, int pos, const float* q, const float* k_new,
              const float* v_new, float* out, bool rotate);
// The same with the split partials in part_o / part_ml and, when timed is
// false, no profiling events taken.
int do_decode_in(slm_attn_ctx* c, int layer, int pos, const float* q, const float* k_new,
                 const float* v_new, float* out, bool rotate, float* part_o, float* part_ml,
                 bool timed);
int do_attend(slm_attn_ctx* c, int layer, int start, int n, const float* q, float* out,
              bool rotate);
int ensure_q8(slm_attn_ctx* c, size_t n, int nb);
int ensure_q8x(slm_attn_ctx* c, size_t n, int nb);
int check_matrix(slm_attn_ctx* c, const slm_q4_matrix* m, int rows, int cols, const char* name);
slm::Q4Job q4_job(const slm_q4_matrix* m, float* out, const float* res = nullptr);
int project(slm_attn_ctx* c, const slm_q4_matrix* w, const float* x, int batch, float* out,
            const float* res);
int project_qkv(slm_attn_ctx* c, int n, const float* xb, const slm_q4_matrix* wq,
                const slm_q4_matrix* wk, const slm_q4_matrix* wv, float** q, float** k,
                float** v);

}  // namespace slm_host
