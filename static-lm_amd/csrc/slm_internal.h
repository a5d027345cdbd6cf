// Internal interface between the C-ABI host code and the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace slm {

// Shapes every kernel launch needs, derived from slm_attn_config exactly as
// TransformerConfig::{head_dim, kv_dim, kv_mul} (transformer.rs:18-33).
struct Shape {
    int dim;
    int num_heads;
    int num_kv_heads;
    int head_dim;
    int kv_dim;
    int kv_mul;
    int half;  // head_dim / 2, the RoPE table row length
    int max_seq_len;
    int cus;   // compute units of the device (sizes the decode split count)
};

// K/V append: rows pos0..pos0+n-1 of the layer's K slice get rope(k row),
// the V slice gets the v row.  f32 products and sums rounded one by one.
hipError_t launch_kv_append(const Shape& s, const float* k, const float* v,
                            float* k_cache, float* v_cache, const float* cos_t,
                            const float* sin_t, int pos0, int n,
                            hipStream_t st);

// Row pos of `rows` consecutive K/V slices ([layer][K|V][msl][kv_dim]; kv_row
// points at row pos of the first) to (to_packed) or from packed
// [rows][kv_dim].
hipError_t launch_kv_rows_copy(const Shape& s, float* kv_row, float* packed, int rows,
                               bool to_packed, hipStream_t st);

// In-place apply_rope_cached on n rows of row_len floats at pos0..pos0+n-1.
hipError_t launch_rope(const Shape& s, float* x, int n, int row_len, int pos0,
                       const float* cos_t, const float* sin_t, hipStream_t st);

bool head_dim_supported(int head_dim);

// Single-token decode: optional KV append at pos fused into split-K
// attention over rows 0..pos, then a merge kernel when there are splits.
struct DecodeArgs {
    const float* q;      // [dim]; rotated at pos when cos_t != nullptr
    const float* k_new;  // [kv_dim] appended at pos when not nullptr
    const float* v_new;
    float* k_cache;
    float* v_cache;
    const float* cos_t;
    const float* sin_t;
    float* out;          // [dim]
    float* part_o;       // [n_splits][num_heads][head_dim]
    float* part_ml;      // [n_splits][num_heads][2]
    int pos;
    int n_splits;
    // when set, the launch (decode or merge) records these at the kernel's
    // start and end
    hipEvent_t ev_start = nullptr;
    hipEvent_t ev_stop = nullptr;
};
// Split count and tile length (positions) at seq_len: split s of n reads
// tiles s, s+n, s+2n, ...  A pure function of seq_len, the shape and the CU
// count.
void decode_split_policy(const Shape& s, int seq_len, int* n_splits, int* tile);
int decode_groups(const Shape& s);
int decode_max_splits();
hipError_t launch_decode(const Shape& s, const DecodeArgs& a, hipStream_t st);
// Merge of the split partials; needed only when a.n_splits > 1.
hipError_t launch_decode_combine(const Shape& s, const DecodeArgs& a, hipStream_t st);

// Causal prefill on fp32 MFMA: rows b < n at positions start + b attend to
// cache rows 0..start+b.  q is un-rotated when cos_t != nullptr.
struct PrefillArgs {
    const float* q;
    const float* k_cache;
    const float* v_cache;
    const float* cos_t;
    const float* sin_t;
    float* out;
    int start;
    int n;
};
hipError_t launch_prefill_mfma(const Shape& s, const PrefillArgs& a,
                               hipStream_t st);

// Q4_0 x Q8_0 projections (quant_gemm.hip).  A job is one weight matrix:
// nibbles [rows][nb][16], f16 scales [rows][q4_scale_stride(nb)],
// out[tok * out_stride + row].  With res, out = res + product, res laid out
// like out (res may be out itself: each element is read, then written, by
// one thread).
struct Q4Job {
    const uint8_t* qs;
    const uint16_t* d;
    float* out;
    int rows;
    int out_stride;
    const float* res;
};
int q4_max_cols();
// scale row length: nb rounded up to 8 (the GEMM reads 8 scales per load)
int q4_scale_stride(int nb);
// whether the GEMV takes a batch of this size (batch 1 always; up to 4 rows of
// at most 256 blocks)
bool q4_gemv_takes(int nb, int batch);
// quantize_row_q8_0 into 34-byte blocks
hipError_t launch_quantize_q8_aos(const float* x, long nblk, uint8_t* out, hipStream_t st);
// quantize_row_q8_0 of ntok rows of nb blocks into q [ntok][nb][32] i8 and
// d [ntok][q4_scale_stride(nb)] f32 (the GEMM's input); with sums, also the
// blocks' sums of quantized values, laid out like d (the GEMV's input)
hipError_t launch_quantize_q8_soa(const float* x, long ntok, int nb, uint32_t* q, float* d,
                                  int* sums, hipStream_t st);
// a batch q4_gemv_takes(): quantizes x [batch][nb*32] itself
hipError_t launch_q4_gemv(const Q4Job* jobs, int njobs, const float* x, int nb, int batch,
                          hipStream_t st);
// one token from pre-quantized activations (q [nb][8] u32, d and block sums
// [nb]); nb at most 512
hipError_t launch_q4_gemv_q8(const Q4Job* jobs, int njobs, const uint32_t* aq, const float* ad,
                             const int* as, int nb, hipStream_t st);
// Q8_0 blocks of a row-major [rows][nb * 32] activation, as the projections
// read them: q [rows][nb][8] (32 i8 per block), d and the blocks' sums of
// quantized values [rows][d_stride] (s may be nullptr; the GEMM needs none).
struct Q8Out {
    uint32_t* q;
    float* d;
    int* s;
    int nb;
    int d_stride;
};
// gate and up rows of one token from pre-quantized activations with SwiGLU
// fused: act = silu(gate . x) * (up . x) for every hidden row, written as
// Q8_0 blocks to q8 (and f32 to act unless nullptr); hidden % 32 == 0
hipError_t launch_q4_gemv_q8_swiglu(const Q4Job& gate, const Q4Job& up, const uint32_t* aq,
                                    const float* ad, const int* as, int nb, float* act,
                                    const Q8Out& q8, hipStream_t st);
// The same two one-token projections from the f32 row x [nb * 32] that the
// RMSNorm with weights w before them reads: every workgroup normalizes x
// itself (the norm kernel's bits) and quantizes it into LDS.
hipError_t launch_q4_gemv_norm(const Q4Job* jobs, int njobs, const float* x, const float* w,
                               float eps, int nb, hipStream_t st);
hipError_t launch_q4_gemv_norm_swiglu(const Q4Job& gate, const Q4Job& up, const float* x,
                                      const float* w, float eps, int nb, float* act,
                                      const Q8Out& q8, hipStream_t st);
// any batch, from pre-quantized activations
hipError_t launch_q4_gemm(const Q4Job* jobs, int njobs, const uint32_t* aq, const float* ad,
                          int nb, int batch, hipStream_t st);

// JIT kernels (norm_act.hip).  RMSNorm (w != nullptr) or L2 norm (w ==
// nullptr) of `rows` rows of n, into out (f32) and/or q8 (n % 32 == 0).
int norm_max_n();
hipError_t launch_rmsnorm(const float* x, long x_stride, const float* w, int rows, int n,
                          float eps, float* out, long out_stride, const Q8Out& q8,
                          hipStream_t st);
// out = silu(gate) * up over `total` elements, into out and/or q8 (rows of
// n elements, n % 32 == 0; n is only read for q8)
hipError_t launch_swiglu(const float* gate, const float* up, long total, int n, float* out,
                         const Q8Out& q8, hipStream_t st);
// out = x + y
hipError_t launch_add(const float* x, const float* y, long n, float* out, hipStream_t st);
// rows tokens[0..n) of a Q4_0 matrix dequantized into out [n][nb*32]; a
// device-side token id outside [0, vocab) sets *bad and leaves its row
hipError_t launch_embed_rows(const uint8_t* qs, const uint16_t* d, int nb, int vocab,
                             const int32_t* tokens, int n, float* out, int* bad,
                             hipStream_t st);
// out[i] = sum over b in order of rows[b][i] * inv (embed_tokens' pooling)
hipError_t launch_mean_pool(const float* rows, int n, int dim, float inv, float* out,
                            hipStream_t st);
// The best (value, index) of a stretch of logits, NaN skipped (index -1: none).
struct ArgmaxPart {
    float v;
    int i;
};
// One token's projection (as launch_q4_gemv_q8, one matrix, no residual) that
// also writes each workgroup's ArgmaxPart of its rows: q4_gemv_rows_per_part()
// rows per part, ceil(rows / that) parts.
int q4_gemv_rows_per_part();
hipError_t launch_q4_gemv_q8_argmax(const Q4Job& job, const uint32_t* aq, const float* ad,
                                    const int* as, int nb, ArgmaxPart* parts, hipStream_t st);
// sample_argmax from those parts: out[0] = the first index of the maximum of x
// (0 when x[0] is NaN or every value is)
hipError_t launch_argmax_parts(const ArgmaxPart* parts, int n_parts, const float* x, int32_t* out,
                               hipStream_t st);

}  // namespace slm
