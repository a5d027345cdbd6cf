// RoPE and KV-cache append kernels for gfx950.
//
// The rotation is apply_rope_cached (transformer.rs:178-194):
//   x[2j]   = x[2j]*cos[j] - x[2j+1]*sin[j]
//   x[2j+1] = x[2j]*sin[j] + x[2j+1]*cos[j]
// with each product and each sum rounded on its own (Rust never fuses), so the
// cache rows written here are bit-identical to the reference's.  Contraction
// into v_fma is switched off in these kernels for that reason.
#include "attn_common.h"
#include "slm_internal.h"

namespace slm {
namespace {

// One thread per (row, pair).  K row pos0+r of the layer slice receives the
// rotated pair, V row receives the v pair unchanged (the Wk/Wv GEMV output the
// reference writes in place, transformer.rs:416-417, 545-561).
__global__ __launch_bounds__(256) void kv_append_kernel(
    const float* __restrict__ k, const float* __restrict__ v,
    float* __restrict__ k_cache, float* __restrict__ v_cache,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t,
    int kv_dim, int half, int pos0, int n) {
    const unsigned pairs = (unsigned)kv_dim >> 1;
    const unsigned idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (unsigned)n * pairs) return;
    const unsigned r = idx / pairs;
    const unsigned p = idx - r * pairs;
    const unsigned j = p % (unsigned)half;
    const long pos = pos0 + (long)r;
    const float c = cos_t[pos * half + j];
    const float s = sin_t[pos * half + j];
    const float2 kk = reinterpret_cast<const float2*>(k + (long)r * kv_dim)[p];
    const float2 vv = reinterpret_cast<const float2*>(v + (long)r * kv_dim)[p];
    reinterpret_cast<float2*>(k_cache + pos * kv_dim)[p] = rope_pair_exact(kk, c, s);
    reinterpret_cast<float2*>(v_cache + pos * kv_dim)[p] = vv;
}

__global__ __launch_bounds__(256) void rope_kernel(
    float* __restrict__ x, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, int row_len, int half, int pos0, int n) {
    const unsigned pairs = (unsigned)row_len >> 1;
    const unsigned idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (unsigned)n * pairs) return;
    const unsigned r = idx / pairs;
    const unsigned p = idx - r * pairs;
    const unsigned j = p % (unsigned)half;
    const long pos = pos0 + (long)r;
    float2* row = reinterpret_cast<float2*>(x + (long)r * row_len);
    row[p] = rope_pair_exact(row[p], cos_t[pos * half + j], sin_t[pos * half + j]);
}

// Row pos of each of the rows K/V slices (kv_row points at row pos of the
// first; the slices are pitch floats apart) to or from packed [rows][kv_dim].
__global__ __launch_bounds__(256) void kv_rows_copy_kernel(float* __restrict__ kv_row,
                                                           float* __restrict__ packed, long pitch,
                                                           int kv_dim4, bool to_packed) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= kv_dim4) return;
    float4* a = reinterpret_cast<float4*>(kv_row + blockIdx.y * pitch) + i;
    float4* b = reinterpret_cast<float4*>(packed) + (long)blockIdx.y * kv_dim4 + i;
    if (to_packed)
        *b = *a;
    else
        *a = *b;
}

}  // namespace

hipError_t launch_kv_rows_copy(const Shape& s, float* kv_row, float* packed, int rows,
                               bool to_packed, hipStream_t st) {
    const int kv_dim4 = s.kv_dim / 4;
    hipLaunchKernelGGL(kv_rows_copy_kernel, dim3((kv_dim4 + 255) / 256, rows), dim3(256), 0, st,
                       kv_row, packed, (long)s.max_seq_len * s.kv_dim, kv_dim4, to_packed);
    return hipGetLastError();
}

// Rows per launch so that the 32-bit thread index cannot overflow.
static int rows_per_launch(int row_len) {
    const long limit = 1L << 30;
    const long pairs = row_len / 2;
    return (int)(limit / pairs);
}

hipError_t launch_kv_append(const Shape& s, const float* k, const float* v,
                            float* k_cache, float* v_cache, const float* cos_t,
                            const float* sin_t, int pos0, int n,
                            hipStream_t st) {
    const int block = 256;
    const int step = rows_per_launch(s.kv_dim);
    for (int r0 = 0; r0 < n; r0 += step) {
        const int nr = (n - r0 < step) ? n - r0 : step;
        const long total = (long)nr * (s.kv_dim / 2);
        const long grid = (total + block - 1) / block;
        hipLaunchKernelGGL(kv_append_kernel, dim3((unsigned)grid), dim3(block),
                           0, st, k + (long)r0 * s.kv_dim,
                           v + (long)r0 * s.kv_dim, k_cache, v_cache, cos_t,
                           sin_t, s.kv_dim, s.half, pos0 + r0, nr);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_rope(const Shape& s, float* x, int n, int row_len, int pos0,
                       const float* cos_t, const float* sin_t, hipStream_t st) {
    const int block = 256;
    const int step = rows_per_launch(row_len);
    for (int r0 = 0; r0 < n; r0 += step) {
        const int nr = (n - r0 < step) ? n - r0 : step;
        const long total = (long)nr * (row_len / 2);
        const long grid = (total + block - 1) / block;
        hipLaunchKernelGGL(rope_kernel, dim3((unsigned)grid), dim3(block), 0, st,
                           x + (long)r0 * row_len, cos_t, sin_t, row_len,
                           s.half, pos0 + r0, nr);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace slm
