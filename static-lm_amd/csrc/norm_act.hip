// The JIT kernels around the projections, for gfx950: RMSNorm, L2 norm,
// SwiGLU and the residual add (FuseGraph, src/jit/graph.rs:130-193), plus
// the token-embedding row lookup (dequantize_row_q4_0, blocks.rs:85-99) and
// greedy argmax (sample_argmax, transformer.rs:654-666).
//
// Bit-exactness.  lower_fuse_graph (src/jit/lower.rs:212-480) evaluates a
// reduction as four lane accumulators over i < n & ~3 (lane k takes
// i = k mod 4, in order), then (l0 + l1) + (l2 + l3), then a scalar tail in
// order; scalars derived from the reduction are hoisted, and the store pass
// applies the elementwise ops per element.  Every f32 operation is IEEE with
// no contraction (Cranelift never fuses), so the kernels keep the same
// operations in the same order: each of the four lane sums is one dependent
// chain of n/4 adds run by one lane, and division and square root are the
// correctly rounded ones.  The normalized rows can be emitted directly as
// Q8_0 blocks (quantize_row_q8_0's arithmetic) for the projection that reads
// them, which is what the reference's next call does with them.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "attn_common.h"
#include "jit_math.h"
#include "norm_common.h"
#include "quant_common.h"
#include "slm_internal.h"

namespace slm {
namespace {

constexpr int kNormThreads = 256;

// ---- RMSNorm / L2 norm: one workgroup per row ----
//
// The squares go to LDS transposed, s_sq[k][i] = x[4i + k]^2, so lane k of
// wave 0 reads its chain contiguously; lanes 0..3 run the four chains, lane 0
// combines them and the tail, and computes the scale.  Then every thread
// writes its share of the output (f32 and/or Q8_0 blocks).

struct NormArgs {
    const float* x;   // [rows][n], row stride x_stride floats
    long x_stride;
    const float* w;   // [n] (RMSNorm) or nullptr (L2 norm)
    int n;
    float eps;
    float* out;       // [rows][n], row stride out_stride, or nullptr
    long out_stride;
    Q8Out q8;         // Q8_0 output of each row, or q8.q == nullptr
};

// Rows of n % 32 == 0: quad q of the workgroup owns blocks q, q + 64, ...
// (lane part p: elements 8p..8p+7 of each) in both phases, so x and w are
// loaded once, up front, and held in registers across the chain.
constexpr int kNormMaxPasses = 8;  // n <= 64 blocks * 8 passes * 32 = 16384

template <bool RMS>
__global__ __launch_bounds__(kNormThreads) void norm_rows_kernel(NormArgs a) {
#pragma clang fp contract(off)
    extern __shared__ __align__(16) float s_sq[];  // [4][norm_sq_stride(n)]
    __shared__ float s_part[4];
    __shared__ float s_tail[4];
    __shared__ float s_scale;
    const int n = a.n;
    const int vq = n / 4;
    const int st = norm_sq_stride(n);
    const float* x = a.x + (long)blockIdx.x * a.x_stride;
    const int tid = threadIdx.x;
    const int part = tid & 3;
    const int nb = n / 32;
    const int passes = (nb + 63) / 64;

    NormRow<kNormMaxPasses> r;
    norm_row_load<kNormMaxPasses, RMS>(r, x, a.w, nb);
    norm_row_squares(r, nb, s_sq);
    __syncthreads();
    norm_scale<RMS>(s_sq, st, vq, n, s_tail, a.eps, s_part, &s_scale);
    __syncthreads();
    const float scale = s_scale;

#pragma unroll
    for (int k = 0; k < kNormMaxPasses; ++k) {
        if (k >= passes) break;
        const int blk = (tid >> 2) + 64 * k;
        if (blk >= nb) break;  // uniform over the quad
        float4 f0, f1;
        norm_row_values<kNormMaxPasses, RMS>(r, k, scale, &f0, &f1);
        const int e0 = 32 * blk + 8 * part;
        if (a.out) {
            float* o = a.out + (long)blockIdx.x * a.out_stride + e0;
            *reinterpret_cast<float4*>(o) = f0;
            *reinterpret_cast<float4*>(o + 4) = f1;
        }
        if (a.q8.q) store_q8_quad(a.q8, blockIdx.x, blk, part, f0, f1);
    }
}

// Any n (f32 output only): float4 squares strided over the workgroup, the
// tail by the first threads, elementwise output.
template <bool RMS>
__global__ __launch_bounds__(kNormThreads) void norm_rows_any_kernel(NormArgs a) {
#pragma clang fp contract(off)
    extern __shared__ __align__(16) float s_sq[];
    __shared__ float s_part[4];
    __shared__ float s_tail[4];
    __shared__ float s_scale;
    const int n = a.n;
    const int vq = n / 4;
    const int st = norm_sq_stride(n);
    const float* x = a.x + (long)blockIdx.x * a.x_stride;
    const int tid = threadIdx.x;
    for (int i = tid; i < vq; i += kNormThreads) {
        const float4 v = ld4(x + 4 * i);
        s_sq[0 * st + i] = v.x * v.x;
        s_sq[1 * st + i] = v.y * v.y;
        s_sq[2 * st + i] = v.z * v.z;
        s_sq[3 * st + i] = v.w * v.w;
    }
    if (tid < n - 4 * vq) {
        const float v = x[4 * vq + tid];
        s_tail[tid] = v * v;
    }
    __syncthreads();
    norm_scale<RMS>(s_sq, st, vq, n, s_tail, a.eps, s_part, &s_scale);
    __syncthreads();
    const float scale = s_scale;
    float* o = a.out + (long)blockIdx.x * a.out_stride;
    for (int e = tid; e < n; e += kNormThreads) {
        float y;
        if (RMS) {
            const float nx = x[e] * scale;
            y = nx * a.w[e];
        } else {
            y = x[e] * scale;
        }
        o[e] = y;
    }
}

// ---- SwiGLU: out[i] = silu(gate[i]) * up[i] over rows of n ----

struct SwigluArgs {
    const float* gate;  // [rows][n] contiguous
    const float* up;
    long total;         // rows * n
    int n;
    float* out;         // [rows][n] or nullptr
    Q8Out q8;           // Q8_0 output, or q8.q == nullptr (then n % 32 == 0)
};

__global__ __launch_bounds__(256) void swiglu_kernel(SwigluArgs a) {
#pragma clang fp contract(off)
    if (a.q8.q) {
        const long nblk = a.total / 32;
        const long i = ((long)blockIdx.x * blockDim.x + threadIdx.x) >> 2;
        const int part = threadIdx.x & 3;
        if (i >= nblk) return;  // uniform over the quad
        const long e0 = i * 32 + 8 * part;
        const float4 g0 = ld4(a.gate + e0), g1 = ld4(a.gate + e0 + 4);
        const float4 u0 = ld4(a.up + e0), u1 = ld4(a.up + e0 + 4);
        const float4 y0 = make_float4(jit_silu(g0.x) * u0.x, jit_silu(g0.y) * u0.y,
                                      jit_silu(g0.z) * u0.z, jit_silu(g0.w) * u0.w);
        const float4 y1 = make_float4(jit_silu(g1.x) * u1.x, jit_silu(g1.y) * u1.y,
                                      jit_silu(g1.z) * u1.z, jit_silu(g1.w) * u1.w);
        if (a.out) {
            *reinterpret_cast<float4*>(a.out + e0) = y0;
            *reinterpret_cast<float4*>(a.out + e0 + 4) = y1;
        }
        const int nb = a.n / 32;
        const long row = i / nb;
        store_q8_quad(a.q8, row, (int)(i - row * nb), part, y0, y1);
        return;
    }
    for (long e = (long)blockIdx.x * blockDim.x + threadIdx.x; e < a.total;
         e += (long)gridDim.x * blockDim.x)
        a.out[e] = jit_silu(a.gate[e]) * a.up[e];
}

// ---- residual_add: out[i] = a[i] + b[i] ----

__global__ __launch_bounds__(256) void add_kernel(const float* x, const float* y, long n,
                                                  float* out) {
    for (long e = (long)blockIdx.x * blockDim.x + threadIdx.x; e < n;
         e += (long)gridDim.x * blockDim.x)
        out[e] = x[e] + y[e];
}

// ---- mean pool of embed_tokens (transformer.rs:934-950) ----
// accum starts at 0 and takes accum[i] += normed_b[i] * inv_batch for b in
// order: a product then a sum per row, thread per element.

__global__ __launch_bounds__(256) void mean_pool_kernel(const float* rows, int n, int dim,
                                                        float inv, float* out) {
#pragma clang fp contract(off)
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= dim) return;
    float acc = 0.0f;
    for (int b = 0; b < n; ++b) {
        const float t = rows[(long)b * dim + i] * inv;
        acc = acc + t;
    }
    out[i] = acc;
}

// ---- token embedding rows: dequantize_row_q4_0 of row tokens[t] ----
// Thread per block: (q - 8) as f32 * d, low nibbles to elements 0..15 and
// high nibbles to 16..31 (blocks.rs:85-99).

__global__ __launch_bounds__(256) void embed_rows_kernel(const uint8_t* qs, const uint16_t* d,
                                                         int d_stride, int nb, int vocab,
                                                         const int32_t* tokens, int n,
                                                         float* out, int* bad) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)n * nb) return;
    const int t = (int)(i / nb), b = (int)(i - (long)t * nb);
    const int tok = tokens[t];
    float* o = out + (long)t * nb * 32 + 32 * b;
    if (tok < 0 || tok >= vocab) {  // the host checks host-side ids; device ids are flagged
        if (b == 0) atomicOr(bad, 1);
        return;
    }
    const uint4 w = *reinterpret_cast<const uint4*>(qs + ((long)tok * nb + b) * 16);
    const float sc = __half2float(__ushort_as_half(d[(long)tok * d_stride + b]));
    const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        float lo[4], hi[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int byte = (wd[k] >> (8 * j)) & 0xFF;
            lo[j] = (float)((byte & 0x0F) - 8) * sc;
            hi[j] = (float)((byte >> 4) - 8) * sc;
        }
        *reinterpret_cast<float4*>(o + 4 * k) = make_float4(lo[0], lo[1], lo[2], lo[3]);
        *reinterpret_cast<float4*>(o + 16 + 4 * k) = make_float4(hi[0], hi[1], hi[2], hi[3]);
    }
}

// ---- sample_argmax: the first index of the maximum ----
// The reference scans in order with `val > best` from logits[0]: NaN never
// wins after the first element, and a NaN first element wins outright.  In
// parallel: each thread keeps its best non-NaN (value, index), ties go to the
// lower index, and logits[0] being NaN short-cuts to 0.

constexpr int kArgmaxThreads = 1024;

// Over the per-workgroup parts of the lm_head projection (its epilogue keeps
// each workgroup's best row): one round of loads, then the wave and
// workgroup merges.
constexpr int kArgmaxPartsPerThread = 16;

__global__ __launch_bounds__(kArgmaxThreads) void argmax_parts_kernel(const ArgmaxPart* parts,
                                                                      int n_parts, const float* x,
                                                                      int32_t* out) {
    __shared__ float s_v[kArgmaxThreads / 64];
    __shared__ int s_i[kArgmaxThreads / 64];
    float bv = 0.0f;
    int bi = -1;
    for (int base = 0; base < n_parts; base += kArgmaxThreads * kArgmaxPartsPerThread) {
        ArgmaxPart q[kArgmaxPartsPerThread];
#pragma unroll
        for (int u = 0; u < kArgmaxPartsPerThread; ++u) {
            const int k = base + u * kArgmaxThreads + (int)threadIdx.x;
            q[u] = k < n_parts ? parts[k] : ArgmaxPart{0.0f, -1};
        }
#pragma unroll
        for (int u = 0; u < kArgmaxPartsPerThread; ++u) argmax_merge(bv, bi, q[u].v, q[u].i);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float v2 = __shfl_xor(bv, off);
        const int i2 = __shfl_xor(bi, off);
        argmax_merge(bv, bi, v2, i2);
    }
    if ((threadIdx.x & 63) == 0) {
        s_v[threadIdx.x >> 6] = bv;
        s_i[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kArgmaxThreads / 64; ++w) argmax_merge(bv, bi, s_v[w], s_i[w]);
        const float x0 = x[0];
        out[0] = (x0 != x0 || bi < 0) ? 0 : bi;
    }
}

template <bool RMS>
hipError_t launch_norm_t(const NormArgs& a, int rows, hipStream_t st) {
    const size_t lds = (size_t)4 * norm_sq_stride(a.n) * sizeof(float);
    const bool blocks = a.n % 32 == 0;
    const void* fn = blocks ? reinterpret_cast<const void*>(norm_rows_kernel<RMS>)
                            : reinterpret_cast<const void*>(norm_rows_any_kernel<RMS>);
    if (lds > 64 * 1024) {
        const hipError_t e =
            hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    if (blocks)
        hipLaunchKernelGGL(norm_rows_kernel<RMS>, dim3(rows), dim3(kNormThreads), lds, st, a);
    else
        hipLaunchKernelGGL(norm_rows_any_kernel<RMS>, dim3(rows), dim3(kNormThreads), lds, st, a);
    return hipGetLastError();
}

}  // namespace

int norm_max_n() { return 16384; }

hipError_t launch_rmsnorm(const float* x, long x_stride, const float* w, int rows, int n,
                          float eps, float* out, long out_stride, const Q8Out& q8,
                          hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    if (n < 1 || n > norm_max_n() || (q8.q && n % 32) || (!q8.q && !out))
        return hipErrorInvalidValue;
    NormArgs a{x, x_stride, w, n, eps, out, out_stride, q8};
    return w ? launch_norm_t<true>(a, rows, st) : launch_norm_t<false>(a, rows, st);
}

hipError_t launch_swiglu(const float* gate, const float* up, long total, int n, float* out,
                         const Q8Out& q8, hipStream_t st) {
    if (total <= 0) return hipSuccess;
    if ((q8.q && (n <= 0 || n % 32 || total % n)) || (!q8.q && !out)) return hipErrorInvalidValue;
    SwigluArgs a{gate, up, total, n, out, q8};
    long grid;
    if (q8.q) {
        grid = (total / 32 + 63) / 64;
    } else {
        grid = (total + 255) / 256;
        if (grid > 65536) grid = 65536;
    }
    hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)grid), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_add(const float* x, const float* y, long n, float* out, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    long grid = (n + 255) / 256;
    if (grid > 65536) grid = 65536;
    hipLaunchKernelGGL(add_kernel, dim3((unsigned)grid), dim3(256), 0, st, x, y, n, out);
    return hipGetLastError();
}

hipError_t launch_embed_rows(const uint8_t* qs, const uint16_t* d, int nb, int vocab,
                             const int32_t* tokens, int n, float* out, int* bad,
                             hipStream_t st) {
    if (n <= 0) return hipSuccess;
    const long threads = (long)n * nb;
    hipLaunchKernelGGL(embed_rows_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                       st, qs, d, q4_scale_stride(nb), nb, vocab, tokens, n, out, bad);
    return hipGetLastError();
}

hipError_t launch_mean_pool(const float* rows, int n, int dim, float inv, float* out,
                            hipStream_t st) {
    if (n <= 0 || dim <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(mean_pool_kernel, dim3((dim + 255) / 256), dim3(256), 0, st, rows, n, dim,
                       inv, out);
    return hipGetLastError();
}

hipError_t launch_argmax_parts(const ArgmaxPart* parts, int n_parts, const float* x, int32_t* out,
                               hipStream_t st) {
    if (n_parts <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(argmax_parts_kernel, dim3(1), dim3(kArgmaxThreads), 0, st, parts, n_parts,
                       x, out);
    return hipGetLastError();
}

}  // namespace slm
