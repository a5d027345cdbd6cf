// The reductions of the JIT normalisation kernels (FuseGraph::rmsnorm and
// l2_norm, graph.rs:141-193, lowered by lower.rs:244-389), shared by the
// standalone norm kernel and the projections that normalize their own input.
#pragma once

#include <hip/hip_runtime.h>

#include "attn_common.h"
#include "jit_math.h"

namespace slm {

// A row of n = 32 nb elements over a 256-thread workgroup: quad q owns
// blocks q, q + 64, ... (lane part p: elements 8p..8p+7), pass k holding
// block q + 64k, so x and the norm weights are loaded once and stay in
// registers across the reduction.
template <int KP>
struct NormRow {
    float4 x[KP][2], w[KP][2];
};

__host__ __device__ constexpr int norm_sq_stride(int n) { return n / 4 + 4; }

// Loads the row's passes; block addresses are clamped into the row (blocks
// past nb are loaded but never used).
template <int KP, bool RMS>
__device__ __forceinline__ void norm_row_load(NormRow<KP>& r, const float* x, const float* w,
                                              int nb) {
    const int tid = threadIdx.x;
    const int part = tid & 3;
    const int passes = (nb + 63) / 64;
#pragma unroll
    for (int k = 0; k < KP; ++k) {
        if (k >= passes) break;  // uniform
        const int e0 = 32 * min((tid >> 2) + 64 * k, nb - 1) + 8 * part;
        r.x[k][0] = ld4(x + e0);
        r.x[k][1] = ld4(x + e0 + 4);
        if (RMS) {
            r.w[k][0] = ld4(w + e0);
            r.w[k][1] = ld4(w + e0 + 4);
        }
    }
}

// The squares, transposed for the lane chains: element e = 32 blk + 8 part
// + j goes to chain j % 4 at position 8 blk + 2 part + j / 4 of s_sq
// ([4][st], st = norm_sq_stride(32 nb)).
template <int KP>
__device__ __forceinline__ void norm_row_squares(const NormRow<KP>& r, int nb, float* s_sq) {
#pragma clang fp contract(off)
    const int tid = threadIdx.x;
    const int part = tid & 3;
    const int st = norm_sq_stride(32 * nb);
    const int passes = (nb + 63) / 64;
#pragma unroll
    for (int k = 0; k < KP; ++k) {
        if (k >= passes) break;
        const int blk = (tid >> 2) + 64 * k;
        if (blk < nb) {
            const int i0 = 8 * blk + 2 * part;
            const float v[8] = {r.x[k][0].x, r.x[k][0].y, r.x[k][0].z, r.x[k][0].w,
                                r.x[k][1].x, r.x[k][1].y, r.x[k][1].z, r.x[k][1].w};
#pragma unroll
            for (int j = 0; j < 8; ++j) s_sq[(j & 3) * st + i0 + (j >> 2)] = v[j] * v[j];
        }
    }
}

// Pass k's eight outputs: x * scale, then times the weight for RMSNorm, per
// element (the store pass of graph.rs:141-156 / 182-193).
template <int KP, bool RMS>
__device__ __forceinline__ void norm_row_values(const NormRow<KP>& r, int k, float scale,
                                                float4* f0, float4* f1) {
#pragma clang fp contract(off)
    float v[8] = {r.x[k][0].x, r.x[k][0].y, r.x[k][0].z, r.x[k][0].w,
                  r.x[k][1].x, r.x[k][1].y, r.x[k][1].z, r.x[k][1].w};
    if (RMS) {
        const float wv[8] = {r.w[k][0].x, r.w[k][0].y, r.w[k][0].z, r.w[k][0].w,
                             r.w[k][1].x, r.w[k][1].y, r.w[k][1].z, r.w[k][1].w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float nx = v[j] * scale;
            v[j] = nx * wv[j];
        }
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = v[j] * scale;
    }
    *f0 = make_float4(v[0], v[1], v[2], v[3]);
    *f1 = make_float4(v[4], v[5], v[6], v[7]);
}

// The four lane chains of the squares in s_sq (lanes 0..3 of wave 0), then
// lane 0 combines them with the tail and returns the scale in s_scale.
// T terms are added while the next T are read from LDS (two buffers of T/4
// float4 registers; a smaller T suits a kernel with other registers live).
template <bool RMS, int T = 32>
__device__ __forceinline__ void norm_scale(const float* s_sq, int st, int vq, int n,
                                           const float* s_tail, float eps, float* s_part,
                                           float* s_scale) {
#pragma clang fp contract(off)
    static_assert(T % 4 == 0 && T >= 8, "T: whole float4 loads");
    constexpr int F4 = T / 4;
    const int tid = threadIdx.x;
    if (tid < 4) {
        // two buffers of T terms take turns (no register copies between
        // the dependent adds): one is added while the other is read
        const float* t = s_sq + tid * st;
        float acc = 0.0f;
        int i = 0;
        if (vq >= 2 * T) {
            float4 A[F4], B[F4];
#define SLM_LOADT(buf, off)                                                               \
    _Pragma("unroll") for (int k = 0; k < F4; ++k) buf[k] =                               \
        *reinterpret_cast<const float4*>(t + (off) + 4 * k)
#define SLM_ADDT(buf)                                                                     \
    _Pragma("unroll") for (int k = 0; k < F4; ++k) {                                      \
        acc = acc + buf[k].x;                                                             \
        acc = acc + buf[k].y;                                                             \
        acc = acc + buf[k].z;                                                             \
        acc = acc + buf[k].w;                                                             \
    }
#define SLM_PIN()                                                                         \
    do {                                                                                  \
        asm volatile("" : "+v"(acc)::"memory");                                           \
        __builtin_amdgcn_sched_barrier(0);                                                \
    } while (0)
            SLM_LOADT(A, 0);
            for (; i + 3 * T <= vq; i += 2 * T) {  // A holds terms [i, i + T)
                // each read group stays where it is: an empty asm that takes
                // the sum and clobbers memory orders the adds and the reads
                // for the IR passes, the scheduling barrier for the machine
                // scheduler (a read hoisted above the adds of the buffer it
                // refills makes the compiler copy that buffer first)
                SLM_LOADT(B, i + T);
                SLM_PIN();
                SLM_ADDT(A);
                SLM_PIN();
                SLM_LOADT(A, i + 2 * T);
                SLM_PIN();
                SLM_ADDT(B);
                SLM_PIN();
            }
            if (i + 2 * T <= vq) {
                SLM_LOADT(B, i + T);
                SLM_ADDT(A);
                SLM_ADDT(B);
                i += 2 * T;
            } else {
                SLM_ADDT(A);
                i += T;
            }
#undef SLM_LOADT
#undef SLM_ADDT
#undef SLM_PIN
        }
        for (; i < vq; ++i) acc = acc + t[i];
        s_part[tid] = acc;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (tid == 0) {
        float s = (s_part[0] + s_part[1]) + (s_part[2] + s_part[3]);
        for (int i = 0; i < n - 4 * vq; ++i) s = s + s_tail[i];
        float scale;
        if (RMS) {  // graph.rs:141-156
            const float inv_n = __fdiv_rn(1.0f, (float)n);
            const float mean = s * inv_n;
            const float var = mean + eps;
            scale = __fdiv_rn(1.0f, sqrt_rn(var));
        } else {    // graph.rs:182-193
            const float var = s + eps;
            scale = __fdiv_rn(1.0f, sqrt_rn(var));
        }
        *s_scale = scale;
    }
}

}  // namespace slm
