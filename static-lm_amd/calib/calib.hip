// Measurement helpers for the bench: the fp32 MFMA issue rate and the HBM
// streaming-read rate this device actually reaches, to set next to the
// published peaks the roofline fractions use.  Not part of the attention
// path; no counterpart in static-lm.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include "slm_calib.h"
#include "attn_common.h"

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kChains = 16;  // independent accumulators per wave

// Each wave issues iters * kChains v_mfma_f32_16x16x4_f32 (2048 flop each)
// over kChains independent accumulators.  Swept on MI355X: 16 chains at two
// waves per SIMD reach 155 TFLOP/s (4 chains: 118, 8 chains: 134).
__global__ __launch_bounds__(256) void mfma_f32_rate_kernel(float* out, int iters, float seed) {
    const float a = seed * (float)(threadIdx.x + 1);
    const float b = seed;
    v4f c[kChains];
#pragma unroll
    for (int k = 0; k < kChains; ++k) c[k] = v4f{0.f, 0.f, 0.f, 0.f};
    for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int k = 0; k < kChains; ++k)
            c[k] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c[k], 0, 0, 0);
    }
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < kChains; ++k) s += c[k].x + c[k].y + c[k].z + c[k].w;
    out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// Each workgroup streams its own contiguous range of per_wg float4, four
// 128-bit loads in flight per thread (the fastest pattern of a sweep over
// grid-stride and per-workgroup ranges, 1-8 loads in flight, 1-32
// workgroups per CU: 7.28 TB/s nontemporal at two workgroups per CU).
template <bool NT>
__global__ __launch_bounds__(256) void hbm_read_kernel(const float* p, size_t per_wg, float* out) {
    constexpr int U = 4;
    float acc[U] = {};
    const float* b = p + 4 * (size_t)blockIdx.x * per_wg;
    size_t i = threadIdx.x;
    for (; i + 256 * (U - 1) < per_wg; i += 256 * U) {
        float4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u)
            v[u] = NT ? slm::ld4_stream(b + 4 * (i + 256 * u)) : slm::ld4(b + 4 * (i + 256 * u));
        // all U loads issue before the first wait
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < U; ++u) acc[u] += (v[u].x + v[u].y) + (v[u].z + v[u].w);
    }
    for (; i < per_wg; i += 256) {
        const float4 v = slm::ld4(b + 4 * i);
        acc[0] += (v.x + v.y) + (v.z + v.w);
    }
    out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
}

struct Session {
    int prev = -1;
    hipStream_t st = nullptr;
    hipEvent_t a = nullptr, b = nullptr;
    float* out = nullptr;
    float* buf = nullptr;
    hipError_t err = hipSuccess;

    bool ok(hipError_t e) {
        if (err == hipSuccess) err = e;
        return err == hipSuccess;
    }
    ~Session() {
        if (buf) (void)hipFree(buf);
        if (out) (void)hipFree(out);
        if (a) (void)hipEventDestroy(a);
        if (b) (void)hipEventDestroy(b);
        if (st) (void)hipStreamDestroy(st);
        if (prev >= 0) (void)hipSetDevice(prev);
    }
};

int open_session(Session& s, int device, int* cus) {
    if (!s.ok(hipGetDevice(&s.prev))) return SLM_ERR_HIP;
    if (!s.ok(hipSetDevice(device))) return SLM_ERR_HIP;
    hipDeviceProp_t prop;
    if (!s.ok(hipGetDeviceProperties(&prop, device))) return SLM_ERR_HIP;
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) return SLM_ERR_DEVICE;
    *cus = prop.multiProcessorCount;
    if (!s.ok(hipStreamCreateWithFlags(&s.st, hipStreamNonBlocking))) return SLM_ERR_HIP;
    if (!s.ok(hipEventCreate(&s.a)) || !s.ok(hipEventCreate(&s.b))) return SLM_ERR_HIP;
    return SLM_OK;
}

// Best of `reps` timed runs of launch(), after one untimed run.
template <class F>
int best_ms(Session& s, int reps, F launch, double* ms) {
    launch();
    if (!s.ok(hipGetLastError()) || !s.ok(hipStreamSynchronize(s.st))) return SLM_ERR_HIP;
    double best = 1e30;
    for (int r = 0; r < reps; ++r) {
        if (!s.ok(hipEventRecord(s.a, s.st))) return SLM_ERR_HIP;
        launch();
        if (!s.ok(hipGetLastError()) || !s.ok(hipEventRecord(s.b, s.st))) return SLM_ERR_HIP;
        if (!s.ok(hipEventSynchronize(s.b))) return SLM_ERR_HIP;
        float t = 0.f;
        if (!s.ok(hipEventElapsedTime(&t, s.a, s.b))) return SLM_ERR_HIP;
        if (t < best) best = t;
    }
    *ms = best;
    return SLM_OK;
}

}  // namespace

extern "C" {

int slm_calib_mfma_f32(int32_t device, int32_t iters, double* tflops, double* ms) {
    if (!tflops || !ms || iters <= 0) return SLM_ERR_ARG;
    Session s;
    int cus = 0;
    int rc = open_session(s, device, &cus);
    if (rc != SLM_OK) return rc;
    const int wgs = 2 * cus;  // 8 waves per CU: two per SIMD
    if (!s.ok(hipMalloc(&s.out, (size_t)wgs * 256 * sizeof(float)))) return SLM_ERR_HIP;
    rc = best_ms(s, 3, [&] {
        hipLaunchKernelGGL(mfma_f32_rate_kernel, dim3(wgs), dim3(256), 0, s.st, s.out, iters,
                           1e-3f);
    }, ms);
    if (rc != SLM_OK) return rc;
    const double flops = (double)wgs * 4 * iters * kChains * 2.0 * 16 * 16 * 4;
    *tflops = flops / (*ms * 1e-3) / 1e12;
    return SLM_OK;
}

int slm_calib_hbm_read(int32_t device, int64_t bytes, int32_t nontemporal, double* gbs) {
    if (!gbs || bytes < (1 << 20) || bytes % 16 != 0) return SLM_ERR_ARG;
    Session s;
    int cus = 0;
    int rc = open_session(s, device, &cus);
    if (rc != SLM_OK) return rc;
    const int wgs = 2 * cus;
    if (!s.ok(hipMalloc(&s.out, (size_t)wgs * 256 * sizeof(float)))) return SLM_ERR_HIP;
    if (!s.ok(hipMalloc(&s.buf, (size_t)bytes))) return SLM_ERR_HIP;
    if (!s.ok(hipMemsetAsync(s.buf, 0, (size_t)bytes, s.st))) return SLM_ERR_HIP;
    // whole float4 per workgroup; the rest of the buffer is not read or counted
    const size_t per_wg = (size_t)bytes / 16 / wgs;
    if (per_wg == 0) return SLM_ERR_ARG;
    double ms = 0.0;
    rc = best_ms(s, 5, [&] {
        if (nontemporal)
            hipLaunchKernelGGL(hbm_read_kernel<true>, dim3(wgs), dim3(256), 0, s.st, s.buf,
                               per_wg, s.out);
        else
            hipLaunchKernelGGL(hbm_read_kernel<false>, dim3(wgs), dim3(256), 0, s.st, s.buf,
                               per_wg, s.out);
    }, &ms);
    if (rc != SLM_OK) return rc;
    *gbs = (double)(per_wg * wgs * 16) / (ms * 1e-3) / 1e9;
    return SLM_OK;
}

}  // extern "C"
