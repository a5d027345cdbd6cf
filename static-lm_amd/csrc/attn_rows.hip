// Batched attention rows for gfx950 (VALU), one workgroup per (row, KV head
// x head batch) walking the row's whole causal range.
//
// Serves the per-row loop of forward_batch_with_kv (transformer.rs:563-593)
// for shapes the MFMA prefill kernel does not take: row r at position
// p = start + r attends to cache rows 0..p with
//   out_h = sum_t softmax_t(q_h . K[t, g] / sqrt(hd)) V[t, g], g = h / kv_mul
// (transformer.rs:273-321).  Lane layout and online softmax as in the decode
// kernel: LPG lanes per position, one softmax state per lane group, merged
// across lane groups with shuffles and across waves through LDS.
#include <math.h>

#include "attn_common.h"
#include "slm_internal.h"

namespace slm {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;

template <int HD, int GB>
constexpr int rows_tp() {
    constexpr int fpl = HD / LaneCfg<HD>::LPG;
    return (fpl <= 8) ? 4 : ((GB <= 2) ? 4 : 2);
}

template <int HD, int GB>
__global__ __launch_bounds__(kThreads) void attn_rows_kernel(RowsArgs a, int dim, int num_heads,
                                                             int kv_dim, int kv_mul, int half,
                                                             float scale_log2) {
    constexpr int LPG = LaneCfg<HD>::LPG;
    constexpr int FPL = HD / LPG;
    constexpr int NV = FPL / 4;
    constexpr int GPW = 64 / LPG;
    constexpr int TP = rows_tp<HD, GB>();
    constexpr int IT = kWaves * GPW * TP;
    static_assert(FPL % 4 == 0, "lane slice must be whole float4s");

    const int row = blockIdx.y;
    const int pos = a.start + row;
    const int seq_len = pos + 1;
    const int nhb = kv_mul / GB;
    const int g = blockIdx.x / nhb;
    const int h0 = g * kv_mul + (blockIdx.x % nhb) * GB;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int li = lane % LPG;
    const int lg = lane / LPG;

    float4 qr[GB][NV];
    {
        const float* qrow = a.q + (long)row * dim;
        const long tr = (long)pos * half;
#pragma unroll
        for (int i = 0; i < GB; ++i) {
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                const int d = 4 * (v * LPG + li);
                float4 x = ld4(qrow + (h0 + i) * HD + d);
                if (a.cos_t != nullptr)
                    x = rope4_exact(x, a.cos_t + tr + (d >> 1), a.sin_t + tr + (d >> 1));
                x.x *= scale_log2;
                x.y *= scale_log2;
                x.z *= scale_log2;
                x.w *= scale_log2;
                qr[i][v] = x;
            }
        }
    }

    float m[GB], l[GB];
    float4 o[GB][NV];
#pragma unroll
    for (int i = 0; i < GB; ++i) {
        m[i] = -INFINITY;
        l[i] = 0.0f;
#pragma unroll
        for (int v = 0; v < NV; ++v) o[i][v] = make_float4(0.f, 0.f, 0.f, 0.f);
    }

    const float* kbase = a.k_cache + g * HD + 4 * li;
    const float* vbase = a.v_cache + g * HD + 4 * li;
    for (int tb = 0; tb < seq_len; tb += IT) {
        float4 kr[TP][NV], vr[TP][NV];
        bool valid[TP];
#pragma unroll
        for (int tp = 0; tp < TP; ++tp) {
            const int t = tb + (tp * kWaves + wave) * GPW + lg;
            valid[tp] = t < seq_len;
            const long tt = valid[tp] ? t : 0;
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                kr[tp][v] = ld4(kbase + tt * kv_dim + 4 * v * LPG);
                vr[tp][v] = ld4(vbase + tt * kv_dim + 4 * v * LPG);
            }
        }
        attend_tile<LPG, NV, GB, TP>(qr, kr, vr, valid, m, l, o);
    }
    merge_lane_groups<LPG, NV, GB>(m, l, o);

    __shared__ __align__(16) float s_o[kWaves][GB][HD];
    __shared__ float s_m[kWaves][GB];
    __shared__ float s_l[kWaves][GB];
    if (lg == 0) {
#pragma unroll
        for (int i = 0; i < GB; ++i) {
#pragma unroll
            for (int v = 0; v < NV; ++v)
                *reinterpret_cast<float4*>(&s_o[wave][i][4 * (v * LPG + li)]) = o[i][v];
            if (li == 0) {
                s_m[wave][i] = m[i];
                s_l[wave][i] = l[i];
            }
        }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < GB * HD; idx += kThreads) {
        const int i = idx / HD;
        const int d = idx - i * HD;
        float mx = s_m[0][i];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) mx = fmaxf(mx, s_m[w][i]);
        const float mu = (mx == -INFINITY) ? 0.0f : mx;
        float acc_o = 0.0f, acc_l = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float wt = fast_exp2(s_m[w][i] - mu);
            acc_o += wt * s_o[w][i][d];
            acc_l += wt * s_l[w][i];
        }
        a.out[(long)row * dim + (h0 + i) * HD + d] = acc_o / acc_l;
    }
}

template <int HD, int GB>
hipError_t launch_rows_t(const Shape& s, const RowsArgs& a, hipStream_t st) {
    const float scale_log2 = 1.4426950408889634f / sqrtf((float)HD);
    const int kMaxRows = 65535;
    for (int r0 = 0; r0 < a.rows; r0 += kMaxRows) {
        RowsArgs b = a;
        b.q = a.q + (long)r0 * s.dim;
        b.out = a.out + (long)r0 * s.dim;
        b.start = a.start + r0;
        b.rows = (a.rows - r0 < kMaxRows) ? a.rows - r0 : kMaxRows;
        const dim3 grid(s.num_kv_heads * (s.kv_mul / GB), b.rows);
        hipLaunchKernelGGL((attn_rows_kernel<HD, GB>), grid, dim3(kThreads), 0, st, b, s.dim,
                           s.num_heads, s.kv_dim, s.kv_mul, s.half, scale_log2);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

template <int HD>
hipError_t launch_rows_hd(const Shape& s, const RowsArgs& a, hipStream_t st) {
    switch (pick_gb(s.kv_mul)) {
        case 4: return launch_rows_t<HD, 4>(s, a, st);
        case 3: return launch_rows_t<HD, 3>(s, a, st);
        case 2: return launch_rows_t<HD, 2>(s, a, st);
        default: return launch_rows_t<HD, 1>(s, a, st);
    }
}

}  // namespace

bool head_dim_supported(int hd) {
    switch (hd) {
        case 16: case 32: case 48: case 64: case 96: case 128: case 256:
            return true;
        default:
            return false;
    }
}

hipError_t launch_attn_rows(const Shape& s, const RowsArgs& a, hipStream_t st) {
    switch (s.head_dim) {
        case 16: return launch_rows_hd<16>(s, a, st);
        case 32: return launch_rows_hd<32>(s, a, st);
        case 48: return launch_rows_hd<48>(s, a, st);
        case 64: return launch_rows_hd<64>(s, a, st);
        case 96: return launch_rows_hd<96>(s, a, st);
        case 128: return launch_rows_hd<128>(s, a, st);
        case 256: return launch_rows_hd<256>(s, a, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace slm
