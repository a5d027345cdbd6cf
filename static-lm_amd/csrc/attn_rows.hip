// Split-K ("flash-decoding") attention over the KV cache for gfx950.
//
// Replaces the per-head loops of causal_multi_head_attention_jit
// (transformer.rs:273-321): for query row r at position p = start + r and
// head h (KV head g = h / kv_mul, transformer.rs:295),
//   out_h = sum_t softmax_t(q_h . K[t, g] / sqrt(hd)) V[t, g],  t = 0..p.
//
// Mapping.  grid = (split, KV head x head batch, row).  A workgroup owns the
// positions [split*chunk, min(p+1, (split+1)*chunk)) of one KV head and GB of
// its kv_mul query heads, so each K/V row segment it loads from HBM serves GB
// heads (GQA sharing; the reference re-reads it once per head).  Inside a
// wave, LPG lanes form a group that holds one position's head_dim floats as
// 128-bit loads, LPG*16 contiguous bytes per group per instruction.  Each
// group keeps its own online-softmax state (running max in the log2 domain,
// running sum, output accumulator) over the positions it sees; the states
// are merged across groups with lane shuffles, across waves through LDS, and
// across splits by attn_combine_kernel (log-sum-exp merge).  A row whose
// sequence fits one split writes its normalised output directly.
//
// Numerics.  q is pre-scaled by log2(e)/sqrt(hd) so exp2 replaces exp; dot
// products and sums use fused multiply-adds in an order different from the
// reference's sequential chains.  The result matches the reference within
// the tolerance its own tests use, not bit for bit.
#include <math.h>

#include "slm_internal.h"

namespace slm {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kMaxSplits = 1024;

// Lanes per position group for each compiled head_dim: every lane holds
// head_dim / LPG floats (a multiple of 4, for 128-bit loads).
template <int HD>
struct RowsCfg;
template <> struct RowsCfg<16> { static constexpr int LPG = 4; };
template <> struct RowsCfg<32> { static constexpr int LPG = 8; };
template <> struct RowsCfg<48> { static constexpr int LPG = 4; };
template <> struct RowsCfg<64> { static constexpr int LPG = 8; };
template <> struct RowsCfg<96> { static constexpr int LPG = 8; };
template <> struct RowsCfg<128> { static constexpr int LPG = 8; };
template <> struct RowsCfg<256> { static constexpr int LPG = 16; };

// Positions each lane group takes per loop iteration.
template <int HD, int GB>
constexpr int rows_tp() {
    constexpr int fpl = HD / RowsCfg<HD>::LPG;
    return (fpl <= 8) ? 4 : ((GB <= 2) ? 4 : 2);
}

template <int HD, int GB>
constexpr int rows_span() {
    return kWaves * (64 / RowsCfg<HD>::LPG) * rows_tp<HD, GB>();
}

int pick_gb(int kv_mul) {
    for (int gb = 4; gb > 1; --gb)
        if (kv_mul % gb == 0) return gb;
    return 1;
}

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __builtin_amdgcn_update_dpp(0.0f, x, CTRL, 0xF, 0xF, false);
}

// Sum over the LPG lanes of a group; every lane of the group gets the total.
template <int LPG>
__device__ __forceinline__ float group_sum(float x) {
    if constexpr (LPG >= 2) x += dpp<0xB1>(x);   // quad_perm [1,0,3,2]
    if constexpr (LPG >= 4) x += dpp<0x4E>(x);   // quad_perm [2,3,0,1]
    if constexpr (LPG >= 8) x += dpp<0x141>(x);  // row_half_mirror
    if constexpr (LPG >= 16) x += dpp<0x140>(x); // row_mirror
    if constexpr (LPG >= 32) x += __shfl_xor(x, 16);
    return x;
}

__device__ __forceinline__ float fast_exp2(float x) {
    return __builtin_amdgcn_exp2f(x);
}

__device__ __forceinline__ float4 ld4(const float* p) {
    return *reinterpret_cast<const float4*>(p);
}

__device__ __forceinline__ float4 rotate4(float4 x, const float* c,
                                          const float* s) {
    // pairs (x, y) and (z, w) at table columns c[0], c[1]
    float4 r;
    r.x = x.x * c[0] - x.y * s[0];
    r.y = x.x * s[0] + x.y * c[0];
    r.z = x.z * c[1] - x.w * s[1];
    r.w = x.z * s[1] + x.w * c[1];
    return r;
}

template <int HD, int GB>
__global__ __launch_bounds__(kThreads) void attn_rows_kernel(
    RowsArgs a, int dim, int num_heads, int kv_dim, int kv_mul, int half,
    float scale_log2) {
    constexpr int LPG = RowsCfg<HD>::LPG;
    constexpr int FPL = HD / LPG;
    constexpr int NV = FPL / 4;
    constexpr int GPW = 64 / LPG;
    constexpr int TP = rows_tp<HD, GB>();
    constexpr int IT = kWaves * GPW * TP;
    static_assert(FPL % 4 == 0, "lane slice must be whole float4s");

    const int row = blockIdx.z;
    const int pos = a.start + row;
    const int seq_len = pos + 1;
    const int n_splits = (seq_len + a.chunk - 1) / a.chunk;
    const int split = blockIdx.x;
    if (split >= n_splits) return;  // uniform over the workgroup
    const int nhb = kv_mul / GB;
    const int g = blockIdx.y / nhb;
    const int h0 = g * kv_mul + (blockIdx.y % nhb) * GB;
    const int t0 = split * a.chunk;
    const int t1 = min(seq_len, t0 + a.chunk);

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int li = lane % LPG;
    const int lg = lane / LPG;

    // q slice of each head: dims 4*(v*LPG + li) .. +3, rotated and pre-scaled.
    float4 qr[GB][NV];
    {
        const float* qrow = a.q + (long)row * dim;
#pragma unroll
        for (int i = 0; i < GB; ++i) {
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                const int d = 4 * (v * LPG + li);
                float4 x = ld4(qrow + (h0 + i) * HD + d);
                if (a.cos_t != nullptr) {
                    const long tr = (long)pos * half + (d >> 1);
                    x = rotate4(x, a.cos_t + tr, a.sin_t + tr);
                }
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

    for (int tb = t0; tb < t1; tb += IT) {
        float4 kr[TP][NV], vr[TP][NV];
        bool valid[TP];
#pragma unroll
        for (int tp = 0; tp < TP; ++tp) {
            const int t = tb + (tp * kWaves + wave) * GPW + lg;
            valid[tp] = t < t1;
            const long tt = valid[tp] ? t : t0;
            const float* kp = kbase + tt * kv_dim;
            const float* vp = vbase + tt * kv_dim;
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                kr[tp][v] = ld4(kp + 4 * v * LPG);
                vr[tp][v] = ld4(vp + 4 * v * LPG);
            }
        }
#pragma unroll
        for (int i = 0; i < GB; ++i) {
            float sc[TP];
#pragma unroll
            for (int tp = 0; tp < TP; ++tp) {
                float acc = 0.0f;
#pragma unroll
                for (int v = 0; v < NV; ++v) {
                    acc = fmaf(qr[i][v].x, kr[tp][v].x, acc);
                    acc = fmaf(qr[i][v].y, kr[tp][v].y, acc);
                    acc = fmaf(qr[i][v].z, kr[tp][v].z, acc);
                    acc = fmaf(qr[i][v].w, kr[tp][v].w, acc);
                }
                acc = group_sum<LPG>(acc);
                sc[tp] = valid[tp] ? acc : -INFINITY;
            }
            float mx = sc[0];
#pragma unroll
            for (int tp = 1; tp < TP; ++tp) mx = fmaxf(mx, sc[tp]);
            const float mn = fmaxf(m[i], mx);
            const float mu = (mn == -INFINITY) ? 0.0f : mn;
            const float alpha = fast_exp2(m[i] - mu);
            float p[TP];
            float ps = 0.0f;
#pragma unroll
            for (int tp = 0; tp < TP; ++tp) {
                p[tp] = fast_exp2(sc[tp] - mu);
                ps += p[tp];
            }
            l[i] = l[i] * alpha + ps;
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                float4 acc = o[i][v];
                acc.x *= alpha;
                acc.y *= alpha;
                acc.z *= alpha;
                acc.w *= alpha;
#pragma unroll
                for (int tp = 0; tp < TP; ++tp) {
                    acc.x = fmaf(p[tp], vr[tp][v].x, acc.x);
                    acc.y = fmaf(p[tp], vr[tp][v].y, acc.y);
                    acc.z = fmaf(p[tp], vr[tp][v].z, acc.z);
                    acc.w = fmaf(p[tp], vr[tp][v].w, acc.w);
                }
                o[i][v] = acc;
            }
            m[i] = mn;
        }
    }

    // Merge the lane groups of the wave (lanes with equal li hold equal dims).
#pragma unroll
    for (int off = LPG; off < 64; off <<= 1) {
#pragma unroll
        for (int i = 0; i < GB; ++i) {
            const float mo = __shfl_xor(m[i], off);
            const float lo = __shfl_xor(l[i], off);
            const float mn = fmaxf(m[i], mo);
            const float mu = (mn == -INFINITY) ? 0.0f : mn;
            const float wa = fast_exp2(m[i] - mu);
            const float wb = fast_exp2(mo - mu);
            l[i] = l[i] * wa + lo * wb;
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                float4 x = o[i][v];
                x.x = x.x * wa + __shfl_xor(x.x, off) * wb;
                x.y = x.y * wa + __shfl_xor(x.y, off) * wb;
                x.z = x.z * wa + __shfl_xor(x.z, off) * wb;
                x.w = x.w * wa + __shfl_xor(x.w, off) * wb;
                o[i][v] = x;
            }
            m[i] = mn;
        }
    }

    // Merge the waves through LDS and write this split's result.
    __shared__ __align__(16) float s_o[kWaves][GB][HD];
    __shared__ float s_m[kWaves][GB];
    __shared__ float s_l[kWaves][GB];
    if (lg == 0) {
#pragma unroll
        for (int i = 0; i < GB; ++i) {
#pragma unroll
            for (int v = 0; v < NV; ++v)
                *reinterpret_cast<float4*>(&s_o[wave][i][4 * (v * LPG + li)]) =
                    o[i][v];
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
        const int h = h0 + i;
        if (n_splits == 1) {
            a.out[(long)row * dim + h * HD + d] = acc_o / acc_l;
        } else {
            const long pi = ((long)row * a.max_splits + split) * num_heads + h;
            a.part_o[pi * HD + d] = acc_o;
            if (d == 0) {
                a.part_ml[pi * 2] = mx;
                a.part_ml[pi * 2 + 1] = acc_l;
            }
        }
    }
}

// Log-sum-exp merge of the split partials of one (head, row).
template <int HD>
__global__ __launch_bounds__(64) void attn_combine_kernel(RowsArgs a, int dim,
                                                          int num_heads) {
    const int h = blockIdx.x;
    const int row = blockIdx.y;
    const int seq_len = a.start + row + 1;
    const int n_splits = (seq_len + a.chunk - 1) / a.chunk;
    if (n_splits <= 1) return;  // written by attn_rows_kernel
    const long base = (long)row * a.max_splits * num_heads + h;
    float mx = -INFINITY;
    for (int sp = 0; sp < n_splits; ++sp)
        mx = fmaxf(mx, a.part_ml[(base + (long)sp * num_heads) * 2]);
    for (int d = threadIdx.x; d < HD; d += 64) {
        float acc_o = 0.0f, acc_l = 0.0f;
        for (int sp = 0; sp < n_splits; ++sp) {
            const long pi = base + (long)sp * num_heads;
            const float wt = fast_exp2(a.part_ml[pi * 2] - mx);
            acc_o += wt * a.part_o[pi * HD + d];
            acc_l += wt * a.part_ml[pi * 2 + 1];
        }
        a.out[(long)row * dim + h * HD + d] = acc_o / acc_l;
    }
}

template <int HD, int GB>
hipError_t launch_rows_t(const Shape& s, const RowsArgs& a, hipStream_t st) {
    const float scale_log2 = 1.4426950408889634f / sqrtf((float)HD);
    const dim3 grid(a.max_splits, s.num_kv_heads * (s.kv_mul / GB), a.rows);
    hipLaunchKernelGGL((attn_rows_kernel<HD, GB>), grid, dim3(kThreads), 0, st,
                       a, s.dim, s.num_heads, s.kv_dim, s.kv_mul, s.half,
                       scale_log2);
    return hipGetLastError();
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

template <int HD>
int span_hd(int kv_mul) {
    switch (pick_gb(kv_mul)) {
        case 4: return rows_span<HD, 4>();
        case 3: return rows_span<HD, 3>();
        case 2: return rows_span<HD, 2>();
        default: return rows_span<HD, 1>();
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

int rows_iteration_span(const Shape& s) {
    switch (s.head_dim) {
        case 16: return span_hd<16>(s.kv_mul);
        case 32: return span_hd<32>(s.kv_mul);
        case 48: return span_hd<48>(s.kv_mul);
        case 64: return span_hd<64>(s.kv_mul);
        case 96: return span_hd<96>(s.kv_mul);
        case 128: return span_hd<128>(s.kv_mul);
        case 256: return span_hd<256>(s.kv_mul);
        default: return 64;
    }
}

void decode_split_policy(const Shape& s, int seq_len, int* n_splits,
                         int* chunk) {
    // Aim for ~2048 workgroups (8 per CU) once the sequence is long enough,
    // with at least two loop iterations per workgroup and at most kMaxSplits
    // splits.  A pure function of seq_len and the shape.
    const int it = rows_iteration_span(s);
    const int groups = s.num_kv_heads * (s.kv_mul / pick_gb(s.kv_mul));
    const int want = groups >= 2048 ? 1 : 2048 / groups;
    int c = (seq_len + want - 1) / want;
    if (c < 2 * it) c = 2 * it;
    c = (c + it - 1) / it * it;
    if ((seq_len + c - 1) / c > kMaxSplits) {
        c = (seq_len + kMaxSplits - 1) / kMaxSplits;
        c = (c + it - 1) / it * it;
    }
    *chunk = c;
    *n_splits = (seq_len + c - 1) / c;
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

hipError_t launch_attn_combine(const Shape& s, const RowsArgs& a,
                               hipStream_t st) {
    const dim3 grid(s.num_heads, a.rows);
    switch (s.head_dim) {
#define SLM_COMBINE(HD)                                                      \
    case HD:                                                                 \
        hipLaunchKernelGGL(attn_combine_kernel<HD>, grid, dim3(64), 0, st, a, \
                           s.dim, s.num_heads);                              \
        return hipGetLastError();
        SLM_COMBINE(16)
        SLM_COMBINE(32)
        SLM_COMBINE(48)
        SLM_COMBINE(64)
        SLM_COMBINE(96)
        SLM_COMBINE(128)
        SLM_COMBINE(256)
#undef SLM_COMBINE
        default:
            return hipErrorInvalidValue;
    }
}

}  // namespace slm
