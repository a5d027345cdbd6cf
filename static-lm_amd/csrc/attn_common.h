// Device helpers shared by the attention kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>

namespace slm {

typedef float vfloat4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 ld4(const float* p) {
    return *reinterpret_cast<const float4*>(p);
}

// K/V rows are read once per step: nontemporal loads keep them from evicting
// what is reused (streaming reads measured ~15% faster this way on MI355X).
__device__ __forceinline__ float4 ld4_stream(const float* p) {
    const vfloat4 v = __builtin_nontemporal_load(reinterpret_cast<const vfloat4*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// One RoPE pair exactly as apply_rope_cached computes it
// (transformer.rs:186-191): every product and sum rounded on its own.
__device__ __forceinline__ float2 rope_pair_exact(float2 x, float c, float s) {
#pragma clang fp contract(off)
    const float t0 = x.x * c;
    const float t1 = x.y * s;
    const float t2 = x.x * s;
    const float t3 = x.y * c;
    float2 r;
    r.x = t0 - t1;
    r.y = t2 + t3;
    return r;
}

// Two consecutive pairs (x,y), (z,w) with table entries (c.x, s.x), (c.y,
// s.y), bit-exact.
__device__ __forceinline__ float4 rope4_exact(float4 x, float2 c, float2 s) {
    const float2 a = rope_pair_exact(make_float2(x.x, x.y), c.x, s.x);
    const float2 b = rope_pair_exact(make_float2(x.z, x.w), c.y, s.y);
    return make_float4(a.x, a.y, b.x, b.y);
}

// The same with the entries read at table columns j, j+1.
__device__ __forceinline__ float4 rope4_exact(float4 x, const float* c, const float* s) {
    return rope4_exact(x, make_float2(c[0], c[1]), make_float2(s[0], s[1]));
}

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __builtin_amdgcn_update_dpp(0.0f, x, CTRL, 0xF, 0xF, false);
}

// Sum over aligned groups of LPG lanes; every lane of a group gets the total.
template <int LPG>
__device__ __forceinline__ float group_sum(float x) {
    if constexpr (LPG >= 2) x += dpp<0xB1>(x);    // quad_perm [1,0,3,2]
    if constexpr (LPG >= 4) x += dpp<0x4E>(x);    // quad_perm [2,3,0,1]
    if constexpr (LPG >= 8) x += dpp<0x141>(x);   // row_half_mirror
    if constexpr (LPG >= 16) x += dpp<0x140>(x);  // row_mirror
    if constexpr (LPG >= 32) x += __shfl_xor(x, 16);
    return x;
}

// Max / sum over lanes l, l^16, l^32, l^48 (the four 16-lane rows of the
// wave) with the VALU lane swaps of gfx950: each swap leaves x[l] and its
// partner's value in the two outputs, in one order or the other, so the max
// (sum) of the outputs is the pairwise max (sum).
// max(a, b) for operands that are not NaN (finite or -inf): one v_max_f32,
// where fmaxf first canonicalizes operands that come out of a lane swap
// (two more instructions per call; the compiler folds a median with +inf
// back into fmaxf)
__device__ __forceinline__ float max_nonan(float a, float b) {
    float r;
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

__device__ __forceinline__ float rows_max(float x) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                    false);
    x = max_nonan(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                    false);
    return max_nonan(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float rows_sum(float x) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                    false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                    false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Online softmax keeps a running max m with the invariant l = sum 2^(s-m),
// o = sum 2^(s-m) v.  The state is rescaled only when some lane's max has
// grown by more than kLazyRescale (log2 units) since m was last set: below
// that the stale m is kept, so terms are at most 2^8 and the rescale (one
// multiply per accumulator element) is skipped for the whole wave.  Any m
// satisfies the invariant, so the normalised result is unchanged.
constexpr float kLazyRescale = 8.0f;

// Max / sum over the wave, every lane getting the result: DPP row rotations
// by 8, 4, 2 and 1 fold each 16-lane row (lane l then holds the whole row's
// value), the lane swaps fold the four rows.  All VALU, no LDS round trips.
// The sum's association differs from lane to lane.
__device__ __forceinline__ float wave_max(float x) {
    x = fmaxf(x, dpp<0x128>(x));  // row_ror:8
    x = fmaxf(x, dpp<0x124>(x));  // row_ror:4
    x = fmaxf(x, dpp<0x122>(x));  // row_ror:2
    x = fmaxf(x, dpp<0x121>(x));  // row_ror:1
    return rows_max(x);
}

__device__ __forceinline__ float wave_sum(float x) {
    x += dpp<0x128>(x);
    x += dpp<0x124>(x);
    x += dpp<0x122>(x);
    x += dpp<0x121>(x);
    return rows_sum(x);
}

// One online-softmax step of a lane group over TP positions (log2 domain):
// scores q.k for GB heads reduced over the LPG lanes of the group, running
// max m, running sum l, accumulator o (lazy rescale, see kLazyRescale).
// Positions with valid[tp] false contribute nothing.  m starts at -FLT_MAX,
// not -inf: the first valid position then rescales by exp2(-FLT_MAX - mx) =
// 0 like any other, and m - m and score - m never meet an infinite m, so the
// exponents need no guard (two VALU instructions per head and position).
template <int LPG, int NV, int GB, int TP>
__device__ __forceinline__ void attend_tile(const float4 (&qr)[GB][NV],
                                            const float4 (&kr)[TP][NV],
                                            const float4 (&vr)[TP][NV], const bool (&valid)[TP],
                                            float (&m)[GB], float (&l)[GB],
                                            float4 (&o)[GB][NV]) {
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
        if (__any(mx > m[i] + kLazyRescale)) {  // wave-uniform
            const float mn = fmaxf(m[i], mx);
            const float alpha = fast_exp2(m[i] - mn);
            l[i] *= alpha;
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                o[i][v].x *= alpha;
                o[i][v].y *= alpha;
                o[i][v].z *= alpha;
                o[i][v].w *= alpha;
            }
            m[i] = mn;
        }
        const float mu = m[i];
        float pr[TP];
        float ps = 0.0f;
#pragma unroll
        for (int tp = 0; tp < TP; ++tp) {
            pr[tp] = fast_exp2(sc[tp] - mu);
            ps += pr[tp];
        }
        l[i] += ps;
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            float4 acc = o[i][v];
#pragma unroll
            for (int tp = 0; tp < TP; ++tp) {
                acc.x = fmaf(pr[tp], vr[tp][v].x, acc.x);
                acc.y = fmaf(pr[tp], vr[tp][v].y, acc.y);
                acc.z = fmaf(pr[tp], vr[tp][v].z, acc.z);
                acc.w = fmaf(pr[tp], vr[tp][v].w, acc.w);
            }
            o[i][v] = acc;
        }
    }
}

// Merges the online-softmax states of the lane groups of a wave (lanes with
// equal index inside their group hold equal head dims); afterwards every
// lane holds the wave's state for its dims.
// The values of lanes l and l ^ OFF, in an order that depends on the lane
// alone (the same for every call): gfx950's VALU lane swaps for OFF 16 and
// 32, a DPP row rotation for 8, a shuffle below that.
template <int OFF>
__device__ __forceinline__ void lane_pair(float x, float& a, float& b) {
    if constexpr (OFF == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                        false, false);
        a = __uint_as_float(r[0]);
        b = __uint_as_float(r[1]);
    } else if constexpr (OFF == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                        false, false);
        a = __uint_as_float(r[0]);
        b = __uint_as_float(r[1]);
    } else if constexpr (OFF == 8) {
        a = x;
        b = dpp<0x128>(x);  // row_ror:8 — lane l ^ 8 within its 16-lane row
    } else {
        a = x;
        b = __shfl_xor(x, OFF);
    }
}

// Max over the lane groups of a wave (lanes with equal index inside their
// LPG-lane group); every lane gets the result.
template <int LPG>
__device__ __forceinline__ float groups_max(float x) {
    if constexpr (LPG < 64) {
        float a, b;
        lane_pair<LPG>(x, a, b);
        return groups_max<2 * LPG>(fmaxf(a, b));
    } else {
        return x;
    }
}

// Sum over the lane groups of a wave (lanes with equal index inside their
// LPG-lane group), pairs of groups LPG apart first; every lane gets the
// result (the two lanes of a pair add the same two values).
template <int LPG>
__device__ __forceinline__ float groups_sum(float x) {
    if constexpr (LPG < 64) {
        float a, b;
        lane_pair<LPG>(x, a, b);
        return groups_sum<2 * LPG>(a + b);
    } else {
        return x;
    }
}

// Query heads that share one loaded K/V segment in a workgroup.
inline int pick_gb(int kv_mul) {
    for (int gb = 4; gb > 1; --gb)
        if (kv_mul % gb == 0) return gb;
    return 1;
}

}  // namespace slm
