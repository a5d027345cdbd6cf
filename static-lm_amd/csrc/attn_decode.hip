// Single-token decode for gfx950: KV append fused into split-K attention,
// then a log-sum-exp merge of the splits.
//
// Replaces, for one layer and position p, the decode attention block of
// forward_token_with_kv (transformer.rs:413-443):
//   K[p] = rope(k), V[p] = v                    (transformer.rs:416-428)
//   out_h = sum_t softmax_t(q_h . K[t, g] / sqrt(hd)) V[t, g], t = 0..p,
//   g = h / kv_mul                              (transformer.rs:273-321)
//
// Mapping.  blockIdx.x = split * groups + group, so workgroups that run at
// the same time cover every KV head of the same positions (whole 4 KiB cache
// rows for the Llama-3-8B shape).  Positions 0..p are cut into tiles of IT
// (the positions one loop iteration of a workgroup covers) and split s of n
// takes tiles s, s+n, s+2n, ...: at any moment the n splits stream one
// contiguous stretch of the cache, every split gets the same number of tiles
// to within one, and no sequence length lines the splits up on a bad
// address stride (contiguous chunks of 4128 rows ran at 74% of HBM peak
// where 4096 rows ran at 89%).  A workgroup covers one KV head and GB of its
// kv_mul query heads: each K/V segment loaded from HBM serves GB heads (the
// reference re-reads it once per head).  In a wave, LPG lanes hold one
// position's head_dim floats (128-bit nontemporal loads, LPG*16 contiguous
// bytes per group); each lane group keeps its own online-softmax state
// (log2 domain) over the positions it sees.  States merge across lane groups
// with shuffles and across waves through LDS; a sequence that fits one split
// is written out directly, otherwise decode_combine_kernel (up to 32 splits)
// or decode_combine_wide_kernel merges the split partials.  (Merging in the
// last workgroup to finish needs device-scope fences, which on this part
// write back and invalidate the whole L2: a second small kernel is cheaper.)
//
// The workgroup owning position p does not read row p back: after its loop,
// its wave 0 rotates k in registers with the reference's f32 arithmetic (no
// FMA contraction), stores K[p] and V[p] (bit-exact with the reference), and
// adds row p to its first lane group's state as one more position.  No other
// workgroup reads row p.
#include <hip/hip_ext.h>
#include <float.h>
#include <math.h>

#include "attn_common.h"
#include "slm_internal.h"

namespace slm {
namespace {

constexpr int kWaves = 4;
constexpr int kMaxSplits = 1024;

// Decode tiling per head_dim: lanes per position (LPG, 8 floats per lane
// where head_dim allows), positions per lane group per loop iteration (TP)
// and waves per workgroup (NW).  Measured on MI355X for hd 128 at 32k and
// 131k context: 16 lanes x 8 floats with one position per iteration keeps
// registers low (~110 VGPRs) and beat 8 lanes x 16 floats by 5-7 points of
// HBM bandwidth; what matters beyond that is two waves per SIMD, which
// 4-wave x 512 and 8-wave x 256 workgroups reach equally (interleaved
// medians 46 us at 32k, 153 us at 131k); 8 waves halve the splits to merge.
// MT: the most tiles a sequence may have and still run as one split (no
// merge launch).  One split walks its tiles one memory round trip after
// another, the split path costs a second launch.  Per layer-step (8 layers,
// replayed as a graph, the two interleaved in one process), one split against
// one tile per split: hd 128 at 4 tiles 6.89 against 6.93 us, at 5 tiles 7.80
// against 6.95; hd 64 (GQA 3) at 5 tiles 6.81 against 5.99; hd 48 (6 heads)
// at 3 tiles 7.52 against 7.01; hd 16, 32 and 96 at 4 tiles 9.70 / 9.78 /
// 6.83 against 8.08 / 7.61 / 6.35; hd 256 at 5 tiles 5.91 against 5.84.
template <int HD>
struct DecodeCfg;
template <> struct DecodeCfg<16> { static constexpr int LPG = 2, TP = 2, NW = 4, MT = 3; };
template <> struct DecodeCfg<32> { static constexpr int LPG = 4, TP = 2, NW = 4, MT = 3; };
template <> struct DecodeCfg<48> { static constexpr int LPG = 4, TP = 2, NW = 4, MT = 2; };
template <> struct DecodeCfg<64> { static constexpr int LPG = 8, TP = 2, NW = 4, MT = 4; };
template <> struct DecodeCfg<96> { static constexpr int LPG = 8, TP = 2, NW = 4, MT = 3; };
template <> struct DecodeCfg<128> { static constexpr int LPG = 16, TP = 1, NW = 8, MT = 4; };
template <> struct DecodeCfg<256> { static constexpr int LPG = 32, TP = 1, NW = 8, MT = 4; };

// Two more tilings, picked by length (decode_plan).  Per layer-step (8
// layers, replayed as a graph, the tilings interleaved in one process):
// kShort, one position per lane group (half the tile, twice the splits), for
// the head dims whose base tiling takes two (hd 16-96), while that stays
// within one merge round and one workgroup per CU: at 1023 rows hd 16 / 32 /
// 48 / 64 / 96 with GQA 4 7.16 / 7.20 / 7.85 / 6.60 / 7.55 us against 7.57 /
// 8.00 / 8.87 / 6.79 / 7.85, the SmolLM2 shape (hd 64, GQA 3) at 513 / 767
// rows 5.81 / 6.06 against 6.05 / 6.28, but MHA with 16 KV heads at 513 rows
// (272 workgroups) 5.77 against 5.48.  kWide, 8-wave workgroups of one
// position per lane group (one workgroup per CU, half the splits), for hd 64
// and 96 once each of its splits holds 1.5 tiles or more: GQA 4 at 8191 rows
// 10.84 / 13.87 us against 12.15 / 15.81 (hd 64 / 96), hd 64 at 32767 24.83
// against 27.44 and MHA with 16 / 32 KV heads 43.7 / 82.5 against 45.7 /
// 86.3; at hd 16, 32 and 48 it lost or tied (hd 48 GQA 4 at 8191 rows 13.36
// against 13.46, Stories-15M shape 12.18 against 11.25).
enum class Tiling { kBase, kShort, kWide };

template <int HD, Tiling T>
struct TilingCfg : DecodeCfg<HD> {};
template <int HD>
struct TilingCfg<HD, Tiling::kShort> {
    static constexpr int LPG = DecodeCfg<HD>::LPG, TP = 1, NW = DecodeCfg<HD>::NW;
};
template <int HD>
struct TilingCfg<HD, Tiling::kWide> {
    static constexpr int LPG = DecodeCfg<HD>::LPG, TP = 1, NW = 8;
};
template <int HD>
constexpr bool has_short() { return DecodeCfg<HD>::TP == 2; }
template <int HD>
constexpr bool has_wide() { return HD == 64 || HD == 96; }

// Rows per tile (the positions one loop iteration of a workgroup covers).
template <int HD, Tiling T = Tiling::kBase>
constexpr int dec_span() {
    using C = TilingCfg<HD, T>;
    return C::NW * (64 / C::LPG) * C::TP;
}

// Waves per CU one decode launch aims for on long sequences: two per SIMD.
constexpr int kWavesPerCu = 8;

struct DecodeParams {
    const float* q;      // [dim]; rotated at p here when cos_t != nullptr
    const float* k_new;  // [kv_dim] appended at p when not nullptr
    const float* v_new;
    float* k_cache;      // layer K slice [max_seq_len][kv_dim]
    float* v_cache;
    const float* cos_t;  // RoPE tables [max_seq_len][head_dim/2]
    const float* sin_t;
    float* out;          // [dim]
    float* part_o;       // [n_splits][num_heads][head_dim]
    float* part_ml;      // [n_splits][num_heads][2]
    int pos;
    int n_splits;
    int num_heads;
    int kv_dim;
    int kv_mul;
    int half;
    float scale_log2;
};

// Tiling of decode_kernel: lanes per position (LPG), positions per lane group
// per loop iteration (TP) and waves per workgroup (NW).
template <int HD, int GB, int LPG_ = DecodeCfg<HD>::LPG, int TP_ = DecodeCfg<HD>::TP,
          int NW = DecodeCfg<HD>::NW>
__global__ __launch_bounds__(64 * NW) void decode_kernel(DecodeParams p) {
    constexpr int LPG = LPG_;
    constexpr int FPL = HD / LPG;
    constexpr int NV = FPL / 4;
    constexpr int GPW = 64 / LPG;
    constexpr int TP = TP_;
    constexpr int IT = NW * GPW * TP;
    static_assert(FPL % 4 == 0, "lane slice must be whole float4s");

    const int nhb = p.kv_mul / GB;
    const int groups = (p.num_heads / p.kv_mul) * nhb;
    const int split = blockIdx.x / groups;
    const int gy = blockIdx.x - split * groups;
    const int g = gy / nhb;
    const int h0 = g * p.kv_mul + (gy % nhb) * GB;
    const int seq_len = p.pos + 1;
    const int t0 = split * IT;
    const int t_step = p.n_splits * IT;
    const bool append = p.k_new != nullptr;
    const bool owner = (p.pos / IT) % p.n_splits == split;  // holds row p's tile
    const int t_end = append ? p.pos : seq_len;  // rows read from the cache

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform, and known to be
    const int li = lane % LPG;
    const int lg = lane / LPG;
    const long trow = (long)p.pos * p.half;
    const float* kbase = p.k_cache + g * HD + 4 * li;
    const float* vbase = p.v_cache + g * HD + 4 * li;

    float4 kr[TP][NV], vr[TP][NV];
    bool valid[TP];
    auto load_tile = [&](int tb) {
#pragma unroll
        for (int tp = 0; tp < TP; ++tp) {
            const int t = tb + (tp * NW + wave) * GPW + lg;
            valid[tp] = t < t_end;
            const long tt = valid[tp] ? t : 0;
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                kr[tp][v] = ld4_stream(kbase + tt * p.kv_dim + 4 * v * LPG);
                vr[tp][v] = ld4_stream(vbase + tt * p.kv_dim + 4 * v * LPG);
            }
        }
    };
    // q of the GB heads, rotated at p and pre-scaled, is built once per
    // workgroup in LDS: one float4 per thread of the first GB*HD/4.  (Loading
    // each lane's own slice from memory replicated it 64*NW/LPG times per
    // workgroup, ~80 KB of q and table traffic per CU for the Llama-3-8B
    // shape.)  Loads complete in issue order, so the set-up's go out first --
    // q with its table row -- and the first tile right after them: the q
    // rotation waits for its own loads while the tile is still in flight.
    // The scheduling barriers keep that order (left to itself the compiler
    // issued the sin row after a wait for every earlier load, the tile's
    // included, and waited again), and the tile is loaded unconditionally
    // (rows past the end are clamped and never used) so that the waits can
    // count the loads.
    // More than one tile in flight per wave measured slower at every context
    // length (4096 rows: 12.8 us with four against 11.7 us with one; 32768
    // rows: 48.4 us against 43.5 us).
    const bool rot = p.cos_t != nullptr;  // always set when appending
    constexpr int NQ4 = GB * HD / 4;
    static_assert(NQ4 <= 64 * NW, "one q float4 per thread");
    __shared__ __align__(16) float s_q[GB * HD];
    const bool qthread = threadIdx.x < NQ4;
    const int qi = threadIdx.x / (HD / 4);
    const int qc = threadIdx.x - qi * (HD / 4);
    float4 xq = make_float4(0.f, 0.f, 0.f, 0.f);
    float2 cq = make_float2(1.0f, 1.0f), sq = make_float2(0.0f, 0.0f);
    if (qthread) {
        xq = ld4(p.q + (h0 + qi) * HD + 4 * qc);
        if (rot) {
            cq = *reinterpret_cast<const float2*>(p.cos_t + trow + 2 * qc);
            sq = *reinterpret_cast<const float2*>(p.sin_t + trow + 2 * qc);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    load_tile(t0);
    // The appended row (k, v and the table entries of its dims) is used only
    // by wave 0 of the owner, after the loop.  Its loads go out behind the
    // first tile, from every wave, through buffer descriptors whose range is
    // empty except in that wave (out-of-range loads return zeros and touch no
    // memory): with the same loads on every path the compiler waits for q
    // and the first tile alone.  (Issued ahead of the tile by the owner only,
    // they were waited for at the set-up barrier -- loads complete in issue
    // order -- and the owner's workgroups passed it 1.4 us after the others.)
    const bool app_wave = append && owner && wave == 0;  // wave-uniform
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    const int row_bytes = app_wave ? HD * 4 : 0;
    const int tab_bytes = app_wave ? HD * 2 : 0;  // half a table row: HD/2 floats
    const __amdgpu_buffer_rsrc_t rkn = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(p.k_new + g * HD), 0, row_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rvn = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(p.v_new + g * HD), 0, row_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rcos = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(p.cos_t + trow), 0, tab_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsin = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(p.sin_t + trow), 0, tab_bytes, 0x00020000);
    float4 kn[NV], vn[NV];
    float2 cr[NV], sr[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) {
        const int d = 4 * (v * LPG + li);  // this lane's dims of the row
        const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(rkn, 4 * d, 0, 0);
        const u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(rvn, 4 * d, 0, 0);
        const u32x2 c = __builtin_amdgcn_raw_buffer_load_b64(rcos, 2 * d, 0, 0);
        const u32x2 e = __builtin_amdgcn_raw_buffer_load_b64(rsin, 2 * d, 0, 0);
        kn[v] = make_float4(__uint_as_float(a.x), __uint_as_float(a.y), __uint_as_float(a.z),
                            __uint_as_float(a.w));
        vn[v] = make_float4(__uint_as_float(b.x), __uint_as_float(b.y), __uint_as_float(b.z),
                            __uint_as_float(b.w));
        cr[v] = make_float2(__uint_as_float(c.x), __uint_as_float(c.y));
        sr[v] = make_float2(__uint_as_float(e.x), __uint_as_float(e.y));
    }
    __builtin_amdgcn_sched_barrier(0);
    if (qthread) {
        float4 x = xq;
        if (rot) x = rope4_exact(x, cq, sq);
        x.x *= p.scale_log2;
        x.y *= p.scale_log2;
        x.z *= p.scale_log2;
        x.w *= p.scale_log2;
        *reinterpret_cast<float4*>(&s_q[qi * HD + 4 * qc]) = x;
    }
    __syncthreads();
    float4 qr[GB][NV];
#pragma unroll
    for (int i = 0; i < GB; ++i) {
#pragma unroll
        for (int v = 0; v < NV; ++v)
            qr[i][v] = *reinterpret_cast<const float4*>(&s_q[i * HD + 4 * (v * LPG + li)]);
    }

    float m[GB], l[GB];
    float4 o[GB][NV];
#pragma unroll
    for (int i = 0; i < GB; ++i) {
        m[i] = -FLT_MAX;  // finite: see attend_tile
        l[i] = 0.0f;
#pragma unroll
        for (int v = 0; v < NV; ++v) o[i][v] = make_float4(0.f, 0.f, 0.f, 0.f);
    }

    // The first tile, loaded with the set-up, is attended outside the loop:
    // there the compiler knows the appended row's loads are younger and waits
    // for the tile alone (merged with the loop's own wait, it waited for
    // most of them too).
    if (t0 < t_end) attend_tile<LPG, NV, GB, TP>(qr, kr, vr, valid, m, l, o);
    // The second half of the waves issues its first loads after the first
    // half's and falls further behind over the loop (each shares a SIMD with
    // an older wave of the first half): at 32k rows its loops ended 1.1-1.4 us
    // later.  Raising its issue priority for the loop took 0.3 us off a 32k
    // layer-step and 0.14 us off a 4096-row one (means of five interleaved
    // runs); from the kernel's start, or alternating per tile, it did not.
    if (wave >= NW / 2) __builtin_amdgcn_s_setprio(1);
    for (int tb = t0 + t_step; tb < t_end; tb += t_step) {
        load_tile(tb);
        // With three float4 per lane and row (hd 48 and 96) the scheduler
        // hoisted the first dot product right behind the first load, whose
        // wait then split each tile into two memory round trips; the barrier
        // sends every load of the tile first (unsplit decode 14.9 -> 13.3 us
        // at 767 rows of the Stories-15M shape, 6.1 -> 5.6 us at 300 rows of
        // hd 96).  The other layouts issue their loads first anyway, and
        // there the barrier only reshuffled the code (2-3% slower at hd 16
        // and 32, no change at hd 128).
        if constexpr (NV == 3) __builtin_amdgcn_sched_barrier(0);
        attend_tile<LPG, NV, GB, TP>(qr, kr, vr, valid, m, l, o);
    }
    if (app_wave) {
        // Row p: k rotated at p with the reference's f32 arithmetic (no FMA
        // contraction), K[p] and V[p] stored bit-exact, then one more
        // position of lane group 0's state.
#pragma unroll
        for (int v = 0; v < NV; ++v) kn[v] = rope4_exact(kn[v], cr[v], sr[v]);
        if (lg == 0 && (gy % nhb) == 0) {
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                const int d = 4 * (v * LPG + li);
                *reinterpret_cast<float4*>(p.k_cache + (long)p.pos * p.kv_dim + g * HD + d) = kn[v];
                *reinterpret_cast<float4*>(p.v_cache + (long)p.pos * p.kv_dim + g * HD + d) = vn[v];
            }
        }
        float4 kt[1][NV], vt[1][NV];
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            kt[0][v] = kn[v];
            vt[0][v] = vn[v];
        }
        const bool mine[1] = {lg == 0};
        attend_tile<LPG, NV, GB, 1>(qr, kt, vt, mine, m, l, o);
    }
    constexpr int F = GB * NV * 4;  // floats of o per lane
    if constexpr ((GPW == 4 || GPW == 8) && F % GPW == 0) {
        // Merge in two levels.  In the wave: each lane group scales its (l, o)
        // by 2^(m - Mw), Mw the wave's max per head, and rounds of lane
        // exchanges sum the lane groups -- register pairs (f, f+F/2) across
        // the wave's halves (v_permlane32_swap), (f, f+F/4) across 16-lane
        // rows (v_permlane16_swap) and, with 8 lanes per position, (f, f+F/8)
        // across the two halves of a row (DPP row_ror:8) -- so that lane group
        // g of register f ends holding flat element g*F/GPW + f of o summed
        // over the groups (for the Llama-3-8B shape: head g, the lane's dims).
        // 24 swaps and 24 adds there, done by each wave as soon as its loop
        // ends.  In the workgroup: one barrier, then each thread combines one
        // (head, dim) over the waves in wave order.  (All lane-group states
        // through LDS with two barriers took ~1.5 us after the last wave's
        // loop at every context length.)
        float mw[GB], lw[GB], of[F];
#pragma unroll
        for (int i = 0; i < GB; ++i) {
            // -FLT_MAX when the wave saw no position
            if constexpr (GPW == 4)
                mw[i] = rows_max(m[i]);
            else
                mw[i] = groups_max<LPG>(m[i]);
            // 0 for a lane group that saw nothing (its l and o are 0 anyway)
            const float sc = fast_exp2(m[i] - mw[i]);
            if constexpr (GPW == 4)
                lw[i] = rows_sum(l[i] * sc);
            else
                lw[i] = groups_sum<LPG>(l[i] * sc);
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                of[(i * NV + v) * 4 + 0] = o[i][v].x * sc;
                of[(i * NV + v) * 4 + 1] = o[i][v].y * sc;
                of[(i * NV + v) * 4 + 2] = o[i][v].z * sc;
                of[(i * NV + v) * 4 + 3] = o[i][v].w * sc;
            }
        }
        float z[F / 2], zz[F / 4], wv[F / GPW];
#pragma unroll
        for (int f = 0; f < F / 2; ++f) {
            const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(of[f]),
                                                            __float_as_uint(of[f + F / 2]), false,
                                                            false);
            z[f] = __uint_as_float(a[0]) + __uint_as_float(a[1]);
        }
#pragma unroll
        for (int f = 0; f < F / 4; ++f) {
            const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(z[f]),
                                                            __float_as_uint(z[f + F / 4]), false,
                                                            false);
            zz[f] = __uint_as_float(b[0]) + __uint_as_float(b[1]);
        }
        if constexpr (GPW == 4) {
#pragma unroll
            for (int f = 0; f < F / 4; ++f) wv[f] = zz[f];
        } else {
            // lanes 0-7 of a row add register f of lanes 8-15, lanes 8-15 add
            // register f+F/8 of lanes 0-7
            const bool hi = (lane & 8) != 0;
#pragma unroll
            for (int f = 0; f < F / 8; ++f) {
                const float t = hi ? zz[f] : zz[f + F / 8];
                const float u = hi ? zz[f + F / 8] : zz[f];
                wv[f] = u + dpp<0x128>(t);  // row_ror:8
            }
        }
        __shared__ __align__(16) float s_ow[NW][GB * HD];
        __shared__ float s_mx[NW][GB];
        __shared__ float s_lw[NW][GB];
#pragma unroll
        for (int f = 0; f < F / GPW; ++f) {
            const int e = lg * (F / GPW) + f;  // flat element of o held by this lane group
            const int i = e / (NV * 4), v = (e / 4) % NV, c = e % 4;
            s_ow[wave][i * HD + 4 * (v * LPG + li) + c] = wv[f];
        }
        if (lane == 0) {
#pragma unroll
            for (int i = 0; i < GB; ++i) {
                s_mx[wave][i] = mw[i];
                s_lw[wave][i] = lw[i];
            }
        }
        __syncthreads();
        for (int idx = threadIdx.x; idx < GB * HD; idx += 64 * NW) {
            const int i = idx / HD;
            const int d = idx - i * HD;
            float mx = s_mx[0][i];
#pragma unroll
            for (int w = 1; w < NW; ++w) mx = fmaxf(mx, s_mx[w][i]);
            float acc_o = 0.0f, acc_l = 0.0f;
#pragma unroll
            for (int w = 0; w < NW; ++w) {
                const float e = fast_exp2(s_mx[w][i] - mx);  // 0 for a wave that saw nothing
                acc_o += e * s_ow[w][idx];
                acc_l += e * s_lw[w][i];
            }
            const int h = h0 + i;
            if (p.n_splits == 1) {
                p.out[h * HD + d] = acc_o / acc_l;
            } else {
                const long pi = (long)split * p.num_heads + h;
                p.part_o[pi * HD + d] = acc_o;
                if (d == 0) {
                    p.part_ml[pi * 2] = mx;
                    p.part_ml[pi * 2 + 1] = acc_l;
                }
            }
        }
    } else {
        // Merge of the workgroup's NS lane-group states per head: the workgroup
        // max M over the lane groups' maxima (max over the wave's lane groups by
        // lane swaps, then over the waves through LDS), every lane group scales
        // its (l, o) once by 2^(m - M) into its own LDS slot, and each thread sums
        // the slots of one (head, dim) in slot order.  (Merging pairs of lane
        // groups in registers first, with a scale per pair and round, cost ~360
        // VALU ops per wave: ~1.5 us between a workgroup's last wave leaving the
        // loop and the barrier, at two waves per SIMD.)
        constexpr int NS = NW * GPW;  // lane-group states per workgroup
        __shared__ float s_mw[NW][GB];
        __shared__ __align__(16) float s_o[NS][GB][HD];
        __shared__ float s_l[GB][NS];
        float mg[GB];
#pragma unroll
        for (int i = 0; i < GB; ++i) mg[i] = groups_max<LPG>(m[i]);
        if (lane == 0) {
#pragma unroll
            for (int i = 0; i < GB; ++i) s_mw[wave][i] = mg[i];
        }
        __syncthreads();
        float mwg[GB];  // the workgroup max per head, -FLT_MAX when no position was seen
#pragma unroll
        for (int i = 0; i < GB; ++i) {
            float mx = s_mw[0][i];
#pragma unroll
            for (int w = 1; w < NW; ++w) mx = fmaxf(mx, s_mw[w][i]);
            mwg[i] = mx;
        }
        const int slot = wave * GPW + lg;
#pragma unroll
        for (int i = 0; i < GB; ++i) {
            const float w = fast_exp2(m[i] - mwg[i]);  // 0 for a lane group that saw nothing
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                float4 x = o[i][v];
                x.x *= w;
                x.y *= w;
                x.z *= w;
                x.w *= w;
                *reinterpret_cast<float4*>(&s_o[slot][i][4 * (v * LPG + li)]) = x;
            }
            if (li == 0) s_l[i][slot] = l[i] * w;
        }
        __syncthreads();
        for (int idx = threadIdx.x; idx < GB * HD; idx += 64 * NW) {
            const int i = idx / HD;
            const int d = idx - i * HD;
            float mx = mwg[0];
#pragma unroll
            for (int j = 1; j < GB; ++j)
                if (i == j) mx = mwg[j];
            float acc_o = 0.0f, acc_l = 0.0f;
#pragma unroll
            for (int sl = 0; sl < NS; ++sl) {
                acc_o += s_o[sl][i][d];
                acc_l += s_l[i][sl];
            }
            const int h = h0 + i;
            if (p.n_splits == 1) {
                p.out[h * HD + d] = acc_o / acc_l;
            } else {
                const long pi = (long)split * p.num_heads + h;
                p.part_o[pi * HD + d] = acc_o;
                if (d == 0) {
                    p.part_ml[pi * 2] = mx;
                    p.part_ml[pi * 2 + 1] = acc_l;
                }
            }
        }
    }
}

// Threads of a merge workgroup: one per head dim, rounded up to whole waves.
template <int HD>
constexpr int combine_threads() {
    return (HD + 63) / 64 * 64;
}
// Split partials a merge thread loads per round: all of them for up to 32
// splits (the Llama-3-8B shape's policy on 256 CUs); more splits go to
// decode_combine_wide_kernel.
constexpr int kCombineRound = 32;

// Log-sum-exp merge of the split partials: one workgroup per head, one
// thread per head dim.  Every thread issues the loads of its dim's partials
// first; wave 0 meanwhile turns the splits' (max, sum) pairs into weights
// 2^(m_s - M) in LDS and the total sum; one barrier; each thread then sums
// its dim over the splits in split order.  (Four waves splitting the splits
// of a 64-dim slice, with a second barrier to add the waves' sums, cost
// ~3 us per step at short contexts where an empty launch costs 2.4 us.)
template <int HD>
__global__ __launch_bounds__(combine_threads<HD>()) void decode_combine_kernel(DecodeParams p) {
    __shared__ float s_w[kMaxSplits];
    __shared__ float s_ltot;
    const int h = blockIdx.x;
    const int d = threadIdx.x;
    const int lane = threadIdx.x & 63;
    const int ns = p.n_splits;
    const bool has_d = d < HD;
    const float* src = p.part_o + (long)h * HD + (has_d ? d : 0);
    const long stride = (long)p.num_heads * HD;

    // the (max, sum) pairs of the first 64 splits go out before the
    // partials: loads complete in issue order, so wave 0 forms the weights
    // while the partials are still in flight.  Every load is unconditional
    // (indices clamped, values past ns never used), so the compiler can
    // count them and wait for the pairs alone.
    const float2* ml = reinterpret_cast<const float2*>(p.part_ml);
    const float2 ml0 = ml[(long)min(lane, ns - 1) * p.num_heads + h];
    asm volatile("" ::: "memory");  // keeps it ahead of the partials' loads
    float x[kCombineRound];
#pragma unroll
    for (int u = 0; u < kCombineRound; ++u) x[u] = src[(long)min(u, ns - 1) * stride];
    if (threadIdx.x < 64) {
        float mx = lane < ns ? ml0.x : -INFINITY;
        for (int sp = lane + 64; sp < ns; sp += 64) mx = fmaxf(mx, ml[(long)sp * p.num_heads + h].x);
        mx = wave_max(mx);
        float ls = 0.0f;
        if (lane < ns) {
            const float w = fast_exp2(ml0.x - mx);
            s_w[lane] = w;
            ls += w * ml0.y;
        }
        for (int sp = lane + 64; sp < ns; sp += 64) {
            const float2 v = ml[(long)sp * p.num_heads + h];
            const float w = fast_exp2(v.x - mx);
            s_w[sp] = w;
            ls += w * v.y;
        }
        ls = wave_sum(ls);
        if (lane == 0) s_ltot = ls;
    }
    __syncthreads();
    float acc = 0.0f;
#pragma unroll
    for (int u = 0; u < kCombineRound; ++u)
        if (u < ns) acc += s_w[u] * x[u];
    for (int base = kCombineRound; base < ns; base += kCombineRound) {
#pragma unroll
        for (int u = 0; u < kCombineRound; ++u)
            x[u] = base + u < ns ? src[(long)(base + u) * stride] : 0.0f;
#pragma unroll
        for (int u = 0; u < kCombineRound; ++u)
            if (base + u < ns) acc += s_w[base + u] * x[u];
    }
    if (has_d) p.out[h * HD + d] = acc / s_ltot;
}

// Threads of a wide merge workgroup, and the most splits it takes.
constexpr int kCombineWideThreads = 1024;
template <int HD>
constexpr int combine_wide_max_splits() {
    return kCombineWideThreads / combine_threads<HD>() * kCombineRound;
}

// The merge for more than kCombineRound splits (shapes with few KV-head
// groups take up to 512/groups splits to fill the CUs: 170 for 3 groups).
// decode_combine_kernel would take one dependent round of loads per 32
// splits, and its wave 0 one more per 64 splits for the (max, sum) pairs
// (ten memory round trips at 170 splits); here R = ceil(ns/32) rows of
// threads, one thread per head dim in each, so every load is in flight at
// once.  Thread t loads the pair of split t and thread (d, r) the partials
// of dim d for splits 32r..32r+31.  The maxima reduce per wave and then over
// the waves in wave order; each row sums its 32 splits in split order and the
// rows are added in row order: a fixed function of n_splits, so results
// reproduce bit for bit.  One memory round trip and three barriers.
template <int HD>
__global__ __launch_bounds__(kCombineWideThreads) void decode_combine_wide_kernel(
    DecodeParams p) {
    constexpr int HDT = combine_threads<HD>();
    constexpr int kMaxRows = kCombineWideThreads / HDT;
    __shared__ float s_w[kMaxRows * kCombineRound];
    __shared__ float s_acc[kCombineWideThreads];
    __shared__ float s_wmax[kCombineWideThreads / 64], s_wsum[kCombineWideThreads / 64];
    const int h = blockIdx.x;
    const int t = threadIdx.x;
    const int d = t % HDT;
    const int r = t / HDT;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int n_waves = blockDim.x >> 6;
    const int rows = blockDim.x / HDT;
    const int ns = p.n_splits;
    const int u0 = r * kCombineRound;
    const bool has_d = d < HD;
    const float* src = p.part_o + (long)h * HD + (has_d ? d : 0);
    const long stride = (long)p.num_heads * HD;

    // the pair first, then the partials (indices clamped, every load
    // unconditional: the compiler waits for the pair alone)
    const float2* ml = reinterpret_cast<const float2*>(p.part_ml);
    const float2 mlt = ml[(long)min(t, ns - 1) * p.num_heads + h];
    asm volatile("" ::: "memory");
    float x[kCombineRound];
#pragma unroll
    for (int u = 0; u < kCombineRound; ++u) x[u] = src[(long)min(u0 + u, ns - 1) * stride];

    const float wm = wave_max(t < ns ? mlt.x : -INFINITY);
    if (lane == 0) s_wmax[wave] = wm;
    __syncthreads();
    float mx = s_wmax[0];
    for (int w = 1; w < n_waves; ++w) mx = fmaxf(mx, s_wmax[w]);
    float wl = 0.0f;
    if (t < ns) {
        const float w = fast_exp2(mlt.x - mx);
        s_w[t] = w;
        wl = w * mlt.y;
    }
    wl = wave_sum(wl);
    if (lane == 0) s_wsum[wave] = wl;
    __syncthreads();
    float acc = 0.0f;
#pragma unroll
    for (int u = 0; u < kCombineRound; ++u)
        if (u0 + u < ns) acc += s_w[u0 + u] * x[u];
    s_acc[t] = acc;
    __syncthreads();
    if (r == 0 && has_d) {
        float ltot = s_wsum[0];
        for (int w = 1; w < n_waves; ++w) ltot += s_wsum[w];
        float o = s_acc[d];
        for (int rr = 1; rr < rows; ++rr) o += s_acc[rr * HDT + d];
        p.out[h * HD + d] = o / ltot;
    }
}

template <int HD, int GB, Tiling T>
hipError_t launch_t(const Shape& s, const DecodeParams& dp, hipStream_t st, hipEvent_t ev0,
                    hipEvent_t ev1) {
    using C = TilingCfg<HD, T>;
    const auto kern = decode_kernel<HD, GB, C::LPG, C::TP, C::NW>;
    const int groups = s.num_kv_heads * (s.kv_mul / GB);
    if (ev0 != nullptr && ev1 != nullptr)
        hipExtLaunchKernelGGL(kern, dim3(dp.n_splits * groups), dim3(64 * C::NW), 0, st, ev0,
                              ev1, 0, dp);
    else
        hipLaunchKernelGGL(kern, dim3(dp.n_splits * groups), dim3(64 * C::NW), 0, st, dp);
    return hipGetLastError();
}

template <int HD>
hipError_t launch_combine_t(const Shape& s, const DecodeParams& dp, hipStream_t st,
                            hipEvent_t ev0, hipEvent_t ev1) {
    if (dp.n_splits > kCombineRound && dp.n_splits <= combine_wide_max_splits<HD>()) {
        const int rows = (dp.n_splits + kCombineRound - 1) / kCombineRound;
        const dim3 block(rows * combine_threads<HD>());
        if (ev0 != nullptr && ev1 != nullptr)
            hipExtLaunchKernelGGL(decode_combine_wide_kernel<HD>, dim3(s.num_heads), block, 0,
                                  st, ev0, ev1, 0, dp);
        else
            hipLaunchKernelGGL(decode_combine_wide_kernel<HD>, dim3(s.num_heads), block, 0, st,
                               dp);
        return hipGetLastError();
    }
    if (ev0 != nullptr && ev1 != nullptr)
        hipExtLaunchKernelGGL(decode_combine_kernel<HD>, dim3(s.num_heads),
                              dim3(combine_threads<HD>()), 0, st, ev0, ev1, 0, dp);
    else
        hipLaunchKernelGGL(decode_combine_kernel<HD>, dim3(s.num_heads),
                           dim3(combine_threads<HD>()), 0, st, dp);
    return hipGetLastError();
}

template <int HD, Tiling T>
hipError_t launch_gb(const Shape& s, const DecodeParams& dp, hipStream_t st, hipEvent_t ev0,
                     hipEvent_t ev1) {
    switch (pick_gb(s.kv_mul)) {
        case 4: return launch_t<HD, 4, T>(s, dp, st, ev0, ev1);
        case 3: return launch_t<HD, 3, T>(s, dp, st, ev0, ev1);
        case 2: return launch_t<HD, 2, T>(s, dp, st, ev0, ev1);
        default: return launch_t<HD, 1, T>(s, dp, st, ev0, ev1);
    }
}

template <int HD>
hipError_t launch_hd(const Shape& s, const DecodeParams& dp, Tiling t, hipStream_t st,
                     hipEvent_t ev0, hipEvent_t ev1) {
    if constexpr (has_short<HD>())
        if (t == Tiling::kShort) return launch_gb<HD, Tiling::kShort>(s, dp, st, ev0, ev1);
    if constexpr (has_wide<HD>())
        if (t == Tiling::kWide) return launch_gb<HD, Tiling::kWide>(s, dp, st, ev0, ev1);
    return launch_gb<HD, Tiling::kBase>(s, dp, st, ev0, ev1);
}

// Rows per tile and waves per workgroup of a tiling.
struct TilingDims {
    int span, nw;
};

template <int HD, Tiling T>
constexpr TilingDims dims_t() {
    return TilingDims{dec_span<HD, T>(), TilingCfg<HD, T>::NW};
}

// The tiling's dims (the base tiling's where the head dim has no such tiling).
template <int HD>
TilingDims dims(Tiling t) {
    if constexpr (has_short<HD>())
        if (t == Tiling::kShort) return dims_t<HD, Tiling::kShort>();
    if constexpr (has_wide<HD>())
        if (t == Tiling::kWide) return dims_t<HD, Tiling::kWide>();
    return dims_t<HD, Tiling::kBase>();
}

TilingDims tiling_dims(int head_dim, Tiling t) {
    switch (head_dim) {
        case 16: return dims<16>(t);
        case 32: return dims<32>(t);
        case 48: return dims<48>(t);
        case 64: return dims<64>(t);
        case 96: return dims<96>(t);
        case 128: return dims<128>(t);
        case 256: return dims<256>(t);
        default: return TilingDims{64, kWaves};
    }
}

// has_short / has_wide of a runtime head dim
template <bool (*F16)(), bool (*F32)(), bool (*F48)(), bool (*F64)(), bool (*F96)(),
          bool (*F128)(), bool (*F256)()>
bool by_head_dim(int head_dim) {
    switch (head_dim) {
        case 16: return F16();
        case 32: return F32();
        case 48: return F48();
        case 64: return F64();
        case 96: return F96();
        case 128: return F128();
        case 256: return F256();
        default: return false;
    }
}
bool tiling_short(int head_dim) {
    return by_head_dim<has_short<16>, has_short<32>, has_short<48>, has_short<64>, has_short<96>,
                       has_short<128>, has_short<256>>(head_dim);
}
bool tiling_wide(int head_dim) {
    return by_head_dim<has_wide<16>, has_wide<32>, has_wide<48>, has_wide<64>, has_wide<96>,
                       has_wide<128>, has_wide<256>>(head_dim);
}

int decode_one_split_tiles(const Shape& s) {
    switch (s.head_dim) {
        case 16: return DecodeCfg<16>::MT;
        case 32: return DecodeCfg<32>::MT;
        case 48: return DecodeCfg<48>::MT;
        case 64: return DecodeCfg<64>::MT;
        case 96: return DecodeCfg<96>::MT;
        case 128: return DecodeCfg<128>::MT;
        case 256: return DecodeCfg<256>::MT;
        default: return 1;
    }
}

struct DecodePlan {
    int n_splits, tile;
    Tiling tiling;
    int tiles, want;  // tiles of the sequence; splits that fill the CUs
};

int decode_groups_of(const Shape& s) { return s.num_kv_heads * (s.kv_mul / pick_gb(s.kv_mul)); }

// As many splits as there are tiles, up to two waves per SIMD (for 8-wave
// workgroups one per CU: a few workgroups more than CUs double some CUs up
// and measured 20-30% slower) and kMaxSplits.  Below that the kernel is
// latency-bound and every tile a split walks costs about one memory round
// trip, so one tile per split wins (Llama-3-8B shape at 4096 rows: 15.0 us
// with 32 splits against 17.4 us with 16; SmolLM2 at 768 rows: 10.8 us with
// 12 splits against 13.0 us with one).  Up to DecodeCfg::MT tiles (2-4 by
// head_dim) the merge launch costs more than it saves, and a single split
// writes the output directly.  hd 16-96 then pick among their tilings (see
// Tiling).  A pure function of seq_len, the shape and the CU count, so the
// launch finds the same tiling and results reproduce run to run on a device.
DecodePlan decode_plan(const Shape& s, int seq_len) {
    const int groups = decode_groups_of(s);
    auto plan = [&](Tiling t) {
        const TilingDims d = tiling_dims(s.head_dim, t);
        const int wgs = kWavesPerCu * s.cus / d.nw;
        const int want = groups >= wgs ? 1 : wgs / groups;
        const int tiles = (seq_len + d.span - 1) / d.span;
        int ns = tiles < want ? tiles : want;
        if (ns > kMaxSplits) ns = kMaxSplits;
        return DecodePlan{ns, d.span, t, tiles, want};
    };
    DecodePlan base = plan(Tiling::kBase);
    if (base.tiles <= decode_one_split_tiles(s)) {
        base.n_splits = 1;
        return base;
    }
    if (tiling_short(s.head_dim)) {
        const DecodePlan sh = plan(Tiling::kShort);
        if (sh.n_splits <= kCombineRound && sh.n_splits * groups <= s.cus) return sh;
    }
    if (tiling_wide(s.head_dim)) {
        const DecodePlan wide = plan(Tiling::kWide);
        if (2 * base.tiles >= 3 * wide.want) return wide;
    }
    return base;
}

}  // namespace

int decode_groups(const Shape& s) { return decode_groups_of(s); }

int decode_max_splits() { return kMaxSplits; }

void decode_split_policy(const Shape& s, int seq_len, int* n_splits, int* tile) {
    const DecodePlan pl = decode_plan(s, seq_len);
    *n_splits = pl.n_splits;
    *tile = pl.tile;
}

static DecodeParams decode_params(const Shape& s, const DecodeArgs& a) {
    return DecodeParams{a.q,        a.k_new,   a.v_new,     a.k_cache,  a.v_cache,
                    a.cos_t,    a.sin_t,   a.out,       a.part_o,   a.part_ml,
                    a.pos,      a.n_splits,  s.num_heads,
                    s.kv_dim,   s.kv_mul,  s.half,
                    1.4426950408889634f / sqrtf((float)s.head_dim)};
}

hipError_t launch_decode_combine(const Shape& s, const DecodeArgs& a, hipStream_t st) {
    const DecodeParams dp = decode_params(s, a);
    if (a.n_splits < 2 || a.n_splits > kMaxSplits) return hipErrorInvalidValue;
    switch (s.head_dim) {
        case 16: return launch_combine_t<16>(s, dp, st, a.ev_start, a.ev_stop);
        case 32: return launch_combine_t<32>(s, dp, st, a.ev_start, a.ev_stop);
        case 48: return launch_combine_t<48>(s, dp, st, a.ev_start, a.ev_stop);
        case 64: return launch_combine_t<64>(s, dp, st, a.ev_start, a.ev_stop);
        case 96: return launch_combine_t<96>(s, dp, st, a.ev_start, a.ev_stop);
        case 128: return launch_combine_t<128>(s, dp, st, a.ev_start, a.ev_stop);
        case 256: return launch_combine_t<256>(s, dp, st, a.ev_start, a.ev_stop);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_decode(const Shape& s, const DecodeArgs& a, hipStream_t st) {
    const DecodeParams dp = decode_params(s, a);
    if (a.n_splits < 1 || a.n_splits > kMaxSplits) return hipErrorInvalidValue;
    // the appended k row is rotated with the tables (the kernel reads them
    // whenever it appends)
    if (a.k_new != nullptr && (a.cos_t == nullptr || a.sin_t == nullptr || a.v_new == nullptr))
        return hipErrorInvalidValue;
    const Tiling t = decode_plan(s, a.pos + 1).tiling;
    switch (s.head_dim) {
        case 16: return launch_hd<16>(s, dp, t, st, a.ev_start, a.ev_stop);
        case 32: return launch_hd<32>(s, dp, t, st, a.ev_start, a.ev_stop);
        case 48: return launch_hd<48>(s, dp, t, st, a.ev_start, a.ev_stop);
        case 64: return launch_hd<64>(s, dp, t, st, a.ev_start, a.ev_stop);
        case 96: return launch_hd<96>(s, dp, t, st, a.ev_start, a.ev_stop);
        case 128: return launch_hd<128>(s, dp, t, st, a.ev_start, a.ev_stop);
        case 256: return launch_hd<256>(s, dp, t, st, a.ev_start, a.ev_stop);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace slm
