// Causal prefill attention on fp32 MFMA (v_mfma_f32_16x16x4_f32) for gfx950.
//
// Replaces the per-row loop of forward_batch_with_kv (transformer.rs:563-593),
// where row b at position p = start + b attends to cache rows 0..p.
//
// Tiling.  A workgroup of HW*QS waves owns one query block and HW query heads
// of one KV head (HW divides kv_mul), so every K/V tile staged in LDS serves
// HW*QS waves.  Each wave owns 16*NQT query rows of one head.  Keys stream
// through LDS in tiles of 32 rows.  For hd 128 with four heads per KV head
// (the Llama-3-8B shape) eight waves share each tile and the tiles go from
// memory straight into two LDS buffers (buffer loads with the lds bit), with
// no registers held for the next tile, four waves per SIMD; otherwise the
// next tile is prefetched into registers while the current one is in use.
//
// Transposed products keep softmax state lane-local.  With the 16x16x4 MFMA
// layout (lane l: A[l%16][l/16], B[l/16][l%16], D[4*(l/16)+r][l%16]):
//   S^T = K . Q^T   A = K rows (keys) , B = Q^T (queries): lane l ends with
//                   scores of query l%16 against keys 4*(l/16)+r;
//   O^T = V^T . P^T A = V^T (head dims), B = P^T: k-step j of a 16-key block
//                   uses key 4*(l/16)+j, which is exactly D register j of S^T,
//                   so probabilities feed the second MFMA with no shuffle;
//                   lane l accumulates O^T[d][query l%16].
// The head dimension is split into four contiguous quarters, one per lane
// group l/16, so Q and K fragments are contiguous (128-bit loads) and the
// RoPE pairs of q stay inside one lane.
//
// Online softmax runs in the log2 domain (q pre-scaled by log2(e)/sqrt(hd));
// the running max is reduced across the four lane groups each tile, the
// running sum stays a per-lane partial until the end.
//
// Which form of the kernel a batch runs (heads and blocks per workgroup,
// paired blocks, key splits, DMA-fed tiles) is decided in prefill_plan.h,
// with the measurements behind each rule.
#include <math.h>

#include <type_traits>

#include "attn_common.h"
#include "prefill_plan.h"
#include "slm_internal.h"
#include "tile_range.h"

namespace slm {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));


__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

struct PrefillParams {
    const float* q;
    const float* k_cache;
    const float* v_cache;
    const float* cos_t;
    const float* sin_t;
    float* out;
    int start;
    int n;
    int dim;
    int num_heads;
    int kv_dim;
    int kv_mul;
    int half;
    float scale_log2;
};

// LDS tile layouts.  Measured on MI355X with the bank-conflict counter over
// single-pattern probes: a 64-lane ds_read_b128 takes 4 cycles when free of
// conflicts (64 banks of 4 bytes), and each cycle serves the 16 lanes of one
// half-wave that agree in the parity of lane bits 2-4 (bit 0 may also count;
// the layouts below are conflict-free either way).  Two lanes of one cycle
// conflict when their addresses differ but agree modulo 64 floats.
//
// K tile: lane (lr, lg) reads row lr of a 16-key block at head dims
// lg*HD/4 + 4c.  With row stride HD + 4 the lanes l and l^8^16 always share
// banks (lg*HD/4 moves by a multiple of 64 floats for every other lg); the
// 128-bit chunk index of a row is therefore XORed with k_swz(row) where that
// helps.  V tile: the lanes of one cycle read rows 4 apart at their own NDT
// head dims; the row stride and the chunk order v_rot (below) are chosen per
// head_dim.  Both checked conflict-free (reads and the tile stores) against
// the measured rule on the CPU for head_dim 128 and 256; for 64 the V reads
// and the K reads are, the K stores are not.
template <int HD>
struct PrefillLds {
    static constexpr int LDK = HD + 4;  // floats per K row
    static constexpr int LDV = HD + 4;  // floats per V row
    static __device__ __forceinline__ int k_swz(int) { return 0; }
};
template <>
struct PrefillLds<64> {
    static constexpr int LDK = 68;
    static constexpr int LDV = 64;
    static __device__ __forceinline__ int k_swz(int r) { return (((r >> 2) ^ (r >> 3)) & 1) << 2; }
};
template <>
struct PrefillLds<128> {
    static constexpr int LDK = 132;
    static constexpr int LDV = 132;
    static __device__ __forceinline__ int k_swz(int r) { return ((r >> 3) & 1) << 3; }
};
template <>
struct PrefillLds<256> {
    static constexpr int LDK = 260;
    static constexpr int LDV = 256;
    static __device__ __forceinline__ int k_swz(int) { return 0; }
};

// Tiles written by buffer->LDS DMA (hd 128): a wave's DMA instruction fills
// 1 KiB of LDS contiguously, so rows cannot be padded.  Rows are 128 floats;
// the K chunk index is XORed with k_swz(row) (bits 0-1 and 3 of the row), and
// lane m reads its two V chunks in the order vrot(m).  Checked conflict-free
// under the rule above on the CPU, for both readings of the lane grouping.
template <int HD>
struct PrefillLdsDma;
template <>
struct PrefillLdsDma<128> {
    static constexpr int LDK = 128;
    static constexpr int LDV = 128;
    static __device__ __forceinline__ int k_swz(int r) { return (r & 3) | (((r >> 3) & 1) << 2); }
    static __device__ __forceinline__ int vrot(int m) { return (m >> 3) & 1; }
};

// First 128-bit chunk lane m reads of its NDT contiguous V dims (NDT a
// multiple of 4; lane m starts at float m*NDT of its row): with the V row
// strides above, every cycle's 16 lanes then cover the 64 banks once.
template <int NDT>
__device__ __forceinline__ int v_rot(int m) {
    if constexpr (NDT == 8) return ((m >> 2) ^ (m >> 3)) & 1;
    if constexpr (NDT == 16) return (((m >> 1) ^ (m >> 3)) & 1) | (((m >> 2) & 1) << 1);
    return 0;
}

// Two waves per SIMD let one wave's MFMAs overlap another's softmax; the
// largest variants keep one wave per SIMD rather than spill.
template <int HD, int HW>
constexpr int prefill_waves_per_simd() {
    return HD > 128 ? 1 : 2;
}

// DMA: K/V tiles go straight from memory to LDS (buffer loads with the lds
// bit) into two buffers, with no registers held for the next tile; four waves
// per SIMD.  Otherwise the next tile is prefetched into registers.
//
// KSP (register prefetch only): key splits.  The workgroup holds KSP sets of
// HW*QS waves; set k attends tiles k, k + KSP, k + 2*KSP, ... of its query
// block, the KSP tiles of a step loaded together into KSP LDS slots, and at
// the end sets 1..KSP-1 hand their (max, sum, O) to set 0 through LDS, which
// merges them in set order.  Used for short prefills with one head per
// workgroup (head_dim <= 64): the heaviest causal block's key tiles are
// walked by KSP SIMDs instead of one.  (Splitting keys among the waves of a workgroup that
// already has a wave on every SIMD gains nothing: the per-SIMD MFMA work of
// the heaviest block stays the same.)
//
// PAIR (with QS = 2): the workgroup's two query blocks are i and n_qb-1-i
// (16-row blocks), so every workgroup has the same causal work, and the
// waves are numbered key split first, then head, then block: the waves of one
// SIMD hold the same head and key split of the heavy and the light block,
// and every SIMD gets the same share.
template <int HD, int HW, int QS, int NQT, int kKT = 32, int NB = 1, bool PRIO = false,
          bool DMA = false, int KSP = 1, bool PAIR = false>
__global__ __launch_bounds__(64 * HW * QS * KSP,
                             (DMA ? 4 : prefill_waves_per_simd<HD, HW>())) void
prefill_mfma_kernel(PrefillParams p) {
    constexpr int KS = kKT / 16;  // 16-key sub-tiles per LDS tile
    constexpr int NWS = HW * QS;  // waves of one key split
    constexpr int NW = NWS * KSP;
    constexpr int NT = 64 * NW;
    using Lds = std::conditional_t<DMA, PrefillLdsDma<HD>, PrefillLds<HD>>;
    constexpr int LDK = Lds::LDK;
    constexpr int LDV = Lds::LDV;
    constexpr int DPL = HD / 4;   // contiguous head dims per lane group
    constexpr int NDT = HD / 16;  // 16-wide head-dim tiles of O^T
    constexpr int QPW = 16 * NQT; // query rows per wave
    constexpr int QB = QPW * QS;  // query rows per workgroup
    constexpr int F4 = kKT * HD / 4;          // float4 per K (or V) tile
    constexpr int NPF = (F4 * KSP + NT - 1) / NT;  // float4 per thread per step
    static_assert(DPL % 4 == 0 && HD % 16 == 0, "head_dim must be a multiple of 16");
    // PV operands.  With NDT a multiple of 4, row m of each 16-dim O^T tile
    // maps to lane m's own NDT contiguous head dims, read from the V tile as
    // VC 128-bit chunks, lane m starting at chunk v_rot<NDT>(m).  (Reading
    // dims dt*16 + lane as 32-bit words gave more bank conflict cycles than
    // LDS instructions on the 4096-row prefill.)
    constexpr bool VEC_V = NDT % 4 == 0;
    constexpr int VC = VEC_V ? NDT / 4 : 1;

    // NB LDS buffers: with two, a tile is stored while the other is read and
    // one barrier per tile suffices.  With key splits, KSP tile slots (one
    // buffer each), in one array so the merge at the end can reuse it whole.
    static_assert(!DMA || NB == 2, "DMA tiles use two buffers");
    static_assert(KSP == 1 || (!DMA && NB == 1), "key splits: register prefetch, one buffer");
    static_assert(KSP == 1 || F4 % 64 == 0, "key splits: a wave's tile loads in one slot");
    constexpr int NSLOT = NB * KSP;
    __shared__ __align__(16) float s_tiles[NSLOT * kKT * (LDK + LDV)];
    float(*sKb)[kKT * LDK] = reinterpret_cast<float(*)[kKT * LDK]>(s_tiles);
    float(*sVb)[kKT * LDV] = reinterpret_cast<float(*)[kKT * LDV]>(s_tiles + NSLOT * kKT * LDK);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    // wave-uniform, and known to be: the per-wave tests below (the causal
    // mask only on diagonal tiles, rows past the wave's last position) then
    // compile to branches instead of per-lane selects on every tile
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 15;
    const int lg = lane >> 4;
    static_assert(!PAIR || (QS == 2 && NQT == 1), "pairs: two 16-row blocks");
    const int hw = PAIR ? (wave / KSP) % HW : wave % HW;
    const int qs = PAIR ? wave / (KSP * HW) : (wave / HW) % QS;
    const int kspl = PAIR ? wave % KSP : wave / NWS;  // key split

    // blockIdx.x = query block * head groups + head group: consecutive
    // workgroups go round-robin to the 8 XCDs, so with 8 head groups each XCD's
    // L2 serves one KV head's K/V; longest causal ranges are launched first.
    // Pairs: blockIdx.x = pair * head groups + head group, pair i holding
    // 16-row blocks n_qb-1-i (qs 0) and i (qs 1); with n_qb odd the middle
    // pair's second block is the first's, and its waves hold no rows.
    const int n_qb = PAIR ? (p.n + QPW - 1) / QPW : (p.n + QB - 1) / QB;
    const int n_hg = p.num_heads / HW;
    const int hg = (int)blockIdx.x % n_hg;
    const int head = hg * HW + hw;
    const int g = (hg * HW) / p.kv_mul;
    int q0, kv_len;  // first query row of this wave; keys 0..kv_len-1
    if constexpr (PAIR) {
        const int pi = (int)blockIdx.x / n_hg;
        const int heavy = n_qb - 1 - pi;
        q0 = qs == 0 ? heavy * QPW : pi < heavy ? pi * QPW : p.n;
        kv_len = p.start + min(p.n, (heavy + 1) * QPW);
    } else {
        const int qb = n_qb - 1 - (int)blockIdx.x / n_hg;
        q0 = qb * QB + qs * QPW;
        kv_len = p.start + qb * QB + min(p.n - qb * QB, QB);
    }
    const int n_tiles = (kv_len + kKT - 1) / kKT;
    const int wave_rows = max(0, min(QPW, p.n - q0));
    const int wave_last_pos = p.start + q0 + wave_rows - 1;

    // Q fragments: row q0 + qt*16 + lr, dims lg*DPL .. +DPL, rotated, scaled.
    // All q and table loads are issued before the first use (a load inside
    // the rotate branch would wait for every earlier load, once per float4).
    const bool rot = p.cos_t != nullptr;
    float4 qx[NQT][DPL / 4];
    float2 qc[NQT][DPL / 4], qsn[NQT][DPL / 4];
    bool qok[NQT];
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
        const int row = q0 + qt * 16 + lr;
        qok[qt] = row < p.n;
        const float* src = p.q + (long)(qok[qt] ? row : 0) * p.dim + head * HD + lg * DPL;
#pragma unroll
        for (int c = 0; c < DPL / 4; ++c) qx[qt][c] = ld4(src + 4 * c);  // zeroed below if !ok
    }
    if (rot) {
#pragma unroll
        for (int qt = 0; qt < NQT; ++qt) {
            const int row = min(q0 + qt * 16 + lr, p.n - 1);
            const long tr = (long)(p.start + row) * p.half + (lg * DPL >> 1);
#pragma unroll
            for (int c = 0; c < DPL / 4; ++c) {
                qc[qt][c] = *reinterpret_cast<const float2*>(p.cos_t + tr + 2 * c);
                qsn[qt][c] = *reinterpret_cast<const float2*>(p.sin_t + tr + 2 * c);
            }
        }
    }
    float qf[NQT][DPL];
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
#pragma unroll
        for (int c = 0; c < DPL / 4; ++c) {
            float4 x = qok[qt] ? qx[qt][c] : make_float4(0.f, 0.f, 0.f, 0.f);
            if (rot) x = rope4_exact(x, qc[qt][c], qsn[qt][c]);
            qf[qt][4 * c + 0] = x.x * p.scale_log2;
            qf[qt][4 * c + 1] = x.y * p.scale_log2;
            qf[qt][4 * c + 2] = x.z * p.scale_log2;
            qf[qt][4 * c + 3] = x.w * p.scale_log2;
        }
    }

    // Softmax state per query tile (log2 domain): m, the running max (-inf
    // before the first key); om, the offset the score accumulators start
    // from (negm holds -om four times: the QK^T MFMAs then return s - om, and
    // exp2 takes them without a subtraction); lim, how far a tile's max may
    // exceed om before the state is rescaled (kLazyRescale once m is set, -inf
    // before the first tile, which therefore always rescales).
    floatx4 o[NQT][NDT];
    float m[NQT], l[NQT], om[NQT], lim[NQT];
    floatx4 negm[NQT];
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
        m[qt] = -INFINITY;
        l[qt] = 0.0f;
        om[qt] = 0.0f;
        lim[qt] = -INFINITY;
        negm[qt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) o[qt][dt] = floatx4{0.f, 0.f, 0.f, 0.f};
    }

    auto vrot_of = [](int m) {
        if constexpr (DMA)
            return Lds::vrot(m);
        else
            return v_rot<NDT>(m);
    };
    int v_off[VC];  // this lane's chunk offsets inside its NDT dims
#pragma unroll
    for (int c = 0; c < VC; ++c) v_off[c] = 4 * ((c + vrot_of(lr)) % VC);

    const float* kg = p.k_cache + g * HD;
    const float* vg = p.v_cache + g * HD;
    // This thread's NPF float4 of a tile sit at fixed byte offsets from the
    // tile's first row, so a tile is loaded through a buffer descriptor built
    // from uniform values (scalar work) plus those offsets: no vector
    // arithmetic per tile (on this part VALU work of one wave does not overlap
    // another wave's fp32 MFMAs on the same SIMD, so every VALU instruction in
    // the loop costs MFMA time).  The descriptor's range ends at row kv_len,
    // and buffer loads past the range return zeros: the rows past the end
    // read as zeros without a branch.
    constexpr int NI = DMA ? F4 / NT : 1;  // DMA instructions per wave, tile and matrix
    static_assert(!DMA || F4 % NT == 0, "DMA tiles: whole instructions per wave");
    int t_off[DMA ? 1 : NPF];
    int d_off_k[NI], d_off_v[NI];
    if constexpr (DMA) {
        // instruction i of this wave fills float4 slots (wave*NI + i)*64 + lane
        // of a tile; K slot (row r, chunk c) receives chunk c ^ k_swz(r)
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int f = (wave * NI + i) * 64 + lane;
            const int r = f / (HD / 4), c = f % (HD / 4);
            d_off_k[i] = (r * p.kv_dim + 4 * (c ^ Lds::k_swz(r))) * 4;
            d_off_v[i] = (r * p.kv_dim + 4 * c) * 4;
        }
    } else {
#pragma unroll
        for (int i = 0; i < NPF; ++i) {
            const int f = (tid + i * NT) % F4;  // within its tile slot
            t_off[i] = ((f / (HD / 4)) * p.kv_dim + (f % (HD / 4)) * 4) * 4;
        }
    }
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    auto bload = [](__amdgpu_buffer_rsrc_t r, int off) {
        const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
        return make_float4(__uint_as_float(x.x), __uint_as_float(x.y), __uint_as_float(x.z),
                           __uint_as_float(x.w));
    };
    float4 pk[DMA ? 1 : NPF], pv[DMA ? 1 : NPF];
    static_assert(tile_range_fits(kKT, kMaxKvDim), "tile ranges must fit 32 bits");
    // Register prefetch of the KSP tiles from tile kt0: this thread's float4 i
    // belongs to slot (wave*64 + i*NT) / F4 (whole waves per slot, so the
    // slot and its descriptor are wave-uniform); slots past the last tile
    // load nothing.
    auto prefetch_regs = [&](int kt0) __attribute__((always_inline)) {
        if constexpr (KSP == 1) {
            // one tile: one descriptor for all of this thread's loads
            const int kb = kt0 * kKT;
            const int bytes = (int)tile_range_bytes(kv_len, kb, kKT, p.kv_dim);
            const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float*>(kg + (long)kb * p.kv_dim), 0, bytes, 0x00020000);
            const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float*>(vg + (long)kb * p.kv_dim), 0, bytes, 0x00020000);
#pragma unroll
            for (int i = 0; i < NPF; ++i) {
                if (tid + i * NT < F4) {
                    pk[i] = bload(rk, t_off[i]);
                    pv[i] = bload(rv, t_off[i]);
                }
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < NPF; ++i) {
            if (wave * 64 + i * NT >= F4 * KSP) continue;  // uniform
            const int slot = (wave * 64 + i * NT) / F4;
            const int kb = (kt0 + slot) * kKT;
            if (kt0 + slot >= n_tiles) continue;  // uniform
            const int bytes = (int)tile_range_bytes(kv_len, kb, kKT, p.kv_dim);
            const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float*>(kg + (long)kb * p.kv_dim), 0, bytes, 0x00020000);
            const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float*>(vg + (long)kb * p.kv_dim), 0, bytes, 0x00020000);
            if (tid + i * NT < F4 * KSP) {
                pk[i] = bload(rk, t_off[i]);
                pv[i] = bload(rv, t_off[i]);
            }
        }
    };
    auto prefetch = [&](int kb, int buf) __attribute__((always_inline)) {
        // rows kb .. min(kv_len, kb + kKT) - 1: bounded by the tile (one
        // layer's K slice may pass 4 GiB)
        const int bytes = (int)tile_range_bytes(kv_len, kb, kKT, p.kv_dim);
        const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(kg + (long)kb * p.kv_dim), 0, bytes, 0x00020000);
        const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(vg + (long)kb * p.kv_dim), 0, bytes, 0x00020000);
        if constexpr (DMA) {
            // Issued as inline assembly: the compiler then sees no LDS store
            // here, so it does not make the current tile's LDS reads wait for
            // this DMA (it cannot tell the two buffers apart); the vmcnt(0)
            // wait and the barrier ahead of the next tile order them instead.
            // M0 holds the wave's LDS destination; lane l's 16 bytes land at
            // M0 + 16*l.
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const unsigned lk = (unsigned)(unsigned long)(
                    __attribute__((address_space(3))) float*)&sKb[buf][(wave * NI + i) * 256];
                const unsigned lv = (unsigned)(unsigned long)(
                    __attribute__((address_space(3))) float*)&sVb[buf][(wave * NI + i) * 256];
                asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(d_off_k[i]),
                             "s"(rk), "{m0}"(lk) : "memory");
                asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(d_off_v[i]),
                             "s"(rv), "{m0}"(lv) : "memory");
            }
        } else {
            (void)buf;  // register prefetch goes through prefetch_regs
            (void)rk;
            (void)rv;
        }
    };

    // One key tile: S^T = K.Q^T, causal mask, online softmax, O^T += V^T.P^T.
    auto attend = [&](int kb, const float* sK, const float* sV) __attribute__((always_inline)) {
        // S^T tiles [key sub-tile][query tile]; the KS*NQT accumulators are
        // updated round-robin so consecutive MFMAs never depend on each other
        if (PRIO) __builtin_amdgcn_s_setprio(1);
        floatx4 s[KS][NQT];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int qt = 0; qt < NQT; ++qt) s[ks][qt] = negm[qt];
#pragma unroll
        for (int c = 0; c < DPL / 4; ++c) {
            float4 kf[KS];
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
                kf[ks] = ld4(&sK[(ks * 16 + lr) * LDK +
                                 4 * ((lg * (DPL / 4) + c) ^ Lds::k_swz(ks * 16 + lr))]);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    const float ke = e == 0 ? kf[ks].x : e == 1 ? kf[ks].y : e == 2 ? kf[ks].z : kf[ks].w;
#pragma unroll
                    for (int qt = 0; qt < NQT; ++qt)
                        s[ks][qt] = mfma4(ke, qf[qt][4 * c + e], s[ks][qt]);
                }
            }
        }

        if (PRIO) __builtin_amdgcn_s_setprio(0);

        // causal mask, online softmax
        const bool diag = kb + kKT - 1 > p.start + q0;  // some key may be masked
#pragma unroll
        for (int qt = 0; qt < NQT; ++qt) {
            const int qpos = p.start + q0 + qt * 16 + lr;
            if (diag) {  // uniform: only tiles that reach past a query of the wave
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (kb + ks * 16 + 4 * lg + r > qpos) s[ks][qt][r] = -INFINITY;
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            float mx = -INFINITY;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
                for (int r = 0; r < 4; ++r) mx = fmaxf(mx, s[ks][qt][r]);
            }
            mx = rows_max(mx);  // of s - om
            // Without key splits the first tile always holds key 0 <= qpos, so
            // mx is finite there.  With them, the first tile a split attends
            // may mask every key of a query (positions below the tile): such a
            // lane has seen no key yet and keeps its empty state (max -inf,
            // no offset), or exp2(-inf - -inf) would make it NaN.
            if (__any(mx > lim[qt])) {  // wave-uniform
                const float mn = fmaxf(m[qt], mx + om[qt]);
                bool none = false;
                if constexpr (KSP > 1) none = mn == -INFINITY;
                const float alpha = none ? 1.0f : __builtin_amdgcn_exp2f(m[qt] - mn);
                l[qt] *= alpha;
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) o[qt][dt] *= alpha;
                // this tile's scores move to the new offset
                const float d = none ? 0.0f : mn - om[qt];
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) s[ks][qt][r] -= d;
                }
                m[qt] = mn;
                if (!none) {
                    om[qt] = mn;
                    lim[qt] = kLazyRescale;
                    negm[qt] = floatx4{-mn, -mn, -mn, -mn};
                }
            }
            float ps = 0.0f;  // starts at the first term (0 + e is e exactly, e >= 0)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float e = __builtin_amdgcn_exp2f(s[ks][qt][r]);
                    s[ks][qt][r] = e;
                    ps = (ks == 0 && r == 0) ? e : ps + e;
                }
            }
            l[qt] += ps;
        }

        // O^T += V^T . P^T
        if (PRIO) __builtin_amdgcn_s_setprio(1);
        if constexpr (VEC_V) {
            // row m of every O^T tile belongs to lane m: its NDT head dims are
            // contiguous, read as 128-bit chunks in the lane's rotated order
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float* vrow = &sV[(ks * 16 + 4 * lg + j) * LDV + lr * NDT];
                    float4 vc[VC];
#pragma unroll
                    for (int c = 0; c < VC; ++c) vc[c] = ld4(vrow + v_off[c]);
#pragma unroll
                    for (int c = 0; c < VC; ++c) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float vf = e == 0 ? vc[c].x : e == 1 ? vc[c].y : e == 2 ? vc[c].z : vc[c].w;
#pragma unroll
                            for (int qt = 0; qt < NQT; ++qt)
                                o[qt][4 * c + e] = mfma4(vf, s[ks][qt][j], o[qt][4 * c + e]);
                        }
                    }
                }
            }
        } else {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float* vrow = &sV[(ks * 16 + 4 * lg + j) * LDV + lr];
#pragma unroll
                    for (int dt = 0; dt < NDT; ++dt) {
                        const float vf = vrow[dt * 16];
#pragma unroll
                        for (int qt = 0; qt < NQT; ++qt)
                            o[qt][dt] = mfma4(vf, s[ks][qt][j], o[qt][dt]);
                    }
                }
            }
        }
        if (PRIO) __builtin_amdgcn_s_setprio(0);
    };

    if constexpr (DMA)
        prefetch(0, 0);
    else
        prefetch_regs(0);
    if constexpr (DMA) {
        // Two tiles per trip, so each tile's buffer is a compile-time constant:
        // the LDS read addresses are then loop-invariant registers plus
        // immediate offsets instead of being recomputed per tile.
        auto step = [&](int it, auto buf_c) __attribute__((always_inline)) {
            constexpr int buf = decltype(buf_c)::value;
            // this wave's DMA of tile it has landed; after the barrier every
            // wave's has, and every wave is done with the other buffer
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            if (it + 1 < n_tiles) prefetch((it + 1) * kKT, buf ^ 1);
            const int kb = it * kKT;
            if (wave_rows == 0 || kb > wave_last_pos) return;  // wave-uniform
            attend(kb, sKb[buf], sVb[buf]);
        };
        for (int it = 0; it < n_tiles; it += 2) {
            step(it, std::integral_constant<int, 0>());
            if (it + 1 < n_tiles) step(it + 1, std::integral_constant<int, 1>());
        }
    } else {
        // step st: tiles st*KSP .. st*KSP + KSP - 1 in slots 0..KSP-1; key
        // split kspl attends slot kspl
        const int n_steps = (n_tiles + KSP - 1) / KSP;
        for (int st = 0; st < n_steps; ++st) {
            const int kt0 = st * KSP;
            if (NB == 1) __syncthreads();  // every wave is done with the previous tiles
#pragma unroll
            for (int i = 0; i < NPF; ++i) {
                const int f = tid + i * NT;
                if constexpr (KSP == 1) {
                    if (f < F4) {
                        const int r = f / (HD / 4), ch = f % (HD / 4);
                        float* sK = sKb[st % NB];
                        float* sV = sVb[st % NB];
                        *reinterpret_cast<float4*>(&sK[r * LDK + 4 * (ch ^ Lds::k_swz(r))]) =
                            pk[i];
                        *reinterpret_cast<float4*>(&sV[r * LDV + 4 * ch]) = pv[i];
                    }
                } else {
                    const int slot = (wave * 64 + i * NT) / F4;  // uniform
                    if (f < F4 * KSP && kt0 + slot < n_tiles) {
                        const int fr = f % F4;
                        const int r = fr / (HD / 4), ch = fr % (HD / 4);
                        float* sK = sKb[(st % NB) * KSP + slot];
                        float* sV = sVb[(st % NB) * KSP + slot];
                        *reinterpret_cast<float4*>(&sK[r * LDK + 4 * (ch ^ Lds::k_swz(r))]) =
                            pk[i];
                        *reinterpret_cast<float4*>(&sV[r * LDV + 4 * ch]) = pv[i];
                    }
                }
            }
            __syncthreads();
            if (st + 1 < n_steps) prefetch_regs(kt0 + KSP);
            const int it = kt0 + kspl;
            const int kb = it * kKT;
            if (it >= n_tiles || wave_rows == 0 || kb > wave_last_pos) continue;  // uniform
            attend(kb, sKb[(st % NB) * KSP + kspl], sVb[(st % NB) * KSP + kspl]);
        }
    }

    if constexpr (KSP > 1) {
        // Merge of the key splits: sets 1..KSP-1 write each lane's O
        // registers, max and sum partial to the tile LDS (lane-contiguous,
        // no bank conflicts), set 0 folds them in set order: M = max of the
        // maxima, every state scaled by 2^(m - M) (0 for a set that saw no
        // key), then summed.
        constexpr int NR = NQT * (NDT * 4 + 2);  // floats per lane
        static_assert((KSP - 1) * NWS * 64 * NR <= NSLOT * kKT * (LDK + LDV),
                      "the merge fits the tile LDS");
        __syncthreads();  // every wave is done with the tiles
        const int ws = qs * HW + hw;  // the wave's place in its key split's set
        if (kspl > 0) {
            float* dst = s_tiles + ((kspl - 1) * NWS + ws) * NR * 64 + lane;
            int r = 0;
#pragma unroll
            for (int qt = 0; qt < NQT; ++qt) {
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                    for (int e = 0; e < 4; ++e) dst[64 * r++] = o[qt][dt][e];
                dst[64 * r++] = m[qt];
                dst[64 * r++] = l[qt];
            }
        }
        __syncthreads();
        if (kspl > 0) return;  // no barrier follows
#pragma unroll
        for (int qt = 0; qt < NQT; ++qt) {
            constexpr int MOFF = NDT * 4;  // m, then l, after a query tile's O
            float mk[KSP];
            mk[0] = m[qt];
            float mx = m[qt];
#pragma unroll
            for (int k = 1; k < KSP; ++k) {
                mk[k] = s_tiles[((k - 1) * NWS + ws) * NR * 64 + lane +
                                64 * (qt * (MOFF + 2) + MOFF)];
                mx = fmaxf(mx, mk[k]);
            }
            const float s0 = __builtin_amdgcn_exp2f(m[qt] - mx);
            l[qt] *= s0;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) o[qt][dt] *= s0;
#pragma unroll
            for (int k = 1; k < KSP; ++k) {
                const float* src = s_tiles + ((k - 1) * NWS + ws) * NR * 64 + lane +
                                   64 * qt * (MOFF + 2);
                const float sk = __builtin_amdgcn_exp2f(mk[k] - mx);
                l[qt] += src[64 * (MOFF + 1)] * sk;
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                    for (int e = 0; e < 4; ++e) o[qt][dt][e] += src[64 * (dt * 4 + e)] * sk;
            }
        }
    }

    // normalise and store
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
        const float lt = rows_sum(l[qt]);
        const int row = q0 + qt * 16 + lr;
        if (row < p.n) {
            const float inv = 1.0f / lt;
            float* dst = p.out + (long)row * p.dim + head * HD;
            if constexpr (VEC_V) {
                // register r of tile 4c+e holds O^T row m = 4*lg + r, whose dims
                // are m*NDT + (chunk c in lane m's rotated order) + e
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int m = 4 * lg + r;
                    const int rot = vrot_of(m);
#pragma unroll
                    for (int c = 0; c < VC; ++c) {
                        float4 x;
                        x.x = o[qt][4 * c + 0][r] * inv;
                        x.y = o[qt][4 * c + 1][r] * inv;
                        x.z = o[qt][4 * c + 2][r] * inv;
                        x.w = o[qt][4 * c + 3][r] * inv;
                        *reinterpret_cast<float4*>(dst + m * NDT + 4 * ((c + rot) % VC)) = x;
                    }
                }
            } else {
                // lane holds out[row][dt*16 + 4*lg .. +3]
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) {
                    float4 r;
                    r.x = o[qt][dt][0] * inv;
                    r.y = o[qt][dt][1] * inv;
                    r.z = o[qt][dt][2] * inv;
                    r.w = o[qt][dt][3] * inv;
                    *reinterpret_cast<float4*>(dst + 4 * lg + dt * 16) = r;
                }
            }
        }
    }
}

template <int HD, int HW, int QS, int KSP, bool PAIR = false>
hipError_t launch_t(const Shape& s, const PrefillParams& pp, hipStream_t st) {
    // 16 query rows per wave: measured on MI355X (hd 128, 4096 rows) 57% of
    // the fp32 MFMA peak against 47% with 32 rows per wave, because the lower
    // register count (~160 VGPRs) allows three waves per SIMD
    constexpr int NQT = 1;
    constexpr int QB = 16 * NQT * QS;
    const int n_qb = PAIR ? ((pp.n + 15) / 16 + 1) / 2 : (pp.n + QB - 1) / QB;
    const dim3 grid(n_qb * (s.num_heads / HW));
    hipLaunchKernelGGL((prefill_mfma_kernel<HD, HW, QS, NQT, 32, 1, false, false, KSP, PAIR>),
                       grid, dim3(64 * HW * QS * KSP), 0, st, pp);
    return hipGetLastError();
}

template <int HD>
hipError_t launch_hd(const Shape& s, const PrefillParams& pp, hipStream_t st) {
    switch (prefill_plan(s.head_dim, s.num_heads, s.kv_mul, s.cus, pp.start, pp.n)) {
        case PrefillKernel::kFourHeads: return launch_t<HD, 4, 1, 1>(s, pp, st);
        case PrefillKernel::kThreeHeads: return launch_t<HD, 3, 1, 1>(s, pp, st);
        case PrefillKernel::kTwoHeads: return launch_t<HD, 2, 2, 1>(s, pp, st);
        case PrefillKernel::kOneHead: return launch_t<HD, 1, 4, 1>(s, pp, st);
        case PrefillKernel::kKeySplit:
            if constexpr (HD <= 64) return launch_t<HD, 1, 1, 4>(s, pp, st);
            break;
        case PrefillKernel::kPairedFourHeads:
            if constexpr (HD <= 96) return launch_t<HD, 4, 2, 1, true>(s, pp, st);
            break;
        case PrefillKernel::kDma:
            if constexpr (HD == 128) {
                const int n_qb = (pp.n + 31) / 32;
                hipLaunchKernelGGL((prefill_mfma_kernel<128, 4, 2, 1, 32, 2, false, true>),
                                   dim3(n_qb * (s.num_heads / 4)), dim3(512), 0, st, pp);
                return hipGetLastError();
            }
            break;
        case PrefillKernel::kDmaPaired:
            if constexpr (HD == 128) {
                const int pwgs = ((pp.n + 15) / 16 + 1) / 2 * (s.num_heads / 4);
                hipLaunchKernelGGL((prefill_mfma_kernel<128, 4, 2, 1, 32, 2, false, true, 1, true>),
                                   dim3(pwgs), dim3(512), 0, st, pp);
                return hipGetLastError();
            }
            break;
        case PrefillKernel::kPairedTwoHeads:
            if constexpr (HD == 128) return launch_t<128, 2, 2, 2, true>(s, pp, st);
            break;
        case PrefillKernel::kPairedOneHead:
            if constexpr (HD == 128) return launch_t<128, 1, 2, 4, true>(s, pp, st);
            break;
    }
    return hipErrorInvalidValue;  // a plan this head_dim has no kernel for
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

hipError_t launch_prefill_mfma(const Shape& s, const PrefillArgs& a, hipStream_t st) {
    PrefillParams pp{a.q,   a.k_cache, a.v_cache,   a.cos_t,  a.sin_t,  a.out, a.start,
                     a.n,   s.dim,     s.num_heads, s.kv_dim, s.kv_mul, s.half,
                     1.4426950408889634f / sqrtf((float)s.head_dim)};
    if (a.n > 65535 * 64) return hipErrorInvalidValue;
    switch (s.head_dim) {
        case 16: return launch_hd<16>(s, pp, st);
        case 32: return launch_hd<32>(s, pp, st);
        case 48: return launch_hd<48>(s, pp, st);
        case 64: return launch_hd<64>(s, pp, st);
        case 96: return launch_hd<96>(s, pp, st);
        case 128: return launch_hd<128>(s, pp, st);
        case 256: return launch_hd<256>(s, pp, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace slm
