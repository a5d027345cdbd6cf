// Q4_0 x Q8_0 projections for gfx950: the Q/K/V projections that feed the
// attention path (transformer.rs:413-417 decode, :530-561 prefill).
//
// Arithmetic.  gemm_q4_0 (kernels.rs:308-394) computes every output as
// vec_dot_q4_0_q8_0 of a Q4_0 weight row and a Q8_0 activation row; the
// scalar dot (kernels.rs:145-161) sums, block by block in order,
//     (isum_b as f32) * (d_w,b * d_a,b)
// into one f32 with no fused multiply-add (the NEON path gives the same
// bits).  Both kernels here keep exactly that: the integer block sums are
// exact (v_dot4 or int8 MFMA), d_w * d_a is exact in f32 (two f16 values),
// and the f32 sum runs over blocks in order, so outputs are bit-identical to
// the scalar reference.  The x86 AVX2 path (kernels.rs:163-212) sums in eight
// FMA lanes and differs from it by at most the reference's own 1e-5 bound.
//
// Activations are quantized with quantize_row_q8_0's arithmetic
// (blocks.rs:102-123): amax, d = amax/127 (correctly rounded divide),
// id = 127/amax, q = round-half-away(x*id) clamped to [-127, 127], d stored
// as f16 (round to nearest even).
//
// Device layout of a weight matrix (slm_q4_matrix): nibbles [rows][nb][16]
// (16-byte aligned rows of blocks) and f16 scales [rows][nb], repacked from
// the reference's 18-byte BlockQ4_0 (blocks.rs:11-19) at upload.
#include <atomic>

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

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

// A token's GEMV reads each weight once: nontemporal loads stream them past
// the caches (measured 6% faster for the 66 MB gate/up GEMV; the GEMM, which
// reuses weights across token tiles, keeps plain loads).
__device__ __forceinline__ uint4 ldq_stream(const uint8_t* p) {
    const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// ---- standalone quantize_row_q8_0: 34-byte BlockQ8_0 output ----
// Four lanes per block (coalesced 32-byte reads per lane).

__global__ __launch_bounds__(256) void quantize_q8_aos_kernel(const float* x, long nblk,
                                                              uint8_t* out) {
    const long i = ((long)blockIdx.x * blockDim.x + threadIdx.x) >> 2;
    const int part = threadIdx.x & 3;
    if (i >= nblk) return;  // uniform over the quad
    const float* blk = x + i * 32 + 8 * part;
    uint2 q;
    uint16_t dbits;
    int sum;
    quantize_q8_quad(ld4(blk), ld4(blk + 4), &q, &dbits, &sum);
    // 34-byte blocks are 2-byte aligned: little-endian u16 stores
    uint16_t* o = reinterpret_cast<uint16_t*>(out + i * 34);
    if (part == 0) o[0] = dbits;
    o[1 + 4 * part + 0] = (uint16_t)(q.x & 0xFFFF);
    o[1 + 4 * part + 1] = (uint16_t)(q.x >> 16);
    o[1 + 4 * part + 2] = (uint16_t)(q.y & 0xFFFF);
    o[1 + 4 * part + 3] = (uint16_t)(q.y >> 16);
}

// ---- activations for the MFMA GEMM: q [n][nb][32] i8, d [n][d_stride] f32 ----
// d rows are padded to d_stride (nb rounded up to 8) so the GEMM reads eight
// blocks' scales with two 128-bit loads.

// With s, the block sums of the quantized values go to s (laid out like d):
// the GEMV's input, whose nibble dot needs them for the -8 offset.
__global__ __launch_bounds__(256) void quantize_q8_soa_kernel(const float* x, long nblk, int nb,
                                                              int d_stride, uint32_t* q,
                                                              float* d, int* s) {
    const long i = ((long)blockIdx.x * blockDim.x + threadIdx.x) >> 2;
    const int part = threadIdx.x & 3;
    if (i >= nblk) return;  // uniform over the quad
    const float* blk = x + i * 32 + 8 * part;
    uint2 qv;
    uint16_t dbits;
    int sum;
    quantize_q8_quad(ld4(blk), ld4(blk + 4), &qv, &dbits, &sum);
    *reinterpret_cast<uint2*>(q + i * 8 + 2 * part) = qv;
    if (part == 0) {
        const long tok = i / nb;
        const long o = tok * d_stride + (i - tok * nb);
        d[o] = h2f(dbits);
        if (s) s[o] = sum;
    }
}

// ---- GEMV: a workgroup per 16-row tile of one matrix ----
//
// Phase 1 quantizes the activation blocks into LDS (four lanes per block;
// max and integer sums are exact, so any reduction order gives the
// reference's values).  Then each wave, owning 4 rows, walks the blocks in
// chunks of 64 (lane l: block 64j + l) in the order the chunks' weight loads
// were issued: it forms the chunk's block terms (isum as f32) * (d_w * d_a),
// passes them through its own LDS rows, and lanes 0..4*NT-1 (one per token
// and row) add them, in block order, to the running sum: the reference's
// single f32 accumulator.  The ordered sum (nb dependent adds per row)
// advances while later chunks are still arriving from HBM.

struct QMat {
    const uint8_t* qs;   // [rows][nb][16]
    const uint16_t* d;   // [rows][d_stride], d_stride = nb rounded up to 8
    float* out;          // out[tok * out_stride + row]
    const float* res;    // nullptr, or the residual added to out (same layout)
    int rows;
    int out_stride;
    int d_stride;
};

constexpr int kGemvRowsPerWave = 4;
constexpr int kGemvRows = 4 * kGemvRowsPerWave;  // rows per workgroup (256 threads)
constexpr int kChunk = 64;                       // blocks per chunk, one per lane
constexpr int kTermStride = kChunk + 4;          // floats per term row in LDS
constexpr int kPrefetch = 2;                     // chunks in flight ahead of the sums

struct GemvParams {
    QMat m[3];
    int nmat;
    int tiles[3];    // kGemvRows-row tiles per matrix
    const float* x;  // [batch][nb*32]
    int nb;
    int batch;
};

__device__ __forceinline__ QMat pick(const QMat (&mm)[3], int m) {
    return m == 0 ? mm[0] : (m == 1 ? mm[1] : mm[2]);
}

// Block b's integer dot with unsigned nibbles: sum(nib_i * a_i) - 8 * sum(a).
__device__ __forceinline__ int block_dot(const uint4 w, const uint32_t (&a)[8], int asum) {
    const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
    int s = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t lo = wd[k] & 0x0F0F0F0Fu;         // weights 4k..4k+3
        const uint32_t hi = (wd[k] >> 4) & 0x0F0F0F0Fu;  // weights 16+4k..
        s = __builtin_amdgcn_sdot4((int)lo, (int)a[k], s, false);
        s = __builtin_amdgcn_sdot4((int)hi, (int)a[4 + k], s, false);
    }
    return s - 8 * asum;
}

// Offset (dwords) of the per-wave term rows: after q [NT][nb][8], d and sum
// [NT][nb], rounded up to 16 bytes.
__host__ __device__ constexpr int gemv_terms_offset(int nt, int nb) {
    return (nt * nb * 10 + 3) & ~3;
}

// Adds t[0..cnt) to s in order; a whole chunk reads its 64 terms at once.
__device__ __forceinline__ float ordered_add(float s, const float* t, int cnt) {
#pragma clang fp contract(off)
    if (cnt == kChunk) {
        float4 v[kChunk / 4];
#pragma unroll
        for (int i = 0; i < kChunk / 4; ++i) v[i] = *reinterpret_cast<const float4*>(t + 4 * i);
#pragma unroll
        for (int i = 0; i < kChunk / 4; ++i) {
            s = s + v[i].x;
            s = s + v[i].y;
            s = s + v[i].z;
            s = s + v[i].w;
        }
        return s;
    }
    for (int i = 0; i < cnt; ++i) s = s + t[i];
    return s;
}

template <int NT, int NBL>
__global__ __launch_bounds__(256) void gemv_q4_kernel(GemvParams p) {
#pragma clang fp contract(off)
    extern __shared__ __align__(16) uint32_t smem[];
    const int nb = p.nb;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    uint32_t* s_q = smem;                                       // [NT][nb][8]
    float* s_d = reinterpret_cast<float*>(smem + NT * nb * 8);  // [NT][nb]
    int* s_sum = reinterpret_cast<int*>(s_d + NT * nb);          // [NT][nb]
    float* s_t = reinterpret_cast<float*>(smem + gemv_terms_offset(NT, nb)) +
                 wave * (NT * kGemvRowsPerWave * kTermStride);   // this wave's [NT*4][kTermStride]

    // workgroup -> (matrix, 16-row tile), uniform
    int tile = blockIdx.x, m = 0;
    while (m < p.nmat - 1 && tile >= p.tiles[m]) {
        tile -= p.tiles[m];
        ++m;
    }
    const QMat M = pick(p.m, m);
    const int rw = tile * kGemvRows + wave * kGemvRowsPerWave;  // this wave's first row

    // Phase 1 quantizes the activation blocks of every token into LDS (pass
    // k: blocks 64k + quad).  The activation loads of the first kPre passes
    // (all of them for one token) go out first, then the weight loads of the
    // first kPrefetch chunks, so the two trips overlap and the wait for the
    // activations (loads complete in issue order) does not include the
    // weights.  Later chunks are loaded kPrefetch chunks ahead of the one
    // being summed: with every chunk in flight at once the memory system
    // returns them in no particular order and the first chunk (which the
    // ordered sums need first) arrives with the last.  Weight addresses are
    // clamped into the matrix instead of guarded (a guarded load with a zero
    // fallback makes the compiler wait for each load before the next); terms
    // of rows or blocks past the end are never used.
    constexpr int kPre = NT * NBL < 8 ? NT * NBL : 8;
    const int nblk = p.batch * nb;
    const int quad = threadIdx.x >> 2;
    const int part = threadIdx.x & 3;
    auto quantize_pass = [&](int idx, float4 f0, float4 f1) {
        uint2 q;
        uint16_t dbits;
        int sum;
        quantize_q8_quad(f0, f1, &q, &dbits, &sum);
        if (idx < nblk) {  // uniform over the quad
            *reinterpret_cast<uint2*>(s_q + idx * 8 + 2 * part) = q;
            if (part == 0) {
                s_d[idx] = h2f(dbits);
                s_sum[idx] = sum;
            }
        }
    };
    float4 xa[kPre][2];
#pragma unroll
    for (int k = 0; k < kPre; ++k) {  // addresses clamped; results past the end not stored
        const float* blk = p.x + (long)min(quad + 64 * k, nblk - 1) * 32 + 8 * part;
        xa[k][0] = ld4(blk);
        xa[k][1] = ld4(blk + 4);
    }
    __builtin_amdgcn_sched_barrier(0);

    uint4 wq[NBL][kGemvRowsPerWave];
    uint16_t wd[NBL][kGemvRowsPerWave];
#define SLM_GEMV_ISSUE(j)                                                                    \
    do {                                                                                     \
        const int b_ = min(kChunk * (j) + lane, nb - 1);                                     \
        _Pragma("unroll") for (int rr = 0; rr < kGemvRowsPerWave; ++rr) {                    \
            const int r_ = min(rw + rr, M.rows - 1);                                         \
            wq[j][rr] = ldq_stream(M.qs + ((long)r_ * nb + b_) * 16);                        \
            wd[j][rr] = __builtin_nontemporal_load(M.d + (long)r_ * M.d_stride + b_);        \
        }                                                                                    \
    } while (0)
#pragma unroll
    for (int j = 0; j < (kPrefetch < NBL ? kPrefetch : NBL); ++j) SLM_GEMV_ISSUE(j);
    __builtin_amdgcn_sched_barrier(0);

#pragma unroll
    for (int k = 0; k < kPre; ++k) {
        if (64 * k >= nblk) break;  // uniform
        quantize_pass(quad + 64 * k, xa[k][0], xa[k][1]);
    }
    for (int k = kPre; 64 * k < nblk; ++k) {
        const int idx = quad + 64 * k;
        const float* blk = p.x + (long)min(idx, nblk - 1) * 32 + 8 * part;
        quantize_pass(idx, ld4(blk), ld4(blk + 4));
    }
    __syncthreads();

    // Chunk j: issue chunk j + kPrefetch, then the block terms of chunk j
    // into this wave's LDS rows, then the ordered sums advance over them.
    // The term rows are the wave's own and a wave's LDS accesses complete in
    // program order, so no workgroup barrier is needed between writing and
    // reading them, nor before the next chunk overwrites them.
    const bool summer = lane < NT * kGemvRowsPerWave && (lane >> 2) < p.batch;
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < NBL; ++j) {  // NBL = ceil(nb / kChunk)
        if (j + kPrefetch < NBL) SLM_GEMV_ISSUE(j + kPrefetch);
        __builtin_amdgcn_sched_barrier(0);
        const int b0 = kChunk * j;
        const int b = b0 + lane;
        if (b < nb) {
#pragma unroll
            for (int tok = 0; tok < NT; ++tok) {
                if (tok >= p.batch) break;
                const int ai = tok * nb + b;
                const uint4 a0 = *reinterpret_cast<const uint4*>(s_q + ai * 8);
                const uint4 a1 = *reinterpret_cast<const uint4*>(s_q + ai * 8 + 4);
                const uint32_t a[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
                const float da = s_d[ai];
                const int asum = s_sum[ai];
#pragma unroll
                for (int rr = 0; rr < kGemvRowsPerWave; ++rr) {
                    const int isum = block_dot(wq[j][rr], a, asum);
                    const float sc = h2f(wd[j][rr]) * da;
                    s_t[(tok * kGemvRowsPerWave + rr) * kTermStride + lane] = (float)isum * sc;
                }
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (summer) acc = ordered_add(acc, s_t + lane * kTermStride, min(kChunk, nb - b0));
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
#undef SLM_GEMV_ISSUE

    if (summer) {
        const int r = rw + (lane & 3);
        if (r < M.rows) {
            const long o = (long)(lane >> 2) * M.out_stride + r;
            // the residual_add JIT kernel, out[i] = a[i] + b[i] (graph.rs:157-164)
            if (M.res) acc = M.res[o] + acc;
            M.out[o] = acc;
        }
    }
}

// ---- GEMV of one token, activations quantized or normalized on the way ----
//
// The activation blocks come quantized (q [nb][32] i8, d and block sums
// [nb]) from the producing kernel, so a workgroup has no quantization phase
// and no barrier: each wave streams its 4 rows chunk by chunk (lane l: block
// 64j + l), loading the weight blocks together with the matching activation
// blocks kPrefetch chunks ahead, and advances the ordered sums chunk by chunk
// as in gemv_q4_kernel.
//
// Or (NORM) the workgroup takes the f32 row the RMSNorm before the
// projection reads (transformer.rs:411 and :448-454: rmsnorm, then the
// projection quantizes its output) and normalizes it itself, with the
// standalone norm kernel's operations in the same order, so the Q8_0 blocks
// it quantizes into LDS carry the same bits: the row and the norm weights
// are loaded and the squares written first, then waves 1-3 issue their
// first weight chunks, so the weights stream in while wave 0 runs the four
// reduction chains.  This takes the norm's launch and its round trip through
// memory off the decode step.

struct GemvAct {
    const uint32_t* aq;  // [nb][8] quantized blocks, or
    const float* ad;     // [nb]
    const int* as;       // [nb]
    const float* x;      // (NORM) the row to normalize, [nb * 32]
    const float* w;      // (NORM) its RMSNorm weights
    float eps;
};

struct GemvQ8Params {
    QMat m[3];
    int nmat;
    int tiles[3];        // kGemvRows-row tiles per matrix
    GemvAct a;
    int nb;
    ArgmaxPart* am;      // (one matrix) each workgroup's best row, or nullptr
};

// LDS of a normalizing workgroup (dwords): the squares [4][norm_sq_stride],
// then the quantized row q [nb][8], d [nb], sums [nb], then the reduction's
// partials [4], tail [4] and scale.
__host__ __device__ constexpr int gemv_norm_q_offset(int nb) {
    return 4 * norm_sq_stride(32 * nb);
}
constexpr size_t gemv_norm_lds_bytes(int nb) {
    return (size_t)(gemv_norm_q_offset(nb) + nb * 10 + 12) * 4;
}

// Waits for the norm weights of the row's passes: they are loaded with the
// row but first read after the reduction, and a wait for them issued behind
// the weight loads would wait for those too (loads complete in order).
template <int KP>
__device__ __forceinline__ void norm_row_wait_w(const NormRow<KP>& r, int nb) {
    const int passes = (nb + 63) / 64;
#pragma unroll
    for (int k = 0; k < KP; ++k) {
        if (k >= passes) break;
#pragma unroll
        for (int h = 0; h < 2; ++h)
            asm volatile("" ::"v"(r.w[k][h].x), "v"(r.w[k][h].y), "v"(r.w[k][h].z),
                         "v"(r.w[k][h].w));
    }
}

// The reduction (wave 0) over the squares the workgroup has written to LDS
// (after a barrier), then the normalized row quantized into LDS; ends at a
// workgroup barrier.
template <int KP, int T>
__device__ __forceinline__ void norm_row_to_lds(const NormRow<KP>& r, int nb, float eps,
                                                uint32_t* smem) {
    float* s_sq = reinterpret_cast<float*>(smem);
    uint32_t* s_q = smem + gemv_norm_q_offset(nb);
    float* s_d = reinterpret_cast<float*>(s_q + nb * 8);
    int* s_sum = reinterpret_cast<int*>(s_d + nb);
    float* s_small = reinterpret_cast<float*>(s_sum + nb);
    const int n = 32 * nb;
    norm_scale<true, T>(s_sq, norm_sq_stride(n), n / 4, n, s_small + 4, eps, s_small,
                        s_small + 8);
    __syncthreads();
    const float scale = s_small[8];
    const int part = threadIdx.x & 3;
#pragma unroll
    for (int k = 0; k < KP; ++k) {
        const int blk = (threadIdx.x >> 2) + 64 * k;
        if (blk < nb) {  // uniform over the quad
            float4 f0, f1;
            norm_row_values<KP, true>(r, k, scale, &f0, &f1);
            uint2 q;
            uint16_t dbits;
            int sum;
            quantize_q8_quad(f0, f1, &q, &dbits, &sum);
            *reinterpret_cast<uint2*>(s_q + blk * 8 + 2 * part) = q;
            if (part == 0) {
                s_d[blk] = h2f(dbits);
                s_sum[blk] = sum;
            }
        }
    }
    __syncthreads();
}

// Activation block b of a chunk: from the prefetched registers, or from the
// workgroup's quantized row in LDS.
struct ActBlock {
    uint32_t a[8];
    float d;
    int s;
};
__device__ __forceinline__ ActBlock act_lds(const uint32_t* smem, int nb, int b) {
    const uint32_t* s_q = smem + gemv_norm_q_offset(nb);
    const uint4 a0 = *reinterpret_cast<const uint4*>(s_q + b * 8);
    const uint4 a1 = *reinterpret_cast<const uint4*>(s_q + b * 8 + 4);
    return ActBlock{{a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w},
                    reinterpret_cast<const float*>(s_q + nb * 8)[b],
                    reinterpret_cast<const int*>(s_q + nb * 9)[b]};
}

template <bool NORM, int NBL>
__global__ __launch_bounds__(256) void gemv_q8in_kernel(GemvQ8Params p) {
#pragma clang fp contract(off)
    __shared__ __align__(16) float s_t[4][kGemvRowsPerWave][kTermStride];
    extern __shared__ __align__(16) uint32_t smem[];  // NORM: gemv_norm_lds_bytes(nb)
    const int nb = p.nb;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    int tile = blockIdx.x, m = 0;
    while (m < p.nmat - 1 && tile >= p.tiles[m]) {
        tile -= p.tiles[m];
        ++m;
    }
    const QMat M = pick(p.m, m);
    const int rw = tile * kGemvRows + wave * kGemvRowsPerWave;

    // (NORM) the row, its squares and its norm weights first; then waves
    // 1-3 issue their first weight chunks while wave 0 runs the reduction,
    // and wave 0 issues its own after it: a wave stalls issuing loads while
    // the memory pipeline is full, which would hold up the reduction
    NormRow<NBL> nr;
    if constexpr (NORM) {
        norm_row_load<NBL, true>(nr, p.a.x, p.a.w, nb);
        norm_row_squares(nr, nb, reinterpret_cast<float*>(smem));
        norm_row_wait_w(nr, nb);
        __syncthreads();
    }
    __builtin_amdgcn_sched_barrier(0);
    uint4 a0[NBL], a1[NBL];
    float da[NBL];
    int as[NBL];
    uint4 wq[NBL][kGemvRowsPerWave];
    uint16_t wd[NBL][kGemvRowsPerWave];
#define SLM_GEMV_ISSUE(j)                                                                    \
    do {                                                                                     \
        const int b_ = min(kChunk * (j) + lane, nb - 1);                                     \
        if constexpr (!NORM) {                                                               \
            a0[j] = *reinterpret_cast<const uint4*>(p.a.aq + (long)b_ * 8);                  \
            a1[j] = *reinterpret_cast<const uint4*>(p.a.aq + (long)b_ * 8 + 4);              \
            da[j] = p.a.ad[b_];                                                              \
            as[j] = p.a.as[b_];                                                              \
        }                                                                                    \
        _Pragma("unroll") for (int rr = 0; rr < kGemvRowsPerWave; ++rr) {                    \
            const int r_ = min(rw + rr, M.rows - 1);                                         \
            wq[j][rr] = ldq_stream(M.qs + ((long)r_ * nb + b_) * 16);                        \
            wd[j][rr] = __builtin_nontemporal_load(M.d + (long)r_ * M.d_stride + b_);        \
        }                                                                                    \
    } while (0)
    if (!NORM || wave != 0) {
#pragma unroll
        for (int j = 0; j < (kPrefetch < NBL ? kPrefetch : NBL); ++j) SLM_GEMV_ISSUE(j);
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (NORM) {
        norm_row_to_lds<NBL, 32>(nr, nb, p.a.eps, smem);
        if (wave == 0) {
#pragma unroll
            for (int j = 0; j < (kPrefetch < NBL ? kPrefetch : NBL); ++j) SLM_GEMV_ISSUE(j);
        }
    }

    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < NBL; ++j) {  // NBL = ceil(nb / kChunk)
        if (j + kPrefetch < NBL) SLM_GEMV_ISSUE(j + kPrefetch);
        __builtin_amdgcn_sched_barrier(0);
        const int b0 = kChunk * j;
        if (b0 + lane < nb) {
            ActBlock ab;
            if constexpr (NORM) {
                ab = act_lds(smem, nb, b0 + lane);
            } else {
                ab = ActBlock{{a0[j].x, a0[j].y, a0[j].z, a0[j].w,
                               a1[j].x, a1[j].y, a1[j].z, a1[j].w}, da[j], as[j]};
            }
#pragma unroll
            for (int rr = 0; rr < kGemvRowsPerWave; ++rr) {
                const int isum = block_dot(wq[j][rr], ab.a, ab.s);
                s_t[wave][rr][lane] = (float)isum * (h2f(wd[j][rr]) * ab.d);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (lane < kGemvRowsPerWave) acc = ordered_add(acc, &s_t[wave][lane][0], min(kChunk, nb - b0));
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
#undef SLM_GEMV_ISSUE

    if (lane < kGemvRowsPerWave) {
        const int r = rw + lane;
        if (r < M.rows) {
            // the residual_add JIT kernel, out[i] = a[i] + b[i] (graph.rs:157-164)
            if (M.res) acc = M.res[r] + acc;
            M.out[r] = acc;
        }
    }
    if (p.am) {  // uniform: the first maximum of the workgroup's rows, NaN skipped
        __shared__ float s_av[4];
        __shared__ int s_ai[4];
        float v = acc;
        int i = rw + lane;
        if (lane >= kGemvRowsPerWave || i >= M.rows || v != v) i = -1;
#pragma unroll
        for (int off = 1; off < kGemvRowsPerWave; off <<= 1) {
            const float v2 = __shfl_xor(v, off);
            const int i2 = __shfl_xor(i, off);
            argmax_merge(v, i, v2, i2);
        }
        if (lane == 0) {
            s_av[wave] = v;
            s_ai[wave] = i;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            for (int w = 1; w < 4; ++w) argmax_merge(v, i, s_av[w], s_ai[w]);
            p.am[blockIdx.x] = ArgmaxPart{v, i};
        }
    }
}

// ---- gate and up of one token, SwiGLU fused ----
//
// FuseGraph::swiglu (graph.rs:131-139) reads the gate and up rows of the same
// hidden index, so a workgroup takes 32 hidden rows of both matrices (wave w:
// rows 8w..8w+7 of each, 16 row streams) and, once its ordered sums are done,
// one quad forms act = silu(gate) * up for the 32 rows and quantizes them as
// the one Q8_0 block the down projection reads (quantize_row_q8_0 of act).
// Gate, up and act carry the same bits as the separate kernels give.  The
// activations come as in gemv_q8in_kernel: quantized, or (NORM) the FFN
// RMSNorm's input row, normalized by the workgroup.

constexpr int kSwRowsPerWave = 8;             // hidden rows per wave (of each matrix)
constexpr int kSwRows = 4 * kSwRowsPerWave;   // hidden rows per workgroup: one Q8_0 block

struct GemvSwigluParams {
    QMat gate, up;       // [hidden][nb]; out/res unused
    GemvAct a;
    int nb;
    float* act;          // [hidden] f32, or nullptr
    Q8Out q8;            // act as Q8_0 blocks (one row of hidden / 32 blocks)
};

template <bool NORM, int NBL>
__global__ __launch_bounds__(256) void gemv_q8in_swiglu_kernel(GemvSwigluParams p) {
#pragma clang fp contract(off)
    constexpr int R = 2 * kSwRowsPerWave;  // row streams per wave: gate rows, then up rows
    // chunks in flight ahead of the sums.  Normalizing, the reduction runs
    // while they stream in: rows of up to two chunks have both in flight
    // (with the reduction's 16-term buffers this fits the 256 registers of
    // two waves per SIMD, so all workgroups of a 14336-row FFN are
    // resident); longer rows keep one ahead.
    constexpr int PF = NORM && NBL > 2 ? 1 : kPrefetch;
    __shared__ __align__(16) float s_t[4][R][kTermStride];
    __shared__ float s_g[kSwRows], s_u[kSwRows];
    extern __shared__ __align__(16) uint32_t smem[];  // NORM: gemv_norm_lds_bytes(nb)
    const int nb = p.nb;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int h0 = blockIdx.x * kSwRows;             // the workgroup's block of hidden rows
    const int hw = h0 + wave * kSwRowsPerWave;       // this wave's first row

    NormRow<NBL> nr;  // (NORM) the row first, the weights around the reduction, as in
    if constexpr (NORM) {  // gemv_q8in_kernel
        norm_row_load<NBL, true>(nr, p.a.x, p.a.w, nb);
        norm_row_squares(nr, nb, reinterpret_cast<float*>(smem));
        norm_row_wait_w(nr, nb);
        __syncthreads();
    }
    __builtin_amdgcn_sched_barrier(0);
    uint4 a0[NBL], a1[NBL];
    float da[NBL];
    int as[NBL];
    uint4 wq[NBL][R];
    uint16_t wd[NBL][R];
#define SLM_SW_ISSUE(j)                                                                      \
    do {                                                                                     \
        const int b_ = min(kChunk * (j) + lane, nb - 1);                                     \
        if constexpr (!NORM) {                                                               \
            a0[j] = *reinterpret_cast<const uint4*>(p.a.aq + (long)b_ * 8);                  \
            a1[j] = *reinterpret_cast<const uint4*>(p.a.aq + (long)b_ * 8 + 4);              \
            da[j] = p.a.ad[b_];                                                              \
            as[j] = p.a.as[b_];                                                              \
        }                                                                                    \
        _Pragma("unroll") for (int rr = 0; rr < R; ++rr) {                                   \
            const QMat& M_ = rr < kSwRowsPerWave ? p.gate : p.up;                            \
            const long r_ = hw + (rr % kSwRowsPerWave);                                      \
            wq[j][rr] = ldq_stream(M_.qs + (r_ * nb + b_) * 16);                             \
            wd[j][rr] = __builtin_nontemporal_load(M_.d + r_ * M_.d_stride + b_);            \
        }                                                                                    \
    } while (0)
    if (!NORM || wave != 0) {
#pragma unroll
        for (int j = 0; j < (PF < NBL ? PF : NBL); ++j) SLM_SW_ISSUE(j);
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (NORM) {
        norm_row_to_lds<NBL, 16>(nr, nb, p.a.eps, smem);
        if (wave == 0) {
#pragma unroll
            for (int j = 0; j < (PF < NBL ? PF : NBL); ++j) SLM_SW_ISSUE(j);
        }
    }

    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < NBL; ++j) {  // NBL = ceil(nb / kChunk)
        if (j + PF < NBL) SLM_SW_ISSUE(j + PF);
        __builtin_amdgcn_sched_barrier(0);
        const int b0 = kChunk * j;
        if (b0 + lane < nb) {
            ActBlock ab;
            if constexpr (NORM) {
                ab = act_lds(smem, nb, b0 + lane);
            } else {
                ab = ActBlock{{a0[j].x, a0[j].y, a0[j].z, a0[j].w,
                               a1[j].x, a1[j].y, a1[j].z, a1[j].w}, da[j], as[j]};
            }
#pragma unroll
            for (int rr = 0; rr < R; ++rr) {
                const int isum = block_dot(wq[j][rr], ab.a, ab.s);
                s_t[wave][rr][lane] = (float)isum * (h2f(wd[j][rr]) * ab.d);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (lane < R) acc = ordered_add(acc, &s_t[wave][lane][0], min(kChunk, nb - b0));
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
#undef SLM_SW_ISSUE

    if (lane < kSwRowsPerWave) s_g[wave * kSwRowsPerWave + lane] = acc;
    else if (lane < R) s_u[wave * kSwRowsPerWave + lane - kSwRowsPerWave] = acc;
    __syncthreads();
    if (threadIdx.x < 4) {  // one quad: elements 8p..8p+7 of the block
        const int part = threadIdx.x;
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = jit_silu(s_g[8 * part + k]) * s_u[8 * part + k];
        const float4 f0 = make_float4(v[0], v[1], v[2], v[3]);
        const float4 f1 = make_float4(v[4], v[5], v[6], v[7]);
        if (p.act) {
            *reinterpret_cast<float4*>(p.act + h0 + 8 * part) = f0;
            *reinterpret_cast<float4*>(p.act + h0 + 8 * part + 4) = f1;
        }
        store_q8_quad(p.q8, 0, blockIdx.x, part, f0, f1);
    }
}

// ---- MFMA GEMM: batches of 5 or more tokens ----
//
// Workgroup tile 64 rows x 64 tokens, four waves of 32 x 32 (2 x 2 tiles of
// v_mfma_i32_16x16x32_i8, one Q-block of K = 32 per instruction).  Lane l
// feeds A[l%16][8*(l/16)..+7] = weights 8g..8g+7 of row l%16 (g = l/16) and
// B[8g..+7][l%16] = the same eight activations of token l%16, and holds
// D[4g+j][l%16].  Per block each element gets acc = acc + float(D) * (dw*da).
// The kernel is bound by that f32 epilogue (VALU), so everything else that
// costs VALU is done once per workgroup at staging: the nibbles are widened
// to i8 weights (in weight order, so a fragment is one 8-byte read) and the
// weight scales to f32.

struct GemmParams {
    QMat m[3];
    int nmat;
    int tiles[3];          // row tiles of the workgroup shape per matrix
    const uint32_t* aq;    // [batch][nb][8]
    const float* ad;       // [batch][d_stride]
    int nb;
    int d_stride;          // nb rounded up to 8 (weights and activations alike)
    int batch;
};

constexpr int kScaleChunk = 8;  // blocks whose scales one 128-bit load covers

// nibbles 0..15 -> weight - 8 as i8, four per dword
__device__ __forceinline__ uint32_t nib_to_i8(uint32_t x) {
    return (x + 0x78787878u) ^ 0x80808080u;
}

// LDS stage of the GEMM: kScaleChunk blocks of the workgroup's RT weight rows
// (widened to i8) and TT tokens.  Row strides are padded to 68 dwords so that
// the 8-byte fragment reads of a half-wave (16 rows or tokens x 2 lane
// groups) hit 64 different banks; scales are stored block-major so a lane's
// four rows are one 16-byte read.
constexpr int kAStride = 68;  // dwords per weight row: 8 blocks x 32 i8 + pad
constexpr int kBStride = 68;  // dwords per token: 8 blocks x 32 B + pad
template <int RT, int TT>
struct GemmStage {
    uint32_t a[RT * kAStride];
    uint32_t b[TT * kBStride];
    float dw[kScaleChunk][RT];
    float da[kScaleChunk][TT];
};

// Workgroup shapes: WRW x WTW waves, each 32 rows x 16*NTS tokens.  64 x 64
// (2 x 2 waves of 32 x 32), or 128 x 128 (4 x 2 waves of 32 x 64) for
// products with enough tiles to fill the CUs (launch_q4_gemm), where each
// lane's 32 outputs share the block's
// fragment and scale reads twice as widely (the loop's VALU cost per output
// element and block falls from ~5.6 to ~4.9 ops, against the epilogue's 4).
template <int WRW, int WTW, int NTS>
struct GemmShape {
    static constexpr int NW = WRW * WTW;
    static constexpr int NT = 64 * NW;
    static constexpr int RT = 32 * WRW;       // rows per workgroup
    static constexpr int TT = 16 * NTS * WTW;  // tokens per workgroup
    static_assert(RT == NT / 4 && TT == NT / 4, "one row and one token per thread quad");
};

template <int WRW, int WTW, int NTS>
__global__ __launch_bounds__(64 * WRW * WTW) void gemm_q4_mfma_kernel(GemmParams p) {
#pragma clang fp contract(off)
    using Sh = GemmShape<WRW, WTW, NTS>;
    constexpr int RT = Sh::RT, TT = Sh::TT;
    __shared__ __align__(16) GemmStage<RT, TT> st[2];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int lr = lane & 15;
    const int g = lane >> 4;

    // workgroup -> (matrix, row tile, token tile); token tiles vary fastest
    const int n_tt = (p.batch + TT - 1) / TT;
    int rt = blockIdx.x / n_tt;
    const int tt = blockIdx.x - rt * n_tt;
    int m = 0;
    while (m < p.nmat - 1 && rt >= p.tiles[m]) {
        rt -= p.tiles[m];
        ++m;
    }
    const QMat M = m == 0 ? p.m[0] : (m == 1 ? p.m[1] : p.m[2]);
    const int nb = p.nb;
    const int ds = p.d_stride;
    const int wr0 = rt * RT;  // workgroup's first row / token
    const int wt0 = tt * TT;

    // Stage loads, all 16 bytes wide and coalesced, addresses clamped into
    // the buffers (rows / tokens / blocks past the end are never used):
    //   nibbles: thread -> (row tid/4, blocks 2*(tid%4), +1)
    //   activations: thread -> (token tid/4, blocks 2*(tid%4), +1)
    //   weight scales: threads 0..RT-1 -> row; activation scales: the next
    //   2*TT threads, half a token's eight each.
    const int lrow = tid >> 2, lsub = tid & 3;
    const uint8_t* asrc = M.qs + (long)min(wr0 + lrow, M.rows - 1) * nb * 16;
    const uint32_t* bsrc = p.aq + (long)min(wt0 + lrow, p.batch - 1) * nb * 8;
    const uint16_t* dwsrc = M.d + (long)min(wr0 + min(tid, RT - 1), M.rows - 1) * ds;
    const int sidx = min(max(tid - RT, 0), 2 * TT - 1);
    const float* dasrc = p.ad + (long)min(wt0 + (sidx >> 1), p.batch - 1) * ds + 4 * (sidx & 1);
    uint4 ra0, ra1, rb0, rb1, rb2, rb3, rs;
#define SLM_GEMM_LOAD_STAGE(b0)                                                          \
    do {                                                                                 \
        const int blk0 = min((b0) + 2 * lsub, nb - 1);                                   \
        const int blk1 = min((b0) + 2 * lsub + 1, nb - 1);                               \
        ra0 = *reinterpret_cast<const uint4*>(asrc + (long)blk0 * 16);                   \
        ra1 = *reinterpret_cast<const uint4*>(asrc + (long)blk1 * 16);                   \
        rb0 = *reinterpret_cast<const uint4*>(bsrc + (long)blk0 * 8);                    \
        rb1 = *reinterpret_cast<const uint4*>(bsrc + (long)blk0 * 8 + 4);                \
        rb2 = *reinterpret_cast<const uint4*>(bsrc + (long)blk1 * 8);                    \
        rb3 = *reinterpret_cast<const uint4*>(bsrc + (long)blk1 * 8 + 4);                \
        if (tid < RT)                                                                    \
            rs = *reinterpret_cast<const uint4*>(dwsrc + (b0));                          \
        else if (tid < RT + 2 * TT)                                                      \
            rs = *reinterpret_cast<const uint4*>(dasrc + (b0));                          \
    } while (0)
    // a block's 16 nibble bytes as its 32 i8 weights in order: byte k holds
    // weight k (low nibble) and weight k + 16 (high nibble)
    auto widen = [](const uint4 q, uint4* lo, uint4* hi) {
        *lo = make_uint4(nib_to_i8(q.x & 0x0F0F0F0Fu), nib_to_i8(q.y & 0x0F0F0F0Fu),
                         nib_to_i8(q.z & 0x0F0F0F0Fu), nib_to_i8(q.w & 0x0F0F0F0Fu));
        *hi = make_uint4(nib_to_i8((q.x >> 4) & 0x0F0F0F0Fu), nib_to_i8((q.y >> 4) & 0x0F0F0F0Fu),
                         nib_to_i8((q.z >> 4) & 0x0F0F0F0Fu), nib_to_i8((q.w >> 4) & 0x0F0F0F0Fu));
    };
#define SLM_GEMM_STORE_STAGE(S)                                                           \
    do {                                                                                  \
        const int kb0 = 2 * lsub;                                                         \
        uint4 w0_, w1_;                                                                   \
        widen(ra0, &w0_, &w1_);                                                           \
        *reinterpret_cast<uint4*>(&(S).a[lrow * kAStride + kb0 * 8]) = w0_;               \
        *reinterpret_cast<uint4*>(&(S).a[lrow * kAStride + kb0 * 8 + 4]) = w1_;           \
        widen(ra1, &w0_, &w1_);                                                           \
        *reinterpret_cast<uint4*>(&(S).a[lrow * kAStride + kb0 * 8 + 8]) = w0_;           \
        *reinterpret_cast<uint4*>(&(S).a[lrow * kAStride + kb0 * 8 + 12]) = w1_;          \
        *reinterpret_cast<uint4*>(&(S).b[lrow * kBStride + kb0 * 8]) = rb0;               \
        *reinterpret_cast<uint4*>(&(S).b[lrow * kBStride + kb0 * 8 + 4]) = rb1;           \
        *reinterpret_cast<uint4*>(&(S).b[lrow * kBStride + kb0 * 8 + 8]) = rb2;           \
        *reinterpret_cast<uint4*>(&(S).b[lrow * kBStride + kb0 * 8 + 12]) = rb3;          \
        if (tid < RT) {                                                                   \
            (S).dw[0][tid] = h2f((uint16_t)(rs.x & 0xFFFF));                              \
            (S).dw[1][tid] = h2f((uint16_t)(rs.x >> 16));                                 \
            (S).dw[2][tid] = h2f((uint16_t)(rs.y & 0xFFFF));                              \
            (S).dw[3][tid] = h2f((uint16_t)(rs.y >> 16));                                 \
            (S).dw[4][tid] = h2f((uint16_t)(rs.z & 0xFFFF));                              \
            (S).dw[5][tid] = h2f((uint16_t)(rs.z >> 16));                                 \
            (S).dw[6][tid] = h2f((uint16_t)(rs.w & 0xFFFF));                              \
            (S).dw[7][tid] = h2f((uint16_t)(rs.w >> 16));                                 \
        } else if (tid < RT + 2 * TT) {                                                   \
            const int t_ = (tid - RT) >> 1, h_ = 4 * ((tid - RT) & 1);                    \
            (S).da[h_ + 0][t_] = __uint_as_float(rs.x);                                   \
            (S).da[h_ + 1][t_] = __uint_as_float(rs.y);                                   \
            (S).da[h_ + 2][t_] = __uint_as_float(rs.z);                                   \
            (S).da[h_ + 3][t_] = __uint_as_float(rs.w);                                   \
        }                                                                                 \
    } while (0)

    // this wave's 32 rows x 16*NTS tokens
    const int qr = (wave % WRW) * 32, qt = (wave / WRW) * (16 * NTS);

    float acc[2][NTS][4];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < NTS; ++b)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[a][b][j] = 0.0f;

    SLM_GEMM_LOAD_STAGE(0);
    SLM_GEMM_STORE_STAGE(st[0]);
    const int n_stages = (nb + kScaleChunk - 1) / kScaleChunk;
    for (int sg = 0; sg < n_stages; ++sg) {
        __syncthreads();  // stage sg is in st[sg & 1]; st[(sg+1) & 1] is free
        if (sg + 1 < n_stages) SLM_GEMM_LOAD_STAGE((sg + 1) * kScaleChunk);
        const GemmStage<RT, TT>& S = st[sg & 1];
        const int b0 = sg * kScaleChunk;
#pragma unroll
        for (int kb = 0; kb < kScaleChunk; ++kb) {
            if (b0 + kb >= nb) break;  // uniform
            long af[2], bf[NTS];
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                const uint2 w = *reinterpret_cast<const uint2*>(
                    &S.a[(qr + 16 * s + lr) * kAStride + kb * 8 + 2 * g]);
                af[s] = (long)(((uint64_t)w.y << 32) | w.x);
            }
#pragma unroll
            for (int s = 0; s < NTS; ++s) {
                const uint2 x = *reinterpret_cast<const uint2*>(
                    &S.b[(qt + 16 * s + lr) * kBStride + kb * 8 + 2 * g]);
                bf[s] = (long)(((uint64_t)x.y << 32) | x.x);
            }
            v4i d[2][NTS];
#pragma unroll
            for (int rs2 = 0; rs2 < 2; ++rs2)
#pragma unroll
                for (int ts = 0; ts < NTS; ++ts)
                    d[rs2][ts] = __builtin_amdgcn_mfma_i32_16x16x32_i8(af[rs2], bf[ts],
                                                                       v4i{0, 0, 0, 0}, 0, 0, 0);
            // the scale products stay on the VALU: on the matrix cores (an
            // f16 or f32 MFMA whose K = 0 slice holds the two scales, exact)
            // the epilogue waits for them and the kernel ran slower
            float dw[2][4], da[NTS];
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                const float4 h = *reinterpret_cast<const float4*>(&S.dw[kb][qr + 16 * s + 4 * g]);
                dw[s][0] = h.x;
                dw[s][1] = h.y;
                dw[s][2] = h.z;
                dw[s][3] = h.w;
            }
#pragma unroll
            for (int s = 0; s < NTS; ++s) da[s] = S.da[kb][qt + 16 * s + lr];
#pragma unroll
            for (int rs2 = 0; rs2 < 2; ++rs2)
#pragma unroll
                for (int ts = 0; ts < NTS; ++ts)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const float sc = dw[rs2][j] * da[ts];
                        acc[rs2][ts][j] = acc[rs2][ts][j] + (float)d[rs2][ts][j] * sc;
                    }
        }
        if (sg + 1 < n_stages) SLM_GEMM_STORE_STAGE(st[(sg + 1) & 1]);
    }

    // Rows r0..r0+3 of token t (r0 a multiple of 4) are contiguous in out and
    // res: with whole 4-row groups and 16-byte aligned rows they move as one
    // 128-bit access, and every residual load (at a clamped, in-bounds
    // address) is issued before the first add, so the epilogue costs one
    // memory round trip rather than one per element.
    const bool vec = (M.rows & 3) == 0 && (M.out_stride & 3) == 0 &&
                     ((reinterpret_cast<uintptr_t>(M.out) | reinterpret_cast<uintptr_t>(M.res)) &
                      15) == 0;
    if (vec) {
        float4 rv[2][NTS];
        if (M.res) {
#pragma unroll
            for (int rs2 = 0; rs2 < 2; ++rs2)
#pragma unroll
                for (int ts = 0; ts < NTS; ++ts) {
                    const int t = min(wt0 + qt + 16 * ts + lr, p.batch - 1);
                    const int r0 = min(wr0 + qr + 16 * rs2 + 4 * g, M.rows - 4);
                    rv[rs2][ts] = ld4(M.res + (long)t * M.out_stride + r0);
                }
        }
#pragma unroll
        for (int rs2 = 0; rs2 < 2; ++rs2)
#pragma unroll
            for (int ts = 0; ts < NTS; ++ts) {
                const int t = wt0 + qt + 16 * ts + lr;
                const int r0 = wr0 + qr + 16 * rs2 + 4 * g;
                if (t >= p.batch || r0 >= M.rows) continue;
                float4 y = make_float4(acc[rs2][ts][0], acc[rs2][ts][1], acc[rs2][ts][2],
                                       acc[rs2][ts][3]);
                if (M.res) {
                    y.x = rv[rs2][ts].x + y.x;
                    y.y = rv[rs2][ts].y + y.y;
                    y.z = rv[rs2][ts].z + y.z;
                    y.w = rv[rs2][ts].w + y.w;
                }
                *reinterpret_cast<float4*>(M.out + (long)t * M.out_stride + r0) = y;
            }
        return;
    }
#pragma unroll
    for (int rs2 = 0; rs2 < 2; ++rs2)
#pragma unroll
        for (int ts = 0; ts < NTS; ++ts) {
            const int t = wt0 + qt + 16 * ts + lr;
            if (t >= p.batch) continue;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int r = wr0 + qr + 16 * rs2 + 4 * g + j;
                if (r >= M.rows) continue;
                const long o = (long)t * M.out_stride + r;
                M.out[o] = M.res ? M.res[o] + acc[rs2][ts][j] : acc[rs2][ts][j];
            }
        }
}
#undef SLM_GEMM_LOAD_STAGE
#undef SLM_GEMM_STORE_STAGE

size_t gemv_lds_bytes(int nt, int nb) {
    return ((size_t)gemv_terms_offset(nt, nb) + (size_t)nt * kGemvRows * kTermStride) * 4;
}

template <int NT, int NBL>
hipError_t launch_gemv_t(const GemvParams& p, int grid, hipStream_t st) {
    if constexpr (NT > 1 && NBL > 4) {
        return hipErrorInvalidValue;  // batches above 1 take rows of at most 256 blocks
    } else {
        const size_t lds = gemv_lds_bytes(NT, p.nb);
        if (lds > 64 * 1024) {
            // above the default dynamic-LDS limit
            const hipError_t e = hipFuncSetAttribute(
                reinterpret_cast<const void*>(gemv_q4_kernel<NT, NBL>),
                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            if (e != hipSuccess) return e;
        }
        hipLaunchKernelGGL((gemv_q4_kernel<NT, NBL>), dim3(grid), dim3(256), lds, st, p);
        return hipGetLastError();
    }
}

template <int NT>
hipError_t launch_gemv_nt(const GemvParams& p, int grid, hipStream_t st) {
    const int nbl = (p.nb + 63) / 64;
    switch (nbl) {
        case 1: return launch_gemv_t<NT, 1>(p, grid, st);
        case 2: return launch_gemv_t<NT, 2>(p, grid, st);
        case 3: return launch_gemv_t<NT, 3>(p, grid, st);
        case 4: return launch_gemv_t<NT, 4>(p, grid, st);
        case 5: return launch_gemv_t<NT, 5>(p, grid, st);
        case 6: return launch_gemv_t<NT, 6>(p, grid, st);
        case 7: return launch_gemv_t<NT, 7>(p, grid, st);
        case 8: return launch_gemv_t<NT, 8>(p, grid, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

int q4_max_cols() { return 64 * 8 * 32; }

hipError_t launch_quantize_q8_aos(const float* x, long nblk, uint8_t* out, hipStream_t st) {
    if (nblk <= 0) return hipSuccess;
    hipLaunchKernelGGL(quantize_q8_aos_kernel, dim3((unsigned)((nblk + 63) / 64)), dim3(256),
                       0, st, x, nblk, out);
    return hipGetLastError();
}

int q4_scale_stride(int nb) { return (nb + kScaleChunk - 1) / kScaleChunk * kScaleChunk; }

hipError_t launch_quantize_q8_soa(const float* x, long ntok, int nb, uint32_t* q, float* d,
                                  int* sums, hipStream_t st) {
    const long nblk = ntok * nb;
    if (nblk <= 0) return hipSuccess;
    hipLaunchKernelGGL(quantize_q8_soa_kernel, dim3((unsigned)((nblk + 63) / 64)), dim3(256),
                       0, st, x, nblk, nb, q4_scale_stride(nb), q, d, sums);
    return hipGetLastError();
}

bool q4_gemv_takes(int nb, int batch) {
    return batch >= 1 && (batch == 1 || (batch <= 4 && nb <= 256));
}

hipError_t launch_q4_gemv(const Q4Job* jobs, int njobs, const float* x, int nb, int batch,
                          hipStream_t st) {
    if (njobs < 1 || njobs > 3 || !q4_gemv_takes(nb, batch)) return hipErrorInvalidValue;
    GemvParams p{};
    int grid = 0;
    for (int i = 0; i < njobs; ++i) {
        p.m[i] = QMat{jobs[i].qs, jobs[i].d, jobs[i].out, jobs[i].res, jobs[i].rows,
                      jobs[i].out_stride, q4_scale_stride(nb)};
        p.tiles[i] = (jobs[i].rows + kGemvRows - 1) / kGemvRows;
        grid += p.tiles[i];
    }
    p.nmat = njobs;
    p.x = x;
    p.nb = nb;
    p.batch = batch;
    return batch == 1 ? launch_gemv_nt<1>(p, grid, st) : launch_gemv_nt<4>(p, grid, st);
}

namespace {

template <bool NORM, int NBL>
hipError_t launch_gemv_q8_t(const GemvQ8Params& p, int grid, hipStream_t st) {
    const size_t lds = NORM ? gemv_norm_lds_bytes(p.nb) : 0;
    if (lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute(
            reinterpret_cast<const void*>(gemv_q8in_kernel<NORM, NBL>),
            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL((gemv_q8in_kernel<NORM, NBL>), dim3(grid), dim3(256), lds, st, p);
    return hipGetLastError();
}

template <bool NORM>
hipError_t launch_gemv_q8_any(const Q4Job* jobs, int njobs, const GemvAct& a, int nb,
                              hipStream_t st) {
    if (njobs < 1 || njobs > 3 || nb < 1 || nb > 8 * kChunk) return hipErrorInvalidValue;
    GemvQ8Params p{};
    int grid = 0;
    for (int i = 0; i < njobs; ++i) {
        p.m[i] = QMat{jobs[i].qs, jobs[i].d, jobs[i].out, jobs[i].res, jobs[i].rows,
                      jobs[i].out_stride, q4_scale_stride(nb)};
        p.tiles[i] = (jobs[i].rows + kGemvRows - 1) / kGemvRows;
        grid += p.tiles[i];
    }
    p.nmat = njobs;
    p.a = a;
    p.nb = nb;
    switch ((nb + kChunk - 1) / kChunk) {
        case 1: return launch_gemv_q8_t<NORM, 1>(p, grid, st);
        case 2: return launch_gemv_q8_t<NORM, 2>(p, grid, st);
        case 3: return launch_gemv_q8_t<NORM, 3>(p, grid, st);
        case 4: return launch_gemv_q8_t<NORM, 4>(p, grid, st);
        case 5: return launch_gemv_q8_t<NORM, 5>(p, grid, st);
        case 6: return launch_gemv_q8_t<NORM, 6>(p, grid, st);
        case 7: return launch_gemv_q8_t<NORM, 7>(p, grid, st);
        case 8: return launch_gemv_q8_t<NORM, 8>(p, grid, st);
        default: return hipErrorInvalidValue;
    }
}

template <bool NORM, int NBL>
hipError_t launch_swiglu_t(const GemvSwigluParams& p, int grid, hipStream_t st) {
    const size_t lds = NORM ? gemv_norm_lds_bytes(p.nb) : 0;
    if (lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute(
            reinterpret_cast<const void*>(gemv_q8in_swiglu_kernel<NORM, NBL>),
            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL((gemv_q8in_swiglu_kernel<NORM, NBL>), dim3(grid), dim3(256), lds, st, p);
    return hipGetLastError();
}

template <bool NORM>
hipError_t launch_swiglu_any(const Q4Job& gate, const Q4Job& up, const GemvAct& a, int nb,
                             float* act, const Q8Out& q8, hipStream_t st) {
    const int hidden = gate.rows;
    if (up.rows != hidden || hidden % kSwRows || nb < 1 || nb > 8 * kChunk || !q8.q)
        return hipErrorInvalidValue;
    GemvSwigluParams p{};
    p.gate = QMat{gate.qs, gate.d, nullptr, nullptr, hidden, 0, q4_scale_stride(nb)};
    p.up = QMat{up.qs, up.d, nullptr, nullptr, hidden, 0, q4_scale_stride(nb)};
    p.a = a;
    p.nb = nb;
    p.act = act;
    p.q8 = q8;
    const int grid = hidden / kSwRows;
    switch ((nb + kChunk - 1) / kChunk) {
        case 1: return launch_swiglu_t<NORM, 1>(p, grid, st);
        case 2: return launch_swiglu_t<NORM, 2>(p, grid, st);
        case 3: return launch_swiglu_t<NORM, 3>(p, grid, st);
        case 4: return launch_swiglu_t<NORM, 4>(p, grid, st);
        case 5: return launch_swiglu_t<NORM, 5>(p, grid, st);
        case 6: return launch_swiglu_t<NORM, 6>(p, grid, st);
        case 7: return launch_swiglu_t<NORM, 7>(p, grid, st);
        case 8: return launch_swiglu_t<NORM, 8>(p, grid, st);
        default: return hipErrorInvalidValue;
    }
}

template <int WRW, int WTW, int NTS>
hipError_t launch_gemm_t(const Q4Job* jobs, int njobs, const uint32_t* aq, const float* ad,
                         int nb, int batch, hipStream_t st) {
    using Sh = GemmShape<WRW, WTW, NTS>;
    GemmParams p{};
    long tiles = 0;
    for (int i = 0; i < njobs; ++i) {
        p.m[i] = QMat{jobs[i].qs, jobs[i].d, jobs[i].out, jobs[i].res, jobs[i].rows,
                      jobs[i].out_stride, q4_scale_stride(nb)};
        p.tiles[i] = (jobs[i].rows + Sh::RT - 1) / Sh::RT;
        tiles += p.tiles[i];
    }
    p.nmat = njobs;
    p.aq = aq;
    p.ad = ad;
    p.nb = nb;
    p.d_stride = q4_scale_stride(nb);
    p.batch = batch;
    const long n_tt = (batch + Sh::TT - 1) / Sh::TT;
    if (tiles * n_tt > 0x7FFFFFFF) return hipErrorInvalidValue;
    hipLaunchKernelGGL((gemm_q4_mfma_kernel<WRW, WTW, NTS>), dim3((unsigned)(tiles * n_tt)),
                       dim3(Sh::NT), 0, st, p);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_q4_gemv_q8(const Q4Job* jobs, int njobs, const uint32_t* aq, const float* ad,
                             const int* as, int nb, hipStream_t st) {
    return launch_gemv_q8_any<false>(jobs, njobs, GemvAct{aq, ad, as, nullptr, nullptr, 0.0f},
                                     nb, st);
}

int q4_gemv_rows_per_part() { return kGemvRows; }

hipError_t launch_q4_gemv_q8_argmax(const Q4Job& job, const uint32_t* aq, const float* ad,
                                    const int* as, int nb, ArgmaxPart* parts, hipStream_t st) {
    if (!parts || job.res || nb < 1 || nb > 8 * kChunk) return hipErrorInvalidValue;
    GemvQ8Params p{};
    p.m[0] = QMat{job.qs, job.d, job.out, nullptr, job.rows, job.out_stride, q4_scale_stride(nb)};
    p.tiles[0] = (job.rows + kGemvRows - 1) / kGemvRows;
    p.nmat = 1;
    p.a = GemvAct{aq, ad, as, nullptr, nullptr, 0.0f};
    p.nb = nb;
    p.am = parts;
    switch ((nb + kChunk - 1) / kChunk) {
        case 1: return launch_gemv_q8_t<false, 1>(p, p.tiles[0], st);
        case 2: return launch_gemv_q8_t<false, 2>(p, p.tiles[0], st);
        case 3: return launch_gemv_q8_t<false, 3>(p, p.tiles[0], st);
        case 4: return launch_gemv_q8_t<false, 4>(p, p.tiles[0], st);
        case 5: return launch_gemv_q8_t<false, 5>(p, p.tiles[0], st);
        case 6: return launch_gemv_q8_t<false, 6>(p, p.tiles[0], st);
        case 7: return launch_gemv_q8_t<false, 7>(p, p.tiles[0], st);
        case 8: return launch_gemv_q8_t<false, 8>(p, p.tiles[0], st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_q4_gemv_norm(const Q4Job* jobs, int njobs, const float* x, const float* w,
                               float eps, int nb, hipStream_t st) {
    if (!x || !w) return hipErrorInvalidValue;
    return launch_gemv_q8_any<true>(jobs, njobs, GemvAct{nullptr, nullptr, nullptr, x, w, eps},
                                    nb, st);
}

hipError_t launch_q4_gemv_q8_swiglu(const Q4Job& gate, const Q4Job& up, const uint32_t* aq,
                                    const float* ad, const int* as, int nb, float* act,
                                    const Q8Out& q8, hipStream_t st) {
    return launch_swiglu_any<false>(gate, up, GemvAct{aq, ad, as, nullptr, nullptr, 0.0f}, nb,
                                    act, q8, st);
}

hipError_t launch_q4_gemv_norm_swiglu(const Q4Job& gate, const Q4Job& up, const float* x,
                                      const float* w, float eps, int nb, float* act,
                                      const Q8Out& q8, hipStream_t st) {
    if (!x || !w) return hipErrorInvalidValue;
    return launch_swiglu_any<true>(gate, up, GemvAct{nullptr, nullptr, nullptr, x, w, eps}, nb,
                                   act, q8, st);
}

namespace {

// Compute units of the current device, looked up once per device.
long device_cus() {
    static std::atomic<int> cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cached[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        cached[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

}  // namespace

// Tile choice: 128 x 128 workgroups (one per CU; 10% less VALU per output
// element and block, measured on the 4096-token Q/K/V GEMM: 0.48 against
// 0.53 ms) or 64 x 64 (two per CU).  The estimate of each is the workgroups
// a CU runs in turn times one workgroup's work; products with few big tiles
// would leave CUs idle (Wo at 512 tokens: 128 workgroups of 128 x 128 on 256
// CUs).  Tile shape does not change results (each output is one thread's
// ordered sum over blocks).
hipError_t launch_q4_gemm(const Q4Job* jobs, int njobs, const uint32_t* aq, const float* ad,
                          int nb, int batch, hipStream_t st) {
    if (njobs < 1 || njobs > 3 || batch < 1) return hipErrorInvalidValue;
    long w128 = 0, w64 = 0;
    for (int i = 0; i < njobs; ++i) {
        w128 += (long)((jobs[i].rows + 127) / 128) * ((batch + 127) / 128);
        w64 += (long)((jobs[i].rows + 63) / 64) * ((batch + 63) / 64);
    }
    const long cus = device_cus();
    const double t128 = (double)((w128 + cus - 1) / cus) * 4.0;
    const double t64 = (double)((w64 + cus - 1) / cus) * 1.1;
    return t128 < t64 ? launch_gemm_t<4, 2, 4>(jobs, njobs, aq, ad, nb, batch, st)
                      : launch_gemm_t<2, 2, 2>(jobs, njobs, aq, ad, nb, batch, st);
}

}  // namespace slm
