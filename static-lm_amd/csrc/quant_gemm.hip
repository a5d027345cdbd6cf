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
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "attn_common.h"
#include "slm_internal.h"

namespace slm {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }
__device__ __forceinline__ uint16_t f2h(float f) { return __half_as_ushort(__float2half_rn(f)); }

// One Q8_0 block from 32 floats: packed i8 (little-endian bytes), the f16
// scale bits, and the sum of the 32 quantized values.
struct Q8Block {
    uint32_t q[8];
    uint16_t dbits;
    int sum;
};

// `(x * id).round().clamp(-127.0, 127.0) as i8`: round half away from zero,
// clamp keeps NaN, the cast sends NaN to 0.
__device__ __forceinline__ int q8_value(float v) {
    float r = roundf(v);
    r = r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r);
    return r != r ? 0 : (int)r;
}

__device__ __forceinline__ Q8Block quantize_q8_block(const float* x) {
#pragma clang fp contract(off)
    float v[32];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 f = ld4(x + 4 * i);
        v[4 * i + 0] = f.x;
        v[4 * i + 1] = f.y;
        v[4 * i + 2] = f.z;
        v[4 * i + 3] = f.w;
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const float av = fabsf(v[i]);
        amax = av > amax ? av : amax;
    }
    const float d = amax / 127.0f;
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    Q8Block b;
    b.dbits = f2h(d);
    b.sum = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        uint32_t w = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int q = q8_value(v[4 * k + e] * id);
            b.sum += q;
            w |= (uint32_t)(q & 0xFF) << (8 * e);
        }
        b.q[k] = w;
    }
    return b;
}

// ---- standalone quantize_row_q8_0: 34-byte BlockQ8_0 output ----

__global__ __launch_bounds__(256) void quantize_q8_aos_kernel(const float* x, long nblk,
                                                              uint8_t* out) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblk) return;
    const Q8Block b = quantize_q8_block(x + i * 32);
    // 34-byte blocks are 2-byte aligned: 17 little-endian u16 stores
    uint16_t* o = reinterpret_cast<uint16_t*>(out + i * 34);
    o[0] = b.dbits;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        o[1 + 2 * k] = (uint16_t)(b.q[k] & 0xFFFF);
        o[2 + 2 * k] = (uint16_t)(b.q[k] >> 16);
    }
}

// ---- activations for the MFMA GEMM: q [n][nb][32] i8, d [n][nb] f32 ----

__global__ __launch_bounds__(256) void quantize_q8_soa_kernel(const float* x, long nblk,
                                                              uint32_t* q, float* d) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblk) return;
    const Q8Block b = quantize_q8_block(x + i * 32);
    uint4* o = reinterpret_cast<uint4*>(q + i * 8);
    o[0] = make_uint4(b.q[0], b.q[1], b.q[2], b.q[3]);
    o[1] = make_uint4(b.q[4], b.q[5], b.q[6], b.q[7]);
    d[i] = h2f(b.dbits);
}

// ---- GEMV: one weight row per wave, blocks lane, lane+64, ... ----

struct QMat {
    const uint8_t* qs;   // [rows][nb][16]
    const uint16_t* d;   // [rows][nb]
    float* out;          // out[tok * out_stride + row]
    int rows;
    int out_stride;
};

struct GemvParams {
    QMat m[3];
    int nmat;
    const float* x;  // [batch][nb*32]
    int nb;
    int batch;
};

constexpr int kGemvWaves = 8;
constexpr int kGemvRowsPerWave = 2;
constexpr int kGemvRows = kGemvWaves * kGemvRowsPerWave;  // rows per workgroup

// Block b's integer dot with unsigned nibbles: sum(nib_i * a_i) - 8 * sum(a).
__device__ __forceinline__ int block_dot(const uint4 w, const uint32_t* a, int asum) {
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

template <int NT, int NBL>
__global__ __launch_bounds__(64 * kGemvWaves) void gemv_q4_kernel(GemvParams p) {
#pragma clang fp contract(off)
    extern __shared__ __align__(16) uint32_t smem[];
    const int nb = p.nb;
    uint32_t* s_q = smem;                                   // [NT][nb][8]
    float* s_d = reinterpret_cast<float*>(smem + NT * nb * 8);  // [NT][nb]
    int* s_sum = reinterpret_cast<int*>(s_d + NT * nb);      // [NT][nb]

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;

    // this wave's rows (over the concatenated matrices), weight loads first
    int mi[kGemvRowsPerWave], row[kGemvRowsPerWave];
    bool act[kGemvRowsPerWave];
    uint4 wq[kGemvRowsPerWave][NBL];
    uint16_t wd[kGemvRowsPerWave][NBL];
#pragma unroll
    for (int rr = 0; rr < kGemvRowsPerWave; ++rr) {
        int r = (blockIdx.x * kGemvWaves + wave) * kGemvRowsPerWave + rr;
        int m = 0;
        while (m < p.nmat - 1 && r >= p.m[m].rows) {
            r -= p.m[m].rows;
            ++m;
        }
        mi[rr] = m;
        row[rr] = r;
        act[rr] = r < p.m[m].rows;
        const QMat& M = p.m[m];
#pragma unroll
        for (int j = 0; j < NBL; ++j) {
            const int b = lane + 64 * j;
            if (act[rr] && b < nb) {
                const long blk = (long)r * nb + b;
                wq[rr][j] = *reinterpret_cast<const uint4*>(M.qs + blk * 16);
                wd[rr][j] = M.d[blk];
            } else {
                wq[rr][j] = make_uint4(0u, 0u, 0u, 0u);
                wd[rr][j] = 0;
            }
        }
    }

    // activations of every token, quantized once per workgroup
    for (int idx = threadIdx.x; idx < p.batch * nb; idx += 64 * kGemvWaves) {
        const Q8Block b = quantize_q8_block(p.x + (long)idx * 32);
        uint4* o = reinterpret_cast<uint4*>(s_q + idx * 8);
        o[0] = make_uint4(b.q[0], b.q[1], b.q[2], b.q[3]);
        o[1] = make_uint4(b.q[4], b.q[5], b.q[6], b.q[7]);
        s_d[idx] = h2f(b.dbits);
        s_sum[idx] = b.sum;
    }
    __syncthreads();

#pragma unroll
    for (int rr = 0; rr < kGemvRowsPerWave; ++rr) {
        if (!act[rr]) continue;  // wave-uniform
        float t[NBL][NT];
#pragma unroll
        for (int j = 0; j < NBL; ++j) {
            const int b = lane + 64 * j;
            const float dw = h2f(wd[rr][j]);
#pragma unroll
            for (int tok = 0; tok < NT; ++tok) {
                t[j][tok] = 0.0f;
                if (b < nb && tok < p.batch) {
                    const int ai = tok * nb + b;
                    uint32_t a[8];
                    const uint4 a0 = *reinterpret_cast<const uint4*>(s_q + ai * 8);
                    const uint4 a1 = *reinterpret_cast<const uint4*>(s_q + ai * 8 + 4);
                    a[0] = a0.x; a[1] = a0.y; a[2] = a0.z; a[3] = a0.w;
                    a[4] = a1.x; a[5] = a1.y; a[6] = a1.z; a[7] = a1.w;
                    const int isum = block_dot(wq[rr][j], a, s_sum[ai]);
                    const float sc = dw * s_d[ai];
                    t[j][tok] = (float)isum * sc;
                }
            }
        }
        // the reference's order: one accumulator over blocks 0, 1, 2, ...
        const QMat& M = p.m[mi[rr]];
#pragma unroll
        for (int tok = 0; tok < NT; ++tok) {
            if (tok >= p.batch) break;
            float s = 0.0f;
#pragma unroll
            for (int j = 0; j < NBL; ++j) {
                const int nl = min(64, nb - 64 * j);
                const int tv = __float_as_int(t[j][tok]);
                for (int l = 0; l < nl; ++l)
                    s = s + __int_as_float(__builtin_amdgcn_readlane(tv, l));
            }
            if (lane == 0) M.out[(long)tok * M.out_stride + row[rr]] = s;
        }
    }
}

// ---- MFMA GEMM: batches of 5 or more tokens ----
//
// Workgroup tile 64 rows x 64 tokens, four waves of 32 x 32 (2 x 2 tiles of
// v_mfma_i32_16x16x32_i8, one Q-block of K = 32 per instruction).  Lane l
// feeds A[l%16][8*(l/16)..+7] = weights 8g..8g+7 of row l%16 (g = l/16: low
// nibbles of bytes 0-7 / 8-15, then high nibbles of bytes 0-7 / 8-15) and
// B[8g..+7][l%16] = the same eight activations of token l%16, and holds
// D[4g+j][l%16].  Per block each element gets acc = acc + float(D) * (dw*da).

struct GemmParams {
    QMat m[3];
    int nmat;
    int tiles[3];          // 64-row tiles per matrix
    const uint32_t* aq;    // [batch][nb][8]
    const float* ad;       // [batch][nb]
    int nb;
    int batch;
};

constexpr int kGemmTile = 64;

// nibbles 0..15 -> weight - 8 as i8, four per dword
__device__ __forceinline__ uint32_t nib_to_i8(uint32_t x) {
    return (x + 0x78787878u) ^ 0x80808080u;
}

__global__ __launch_bounds__(256) void gemm_q4_mfma_kernel(GemmParams p) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int lr = lane & 15;
    const int g = lane >> 4;

    // workgroup -> (matrix, row tile, token tile); token tiles vary fastest
    const int n_tt = (p.batch + kGemmTile - 1) / kGemmTile;
    int rt = blockIdx.x / n_tt;
    const int tt = blockIdx.x - rt * n_tt;
    int m = 0;
    while (m < p.nmat - 1 && rt >= p.tiles[m]) {
        rt -= p.tiles[m];
        ++m;
    }
    const QMat& M = p.m[m];
    const int nb = p.nb;
    const int r0 = rt * kGemmTile + (wave & 1) * 32;
    const int t0 = tt * kGemmTile + (wave >> 1) * 32;

    // rows / tokens this lane loads fragments for (clamped in bounds)
    long wrow[2], atok[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        const int r = r0 + 16 * s + lr;
        wrow[s] = r < M.rows ? r : 0;
        const int t = t0 + 16 * s + lr;
        atok[s] = t < p.batch ? t : 0;
    }
    // rows whose scales this lane needs: r0 + 16 s + 4 g + j
    long srow[2][4];
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int r = r0 + 16 * s + 4 * g + j;
            srow[s][j] = r < M.rows ? r : 0;
        }
    const int half = (g & 1) * 8;        // byte offset of this lane's 8 nibble bytes
    const int shift = (g >> 1) * 4;      // low or high nibbles

    float acc[2][2][4];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[a][b][j] = 0.0f;

    for (int b = 0; b < nb; ++b) {
        long afrag[2], bfrag[2];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const uint2 w = *reinterpret_cast<const uint2*>(M.qs + (wrow[s] * nb + b) * 16 + half);
            const uint32_t lo = nib_to_i8((w.x >> shift) & 0x0F0F0F0Fu);
            const uint32_t hi = nib_to_i8((w.y >> shift) & 0x0F0F0F0Fu);
            afrag[s] = (long)(((uint64_t)hi << 32) | lo);
            const uint2 a = *reinterpret_cast<const uint2*>(p.aq + (atok[s] * nb + b) * 8 + 2 * g);
            bfrag[s] = (long)(((uint64_t)a.y << 32) | a.x);
        }
        float dw[2][4], da[2];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
#pragma unroll
            for (int j = 0; j < 4; ++j) dw[s][j] = h2f(M.d[srow[s][j] * nb + b]);
            da[s] = p.ad[atok[s] * nb + b];
        }
        v4i d[2][2];
#pragma unroll
        for (int rs = 0; rs < 2; ++rs)
#pragma unroll
            for (int ts = 0; ts < 2; ++ts)
                d[rs][ts] = __builtin_amdgcn_mfma_i32_16x16x32_i8(afrag[rs], bfrag[ts],
                                                                  v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
        for (int rs = 0; rs < 2; ++rs)
#pragma unroll
            for (int ts = 0; ts < 2; ++ts)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float sc = dw[rs][j] * da[ts];
                    acc[rs][ts][j] = acc[rs][ts][j] + (float)d[rs][ts][j] * sc;
                }
    }

#pragma unroll
    for (int rs = 0; rs < 2; ++rs)
#pragma unroll
        for (int ts = 0; ts < 2; ++ts) {
            const int t = t0 + 16 * ts + lr;
            if (t >= p.batch) continue;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int r = r0 + 16 * rs + 4 * g + j;
                if (r < M.rows) M.out[(long)t * M.out_stride + r] = acc[rs][ts][j];
            }
        }
}

template <int NT, int NBL>
hipError_t launch_gemv_t(const GemvParams& p, int total_rows, hipStream_t st) {
    const size_t lds = (size_t)NT * p.nb * (8 * 4 + 4 + 4);
    if (lds > 64 * 1024) {
        // above the default dynamic-LDS limit (up to 80 KiB of the 160 KiB)
        const hipError_t e = hipFuncSetAttribute(
            reinterpret_cast<const void*>(gemv_q4_kernel<NT, NBL>),
            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    const int grid = (total_rows + kGemvRows - 1) / kGemvRows;
    hipLaunchKernelGGL((gemv_q4_kernel<NT, NBL>), dim3(grid), dim3(64 * kGemvWaves), lds, st, p);
    return hipGetLastError();
}

template <int NT>
hipError_t launch_gemv_nt(const GemvParams& p, int total_rows, hipStream_t st) {
    const int nbl = (p.nb + 63) / 64;
    switch (nbl) {
        case 1: return launch_gemv_t<NT, 1>(p, total_rows, st);
        case 2: return launch_gemv_t<NT, 2>(p, total_rows, st);
        case 3: case 4: return launch_gemv_t<NT, 4>(p, total_rows, st);
        case 5: case 6: case 7: case 8: return launch_gemv_t<NT, 8>(p, total_rows, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

int q4_max_cols() { return 64 * 8 * 32; }
int q4_gemv_max_batch() { return 4; }

hipError_t launch_quantize_q8_aos(const float* x, long nblk, uint8_t* out, hipStream_t st) {
    if (nblk <= 0) return hipSuccess;
    hipLaunchKernelGGL(quantize_q8_aos_kernel, dim3((unsigned)((nblk + 255) / 256)), dim3(256),
                       0, st, x, nblk, out);
    return hipGetLastError();
}

hipError_t launch_quantize_q8_soa(const float* x, long nblk, uint32_t* q, float* d,
                                  hipStream_t st) {
    if (nblk <= 0) return hipSuccess;
    hipLaunchKernelGGL(quantize_q8_soa_kernel, dim3((unsigned)((nblk + 255) / 256)), dim3(256),
                       0, st, x, nblk, q, d);
    return hipGetLastError();
}

hipError_t launch_q4_gemv(const Q4Job* jobs, int njobs, const float* x, int nb, int batch,
                          hipStream_t st) {
    if (njobs < 1 || njobs > 3 || batch < 1 || batch > q4_gemv_max_batch()) return hipErrorInvalidValue;
    GemvParams p{};
    int total = 0;
    for (int i = 0; i < njobs; ++i) {
        p.m[i] = QMat{jobs[i].qs, jobs[i].d, jobs[i].out, jobs[i].rows, jobs[i].out_stride};
        total += jobs[i].rows;
    }
    p.nmat = njobs;
    p.x = x;
    p.nb = nb;
    p.batch = batch;
    return batch == 1 ? launch_gemv_nt<1>(p, total, st) : launch_gemv_nt<4>(p, total, st);
}

hipError_t launch_q4_gemm(const Q4Job* jobs, int njobs, const uint32_t* aq, const float* ad,
                          int nb, int batch, hipStream_t st) {
    if (njobs < 1 || njobs > 3 || batch < 1) return hipErrorInvalidValue;
    GemmParams p{};
    long tiles = 0;
    for (int i = 0; i < njobs; ++i) {
        p.m[i] = QMat{jobs[i].qs, jobs[i].d, jobs[i].out, jobs[i].rows, jobs[i].out_stride};
        p.tiles[i] = (jobs[i].rows + kGemmTile - 1) / kGemmTile;
        tiles += p.tiles[i];
    }
    p.nmat = njobs;
    p.aq = aq;
    p.ad = ad;
    p.nb = nb;
    p.batch = batch;
    const long n_tt = (batch + kGemmTile - 1) / kGemmTile;
    if (tiles * n_tt > 0x7FFFFFFF) return hipErrorInvalidValue;
    hipLaunchKernelGGL(gemm_q4_mfma_kernel, dim3((unsigned)(tiles * n_tt)), dim3(256), 0, st, p);
    return hipGetLastError();
}

}  // namespace slm
