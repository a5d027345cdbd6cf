// Q8_0 quantization shared by the kernels that emit or consume it:
// quantize_row_q8_0 (blocks.rs:102-123) for one block, four lanes per block.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "attn_common.h"
#include "slm_internal.h"

namespace slm {

__device__ __forceinline__ float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }
__device__ __forceinline__ uint16_t f2h(float f) { return __half_as_ushort(__float2half_rn(f)); }

// `(x * id).round().clamp(-127.0, 127.0) as i8`: round half away from zero,
// clamp keeps NaN, the cast sends NaN to 0.
__device__ __forceinline__ int q8_value(float v) {
    float r = roundf(v);
    r = r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r);
    return r != r ? 0 : (int)r;
}

// Four consecutive lanes quantize one block: lane part p holds elements
// 8p..8p+7; returns them packed (2 dwords), with the block's f16 scale and
// the sum of its 32 quantized values in every lane of the quad.
__device__ __forceinline__ void quantize_q8_quad(const float4 f0, const float4 f1, uint2* q,
                                                 uint16_t* dbits, int* sum) {
#pragma clang fp contract(off)
    const float v[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float av = fabsf(v[i]);
        amax = av > amax ? av : amax;
    }
    float o = dpp<0xB1>(amax);  // quad_perm [1,0,3,2]
    amax = o > amax ? o : amax;
    o = dpp<0x4E>(amax);        // quad_perm [2,3,0,1]
    amax = o > amax ? o : amax;
    const float d = amax / 127.0f;
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    int s = 0;
    uint32_t w[2] = {0u, 0u};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int qv = q8_value(v[i] * id);
        s += qv;
        w[i >> 2] |= (uint32_t)(qv & 0xFF) << (8 * (i & 3));
    }
    s += __builtin_amdgcn_update_dpp(0, s, 0xB1, 0xF, 0xF, false);
    s += __builtin_amdgcn_update_dpp(0, s, 0x4E, 0xF, 0xF, false);
    *q = make_uint2(w[0], w[1]);
    *dbits = f2h(d);
    *sum = s;
}

// Quantizes block blk of row `row` from four lanes (part p: elements
// 8p..8p+7) and stores it.  All four lanes of the quad must be active.
__device__ __forceinline__ void store_q8_quad(const Q8Out& o, long row, int blk, int part,
                                              float4 f0, float4 f1) {
    uint2 qv;
    uint16_t dbits;
    int sum;
    quantize_q8_quad(f0, f1, &qv, &dbits, &sum);
    *reinterpret_cast<uint2*>(o.q + (row * o.nb + blk) * 8 + 2 * part) = qv;
    if (part == 0) {
        const long k = row * o.d_stride + blk;
        o.d[k] = h2f(dbits);
        if (o.s) o.s[k] = sum;
    }
}

// sample_argmax's order (transformer.rs:654-666) for a parallel scan: the
// larger value wins, a tie goes to the lower index; i < 0 marks "none".
__device__ __forceinline__ void argmax_merge(float& v, int& i, float v2, int i2) {
    if (i2 < 0) return;
    if (i < 0 || v2 > v || (v2 == v && i2 < i)) {
        v = v2;
        i = i2;
    }
}

}  // namespace slm
