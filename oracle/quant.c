/*
 * CPU oracle, quantized projections -- TEST INFRASTRUCTURE ONLY.
 *
 * Restates static-lm's Q4_0 / Q8_0 block formats and dot products
 * (src/quant/blocks.rs, src/quant/kernels.rs) operation for operation.
 * Built with -fno-fast-math -ffp-contract=off: every f32 product and sum is
 * rounded on its own, as Rust does; the AVX2 restatement spells its fused
 * multiply-adds out with fmaf.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "slm_oracle.h"

/* IEEE binary32 -> binary16, round to nearest even, as half::f16::from_f32
 * (half 2.7.1, the crate blocks.rs uses for block scales).  Overflow goes to
 * infinity, small values to subnormals or zero, NaN stays a quiet NaN. */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t exp = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (exp == 0xFFu) {  // inf / NaN
        return (uint16_t)(sign | 0x7C00u | (man ? (0x0200u | (man >> 13)) : 0u));
    }
    const int e = (int)exp - 127 + 15;  // rebiased exponent
    if (e >= 0x1F) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        // subnormal half (or zero): shift the significand with its hidden bit
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000u;
        const int shift = 14 - e;  // 24-bit significand -> 10-bit field
        uint32_t h = man >> shift;
        const uint32_t rem = man & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (h & 1u))) ++h;
        return (uint16_t)(sign | h);
    }
    uint32_t h = ((uint32_t)e << 10) | (man >> 13);
    const uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;  // may carry into exp: correct
    return (uint16_t)(sign | h);
}

/* binary16 -> binary32 (exact), as half::f16::to_f32. */
float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t exp = ((uint32_t)h >> 10) & 0x1Fu;
    uint32_t man = (uint32_t)h & 0x3FFu;
    uint32_t x;
    if (exp == 0) {
        if (man == 0) {
            x = sign;
        } else {  // subnormal: normalise
            int e = -1;
            do {
                ++e;
                man <<= 1;
            } while (!(man & 0x400u));
            x = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3FFu) << 13);
        }
    } else if (exp == 0x1F) {
        x = sign | 0x7F800000u | (man << 13);
    } else {
        x = sign | ((exp - 15 + 127) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* Rust's `f as i32`: NaN -> 0, saturating at the i32 range. */
static inline int32_t rust_f32_as_i32(float f) {
    if (f != f) return 0;
    if (f >= 2147483648.0f) return INT32_MAX;
    if (f <= -2147483648.0f) return INT32_MIN;
    return (int32_t)f;
}

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline void wr16(uint8_t* p, uint16_t v) {
    p[0] = (uint8_t)(v & 0xFF);
    p[1] = (uint8_t)(v >> 8);
}

/* quantize_row_q4_0 (blocks.rs:50-82). */
void orc_quantize_row_q4_0(const float* src, size_t n, uint8_t* dst) {
    for (size_t b = 0; b < n / ORC_QK; ++b) {
        const float* chunk = src + b * ORC_QK;
        uint8_t* blk = dst + b * ORC_Q4_BYTES;
        float min_val = 0.0f, max_val = 0.0f;
        for (int i = 0; i < ORC_QK; ++i) {
            const float v = chunk[i];
            if (v < min_val) min_val = v;
            if (v > max_val) max_val = v;
        }
        const float d_pos = fmaxf(-min_val / 8.0f, max_val / 7.0f);
        const float d_neg = fmaxf(max_val / 8.0f, -min_val / 7.0f);
        const float d = d_pos <= d_neg ? d_pos : -d_neg;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        wr16(blk, orc_f32_to_f16(d));
        for (int j = 0; j < ORC_QK / 2; ++j) {
            const float x0 = chunk[j] * id;
            const float x1 = chunk[j + ORC_QK / 2] * id;
            // `x.round() as i32 + 8`, then clamp(0, 15); the add wraps as in a
            // release build (Cargo.toml's release profile keeps the default
            // overflow-checks = false), so +inf -> i32::MAX + 8 -> 0
            int32_t q0 = (int32_t)((uint32_t)rust_f32_as_i32(roundf(x0)) + 8u);
            int32_t q1 = (int32_t)((uint32_t)rust_f32_as_i32(roundf(x1)) + 8u);
            q0 = q0 < 0 ? 0 : (q0 > 15 ? 15 : q0);
            q1 = q1 < 0 ? 0 : (q1 > 15 ? 15 : q1);
            blk[2 + j] = (uint8_t)(q0 | (q1 << 4));
        }
    }
}

/* dequantize_row_q4_0 (blocks.rs:85-99). */
void orc_dequantize_row_q4_0(const uint8_t* src, size_t nblocks, float* dst) {
    for (size_t b = 0; b < nblocks; ++b) {
        const uint8_t* blk = src + b * ORC_Q4_BYTES;
        const float d = orc_f16_to_f32(rd16(blk));
        for (int j = 0; j < ORC_QK / 2; ++j) {
            const uint8_t packed = blk[2 + j];
            dst[b * ORC_QK + j] = (float)((int)(packed & 0x0F) - 8) * d;
            dst[b * ORC_QK + j + ORC_QK / 2] = (float)((int)(packed >> 4) - 8) * d;
        }
    }
}

/* quantize_row_q8_0 (blocks.rs:102-123). */
void orc_quantize_row_q8_0(const float* src, size_t n, uint8_t* dst) {
    for (size_t b = 0; b < n / ORC_QK; ++b) {
        const float* chunk = src + b * ORC_QK;
        uint8_t* blk = dst + b * ORC_Q8_BYTES;
        float amax = 0.0f;
        for (int i = 0; i < ORC_QK; ++i) {
            const float av = fabsf(chunk[i]);
            if (av > amax) amax = av;
        }
        const float d = amax / 127.0f;
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        wr16(blk, orc_f32_to_f16(d));
        for (int j = 0; j < ORC_QK; ++j) {
            // `.round().clamp(-127.0, 127.0) as i8`: clamp keeps NaN, the cast
            // sends it to 0
            float v = roundf(chunk[j] * id);
            if (v < -127.0f) v = -127.0f;
            if (v > 127.0f) v = 127.0f;
            blk[2 + j] = (uint8_t)(int8_t)rust_f32_as_i32(v);
        }
    }
}

/* dequantize_row_q8_0 (blocks.rs:126-135). */
void orc_dequantize_row_q8_0(const uint8_t* src, size_t nblocks, float* dst) {
    for (size_t b = 0; b < nblocks; ++b) {
        const uint8_t* blk = src + b * ORC_Q8_BYTES;
        const float d = orc_f16_to_f32(rd16(blk));
        for (int j = 0; j < ORC_QK; ++j) dst[b * ORC_QK + j] = (float)(int8_t)blk[2 + j] * d;
    }
}

/* Integer dot of one Q4_0 block with one Q8_0 block, weight i at nibble
 * (i < 16: low of byte i, else high of byte i-16) minus 8. */
static inline int32_t block_isum(const uint8_t* w, const uint8_t* a) {
    int32_t s = 0;
    for (int j = 0; j < ORC_QK / 2; ++j) {
        const uint8_t packed = w[2 + j];
        const int v0 = (int)(packed & 0x0F) - 8;
        const int v1 = (int)(packed >> 4) - 8;
        s += v0 * (int)(int8_t)a[2 + j] + v1 * (int)(int8_t)a[2 + j + ORC_QK / 2];
    }
    return s;
}

/* vec_dot_q4_0_q8_0_scalar (kernels.rs:145-161): one f32 accumulator, block
 * sums in order, each term (sum_i as f32) * (d_w * d_a). */
float orc_vec_dot_q4_0_q8_0_scalar(const uint8_t* w, const uint8_t* a, size_t nblocks) {
    float sumf = 0.0f;
    for (size_t b = 0; b < nblocks; ++b) {
        const uint8_t* wb = w + b * ORC_Q4_BYTES;
        const uint8_t* ab = a + b * ORC_Q8_BYTES;
        const int32_t s = block_isum(wb, ab);
        const float d = orc_f16_to_f32(rd16(wb)) * orc_f16_to_f32(rd16(ab));
        sumf += (float)s * d;
    }
    return sumf;
}

/* vec_dot_q4_0_q8_0_avx2 (kernels.rs:163-212): eight f32 lanes; lane k takes
 * the exact integer dot of elements 4k..4k+3 of each block (maddubs + madd),
 * converts it and accumulates fma(d, lane, acc_k); then the horizontal sum
 * ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)) of kernels.rs:203-210.  Activations
 * are clamped to >= -127 (kernels.rs:190-191), a no-op for quantize_row_q8_0
 * output. */
float orc_vec_dot_q4_0_q8_0_avx2(const uint8_t* w, const uint8_t* a, size_t nblocks) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (size_t b = 0; b < nblocks; ++b) {
        const uint8_t* wb = w + b * ORC_Q4_BYTES;
        const uint8_t* ab = a + b * ORC_Q8_BYTES;
        const float d = orc_f16_to_f32(rd16(wb)) * orc_f16_to_f32(rd16(ab));
        int wi[ORC_QK], ai[ORC_QK];
        for (int j = 0; j < ORC_QK / 2; ++j) {
            wi[j] = (int)(wb[2 + j] & 0x0F) - 8;
            wi[j + ORC_QK / 2] = (int)(wb[2 + j] >> 4) - 8;
        }
        for (int j = 0; j < ORC_QK; ++j) {
            const int v = (int)(int8_t)ab[2 + j];
            ai[j] = v < -127 ? -127 : v;
        }
        for (int k = 0; k < 8; ++k) {
            int32_t lane = 0;
            for (int i = 4 * k; i < 4 * k + 4; ++i) lane += wi[i] * ai[i];
            acc[k] = fmaf(d, (float)lane, acc[k]);
        }
    }
    const float s0 = acc[0] + acc[4], s1 = acc[1] + acc[5];
    const float s2 = acc[2] + acc[6], s3 = acc[3] + acc[7];
    return (s0 + s1) + (s2 + s3);
}

/* gemm_q4_0 (kernels.rs:308-394): out[b*rows + r] = vec_dot(W row r, x row b)
 * for every b < batch, r < rows; x_q8 holds batch rows of cols/32 blocks.
 * avx2 selects the AVX2 dot product (the x86 production path), else the
 * scalar one (which the NEON path equals bit for bit). */
void orc_gemm_q4_0(const uint8_t* w, const uint8_t* x_q8, float* out, int batch, int rows,
                   int cols, int avx2) {
    const size_t nb = (size_t)cols / ORC_QK;
    for (int b = 0; b < batch; ++b)
        for (int r = 0; r < rows; ++r) {
            const uint8_t* wr = w + (size_t)r * nb * ORC_Q4_BYTES;
            const uint8_t* xr = x_q8 + (size_t)b * nb * ORC_Q8_BYTES;
            out[(size_t)b * rows + r] = avx2 ? orc_vec_dot_q4_0_q8_0_avx2(wr, xr, nb)
                                             : orc_vec_dot_q4_0_q8_0_scalar(wr, xr, nb);
        }
}
