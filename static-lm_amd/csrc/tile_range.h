// Byte range of a buffer descriptor that covers one key tile of a layer's
// K or V slice.  No HIP dependencies, so host code and CPU tests can include
// it as well as the kernels.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define SLM_HD __host__ __device__
#else
#define SLM_HD
#endif

namespace slm {

// Largest kv_dim a context accepts: the prefill kernels keep each thread's
// byte offset inside a 32-row tile in 32 bits (32 * kMaxKvDim * 4 < 2^31).
constexpr int kMaxKvDim = 1 << 20;

// Bytes from the tile's first row kb to the end of the rows the tile may
// read: rows kb .. min(kv_len, kb + tile_rows) - 1 of kv_dim floats.  A load
// past that range returns zeros, which is how rows at or past kv_len read.
// Bounded by the tile, never by the whole rest of the slice: (kv_len - kb) *
// kv_dim * 4 wraps in 32 bits once one layer's slice passes 4 GiB, and the
// rows it then cuts off would read as zeros.  Needs tile_rows * kv_dim * 4 <
// 2^32 (tile_range_fits) and 0 <= kb <= kv_len.  One 32-bit subtract, min
// and multiply, so for uniform operands the kernels compute it on the scalar
// unit: 64-bit signed compares, or a min and a max (which the compiler fuses
// into v_med3), take vector instructions, and a descriptor range held in a
// vector register makes the compiler wrap every buffer load in a
// readfirstlane loop.
SLM_HD constexpr bool tile_range_fits(int tile_rows, int kv_dim) {
    return (int64_t)tile_rows * kv_dim * 4 <= (int64_t)0xFFFFFFFF;
}

SLM_HD inline uint32_t tile_range_bytes(int kv_len, int kb, int tile_rows, int kv_dim) {
    const int left = kv_len - kb;  // 0 <= left: both non-negative, no overflow
    const int rows = left < tile_rows ? left : tile_rows;
    return (uint32_t)rows * (uint32_t)kv_dim * 4u;
}

}  // namespace slm

#undef SLM_HD
