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
// Computed in 64 bits and clamped to the descriptor's 32-bit field: a tile
// never reads more than tile_rows rows from kb, so the clamp only matters
// for a tile far larger than any kernel uses, and without the tile bound a
// layer slice past 4 GiB would wrap the range and zero rows that exist.
SLM_HD inline uint32_t tile_range_bytes(int kv_len, int kb, int tile_rows, int kv_dim) {
    int64_t rows = (int64_t)kv_len - (int64_t)kb;
    if (rows > tile_rows) rows = tile_rows;
    if (rows < 0) rows = 0;
    const int64_t bytes = rows * (int64_t)kv_dim * 4;
    return bytes > (int64_t)0xFFFFFFFF ? 0xFFFFFFFFu : (uint32_t)bytes;
}

}  // namespace slm

#undef SLM_HD
