// Which prefill kernel runs for a batch.  No HIP dependencies, so host code
// and CPU tests can include it as well as the launcher.
#pragma once

namespace slm {

// The prefill kernels, numbered as SLM_PF_* in slm_attn.h.
enum class PrefillKernel : int {
    kFourHeads = 0,
    kThreeHeads = 1,
    kTwoHeads = 2,
    kOneHead = 3,
    kKeySplit = 4,
    kPairedFourHeads = 5,
    kDma = 6,
    kDmaPaired = 7,
    kPairedTwoHeads = 8,
    kPairedOneHead = 9,
};

// Query heads per workgroup (hw, all of one KV head) and 16-row query blocks
// per workgroup (qs) of the head-group tiling.
struct PrefillTiling {
    int hw;
    int qs;
};

inline PrefillTiling prefill_tiling(int kv_mul) {
    if (kv_mul % 4 == 0) return {4, 1};
    if (kv_mul % 3 == 0) return {3, 1};
    if (kv_mul % 2 == 0) return {2, 2};
    return {1, 4};
}

// Which kernel a prefill of n rows from row `start` runs, for head_dim,
// num_heads query heads (kv_mul per KV head) on a device of `cus` CUs: a pure
// function of the batch, the shape and the CU count.  The launcher and the
// kernel query of the C ABI both call it.
inline PrefillKernel prefill_plan(int head_dim, int num_heads, int kv_mul, int cus, int start,
                                  int n) {
    const PrefillTiling t = prefill_tiling(kv_mul);
    if (head_dim == 128) {
        // Short prefills whose head-group tiling gives at most one workgroup
        // per CU run one wave per SIMD, and the heaviest causal block sets
        // the time (its tiles in series: 16 at 512 rows, against 8.5 on
        // average).  Pairs of blocks i and n_qb-1-i, two heads and two key
        // splits per workgroup give every SIMD the same share.  Measured for
        // the Llama-3-8B shape (interleaved, per call): 256 rows 25.6 against
        // 28.2 us, 512 rows 39.9 against 49.7, 512 rows at start 1000 111.2
        // against 125.6; 1024 rows (two workgroups per CU) even; 2048 / 3072
        // rows 368 / 785 against 301 / 607 us (158 VGPRs: one 8-wave workgroup
        // per CU against three 4-wave ones); below 256 rows 13% slower.
        // With one head and four key splits per workgroup (no GQA sharing of
        // the tiles, 200 VGPRs), while that grid still fits the CUs once: 256
        // rows 22.2 against 25.6 us (Llama-3-8B shape) and 24.9 against 31.1
        // (MHA, 32 KV heads, where two heads per workgroup are not possible);
        // at 512 rows, two rounds of 512 workgroups, 53.2 against 39.7 and
        // 54.9 against 53.9.
        const long wgs = (long)((n + 16 * t.qs - 1) / (16 * t.qs)) * (num_heads / t.hw);
        const long pairs = ((n + 15) / 16 + 1) / 2;
        if (n >= 256 && wgs <= cus) {
            if (pairs * num_heads <= cus) return PrefillKernel::kPairedOneHead;
            if (kv_mul % 2 == 0 && pairs * (num_heads / 2) <= cus)
                return PrefillKernel::kPairedTwoHeads;
        }
        // Four heads of one KV head and two 16-row query blocks per workgroup
        // (8 waves), DMA-fed LDS tiles: the same K/V tile serves eight waves,
        // and two 64 KiB workgroups fit a CU's LDS.  With consecutive blocks
        // its grid is half the other kernel's, so that form runs only when it
        // still gives four workgroups per CU: measured for the Llama-3-8B
        // shape, the DMA kernel against the register-prefetch one took 73.5 /
        // 48.8 us at 512 rows, 141 / 114 at 1024, 388 / 324 at 2048, 625 /
        // 619-637 at 3072 and 985-991 / 1025 at 4096.  With paired blocks (i
        // and n_qb-1-i, 16 rows each; same bits) every workgroup has the same
        // work, so the time follows the workgroups per CU: it runs when they
        // are at most one or a whole number.  Interleaved per call, against
        // the kernel that ran before: 600 / 768 / 1024 rows (152 / 192 / 256
        // workgroups) 55.1 / 67.4 / 91 against 62.5 / 80.4 / 115 us, 2048 /
        // 3072 / 4096 / 5120 / 8192 rows (2, 3, 4, 5, 8 per CU) 270 / 577 /
        // 997 / 1535 / 3843 against 305 / 607 / 1003 / 1590 / 3880; with
        // fractions per CU it lost (1152 / 1280 / 2560 / 3584 rows: +16 / +11
        // / +7 / +7%), and below 512 rows too (64 / 100 / 200 rows +21 / +21
        // / +9%, 77 rows at start 300 +45%).  Pairing halves the grid, so it
        // runs only where the four-head kernel's grid has more workgroups
        // than CUs (with one per CU it only idles half of them: hd 96 at 512
        // rows from start 1000, +32%).
        if (t.hw == 4) {
            const long pwgs = (((long)n + 15) / 16 + 1) / 2 * (num_heads / 4);
            if (n >= 512 && wgs > cus && (pwgs <= cus || pwgs % cus == 0))
                return PrefillKernel::kDmaPaired;
            if ((long)((n + 31) / 32) * (num_heads / 4) >= 4L * cus)
                return PrefillKernel::kDma;
        }
    }
    // Short prefills, head_dim <= 64: when the head-group tiling gives fewer
    // than two workgroups per CU, one head and one 16-row query block per
    // workgroup with its key tiles split over four waves, as long as the
    // heaviest block keeps two tiles per split: more workgroups, and the
    // heaviest block's tiles walked by four SIMDs instead of one.  (Each
    // thread then prefetches four tiles' share: 169 VGPRs at hd 64, 312 at
    // hd 128.)
    if (head_dim <= 64) {
        constexpr int KSP = 4;
        const int qs = t.hw == 1 ? 4 : t.hw == 2 ? 2 : 1;
        const long wgs = (long)((n + 16 * qs - 1) / (16 * qs)) * (num_heads / t.hw);
        const long tiles = ((long)start + n + 31) / 32;  // the heaviest block's
        if (wgs < 2L * cus && tiles >= 2L * KSP) return PrefillKernel::kKeySplit;
    }
    if (head_dim <= 96 && t.hw == 4) {
        // Paired blocks (i and n_qb-1-i) in the four-head register kernel, as
        // in the DMA-fed one: where the four-head grid has more workgroups
        // than CUs and the paired grid (8-wave workgroups, one per CU) is at
        // most one or two per CU.  Interleaved per call against the four-head
        // kernel, GQA 4 (32 heads): at 1024 rows hd 16 / 32 / 48 / 64 / 96
        // 23.8 / 35.5 / 48.2 / 53.5 / 77.8 against 26.8 / 38.7 / 54.8 / 63.5 /
        // 91.9 us, at 2048 rows 55.7 / 87.4 / 123.3 / 149.1 / 222.2 against
        // 60.8 / 97.2 / 137.9 / 167.6 / 248.9, hd 96 at 768 rows 59.3 against
        // 66.0; it lost with 1.5 per CU (1536 rows: +1.4 / +2.4% at hd 64 /
        // 96) and from three per CU (4096 rows: +3.5 / +1.8%, against the
        // four-head kernel's three 4-wave workgroups per CU); with three heads
        // per workgroup (SmolLM2 shape) and for MHA it gained nothing or lost
        // (MHA at 2048 rows +19%).
        const long wgs = (long)((n + 15) / 16) * (num_heads / 4);
        const long pwgs = (((long)n + 15) / 16 + 1) / 2 * (num_heads / 4);
        if (wgs > cus && (pwgs <= cus || pwgs == 2L * cus))
            return PrefillKernel::kPairedFourHeads;
    }
    if (t.hw == 4) return PrefillKernel::kFourHeads;
    if (t.hw == 3) return PrefillKernel::kThreeHeads;
    if (t.hw == 2) return PrefillKernel::kTwoHeads;
    return PrefillKernel::kOneHead;
}

}  // namespace slm
