/*
 * slm_calib -- measurement probes for the bench (libslm_calib.so), kept out
 * of the product library.
 *
 * No counterpart in static-lm.  slm_calib_mfma_f32 times the fp32 matrix
 * cores with every SIMD busy; slm_calib_hbm_read times a plain streaming
 * read.  Neither is a ceiling of the product kernels: the decode kernel at
 * 131k positions streams faster than this read probe does.  The bench
 * reports them next to the published peaks (8 TB/s HBM, 157.3 TFLOP/s dense
 * fp32 MFMA), which remain the roofline denominators.  Both calls are
 * synchronous, allocate and free their own device memory and stream, and
 * restore the caller's current device.  Return codes are those of
 * slm_attn.h.
 */
#ifndef SLM_CALIB_H
#define SLM_CALIB_H

#include <stdint.h>

#include "../../include/slm_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Rate of v_mfma_f32_16x16x4_f32 with every SIMD of the device busy: each of
 * 2 waves per SIMD issues iters * 16 independent MFMAs.  *tflops is the best of
 * three timed launches (2048 flop per MFMA), *ms that launch's duration. */
int slm_calib_mfma_f32(int32_t device, int32_t iters, double* tflops, double* ms);

/* Streaming read of a fresh `bytes`-byte buffer (a multiple of 16, at least
 * 1 MiB; pick it well above the 256 MB Infinity Cache) with 128-bit loads,
 * nontemporal when `nontemporal` is nonzero, each workgroup reading its own
 * contiguous range.  *gbs is the best of five runs. */
int slm_calib_hbm_read(int32_t device, int64_t bytes, int32_t nontemporal, double* gbs);

#ifdef __cplusplus
}
#endif

#endif /* SLM_CALIB_H */
