// Causal prefill attention on fp32 MFMA for gfx950 (not yet enabled: the
// split-K rows kernel serves prefill until this path is parity-checked).
#include "slm_internal.h"

namespace slm {

bool prefill_mfma_supported(const Shape&) { return false; }

hipError_t launch_prefill_mfma(const Shape&, const PrefillArgs&, hipStream_t) {
    return hipErrorNotSupported;
}

}  // namespace slm
