// k_gemm.hip -- prefill GEMM (m > 8) for gfx950.  Placeholder until the
// MFMA kernel lands: reports "not supported" so the caller uses the matvec.
#include "aq_internal.h"

namespace aq {

size_t gemm_workspace_bytes(int, int64_t, int64_t, int64_t) { return (size_t)-1; }

hipError_t launch_gemm(const WLayout &, int64_t, int64_t, const ActPlanes &, int64_t, float *, int32_t *, int32_t *,
                       void *, size_t, hipStream_t) {
    return hipErrorNotSupported;
}

}  // namespace aq
