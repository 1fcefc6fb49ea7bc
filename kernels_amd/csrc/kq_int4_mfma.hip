// kq_int4_mfma.hip -- int4 skinny GEMM on the matrix cores (gfx950).
// (placeholder until the MFMA path lands: reports "unsupported")
#include "kq_device.h"
#include "kq_internal.h"

namespace kq {

Int4Cfg int4_mfma_default(uint32_t, uint32_t, uint32_t) { return Int4Cfg{1, 1}; }

bool int4_mfma_supported(uint32_t, uint32_t, uint32_t, Int4Cfg) { return false; }

hipError_t launch_int4_mfma(const uint32_t*, const uint16_t*, const uint16_t*, int, bool,
                            const uint16_t*, void*, bool, uint32_t, uint32_t, uint32_t, uint32_t,
                            Int4Cfg, hipStream_t) {
    return hipErrorNotSupported;
}

}  // namespace kq
