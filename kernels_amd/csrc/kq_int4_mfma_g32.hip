// kq_int4_mfma_g32.hip -- matrix-core int4 kernels for quant group size 32.
#include "kq_int4_mfma_kernel.h"

namespace kq {

hipError_t launch_mfma_g32(const mfma::Args& a, const mfma::Plan& pl, bool sb, bool bf,
                           hipStream_t s) {
    return mfma::dispatch<32>(a, pl, sb, bf, s);
}

}  // namespace kq
