// kq_int4_mfma_g64.hip -- matrix-core int4 kernels for quant group size 64.
#include "kq_int4_mfma_kernel.h"

namespace kq {

hipError_t launch_mfma_g64(const mfma::Args& a, const mfma::Plan& pl, bool sb, bool bf,
                           hipStream_t s) {
    return mfma::dispatch<64>(a, pl, sb, bf, s);
}

}  // namespace kq
