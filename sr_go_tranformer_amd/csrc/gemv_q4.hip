// Q4 instantiations of the dequant GEMV kernels (gemv_kernels.h).
#include "gemv_kernels.h"

namespace srq {

int gemv_launch_q4(hipStream_t s, const GemvArgs &a, bool fast) {
    return fast ? launch_epi<SRQ_Q4, true>(s, a) : launch_epi<SRQ_Q4, false>(s, a);
}

hipError_t gemv_prepare_q4() {
    const hipError_t e = prepare_epi<SRQ_Q4, true>();
    return e != hipSuccess ? e : prepare_epi<SRQ_Q4, false>();
}

}  // namespace srq
