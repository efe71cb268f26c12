// Q8 instantiations of the dequant GEMV kernels (gemv_kernels.h).
#include "gemv_kernels.h"

namespace srq {

int gemv_launch_q8(hipStream_t s, const GemvArgs &a, bool fast) {
    return fast ? launch_epi<SRQ_Q8, true>(s, a) : launch_epi<SRQ_Q8, false>(s, a);
}

hipError_t gemv_prepare_q8() {
    const hipError_t e = prepare_epi<SRQ_Q8, true>();
    return e != hipSuccess ? e : prepare_epi<SRQ_Q8, false>();
}

}  // namespace srq
