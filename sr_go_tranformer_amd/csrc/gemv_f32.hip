// F32 instantiations of the dequant GEMV kernels (gemv_kernels.h).
#include "gemv_kernels.h"

namespace srq {

int gemv_launch_f32(hipStream_t s, const GemvArgs &a, bool fast) {
    return fast ? launch_epi<SRQ_F32, true>(s, a) : launch_epi<SRQ_F32, false>(s, a);
}

hipError_t gemv_prepare_f32() {
    const hipError_t e = prepare_epi<SRQ_F32, true>();
    return e != hipSuccess ? e : prepare_epi<SRQ_F32, false>();
}

}  // namespace srq
