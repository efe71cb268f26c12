// Dequant GEMV dispatch: format, layout and batch checks, then the
// per-format launchers (gemv_q8.hip, gemv_q4.hip, gemv_f32.hip; kernels in
// gemv_kernels.h).
#include "gemv_kernels.h"

namespace srq {

// Raise the dynamic LDS limit of every GEMV instantiation once per device,
// before any launch (also before graph capture).
int gemv_prepare() {
    const hipError_t errs[] = {gemv_prepare_q8(), gemv_prepare_q4(), gemv_prepare_f32()};
    for (hipError_t e : errs)
        if (e != hipSuccess) return fail(SRQ_EDEVICE, "gemv LDS attribute: %s", hipGetErrorString(e));
    return SRQ_OK;
}

// Largest batch (8, 4, 2 or 1) whose staged activations fit the LDS budget,
// or 0 when even one row does not fit.
int gemv_max_rows(int fmt, int64_t cols, bool norm, int64_t extra_floats) {
    const bool fast = gemv_fast_ok(fmt, cols);
    const int64_t cw = !fast ? 256 : fmt == SRQ_Q8 ? 1024 : fmt == SRQ_Q4 ? 2048 : 256;
    const int64_t ld = (cols + cw - 1) / cw * cw;
    // Fast layouts stream at most 8 rows per launch (Q4: 2); larger batches
    // are chunked by the caller.  Their LDS also holds the norm weight and
    // the epilogue's per-row data (extra_floats bounds it).
    for (int nb = !fast ? 8 : fmt == SRQ_Q4 ? 2 : 8; nb >= 1; nb /= 2) {
        const int64_t floats = fast ? nb * ld + (norm ? ld : 0) + extra_floats : nb * ld;
        if (floats * 4 <= (int64_t)kMaxLds) return nb;
    }
    return 0;
}
bool gemv_fast_ok(int fmt, int64_t cols) {
    if (fmt == SRQ_Q8) return cols % 16 == 0;
    if (fmt == SRQ_Q4) return cols % 32 == 0;
    return cols % 4 == 0;
}

int launch_gemv(hipStream_t s, const GemvArgs &a) {
    if (a.n < 1 || a.n > 8) return fail(SRQ_EINVAL, "gemv: n=%d outside 1..8", a.n);
    if (a.rows <= 0 || a.cols <= 0) return SRQ_OK;
    const bool fast = gemv_fast_ok(a.fmt, a.cols) && ((uintptr_t)a.values & 15) == 0;
    switch (a.fmt) {
        case SRQ_Q8: return gemv_launch_q8(s, a, fast);
        case SRQ_Q4: return gemv_launch_q4(s, a, fast);
        case SRQ_F32: return gemv_launch_f32(s, a, fast);
    }
    return fail(SRQ_EINVAL, "gemv: bad format");
}

}  // namespace srq
