// C-ABI runtime of the gfx950 quantized-weight inference path.
//
// Host side of the drop-in boundary declared in include/srq.h: executor
// (kernelExecutor), weight handles (Param), model storage and loading
// (loadHFModelFormatKV + readParam), paged KV pools (pagePool/KVCache), the
// batched step (prefillSelected) and greedy generation (inferHFIDs), all of
// cmd/monolith/monolith.go.  Every GPU computation is a HIP kernel of this
// library; there is no CPU fallback.
#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "srq_internal.h"

// Scratch of srq_linear_noalloc (split-K partial sums and wide-row flags of
// the GEMM path): a fixed array of the code object, one copy per GPU, held
// until the process ends.  Host code never passes its name to a kernel (on
// the host it is only a stand-in for the symbol): each device's address is
// looked up once, when the device is prepared, and used from then on.
static __device__ __align__(256) unsigned char scratch[SRQ_NOALLOC_SCRATCH_BYTES];

namespace srq {

static thread_local std::string g_err;

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

void clear_error() { g_err.clear(); }

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_prep_mu;
bool g_prepared[kMaxDevices];
// Device address of `scratch` on each prepared device (written under
// g_prep_mu before g_prepared is set; read only through an executor of that
// device, which exists only after its preparation).
void *g_noalloc_scratch[kMaxDevices];

// Once per device, with that device current: kernel attributes, and the
// device's address of the no-allocation scratch array.
int prepare_device(int device) {
    if (device < 0 || device >= kMaxDevices) return fail(SRQ_EINVAL, "device %d above the supported %d", device, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_prep_mu);
    if (g_prepared[device]) return SRQ_OK;
    SRQ_CHECK(gemv_prepare());
    SRQ_CHECK(attention_prepare());
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
        return fail(SRQ_EDEVICE, "no-allocation scratch lookup failed: %s", hipGetErrorString(e));
    g_noalloc_scratch[device] = p;
    g_prepared[device] = true;
    return SRQ_OK;
}

struct DevBuf {
    void *p = nullptr;
    size_t n = 0;
};

// Grows b to at least `bytes`.  A buffer that has to grow again takes half
// as much again as it held, so steps whose shapes creep up (the attention
// scratch gains a split every 64 positions) reallocate -- a stream
// synchronisation, a free and an allocation -- a logarithmic number of times.
int ensure(DevBuf &b, size_t bytes, hipStream_t s) {
    if (bytes <= b.n) return SRQ_OK;
    size_t want = std::max(bytes, (size_t)256);
    if (b.p) {
        want = std::max(want, b.n + b.n / 2);
        SRQ_HIP(hipStreamSynchronize(s));
        SRQ_HIP(hipFree(b.p));
        b.p = nullptr;
        b.n = 0;
    }
    if (hipMalloc(&b.p, want) != hipSuccess) {
        b.p = nullptr;
        return fail(SRQ_ENOMEM, "device allocation of %zu bytes failed", want);
    }
    b.n = want;
    return SRQ_OK;
}

void release(DevBuf &b) {
    if (b.p) (void)hipFree(b.p);
    b.p = nullptr;
    b.n = 0;
}

template <class T>
T *as(DevBuf &b) {
    return (T *)b.p;
}

int matrix_format(const std::string &format, bool embed_or_head) {
    if (format == "f32") return SRQ_F32;
    if (format == "q8") return SRQ_Q8;
    if (format == "q4") return SRQ_Q4;
    return embed_or_head ? SRQ_Q8 : SRQ_Q4;  // q4-mixed (M:572-582)
}

// hfInverseFrequency (M:4961-4977) with Transformers' f32 steps.
float inverse_frequency(const srq_model_config &c, int head_dim, int index) {
    float e = (float)(2 * index) / (float)head_dim;
    float inv = 1.0f / (float)std::pow(c.rope_theta, (double)e);
    if (!c.rope_llama3) return inv;
    volatile float two_pi = (float)(2 * M_PI);
    float wave = two_pi / inv;
    float low_wave = (float)((double)c.rope_original / c.rope_low);
    float high_wave = (float)((double)c.rope_original / c.rope_high);
    float factor = (float)c.rope_factor;
    if (wave > low_wave) return inv / factor;
    if (wave >= high_wave) {
        volatile float t = (float)c.rope_original / wave;
        float smooth = (t - (float)c.rope_low) / (float)(c.rope_high - c.rope_low);
        volatile float a = (1 - smooth) * inv;
        volatile float b = a / factor;
        volatile float d = smooth * inv;
        return b + d;
    }
    return inv;
}

}  // namespace
}  // namespace srq

using namespace srq;

// ------------------------------------------------------------------ handles
// Activation workspace of one executor or decoder (decodeWorkspace,
// M:6062-6100).  Captured graphs point into a decoder's own workspace, so a
// later step that grows the executor's workspace cannot invalidate them.
struct Workspace {
    DevBuf X, N, Q, A, T, H, W2, LOG, LOGC, meta, flags, ATT, ATTC, PLAN, SMP, SMPS;
    void release_all() {
        for (DevBuf *b : {&X, &N, &Q, &A, &T, &H, &W2, &LOG, &LOGC, &meta, &flags, &ATT, &ATTC, &PLAN, &SMP, &SMPS})
            release(*b);
    }
};

// Handles are reference counted: a model holds its executor, a pool its
// model, a cache its pool and a decoder its executor, model and cache, so
// destroy calls may come in any order (Go finalizers, Python's collector)
// without a handle outliving what it points to.  *_destroy drops the
// caller's reference.
struct srq_exec {
    std::atomic<int> refs{1};
    int device = 0;
    hipStream_t stream = nullptr;
    int32_t *d_err = nullptr;  // [4] device error words
    int32_t *h_err = nullptr;  // pinned mirror
    Workspace ws;
    int32_t *h_meta = nullptr;  // pinned metadata staging
    size_t h_meta_n = 0;
    int32_t *h_smp = nullptr;   // pinned staging of srq_sample's per-row words
    size_t h_smp_n = 0;
    hipEvent_t layer_done[2] = {};  // in-flight cancellation: progress events of the last layer groups
};

struct srq_weight {
    int fmt = SRQ_F32;
    int64_t rows = 0, cols = 0;
    void *values = nullptr;
    float *scales = nullptr;
    bool owned = false;
};

struct Layer {
    srq_weight qkv, o, gu, down;          // fused storage used by the step
    srq_weight q, k, v, gate, up;         // views into qkv / gu
    float *n1 = nullptr, *n2 = nullptr, *bias = nullptr;
};

struct srq_model {
    std::atomic<int> refs{1};
    int device = 0;
    srq_exec *e = nullptr;
    srq_model_config c{};
    std::string format;
    int hd = 0, kvdim = 0;
    srq_weight embed, output;
    bool has_output = false;
    float *final_norm = nullptr;
    std::vector<Layer> L;
    float *cos_t = nullptr, *sin_t = nullptr;
    std::vector<float> h_cos, h_sin;
    std::vector<void *> allocs;
    int64_t resident = 0;
};

struct srq_pool {
    std::atomic<int> refs{1};
    int device = 0;
    srq_model *m = nullptr;
    float *base = nullptr;
    int32_t max_pages = 0, reserved = 0;
    int64_t page_elems = 0;
    std::vector<int32_t> free_list;
};

struct srq_cache {
    std::atomic<int> refs{1};
    srq_pool *p = nullptr;
    int32_t pos = 0, reserve = 0;
    std::vector<int32_t> pages;
    bool released = false;
    bool busy = false;  // a live decoder owns the cache's position and rows
};

namespace {

struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) (void)hipSetDevice(dev);
        // Drop any error left by an earlier best-effort call (a release on
        // a teardown path) so launch checks report only their own errors.
        (void)hipGetLastError();
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

int check_err_flag(srq_exec *e, int code, const char *what) {
    SRQ_HIP(hipMemcpyAsync(e->h_err, e->d_err, sizeof(int32_t) * 4, hipMemcpyDeviceToHost, e->stream));
    SRQ_HIP(hipStreamSynchronize(e->stream));
    if (e->h_err[0]) {
        SRQ_HIP(hipMemsetAsync(e->d_err, 0, sizeof(int32_t) * 4, e->stream));
        SRQ_HIP(hipStreamSynchronize(e->stream));
        return fail(code, "%s", what);
    }
    return SRQ_OK;
}

int alloc_weight(srq_model *m, srq_weight &w, int fmt, int64_t rows, int64_t cols) {
    w.fmt = fmt;
    w.rows = rows;
    w.cols = cols;
    int64_t vb = rows * row_bytes(fmt, cols), sb = fmt == SRQ_F32 ? 0 : rows * groups_of(cols) * 4;
    if (hipMalloc(&w.values, (size_t)std::max<int64_t>(vb, 16)) != hipSuccess)
        return fail(SRQ_ENOMEM, "weight allocation (%lld bytes) failed", (long long)vb);
    m->allocs.push_back(w.values);
    if (sb) {
        if (hipMalloc((void **)&w.scales, (size_t)sb) != hipSuccess)
            return fail(SRQ_ENOMEM, "scale allocation failed");
        m->allocs.push_back(w.scales);
    }
    m->resident += vb + sb;
    return SRQ_OK;
}

srq_weight view_rows(const srq_weight &w, int64_t row0, int64_t rows) {
    srq_weight v;
    v.fmt = w.fmt;
    v.rows = rows;
    v.cols = w.cols;
    v.values = (uint8_t *)w.values + row0 * row_bytes(w.fmt, w.cols);
    v.scales = w.scales ? w.scales + row0 * groups_of(w.cols) : nullptr;
    return v;
}

int alloc_f32(srq_model *m, float **p, int64_t count) {
    if (hipMalloc((void **)p, (size_t)std::max<int64_t>(count * 4, 16)) != hipSuccess)
        return fail(SRQ_ENOMEM, "allocation failed");
    m->allocs.push_back(*p);
    m->resident += count * 4;
    return SRQ_OK;
}

// Fill a weight from a device source (pack or convert).
int fill_weight(srq_exec *e, const srq_weight &w, const void *src, int dtype) {
    if (w.fmt == SRQ_F32) return launch_convert_f32(e->stream, w.rows * w.cols, src, dtype, (float *)w.values, e->d_err);
    return launch_pack(e->stream, w.fmt, w.rows, w.cols, src, dtype, w.values, w.scales, e->d_err);
}

RowMeta make_meta(srq_exec *e, srq_model *m, int layer, int32_t pt_stride, const int32_t *pos, const int32_t *sess,
                  const int32_t *pages, srq_pool *pool) {
    (void)e;
    RowMeta r;
    r.pos = pos;
    r.sess = sess;
    r.pages = pages;
    r.pt_stride = pt_stride;
    r.kv_pool = pool->base;
    r.page_elems = pool->page_elems;
    r.layer = layer;
    r.kvoff = nullptr;
    r.rope_cs = nullptr;
    r.one_sess = 0;
    (void)m;
    return r;
}

// Rows above which srq_linear takes the MFMA GEMM: up to here a row's bits
// do not depend on the batch (the GEMV computes rows independently).
constexpr int32_t kLinearGemmRows = 16;
// Rows above which a step's layers and its head take the MFMA GEMM (with
// separate norm, RoPE and SwiGLU kernels).  At 5-8 rows the GEMM and its
// reduction beat the GEMV (Llama-3.2-3B shape: gate/up 33 against 21 us,
// q/k/v 23 against 15 us, down 31 us as two 4-row GEMV passes -- 8 rows of
// 8192 activations exceed LDS -- against 19 us; the 128256-id head 164
// against about 128 us); at 3-4 rows they are even or the GEMV wins.
// Continuous batching (32 sessions): 1311 -> 1349 tokens/s against a
// boundary at 8 rows.
constexpr int32_t kStepGemmRows = 4;

// Device scratch the GEMM of y = x . W^T needs for n rows (split-K partial
// sums and wide-row flags); 0 on the GEMV path.
size_t linear_scratch_bytes(const srq_weight &w, int32_t n, int32_t gemm_rows = kLinearGemmRows) {
    return n > gemm_rows && gemm_ok(w.fmt, w.cols) ? gemm_scratch_bytes(w.fmt, n, w.rows, w.cols) : 0;
}

// y[n x w.rows] = x . W^T for n rows through the GEMV (chunks of 8) or the
// MFMA GEMM (n > gemm_rows, K multiple of 32), with optional fused RMSNorm.
// fixed (non-null): the GEMM's scratch is that caller-provided buffer of
// fixed_bytes instead of the workspace, which then never grows.
int run_linear(srq_exec *e, Workspace &ws, const srq_weight &w, const float *x, int32_t n, float *y, int64_t y_stride,
               const float *norm_w, double eps, const float *residual, int32_t gemm_rows = kLinearGemmRows,
               void *fixed = nullptr, size_t fixed_bytes = 0) {
    if (n > gemm_rows && gemm_ok(w.fmt, w.cols) && !norm_w) {
        GemmArgs g{w.fmt, w.values, w.scales, w.rows, w.cols, x, n, y, y_stride, residual, nullptr};
        if (fixed) return launch_gemm(e->stream, g, fixed, fixed_bytes);
        SRQ_CHECK(ensure(ws.flags, gemm_scratch_bytes(w.fmt, n, w.rows, w.cols), e->stream));
        return launch_gemm(e->stream, g, ws.flags.p, ws.flags.n);
    }
    const int nb = gemv_max_rows(w.fmt, w.cols, norm_w != nullptr, 0);
    if (nb < 1) return fail(SRQ_EINVAL, "input width %lld exceeds the GEMV staging limit", (long long)w.cols);
    for (int32_t r0 = 0; r0 < n; r0 += nb) {
        GemvArgs a{};
        a.fmt = w.fmt;
        a.values = w.values;
        a.scales = w.scales;
        a.rows = w.rows;
        a.cols = w.cols;
        a.x = x + (int64_t)r0 * w.cols;
        a.n = std::min(nb, n - r0);
        a.row0 = r0;
        a.norm_w = norm_w;
        a.norm_eps = eps;
        a.y = y + (int64_t)r0 * y_stride;
        a.y_stride = y_stride;
        a.epilogue = residual ? EPI_RESID : EPI_PLAIN;
        a.residual = residual ? residual + (int64_t)r0 * y_stride : nullptr;
        SRQ_CHECK(launch_gemv(e->stream, a));
    }
    return SRQ_OK;
}

}  // namespace

static void exec_unref(srq_exec *e);
static void model_unref(srq_model *m);

// ====================================================================== ABI
extern "C" {

int srq_abi_version(void) { return SRQ_ABI_VERSION; }

const char *srq_last_error(void) { return g_err.c_str(); }

int srq_device_count(int *count) {
    if (!count) return fail(SRQ_EINVAL, "null count");
    SRQ_HIP(hipGetDeviceCount(count));
    return SRQ_OK;
}

int srq_alloc(int device, size_t bytes, void **dptr) {
    if (!dptr) return fail(SRQ_EINVAL, "null pointer");
    DeviceGuard g(device);
    if (hipMalloc(dptr, std::max<size_t>(bytes, 1)) != hipSuccess) {
        *dptr = nullptr;
        return fail(SRQ_ENOMEM, "device allocation of %zu bytes failed", bytes);
    }
    return SRQ_OK;
}

int srq_free(void *dptr) {
    if (dptr) SRQ_HIP(hipFree(dptr));
    return SRQ_OK;
}

static int copy(srq_exec *e, void *dst, const void *src, size_t bytes, hipMemcpyKind kind) {
    if (!e || (!dst && bytes) || (!src && bytes)) return fail(SRQ_EINVAL, "null pointer");
    if (!bytes) return SRQ_OK;
    DeviceGuard g(e->device);
    SRQ_HIP(hipMemcpyAsync(dst, src, bytes, kind, e->stream));
    SRQ_HIP(hipStreamSynchronize(e->stream));
    return SRQ_OK;
}

int srq_copy_h2d(srq_exec *e, void *dst, const void *src, size_t bytes) {
    return copy(e, dst, src, bytes, hipMemcpyHostToDevice);
}
int srq_copy_d2h(srq_exec *e, void *dst, const void *src, size_t bytes) {
    return copy(e, dst, src, bytes, hipMemcpyDeviceToHost);
}
int srq_copy_d2d(srq_exec *e, void *dst, const void *src, size_t bytes) {
    return copy(e, dst, src, bytes, hipMemcpyDeviceToDevice);
}

// ---------------------------------------------------------------- executor
int srq_exec_create(int device, srq_exec **out) {
    if (!out) return fail(SRQ_EINVAL, "null out");
    *out = nullptr;
    int count = 0;
    SRQ_HIP(hipGetDeviceCount(&count));
    if (device < 0 || device >= count) return fail(SRQ_EINVAL, "device %d of %d", device, count);
    DeviceGuard g(device);
    SRQ_CHECK(prepare_device(device));
    srq_exec *e = new srq_exec();
    e->device = device;
    if (hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking) != hipSuccess) {
        delete e;
        return fail(SRQ_EDEVICE, "stream creation failed");
    }
    if (hipMalloc((void **)&e->d_err, sizeof(int32_t) * 4) != hipSuccess ||
        hipHostMalloc((void **)&e->h_err, sizeof(int32_t) * 4) != hipSuccess) {
        exec_unref(e);
        return fail(SRQ_ENOMEM, "executor allocation failed");
    }
    SRQ_HIP(hipMemsetAsync(e->d_err, 0, sizeof(int32_t) * 4, e->stream));
    SRQ_HIP(hipStreamSynchronize(e->stream));
    *out = e;
    return SRQ_OK;
}

static void exec_unref(srq_exec *e) {
    if (!e || --e->refs > 0) return;
    DeviceGuard g(e->device);
    if (e->stream) (void)hipStreamSynchronize(e->stream);
    e->ws.release_all();
    if (e->d_err) (void)hipFree(e->d_err);
    if (e->h_err) (void)hipHostFree(e->h_err);
    if (e->h_meta) (void)hipHostFree(e->h_meta);
    if (e->h_smp) (void)hipHostFree(e->h_smp);
    for (hipEvent_t ev : e->layer_done)
        if (ev) (void)hipEventDestroy(ev);
    if (e->stream) (void)hipStreamDestroy(e->stream);
    delete e;
}

int srq_exec_destroy(srq_exec *e) {
    exec_unref(e);
    return SRQ_OK;
}

int srq_exec_synchronize(srq_exec *e) {
    if (!e) return fail(SRQ_EINVAL, "null executor");
    DeviceGuard g(e->device);
    SRQ_HIP(hipStreamSynchronize(e->stream));
    return SRQ_OK;
}

void *srq_exec_stream(srq_exec *e) { return e ? (void *)e->stream : nullptr; }

// ----------------------------------------------------------------- packing
int srq_packed_bytes(srq_format fmt, int64_t rows, int64_t cols, int64_t *values_bytes, int64_t *scales_bytes) {
    if (rows < 0 || cols < 0 || fmt < SRQ_F32 || fmt > SRQ_Q4) return fail(SRQ_EINVAL, "bad shape or format");
    if (values_bytes) *values_bytes = rows * row_bytes(fmt, cols);
    if (scales_bytes) *scales_bytes = fmt == SRQ_F32 ? 0 : rows * groups_of(cols) * 4;
    return SRQ_OK;
}

int srq_pack(srq_exec *e, srq_format fmt, int64_t rows, int64_t cols, const void *src, srq_src_dtype dtype,
             void *values, float *scales) {
    if (!e || !src || !values || !scales) return fail(SRQ_EINVAL, "null pointer");
    if (fmt != SRQ_Q8 && fmt != SRQ_Q4) return fail(SRQ_EINVAL, "pack format must be Q8 or Q4");
    if (rows < 0 || cols < 0 || dtype < SRQ_SRC_F32 || dtype > SRQ_SRC_F16) return fail(SRQ_EINVAL, "bad shape or dtype");
    DeviceGuard g(e->device);
    SRQ_CHECK(launch_pack(e->stream, fmt, rows, cols, src, dtype, values, scales, e->d_err));
    return check_err_flag(e, SRQ_ENONFINITE, "non-finite weight in pack source");
}

int srq_fill_normal(srq_exec *e, float *dst, int64_t count, uint64_t seed, double scale) {
    if (!e || (count > 0 && !dst)) return fail(SRQ_EINVAL, "null pointer");
    if (count < 0) return fail(SRQ_EINVAL, "negative count");
    DeviceGuard g(e->device);
    SRQ_CHECK(launch_fill_normal(e->stream, dst, count, seed, scale));
    SRQ_HIP(hipStreamSynchronize(e->stream));
    return SRQ_OK;
}

// ----------------------------------------------------------------- weights
int srq_weight_create(srq_exec *e, srq_format fmt, int64_t rows, int64_t cols, const void *src, srq_src_dtype dtype,
                      srq_weight **out) {
    if (!e || !out || !src) return fail(SRQ_EINVAL, "null pointer");
    *out = nullptr;
    if (rows <= 0 || cols <= 0 || fmt < SRQ_F32 || fmt > SRQ_Q4 || dtype < SRQ_SRC_F32 || dtype > SRQ_SRC_F16)
        return fail(SRQ_EINVAL, "bad weight shape, format or dtype");
    DeviceGuard g(e->device);
    srq_weight *w = new srq_weight();
    w->fmt = fmt;
    w->rows = rows;
    w->cols = cols;
    w->owned = true;
    int64_t vb = rows * row_bytes(fmt, cols), sb = fmt == SRQ_F32 ? 0 : rows * groups_of(cols) * 4;
    if (hipMalloc(&w->values, (size_t)vb) != hipSuccess || (sb && hipMalloc((void **)&w->scales, (size_t)sb) != hipSuccess)) {
        srq_weight_destroy(w);
        return fail(SRQ_ENOMEM, "weight allocation failed");
    }
    int rc = fmt == SRQ_F32 ? launch_convert_f32(e->stream, rows * cols, src, dtype, (float *)w->values, e->d_err)
                            : launch_pack(e->stream, fmt, rows, cols, src, dtype, w->values, w->scales, e->d_err);
    if (rc == SRQ_OK) rc = check_err_flag(e, SRQ_ENONFINITE, "non-finite weight");
    if (rc != SRQ_OK) {
        srq_weight_destroy(w);
        return rc;
    }
    *out = w;
    return SRQ_OK;
}

int srq_weight_wrap(srq_format fmt, int64_t rows, int64_t cols, void *values, float *scales, srq_weight **out) {
    if (!out || !values || (fmt != SRQ_F32 && !scales)) return fail(SRQ_EINVAL, "null pointer");
    if (rows <= 0 || cols <= 0 || fmt < SRQ_F32 || fmt > SRQ_Q4) return fail(SRQ_EINVAL, "bad weight shape or format");
    srq_weight *w = new srq_weight();
    w->fmt = fmt;
    w->rows = rows;
    w->cols = cols;
    w->values = values;
    w->scales = fmt == SRQ_F32 ? nullptr : scales;
    w->owned = false;
    *out = w;
    return SRQ_OK;
}

int srq_weight_destroy(srq_weight *w) {
    if (!w) return SRQ_OK;
    if (w->owned) {
        if (w->values) (void)hipFree(w->values);
        if (w->scales) (void)hipFree(w->scales);
    }
    delete w;
    return SRQ_OK;
}

int srq_weight_info(const srq_weight *w, int *fmt, int64_t *rows, int64_t *cols, void **values, float **scales) {
    if (!w) return fail(SRQ_EINVAL, "null weight");
    if (fmt) *fmt = w->fmt;
    if (rows) *rows = w->rows;
    if (cols) *cols = w->cols;
    if (values) *values = w->values;
    if (scales) *scales = w->scales;
    return SRQ_OK;
}

int srq_dequant_rows(srq_exec *e, const srq_weight *w, const int32_t *rows, int32_t count, float *dst) {
    if (!e || !w || (count > 0 && (!rows || !dst))) return fail(SRQ_EINVAL, "null pointer");
    if (count < 0) return fail(SRQ_EINVAL, "negative count");
    DeviceGuard g(e->device);
    SRQ_CHECK(launch_dequant_rows(e->stream, w->fmt, w->cols, w->values, w->scales, rows, count, dst));
    SRQ_HIP(hipStreamSynchronize(e->stream));
    return SRQ_OK;
}

// ------------------------------------------------------------------ linear
int srq_linear(srq_exec *e, float *y, const float *x, const srq_weight *w, int32_t n) {
    if (!e || !y || !x || !w) return fail(SRQ_EINVAL, "null pointer");
    if (n < 1 || n > 1024) return fail(SRQ_EINVAL, "linear rows n=%d outside 1..1024", n);
    const char *yb = (const char *)y, *xb = (const char *)x;
    if (yb < xb + (size_t)n * w->cols * 4 && xb < yb + (size_t)n * w->rows * 4)
        return fail(SRQ_EINVAL, "y overlaps x");
    DeviceGuard g(e->device);
    SRQ_CHECK(run_linear(e, e->ws, *w, x, n, y, w->rows, nullptr, 0.0, nullptr));
    SRQ_HIP(hipStreamSynchronize(e->stream));
    return SRQ_OK;
}

int srq_linear_enqueue(srq_exec *e, float *y, const float *x, const srq_weight *w, int32_t n) {
    if (!e || !y || !x || !w) return fail(SRQ_EINVAL, "null pointer");
    if (n < 1 || n > 1024) return fail(SRQ_EINVAL, "linear rows n=%d outside 1..1024", n);
    const char *yb = (const char *)y, *xb = (const char *)x;
    if (yb < xb + (size_t)n * w->cols * 4 && xb < yb + (size_t)n * w->rows * 4)
        return fail(SRQ_EINVAL, "y overlaps x");
    DeviceGuard g(e->device);
    return run_linear(e, e->ws, *w, x, n, y, w->rows, nullptr, 0.0, nullptr);
}

// srq_linear_enqueue with the split-K scratch in the library's fixed device
// array: no allocation of any kind (no executor workspace growth).
int srq_linear_noalloc(srq_exec *e, float *y, const float *x, const srq_weight *w, int32_t n) {
    if (!e || !y || !x || !w) return fail(SRQ_EINVAL, "null pointer");
    if (n < 1 || n > 1024) return fail(SRQ_EINVAL, "linear rows n=%d outside 1..1024", n);
    const char *yb = (const char *)y, *xb = (const char *)x;
    if (yb < xb + (size_t)n * w->cols * 4 && xb < yb + (size_t)n * w->rows * 4)
        return fail(SRQ_EINVAL, "y overlaps x");
    // The GEMM's scratch grows linearly with n and its K slices depend on
    // the matrix alone, so a row's bits do not change when the rows run in
    // sub-batches of more than kLinearGemmRows: a call whose scratch exceeds
    // the array runs in the fewest such sub-batches that fit it (with 64 MiB
    // every n up to 1024 fits: the plan needs at most 512 KiB per row).
    const size_t cap = (size_t)SRQ_NOALLOC_SCRATCH_BYTES;
    const size_t need = linear_scratch_bytes(*w, n);
    int32_t batches = 1;
    if (need > cap) {
        const size_t per_row = need / (size_t)n;
        const int32_t fit = (int32_t)(cap / per_row);
        batches = (n + fit - 1) / std::max<int32_t>(fit, 1);
        if (fit <= kLinearGemmRows || n / batches <= kLinearGemmRows)
            return fail(SRQ_EINVAL,
                        "srq_linear_noalloc: a %lld x %lld matrix needs %zu bytes of scratch per row, above what "
                        "the fixed %zu holds for %d rows (use srq_linear)",
                        (long long)w->rows, (long long)w->cols, per_row, cap, kLinearGemmRows + 1);
    }
    void *buf = g_noalloc_scratch[e->device];  // set when e's device was prepared
    if (!buf) return fail(SRQ_EDEVICE, "no-allocation scratch missing on device %d", e->device);
    DeviceGuard g(e->device);
    // Sub-batches of n / batches rows, the first n % batches one row more;
    // each is ordered after the previous one on the stream, so they share
    // the array.
    for (int32_t b = 0, r0 = 0; b < batches; ++b) {
        const int32_t cnt = n / batches + (b < n % batches ? 1 : 0);
        SRQ_CHECK(run_linear(e, e->ws, *w, x + (int64_t)r0 * w->cols, cnt, y + (int64_t)r0 * w->rows, w->rows,
                             nullptr, 0.0, nullptr, kLinearGemmRows, buf, cap));
        r0 += cnt;
    }
    return SRQ_OK;
}

// ------------------------------------------------------------------- model
int srq_model_create(srq_exec *e, const srq_model_config *c, const char *weight_format, srq_model **out) {
    if (!e || !c || !weight_format || !out) return fail(SRQ_EINVAL, "null pointer");
    *out = nullptr;
    std::string f(weight_format);
    if (f != "f32" && f != "q8" && f != "q4" && f != "q4-mixed")
        return fail(SRQ_EINVAL, "weight-format must be f32, q8, q4 or q4-mixed");
    if (c->vocab < 1 || c->dim < 2 || c->layers < 1 || c->heads < 1 || c->kv_heads < 1 || c->hidden < 1 ||
        c->context < 1 || c->context > 32768 || c->dim % c->heads || c->heads % c->kv_heads ||
        (c->dim / c->heads) % 2 || c->dim / c->heads > 256 || !(c->rope_theta > 1) || !(c->norm_eps >= 1e-12) ||
        !(c->norm_eps <= 1))
        return fail(SRQ_EINVAL, "invalid model configuration");
    DeviceGuard g(e->device);
    srq_model *m = new srq_model();
    m->device = e->device;
    m->e = e;
    e->refs++;
    m->c = *c;
    m->format = f;
    m->hd = c->dim / c->heads;
    m->kvdim = m->hd * c->kv_heads;
    const int fm = matrix_format(f, false), fe = matrix_format(f, true);
    const int64_t d = c->dim, kd = m->kvdim, H = c->hidden;
    int rc = alloc_weight(m, m->embed, fe, c->vocab, d);
    if (rc == SRQ_OK && !c->tied) {
        rc = alloc_weight(m, m->output, fe, c->vocab, d);
        m->has_output = true;
    }
    if (rc == SRQ_OK) rc = alloc_f32(m, &m->final_norm, d);
    m->L.resize(c->layers);
    for (int l = 0; l < c->layers && rc == SRQ_OK; ++l) {
        Layer &L = m->L[l];
        rc = alloc_weight(m, L.qkv, fm, d + 2 * kd, d);
        if (rc == SRQ_OK) rc = alloc_weight(m, L.o, fm, d, d);
        if (rc == SRQ_OK) rc = alloc_weight(m, L.gu, fm, 2 * H, d);
        if (rc == SRQ_OK) rc = alloc_weight(m, L.down, fm, d, H);
        if (rc == SRQ_OK) rc = alloc_f32(m, &L.n1, d);
        if (rc == SRQ_OK) rc = alloc_f32(m, &L.n2, d);
        if (rc == SRQ_OK && c->qkv_bias) rc = alloc_f32(m, &L.bias, d + 2 * kd);
        if (rc == SRQ_OK) {
            L.q = view_rows(L.qkv, 0, d);
            L.k = view_rows(L.qkv, d, kd);
            L.v = view_rows(L.qkv, d + kd, kd);
            L.gate = view_rows(L.gu, 0, H);
            L.up = view_rows(L.gu, H, H);
        }
    }
    // RoPE tables (M:5034-5043), computed once on the host as the reference
    // does at load time, then resident on the device.
    if (rc == SRQ_OK) {
        const int half = m->hd / 2;
        m->h_cos.resize((size_t)c->context * half);
        m->h_sin.resize((size_t)c->context * half);
        std::vector<float> inv(half);
        for (int j = 0; j < half; ++j) inv[j] = inverse_frequency(*c, m->hd, j);
        for (int p = 0; p < c->context; ++p)
            for (int j = 0; j < half; ++j) {
                volatile float prod = (float)p * inv[j];
                double angle = (double)prod;
                m->h_cos[(size_t)p * half + j] = (float)std::cos(angle);
                m->h_sin[(size_t)p * half + j] = (float)std::sin(angle);
            }
        const int64_t tbytes = (int64_t)c->context * half * 4;
        if (hipMalloc((void **)&m->cos_t, tbytes) != hipSuccess || hipMalloc((void **)&m->sin_t, tbytes) != hipSuccess)
            rc = fail(SRQ_ENOMEM, "RoPE table allocation failed");
        else {
            m->allocs.push_back(m->cos_t);
            m->allocs.push_back(m->sin_t);
            if (hipMemcpy(m->cos_t, m->h_cos.data(), tbytes, hipMemcpyHostToDevice) != hipSuccess ||
                hipMemcpy(m->sin_t, m->h_sin.data(), tbytes, hipMemcpyHostToDevice) != hipSuccess)
                rc = fail(SRQ_EDEVICE, "RoPE table upload failed");
        }
    }
    if (rc != SRQ_OK) {
        model_unref(m);
        return rc;
    }
    *out = m;
    return SRQ_OK;
}

static void model_unref(srq_model *m) {
    if (!m || --m->refs > 0) return;
    {
        DeviceGuard g(m->device);
        (void)hipDeviceSynchronize();
        for (void *p : m->allocs) (void)hipFree(p);
    }
    exec_unref(m->e);
    delete m;
}

int srq_model_destroy(srq_model *m) {
    model_unref(m);
    return SRQ_OK;
}

int srq_model_resident_bytes(const srq_model *m, int64_t *bytes) {
    if (!m || !bytes) return fail(SRQ_EINVAL, "null pointer");
    // RoPE tables are not weights: hfWeightLayoutFor counts parameters only.
    *bytes = m->resident;
    return SRQ_OK;
}

static srq_weight *model_matrix(srq_model *m, int kind, int layer) {
    if (kind == SRQ_T_EMBED) return &m->embed;
    if (kind == SRQ_T_OUTPUT) return m->has_output ? &m->output : nullptr;
    if (layer < 0 || layer >= m->c.layers) return nullptr;
    Layer &L = m->L[layer];
    switch (kind) {
        case SRQ_T_Q: return &L.q;
        case SRQ_T_K: return &L.k;
        case SRQ_T_V: return &L.v;
        case SRQ_T_O: return &L.o;
        case SRQ_T_GATE: return &L.gate;
        case SRQ_T_UP: return &L.up;
        case SRQ_T_DOWN: return &L.down;
    }
    return nullptr;
}

int srq_model_weight(srq_model *m, int kind, int layer, srq_weight **out) {
    if (!m || !out) return fail(SRQ_EINVAL, "null pointer");
    srq_weight *w = nullptr;
    if (kind == SRQ_T_QKV || kind == SRQ_T_GATE_UP) {
        // The fused storage the step streams (borrow only).
        if (layer >= 0 && layer < m->c.layers) w = kind == SRQ_T_QKV ? &m->L[layer].qkv : &m->L[layer].gu;
    } else {
        w = model_matrix(m, kind, layer);
    }
    if (!w) return fail(SRQ_EINVAL, "no matrix of kind %d at layer %d", kind, layer);
    *out = w;
    return SRQ_OK;
}

}  // extern "C"

namespace srq {
// srq_model_load without the join: the convert/pack kernels are queued on
// the executor's stream and a non-finite value sets error word 0.
int model_load_enqueue(srq_model *m, int kind, int layer, const void *src, int dtype) {
    if (!m || !src) return fail(SRQ_EINVAL, "null pointer");
    if (dtype < SRQ_SRC_F32 || dtype > SRQ_SRC_F16) return fail(SRQ_EINVAL, "bad source dtype");
    srq_exec *e = m->e;
    DeviceGuard g(m->device);
    const int64_t d = m->c.dim, kd = m->kvdim;
    float *vec = nullptr;
    int64_t count = 0;
    switch (kind) {
        case SRQ_T_FINAL_NORM: vec = m->final_norm, count = d; break;
        case SRQ_T_ATTN_NORM:
        case SRQ_T_FFN_NORM:
            if (layer < 0 || layer >= m->c.layers) return fail(SRQ_EINVAL, "layer %d out of range", layer);
            vec = kind == SRQ_T_ATTN_NORM ? m->L[layer].n1 : m->L[layer].n2;
            count = d;
            break;
        case SRQ_T_Q_BIAS:
        case SRQ_T_K_BIAS:
        case SRQ_T_V_BIAS:
            if (!m->c.qkv_bias) return fail(SRQ_EINVAL, "model has no q/k/v biases");
            if (layer < 0 || layer >= m->c.layers) return fail(SRQ_EINVAL, "layer %d out of range", layer);
            vec = m->L[layer].bias + (kind == SRQ_T_Q_BIAS ? 0 : kind == SRQ_T_K_BIAS ? d : d + kd);
            count = kind == SRQ_T_Q_BIAS ? d : kd;
            break;
        default: break;
    }
    if (vec) return launch_convert_f32(e->stream, count, src, dtype, vec, e->d_err);
    srq_weight *w = model_matrix(m, kind, layer);
    if (!w) return fail(SRQ_EINVAL, "no tensor of kind %d at layer %d", kind, layer);
    return fill_weight(e, *w, src, dtype);
}

const srq_model_config &model_config(const srq_model *m) { return m->c; }
int model_device(const srq_model *m) { return m->device; }
hipStream_t model_stream(const srq_model *m) { return m->e->stream; }
const int32_t *model_error_word(const srq_model *m) { return m->e->d_err; }
int model_join_nonfinite(srq_model *m, const char *what) {
    DeviceGuard g(m->device);
    return check_err_flag(m->e, SRQ_ENONFINITE, what);
}
}  // namespace srq

extern "C" {

int srq_model_load(srq_model *m, int kind, int layer, const void *src, srq_src_dtype dtype) {
    SRQ_CHECK(model_load_enqueue(m, kind, layer, src, dtype));
    return model_join_nonfinite(m, "non-finite HF weight");
}

// ---------------------------------------------------------- host sources
// readParam streams a tensor's values from host memory (M:857-880).  Here
// the source bytes travel through two pinned 16 MiB chunks into one device
// staging buffer -- the host copy of a chunk overlaps the transfer of the
// previous one -- and are then packed or converted on the device exactly
// as a device source is.  cancel (nullable) is polled between chunks.
namespace {
constexpr size_t kHostChunk = 16 << 20;

struct HostStage {
    hipStream_t stream = nullptr;
    void *dev = nullptr;
    void *slot[2] = {};
    hipEvent_t done[2] = {};
    ~HostStage() {
        if (stream) (void)hipStreamSynchronize(stream);
        if (dev) (void)hipFree(dev);
        for (int i = 0; i < 2; ++i) {
            if (slot[i]) (void)hipHostFree(slot[i]);
            if (done[i]) (void)hipEventDestroy(done[i]);
        }
    }
};

int stage_host(hipStream_t stream, const void *src, size_t bytes, const volatile int32_t *cancel, HostStage &hs) {
    hs.stream = stream;
    if (hipMalloc(&hs.dev, std::max<size_t>(bytes, 256)) != hipSuccess)
        return fail(SRQ_ENOMEM, "device staging of %zu bytes does not fit", bytes);
    const size_t slot_bytes = std::min(bytes, kHostChunk);
    for (int i = 0; i < 2 && slot_bytes > 0; ++i) {
        if (hipHostMalloc(&hs.slot[i], slot_bytes, hipHostMallocDefault) != hipSuccess)
            return fail(SRQ_ENOMEM, "pinned staging of %zu bytes failed", slot_bytes);
        SRQ_HIP(hipEventCreateWithFlags(&hs.done[i], hipEventDisableTiming));
    }
    bool used[2] = {false, false};
    int chunk = 0;
    for (size_t pos = 0; pos < bytes; pos += kHostChunk, ++chunk) {
        if (cancel && *cancel) return fail(SRQ_ECANCELED, "load canceled");
        const int k = chunk & 1;
        if (used[k] && hipEventSynchronize(hs.done[k]) != hipSuccess) return fail(SRQ_EDEVICE, "staging copy failed");
        const size_t len = std::min(kHostChunk, bytes - pos);
        memcpy(hs.slot[k], (const char *)src + pos, len);
        if (hipMemcpyAsync((char *)hs.dev + pos, hs.slot[k], len, hipMemcpyHostToDevice, stream) != hipSuccess ||
            hipEventRecord(hs.done[k], stream) != hipSuccess)
            return fail(SRQ_EDEVICE, "staging copy failed");
        used[k] = true;
    }
    return SRQ_OK;
}

size_t src_elem_bytes(int dtype) { return dtype == SRQ_SRC_F32 ? 4 : 2; }

// Element count of tensor (kind, layer) of m, or -1.
int64_t model_tensor_elems(srq_model *m, int kind, int layer) {
    const int64_t d = m->c.dim, kd = m->kvdim;
    const bool in_layer = layer >= 0 && layer < m->c.layers;
    switch (kind) {
        case SRQ_T_FINAL_NORM: return d;
        case SRQ_T_ATTN_NORM:
        case SRQ_T_FFN_NORM: return in_layer ? d : -1;
        case SRQ_T_Q_BIAS: return in_layer && m->c.qkv_bias ? d : -1;
        case SRQ_T_K_BIAS:
        case SRQ_T_V_BIAS: return in_layer && m->c.qkv_bias ? kd : -1;
        default: break;
    }
    const srq_weight *w = model_matrix(m, kind, layer);
    return w ? w->rows * w->cols : -1;
}
}  // namespace

int srq_pack_host(srq_exec *e, srq_format fmt, int64_t rows, int64_t cols, const void *src_host,
                  srq_src_dtype dtype, void *values, float *scales, const volatile int32_t *cancel) {
    if (!e || !src_host || !values || !scales) return fail(SRQ_EINVAL, "null pointer");
    if (fmt != SRQ_Q8 && fmt != SRQ_Q4) return fail(SRQ_EINVAL, "pack format must be Q8 or Q4");
    if (rows < 0 || cols < 0 || dtype < SRQ_SRC_F32 || dtype > SRQ_SRC_F16) return fail(SRQ_EINVAL, "bad shape or dtype");
    DeviceGuard g(e->device);
    HostStage hs;
    SRQ_CHECK(stage_host(e->stream, src_host, (size_t)(rows * cols) * src_elem_bytes(dtype), cancel, hs));
    SRQ_CHECK(launch_pack(e->stream, fmt, rows, cols, hs.dev, dtype, values, scales, e->d_err));
    return check_err_flag(e, SRQ_ENONFINITE, "non-finite weight in pack source");
}

int srq_weight_create_host(srq_exec *e, srq_format fmt, int64_t rows, int64_t cols, const void *src_host,
                           srq_src_dtype dtype, const volatile int32_t *cancel, srq_weight **out) {
    if (!e || !out || !src_host) return fail(SRQ_EINVAL, "null pointer");
    *out = nullptr;
    if (rows <= 0 || cols <= 0 || fmt < SRQ_F32 || fmt > SRQ_Q4 || dtype < SRQ_SRC_F32 || dtype > SRQ_SRC_F16)
        return fail(SRQ_EINVAL, "bad weight shape, format or dtype");
    DeviceGuard g(e->device);
    HostStage hs;
    SRQ_CHECK(stage_host(e->stream, src_host, (size_t)(rows * cols) * src_elem_bytes(dtype), cancel, hs));
    return srq_weight_create(e, fmt, rows, cols, hs.dev, dtype, out);
}

int srq_model_load_host(srq_model *m, int kind, int layer, const void *src_host, srq_src_dtype dtype,
                        const volatile int32_t *cancel) {
    if (!m || !src_host) return fail(SRQ_EINVAL, "null pointer");
    if (dtype < SRQ_SRC_F32 || dtype > SRQ_SRC_F16) return fail(SRQ_EINVAL, "bad source dtype");
    const int64_t count = model_tensor_elems(m, kind, layer);
    if (count < 0) return fail(SRQ_EINVAL, "no tensor of kind %d at layer %d", kind, layer);
    DeviceGuard g(m->device);
    HostStage hs;
    SRQ_CHECK(stage_host(m->e->stream, src_host, (size_t)count * src_elem_bytes(dtype), cancel, hs));
    SRQ_CHECK(model_load_enqueue(m, kind, layer, hs.dev, dtype));
    return model_join_nonfinite(m, "non-finite HF weight");
}

int srq_model_rope_tables(const srq_model *m, float *cos_out, float *sin_out) {
    if (!m || !cos_out || !sin_out) return fail(SRQ_EINVAL, "null pointer");
    memcpy(cos_out, m->h_cos.data(), m->h_cos.size() * 4);
    memcpy(sin_out, m->h_sin.data(), m->h_sin.size() * 4);
    return SRQ_OK;
}

// -------------------------------------------------------------------- pool
int srq_pool_create(srq_model *m, int32_t max_pages, srq_pool **out) {
    if (!m || !out) return fail(SRQ_EINVAL, "null pointer");
    *out = nullptr;
    if (max_pages < 1) return fail(SRQ_EINVAL, "pool needs at least one page");
    DeviceGuard g(m->device);
    srq_pool *p = new srq_pool();
    p->m = m;
    p->device = m->device;
    p->max_pages = max_pages;
    p->page_elems = (int64_t)2 * kPageTokens * m->kvdim * m->c.layers;
    const size_t bytes = (size_t)max_pages * p->page_elems * 4;
    if (hipMalloc((void **)&p->base, bytes) != hipSuccess) {
        delete p;
        return fail(SRQ_ENOMEM, "KV pool of %zu bytes does not fit", bytes);
    }
    if (hipMemset(p->base, 0, bytes) != hipSuccess) {
        (void)hipFree(p->base);
        delete p;
        return fail(SRQ_EDEVICE, "KV pool clear failed");
    }
    for (int32_t i = max_pages - 1; i >= 0; --i) p->free_list.push_back(i);
    m->refs++;
    *out = p;
    return SRQ_OK;
}

static void pool_unref(srq_pool *p) {
    if (!p || --p->refs > 0) return;
    {
        DeviceGuard g(p->device);
        (void)hipDeviceSynchronize();
        if (p->base) (void)hipFree(p->base);
    }
    model_unref(p->m);
    delete p;
}

int srq_pool_destroy(srq_pool *p) {
    pool_unref(p);
    return SRQ_OK;
}

int srq_cache_create(srq_pool *p, int32_t reserve_pages, srq_cache **out) {
    if (!p || !out) return fail(SRQ_EINVAL, "null pointer");
    *out = nullptr;
    const int32_t limit = (p->m->c.context + kPageTokens - 1) / kPageTokens;
    if (reserve_pages < 1 || reserve_pages > limit) return fail(SRQ_EINVAL, "reservation must be 1..%d pages", limit);
    if (p->reserved + reserve_pages > p->max_pages)
        return fail(SRQ_ENOSPC, "KV pool reservation exceeded: %d + %d > %d pages", p->reserved, reserve_pages,
                    p->max_pages);
    srq_cache *c = new srq_cache();
    c->p = p;
    c->reserve = reserve_pages;
    p->reserved += reserve_pages;
    p->refs++;
    *out = c;
    return SRQ_OK;
}

static void cache_unref(srq_cache *c) {
    if (!c || --c->refs > 0) return;
    for (int32_t pg : c->pages) c->p->free_list.push_back(pg);
    c->p->reserved -= c->reserve;
    pool_unref(c->p);
    delete c;
}

// Returns the cache's pages to its pool (Close, M:6044-6061) once no
// decoder uses it any more.
int srq_cache_destroy(srq_cache *c) {
    if (!c) return SRQ_OK;
    c->released = true;
    cache_unref(c);
    return SRQ_OK;
}

int srq_cache_pos(const srq_cache *c, int32_t *pos) {
    if (!c || !pos) return fail(SRQ_EINVAL, "null pointer");
    *pos = c->pos;
    return SRQ_OK;
}

int srq_cache_read(srq_exec *e, const srq_cache *c, int32_t layer, int32_t pos0, int32_t count, float *k, float *v) {
    if (!e || !c || (count > 0 && (!k || !v))) return fail(SRQ_EINVAL, "null pointer");
    srq_model *m = c->p->m;
    if (layer < 0 || layer >= m->c.layers || pos0 < 0 || count < 0 ||
        (int64_t)pos0 + count > (int64_t)c->pages.size() * kPageTokens)
        return fail(SRQ_EINVAL, "KV rows outside the cache's pages");
    DeviceGuard g(e->device);
    const int64_t kd = m->kvdim;
    for (int32_t i = 0; i < count; ++i) {
        const int32_t pos = pos0 + i;
        const float *base = c->p->base + (int64_t)c->pages[pos / kPageTokens] * c->p->page_elems +
                            (int64_t)layer * 2 * kPageTokens * kd + (int64_t)(pos % kPageTokens) * kd;
        SRQ_HIP(hipMemcpyAsync(k + i * kd, base, kd * 4, hipMemcpyDeviceToHost, e->stream));
        SRQ_HIP(hipMemcpyAsync(v + i * kd, base + kPageTokens * kd, kd * 4, hipMemcpyDeviceToHost, e->stream));
    }
    SRQ_HIP(hipStreamSynchronize(e->stream));
    return SRQ_OK;
}

}  // extern "C"

// -------------------------------------------------------------------- step
namespace {

// Validation of prefillSelected (M:6246-6339) without mutating anything.
int validate_step(srq_model *m, int32_t sessions, srq_cache *const *caches, const int32_t *lens, const int32_t *tokens,
                  int32_t *n_out, int32_t *max_pos) {
    if (sessions < 1 || sessions > 256 || !caches || !lens || !tokens)
        return fail(SRQ_EINVAL, "invalid prefill batch (1..256 sessions)");
    int32_t n = 0, mp = 0;
    std::vector<const srq_cache *> seen;
    std::vector<std::pair<srq_pool *, int32_t>> need;
    for (int32_t i = 0; i < sessions; ++i) {
        const srq_cache *c = caches[i];
        if (!c || c->released || c->p->m != m || std::find(seen.begin(), seen.end(), c) != seen.end())
            return fail(SRQ_EINVAL, "foreign, stale, released, or duplicate KV cache");
        if (c->busy) return fail(SRQ_EINVAL, "KV cache is owned by a live decoder");
        seen.push_back(c);
        const int32_t len = lens[i];
        if (len < 1 || len > 1024 - n)
            return fail(SRQ_EINVAL, "prefill requires nonempty chunks totaling at most 1024 tokens");
        if (c->pos < 0 || c->pos > m->c.context || len > m->c.context - c->pos)
            return fail(SRQ_ERANGE, "KV cache context exhausted or invalid position");
        for (int32_t j = 0; j < len; ++j)
            if (tokens[n + j] < 0 || tokens[n + j] >= m->c.vocab) return fail(SRQ_EINVAL, "token outside vocabulary");
        const int32_t end = c->pos + len;
        const int32_t pages = (end + kPageTokens - 1) / kPageTokens;
        if (pages > c->reserve) return fail(SRQ_ENOSPC, "insufficient KV page reservation");
        const int32_t extra = std::max<int32_t>(0, pages - (int32_t)c->pages.size());
        bool found = false;
        for (auto &pr : need)
            if (pr.first == c->p) pr.second += extra, found = true;
        if (!found) need.push_back({c->p, extra});
        n += len;
        mp = std::max(mp, end);
    }
    for (auto &pr : need)
        if (pr.second > (int32_t)pr.first->free_list.size()) return fail(SRQ_ENOSPC, "insufficient KV page reservation");
    *n_out = n;
    *max_pos = mp;
    return SRQ_OK;
}

struct StepMeta {
    int32_t *tokens, *pos, *sess, *pages, *sel, *expand;
    int32_t pt_stride;
    int32_t *tiles = nullptr;  // query tiles {first row, rows} (AttnArgs::tiles)
    int32_t ntiles = 0;
    bool plan_ready = false;   // the row plan in ws.PLAN is already current (decoder)
    bool one_sess = false;     // every row belongs to session 0 (RowMeta::one_sess)
};

// Layout of the packed metadata buffer (device and pinned host mirror): at
// most n query tiles follow the per-session tables.
size_t meta_words(int32_t n, int32_t sessions, int32_t pt_stride) {
    return (size_t)n * 5 + (size_t)sessions * pt_stride + (size_t)sessions * 2;
}

StepMeta carve(int32_t *base, int32_t n, int32_t sessions, int32_t pt_stride) {
    StepMeta s;
    s.tokens = base;
    s.pos = base + n;
    s.sess = base + 2 * n;
    s.pages = base + 3 * n;
    s.sel = s.pages + (size_t)sessions * pt_stride;
    s.expand = s.sel + sessions;
    s.tiles = s.expand + sessions;
    s.pt_stride = pt_stride;
    return s;
}

int ensure_host_meta(srq_exec *e, size_t words) {
    if (words <= e->h_meta_n) return SRQ_OK;
    if (e->h_meta) {
        SRQ_HIP(hipStreamSynchronize(e->stream));
        (void)hipHostFree(e->h_meta);
        e->h_meta = nullptr;
    }
    size_t want = std::max<size_t>(words, 4096);
    if (hipHostMalloc((void **)&e->h_meta, want * 4) != hipSuccess) return fail(SRQ_ENOMEM, "pinned allocation failed");
    e->h_meta_n = want;
    return SRQ_OK;
}

// In-flight cancellation (the reference checks its context as each layer
// starts, M:6376-6378): with a cancel flag the host stays at most
// kLayerWindow layers ahead of the device, polling the flag while it waits
// for the layers kLayerWindow back to finish (and checking it as every layer
// is enqueued), so a flag raised during a step stops it within about
// kLayerWindow + kEventEvery layers.  Without a flag everything is enqueued
// at once.
// Progress is an event every kEventEvery layers: an event per layer (a
// marker packet the GPU processes between kernels, about 1.5 us) made a
// one-row 7B decode step 3.5-3.9% slower with a flag than without one;
// every fourth layer costs 0.4%.
constexpr int kLayerWindow = 8;
constexpr int kEventEvery = 4;  // layers per progress event
static_assert(kLayerWindow / kEventEvery == sizeof(srq_exec::layer_done) / sizeof(hipEvent_t),
              "one event per group of the window");

static int wait_layer(hipEvent_t ev, const volatile int32_t *cancel) {
    // Poll without sleeping for the first 200 us (a layer of a small step
    // ends within that), then sleep between polls.
    const auto t0 = std::chrono::steady_clock::now();
    for (;;) {
        const hipError_t q = hipEventQuery(ev);
        if (q == hipSuccess) return SRQ_OK;
        if (q != hipErrorNotReady) return fail(SRQ_EDEVICE, "layer wait failed: %s", hipGetErrorString(q));
        if (*cancel) return fail(SRQ_ECANCELED, "context canceled");
        if (std::chrono::steady_clock::now() - t0 > std::chrono::microseconds(200))
            std::this_thread::sleep_for(std::chrono::microseconds(20));
    }
}

// Enqueue the layers of one step for n rows whose metadata is on device.
int enqueue_layers(srq_exec *e, Workspace &ws, srq_model *m, srq_pool *pool, int32_t n, int32_t max_len,
                   const StepMeta &dm, const volatile int32_t *cancel) {
    const srq_model_config &c = m->c;
    const int64_t d = c.dim, kd = m->kvdim, H = c.hidden;
    float *X = as<float>(ws.X), *N = as<float>(ws.N), *Q = as<float>(ws.Q), *A = as<float>(ws.A);
    float *Hh = as<float>(ws.H), *W2 = as<float>(ws.W2);
    const bool use_gemm = n > kStepGemmRows && gemm_ok(m->L[0].qkv.fmt, d) && gemm_ok(m->L[0].down.fmt, H);
    int64_t *kvoff = nullptr;
    float *rope_cs = nullptr;
    if (!use_gemm) {
        // Row plan once per step: KV offsets and RoPE rows for the fused
        // q/k/v epilogue (ws.PLAN is sized by ensure_workspace).
        kvoff = as<int64_t>(ws.PLAN);
        rope_cs = (float *)(kvoff + n);
        if (!dm.plan_ready) {
            RowMeta meta0 = make_meta(e, m, 0, dm.pt_stride, dm.pos, dm.sess, dm.pages, pool);
            SRQ_CHECK(launch_row_plan(e->stream, meta0, n, (int32_t)kd, m->hd, m->cos_t, m->sin_t, kvoff, rope_cs));
        }
    }
    // Batch rows per fused launch: q/k/v (norm, RoPE rows, bias) and gate/up (norm).
    const int nbq = gemv_max_rows(m->L[0].qkv.fmt, d, true, 8 * (int64_t)m->hd + (m->L[0].bias ? d + 2 * kd : 0));
    const int nbg = gemv_max_rows(m->L[0].gu.fmt, d, true, 0);
    if (nbq < 1 || nbg < 1) return fail(SRQ_EINVAL, "model width %lld exceeds the GEMV staging limit", (long long)d);
    if (cancel)
        for (hipEvent_t &ev : e->layer_done)
            if (!ev) SRQ_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    for (int l = 0; l < c.layers; ++l) {
        // before layer l of a group, wait for the group kLayerWindow layers back
        constexpr int kSlots = kLayerWindow / kEventEvery;
        if (cancel && l >= kLayerWindow && l % kEventEvery == 0)
            SRQ_CHECK(wait_layer(e->layer_done[((l - kLayerWindow) / kEventEvery) % kSlots], cancel));
        if (cancel && *cancel) return fail(SRQ_ECANCELED, "context canceled");
        Layer &L = m->L[l];
        RowMeta meta = make_meta(e, m, l, dm.pt_stride, dm.pos, dm.sess, dm.pages, pool);
        meta.kvoff = kvoff;
        meta.rope_cs = rope_cs;
        meta.one_sess = dm.one_sess ? 1 : 0;
        if (!use_gemm) {
            for (int32_t r0 = 0; r0 < n; r0 += nbq) {
                GemvArgs a{};
                a.fmt = L.qkv.fmt;
                a.values = L.qkv.values;
                a.scales = L.qkv.scales;
                a.rows = L.qkv.rows;
                a.cols = d;
                a.x = X + r0 * d;
                a.n = std::min(nbq, n - r0);
                a.row0 = r0;
                a.norm_w = L.n1;
                a.norm_eps = c.norm_eps;
                a.y = Q + r0 * d;
                a.y_stride = d;
                a.epilogue = EPI_ROPE_KV;
                a.dim = (int32_t)d;
                a.kvdim = (int32_t)kd;
                a.head_dim = m->hd;
                a.cos_t = m->cos_t;
                a.sin_t = m->sin_t;
                a.bias = L.bias;
                a.meta = meta;
                SRQ_CHECK(launch_gemv(e->stream, a));
            }
        } else {
            // N holds RMSNorm(X, n1) already when the previous layer's down
            // projection wrote it from its reduction.
            if (l == 0) SRQ_CHECK(launch_rmsnorm(e->stream, X, L.n1, N, n, (int32_t)d, c.norm_eps));
            // q/k/v GEMM with bias, RoPE and the KV write in its reduction.
            SRQ_CHECK(ensure(ws.flags, gemm_scratch_bytes(L.qkv.fmt, n, L.qkv.rows, L.qkv.cols), e->stream));
            GemmArgs g{L.qkv.fmt, L.qkv.values, L.qkv.scales, L.qkv.rows, L.qkv.cols, N, n, W2, d + 2 * kd,
                       nullptr, nullptr};
            g.rope = GemmRope{Q, L.bias, (int32_t)d, (int32_t)kd, m->hd, m->cos_t, m->sin_t, meta};
            SRQ_CHECK(launch_gemm(e->stream, g, ws.flags.p, ws.flags.n));
        }
        AttnArgs at{};
        at.q = Q;
        at.out = A;
        at.n = n;
        at.heads = c.heads;
        at.kv_heads = c.kv_heads;
        at.head_dim = m->hd;
        at.max_len = max_len;
        at.meta = meta;
        at.tiles = dm.tiles;
        at.ntiles = dm.ntiles;
        SRQ_CHECK(launch_attention(e->stream, at, as<float>(ws.ATT), as<int32_t>(ws.ATTC)));
        // O projection + residual (M:6398-6400).
        if (!use_gemm) {
            SRQ_CHECK(run_linear(e, ws, L.o, A, n, X, d, nullptr, 0.0, X, kStepGemmRows));
        } else {
            // with RMSNorm(X, n2) -> N in its reduction
            SRQ_CHECK(ensure(ws.flags, gemm_scratch_bytes(L.o.fmt, n, L.o.rows, L.o.cols), e->stream));
            GemmArgs g{L.o.fmt, L.o.values, L.o.scales, L.o.rows, L.o.cols, A, n, X, d, X, nullptr};
            g.norm_w = L.n2;
            g.norm_eps = c.norm_eps;
            g.norm_out = N;
            SRQ_CHECK(launch_gemm(e->stream, g, ws.flags.p, ws.flags.n));
        }
        if (!use_gemm) {
            for (int32_t r0 = 0; r0 < n; r0 += nbg) {
                GemvArgs a{};
                a.fmt = L.gu.fmt;
                a.values = L.gu.values;
                a.scales = L.gu.scales;
                a.rows = 2 * H;
                a.cols = d;
                a.x = X + r0 * d;
                a.n = std::min(nbg, n - r0);
                a.row0 = r0;
                a.norm_w = L.n2;
                a.norm_eps = c.norm_eps;
                a.y = Hh + r0 * H;
                a.y_stride = H;
                a.epilogue = EPI_SWIGLU;
                SRQ_CHECK(launch_gemv(e->stream, a));
            }
        } else {
            // gate/up GEMM with SwiGLU in its split-K reduction (W2 is only
            // a temporary when K is not split).
            SRQ_CHECK(ensure(ws.flags, gemm_scratch_bytes(L.gu.fmt, n, L.gu.rows, L.gu.cols), e->stream));
            GemmArgs g{L.gu.fmt, L.gu.values, L.gu.scales, L.gu.rows, L.gu.cols, N, n, W2, 2 * H, nullptr, Hh};
            SRQ_CHECK(launch_gemm(e->stream, g, ws.flags.p, ws.flags.n));
        }
        // down + residual (M:6415-6417).
        if (!use_gemm || l + 1 == c.layers) {
            SRQ_CHECK(run_linear(e, ws, L.down, Hh, n, X, d, nullptr, 0.0, X, kStepGemmRows));
        } else {
            // with the next layer's RMSNorm(X, n1) -> N in its reduction
            SRQ_CHECK(ensure(ws.flags, gemm_scratch_bytes(L.down.fmt, n, L.down.rows, L.down.cols), e->stream));
            GemmArgs g{L.down.fmt, L.down.values, L.down.scales, L.down.rows, L.down.cols, Hh, n, X, d, X, nullptr};
            g.norm_w = m->L[l + 1].n1;
            g.norm_eps = c.norm_eps;
            g.norm_out = N;
            SRQ_CHECK(launch_gemm(e->stream, g, ws.flags.p, ws.flags.n));
        }
        if (cancel && (l + 1) % kEventEvery == 0)
            SRQ_HIP(hipEventRecord(e->layer_done[(l / kEventEvery) % kSlots], e->stream));
    }
    return SRQ_OK;
}

// Final norm + head on `heads` compacted rows (already in T) -> LOGC.
int enqueue_head(srq_exec *e, Workspace &ws, srq_model *m, const float *rows, int32_t heads) {
    const srq_weight &head = m->has_output ? m->output : m->embed;
    float *N = as<float>(ws.N), *LOGC = as<float>(ws.LOGC);
    if (heads > kStepGemmRows && gemm_ok(head.fmt, m->c.dim)) {
        SRQ_CHECK(launch_rmsnorm(e->stream, rows, m->final_norm, N, heads, m->c.dim, m->c.norm_eps));
        return run_linear(e, ws, head, N, heads, LOGC, m->c.vocab, nullptr, 0.0, nullptr, kStepGemmRows);
    }
    return run_linear(e, ws, head, rows, heads, LOGC, m->c.vocab, m->final_norm, m->c.norm_eps, nullptr);
}

int ensure_workspace(srq_exec *e, Workspace &ws, srq_model *m, int32_t n, int32_t sessions, int32_t max_len) {
    const int64_t d = m->c.dim, kd = m->kvdim, H = m->c.hidden, V = m->c.vocab;
    const size_t nd = (size_t)n * d * 4;
    SRQ_CHECK(ensure(ws.X, nd, e->stream));
    SRQ_CHECK(ensure(ws.N, nd, e->stream));
    SRQ_CHECK(ensure(ws.Q, nd, e->stream));
    SRQ_CHECK(ensure(ws.A, nd, e->stream));
    SRQ_CHECK(ensure(ws.T, (size_t)std::max<int64_t>(n, sessions) * d * 4, e->stream));
    SRQ_CHECK(ensure(ws.H, (size_t)n * H * 4, e->stream));
    SRQ_CHECK(ensure(ws.W2, (size_t)n * std::max<int64_t>(d + 2 * kd, 2 * H) * 4, e->stream));
    SRQ_CHECK(ensure(ws.LOGC, (size_t)sessions * V * 4, e->stream));
    SRQ_CHECK(ensure(ws.LOG, (size_t)sessions * V * 4, e->stream));
    SRQ_CHECK(ensure(ws.ATT, attention_scratch_bytes(n, m->c.heads, m->hd, max_len), e->stream));
    SRQ_CHECK(ensure(ws.PLAN, (size_t)n * 8 + (size_t)n * m->hd * 4, e->stream));
    // Attention merge counters start at zero; the kernels leave them zero.
    const size_t cbytes = (size_t)n * m->c.heads * 4;
    if (cbytes > ws.ATTC.n) {
        SRQ_CHECK(ensure(ws.ATTC, cbytes, e->stream));
        SRQ_CHECK(launch_zero(e->stream, as<int32_t>(ws.ATTC), (int64_t)(ws.ATTC.n / 4)));
    }
    return SRQ_OK;
}

}  // namespace

extern "C" int srq_step(srq_exec *e, srq_model *m, int32_t sessions, srq_cache *const *caches,
                        const int32_t *chunk_lens, const int32_t *tokens, const uint8_t *want, float **logits,
                        float *logits_host, const volatile int32_t *cancel) {
    if (!e || !m) return fail(SRQ_EINVAL, "null executor or model");
    if (logits) *logits = nullptr;
    if (cancel && *cancel) return fail(SRQ_ECANCELED, "context canceled");
    int32_t n = 0, max_pos = 0;
    SRQ_CHECK(validate_step(m, sessions, caches, chunk_lens, tokens, &n, &max_pos));
    DeviceGuard g(e->device);
    srq_pool *pool = caches[0]->p;
    for (int32_t i = 1; i < sessions; ++i)
        if (caches[i]->p != pool) return fail(SRQ_EINVAL, "sessions of one step must share a KV pool");
    Workspace &ws = e->ws;
    SRQ_CHECK(ensure_workspace(e, ws, m, n, sessions, max_pos));
    const int32_t pt_stride = (m->c.context + kPageTokens - 1) / kPageTokens;
    const size_t words = meta_words(n, sessions, pt_stride);
    SRQ_CHECK(ensure(ws.meta, words * 4, e->stream));
    SRQ_CHECK(ensure_host_meta(e, words));
    SRQ_HIP(hipStreamSynchronize(e->stream));  // the pinned staging may still feed a copy

    // Acquire pages (validation proved they exist), then fill metadata.
    for (int32_t i = 0; i < sessions; ++i) {
        srq_cache *c = caches[i];
        const int32_t pages = (c->pos + chunk_lens[i] + kPageTokens - 1) / kPageTokens;
        while ((int32_t)c->pages.size() < pages) {
            c->pages.push_back(pool->free_list.back());
            pool->free_list.pop_back();
        }
    }
    StepMeta hm = carve(e->h_meta, n, sessions, pt_stride);
    std::vector<int32_t> last_rows(sessions);
    int32_t r = 0, ntiles = 0;
    for (int32_t i = 0; i < sessions; ++i) {
        // Query tiles: up to kAttnTileRows consecutive rows of this session.
        for (int32_t t0 = 0; t0 < chunk_lens[i]; t0 += kAttnTileRows) {
            hm.tiles[2 * ntiles] = r + t0;
            hm.tiles[2 * ntiles + 1] = std::min<int32_t>(kAttnTileRows, chunk_lens[i] - t0);
            ++ntiles;
        }
        for (int32_t j = 0; j < chunk_lens[i]; ++j, ++r) {
            hm.tokens[r] = tokens[r];
            hm.pos[r] = caches[i]->pos + j;
            hm.sess[r] = i;
        }
        last_rows[i] = r - 1;
        int32_t *pt = hm.pages + (size_t)i * pt_stride;
        for (int32_t p = 0; p < pt_stride; ++p) pt[p] = p < (int32_t)caches[i]->pages.size() ? caches[i]->pages[p] : 0;
    }
    int32_t heads = 0;
    for (int32_t i = 0; i < sessions; ++i) {
        if (!want || want[i]) {
            hm.sel[heads] = last_rows[i];
            hm.expand[i] = heads++;
        } else {
            hm.expand[i] = -1;
        }
    }
    SRQ_HIP(hipMemcpyAsync(ws.meta.p, e->h_meta, words * 4, hipMemcpyHostToDevice, e->stream));
    StepMeta dm = carve(as<int32_t>(ws.meta), n, sessions, pt_stride);
    dm.one_sess = sessions == 1;
    dm.ntiles = ntiles;

    // Embedding rows (copyRow, M:6364-6375).
    SRQ_CHECK(launch_dequant_rows(e->stream, m->embed.fmt, m->c.dim, m->embed.values, m->embed.scales, dm.tokens, n,
                                  as<float>(ws.X)));
    int rc = enqueue_layers(e, ws, m, pool, n, max_pos, dm, cancel);
    if (rc == SRQ_OK && heads > 0) {
        rc = launch_gather_rows(e->stream, as<float>(ws.X), m->c.dim, dm.sel, heads, as<float>(ws.T));
        if (rc == SRQ_OK) rc = enqueue_head(e, ws, m, as<float>(ws.T), heads);
    }
    float *out = as<float>(ws.LOGC);
    if (rc == SRQ_OK && want) {
        rc = launch_gather_rows(e->stream, as<float>(ws.LOGC), m->c.vocab, dm.expand, sessions, as<float>(ws.LOG));
        out = as<float>(ws.LOG);
    }
    // With neither a host copy nor a cancel flag the step returns queued:
    // the executor's later calls run after it on the same stream.
    const bool queued = !logits_host && !cancel;
    hipError_t he = queued ? hipSuccess : hipStreamSynchronize(e->stream);
    if (rc != SRQ_OK) return rc;
    if (he != hipSuccess) return fail(SRQ_EDEVICE, "step failed: %s", hipGetErrorString(he));
    if (cancel && *cancel) return fail(SRQ_ECANCELED, "context canceled");
    if (logits_host)
        SRQ_HIP(hipMemcpy(logits_host, out, (size_t)sessions * m->c.vocab * 4, hipMemcpyDeviceToHost));
    for (int32_t i = 0; i < sessions; ++i) caches[i]->pos += chunk_lens[i];
    if (logits) *logits = out;
    return SRQ_OK;
}

extern "C" int srq_argmax(srq_exec *e, const float *logits, int32_t rows, int32_t vocab, int32_t *ids) {
    if (!e || !logits || !ids) return fail(SRQ_EINVAL, "null pointer");
    if (rows < 1 || vocab < 1) return fail(SRQ_EINVAL, "empty logits");
    DeviceGuard g(e->device);
    SRQ_CHECK(ensure(e->ws.flags, sizeof(int32_t) * (size_t)rows, e->stream));
    SRQ_CHECK(launch_argmax(e->stream, logits, rows, vocab, as<int32_t>(e->ws.flags), e->d_err));
    SRQ_HIP(hipMemcpyAsync(ids, e->ws.flags.p, sizeof(int32_t) * rows, hipMemcpyDeviceToHost, e->stream));
    return check_err_flag(e, SRQ_ENONFINITE, "non-finite HF logits");
}

extern "C" int srq_sample(srq_exec *e, const float *logits, int32_t rows, const int32_t *row_ids, int32_t vocab,
                          const srq_sampling *params, const int32_t *history, const int32_t *history_len,
                          int32_t history_stride, const int32_t *blocked, uint64_t *rng_state, int32_t *ids) {
    if (!e || !logits || !params || !rng_state || !ids) return fail(SRQ_EINVAL, "null pointer");
    if (rows < 1 || vocab < 1) return fail(SRQ_EINVAL, "empty logits");
    if (!(params->temperature >= 0) || !(params->repeat_penalty > 0) || params->top_k < 0 || !(params->top_p > 0))
        return fail(SRQ_EINVAL, "bad sampling parameters");
    if (history && (!history_len || history_stride < 0)) return fail(SRQ_EINVAL, "history without lengths");
    for (int32_t r = 0; history && r < rows; ++r)
        if (history_len[r] < 0 || history_len[r] > history_stride) return fail(SRQ_EINVAL, "bad history length");
    for (int32_t r = 0; row_ids && r < rows; ++r)
        if (row_ids[r] < 0) return fail(SRQ_EINVAL, "negative logits row");
    DeviceGuard g(e->device);
    Workspace &ws = e->ws;
    const size_t hist_words = history ? (size_t)rows * history_stride : 0;
    // [rng: 2*rows][ids: rows][blocked: rows][history_len: rows][row_ids: rows][history]
    const size_t words = (size_t)rows * 6 + hist_words;
    SRQ_CHECK(ensure(ws.SMP, words * 4, e->stream));
    SRQ_CHECK(ensure(ws.SMPS, sample_scratch_bytes(rows, vocab), e->stream));
    int32_t *d = as<int32_t>(ws.SMP);
    uint64_t *d_rng = (uint64_t *)d;
    int32_t *d_ids = d + 2 * rows, *d_blk = d + 3 * rows, *d_hl = d + 4 * rows, *d_rows = d + 5 * rows;
    int32_t *d_hist = d + 6 * rows;
    // The per-row words go through a pinned staging buffer of their own (a
    // queued step may still be copying the metadata buffer; the previous
    // sampling call ended synchronised) as one copy each way: copies from
    // pageable memory would each stage and wait on their own.
    if ((size_t)rows * 6 > e->h_smp_n) {
        if (e->h_smp) (void)hipHostFree(e->h_smp);
        e->h_smp = nullptr;
        e->h_smp_n = 0;
        const size_t want = std::max<size_t>((size_t)rows * 6, 1536);
        if (hipHostMalloc((void **)&e->h_smp, want * 4) != hipSuccess) return fail(SRQ_ENOMEM, "pinned allocation failed");
        e->h_smp_n = want;
    }
    int32_t *h = e->h_smp;
    std::memcpy(h, rng_state, (size_t)rows * 8);
    for (int32_t r = 0; r < rows; ++r) {
        h[3 * rows + r] = blocked ? blocked[r] : 0;
        h[4 * rows + r] = history ? history_len[r] : 0;
        h[5 * rows + r] = row_ids ? row_ids[r] : 0;
    }
    SRQ_HIP(hipMemcpyAsync(d, h, (size_t)rows * 6 * 4, hipMemcpyHostToDevice, e->stream));
    if (hist_words) SRQ_HIP(hipMemcpyAsync(d_hist, history, hist_words * 4, hipMemcpyHostToDevice, e->stream));
    SampleArgs a{};
    a.logits = logits;
    a.row_ids = row_ids ? d_rows : nullptr;
    a.rows = rows;
    a.vocab = vocab;
    a.temperature = params->temperature;
    a.top_k = params->top_k;
    a.top_p = params->top_p;
    a.repeat_penalty = params->repeat_penalty;
    a.history = history ? d_hist : nullptr;
    a.history_len = history ? d_hl : nullptr;
    a.history_stride = history_stride;
    a.blocked = blocked ? d_blk : nullptr;
    a.rng = d_rng;
    a.ids = d_ids;
    a.err = e->d_err;
    SRQ_CHECK(launch_sample(e->stream, a, ws.SMPS.p));
    // [rng: 2*rows][ids: rows] back in one copy
    SRQ_HIP(hipMemcpyAsync(h, d, (size_t)rows * 3 * 4, hipMemcpyDeviceToHost, e->stream));
    SRQ_HIP(hipMemcpyAsync(e->h_err, e->d_err, sizeof(int32_t) * 4, hipMemcpyDeviceToHost, e->stream));
    SRQ_HIP(hipStreamSynchronize(e->stream));
    std::memcpy(rng_state, h, (size_t)rows * 8);
    std::memcpy(ids, h + 2 * rows, (size_t)rows * 4);
    const int32_t err = e->h_err[0];
    if (err) {
        SRQ_HIP(hipMemsetAsync(e->d_err, 0, sizeof(int32_t) * 4, e->stream));
        SRQ_HIP(hipStreamSynchronize(e->stream));
        if (err & 1) return fail(SRQ_ENONFINITE, "non-finite logits");
        if (err & 2) return fail(SRQ_EINVAL, "no candidate token");
        return fail(SRQ_EINVAL, "sampling selection limit exceeded (more than 2048 equal-ranked candidates)");
    }
    return SRQ_OK;
}

// ----------------------------------------------------------- greedy decoder
struct srq_decoder {
    srq_exec *e = nullptr;
    srq_model *m = nullptr;
    srq_cache *c = nullptr;
    int32_t start_pos = 0, max_steps = 0, steps = 0;
    int32_t *dbuf = nullptr;  // pos, sess, counter, embed_id, token, err, pages[pt], out[max]
    int32_t pt_stride = 0;
    Workspace ws;             // private: the captured graph points into it
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    bool eager = false;
};

extern "C" {

int srq_decoder_destroy(srq_decoder *d);

// The first step's input: the embedding row of the first token and the row
// plan of its position.  Every step's tail then prepares the next one's.
static int enqueue_decode_input(srq_decoder *d) {
    srq_exec *e = d->e;
    srq_model *m = d->m;
    int32_t *pos = d->dbuf, *sess = d->dbuf + 1, *embed_id = d->dbuf + 3, *pt = d->dbuf + 6;
    Workspace &ws = d->ws;
    SRQ_CHECK(launch_dequant_rows(e->stream, m->embed.fmt, m->c.dim, m->embed.values, m->embed.scales, embed_id, 1,
                                  as<float>(ws.X)));
    int64_t *kvoff = as<int64_t>(ws.PLAN);
    RowMeta meta0 = make_meta(e, m, 0, d->pt_stride, pos, sess, pt, d->c->p);
    return launch_row_plan(e->stream, meta0, 1, (int32_t)m->kvdim, m->hd, m->cos_t, m->sin_t, kvoff,
                           (float *)(kvoff + 1));
}

// One step: layers -> final norm + head -> the tail (argmax, advance, the
// next step's embedding row and row plan).
static int enqueue_decode_step(srq_decoder *d) {
    srq_exec *e = d->e;
    srq_model *m = d->m;
    StepMeta dm{};
    int32_t *pos = d->dbuf, *sess = d->dbuf + 1, *counter = d->dbuf + 2, *embed_id = d->dbuf + 3;
    int32_t *token = d->dbuf + 4, *err = d->dbuf + 5, *pt = d->dbuf + 6, *outbuf = d->dbuf + 6 + d->pt_stride;
    dm.pos = pos;
    dm.sess = sess;
    dm.pages = pt;
    dm.pt_stride = d->pt_stride;
    dm.plan_ready = true;
    dm.one_sess = true;  // the decoder's one session is session 0
    Workspace &ws = d->ws;
    SRQ_CHECK(enqueue_layers(e, ws, m, d->c->p, 1, d->start_pos + d->max_steps, dm, nullptr));
    SRQ_CHECK(enqueue_head(e, ws, m, as<float>(ws.X), 1));
    const RowMeta meta0 = make_meta(e, m, 0, d->pt_stride, pos, sess, pt, d->c->p);
    DecodeTailArgs t{};
    t.logits = as<float>(ws.LOGC);
    t.vocab = m->c.vocab;
    t.token = token;
    t.err = err;
    t.pos = pos;
    t.out = outbuf;
    t.counter = counter;
    t.embed_id = embed_id;
    t.steps = d->max_steps;
    t.fmt = m->embed.fmt;
    t.values = m->embed.values;
    t.scales = m->embed.scales;
    t.dim = m->c.dim;
    t.x = as<float>(ws.X);
    t.sess = sess;
    t.pages = pt;
    t.pt_stride = d->pt_stride;
    t.page_elems = meta0.page_elems;
    t.kvdim = (int32_t)m->kvdim;
    t.half = m->hd / 2;
    t.cos_t = m->cos_t;
    t.sin_t = m->sin_t;
    t.kvoff = as<int64_t>(ws.PLAN);
    t.rope_cs = (float *)(t.kvoff + 1);
    return launch_decode_tail(e->stream, t);
}

int srq_decoder_create(srq_exec *e, srq_model *m, srq_cache *c, int32_t first_token, int32_t max_steps,
                       int32_t flags, srq_decoder **out) {
    if (!e || !m || !c || !out) return fail(SRQ_EINVAL, "null pointer");
    *out = nullptr;
    if (c->released || c->p->m != m) return fail(SRQ_EINVAL, "foreign or released KV cache");
    if (c->busy) return fail(SRQ_EINVAL, "KV cache is owned by a live decoder");
    if (first_token < 0 || first_token >= m->c.vocab) return fail(SRQ_EINVAL, "token outside vocabulary");
    if (max_steps < 1 || max_steps > m->c.context - c->pos) return fail(SRQ_ERANGE, "KV cache context exhausted");
    const int32_t end = c->pos + max_steps;
    const int32_t pages = (end + kPageTokens - 1) / kPageTokens;
    if (pages > c->reserve || pages - (int32_t)c->pages.size() > (int32_t)c->p->free_list.size())
        return fail(SRQ_ENOSPC, "insufficient KV page reservation");
    DeviceGuard g(e->device);
    srq_decoder *d = new srq_decoder();
    d->e = e;
    d->m = m;
    d->c = c;
    e->refs++;
    m->refs++;
    c->refs++;
    d->start_pos = c->pos;
    d->max_steps = max_steps;
    c->busy = true;
    d->pt_stride = (m->c.context + kPageTokens - 1) / kPageTokens;
    while ((int32_t)c->pages.size() < pages) {
        c->pages.push_back(c->p->free_list.back());
        c->p->free_list.pop_back();
    }
    const size_t words = 6 + (size_t)d->pt_stride + (size_t)max_steps;
    if (hipMalloc((void **)&d->dbuf, words * 4) != hipSuccess) {
        d->dbuf = nullptr;
        srq_decoder_destroy(d);
        return fail(SRQ_ENOMEM, "decoder allocation failed");
    }
    std::vector<int32_t> h(words, 0);
    h[0] = c->pos;
    h[1] = 0;
    h[2] = 0;
    h[3] = first_token;
    for (int32_t p = 0; p < d->pt_stride; ++p) h[6 + p] = p < (int32_t)c->pages.size() ? c->pages[p] : 0;
    int rc = ensure_workspace(e, d->ws, m, 1, 1, end);
    if (rc == SRQ_OK && hipMemcpy(d->dbuf, h.data(), words * 4, hipMemcpyHostToDevice) != hipSuccess)
        rc = fail(SRQ_EDEVICE, "decoder upload failed");
    if (rc == SRQ_OK && hipStreamSynchronize(e->stream) != hipSuccess) rc = fail(SRQ_EDEVICE, "sync failed");
    if (rc != SRQ_OK) {
        srq_decoder_destroy(d);
        return rc;
    }
    // One decode step: layers -> final norm + head -> argmax -> record
    // token, advance position, next step's embedding row and row plan.
    // Captured once as a HIP graph and replayed, unless the caller asked for
    // eager launches; the first step's input is prepared here.
    d->eager = (flags & SRQ_DECODER_EAGER) != 0;
    rc = enqueue_decode_input(d);
    if (rc != SRQ_OK) {
        srq_decoder_destroy(d);
        return rc;
    }
    if (!d->eager) {
        if (hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal) != hipSuccess) {
            srq_decoder_destroy(d);
            return fail(SRQ_EDEVICE, "graph capture failed to start");
        }
        rc = enqueue_decode_step(d);
        hipError_t ce = hipStreamEndCapture(e->stream, &d->graph);
        if (rc == SRQ_OK && ce != hipSuccess) rc = fail(SRQ_EDEVICE, "graph capture failed: %s", hipGetErrorString(ce));
        if (rc == SRQ_OK && hipGraphInstantiate(&d->exec, d->graph, nullptr, nullptr, 0) != hipSuccess)
            rc = fail(SRQ_EDEVICE, "graph instantiation failed");
        if (rc != SRQ_OK) {
            srq_decoder_destroy(d);
            return rc;
        }
    }
    *out = d;
    return SRQ_OK;
}

// Enqueue `steps` decode steps (asynchronous; join with srq_exec_synchronize
// or srq_decoder_tokens).
int srq_decoder_run(srq_decoder *d, int32_t steps) {
    if (!d) return fail(SRQ_EINVAL, "null decoder");
    if (steps < 0 || d->steps + steps > d->max_steps) return fail(SRQ_ERANGE, "decoder step budget exceeded");
    DeviceGuard g(d->e->device);
    for (int32_t i = 0; i < steps; ++i) {
        if (d->eager)
            SRQ_CHECK(enqueue_decode_step(d));
        else
            SRQ_HIP(hipGraphLaunch(d->exec, d->e->stream));
    }
    d->steps += steps;
    return SRQ_OK;
}

// Join, copy the tokens produced so far and commit the cache position.  A
// step whose logits were not finite produced no token: the tokens before it
// are returned with SRQ_ENONFINITE, and the position is committed through
// that step (its KV row was written, as the reference's DecodeBatch commits
// before inferHFIDs inspects the logits, M:1212-1238); later replays are
// discarded.
int srq_decoder_tokens(srq_decoder *d, int32_t *out, int32_t *count) {
    if (!d || !count) return fail(SRQ_EINVAL, "null pointer");
    DeviceGuard g(d->e->device);
    SRQ_HIP(hipStreamSynchronize(d->e->stream));
    int32_t err = 0;
    SRQ_HIP(hipMemcpy(&err, d->dbuf + 5, 4, hipMemcpyDeviceToHost));
    const int32_t good = err > 0 ? std::min(err - 1, d->steps) : d->steps;
    if (out && good) SRQ_HIP(hipMemcpy(out, d->dbuf + 6 + d->pt_stride, (size_t)good * 4, hipMemcpyDeviceToHost));
    *count = good;
    d->c->pos = d->start_pos + (err > 0 ? std::min(err, d->steps) : d->steps);
    if (err) return fail(SRQ_ENONFINITE, "non-finite HF logits");
    return SRQ_OK;
}

int srq_decoder_destroy(srq_decoder *d) {
    if (!d) return SRQ_OK;
    {
        DeviceGuard g(d->e->device);
        (void)hipStreamSynchronize(d->e->stream);
        if (d->exec) (void)hipGraphExecDestroy(d->exec);
        if (d->graph) (void)hipGraphDestroy(d->graph);
        if (d->dbuf) (void)hipFree(d->dbuf);
        d->ws.release_all();
    }
    d->c->busy = false;
    cache_unref(d->c);
    model_unref(d->m);
    exec_unref(d->e);
    delete d;
    return SRQ_OK;
}

int srq_generate_greedy(srq_exec *e, srq_model *m, srq_cache *c, const int32_t *ids, int32_t n_ids, int32_t chunk,
                        int32_t count, int32_t eos, int32_t *out_tokens, int32_t *produced) {
    if (!e || !m || !c || !ids || !out_tokens || !produced) return fail(SRQ_EINVAL, "null pointer");
    *produced = 0;
    if (n_ids < 1 || count < 1 || count > 256 || chunk < 1 || chunk > 1024 || n_ids > m->c.context - count - c->pos)
        return fail(SRQ_EINVAL, "invalid HF probe: nonempty IDs, 1..256 outputs, 1..1024 chunk, total within context");
    for (int32_t i = 0; i < n_ids; ++i)
        if (ids[i] < 0 || ids[i] >= m->c.vocab) return fail(SRQ_EINVAL, "HF token ID outside vocabulary");
    float *logits = nullptr;
    for (int32_t lo = 0; lo < n_ids; lo += chunk) {
        int32_t len = std::min(chunk, n_ids - lo);
        srq_cache *cs[1] = {c};
        SRQ_CHECK(srq_step(e, m, 1, cs, &len, ids + lo, nullptr, &logits, nullptr, nullptr));
    }
    int32_t first = 0;
    SRQ_CHECK(srq_argmax(e, logits, 1, m->c.vocab, &first));
    out_tokens[0] = first;
    *produced = 1;
    if (count == 1 || first == eos) return SRQ_OK;
    srq_decoder *d = nullptr;
    SRQ_CHECK(srq_decoder_create(e, m, c, first, count - 1, 0, &d));
    int rc = SRQ_OK;
    int32_t done = 0;
    const int32_t seg = eos >= 0 ? 16 : count - 1;
    while (rc == SRQ_OK && done < count - 1) {
        const int32_t k = std::min(seg, count - 1 - done);
        rc = srq_decoder_run(d, k);
        int32_t got = 0;
        if (rc == SRQ_OK) rc = srq_decoder_tokens(d, out_tokens + 1, &got);
        if (rc != SRQ_OK) {
            // Non-finite logits: the tokens before that step stand (the
            // reference returns them with the error, M:1212-1238).
            if (rc == SRQ_ENONFINITE) *produced = 1 + got;
            break;
        }
        done = got;
        bool stop = false;
        if (eos >= 0)
            for (int32_t i = 0; i < got; ++i)
                if (out_tokens[1 + i] == eos) {
                    // Tokens after the EOS step are not produced; the EOS
                    // token itself is never decoded (M:1224-1232).
                    done = i + 1;
                    c->pos = d->start_pos + i + 1;
                    stop = true;
                    break;
                }
        *produced = 1 + done;
        if (stop) break;
    }
    srq_decoder_destroy(d);
    return rc;
}

}  // extern "C"
