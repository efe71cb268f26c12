// Internal declarations shared by the gfx950 kernels and the C-ABI runtime.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/srq.h"

namespace srq {

constexpr int kBlock = 64;       // q8Block (M:3793): scale block width
constexpr int kPageTokens = 32;  // pageTokens (M:5846)
constexpr int kAttnTileRows = 16;  // rows per query tile of a step (AttnArgs::tiles)
constexpr int kWave = 64;

// f32(MaxFloat32 / (2*64*127)) (M:4346-4354): above it a row takes the
// FP64 path.  The constant is the correctly rounded f32 of the quotient.
constexpr float kWideLimit = 0x1.020408p+114f;  // 2.0932724e34

// Streaming (read-once) loads of packed weights: global_load ... nt.
typedef uint32_t srq_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t srq_u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 ld_stream16(const void *p) {
    const srq_u32x4 v = __builtin_nontemporal_load((const srq_u32x4 *)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ld_stream8(const void *p) {
    const srq_u32x2 v = __builtin_nontemporal_load((const srq_u32x2 *)p);
    return make_uint2(v.x, v.y);
}

// code/16 of the signed nibble in bits [3:0] of byte B of w: one
// v_cvt_off_f32_i4 with an SDWA byte select (exact; 8 -> -0.5, 7 -> 0.4375).
template <int B>
__device__ __forceinline__ float nib16(uint32_t w) {
    float r;
    if constexpr (B == 0)
        asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0" : "=v"(r) : "v"(w));
    else if constexpr (B == 1)
        asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1" : "=v"(r) : "v"(w));
    else if constexpr (B == 2)
        asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2" : "=v"(r) : "v"(w));
    else
        asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3" : "=v"(r) : "v"(w));
    return r;
}

// Error reporting: sets the calling thread's message and returns code.
int fail(int code, const char *fmt, ...);
void clear_error();

#define SRQ_HIP(expr)                                                                          \
    do {                                                                                       \
        hipError_t _e = (expr);                                                                \
        if (_e != hipSuccess) return ::srq::fail(SRQ_EDEVICE, "%s: %s", #expr, hipGetErrorString(_e)); \
    } while (0)

#define SRQ_CHECK(expr)           \
    do {                          \
        int _rc = (expr);         \
        if (_rc != SRQ_OK) return _rc; \
    } while (0)

// Byte stride of one packed row.
__host__ __device__ inline int64_t row_bytes(int fmt, int64_t cols) {
    return fmt == SRQ_Q8 ? cols : fmt == SRQ_Q4 ? (cols + 1) / 2 : cols * 4;
}
__host__ __device__ inline int64_t groups_of(int64_t cols) { return (cols + kBlock - 1) / kBlock; }

// ---------------------------------------------------------------- packing
int launch_pack(hipStream_t s, int fmt, int64_t rows, int64_t cols, const void *src, int dtype, void *values,
                float *scales, int *err_flag);
int launch_convert_f32(hipStream_t s, int64_t count, const void *src, int dtype, float *dst, int *err_flag);
int launch_dequant_rows(hipStream_t s, int fmt, int64_t cols, const void *values, const float *scales,
                        const int32_t *rows, int32_t count, float *dst);
int launch_fill_normal(hipStream_t s, float *dst, int64_t count, uint64_t seed, double scale);
int launch_zero(hipStream_t s, int32_t *dst, int64_t count);

// ------------------------------------------------------------------ GEMV
enum Epilogue { EPI_PLAIN = 0, EPI_RESID = 1, EPI_SWIGLU = 2, EPI_ROPE_KV = 3 };

// Row metadata of a step: per activation row its position and session,
// per session a page table of pt_stride int32 page ids.
struct RowMeta {
    const int32_t *pos;        // [n]
    const int32_t *sess;       // [n]
    const int32_t *pages;      // [sessions x pt_stride]
    int32_t pt_stride;
    float *kv_pool;            // page 0
    int64_t page_elems;        // 2*32*kvdim*layers
    int32_t layer;
    // Row plan (launch_row_plan), used by the fused GEMV epilogue:
    const int64_t *kvoff;      // [n] element offset of the row's K row in layer 0
    const float *rope_cs;      // [n x head_dim] {cos, sin} of the row's position, interleaved
    // Every row belongs to session 0 (one-session steps, the decoder): a
    // row's page-table entries need no load of its session first.
    int32_t one_sess;
};

struct GemvArgs {
    int fmt;
    const void *values;
    const float *scales;
    int64_t rows, cols;        // W is [rows x cols]
    const float *x;            // [n x cols]
    int32_t n;                 // activation rows (1..8 per launch)
    int32_t row0;              // index of x's first row in the step (RowMeta)
    const float *norm_w;       // fused RMSNorm weight [cols] or null
    double norm_eps;
    float *y;                  // output
    int64_t y_stride;
    int epilogue;
    const float *residual;     // EPI_RESID: y = residual + dot (may alias y)
    // EPI_ROPE_KV: W rows are [q: dim | k: kvdim | v: kvdim]
    int32_t dim, kvdim, head_dim;
    const float *cos_t, *sin_t; // [context x head_dim/2]
    const float *bias;          // [rows] or null, added before RoPE
    RowMeta meta;
};
int launch_gemv(hipStream_t s, const GemvArgs &a);
bool gemv_fast_ok(int fmt, int64_t cols);
// Batch rows per GEMV launch for a weight of `cols` inputs; norm: fused
// RMSNorm; extra_floats: LDS floats of the epilogue's per-launch data.
int gemv_max_rows(int fmt, int64_t cols, bool norm, int64_t extra_floats);
int gemv_prepare();

// ------------------------------------------------------------------ GEMM
// RoPE/KV output of a q/k/v GEMM: W's rows are [q: dim | k: kvdim | v: kvdim]
// (bias added first, then the half-split RoPE of M:5264-5289 on q and k); q
// goes to q (stride dim), k and v into the rows' KV pages (M:6393-6395).
struct GemmRope {
    float *q;               // null: no RoPE/KV output
    const float *bias;      // [dim + 2*kvdim] or null
    int32_t dim, kvdim, head_dim;
    const float *cos_t, *sin_t;  // [context x head_dim/2]
    RowMeta meta;
};

struct GemmArgs {
    int fmt;
    const void *values;
    const float *scales;
    int64_t rows, cols;
    const float *x;     // [n x cols]
    int32_t n;
    float *y;           // [n x y_stride]
    int64_t y_stride;
    const float *residual;  // y = residual + acc when non-null (may alias y)
    // SwiGLU output (nullable): W's rows are [gate (rows/2); up (rows/2)] and
    // swiglu_out[m][u] = f32(g/(1+exp(-g))) * up (M:6411-6413), stride
    // rows/2; y is then only a temporary (written when K is not split).
    float *swiglu_out;
    // RMSNorm output (nullable): norm_out[m] = rmsInto(y[m], norm_w, eps)
    // (M:6182-6194), the next matrix's input, stride rows; needs y_stride ==
    // rows.  y is still written.
    const float *norm_w;
    double norm_eps;
    float *norm_out;
    GemmRope rope;  // rope.q non-null: RoPE/KV output; y is then only a temporary
};
// y = x . W^T (+ residual) on MFMA.  Rows holding a wide |x| are computed
// in FP64.  scratch: gemm_scratch_bytes(fmt, n, rows, cols) bytes of device
// memory for split-K partial sums (0: none needed).
int launch_gemm(hipStream_t s, const GemmArgs &a, void *scratch, size_t scratch_bytes);
size_t gemm_scratch_bytes(int fmt, int32_t n, int64_t rows, int64_t cols);
bool gemm_ok(int fmt, int64_t cols);

// ------------------------------------------------------------------ glue
int launch_rmsnorm(hipStream_t s, const float *x, const float *w, float *y, int32_t n, int32_t d, double eps);
int launch_rope_kv(hipStream_t s, const float *qkv, const float *bias, int32_t n, int32_t dim, int32_t kvdim,
                   int32_t head_dim, const float *cos_t, const float *sin_t, float *q_out, const RowMeta &meta);
int launch_swiglu(hipStream_t s, const float *gu, int32_t n, int32_t hidden, float *h);
int launch_gather_rows(hipStream_t s, const float *src, int64_t d, const int32_t *rows, int32_t count, float *dst);
int launch_argmax(hipStream_t s, const float *logits, int32_t rows, int32_t vocab, int32_t *ids, int32_t *err);
// Tail of a replayed greedy decode step (one row): argmax of `logits` ->
// token; out[counter] = token, counter + 1, embed_id = token, pos + 1; then,
// if counter < steps, x = the token's embedding row and the row plan
// (kvoff[0], rope_cs[0..head_dim)) of the new position.  err[0] records
// the first step whose logits held a non-finite value, as its counter + 1.
struct DecodeTailArgs {
    const float *logits;
    int32_t vocab;
    int32_t *token, *err, *pos, *out, *counter, *embed_id;
    int32_t steps;
    int fmt;                   // embedding table
    const void *values;
    const float *scales;
    int64_t dim;
    float *x;
    const int32_t *sess, *pages;  // row plan inputs (RowMeta's)
    int32_t pt_stride;
    int64_t page_elems;
    int32_t kvdim, half;
    const float *cos_t, *sin_t;
    int64_t *kvoff;
    float *rope_cs;
};
int launch_decode_tail(hipStream_t s, const DecodeTailArgs &a);
// Row plan of a step's n rows: kvoff[r] = page*page_elems + (pos%32)*kvdim
// and rope_cs[r] = {cos, sin} pairs of pos (tables [context x head_dim/2]).
int launch_row_plan(hipStream_t s, const RowMeta &meta, int32_t n, int32_t kvdim, int32_t head_dim,
                    const float *cos_t, const float *sin_t, int64_t *kvoff, float *rope_cs);

// -------------------------------------------------------------- sampling
struct SampleArgs {
    const float *logits;         // [* x vocab]
    const int32_t *row_ids;      // [rows]: logits row of each sampled row, or null (row k)
    int32_t rows, vocab;
    double temperature;          // 0: greedy
    int32_t top_k;               // 0: off
    double top_p;                // >= 1: off
    double repeat_penalty;       // 1: off
    const int32_t *history;      // [rows x history_stride] or null
    const int32_t *history_len;  // [rows] or null
    int32_t history_stride;
    const int32_t *blocked;      // [rows] (-1: none) or null
    uint64_t *rng;               // [rows] SplitMix64 states, advanced per draw
    int32_t *ids;                // [rows] out
    int32_t *err;                // |= 1 non-finite logit, 2 no candidate, 4/8 selection limits
    // Set by launch_sample: rows are cut into `chunks` chunks of chunk_len
    // ids, each chunk's range and histogram kept in scratch.
    int32_t chunks, chunk_len;
    struct SampleRange *range;   // [rows x chunks]
    unsigned long long *hmass;   // [rows x chunks x 2048]
    uint32_t *hcount;            // [rows x chunks x 2048]
    uint32_t *hoff;              // [rows x chunks x 2048] bucket starts in `order`
    int32_t *order;              // [rows x chunks x chunk_len] a chunk's candidate ids by bucket
};
struct SampleRange {  // one chunk of a row
    double vmax, vmin, best_v;
    int32_t best_id, cnt, bad, pad;
    unsigned long long total;  // integer mass (temperature != 0)
};
// scratch: sample_scratch_bytes(rows, vocab) bytes, 16-byte aligned.
int launch_sample(hipStream_t s, const SampleArgs &a, void *scratch);
size_t sample_scratch_bytes(int32_t rows, int32_t vocab);

// ------------------------------------------------------------- attention
struct AttnArgs {
    const float *q;     // [n x heads*head_dim]
    float *out;         // [n x heads*head_dim]
    int32_t n, heads, kv_heads, head_dim;
    int32_t max_len;    // upper bound of pos+1 over rows (sizes LDS)
    RowMeta meta;
    // Query tiles of a step (nullable): ntiles pairs {first row, rows} of at
    // most 16 consecutive rows of one session, covering every row once.
    // Prefill-sized steps use them for the MFMA flash kernel.
    const int32_t *tiles;
    int32_t ntiles;
};
// scratch: attention_scratch_bytes(n, heads, head_dim, max_len) bytes;
// counters: n*heads int32, zero before the first launch (the kernels leave
// them zero).
int launch_attention(hipStream_t s, const AttnArgs &a, float *scratch, int32_t *counters);
size_t attention_scratch_bytes(int32_t n, int32_t heads, int32_t head_dim, int32_t max_len);
int attention_prepare();

// ----------------------------------------------------------- model hooks
// For the archive loader.  model_load_enqueue is srq_model_load without the
// join: it queues the convert/pack on the model's executor stream, and a
// non-finite source value sets the executor's device error word 0, which
// stays set until model_join_nonfinite (which joins the stream) clears it
// and fails with SRQ_ENONFINITE and the message `what`.
int model_load_enqueue(srq_model *m, int kind, int layer, const void *src, int dtype);
int model_join_nonfinite(srq_model *m, const char *what);
const srq_model_config &model_config(const srq_model *m);
int model_device(const srq_model *m);
hipStream_t model_stream(const srq_model *m);
const int32_t *model_error_word(const srq_model *m);

}  // namespace srq
