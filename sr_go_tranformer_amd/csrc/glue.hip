// Step glue kernels used on the batched (GEMM) path and around it.
// cmd/monolith/monolith.go: rmsInto M:6182-6194, rope M:5264-5289, KV row
// write M:6393-6395, SwiGLU M:6411-6413, selective-head compaction and
// expansion M:6420-6448, greedy argmax M:1215-1223.
#include <algorithm>

#include "srq_internal.h"

namespace srq {
namespace {

__device__ __forceinline__ double block_sum_d(double v, double *red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    double t = 0.0;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) t += red[w];
    __syncthreads();
    return t;
}

// rmsInto: a = f32(1/sqrt(sum f64(x^2)/d + eps)); y = (x*a)*w.
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                      float *__restrict__ y, int32_t d, double eps) {
    __shared__ double red[4];
    const float *xr = x + (int64_t)blockIdx.x * d;
    float *yr = y + (int64_t)blockIdx.x * d;
    double ss = 0.0;
    for (int j = threadIdx.x; j < d; j += 256) ss += (double)xr[j] * (double)xr[j];
    ss = block_sum_d(ss, red);
    const float a = (float)(1.0 / sqrt(ss / (double)d + eps));
    for (int j = threadIdx.x; j < d; j += 256) yr[j] = __fmul_rn(__fmul_rn(xr[j], a), w[j]);
}

// qkv row [q: dim | k: kvdim | v: kvdim] (+bias) -> q_out (roped), K (roped)
// and V into the row's KV page.
__global__ __launch_bounds__(256) void rope_kv_kernel(const float *__restrict__ qkv, const float *__restrict__ bias,
                                                      int32_t dim, int32_t kvdim, int32_t head_dim,
                                                      const float *__restrict__ cos_t,
                                                      const float *__restrict__ sin_t, float *__restrict__ q_out,
                                                      const RowMeta meta) {
    const int row = blockIdx.x;
    const int width = dim + 2 * kvdim;
    const float *src = qkv + (int64_t)row * width;
    const int pos = meta.pos[row];
    const int half = head_dim / 2;
    const int page = meta.pages[(int64_t)meta.sess[row] * meta.pt_stride + pos / kPageTokens];
    float *kr = meta.kv_pool + (int64_t)page * meta.page_elems + (int64_t)meta.layer * 2 * kPageTokens * kvdim +
                (int64_t)(pos % kPageTokens) * kvdim;
    float *vr = kr + (int64_t)kPageTokens * kvdim;
    const int pairs = (dim + kvdim) / 2;
    for (int p = threadIdx.x; p < pairs; p += 256) {
        const int h = p / half, j = p - h * half;
        const int i0 = h * head_dim + j, i1 = i0 + half;
        float a = src[i0], z = src[i1];
        if (bias) {
            a = __fadd_rn(a, bias[i0]);
            z = __fadd_rn(z, bias[i1]);
        }
        const float c = cos_t[(int64_t)pos * half + j], s = sin_t[(int64_t)pos * half + j];
        const float na = __fsub_rn(__fmul_rn(a, c), __fmul_rn(z, s));
        const float nz = __fadd_rn(__fmul_rn(a, s), __fmul_rn(z, c));
        if (i0 < dim) {
            q_out[(int64_t)row * dim + i0] = na;
            q_out[(int64_t)row * dim + i1] = nz;
        } else {
            kr[i0 - dim] = na;
            kr[i1 - dim] = nz;
        }
    }
    for (int j = threadIdx.x; j < kvdim; j += 256) {
        float v = src[dim + kvdim + j];
        if (bias) v = __fadd_rn(v, bias[dim + kvdim + j]);
        vr[j] = v;
    }
}

// gu row [gate: hidden | up: hidden] -> h = f32(g/(1+exp(-g))) * u.
__global__ __launch_bounds__(256) void swiglu_kernel(const float *__restrict__ gu, int32_t hidden,
                                                     float *__restrict__ h) {
    const float *src = gu + (int64_t)blockIdx.y * 2 * hidden;
    float *dst = h + (int64_t)blockIdx.y * hidden;
    for (int j = blockIdx.x * 256 + threadIdx.x; j < hidden; j += gridDim.x * 256) {
        const double g = (double)src[j];
        const float sg = (float)(g / (1.0 + exp(-g)));
        dst[j] = __fmul_rn(sg, src[hidden + j]);
    }
}

// dst[i] = src[rows[i]] (rows[i] < 0: zero row).
__global__ __launch_bounds__(256) void gather_kernel(const float *__restrict__ src, int64_t d,
                                                     const int32_t *__restrict__ rows, float *__restrict__ dst) {
    const int32_t r = rows[blockIdx.y];
    float *out = dst + (int64_t)blockIdx.y * d;
    for (int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x; j < d; j += (int64_t)gridDim.x * 256)
        out[j] = r >= 0 ? src[(int64_t)r * d + j] : 0.0f;
}

// First maximum with strict '>' (lowest id wins ties); non-finite -> err.
// One 1024-thread workgroup per row; each thread scans its ids in ascending
// order with 8 float4 loads in flight, then the (value, id) pairs reduce
// with ties to the lower id.
constexpr int kArgThreads = 1024;

__device__ __forceinline__ void arg_take(float &best, int &idx, float v, int j) {
    if (idx < 0 || v > best) best = v, idx = j;
}
__device__ __forceinline__ void arg_merge(float &best, int &idx, float ov, int oi) {
    if (oi >= 0 && (idx < 0 || ov > best || (ov == best && oi < idx))) best = ov, idx = oi;
}

// First maximum of one row by the whole 1024-thread workgroup; thread 0
// gets the id (lowest on ties) and whether any value was non-finite.
__device__ __forceinline__ void argmax_row(const float *__restrict__ row, int32_t vocab, int &id, int &nonfinite_any) {
    constexpr int NW = kArgThreads / 64, U = 8;
    __shared__ float bv[NW];
    __shared__ int bi[NW];
    __shared__ int bad;
    const int tid = threadIdx.x;
    if (tid == 0) bad = 0;
    __syncthreads();
    float best = 0.0f;
    int idx = -1;
    int nonfinite = 0;
    if ((vocab & 3) == 0) {
        const int n4 = vocab / 4;
        for (int base = 0; base < n4; base += kArgThreads * U) {
            float4 t[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int j4 = base + u * kArgThreads + tid;
                t[u] = j4 < n4 ? ((const float4 *)row)[j4] : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int j4 = base + u * kArgThreads + tid;
                if (j4 >= n4) continue;
                const float v[4] = {t[u].x, t[u].y, t[u].z, t[u].w};
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    nonfinite |= !isfinite(v[c]);
                    arg_take(best, idx, v[c], 4 * j4 + c);
                }
            }
        }
    } else {
        for (int base = 0; base < vocab; base += kArgThreads * U) {
            float t[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int j = base + u * kArgThreads + tid;
                t[u] = j < vocab ? row[j] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int j = base + u * kArgThreads + tid;
                if (j >= vocab) continue;
                nonfinite |= !isfinite(t[u]);
                arg_take(best, idx, t[u], j);
            }
        }
    }
    if (nonfinite) bad = 1;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) arg_merge(best, idx, __shfl_xor(best, o, 64), __shfl_xor(idx, o, 64));
    const int lane = tid & 63, wave = tid >> 6;
    if (lane == 0) bv[wave] = best, bi[wave] = idx;
    __syncthreads();
    if (tid == 0) {
        float b = bv[0];
        int i = bi[0];
        for (int w = 1; w < NW; ++w) arg_merge(b, i, bv[w], bi[w]);
        id = i;
        nonfinite_any = bad;
    }
}

__global__ __launch_bounds__(kArgThreads) void argmax_kernel(const float *__restrict__ logits, int32_t vocab,
                                                             int32_t *__restrict__ ids, int32_t *__restrict__ err) {
    int id = 0, bad = 0;
    argmax_row(logits + (int64_t)blockIdx.x * vocab, vocab, id, bad);
    if (threadIdx.x == 0) {
        ids[blockIdx.x] = id;
        if (bad) err[0] = 1;
    }
}

// The tail of one step of a replayed greedy decoder, in one launch: the
// argmax of the logits row (argmax_kernel's rule), the advance (token
// recorded, counter and position + 1), and, while steps remain, the next
// step's input: the token's embedding row (copyRow's f32(code) * scale,
// M:3900-3921) and the row plan of the new position (row_plan_kernel's).
template <int FMT>
__global__ __launch_bounds__(kArgThreads) void decode_tail_kernel(const DecodeTailArgs A) {
    __shared__ int tok, next_pos;
    int id = 0, bad = 0;
    argmax_row(A.logits, A.vocab, id, bad);
    const int tid = threadIdx.x;
    if (tid == 0) {
        A.token[0] = id;
        const int c = A.counter[0], p = A.pos[0] + 1;
        // The first step with non-finite logits, as c + 1 (0: none yet).
        if (bad && A.err[0] == 0) A.err[0] = c + 1;
        A.out[c] = id;
        A.counter[0] = c + 1;
        A.embed_id[0] = id;
        A.pos[0] = p;
        tok = id;
        next_pos = c + 1 < A.steps ? p : -1;
    }
    __syncthreads();
    const int p = next_pos, r = tok;
    if (p < 0) return;
    const int64_t cols = A.dim, groups = groups_of(cols);
    for (int64_t j = tid; j < cols; j += kArgThreads) {
        if constexpr (FMT == SRQ_F32) {
            A.x[j] = ((const float *)A.values)[(int64_t)r * cols + j];
        } else {
            float w;
            if constexpr (FMT == SRQ_Q8) {
                w = (float)((const int8_t *)A.values)[(int64_t)r * cols + j];
            } else {
                const uint32_t b = ((const uint8_t *)A.values)[(int64_t)r * ((cols + 1) / 2) + j / 2];
                const uint32_t nib = (j & 1) ? (b >> 4) : (b & 15u);
                w = (float)(((int32_t)(nib << 28)) >> 28);
            }
            A.x[j] = w * A.scales[(int64_t)r * groups + j / kBlock];
        }
    }
    if (tid == 0) {
        const int page = A.pages[(int64_t)A.sess[0] * A.pt_stride + p / kPageTokens];
        A.kvoff[0] = (int64_t)page * A.page_elems + (int64_t)(p % kPageTokens) * A.kvdim;
    }
    for (int j = tid; j < A.half; j += kArgThreads) {
        A.rope_cs[2 * j] = A.cos_t[(int64_t)p * A.half + j];
        A.rope_cs[2 * j + 1] = A.sin_t[(int64_t)p * A.half + j];
    }
}

// One workgroup per row: the row's KV element offset and its RoPE row.
__global__ void row_plan_kernel(const int32_t *pos, const int32_t *sess, const int32_t *pages, int32_t pt_stride,
                                int64_t page_elems, int32_t kvdim, int32_t half, const float *cos_t,
                                const float *sin_t, int64_t *kvoff, float *rope_cs) {
    const int row = blockIdx.x;
    const int p = pos[row];
    if (threadIdx.x == 0) {
        const int page = pages[(int64_t)sess[row] * pt_stride + p / kPageTokens];
        kvoff[row] = (int64_t)page * page_elems + (int64_t)(p % kPageTokens) * kvdim;
    }
    for (int j = threadIdx.x; j < half; j += blockDim.x) {
        rope_cs[((int64_t)row * half + j) * 2] = cos_t[(int64_t)p * half + j];
        rope_cs[((int64_t)row * half + j) * 2 + 1] = sin_t[(int64_t)p * half + j];
    }
}

__global__ void zero_kernel(int32_t *dst, int64_t count) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x)
        dst[i] = 0;
}

}  // namespace

int launch_zero(hipStream_t s, int32_t *dst, int64_t count) {
    if (count <= 0) return SRQ_OK;
    const int64_t blocks = std::min<int64_t>((count + 255) / 256, 1024);
    zero_kernel<<<(unsigned)blocks, 256, 0, s>>>(dst, count);
    SRQ_HIP(hipGetLastError());
    return SRQ_OK;
}

int launch_row_plan(hipStream_t s, const RowMeta &meta, int32_t n, int32_t kvdim, int32_t head_dim,
                    const float *cos_t, const float *sin_t, int64_t *kvoff, float *rope_cs) {
    if (n <= 0) return SRQ_OK;
    row_plan_kernel<<<n, 64, 0, s>>>(meta.pos, meta.sess, meta.pages, meta.pt_stride, meta.page_elems, kvdim,
                                     head_dim / 2, cos_t, sin_t, kvoff, rope_cs);
    SRQ_HIP(hipGetLastError());
    return SRQ_OK;
}

int launch_rmsnorm(hipStream_t s, const float *x, const float *w, float *y, int32_t n, int32_t d, double eps) {
    if (n <= 0) return SRQ_OK;
    rmsnorm_kernel<<<n, 256, 0, s>>>(x, w, y, d, eps);
    SRQ_HIP(hipGetLastError());
    return SRQ_OK;
}

int launch_rope_kv(hipStream_t s, const float *qkv, const float *bias, int32_t n, int32_t dim, int32_t kvdim,
                   int32_t head_dim, const float *cos_t, const float *sin_t, float *q_out, const RowMeta &meta) {
    if (n <= 0) return SRQ_OK;
    rope_kv_kernel<<<n, 256, 0, s>>>(qkv, bias, dim, kvdim, head_dim, cos_t, sin_t, q_out, meta);
    SRQ_HIP(hipGetLastError());
    return SRQ_OK;
}

int launch_swiglu(hipStream_t s, const float *gu, int32_t n, int32_t hidden, float *h) {
    if (n <= 0) return SRQ_OK;
    int bx = (hidden + 255) / 256;
    if (bx > 64) bx = 64;
    swiglu_kernel<<<dim3(bx, n), 256, 0, s>>>(gu, hidden, h);
    SRQ_HIP(hipGetLastError());
    return SRQ_OK;
}

int launch_gather_rows(hipStream_t s, const float *src, int64_t d, const int32_t *rows, int32_t count, float *dst) {
    if (count <= 0) return SRQ_OK;
    int64_t bx = (d + 255) / 256;
    if (bx > 64) bx = 64;
    gather_kernel<<<dim3((unsigned)bx, count), 256, 0, s>>>(src, d, rows, dst);
    SRQ_HIP(hipGetLastError());
    return SRQ_OK;
}

int launch_decode_tail(hipStream_t s, const DecodeTailArgs &a) {
    if (a.vocab < 1 || a.dim < 1) return fail(SRQ_EINVAL, "decode tail: empty vocabulary or width");
    if (a.fmt == SRQ_Q8)
        decode_tail_kernel<SRQ_Q8><<<1, kArgThreads, 0, s>>>(a);
    else if (a.fmt == SRQ_Q4)
        decode_tail_kernel<SRQ_Q4><<<1, kArgThreads, 0, s>>>(a);
    else
        decode_tail_kernel<SRQ_F32><<<1, kArgThreads, 0, s>>>(a);
    SRQ_HIP(hipGetLastError());
    return SRQ_OK;
}

int launch_argmax(hipStream_t s, const float *logits, int32_t rows, int32_t vocab, int32_t *ids, int32_t *err) {
    if (rows <= 0) return SRQ_OK;
    argmax_kernel<<<rows, kArgThreads, 0, s>>>(logits, vocab, ids, err);
    SRQ_HIP(hipGetLastError());
    return SRQ_OK;
}

}  // namespace srq
