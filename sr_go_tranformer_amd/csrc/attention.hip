// Paged GQA attention over the reference's KV page layout.
//
// attend (cmd/monolith/monolith.go M:5293-5352) for every (row, query head)
// of a step (attentionRange M:6131-6147): scores = f32 dot(q, k_s) *
// f32(1/sqrt(hd)) over positions 0..pos of the row's own cache (earlier rows
// of the same chunk included, their K/V already written), max, FP64 sum of
// exp(score - max), lse = max + log(sum), p = f32(exp(score - lse)),
// out = sum_s p * v_s.  Query head h reads KV head h / (heads/kv_heads).
//
// Pages are [layer][K 32 x kvdim | V 32 x kvdim] (M:6038-6043); a row's page
// table maps position/32 to a page of the pool.
//
// One workgroup per (row, head).  Scores live in LDS (up to the model
// context, 32768 positions = 128 KiB).  Keys are scored by 16-lane groups
// (4 keys per wave at a time, lanes strided over the head dimension, a
// 16-lane xor tree); the value pass gives each thread one output element
// and a contiguous range of positions, combined in a fixed order.
#include "srq_internal.h"

namespace srq {
namespace {

__device__ __forceinline__ const float *kv_row(const RowMeta &m, int sess, int pos, int kvdim, int which) {
    const int page = m.pages[(int64_t)sess * m.pt_stride + pos / kPageTokens];
    return m.kv_pool + (int64_t)page * m.page_elems + (int64_t)m.layer * 2 * kPageTokens * kvdim +
           (int64_t)which * kPageTokens * kvdim + (int64_t)(pos % kPageTokens) * kvdim;
}

__global__ __launch_bounds__(256) void attention_kernel(const AttnArgs A) {
    extern __shared__ float scores[];
    __shared__ float qs[256];
    __shared__ float redf[4];
    __shared__ double redd[4];
    __shared__ float part[256];

    const int row = blockIdx.x, h = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int hd = A.head_dim, kvdim = A.kv_heads * hd;
    const int kh = h / (A.heads / A.kv_heads);
    const int pos = A.meta.pos[row], sess = A.meta.sess[row];
    const int len = pos + 1;
    const float *q = A.q + (int64_t)row * A.heads * hd + (int64_t)h * hd;
    for (int j = tid; j < hd; j += 256) qs[j] = q[j];
    __syncthreads();
    const float scale = (float)(1.0 / sqrt((double)hd));

    // ---- scores -----------------------------------------------------------
    const int sub = lane >> 4, l16 = lane & 15;
    float mx = -3.402823466e38f;
    for (int s0 = wave * 4; s0 < len; s0 += 16) {
        const int s = s0 + sub;
        float dot = 0.0f;
        if (s < len) {
            const float *k = kv_row(A.meta, sess, s, kvdim, 0) + (int64_t)kh * hd;
            for (int j = l16; j < hd; j += 16) dot = __builtin_fmaf(qs[j], k[j], dot);
        }
#pragma unroll
        for (int o = 8; o > 0; o >>= 1) dot += __shfl_xor(dot, o, 64);
        if (s < len) {
            const float sc = dot * scale;
            if (l16 == 0) scores[s] = sc;
            mx = fmaxf(mx, sc);
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if (lane == 0) redf[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(redf[0], redf[1]), fmaxf(redf[2], redf[3]));

    // ---- FP64 normaliser ----------------------------------------------------
    double sum = 0.0;
    for (int s = tid; s < len; s += 256) sum += exp((double)scores[s] - (double)mx);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
    if (lane == 0) redd[wave] = sum;
    __syncthreads();
    sum = redd[0] + redd[1] + redd[2] + redd[3];
    const double lse = (double)mx + log(sum);
    for (int s = tid; s < len; s += 256) scores[s] = (float)exp((double)scores[s] - lse);
    __syncthreads();

    // ---- values ---------------------------------------------------------------
    const int nparts = 256 / hd;  // hd <= 256
    const int j = tid % hd, pidx = tid / hd;
    float acc = 0.0f;
    if (pidx < nparts) {
        const int per = (len + nparts - 1) / nparts;
        const int lo = pidx * per, hi = min(len, lo + per);
        for (int s = lo; s < hi; ++s) {
            const float *v = kv_row(A.meta, sess, s, kvdim, 1) + (int64_t)kh * hd;
            acc = __builtin_fmaf(scores[s], v[j], acc);
        }
        part[tid] = acc;
    }
    __syncthreads();
    if (tid < hd) {
        float o = 0.0f;
        for (int p = 0; p < nparts; ++p) o += part[p * hd + tid];
        A.out[(int64_t)row * A.heads * hd + (int64_t)h * hd + tid] = o;
    }
}

}  // namespace

int launch_attention(hipStream_t s, const AttnArgs &a) {
    if (a.n <= 0) return SRQ_OK;
    if (a.head_dim > 256 || a.head_dim < 1) return fail(SRQ_EINVAL, "attention: head_dim %d unsupported", a.head_dim);
    const size_t lds = (size_t)(a.max_len > 0 ? a.max_len : 1) * sizeof(float);
    if (lds > 140 * 1024) return fail(SRQ_EINVAL, "attention: %d positions exceed LDS", a.max_len);
    attention_kernel<<<dim3(a.n, a.heads), 256, lds, s>>>(a);
    SRQ_HIP(hipGetLastError());
    return SRQ_OK;
}

int attention_prepare() {
    SRQ_HIP(hipFuncSetAttribute((const void *)attention_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                140 * 1024));
    return SRQ_OK;
}

}  // namespace srq
