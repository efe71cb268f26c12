// Paged GQA attention over the reference's KV page layout.
//
// attend (cmd/monolith/monolith.go M:5293-5352) for every (row, query head)
// of a step (attentionRange M:6131-6147): scores = f32 dot(q, k_s) *
// f32(1/sqrt(hd)) over positions 0..pos of the row's own cache (earlier rows
// of the same chunk included: their K/V were written first), max, FP64 sum
// of exp(score - max), lse = max + log(sum), out = sum_s p_s v_s with
// p_s = exp(score_s - lse).  Query head h reads KV head h / (heads/kv_heads).
// Pages are [layer][K 32 x kvdim | V 32 x kvdim] (M:6038-6043); a row's page
// table maps position/32 to a pool page.
//
// Split over positions (flash-decoding): workgroup (row, kv head, split)
// scores kSplit positions for all query heads of its GQA group, so each K/V
// row is read once per group.  It keeps the split's max m_i, FP64 sum
// l_i = sum exp(score - m_i) and o_i = sum f32(exp(score - m_i)) v_s.  The
// combine kernel forms lse = M + log(sum_i l_i exp(m_i - M)) and
// out = sum_i f32(exp(m_i - lse)) o_i, which equals the reference's
// sum_s exp(score_s - lse) v_s up to f32 rounding of the factors.
#include <algorithm>
#include <cfloat>

#include "srq_internal.h"

namespace srq {
namespace {

constexpr int kSplit = 64;     // positions per split (two pages)
constexpr int kMaxGroup = 8;   // query heads per KV head handled together
constexpr int kMaxHd = 256;
// Batches up to this many rows use the fused split+merge kernel; larger
// ones (prefill) the split and combine kernels, whose many workgroups would
// otherwise each pay the merge's cache write-back and invalidation.
constexpr int kFusedRows = 4;
constexpr int kFusedSplits = 16;  // splits of 64 positions: context <= 1024
static_assert(kFusedSplits <= 64, "the fused kernel's one-wave merge holds one split per lane");

__device__ __forceinline__ const float *kv_row(const RowMeta &m, int sess, int pos, int kvdim, int which) {
    const int page = m.pages[(int64_t)sess * m.pt_stride + pos / kPageTokens];
    return m.kv_pool + (int64_t)page * m.page_elems + (int64_t)m.layer * 2 * kPageTokens * kvdim +
           (int64_t)which * kPageTokens * kvdim + (int64_t)(pos % kPageTokens) * kvdim;
}

// Partials: [row][head][split] -> {m, l(double as 2 floats), o[hd]}.
__device__ __forceinline__ float *partial(float *base, int row, int h, int sp, int heads, int nsplit, int hd) {
    return base + (((int64_t)row * heads + h) * nsplit + sp) * (hd + 4);
}

__global__ __launch_bounds__(256) void attn_split_kernel(const AttnArgs A, float *__restrict__ part, int nsplit) {
    __shared__ float qs[kMaxGroup * kMaxHd];
    __shared__ float sc[kMaxGroup][kSplit];
    __shared__ float mx[kMaxGroup];
    __shared__ float ov[2][kMaxGroup * kMaxHd];

    const int row = blockIdx.x, kh = blockIdx.y, sp = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int hd = A.head_dim, kvdim = A.kv_heads * hd, G = A.heads / A.kv_heads;
    const int pos = A.meta.pos[row], sess = A.meta.sess[row];
    const int len = pos + 1, s0 = sp * kSplit, s1 = min(len, s0 + kSplit), ns = s1 - s0;
    if (ns <= 0) {
        // Empty split: contributes nothing to the combine.
        for (int i = tid; i < G * (hd + 4); i += 256) {
            const int g = i / (hd + 4), k = i - g * (hd + 4);
            float *p = partial(part, row, kh * G + g, sp, A.heads, nsplit, hd);
            p[k] = k == 0 ? -FLT_MAX : 0.0f;
        }
        return;
    }
    for (int i = tid; i < G * hd; i += 256) {
        const int g = i / hd, j = i - g * hd;
        qs[i] = A.q[(int64_t)row * A.heads * hd + (int64_t)(kh * G + g) * hd + j];
    }
    __syncthreads();
    const float scale = (float)(1.0 / sqrt((double)hd));

    // ---- scores: one 16-lane group per key, all G heads of the group ----
    const int sub = lane >> 4, l16 = lane & 15;
    for (int s = wave * 4 + sub; s < ((ns + 15) / 16) * 16; s += 16) {
        float dot[kMaxGroup];
#pragma unroll
        for (int g = 0; g < kMaxGroup; ++g) dot[g] = 0.0f;
        if (s < ns) {
            const float *k = kv_row(A.meta, sess, s0 + s, kvdim, 0) + (int64_t)kh * hd;
            for (int j = l16; j < hd; j += 16) {
                const float kj = k[j];
#pragma unroll
                for (int g = 0; g < kMaxGroup; ++g)
                    if (g < G) dot[g] = __builtin_fmaf(qs[g * hd + j], kj, dot[g]);
            }
        }
#pragma unroll
        for (int g = 0; g < kMaxGroup; ++g) {
            float d = dot[g];
#pragma unroll
            for (int o = 8; o > 0; o >>= 1) d += __shfl_xor(d, o, 64);
            if (g < G && s < ns && l16 == 0) sc[g][s] = d * scale;
        }
    }
    __syncthreads();

    // ---- per-head split max and FP64 sum ---------------------------------
    if (wave == 0) {
        for (int g = 0; g < G; ++g) {
            float m = -FLT_MAX;
            for (int s = lane; s < ns; s += 64) m = fmaxf(m, sc[g][s]);
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
            double l = 0.0;
            for (int s = lane; s < ns; s += 64) {
                const double e = exp((double)sc[g][s] - (double)m);
                l += e;
                sc[g][s] = (float)e;  // weight of position s inside this split
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) l += __shfl_xor(l, o, 64);
            if (lane == 0) {
                mx[g] = m;
                float *p = partial(part, row, kh * G + g, sp, A.heads, nsplit, hd);
                p[0] = m;
                *(double *)(p + 2) = l;
            }
        }
    }
    __syncthreads();

    // ---- o_i = sum_s w_s v_s: thread = (half of the keys, dim j) ----------
    const int halfk = tid / 128, j = tid & 127;
    for (int jj = j; jj < hd; jj += 128) {
        float acc[kMaxGroup];
#pragma unroll
        for (int g = 0; g < kMaxGroup; ++g) acc[g] = 0.0f;
        const int mid = (ns + 1) / 2;
        const int lo = halfk ? mid : 0, hi = halfk ? ns : mid;
        for (int s = lo; s < hi; ++s) {
            const float vj = kv_row(A.meta, sess, s0 + s, kvdim, 1)[(int64_t)kh * hd + jj];
#pragma unroll
            for (int g = 0; g < kMaxGroup; ++g)
                if (g < G) acc[g] = __builtin_fmaf(sc[g][s], vj, acc[g]);
        }
#pragma unroll
        for (int g = 0; g < kMaxGroup; ++g)
            if (g < G) ov[halfk][g * hd + jj] = acc[g];
    }
    __syncthreads();
    for (int i = tid; i < G * hd; i += 256) {
        const int g = i / hd, jj = i - g * hd;
        float *p = partial(part, row, kh * G + g, sp, A.heads, nsplit, hd);
        p[4 + jj] = ov[0][i] + ov[1][i];
    }
}


// Fast split kernel for head_dim 64 / 128: every K and V element of the
// split is loaded by exactly one thread with independent float4 loads, so a
// split costs one round of memory latency per pass.
//  scores: thread t -> key t/4 of the split, dims [(t%4)*HD/4, +HD/4)
//  values: thread t -> dims 4*(t%(HD/4)) .. +3, keys t/(HD/4) + KG*i
template <int HD>
__global__ __launch_bounds__(256) void attn_split_fast_kernel(const AttnArgs A, float *__restrict__ part,
                                                              int nsplit) {
    constexpr int QD = HD / 4;           // dims per scoring thread
    constexpr int DG = HD / 4;           // float4 dim groups in the value pass
    constexpr int KG = 256 / DG;         // key groups in the value pass
    constexpr int KPG = kSplit / KG;     // keys per value thread
    __shared__ float qs[kMaxGroup * HD];
    __shared__ float sc[kMaxGroup][kSplit];
    __shared__ float4 red[KG][kMaxGroup][DG];

    const int row = blockIdx.x, kh = blockIdx.y, sp = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63;
    const int kvdim = A.kv_heads * HD, G = A.heads / A.kv_heads;
    const int pos = A.meta.pos[row], sess = A.meta.sess[row];
    const int len = pos + 1, s0 = sp * kSplit, s1 = min(len, s0 + kSplit), ns = s1 - s0;
    if (ns <= 0) {
        for (int i = tid; i < G * (HD + 4); i += 256) {
            const int g = i / (HD + 4), k = i - g * (HD + 4);
            float *p = partial(part, row, kh * G + g, sp, A.heads, nsplit, HD);
            p[k] = k == 0 ? -FLT_MAX : 0.0f;
        }
        return;
    }
    // Every K and V load of the split at once (one round of memory latency).
    const int part4 = tid & 3;
    float4 kr[QD / 4];
    {
        const int s = tid >> 2, sk = s < ns ? s : 0;  // clamp: load a valid row, drop below
        const float *k = kv_row(A.meta, sess, s0 + sk, kvdim, 0) + (int64_t)kh * HD + part4 * QD;
#pragma unroll
        for (int u = 0; u < QD / 4; ++u) kr[u] = ((const float4 *)k)[u];
    }
    const int dg = tid % DG, kg = tid / DG;
    float4 vr[KPG];
#pragma unroll
    for (int i = 0; i < KPG; ++i) {
        const int s = kg + KG * i;
        const int sk = s < ns ? s : 0;
        vr[i] = ((const float4 *)(kv_row(A.meta, sess, s0 + sk, kvdim, 1) + (int64_t)kh * HD))[dg];
    }
    for (int i = tid; i < G * HD; i += 256) {
        const int g = i / HD, j = i - g * HD;
        qs[i] = A.q[(int64_t)row * A.heads * HD + (int64_t)(kh * G + g) * HD + j];
    }
    // Keep the V loads ahead of the barrier (the compiler would sink them).
#pragma unroll
    for (int i = 0; i < KPG; ++i) asm volatile("" ::"v"(vr[i].x), "v"(vr[i].y), "v"(vr[i].z), "v"(vr[i].w));
    __syncthreads();
    const float scale = (float)(1.0 / sqrt((double)HD));

    // ---- scores -------------------------------------------------------------
    {
        const int s = tid >> 2;
#pragma unroll
        for (int g = 0; g < kMaxGroup; ++g) {
            if (g >= G) break;
            const float *q = qs + g * HD + part4 * QD;
            float d = 0.0f;
#pragma unroll
            for (int u = 0; u < QD / 4; ++u) {
                d = __builtin_fmaf(q[4 * u + 0], kr[u].x, d);
                d = __builtin_fmaf(q[4 * u + 1], kr[u].y, d);
                d = __builtin_fmaf(q[4 * u + 2], kr[u].z, d);
                d = __builtin_fmaf(q[4 * u + 3], kr[u].w, d);
            }
            d += __shfl_xor(d, 1, 64);
            d += __shfl_xor(d, 2, 64);
            if (part4 == 0 && s < ns) sc[g][s] = d * scale;
        }
    }
    __syncthreads();

    // ---- per-head split max and FP64 sum (one wave per head) ----------------
    const int wave = tid >> 6;
    for (int g = wave; g < G; g += 4) {
        float m = -FLT_MAX;
        if (lane < ns) m = sc[g][lane];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        double e = 0.0;
        if (lane < ns) {
            e = exp((double)sc[g][lane] - (double)m);
            sc[g][lane] = (float)e;
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) e += __shfl_xor(e, o, 64);
        if (lane == 0) {
            float *p = partial(part, row, kh * G + g, sp, A.heads, nsplit, HD);
            p[0] = m;
            *(double *)(p + 2) = e;
        }
    }
    __syncthreads();

    // ---- values: every head of the group at once, one tree ------------------
    {
        float4 acc[kMaxGroup];
#pragma unroll
        for (int g = 0; g < kMaxGroup; ++g) acc[g] = make_float4(0.f, 0.f, 0.f, 0.f);
        // Per head: its KPG weights are read from LDS together, then the
        // FMAs (keys in order, as the reduction below expects).
#pragma unroll
        for (int g = 0; g < kMaxGroup; ++g) {
            if (g < G) {
                float w[KPG];
#pragma unroll
                for (int i = 0; i < KPG; ++i) {
                    const int s = kg + KG * i;
                    w[i] = s < ns ? sc[g][s] : 0.0f;
                }
#pragma unroll
                for (int i = 0; i < KPG; ++i) {
                    acc[g].x = __builtin_fmaf(w[i], vr[i].x, acc[g].x);
                    acc[g].y = __builtin_fmaf(w[i], vr[i].y, acc[g].y);
                    acc[g].z = __builtin_fmaf(w[i], vr[i].z, acc[g].z);
                    acc[g].w = __builtin_fmaf(w[i], vr[i].w, acc[g].w);
                }
            }
        }
#pragma unroll
        for (int g = 0; g < kMaxGroup; ++g)
            if (g < G) red[kg][g][dg] = acc[g];
    }
    __syncthreads();
    for (int t = tid; t < G * DG; t += 256) {
        const int g = t / DG, j = t - g * DG;
        float4 o = red[0][g][j];
        for (int k2 = 1; k2 < KG; ++k2) {
            const float4 u = red[k2][g][j];
            o.x += u.x, o.y += u.y, o.z += u.z, o.w += u.w;
        }
        float *p = partial(part, row, kh * G + g, sp, A.heads, nsplit, HD);
        ((float4 *)(p + 4))[j] = o;
    }
}

constexpr int kMergeChunk = 256;  // splits per pass of the weight table
constexpr int kMergePairs = kMaxGroup * kMaxHd / 256;
constexpr int kMergeBatch = 16;   // partial loads in flight per (head, dim) pair

// Merge of at most 64 split partials for head h of a row by one wave, with no
// barrier: the same arithmetic and order as merge_splits below (lane i holds
// split i's factor; each lane's dims accumulate the splits in order).
__device__ __forceinline__ void merge_wave(const AttnArgs &A, const float *part, int nsplit, int row, int h, int hd,
                                           int used) {
    // One round of loads: every split's {m, l} (lane = split) and, for
    // used <= kMergeBatch, the o values of this lane's first two dims.
    const int lane = threadIdx.x & 63;
    const float *pb = partial((float *)part, row, h, 0, A.heads, nsplit, hd) + 4;
    float mi = 0.0f;
    double li = 0.0;
    if (lane < used) {
        const float *p = partial((float *)part, row, h, lane, A.heads, nsplit, hd);
        mi = p[0];
        li = *(const double *)(p + 2);
    }
    float v0[kMergeBatch], v1[kMergeBatch];
    const bool pre = used <= kMergeBatch;
    if (pre) {
        const int j0 = min(lane, hd - 1), j1 = min(lane + 64, hd - 1);
#pragma unroll
        for (int b = 0; b < kMergeBatch; ++b) {
            const int64_t off = (int64_t)min(b, used - 1) * (hd + 4);
            v0[b] = pb[off + j0];
            v1[b] = pb[off + j1];
        }
    }
    float M = lane < used ? mi : -FLT_MAX;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
    double l = lane < used ? li * exp((double)mi - (double)M) : 0.0;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) l += __shfl_xor(l, o, 64);
    const double lse = (double)M + log(l);
    const float cf = lane < used ? (float)exp((double)mi - lse) : 0.0f;
    for (int j = lane; j < hd; j += 64) {
        float o = 0.0f;
        if (pre && j < lane + 128) {
            const float *v = j == lane ? v0 : v1;
#pragma unroll
            for (int b = 0; b < kMergeBatch; ++b)
                if (b < used)
                    o = __builtin_fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(cf), b)), v[b], o);
        } else {
            for (int i0 = 0; i0 < used; i0 += kMergeBatch) {
                float v[kMergeBatch];
#pragma unroll
                for (int b = 0; b < kMergeBatch; ++b) v[b] = pb[(int64_t)min(i0 + b, used - 1) * (hd + 4) + j];
#pragma unroll
                for (int b = 0; b < kMergeBatch; ++b)
                    if (i0 + b < used)
                        o = __builtin_fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(cf), i0 + b)), v[b],
                                           o);
            }
        }
        A.out[(int64_t)row * A.heads * hd + (int64_t)h * hd + j] = o;
    }
}

// Sum over splits i in [b0, b1) of cf[i] * pb[i * (hd + 4)] added to o by
// FMA in split order, with two batches of kMergeBatch loads in flight (the
// next batch loads while this one's FMAs run).
__device__ __forceinline__ float merge_range(const float *pb, int hd, const float *cf, int b0, int b1, float o) {
    if (b0 >= b1) return o;
    const int64_t st = hd + 4;
    const int last = b1 - 1;
    float va[kMergeBatch], vb[kMergeBatch];
#pragma unroll
    for (int b = 0; b < kMergeBatch; ++b) va[b] = pb[(int64_t)min(b0 + b, last) * st];
    for (int i0 = b0; i0 < b1; i0 += 2 * kMergeBatch) {
        const int i1 = i0 + kMergeBatch;
        if (i1 < b1) {
#pragma unroll
            for (int b = 0; b < kMergeBatch; ++b) vb[b] = pb[(int64_t)min(i1 + b, last) * st];
        }
#pragma unroll
        for (int b = 0; b < kMergeBatch; ++b)
            if (i0 + b < b1) o = __builtin_fmaf(cf[i0 + b], va[b], o);
        if (i1 >= b1) break;
        if (i1 + kMergeBatch < b1) {
#pragma unroll
            for (int b = 0; b < kMergeBatch; ++b) va[b] = pb[(int64_t)min(i1 + kMergeBatch + b, last) * st];
        }
#pragma unroll
        for (int b = 0; b < kMergeBatch; ++b)
            if (i1 + b < b1) o = __builtin_fmaf(cf[i1 + b], vb[b], o);
    }
    return o;
}

// Merge of split partials (m_i, l_i, o_i) for heads h0 .. h0+nh-1 of a row,
// by all 256 threads of the workgroup:
//   M = max_i m_i, l = sum_i l_i exp(m_i - M) (FP64), lse = M + log(l),
//   out_j = sum_i f32(exp(m_i - lse)) * o_i[j], FMA in split order.
// One wave per head forms M and l (lanes stride the splits, then a
// butterfly); the (head, dim) pairs spread over the threads, each pair
// keeping two batches of kMergeBatch splits in flight.  Up to 256 splits a
// lane loads all its {m, l} in one round.
template <bool GROUPS>
__device__ __forceinline__ void merge_splits(const AttnArgs &A, const float *part, int nsplit, int row, int h0,
                                             int nh, int hd, int used, float (*cf)[kMergeChunk], double *lse) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int g = wave; g < nh; g += 4) {
        const int h = h0 + g;
        float M = -FLT_MAX;
        double l = 0.0;
        if (used <= 256) {
            float mv[4];
            double lv[4];
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int i = lane + 64 * b;
                mv[b] = -FLT_MAX;
                lv[b] = 0.0;
                if (i < used) {
                    const float *p = partial((float *)part, row, h, i, A.heads, nsplit, hd);
                    mv[b] = p[0];
                    lv[b] = *(const double *)(p + 2);
                }
            }
#pragma unroll
            for (int b = 0; b < 4; ++b) M = fmaxf(M, mv[b]);
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
#pragma unroll
            for (int b = 0; b < 4; ++b)
                if (lane + 64 * b < used) l += lv[b] * exp((double)mv[b] - (double)M);
        } else {
            for (int i = lane; i < used; i += 64) M = fmaxf(M, partial((float *)part, row, h, i, A.heads, nsplit, hd)[0]);
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
            for (int i = lane; i < used; i += 64) {
                const float *p = partial((float *)part, row, h, i, A.heads, nsplit, hd);
                l += *(const double *)(p + 2) * exp((double)p[0] - (double)M);
            }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) l += __shfl_xor(l, o, 64);
        if (lane == 0) lse[g] = (double)M + log(l);
    }
    __syncthreads();
    float o[kMergePairs];
#pragma unroll
    for (int k = 0; k < kMergePairs; ++k) o[k] = 0.0f;
    // Summation order of a (head, dim) pair, fixed by head_dim and the
    // head's split count alone, so a row's output does not depend on the
    // other rows of its step: up to kFusedSplits splits (and past
    // kMergeChunk) one FMA chain over the splits in order, the fused
    // kernel's order; in between, ng groups of consecutive splits, each
    // summed from zero, then the group sums added in group order.
    // GROUPS (the one-head combine of decode-sized batches): the groups run
    // on separate threads, so none idles; otherwise one thread sums its
    // pair's groups one after another, in the same order.
    __shared__ float gs[GROUPS ? 256 : 1];
    const int ng = hd <= 128 && 256 % hd == 0 && used > kFusedSplits && used <= kMergeChunk ? 256 / hd : 1;
    for (int c0 = 0; c0 < used; c0 += kMergeChunk) {
        const int cnt = min(kMergeChunk, used - c0);
        for (int t = tid; t < nh * cnt; t += 256) {
            const int g = t / cnt, i = t - g * cnt;
            cf[g][i] = (float)exp((double)partial((float *)part, row, h0 + g, c0 + i, A.heads, nsplit, hd)[0] - lse[g]);
        }
        __syncthreads();
        const int per = (cnt + ng - 1) / ng;
        if (GROUPS && ng > 1 && nh == 1) {
            // Thread group q of ng sums splits [q*per, (q+1)*per) of its
            // (head, dim) pair; the groups' sums are added in group order.
            const int j = tid % hd, q = tid / hd;
            const float *pb = partial((float *)part, row, h0, c0, A.heads, nsplit, hd) + 4 + j;
            gs[tid] = merge_range(pb, hd, cf[0], q * per, min(cnt, q * per + per), 0.0f);
            __syncthreads();
            if (q == 0) {
                float v = gs[j];
                for (int r = 1; r < ng; ++r) v += gs[r * hd + j];
                A.out[(int64_t)row * A.heads * hd + (int64_t)h0 * hd + j] = v;
            }
            return;
        }
#pragma unroll
        for (int k = 0; k < kMergePairs; ++k) {
            const int pidx = tid + 256 * k;
            if (pidx >= nh * hd) break;
            const int g = pidx / hd, j = pidx - g * hd;
            const float *pb = partial((float *)part, row, h0 + g, c0, A.heads, nsplit, hd) + 4 + j;
            if (ng > 1) {
                float v = merge_range(pb, hd, cf[g], 0, min(cnt, per), 0.0f);
                for (int q = 1; q < ng; ++q) v += merge_range(pb, hd, cf[g], q * per, min(cnt, q * per + per), 0.0f);
                o[k] = v;
            } else {
                o[k] = merge_range(pb, hd, cf[g], 0, cnt, o[k]);
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int k = 0; k < kMergePairs; ++k) {
        const int pidx = tid + 256 * k;
        if (pidx >= nh * hd) break;
        const int g = pidx / hd, j = pidx - g * hd;
        A.out[(int64_t)row * A.heads * hd + (int64_t)(h0 + g) * hd + j] = o[k];
    }
}

// Fused split + combine for decode-sized batches, head_dim 64 / 128.
// Workgroup (row, kv head, split) loads its K and V rows together (one round
// of memory latency), scores all query heads of the GQA group, writes its
// partial {m, l, o}, and the last split of a (row, kv head) to finish merges
// all partials of the group with the combine rule (counter per (row, kv
// head), reset by the merging workgroup, so the kernel replays without
// clearing).
//  scores: thread t -> key t/4 of the split, dims [(t%4)*HD/4, +HD/4)
//  values: thread t -> dims 4*(t%(HD/4)) .. +3, keys t/(HD/4) + KG*i
template <int HD>
__global__ __launch_bounds__(256) void attn_fused_kernel(const AttnArgs A, float *__restrict__ part, int nsplit,
                                                         int32_t *__restrict__ counters) {
    constexpr int QD = HD / 4;        // dims per scoring thread
    constexpr int DG = HD / 4;        // float4 dim groups in the value pass
    constexpr int KG = 256 / DG;      // key groups in the value pass
    constexpr int KPG = kSplit / KG;  // keys per value thread
    __shared__ float qs[kMaxGroup * HD];
    __shared__ float sc[kMaxGroup][kSplit];
    __shared__ float4 red[KG][kMaxGroup][DG];
    __shared__ int last;

    const int row = blockIdx.x, kh = blockIdx.y, sp = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kvdim = A.kv_heads * HD, G = A.heads / A.kv_heads;
    const int pos = A.meta.pos[row], sess = A.meta.sess[row];
    const int len = pos + 1, s0 = sp * kSplit, s1 = min(len, s0 + kSplit), ns = s1 - s0;
    if (ns <= 0) return;  // past the row's positions: no partial, no count
    const int used = (len + kSplit - 1) / kSplit;

    // Page bases of the split's two pages; then every K and V load at once.
    const int32_t *pt = A.meta.pages + (int64_t)sess * A.meta.pt_stride + s0 / kPageTokens;
    const float *pb0 = A.meta.kv_pool + (int64_t)pt[0] * A.meta.page_elems +
                       (int64_t)A.meta.layer * 2 * kPageTokens * kvdim + (int64_t)kh * HD;
    const float *pb1 = ns > kPageTokens ? A.meta.kv_pool + (int64_t)pt[1] * A.meta.page_elems +
                                              (int64_t)A.meta.layer * 2 * kPageTokens * kvdim + (int64_t)kh * HD
                                        : pb0;
    auto key_row = [&](int s, int which) {  // s < ns
        const float *pb = s < kPageTokens ? pb0 : pb1;
        return pb + (int64_t)which * kPageTokens * kvdim + (int64_t)(s & (kPageTokens - 1)) * kvdim;
    };
    const int ks = tid >> 2, part4 = tid & 3;
    float4 kr[QD / 4];
    {
        const float *k = key_row(ks < ns ? ks : 0, 0) + part4 * QD;
#pragma unroll
        for (int u = 0; u < QD / 4; ++u) kr[u] = ((const float4 *)k)[u];
    }
    const int dg = tid % DG, kg = tid / DG;
    float4 vr[KPG];
#pragma unroll
    for (int i = 0; i < KPG; ++i) {
        const int sv = kg + KG * i;
        vr[i] = ((const float4 *)key_row(sv < ns ? sv : 0, 1))[dg];
    }
    for (int i = tid; i < G * HD; i += 256) {
        const int g = i / HD, j = i - g * HD;
        qs[i] = A.q[(int64_t)row * A.heads * HD + (int64_t)(kh * G + g) * HD + j];
    }
    // The V rows are consumed only after the softmax; without this the
    // compiler sinks their loads past the barrier, which then costs a second
    // round of memory latency instead of overlapping the K loads.
#pragma unroll
    for (int i = 0; i < KPG; ++i) asm volatile("" ::"v"(vr[i].x), "v"(vr[i].y), "v"(vr[i].z), "v"(vr[i].w));
    __syncthreads();
    const float scale = (float)(1.0 / sqrt((double)HD));

    // ---- scores -------------------------------------------------------------
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g) {
        if (g >= G) break;
        const float *q = qs + g * HD + part4 * QD;
        float d = 0.0f;
#pragma unroll
        for (int u = 0; u < QD / 4; ++u) {
            d = __builtin_fmaf(q[4 * u + 0], kr[u].x, d);
            d = __builtin_fmaf(q[4 * u + 1], kr[u].y, d);
            d = __builtin_fmaf(q[4 * u + 2], kr[u].z, d);
            d = __builtin_fmaf(q[4 * u + 3], kr[u].w, d);
        }
        d += __shfl_xor(d, 1, 64);
        d += __shfl_xor(d, 2, 64);
        if (part4 == 0 && ks < ns) sc[g][ks] = d * scale;
    }
    __syncthreads();

    // ---- per-head split max and FP64 sum (one wave per head) ----------------
    for (int g = wave; g < G; g += 4) {
        float m = -FLT_MAX;
        if (lane < ns) m = sc[g][lane];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        double e = 0.0;
        if (lane < ns) {
            e = exp((double)sc[g][lane] - (double)m);
            sc[g][lane] = (float)e;
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) e += __shfl_xor(e, o, 64);
        if (lane == 0) {
            float *p = partial(part, row, kh * G + g, sp, A.heads, nsplit, HD);
            p[0] = m;
            *(double *)(p + 2) = e;
        }
    }
    __syncthreads();

    // ---- values: every head of the group at once, one tree ------------------
    {
        float4 acc[kMaxGroup];
#pragma unroll
        for (int g = 0; g < kMaxGroup; ++g) acc[g] = make_float4(0.f, 0.f, 0.f, 0.f);
        // Per head: its KPG weights are read from LDS together, then the
        // FMAs (keys in order, as the reduction below expects).
#pragma unroll
        for (int g = 0; g < kMaxGroup; ++g) {
            if (g < G) {
                float w[KPG];
#pragma unroll
                for (int i = 0; i < KPG; ++i) {
                    const int sv = kg + KG * i;
                    w[i] = sv < ns ? sc[g][sv] : 0.0f;
                }
#pragma unroll
                for (int i = 0; i < KPG; ++i) {
                    acc[g].x = __builtin_fmaf(w[i], vr[i].x, acc[g].x);
                    acc[g].y = __builtin_fmaf(w[i], vr[i].y, acc[g].y);
                    acc[g].z = __builtin_fmaf(w[i], vr[i].z, acc[g].z);
                    acc[g].w = __builtin_fmaf(w[i], vr[i].w, acc[g].w);
                }
            }
        }
#pragma unroll
        for (int g = 0; g < kMaxGroup; ++g)
            if (g < G) red[kg][g][dg] = acc[g];
    }
    __syncthreads();
    for (int t = tid; t < G * DG; t += 256) {
        const int g = t / DG, j = t - g * DG;
        float4 o = red[0][g][j];
        for (int k2 = 1; k2 < KG; ++k2) {
            const float4 u = red[k2][g][j];
            o.x += u.x, o.y += u.y, o.z += u.z, o.w += u.w;
        }
        float *p = partial(part, row, kh * G + g, sp, A.heads, nsplit, HD);
        ((float4 *)(p + 4))[j] = o;
    }

    // ---- the last split of (row, kv head) merges ------------------------------
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");  // publish this split's partials
    __syncthreads();
    int32_t *cnt = counters + (int64_t)row * A.kv_heads + kh;
    if (tid == 0) last = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == used - 1;
    __syncthreads();
    if (!last) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    if (tid == 0) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // used <= kFusedSplits <= 64: one wave per head merges on its own.
    for (int g = wave; g < G; g += 4) merge_wave(A, part, nsplit, row, kh * G + g, HD, used);
}

// lse and the weighted sum of split partials for one (row, head); split i
// covers positions [i*split_len, (i+1)*split_len).  GROUPS (decode-sized
// batches): thread groups share a head's split range; larger batches keep
// the smaller register footprint, many workgroups being resident anyway.
// Both give the same bits (merge_splits).
template <bool GROUPS>
__global__ __launch_bounds__(256) void attn_combine_kernel(const AttnArgs A, const float *__restrict__ part,
                                                           int nsplit, int split_len) {
    __shared__ float cf[kMaxGroup][kMergeChunk];
    __shared__ double lse[kMaxGroup];
    const int row = blockIdx.x, h = blockIdx.y;
    const int len = A.meta.pos[row] + 1;
    const int used = min(nsplit, (len + split_len - 1) / split_len);
    merge_splits<GROUPS>(A, part, nsplit, row, h, 1, A.head_dim, used, cf, lse);
}

// The same for heads h0 .. h0+nh-1 of a row per workgroup (nh <= kMaxGroup):
// fewer, fuller workgroups for prefill-sized steps.
__global__ __launch_bounds__(256) void attn_combine_heads_kernel(const AttnArgs A, const float *__restrict__ part,
                                                                 int nsplit, int split_len, int nh) {
    __shared__ float cf[kMaxGroup][kMergeChunk];
    __shared__ double lse[kMaxGroup];
    const int row = blockIdx.x, h0 = blockIdx.y * nh;
    const int len = A.meta.pos[row] + 1;
    const int used = min(nsplit, (len + split_len - 1) / split_len);
    merge_splits<false>(A, part, nsplit, row, h0, nh, A.head_dim, used, cf, lse);
}

// ------------------------------------------------------------ prefill
// Causal attention for prefill-sized steps on FP32 MFMA
// (v_mfma_f32_16x16x4f32), flash style.  Workgroup (query tile, kv head,
// key split): a tile is up to 16 consecutive rows of one session, whose
// positions are consecutive.  Wave w takes query head kh*G + w for the
// tile's rows (G > 4: a second pass over the keys for heads 4..7; waves past
// G only stage), so every K/V row staged in LDS serves all the GQA group's
// heads and all 16 rows -- the split kernel re-reads K/V per row.
//  S^T = K Q^T per 16-key step: MFMA step s feeds lane group g = lane/16
//  the head dims (HD/4)g + s, so a lane's q and K values are contiguous; the
//  result gives lane l the scores S[q = l%16][key = 4(l/16) + r], r = 0..3.
//  P V: those registers are P's A operand, MFMA step r taking keys
//  4(l/16) + r; lane l then holds O[q = 4(l/16) + rr][dim = 16b + l%16].
//  Per query row an online softmax: running max m (f32), FP64 sum l of
//  f32 exp(s - m), O rescaled by f32 exp(m_old - m_new) when the max grows.
// Scores are f32 dot(q, k) * f32(1/sqrt(hd)) as in attend (M:5293-5352);
// the split's {m, l, o} feed attn_combine_kernel, split sp covering keys
// [sp*ks, (sp+1)*ks).  K/V chunks of 64 keys are double buffered through
// registers: the next chunk's loads are in flight during this chunk's MFMAs.
constexpr int kFlashChunk = 32;   // keys staged in LDS per pass
constexpr int kFlashFill = 512;   // workgroups the key splits aim for
typedef float flashx4 __attribute__((ext_vector_type(4)));

template <int HD>
__global__ __launch_bounds__(256) void attn_flash_kernel(const AttnArgs A, float *__restrict__ part, int nsplit,
                                                         int ks) {
    constexpr int LDH = HD + 4;           // LDS row stride (floats)
    constexpr int QF = HD / 4;            // q values per lane
    constexpr int NB = HD / 16;           // 16-dim output blocks
    constexpr int CH = kFlashChunk;
    constexpr int D4 = HD / 4;            // float4 per K/V row
    constexpr int LPT = CH * D4 / 256;    // float4 per thread per chunk (K and V each)
    __shared__ __attribute__((aligned(16))) float Ks[CH * LDH];
    __shared__ __attribute__((aligned(16))) float Vs[CH * LDH];

    const int tile = blockIdx.x, kh = blockIdx.y, sp = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, gq = lane >> 4;
    static_assert(kAttnTileRows == 16, "a query tile is one 16-row MFMA operand");
    const int r0 = A.tiles[2 * tile], cnt = A.tiles[2 * tile + 1];
    const int sess = A.meta.sess[r0], pos0 = A.meta.pos[r0];
    const int kvdim = A.kv_heads * HD, G = A.heads / A.kv_heads;
    const int k_lo = sp * ks, k_hi = min(k_lo + ks, pos0 + cnt);
    if (k_lo >= k_hi) return;  // no row of the tile reaches this split
    const float scale = (float)(1.0 / sqrt((double)HD));
    const int32_t *pt = A.meta.pages + (int64_t)sess * A.meta.pt_stride;
    const float *lbase = A.meta.kv_pool + (int64_t)A.meta.layer * 2 * kPageTokens * kvdim + (int64_t)kh * HD;

    for (int g0 = 0; g0 < G; g0 += 4) {
        // K/V chunk registers, indexed only by unrolled loops (native vector
        // type: HIP's float4 struct copies would go through scratch).
        flashx4 kr[LPT], vr[LPT];
        const int g = g0 + wave;
        const bool active = g < G;
        const int h = kh * G + (active ? g : 0);
        float qf[QF];
        {
            const float *qp = A.q + (int64_t)(r0 + min(li, cnt - 1)) * A.heads * HD + (int64_t)h * HD + QF * gq;
#pragma unroll
            for (int u = 0; u < QF; u += 4) {
                const flashx4 t = *(const flashx4 *)(qp + u);
                qf[u] = t[0], qf[u + 1] = t[1], qf[u + 2] = t[2], qf[u + 3] = t[3];
            }
        }
        flashx4 o[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) o[b] = flashx4{0.f, 0.f, 0.f, 0.f};
        float m = -FLT_MAX;
        double l = 0.0;

        {
            const int NEXT = k_lo;
#pragma unroll
            for (int i = 0; i < LPT; ++i) {
                const int f = tid + 256 * i, key = min(NEXT + f / D4, k_hi - 1), d4 = f % D4;
                const float *row = lbase + (int64_t)pt[key / kPageTokens] * A.meta.page_elems +
                                   (int64_t)(key % kPageTokens) * kvdim;
                kr[i] = *(const flashx4 *)(row + 4 * d4);
                vr[i] = *(const flashx4 *)(row + (int64_t)kPageTokens * kvdim + 4 * d4);
            }
        }
        for (int c0 = k_lo; c0 < k_hi; c0 += CH) {
            __syncthreads();  // the previous chunk's LDS reads are done
#pragma unroll
            for (int i = 0; i < LPT; ++i) {
                const int f = tid + 256 * i, k = f / D4, d4 = f % D4;
                *(flashx4 *)(Ks + k * LDH + 4 * d4) = kr[i];
                *(flashx4 *)(Vs + k * LDH + 4 * d4) = vr[i];
            }
            __syncthreads();
            // The next chunk (keys clamped to the split: past its end this
            // re-reads the last key, unused).
            {
                const int NEXT = c0 + CH;
#pragma unroll
            for (int i = 0; i < LPT; ++i) {
                const int f = tid + 256 * i, key = min(NEXT + f / D4, k_hi - 1), d4 = f % D4;
                const float *row = lbase + (int64_t)pt[key / kPageTokens] * A.meta.page_elems +
                                   (int64_t)(key % kPageTokens) * kvdim;
                kr[i] = *(const flashx4 *)(row + 4 * d4);
                vr[i] = *(const flashx4 *)(row + (int64_t)kPageTokens * kvdim + 4 * d4);
            }
            }
            if (!active) continue;
            for (int st = 0; st < CH; st += 32) {
                if (c0 + st >= k_hi) break;
                // ---- S^T = K Q^T for 32 keys: two independent 16-key chains ----
                flashx4 sa = {0.f, 0.f, 0.f, 0.f}, sb = {0.f, 0.f, 0.f, 0.f};
                const float *ka = Ks + (st + li) * LDH + QF * gq, *kb = ka + 16 * LDH;
#pragma unroll
                for (int u = 0; u < QF; u += 4) {
                    const flashx4 va = *(const flashx4 *)(ka + u), vb = *(const flashx4 *)(kb + u);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        sa = __builtin_amdgcn_mfma_f32_16x16x4f32(va[e], qf[u + e], sa, 0, 0, 0);
                        sb = __builtin_amdgcn_mfma_f32_16x16x4f32(vb[e], qf[u + e], sb, 0, 0, 0);
                    }
                }
                // ---- causal mask, online softmax of query row li ----
                float sv[8], p[8];
                bool ok[8];
                float tm = -FLT_MAX;
#pragma unroll
                for (int r = 0; r < 8; ++r) {
                    const int key = c0 + st + 16 * (r >> 2) + 4 * gq + (r & 3);
                    ok[r] = key < k_hi && key <= pos0 + li;
                    sv[r] = (r < 4 ? sa[r & 3] : sb[r & 3]) * scale;
                    if (ok[r]) tm = fmaxf(tm, sv[r]);
                }
                tm = fmaxf(tm, __shfl_xor(tm, 16, 64));
                tm = fmaxf(tm, __shfl_xor(tm, 32, 64));
                const float mn = fmaxf(m, tm);
                const float alpha = expf(m - mn);
                double ps = 0.0;
#pragma unroll
                for (int r = 0; r < 8; ++r) {
                    p[r] = ok[r] ? expf(sv[r] - mn) : 0.0f;
                    ps += (double)p[r];
                }
                ps += __shfl_xor(ps, 16, 64);
                ps += __shfl_xor(ps, 32, 64);
                l = l * (double)alpha + ps;
                m = mn;
                if (__any(alpha != 1.0f)) {  // some row's max grew: rescale O
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr) {
                        const float a = __shfl(alpha, 4 * gq + rr, 64);
#pragma unroll
                        for (int b = 0; b < NB; ++b) o[b][rr] *= a;
                    }
                }
                // ---- O += P V (keys st + 16*half + 4*gq + r at MFMA step r) ----
#pragma unroll
                for (int r = 0; r < 8; ++r) {
                    const float *vp = Vs + (st + 16 * (r >> 2) + 4 * gq + (r & 3)) * LDH + li;
#pragma unroll
                    for (int b = 0; b < NB; ++b)
                        o[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(p[r], vp[16 * b], o[b], 0, 0, 0);
                }
            }
        }
        if (active) {
            // {m, l} of row li (held by every lane group), o of rows 4*gq + rr.
            if (gq == 0 && li < cnt && pos0 + li + 1 > k_lo) {
                float *pp = partial(part, r0 + li, h, sp, A.heads, nsplit, HD);
                pp[0] = m;
                *(double *)(pp + 2) = l;
            }
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const int j = 4 * gq + rr;
                if (j < cnt && pos0 + j + 1 > k_lo) {
                    float *pp = partial(part, r0 + j, h, sp, A.heads, nsplit, HD) + 4 + li;
#pragma unroll
                    for (int b = 0; b < NB; ++b) pp[16 * b] = o[b][rr];
                }
            }
        }
    }
}

}  // namespace

int attention_splits(int32_t max_len) { return (max_len + kSplit - 1) / kSplit; }

size_t attention_scratch_bytes(int32_t n, int32_t heads, int32_t head_dim, int32_t max_len) {
    return (size_t)n * heads * attention_splits(max_len) * (head_dim + 4) * sizeof(float);
}

int launch_attention(hipStream_t s, const AttnArgs &a, float *scratch, int32_t *counters) {
    if (a.n <= 0) return SRQ_OK;
    if (a.head_dim > kMaxHd || a.head_dim < 1) return fail(SRQ_EINVAL, "attention: head_dim %d unsupported", a.head_dim);
    const int G = a.heads / a.kv_heads;
    if (G > kMaxGroup) return fail(SRQ_EINVAL, "attention: %d query heads per KV head exceed %d", G, kMaxGroup);
    const int nsplit = attention_splits(a.max_len);
    if (nsplit > 1024) return fail(SRQ_EINVAL, "attention: %d positions exceed the split table", a.max_len);
    const dim3 grid(a.n, a.kv_heads, nsplit);
    const bool fast = a.head_dim == 128 || a.head_dim == 64;
    if (fast && a.tiles && a.ntiles > 0 && a.n >= 32 && a.n >= 8 * a.ntiles) {
        // Prefill-sized steps: MFMA flash tiles, key splits sized so the
        // grid reaches about kFlashFill workgroups, then the combine.
        const int64_t wgs = (int64_t)a.ntiles * a.kv_heads;
        const int want = (int)std::max<int64_t>(1, (kFlashFill + wgs - 1) / wgs);
        // Split lengths are multiples of kSplit, so there are never more
        // splits than attention_scratch_bytes provides for.
        int ks = (a.max_len + want - 1) / want;
        ks = std::max(kSplit, (ks + kSplit - 1) / kSplit * kSplit);
        const int fsplit = (a.max_len + ks - 1) / ks;
        if (fsplit > nsplit) return fail(SRQ_EINVAL, "attention: %d key splits exceed the scratch's %d", fsplit, nsplit);
        const dim3 fg(a.ntiles, a.kv_heads, fsplit);
        if (a.head_dim == 128)
            attn_flash_kernel<128><<<fg, 256, 0, s>>>(a, scratch, fsplit, ks);
        else
            attn_flash_kernel<64><<<fg, 256, 0, s>>>(a, scratch, fsplit, ks);
        SRQ_HIP(hipGetLastError());
        int nh = std::min(kMaxGroup, a.heads);
        while (a.heads % nh) --nh;
        attn_combine_heads_kernel<<<dim3(a.n, a.heads / nh), 256, 0, s>>>(a, scratch, fsplit, ks, nh);
        SRQ_HIP(hipGetLastError());
        return SRQ_OK;
    }
    if (fast && a.n <= kFusedRows && nsplit <= kFusedSplits) {
        // Decode-sized batches at short context: one launch, the last split
        // merges.  Each split then publishes its partials with an agent-scope
        // release (an L2 writeback on its XCD); past kFusedSplits splits those
        // cost more than the second launch of split + combine.
        if (a.head_dim == 128)
            attn_fused_kernel<128><<<grid, 256, 0, s>>>(a, scratch, nsplit, counters);
        else
            attn_fused_kernel<64><<<grid, 256, 0, s>>>(a, scratch, nsplit, counters);
        SRQ_HIP(hipGetLastError());
        return SRQ_OK;
    }
    if (a.head_dim == 128)
        attn_split_fast_kernel<128><<<grid, 256, 0, s>>>(a, scratch, nsplit);
    else if (a.head_dim == 64)
        attn_split_fast_kernel<64><<<grid, 256, 0, s>>>(a, scratch, nsplit);
    else
        attn_split_kernel<<<grid, 256, 0, s>>>(a, scratch, nsplit);
    SRQ_HIP(hipGetLastError());
    if (a.n <= kFusedRows)
        attn_combine_kernel<true><<<dim3(a.n, a.heads), 256, 0, s>>>(a, scratch, nsplit, kSplit);
    else
        attn_combine_kernel<false><<<dim3(a.n, a.heads), 256, 0, s>>>(a, scratch, nsplit, kSplit);
    SRQ_HIP(hipGetLastError());
    return SRQ_OK;
}

int attention_prepare() { return SRQ_OK; }

}  // namespace srq
