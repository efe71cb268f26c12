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
// l_i = sum exp(score - m_i) and o_i = sum f32(exp(score - m_i)) v_s (for
// head_dim 64 / 128 each of its four waves keeps such a partial over 16
// positions, and the split's partial merges those four the way the combine
// merges splits).  The combine forms lse = M + log(sum_i l_i exp(m_i - M))
// and out = sum_i f32(exp(m_i - lse)) o_i, which equals the reference's
// sum_s exp(score_s - lse) v_s up to f32 rounding of the factors.
#include <algorithm>
#include <cfloat>
#include <type_traits>

#include "srq_internal.h"

namespace srq {
namespace {

constexpr int kSplit = 64;     // positions per split (two pages)
constexpr int kMaxGroup = 8;   // query heads per KV head handled together
constexpr int kMaxHd = 256;
// Steps up to this many rows, over at most kFusedSplits splits, use the
// fused split+merge kernel; the others the split and combine kernels.  Both
// merge in the same order (merge_wave follows merge_splits), so which one a
// step takes does not change its bits.  Past kFusedSplits the fused
// kernel's one-wave merge of a head is the slower (7B decode, fused against
// split + combine: 425 / 421 tokens/s at 2k context, 376 / 395 at 4k, 325 /
// 354 at 8k); on 3B continuous-batching steps of up to 64 rows the fused
// kernel is the faster (1067-1072 against 1060 tokens/s).
constexpr int kFusedRows = 64;
constexpr int kFusedSplits = 48;
// The combine kernel's grouped variant (thread groups sharing a head's
// split range) serves steps up to this many rows.
constexpr int kGroupRows = 8;

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
    const int pos = A.meta.pos[row], sess = A.meta.one_sess ? 0 : A.meta.sess[row];
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


// The fused kernel's split partials travel between workgroups that may sit
// on different XCDs, each with its own L2.  They are written and read by
// agent-scope atomic stores and loads (written through to, and read from,
// the device's coherence point), so publishing them needs no L2 write-back
// and merging them no L2 invalidation: the writer waits for its stores to
// complete before it counts its split, and the merger loads only after the
// count says every split is in.
template <typename T>
__device__ __forceinline__ void publish(T *p, T v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ T fetch(const T *p) {
    return __hip_atomic_load(const_cast<T *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One step of a butterfly over a wave: this lane's value and the value of
// lane (lane ^ K), by DPP (K = 1, 2, 8), ds_swizzle (K = 4) and the gfx950
// permlane swaps (K = 16, 32) rather than LDS permutes.  a and b are the two
// values in some order; op(a, b) equals op(b, a) bit for bit for the sums
// and maxima below, so every lane holds what a __shfl_xor butterfly gives.
template <int K>
__device__ __forceinline__ void xor_pair(int v, int &a, int &b) {
    if constexpr (K == 1) {
        a = v, b = __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    } else if constexpr (K == 2) {
        a = v, b = __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    } else if constexpr (K == 4) {
        a = v, b = __builtin_amdgcn_ds_swizzle(v, 0x101F);  // bit mode, xor mask 4
    } else if constexpr (K == 8) {
        a = v, b = __builtin_amdgcn_mov_dpp(v, 0x128, 0xF, 0xF, false);  // row_ror 8
    } else if constexpr (K == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        a = r[0], b = r[1];
    } else {
        static_assert(K == 32, "lane distance");
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        a = r[0], b = r[1];
    }
}
template <int K>
__device__ __forceinline__ float xor_max(float v) {
    int a, b;
    xor_pair<K>(__float_as_int(v), a, b);
    return fmaxf(__int_as_float(a), __int_as_float(b));
}
template <int K>
__device__ __forceinline__ double xor_add(double v) {
    const int64_t u = __double_as_longlong(v);
    int alo, blo, ahi, bhi;
    xor_pair<K>((int)u, alo, blo);
    xor_pair<K>((int)(u >> 32), ahi, bhi);
    const double a = __longlong_as_double((int64_t)(uint32_t)alo | ((int64_t)ahi << 32));
    const double b = __longlong_as_double((int64_t)(uint32_t)blo | ((int64_t)bhi << 32));
    return a + b;
}
// Maximum and FP64 sum over the 64 lanes, in the order of a __shfl_xor
// butterfly with distances 32, 16, ..., 1.
__device__ __forceinline__ float wave_max(float v) {
    v = xor_max<32>(v), v = xor_max<16>(v), v = xor_max<8>(v);
    v = xor_max<4>(v), v = xor_max<2>(v), v = xor_max<1>(v);
    return v;
}
__device__ __forceinline__ double wave_sum(double v) {
    v = xor_add<32>(v), v = xor_add<16>(v), v = xor_add<8>(v);
    v = xor_add<4>(v), v = xor_add<2>(v), v = xor_add<1>(v);
    return v;
}

// Butterfly steps over lane distances K, 2K, ..., up to KMAX.
template <int K, int KMAX>
__device__ __forceinline__ float xor_max_from(float v) {
    if constexpr (K <= KMAX) return xor_max_from<2 * K, KMAX>(xor_max<K>(v));
    return v;
}
template <int K, int KMAX>
__device__ __forceinline__ double xor_add_from(double v) {
    if constexpr (K <= KMAX) return xor_add_from<2 * K, KMAX>(xor_add<K>(v));
    return v;
}
template <int K, int KMAX>
__device__ __forceinline__ float xor_fadd_from(float v) {
    if constexpr (K <= KMAX) {
        int a, b;
        xor_pair<K>(__float_as_int(v), a, b);
        return xor_fadd_from<2 * K, KMAX>(__int_as_float(a) + __int_as_float(b));
    }
    return v;
}

// LDS of split_partial: the GQA group's queries, each wave's softmax
// weights and each wave's partial over its keys.
constexpr int kSplitWaves = 8;                   // waves per split workgroup
constexpr int kSplitThreads = 64 * kSplitWaves;
constexpr int kWaveKeys = kSplit / kSplitWaves;  // keys per wave
constexpr int kKeyLanes = 64 / kWaveKeys;        // lanes per key while scoring
static_assert(kWaveKeys % 4 == 0 && kKeyLanes >= 4, "split layout");
template <int HD>
struct SplitStage {
    alignas(16) float qs[kMaxGroup * HD];
    alignas(16) float ps[kSplitWaves][kMaxGroup][kWaveKeys];  // [wave][head][key]
    float wm[kSplitWaves][kMaxGroup];                         // wave partials: max,
    double wl[kSplitWaves][kMaxGroup];                        //   FP64 sum,
    float wo[kSplitWaves][kMaxGroup][HD];                     //   weighted V sum
};

// Partial {m, l, o} of split sp of (row, kv head kh) for every query head of
// the group, head_dim 64 / 128, kSplitThreads threads.  All K and V rows of
// the split are loaded into registers at once (one round of memory
// latency).  Wave w takes keys 8w .. 8w+7 of the split for every head of the
// group:
//   scores: lane 8k + t holds the float4s t, t+8, t+16, ... of key k (so
//     one load instruction reads whole 128-byte lines of eight keys); per
//     head a dot over those dims (FMA in dim order), then the eight parts
//     added by a butterfly over distances 1, 2, 4, * f32(1/sqrt(hd)); lane
//     8k + t keeps head t (of four per pass)
//   wave softmax per head: m_w = max over its keys, e = exp((double)s - m_w),
//     l_w = FP64 butterfly sum, p = f32(e)
//   o_w[j] = sum over its keys of p_k v_k[j], FMA in key order; lane holds
//     dims HD/64 * lane + ...
// then wave w merges head w over the eight waves, in wave order:
//   m = max m_w, c_w = exp((double)m_w - m), l = sum l_w c_w (FP64,
//   butterfly over the eight), o[j] = sum f32(c_w) o_w[j] (FMA).
// Eight waves of eight keys rather than four of sixteen: each wave's
// dependent chain of scoring, softmax and P.V is half as long, and two
// waves share each SIMD.  Keys past the row's positions weigh nothing.
// COHERENT: stored with agent-scope stores (publish) for the fused merge,
// except that a row of one split stores its merged output itself.
// Returns false, writing nothing, for a split past the row's positions.
template <int HD, bool COHERENT>
__device__ __forceinline__ bool split_partial(const AttnArgs &A, float *part, int nsplit, int row, int kh, int sp,
                                              SplitStage<HD> &S) {
    constexpr int QV = HD / (4 * kKeyLanes);  // float4s of a key per scoring lane
    constexpr int DPL = HD / 64;              // V dims per lane
    typedef typename std::conditional<DPL == 2, float2, float>::type VDims;
    constexpr int QPT = (kMaxGroup * HD + kSplitThreads - 1) / kSplitThreads;  // query values per thread, at most
    static_assert(QV >= 1, "head_dim");
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kvdim = A.kv_heads * HD, G = A.heads / A.kv_heads;
    // The loads form a chain (row meta -> page table -> K/V): the queries,
    // which need only the arguments, go first, the row's position and
    // session together, then both page-table entries of the split together
    // (the second clamped into the session's row; used only when the split
    // spans two pages).
    float qv[QPT];
#pragma unroll
    for (int r = 0; r < QPT; ++r) {
        const int i = tid + kSplitThreads * r, g = i / HD, j = i - g * HD;
        qv[r] = i < G * HD ? A.q[(int64_t)row * A.heads * HD + (int64_t)(kh * G + g) * HD + j] : 0.0f;
    }
    const int pos = A.meta.pos[row], sess = A.meta.one_sess ? 0 : A.meta.sess[row];
    const int s0 = sp * kSplit, pi = s0 / kPageTokens;
    const int32_t *ptrow = A.meta.pages + (int64_t)sess * A.meta.pt_stride;
    const int pg0 = ptrow[min(pi, A.meta.pt_stride - 1)], pg1 = ptrow[min(pi + 1, A.meta.pt_stride - 1)];
    asm volatile("" ::"s"(pos), "s"(pg0), "s"(pg1));  // issue all of them before the exit test
    const int len = pos + 1, ns = min(len, s0 + kSplit) - s0;
    if (ns <= 0) return false;

    // Page bases of the split's two pages, then every K and V load at once.
    const int64_t lay = (int64_t)A.meta.layer * 2 * kPageTokens * kvdim + (int64_t)kh * HD;
    const float *pb0 = A.meta.kv_pool + (int64_t)pg0 * A.meta.page_elems + lay;
    const float *pb1 = A.meta.kv_pool + (int64_t)pg1 * A.meta.page_elems + lay;
    auto key_row = [&](int s, int which) {  // keys past ns read key 0 (finite, weight 0)
        s = s < ns ? s : 0;
        const float *pb = s < kPageTokens ? pb0 : pb1;
        return pb + (int64_t)which * kPageTokens * kvdim + (int64_t)(s & (kPageTokens - 1)) * kvdim;
    };
    const int kq = lane / kKeyLanes, qt = lane % kKeyLanes;  // scoring: key kq of the wave, part qt
    const int key0 = kWaveKeys * wave;
    float4 kr[QV];
    {
        const float4 *k = (const float4 *)key_row(key0 + kq, 0) + qt;
#pragma unroll
        for (int u = 0; u < QV; ++u) kr[u] = k[u * kKeyLanes];
    }
    VDims vr[kWaveKeys];
#pragma unroll
    for (int k = 0; k < kWaveKeys; ++k) vr[k] = ((const VDims *)key_row(key0 + k, 1))[lane];
#pragma unroll
    for (int r = 0; r < QPT; ++r)
        if (tid + kSplitThreads * r < G * HD) S.qs[tid + kSplitThreads * r] = qv[r];
    __syncthreads();

    const float scale = (float)(1.0 / sqrt((double)HD));
    const bool kvalid = key0 + kq < ns;
    for (int h0 = 0; h0 < G; h0 += 4) {
        const int nh = min(4, G - h0);
        // scores of this lane's key part for heads h0 .. h0+3 (slots past
        // the group repeat its last head, unused)
        int hs[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) hs[g] = min(h0 + g, G - 1);
        float d[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) d[g] = 0.0f;
#pragma unroll
        for (int u = 0; u < QV; ++u) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const float4 q = ((const float4 *)(S.qs + hs[g] * HD))[u * kKeyLanes + qt];
                d[g] = __builtin_fmaf(q.x, kr[u].x, d[g]);
                d[g] = __builtin_fmaf(q.y, kr[u].y, d[g]);
                d[g] = __builtin_fmaf(q.z, kr[u].z, d[g]);
                d[g] = __builtin_fmaf(q.w, kr[u].w, d[g]);
            }
        }
#pragma unroll
        for (int g = 0; g < 4; ++g) d[g] = xor_fadd_from<1, kKeyLanes / 2>(d[g]);
        // lane kKeyLanes*k + p: head h0 + p
        const float sc = (qt == 0 ? d[0] : qt == 1 ? d[1] : qt == 2 ? d[2] : d[3]) * scale;
        const bool valid = kvalid && qt < nh;
        float m = valid ? sc : -FLT_MAX;
        m = xor_max_from<kKeyLanes, 32>(m);
        double e = valid ? exp((double)sc - (double)m) : 0.0;
        const double l = xor_add_from<kKeyLanes, 32>(e);
        if (qt < nh) {
            S.ps[wave][h0 + qt][kq] = (float)e;
            if (kq == 0) {
                S.wm[wave][h0 + qt] = m;
                S.wl[wave][h0 + qt] = l;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // o_w of heads h0 .. h0+3 over the wave's keys (slots past the group
        // repeat its last head and are not stored)
        float o[4][DPL];
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int t = 0; t < DPL; ++t) o[g][t] = 0.0f;
#pragma unroll
        for (int k4 = 0; k4 < kWaveKeys / 4; ++k4) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const float4 pw = ((const float4 *)S.ps[wave][hs[g]])[k4];
                const float pk[4] = {pw.x, pw.y, pw.z, pw.w};
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if constexpr (DPL == 2) {
                        o[g][0] = __builtin_fmaf(pk[r], vr[4 * k4 + r].x, o[g][0]);
                        o[g][1] = __builtin_fmaf(pk[r], vr[4 * k4 + r].y, o[g][1]);
                    } else {
                        o[g][0] = __builtin_fmaf(pk[r], vr[4 * k4 + r], o[g][0]);
                    }
                }
            }
        }
#pragma unroll
        for (int g = 0; g < 4; ++g)
            if (g < nh)
#pragma unroll
                for (int t = 0; t < DPL; ++t) S.wo[wave][h0 + g][DPL * lane + t] = o[g][t];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    __syncthreads();

    // wave w merges head w over the eight waves
    for (int h = wave; h < G; h += kSplitWaves) {
        const int src = lane & (kSplitWaves - 1);
        const float mw = S.wm[src][h];
        const double lw = S.wl[src][h];
        const float M = xor_max_from<1, kSplitWaves / 2>(mw);
        const double c = exp((double)mw - (double)M);
        const double l = xor_add_from<1, kSplitWaves / 2>(lw * c);
        const float cf = (float)c;
        float o[DPL];
#pragma unroll
        for (int t = 0; t < DPL; ++t) o[t] = 0.0f;
#pragma unroll
        for (int w = 0; w < kSplitWaves; ++w) {
            const float cw = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cf), w));
#pragma unroll
            for (int t = 0; t < DPL; ++t) o[t] = __builtin_fmaf(cw, S.wo[w][h][DPL * lane + t], o[t]);
        }
        if (COHERENT && len <= kSplit) {
            // The row's only split: merge_wave's arithmetic on one partial
            // (M and l pass through unchanged, the factor f32(exp(m - lse)),
            // one FMA from zero), stored as the output with no exchange.
            const double lse = (double)M + log(l);
            const float cf1 = (float)exp((double)M - lse);
            float *out = A.out + (int64_t)row * A.heads * HD + (int64_t)(kh * G + h) * HD + DPL * lane;
#pragma unroll
            for (int t = 0; t < DPL; ++t) out[t] = __builtin_fmaf(cf1, o[t], 0.0f);
            continue;
        }
        float *p = partial(part, row, kh * G + h, sp, A.heads, nsplit, HD);
        if constexpr (COHERENT) {
            if (lane == 0) {
                publish(p, M);
                publish((double *)(p + 2), l);
            }
            if constexpr (DPL == 2)
                publish((uint64_t *)(p + 4) + lane,
                        (uint64_t)__float_as_uint(o[0]) | ((uint64_t)__float_as_uint(o[1]) << 32));
            else
                publish(p + 4 + lane, o[0]);
        } else {
            if (lane == 0) {
                p[0] = M;
                *(double *)(p + 2) = l;
            }
#pragma unroll
            for (int t = 0; t < DPL; ++t) p[4 + DPL * lane + t] = o[t];
        }
    }
    return true;
}

// Split kernel for head_dim 64 / 128 (split_partial); the combine kernel
// merges.  Splits past a row's positions write the empty partial.
template <int HD>
__global__ __launch_bounds__(kSplitThreads) void attn_split_fast_kernel(const AttnArgs A, float *__restrict__ part,
                                                                        int nsplit) {
    __shared__ SplitStage<HD> S;
    const int row = blockIdx.x, kh = blockIdx.y, sp = blockIdx.z;
    if (split_partial<HD, false>(A, part, nsplit, row, kh, sp, S)) return;
    const int G = A.heads / A.kv_heads;
    for (int i = threadIdx.x; i < G * (HD + 4); i += kSplitThreads) {
        const int g = i / (HD + 4), k = i - g * (HD + 4);
        float *p = partial(part, row, kh * G + g, sp, A.heads, nsplit, HD);
        p[k] = k == 0 ? -FLT_MAX : 0.0f;
    }
}

constexpr int kMergeChunk = 256;  // splits per pass of the weight table
constexpr int kChainSplits = 16;  // merge_splits: one FMA chain up to this many splits
constexpr int kMergePairs = kMaxGroup * kMaxHd / 256;
constexpr int kMergeBatch = 16;   // partial loads in flight per (head, dim) pair

// Merge of the split partials for head h of a row by one wave, with no
// barrier.  M, l, the factors and the order of the sums are merge_splits'
// below, so the fused kernel and the split + combine kernels give the same
// bits: past 64 splits each lane first folds its splits lane, lane+64, ...
// in order; each dim accumulates the splits by FMA in split order (lane i
// holds split i's factor), in the groups merge_splits uses past
// kChainSplits.  The partials are read with agent-scope loads (publish / fetch);
// lane holds dims HD/64 * lane + ....
template <int HD>
__device__ __forceinline__ void merge_wave(const AttnArgs &A, const float *part, int nsplit, int row, int h,
                                           int used) {
    // One round of loads, none of them under a lane condition (that would
    // make the compiler wait for it before issuing the rest): split
    // min(lane, used-1)'s {m, l} and, for used <= kMergeBatch, this lane's
    // dims of every split.
    constexpr int DL = HD / 64;  // dims per lane
    typedef typename std::conditional<DL == 2, uint64_t, float>::type Dims;
    const int lane = threadIdx.x & 63;
    const float *pb = partial((float *)part, row, h, 0, A.heads, nsplit, HD) + 4 + DL * lane;
    const float *pl = partial((float *)part, row, h, min(lane, used - 1), A.heads, nsplit, HD);
    const float mraw = fetch(pl);
    const double lraw = fetch((const double *)(pl + 2));
    // The first kPre splits' dims load with {m, l}; up to kMergeBatch
    // splits, the rest load after the factors (a second round, only past
    // kPre splits), so that the fused kernel keeps to 128 registers.
    constexpr int kPre = kMergeBatch / 2;
    Dims v[kPre];
    const bool pre = used <= kMergeBatch;
    if (pre) {
#pragma unroll
        for (int b = 0; b < kPre; ++b)
            if (b < used) v[b] = fetch((const Dims *)(pb + (int64_t)b * (HD + 4)));
    }
    float M = lane < used ? mraw : -FLT_MAX;
    for (int i = lane + 64; i < used; i += 64)
        M = fmaxf(M, fetch(partial((float *)part, row, h, i, A.heads, nsplit, HD)));
    M = wave_max(M);
    double l = lane < used ? lraw * exp((double)mraw - (double)M) : 0.0;
    for (int i = lane + 64; i < used; i += 64) {
        const float *p = partial((float *)part, row, h, i, A.heads, nsplit, HD);
        l += fetch((const double *)(p + 2)) * exp((double)fetch(p) - (double)M);
    }
    l = wave_sum(l);
    const double lse = (double)M + log(l);
    float o[DL];
#pragma unroll
    for (int d = 0; d < DL; ++d) o[d] = 0.0f;
    auto acc = [&](float c, Dims w) {
        if constexpr (DL == 2) {
            o[0] = __builtin_fmaf(c, __uint_as_float((uint32_t)w), o[0]);
            o[1] = __builtin_fmaf(c, __uint_as_float((uint32_t)(w >> 32)), o[1]);
        } else {
            o[0] = __builtin_fmaf(c, w, o[0]);
        }
    };
    if (pre) {
        const float cf = lane < used ? (float)exp((double)mraw - lse) : 0.0f;
#pragma unroll
        for (int b = 0; b < kPre; ++b)
            if (b < used) acc(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(cf), b)), v[b]);
        if (used > kPre) {
#pragma unroll
            for (int b = 0; b < kPre; ++b)
                if (kPre + b < used) v[b] = fetch((const Dims *)(pb + (int64_t)(kPre + b) * (HD + 4)));
#pragma unroll
            for (int b = 0; b < kPre; ++b)
                if (kPre + b < used)
                    acc(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(cf), kPre + b)), v[b]);
        }
    } else {
        // merge_splits' order: past kChainSplits (up to kMergeChunk) splits
        // the dims sum ng groups of `per` consecutive splits, each from
        // zero, then add the group sums in group order; past kMergeChunk one
        // chain.  `tot` holds the groups before the current one.
        static_assert(kMergeBatch == kChainSplits && 256 % HD == 0, "merge_splits' grouping");
        const int ng = used <= kMergeChunk ? 256 / HD : 1;
        const int per = (used + ng - 1) / ng;
        float tot[DL];
        int next = per, q = 0;
        for (int c0 = 0; c0 < used; c0 += 64) {
            // lane i holds the factor of split c0 + i
            const int ci = min(c0 + lane, used - 1);
            const float mi = c0 == 0 ? mraw : fetch(partial((float *)part, row, h, ci, A.heads, nsplit, HD));
            const float cf = c0 + lane < used ? (float)exp((double)mi - lse) : 0.0f;
            const int cnt = min(64, used - c0);
            for (int i0 = 0; i0 < cnt; i0 += kMergeBatch) {
                Dims w[kMergeBatch];
#pragma unroll
                for (int b = 0; b < kMergeBatch; ++b)
                    if (i0 + b < cnt) w[b] = fetch((const Dims *)(pb + (int64_t)(c0 + i0 + b) * (HD + 4)));
#pragma unroll
                for (int b = 0; b < kMergeBatch; ++b) {
                    if (i0 + b >= cnt) continue;
                    if (c0 + i0 + b == next) {  // a group ends (wave-uniform)
#pragma unroll
                        for (int d = 0; d < DL; ++d) {
                            tot[d] = q == 0 ? o[d] : tot[d] + o[d];
                            o[d] = 0.0f;
                        }
                        ++q;
                        next += per;
                    }
                    acc(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(cf), i0 + b)), w[b]);
                }
            }
        }
        if (q > 0)
#pragma unroll
            for (int d = 0; d < DL; ++d) o[d] = tot[d] + o[d];
    }
    float *out = A.out + (int64_t)row * A.heads * HD + (int64_t)h * HD + DL * lane;
#pragma unroll
    for (int d = 0; d < DL; ++d) out[d] = o[d];
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
        // each batch's factors into registers before its FMAs (an LDS read
        // inside the chain would cost every FMA an LDS latency)
        float ca[kMergeBatch], cb[kMergeBatch];
#pragma unroll
        for (int b = 0; b < kMergeBatch; ++b) ca[b] = cf[min(i0 + b, last)];
#pragma unroll
        for (int b = 0; b < kMergeBatch; ++b)
            if (i0 + b < b1) o = __builtin_fmaf(ca[b], va[b], o);
        if (i1 >= b1) break;
        if (i1 + kMergeBatch < b1) {
#pragma unroll
            for (int b = 0; b < kMergeBatch; ++b) va[b] = pb[(int64_t)min(i1 + kMergeBatch + b, last) * st];
        }
#pragma unroll
        for (int b = 0; b < kMergeBatch; ++b) cb[b] = cf[min(i1 + b, last)];
#pragma unroll
        for (int b = 0; b < kMergeBatch; ++b)
            if (i1 + b < b1) o = __builtin_fmaf(cb[b], vb[b], o);
    }
    return o;
}

// merge_splits for one head of a decode-sized step past kChainSplits splits
// (at most kMergeChunk; head_dim a multiple of kMergeSlices dividing 256), on
// a slice of the head's dims: workgroup z of kMergeSlices takes dims
// [z*hd/kMergeSlices, +hd/kMergeSlices), so a head's partial loads spread over
// that many CUs.  Each workgroup forms M, l, lse and the factors itself, one
// split's exps per thread; wave 0 folds l as merge_splits' lanes do (lane i:
// splits i, i+64, ... in order, then the butterfly).  Each chain thread
// (dim, group) preloads its group's first 4*kMergeBatch partials and the next
// kMergeBatch, and reads its factors into registers ahead of the FMA chain.
// The same values in the same order as merge_splits, so the same bits.
constexpr int kMergeSlices = 8;
__device__ __forceinline__ void merge_one_head_slice(const AttnArgs &A, const float *part, int nsplit, int row, int h,
                                                     int hd, int used, float *cf) {
    __shared__ double terms[kMergeChunk];
    __shared__ float wmax[4];
    __shared__ double s_lse;
    __shared__ float gs[256];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int ng = 256 / hd, per = (used + ng - 1) / ng;
    const int dn = hd / kMergeSlices, d0 = (int)blockIdx.z * dn;
    // chain threads: (dim d0 + tid % dn, group tid / dn), tid < dn * ng
    const bool chain = tid < dn * ng;
    const int j = d0 + tid % dn, q = tid / dn;
    const int b0 = q * per, b1 = min(used, b0 + per), last = max(b1 - 1, 0);
    const int64_t st = hd + 4;
    const float *pb = partial((float *)part, row, h, 0, A.heads, nsplit, hd) + 4 + j;
    constexpr int PRE = 4 * kMergeBatch;  // partials preloaded per chain thread
    float vp[PRE], vq[kMergeBatch];         // the group's first PRE splits, then the next batch
    if (chain) {
#pragma unroll
        for (int b = 0; b < PRE; ++b) vp[b] = pb[(int64_t)min(b0 + b, last) * st];
#pragma unroll
        for (int b = 0; b < kMergeBatch; ++b) vq[b] = pb[(int64_t)min(b0 + PRE + b, last) * st];
    }
    // split tid's {m, l}
    float mt = -FLT_MAX;
    double lt = 0.0;
    if (tid < used) {
        const float *p = partial((float *)part, row, h, tid, A.heads, nsplit, hd);
        mt = p[0];
        lt = *(const double *)(p + 2);
    }
    // butterflies by DPP / permlane (wave_max, wave_sum: a __shfl_xor
    // butterfly's bits)
    float M = wave_max(mt);
    if (lane == 0) wmax[wave] = M;
    __syncthreads();
    M = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    if (tid < used) terms[tid] = lt * exp((double)mt - (double)M);
    __syncthreads();
    if (wave == 0) {
        double l = 0.0;
#pragma unroll
        for (int b = 0; b < 4; ++b)
            if (lane + 64 * b < used) l += terms[lane + 64 * b];
        l = wave_sum(l);
        if (lane == 0) s_lse = (double)M + log(l);
    }
    __syncthreads();
    if (tid < used) cf[tid] = (float)exp((double)mt - s_lse);
    __syncthreads();
    if (chain) {
        // One FMA chain over [b0, b1) in split order (merge_range's).  The
        // factors are read into registers ahead of the chain: read from LDS
        // inside it, each FMA waited a full LDS latency (3 us for 64).
        float c[PRE];
#pragma unroll
        for (int b = 0; b < PRE; ++b) c[b] = cf[min(b0 + b, used - 1)];
        float o = 0.0f;
#pragma unroll
        for (int b = 0; b < PRE; ++b)
            if (b0 + b < b1) o = __builtin_fmaf(c[b], vp[b], o);
        for (int i0 = b0 + PRE; i0 < b1; i0 += kMergeBatch) {
            float cc[kMergeBatch];
#pragma unroll
            for (int b = 0; b < kMergeBatch; ++b) cc[b] = cf[min(i0 + b, used - 1)];
            if (i0 > b0 + PRE) {
#pragma unroll
                for (int b = 0; b < kMergeBatch; ++b) vq[b] = pb[(int64_t)min(i0 + b, last) * st];
            }
#pragma unroll
            for (int b = 0; b < kMergeBatch; ++b)
                if (i0 + b < b1) o = __builtin_fmaf(cc[b], vq[b], o);
        }
        gs[tid] = o;
    }
    __syncthreads();
    if (tid < dn) {
        float v = gs[tid];
        for (int r = 1; r < ng; ++r) v += gs[r * dn + tid];
        A.out[(int64_t)row * A.heads * hd + (int64_t)h * hd + d0 + tid] = v;
    }
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
    if constexpr (GROUPS) {
        // Launched with kMergeSlices workgroups per head (gridDim.z): the
        // sliced merge where it applies, else workgroup 0 merges alone.
        if (nh == 1 && used > kChainSplits && used <= kMergeChunk && hd <= 128 && 256 % hd == 0 &&
            hd % kMergeSlices == 0 && gridDim.z == kMergeSlices) {
            merge_one_head_slice(A, part, nsplit, row, h0, hd, used, cf[0]);
            return;
        }
        if (blockIdx.z != 0) return;
    }
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
    // other rows of its step: up to kChainSplits splits (and past
    // kMergeChunk) one FMA chain over the splits in order; in between, ng
    // groups of consecutive splits, each summed from zero, then the group
    // sums added in group order.
    // GROUPS (the one-head combine of decode-sized batches): the groups run
    // on separate threads, so none idles; otherwise one thread sums its
    // pair's groups one after another, in the same order.
    __shared__ float gs[GROUPS ? 256 : 1];
    const int ng = hd <= 128 && 256 % hd == 0 && used > kChainSplits && used <= kMergeChunk ? 256 / hd : 1;
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

// Fused split + combine for decode steps, head_dim 64 / 128: 1-D
// grid, workgroup (row, kv head, split) with row fastest, then kv head.
// Each writes its split_partial, and the last split of a (row, kv head) to
// finish merges all partials of the group with the combine rule (counter
// per (row, kv head), reset by the merging workgroup, so the kernel replays
// without clearing).
template <int HD>
__global__ __launch_bounds__(kSplitThreads, 4) void attn_fused_kernel(const AttnArgs A, float *__restrict__ part,
                                                                   int nsplit, int32_t *__restrict__ counters) {
    __shared__ SplitStage<HD> S;
    __shared__ int last;
    const int bid = blockIdx.x, row = bid % A.n, kh = (bid / A.n) % A.kv_heads, sp = bid / (A.n * A.kv_heads);
    const int tid = threadIdx.x, wave = tid >> 6;
    if (!split_partial<HD, true>(A, part, nsplit, row, kh, sp, S)) return;  // no partial, no count
    const int G = A.heads / A.kv_heads, used = (A.meta.pos[row] + kSplit) / kSplit;
    if (used == 1) return;  // a row's only split wrote its output
    // Each wave's partial stores complete before the barrier, so the split
    // is counted only once all of them are visible device-wide.
    //
    // Ordering of the exchange.  Every value that crosses workgroups is an
    // agent-scope atomic access: the partials are written with sc1 stores
    // (written through L2 to the device's coherence point) and read with sc1
    // loads (served from it), and the count is an agent-scope atomic.  The
    // writer waits for its stores' completion (s_waitcnt 0) before the
    // barrier that precedes its count, and the merger issues its loads only
    // after the barrier that follows the count's result; both barriers are
    // compiler barriers for memory operations.  An acq_rel count would add a
    // whole-L2 write-back before it and an L2 invalidation after it, which
    // only non-atomic data needs; measured, it cost 0.3% of 7B decode at 150
    // positions and 1.8% at 2k.
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    int32_t *cnt = counters + (int64_t)row * A.kv_heads + kh;
    if (tid == 0) last = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == used - 1;
    __syncthreads();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);  // no load of the merge moves above the count
    if (!last) return;
    if (tid == 0) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // one wave per head merges on its own
    for (int g = wave; g < G; g += kSplitWaves) merge_wave<HD>(A, part, nsplit, row, kh * G + g, used);
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
        // Decode steps: one launch, the last split of each (row, kv head)
        // merges.
        const dim3 g1((unsigned)((int64_t)a.n * a.kv_heads * nsplit));
        if (a.head_dim == 128)
            attn_fused_kernel<128><<<g1, kSplitThreads, 0, s>>>(a, scratch, nsplit, counters);
        else
            attn_fused_kernel<64><<<g1, kSplitThreads, 0, s>>>(a, scratch, nsplit, counters);
        SRQ_HIP(hipGetLastError());
        return SRQ_OK;
    }
    if (a.head_dim == 128)
        attn_split_fast_kernel<128><<<grid, kSplitThreads, 0, s>>>(a, scratch, nsplit);
    else if (a.head_dim == 64)
        attn_split_fast_kernel<64><<<grid, kSplitThreads, 0, s>>>(a, scratch, nsplit);
    else
        attn_split_kernel<<<grid, 256, 0, s>>>(a, scratch, nsplit);
    SRQ_HIP(hipGetLastError());
    if (a.n <= kGroupRows)
        attn_combine_kernel<true><<<dim3(a.n, a.heads, kMergeSlices), 256, 0, s>>>(a, scratch, nsplit, kSplit);
    else
        attn_combine_kernel<false><<<dim3(a.n, a.heads), 256, 0, s>>>(a, scratch, nsplit, kSplit);
    SRQ_HIP(hipGetLastError());
    return SRQ_OK;
}

int attention_prepare() { return SRQ_OK; }

}  // namespace srq
