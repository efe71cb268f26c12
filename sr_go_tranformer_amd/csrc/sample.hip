// Token sampling on the device: sampleWithBlocked
// (cmd/monolith/monolith.go M:7320-7426) for rows of logits.
//
// Per row (one 1024-thread workgroup):
//  - value v_i = f64(logit_i), divided (v > 0) or multiplied (v <= 0) by the
//    repeat penalty when id i occurs in the row's history; the blocked id is
//    no candidate; any non-finite logit is an error (M:7331-7358).
//  - temperature 0: the first maximum (lowest id on ties), no draw.
//  - otherwise candidates are ordered by value descending, then id
//    ascending (candidateBefore, M:7284-7289); top_k keeps the first k;
//    p_i = exp((v_i - v_max) / T); top_p keeps the shortest prefix whose
//    mass reaches top_p * total; one SplitMix64 Float64 draw u picks the
//    first candidate whose running mass exceeds u * total.
//
// No sort of the whole row: each of the three cuts (k-th candidate, nucleus
// end, drawn candidate) is located by histogramming the candidates over
// 2048 value buckets (bucket index is monotone in the value), narrowing to
// the bucket holding the cut, and sorting only that bucket's candidates in
// LDS.  Masses are integers (p * 2^44, rounded), so every sum is exact and
// independent of the order threads add in: results are deterministic.  The
// reference sums f64 probabilities in sorted order; the two agree except
// when a cut falls within ~1e-12 of a candidate boundary.
//
// Passes over the row: one for the range and the first maximum, one for the
// masses and the first-level histogram of every candidate, then one per cut
// that gathers its bucket (more only when a bucket holds over 2048
// candidates).  The first-level histogram serves all three cuts: every cut
// is a prefix of the candidate order whose target lies within the prefix
// kept so far, so the buckets before the one holding it are kept whole and
// the unfiltered histogram finds the same bucket.  A candidate's mass is
// recomputed where it is needed (it is a pure function of its value).
#include <cfloat>
#include <climits>

#include "srq_internal.h"

namespace srq {
namespace {

constexpr int kST = 1024;      // threads per row
constexpr int kBuckets = 2048;
constexpr int kList = 2048;    // candidates of one bucket sorted in LDS
constexpr int kLevels = 4;     // bucket refinements before giving up
constexpr double kFix = 17592186044416.0;  // 2^44: mass of probability 1
// The scans give each thread two buckets / two sorted candidates.
static_assert(kBuckets == 2 * kST && kList == 2 * kST, "two entries per thread");

struct Cand {  // a position in candidate order; id INT_MAX = past every candidate
    double v;
    int id;
};

__device__ __forceinline__ bool before(double va, int ia, double vb, int ib) {
    return va > vb || (va == vb && ia < ib);
}

struct SampleLds {
    uint32_t hcount[kBuckets];
    unsigned long long hmass[kBuckets];
    uint32_t h0count[kBuckets];           // first-level histogram over [vmin, vmax]
    unsigned long long h0mass[kBuckets];
    double lv[kList];
    int li[kList];
    unsigned long long lp[kList];
    unsigned long long scan[kST];
    double red_d[kST / 64];
    int red_i[kST / 64];
    unsigned long long red_u[kST / 64];
    int list_n;
    int bucket;            // chosen bucket
    unsigned long long above;
    Cand cut;
    unsigned long long cum;  // running count/mass through the cut
    int found;
};

__device__ __forceinline__ double block_max(double v, SampleLds &s) {
    for (int o = 32; o > 0; o >>= 1) v = fmax(v, __shfl_xor(v, o, 64));
    if ((threadIdx.x & 63) == 0) s.red_d[threadIdx.x >> 6] = v;
    __syncthreads();
    double r = s.red_d[0];
    for (int w = 1; w < kST / 64; ++w) r = fmax(r, s.red_d[w]);
    __syncthreads();
    return r;
}
__device__ __forceinline__ double block_min(double v, SampleLds &s) {
    for (int o = 32; o > 0; o >>= 1) v = fmin(v, __shfl_xor(v, o, 64));
    if ((threadIdx.x & 63) == 0) s.red_d[threadIdx.x >> 6] = v;
    __syncthreads();
    double r = s.red_d[0];
    for (int w = 1; w < kST / 64; ++w) r = fmin(r, s.red_d[w]);
    __syncthreads();
    return r;
}
__device__ __forceinline__ unsigned long long block_sum(unsigned long long v, SampleLds &s) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    if ((threadIdx.x & 63) == 0) s.red_u[threadIdx.x >> 6] = v;
    __syncthreads();
    unsigned long long r = 0;
    for (int w = 0; w < kST / 64; ++w) r += s.red_u[w];
    __syncthreads();
    return r;
}
// First candidate in order among (v, id) pairs: the largest v, lowest id.
__device__ __forceinline__ Cand block_first(Cand c, SampleLds &s) {
    for (int o = 32; o > 0; o >>= 1) {
        const double ov = __shfl_xor(c.v, o, 64);
        const int oi = __shfl_xor(c.id, o, 64);
        if (before(ov, oi, c.v, c.id)) c.v = ov, c.id = oi;
    }
    if ((threadIdx.x & 63) == 0) s.red_d[threadIdx.x >> 6] = c.v, s.red_i[threadIdx.x >> 6] = c.id;
    __syncthreads();
    Cand r{s.red_d[0], s.red_i[0]};
    for (int w = 1; w < kST / 64; ++w)
        if (before(s.red_d[w], s.red_i[w], r.v, r.id)) r.v = s.red_d[w], r.id = s.red_i[w];
    __syncthreads();
    return r;
}
// Last candidate in order: the smallest v, highest id.
__device__ __forceinline__ Cand block_last(Cand c, SampleLds &s) {
    for (int o = 32; o > 0; o >>= 1) {
        const double ov = __shfl_xor(c.v, o, 64);
        const int oi = __shfl_xor(c.id, o, 64);
        if (before(c.v, c.id, ov, oi)) c.v = ov, c.id = oi;
    }
    if ((threadIdx.x & 63) == 0) s.red_d[threadIdx.x >> 6] = c.v, s.red_i[threadIdx.x >> 6] = c.id;
    __syncthreads();
    Cand r{s.red_d[0], s.red_i[0]};
    for (int w = 1; w < kST / 64; ++w)
        if (before(r.v, r.id, s.red_d[w], s.red_i[w])) r.v = s.red_d[w], r.id = s.red_i[w];
    __syncthreads();
    return r;
}

__device__ __forceinline__ int bucket_of(double v, double lo, double scale) {
    int b = (int)((v - lo) * scale);
    return b < 0 ? 0 : b > kBuckets - 1 ? kBuckets - 1 : b;
}

enum { CUT_COUNT = 0, CUT_MASS_GE = 1, CUT_MASS_GT = 2 };

// Smallest v over the workgroup (wave butterfly, then the waves' minima).
__device__ __forceinline__ int block_min_int(int v, SampleLds &s) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o, 64));
    if ((tid & 63) == 0) s.red_i[tid >> 6] = v;
    __syncthreads();
    int r = s.red_i[0];
    for (int w = 1; w < kST / 64; ++w) r = min(r, s.red_i[w]);
    __syncthreads();
    return r;
}

__global__ __launch_bounds__(kST) void sample_kernel(const SampleArgs A) {
    extern __shared__ uint32_t seen[];  // history bitmap, (vocab + 31) / 32 words
    __shared__ SampleLds s;
    const int row = blockIdx.x, tid = threadIdx.x;
    const int vocab = A.vocab;
    const float *lg = A.logits + (int64_t)(A.row_ids ? A.row_ids[row] : row) * vocab;
    const int blocked = A.blocked ? A.blocked[row] : -1;
    const double T = A.temperature, rp = A.repeat_penalty;
    const bool use_seen = T != 0.0 || rp != 1.0;
    const int words = (vocab + 31) / 32;
    if (use_seen) {
        for (int i = tid; i < words; i += kST) seen[i] = 0;
        __syncthreads();
        const int hn = A.history_len ? A.history_len[row] : 0;
        const int32_t *h = A.history + (int64_t)row * A.history_stride;
        for (int i = tid; i < hn; i += kST) {
            const int t = h[i];
            if (t >= 0 && t < vocab) atomicOr(&seen[t >> 5], 1u << (t & 31));
        }
        __syncthreads();
    }
    auto value = [&](int i, float x) {
        double v = x;
        if (use_seen && ((seen[i >> 5] >> (i & 31)) & 1u)) v = v > 0 ? v / rp : v * rp;
        return v;
    };

    // ---- pass A: finiteness, range, first maximum --------------------------
    constexpr int U = 8;
    int bad = 0, cnt = 0;
    double vmax = -DBL_MAX, vmin = DBL_MAX;
    Cand best{-DBL_MAX, INT_MAX};
    for (int base = 0; base < vocab; base += kST * U) {
        float x[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = base + u * kST + tid;
            x[u] = i < vocab ? lg[i] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = base + u * kST + tid;
            if (i >= vocab) continue;
            bad |= !isfinite(x[u]);
            if (i == blocked) continue;
            const double v = value(i, x[u]);
            vmax = fmax(vmax, v);
            vmin = fmin(vmin, v);
            ++cnt;
            if (before(v, i, best.v, best.id)) best.v = v, best.id = i;
        }
    }
    bad = (int)block_sum((unsigned long long)bad, s);
    cnt = (int)block_sum((unsigned long long)cnt, s);
    vmax = block_max(vmax, s);
    vmin = block_min(vmin, s);
    best = block_first(best, s);
    if (bad || cnt == 0) {
        if (tid == 0) {
            A.ids[row] = -1;
            atomicOr(A.err, bad ? 1 : 2);
        }
        return;
    }
    if (T == 0.0) {
        if (tid == 0) A.ids[row] = best.id;
        return;
    }

    // Integer mass of a candidate of value v: p = exp((v - vmax) / T) scaled
    // by 2^44 and rounded.
    auto mass_of = [&](double v) { return (unsigned long long)(exp((v - vmax) / T) * kFix + 0.5); };

    // Candidates precede the bounds kcut (top_k) and pcut (top_p) in order.
    Cand kcut{-DBL_MAX, INT_MAX}, pcut{-DBL_MAX, INT_MAX};
    auto member = [&](int i, double v) {
        return i != blocked && !before(kcut.v, kcut.id, v, i) && !before(pcut.v, pcut.id, v, i);
    };

    // Locate the first candidate (in order) at which the running count or
    // mass satisfies the cut; s.cut / s.cum / s.found hold the result.
    auto locate = [&](int mode, unsigned long long target) {
        double lo = vmin, hi = vmax;
        double los[kLevels], scales[kLevels];
        int chosen[kLevels];
        unsigned long long above = 0;
        if (tid == 0) s.found = 0;
        for (int level = 0; level < kLevels; ++level) {
            const double scale = hi > lo ? (double)kBuckets / (hi - lo) : 0.0;
            los[level] = lo;
            scales[level] = scale;
            auto inside = [&](double v) {  // in the chosen bucket of every earlier level
                for (int l = 0; l < level; ++l)
                    if (bucket_of(v, los[l], scales[l]) != chosen[l]) return false;
                return true;
            };
            if (level == 0) {
                // the first-level histogram of every candidate (pass B)
                for (int b = tid; b < kBuckets; b += kST) s.hcount[b] = s.h0count[b], s.hmass[b] = s.h0mass[b];
                __syncthreads();
            } else {
                for (int b = tid; b < kBuckets; b += kST) s.hcount[b] = 0, s.hmass[b] = 0;
                __syncthreads();
                for (int base = 0; base < vocab; base += kST * U) {
                    float x[U];
#pragma unroll
                    for (int u = 0; u < U; ++u) {
                        const int i = base + u * kST + tid;
                        x[u] = i < vocab ? lg[i] : 0.0f;
                    }
#pragma unroll
                    for (int u = 0; u < U; ++u) {
                        const int i = base + u * kST + tid;
                        if (i >= vocab) continue;
                        const double v = value(i, x[u]);
                        if (!member(i, v) || !inside(v)) continue;
                        const int b = bucket_of(v, lo, scale);
                        atomicAdd(&s.hcount[b], 1u);
                        atomicAdd(&s.hmass[b], mass_of(v));
                    }
                }
                __syncthreads();
            }
            // Running totals over buckets in descending order (bucket 2047
            // first): thread t owns buckets 2047-2t and 2046-2t.
            {
                const int b0 = kBuckets - 1 - 2 * tid, b1 = b0 - 1;
                const unsigned long long w0 = mode == CUT_COUNT ? s.hcount[b0] : s.hmass[b0];
                const unsigned long long w1 = mode == CUT_COUNT ? s.hcount[b1] : s.hmass[b1];
                s.scan[tid] = w0 + w1;
                __syncthreads();
                for (int o = 1; o < kST; o <<= 1) {  // inclusive scan
                    const unsigned long long add = tid >= o ? s.scan[tid - o] : 0ull;
                    __syncthreads();
                    s.scan[tid] += add;
                    __syncthreads();
                }
                const unsigned long long before_t = above + (tid ? s.scan[tid - 1] : 0ull);
                auto hit = [&](unsigned long long c) {
                    return mode == CUT_MASS_GT ? c > target : c >= target;
                };
                // the first bucket (in order) whose inclusive total hits
                int mine = INT_MAX;
                if (hit(before_t + w0) && (w0 > 0 || mode == CUT_COUNT)) mine = 2 * tid;
                else if (hit(before_t + w0 + w1)) mine = 2 * tid + 1;
                if (mine != INT_MAX && s.hcount[kBuckets - 1 - mine] == 0) mine = INT_MAX;
                const int first = block_min_int(mine, s);
                if (tid == 0) {
                    s.bucket = first;
                    if (first != INT_MAX) {
                        const int owner = first / 2;
                        unsigned long long a = above + (owner ? s.scan[owner - 1] : 0ull);
                        if (first & 1)
                            a += mode == CUT_COUNT ? s.hcount[kBuckets - 1 - 2 * owner]
                                                   : s.hmass[kBuckets - 1 - 2 * owner];
                        s.above = a;
                    }
                }
                __syncthreads();
            }
            if (s.bucket == INT_MAX) return;  // never reached: s.found stays 0
            const int b = kBuckets - 1 - s.bucket;
            above = s.above;
            chosen[level] = b;
            const uint32_t n = s.hcount[b];
            if (n > (uint32_t)kList && level + 1 < kLevels && hi > lo) {
                lo = lo + (double)b / scale;  // narrow to the bucket's value range
                hi = lo + 1.0 / scale;
                __syncthreads();
                continue;
            }
            if (n > (uint32_t)kList) {
                // More candidates than one sort holds.  If they all hold one
                // value their order is by id alone: take the m-th smallest id.
                double bmn = DBL_MAX, bmx = -DBL_MAX;
                unsigned long long pe = 0;
                for (int i = tid; i < vocab; i += kST) {
                    const double v = value(i, lg[i]);
                    if (!member(i, v) || !inside(v) || bucket_of(v, lo, scale) != b) continue;
                    bmn = fmin(bmn, v), bmx = fmax(bmx, v), pe = mass_of(v);
                }
                bmn = block_min(bmn, s);
                bmx = block_max(bmx, s);
                for (int o = 32; o > 0; o >>= 1) pe = max(pe, (unsigned long long)__shfl_xor(pe, o, 64));
                if ((tid & 63) == 0) s.red_u[tid >> 6] = pe;
                __syncthreads();
                pe = 0;
                for (int w = 0; w < kST / 64; ++w) pe = max(pe, s.red_u[w]);
                __syncthreads();
                const unsigned long long need = target - above;  // > 0: the cut lies in this bucket
                if (bmn != bmx || (mode != CUT_COUNT && pe == 0)) {
                    if (tid == 0) atomicOr(A.err, 4);
                    return;
                }
                const unsigned long long m = mode == CUT_COUNT    ? need
                                             : mode == CUT_MASS_GE ? (need + pe - 1) / pe
                                                                   : need / pe + 1;
                const int width = (vocab + kBuckets - 1) / kBuckets;  // ids per id bucket
                for (int k = tid; k < kBuckets; k += kST) s.hcount[k] = 0;
                __syncthreads();
                for (int i = tid; i < vocab; i += kST) {
                    const double v = value(i, lg[i]);
                    if (member(i, v) && inside(v) && bucket_of(v, lo, scale) == b) atomicAdd(&s.hcount[i / width], 1u);
                }
                __syncthreads();
                {
                    // first id bucket whose running count reaches m: thread t
                    // owns id buckets 2t and 2t+1 (ascending ids)
                    const unsigned long long w0 = s.hcount[2 * tid], w1 = s.hcount[2 * tid + 1];
                    s.scan[tid] = w0 + w1;
                    __syncthreads();
                    for (int o = 1; o < kST; o <<= 1) {  // inclusive scan
                        const unsigned long long add = tid >= o ? s.scan[tid - o] : 0ull;
                        __syncthreads();
                        s.scan[tid] += add;
                        __syncthreads();
                    }
                    const unsigned long long b0 = tid ? s.scan[tid - 1] : 0ull;
                    const int mine = b0 + w0 >= m ? 2 * tid : b0 + w0 + w1 >= m ? 2 * tid + 1 : INT_MAX;
                    const int first = block_min_int(mine, s);
                    if (first != INT_MAX && mine == first) {
                        s.bucket = first;
                        s.above = (first & 1) ? b0 + w0 : b0;  // candidates of lower ids
                    }
                    if (tid == 0) s.list_n = 0;
                    __syncthreads();
                }
                const int ib = s.bucket;
                for (int i = ib * width + tid; i < min(vocab, (ib + 1) * width); i += kST) {
                    const double v = value(i, lg[i]);
                    if (member(i, v) && inside(v) && bucket_of(v, lo, scale) == b) s.li[atomicAdd(&s.list_n, 1)] = i;
                }
                __syncthreads();
                {
                    // the (m - above)-th smallest gathered id (ids are distinct,
                    // at most `width` of them): the one with that many below it
                    const int want = (int)(m - s.above) - 1, ln = s.list_n;
                    for (int t = tid; t < ln; t += kST) {
                        const int id = s.li[t];
                        int rank = 0;
                        for (int c2 = 0; c2 < ln; ++c2) rank += s.li[c2] < id;
                        if (rank == want) {
                            s.cut = Cand{bmn, id};
                            s.cum = above + (mode == CUT_COUNT ? m : m * pe);
                            s.found = 1;
                        }
                    }
                }
                __syncthreads();
                return;
            }
            // Gather the bucket's candidates, sort them in order, scan.
            if (tid == 0) s.list_n = 0;
            __syncthreads();
            for (int base = 0; base < vocab; base += kST * U) {
                float x[U];
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int i = base + u * kST + tid;
                    x[u] = i < vocab ? lg[i] : 0.0f;
                }
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int i = base + u * kST + tid;
                    if (i >= vocab) continue;
                    const double v = value(i, x[u]);
                    if (!member(i, v) || !inside(v) || bucket_of(v, lo, scale) != b) continue;
                    const int k = atomicAdd(&s.list_n, 1);
                    s.lv[k] = v, s.li[k] = i, s.lp[k] = mass_of(v);
                }
            }
            __syncthreads();
            const int ln = s.list_n;
            int pw = 1;
            while (pw < ln) pw <<= 1;
            for (int k = ln + tid; k < pw; k += kST) s.lv[k] = -DBL_MAX, s.li[k] = INT_MAX, s.lp[k] = 0;
            __syncthreads();
            for (int size = 2; size <= pw; size <<= 1) {  // bitonic sort into candidate order
                for (int stride = size >> 1; stride > 0; stride >>= 1) {
                    for (int k = tid; k < pw; k += kST) {
                        const int j = k ^ stride;
                        if (j <= k) continue;
                        const bool up = (k & size) == 0;
                        const bool swap = up ? before(s.lv[j], s.li[j], s.lv[k], s.li[k])
                                             : before(s.lv[k], s.li[k], s.lv[j], s.li[j]);
                        if (swap) {
                            const double tv = s.lv[k];
                            const int ti = s.li[k];
                            const unsigned long long tp = s.lp[k];
                            s.lv[k] = s.lv[j], s.li[k] = s.li[j], s.lp[k] = s.lp[j];
                            s.lv[j] = tv, s.li[j] = ti, s.lp[j] = tp;
                        }
                    }
                    __syncthreads();
                }
            }
            // The first sorted candidate whose running total hits: thread t
            // owns entries 2t and 2t+1; an inclusive scan of the pairs gives
            // every running total at once.
            {
                const int k0 = 2 * tid, k1 = k0 + 1;
                const unsigned long long w0 = k0 < ln ? (mode == CUT_COUNT ? 1ull : s.lp[k0]) : 0ull;
                const unsigned long long w1 = k1 < ln ? (mode == CUT_COUNT ? 1ull : s.lp[k1]) : 0ull;
                s.scan[tid] = w0 + w1;
                __syncthreads();
                for (int o = 1; o < kST; o <<= 1) {  // inclusive scan
                    const unsigned long long add = tid >= o ? s.scan[tid - o] : 0ull;
                    __syncthreads();
                    s.scan[tid] += add;
                    __syncthreads();
                }
                const unsigned long long c0 = above + (tid ? s.scan[tid - 1] : 0ull) + w0, c1 = c0 + w1;
                auto hit = [&](unsigned long long c) { return mode == CUT_MASS_GT ? c > target : c >= target; };
                const int mine = k0 < ln && hit(c0) ? k0 : k1 < ln && hit(c1) ? k1 : INT_MAX;
                const int first = block_min_int(mine, s);
                if (first != INT_MAX && mine == first) {
                    s.cut = Cand{s.lv[first], s.li[first]};
                    s.cum = (first & 1) ? c1 : c0;
                    s.found = 1;
                }
            }
            __syncthreads();
            return;
        }
    };

    // ---- pass B: integer masses, the total and the first-level histogram -----
    // (buckets over [vmin, vmax], as locate's first level computes them)
    for (int b = tid; b < kBuckets; b += kST) s.h0count[b] = 0, s.h0mass[b] = 0;
    __syncthreads();
    const double scale0 = vmax > vmin ? (double)kBuckets / (vmax - vmin) : 0.0;
    unsigned long long total = 0;
    for (int base = 0; base < vocab; base += kST * U) {
        float x[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = base + u * kST + tid;
            x[u] = i < vocab ? lg[i] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = base + u * kST + tid;
            if (i >= vocab || i == blocked) continue;
            const double v = value(i, x[u]);
            const unsigned long long m = mass_of(v);
            total += m;
            const int b = bucket_of(v, vmin, scale0);
            atomicAdd(&s.h0count[b], 1u);
            atomicAdd(&s.h0mass[b], m);
        }
    }
    total = block_sum(total, s);

    // top_k: keep the first k candidates (M:7390-7395).
    if (A.top_k > 0 && A.top_k < cnt) {
        locate(CUT_COUNT, (unsigned long long)A.top_k);
        if (!s.found) {
            if (tid == 0) atomicOr(A.err, 8), A.ids[row] = -1;
            return;
        }
        kcut = s.cut;
        // mass of the kept candidates
        unsigned long long m = 0;
        for (int i = tid; i < vocab; i += kST) {
            const double v = value(i, lg[i]);
            if (member(i, v)) m += mass_of(v);
        }
        total = block_sum(m, s);
    }
    // top_p: the shortest prefix with mass >= top_p * total (M:7398-7409).
    if (A.top_p < 1.0) {
        const double want = A.top_p * (double)total;
        unsigned long long target = (unsigned long long)ceil(want);
        if (target < 1) target = 1;
        locate(CUT_MASS_GE, target);
        if (s.found) {
            pcut = s.cut;
            total = s.cum;
        }
    }
    // Draw: the first candidate whose running mass exceeds u * total.
    uint64_t st = A.rng[row] + 0x9e3779b97f4a7c15ULL;
    uint64_t z = st;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    z ^= z >> 31;
    const double u = (double)(z >> 11) * (1.0 / 9007199254740992.0);
    const unsigned long long draw = (unsigned long long)(u * (double)total);
    locate(CUT_MASS_GT, draw);
    int id;
    if (s.found) {
        id = s.cut.id;
    } else {  // rounding left the draw at the total: the last candidate
        Cand last{DBL_MAX, -1};
        for (int i = tid; i < vocab; i += kST) {
            const double v = value(i, lg[i]);
            if (member(i, v) && before(last.v, last.id, v, i)) last.v = v, last.id = i;
        }
        id = block_last(last, s).id;
    }
    if (tid == 0) {
        A.ids[row] = id;
        A.rng[row] = st;
    }
}

}  // namespace

int launch_sample(hipStream_t s, const SampleArgs &a) {
    if (a.rows <= 0) return SRQ_OK;
    const size_t lds = (size_t)((a.vocab + 31) / 32) * 4;
    if (lds > 48 * 1024) return fail(SRQ_EINVAL, "sample: vocabulary of %d ids exceeds the history bitmap", a.vocab);
    sample_kernel<<<a.rows, kST, lds, s>>>(a);
    SRQ_HIP(hipGetLastError());
    return SRQ_OK;
}

}  // namespace srq
