// Token sampling on the device: sampleWithBlocked
// (cmd/monolith/monolith.go M:7320-7426) for rows of logits.
//
// Per row:
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
// Three launches.  The first two split each row into chunks, one 256-thread
// workgroup per (chunk, row): sample_range_kernel finds a chunk's range,
// candidate count and first maximum; sample_mass_kernel combines the
// chunks' ranges and writes the chunk's total integer mass and its
// first-level histogram (2048 buckets over [vmin, vmax]).  sample_kernel,
// one 1024-thread workgroup per row, adds the chunks' results (exact
// integer sums, order-free maxima) and makes the cuts: one pass over the
// row per cut gathers its bucket (more only when a bucket holds over 2048
// candidates).  The first-level histogram serves all three cuts: every cut
// is a prefix of the candidate order whose target lies within the prefix
// kept so far, so the buckets before the one holding it are kept whole and
// the unfiltered histogram finds the same bucket.  A candidate's mass is
// recomputed where it is needed (it is a pure function of its value).
#include <algorithm>
#include <cfloat>
#include <climits>

#include "srq_internal.h"

namespace srq {
namespace {

constexpr int kST = 1024;      // threads of the row kernel
constexpr int kCT = 256;       // threads of a chunk kernel
constexpr int kBuckets = 2048;
constexpr int kList = 2048;    // candidates of one bucket sorted in LDS
constexpr int kLevels = 4;     // bucket refinements before giving up
constexpr int kMaxChunks = 64; // chunks per row (one wave scans their shares)
constexpr int kChunkMax = 8192; // ids per chunk, at most
constexpr int kRankSort = 128;  // gathered candidates sorted by rank, at most (8 threads each)
constexpr double kFix = 17592186044416.0;  // 2^44: mass of probability 1
// Device scratch of one launch group (ranges, histograms, ids in bucket
// order: about 1 MiB per row of a 128256-id vocabulary); calls with more
// rows run in groups that fit it.
constexpr size_t kSampleScratchMax = (size_t)64 << 20;
// The scans give each thread two buckets / two sorted candidates.
static_assert(kBuckets == 2 * kST && kList == 2 * kST, "two entries per thread");
static_assert(8 * kRankSort <= kST, "8 threads per ranked candidate");
static_assert(kMaxChunks <= 64, "one wave combines a row's chunks");
static_assert(kChunkMax % 256 == 0 && kChunkMax <= 65536, "a chunk in registers, 16-bit ids in a chunk");

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
    uint32_t cstart[kMaxChunks + 1];  // level-0 gather: running counts of the chunks' shares
    uint32_t coff[kMaxChunks];        //   and each share's offset in its chunk's bucket order
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

// Inclusive running sum of v over the workgroup's threads in order: the
// waves' running sums (shuffles), then each adds the totals of the waves
// before it.
__device__ __forceinline__ unsigned long long block_scan(unsigned long long v, SampleLds &s) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const unsigned long long t = __shfl_up(v, o, 64);
        if (lane >= o) v += t;
    }
    if (lane == 63) s.red_u[w] = v;
    __syncthreads();
    unsigned long long add = 0;
    for (int k = 0; k < w; ++k) add += s.red_u[k];
    __syncthreads();
    return v + add;
}

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

// Logits row of sampled row `row`.
__device__ __forceinline__ const float *row_logits(const SampleArgs &A, int row) {
    return A.logits + (int64_t)(A.row_ids ? A.row_ids[row] : row) * A.vocab;
}

// History bits of ids [c0, c0 + 32 * words) of a row, for the repeat penalty.
__device__ __forceinline__ void seen_bits(const SampleArgs &A, int row, int c0, int words, uint32_t *seen,
                                          int nthreads) {
    const int tid = threadIdx.x;
    for (int i = tid; i < words; i += nthreads) seen[i] = 0;
    __syncthreads();
    const int hn = A.history_len ? A.history_len[row] : 0;
    const int32_t *h = A.history + (int64_t)row * A.history_stride;
    for (int i = tid; i < hn; i += nthreads) {
        const int t = h[i] - c0;
        if (t >= 0 && t < 32 * words && t + c0 < A.vocab) atomicOr(&seen[t >> 5], 1u << (t & 31));
    }
    __syncthreads();
}

// Value of id i (logit x): f64, then the repeat penalty for ids in the
// history (a v / 1 or v * 1 is exact, so rp = 1 needs no history).
__device__ __forceinline__ double penalised(const SampleArgs &A, const uint32_t *seen, int c0, int i, float x) {
    double v = x;
    if (A.repeat_penalty != 1.0 && ((seen[(i - c0) >> 5] >> ((i - c0) & 31)) & 1u))
        v = v > 0 ? v / A.repeat_penalty : v * A.repeat_penalty;
    return v;
}

template <int NT, typename T, typename Op>
__device__ __forceinline__ T wg_reduce(T v, T *red, Op op) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = op(v, __shfl_xor(v, o, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    T r = red[0];
#pragma unroll
    for (int w = 1; w < NT / 64; ++w) r = op(r, red[w]);
    __syncthreads();
    return r;
}

struct ChunkRed {
    double d[kCT / 64];
    unsigned long long u[kCT / 64];
    int i[kCT / 64];
};

__device__ __forceinline__ Cand wg_first(Cand c, ChunkRed &r) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const double ov = __shfl_xor(c.v, o, 64);
        const int oi = __shfl_xor(c.id, o, 64);
        if (before(ov, oi, c.v, c.id)) c.v = ov, c.id = oi;
    }
    if ((threadIdx.x & 63) == 0) r.d[threadIdx.x >> 6] = c.v, r.i[threadIdx.x >> 6] = c.id;
    __syncthreads();
    Cand b{r.d[0], r.i[0]};
#pragma unroll
    for (int w = 1; w < kCT / 64; ++w)
        if (before(r.d[w], r.i[w], b.v, b.id)) b.v = r.d[w], b.id = r.i[w];
    __syncthreads();
    return b;
}

constexpr int kCE = kChunkMax / kCT;  // ids of a chunk per thread

// A chunk's logits, all loads issued at once: x[k] is id c0 + k*kCT + tid.
__device__ __forceinline__ void load_chunk(const float *lg, int c0, int c1, float (&x)[kCE]) {
#pragma unroll
    for (int k = 0; k < kCE; ++k) {
        const int i = c0 + k * kCT + (int)threadIdx.x;
        x[k] = i < c1 ? lg[i] : 0.0f;
    }
}

// Chunk c of row `row`: finiteness, candidate count, range and first
// maximum of the values (pass A of sampleWithBlocked's value scan).
__global__ __launch_bounds__(kCT) void sample_range_kernel(const SampleArgs A) {
    extern __shared__ uint32_t seen[];
    __shared__ ChunkRed red;
    const int c = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
    const int c0 = c * A.chunk_len, c1 = min(A.vocab, c0 + A.chunk_len);
    const float *lg = row_logits(A, row);
    float x[kCE];
    load_chunk(lg, c0, c1, x);
    const int blocked = A.blocked ? A.blocked[row] : -1;
    if (A.repeat_penalty != 1.0) seen_bits(A, row, c0, (A.chunk_len + 31) / 32, seen, kCT);
    int bad = 0, cnt = 0;
    double vmax = -DBL_MAX, vmin = DBL_MAX;
    Cand best{-DBL_MAX, INT_MAX};
#pragma unroll
    for (int k = 0; k < kCE; ++k) {
        const int i = c0 + k * kCT + tid;
        if (i >= c1) continue;
        bad |= !isfinite(x[k]);
        if (i == blocked) continue;
        const double v = penalised(A, seen, c0, i, x[k]);
        vmax = fmax(vmax, v);
        vmin = fmin(vmin, v);
        ++cnt;
        if (before(v, i, best.v, best.id)) best.v = v, best.id = i;
    }
    auto add = [](unsigned long long a, unsigned long long b) { return a + b; };
    // bad flags in the low word, counts in the high one (at most 2^31 ids)
    const unsigned long long bc = wg_reduce<kCT>((unsigned long long)bad + ((unsigned long long)cnt << 32), red.u, add);
    vmax = wg_reduce<kCT>(vmax, red.d, [](double a, double b) { return fmax(a, b); });
    vmin = wg_reduce<kCT>(vmin, red.d, [](double a, double b) { return fmin(a, b); });
    best = wg_first(best, red);
    if (tid == 0) {
        SampleRange &o = A.range[(int64_t)row * A.chunks + c];
        o.vmax = vmax, o.vmin = vmin, o.best_v = best.v;
        o.best_id = best.id, o.cnt = (int)(bc >> 32), o.bad = (bc & 0xffffffffull) != 0;
    }
}

// The row's range from its chunks' (the maxima and minima are order-free,
// the counts exact), combined by wave 0 (at most 64 chunks): what one pass
// over the whole row finds.
__device__ __forceinline__ void row_range(const SampleArgs &A, int row, ChunkRed &red, int &bad, int &cnt, double &vmax,
                                          double &vmin) {
    bad = 0, cnt = 0, vmax = -DBL_MAX, vmin = DBL_MAX;
    if (threadIdx.x < 64) {
        if ((int)threadIdx.x < A.chunks) {
            const SampleRange &r = A.range[(int64_t)row * A.chunks + threadIdx.x];
            bad = r.bad, cnt = r.cnt, vmax = r.vmax, vmin = r.vmin;
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            bad |= __shfl_xor(bad, o, 64);
            cnt += __shfl_xor(cnt, o, 64);
            vmax = fmax(vmax, __shfl_xor(vmax, o, 64));
            vmin = fmin(vmin, __shfl_xor(vmin, o, 64));
        }
        if (threadIdx.x == 0) red.d[0] = vmax, red.d[1] = vmin, red.i[0] = bad, red.i[1] = cnt;
    }
    __syncthreads();
    vmax = red.d[0], vmin = red.d[1], bad = red.i[0], cnt = red.i[1];
    __syncthreads();
}

// Chunk c of row `row`: every candidate's integer mass, the chunk's total
// and its counts and masses over the first-level buckets (pass B).
__global__ __launch_bounds__(kCT) void sample_mass_kernel(const SampleArgs A) {
    extern __shared__ uint32_t seen[];
    __shared__ ChunkRed red;
    __shared__ uint32_t hcount[kBuckets];
    __shared__ unsigned long long hmass[kBuckets];
    __shared__ uint16_t lorder[kChunkMax];  // the chunk's ids (less c0) in bucket order
    const int c = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
    const int c0 = c * A.chunk_len, c1 = min(A.vocab, c0 + A.chunk_len);
    const float *lg = row_logits(A, row);
    float x[kCE];
    load_chunk(lg, c0, c1, x);  // in flight while the chunks' ranges combine
    int bad, cnt;
    double vmax, vmin;
    row_range(A, row, red, bad, cnt, vmax, vmin);
    if (bad || cnt == 0) return;  // sample_kernel reports the row
    const int blocked = A.blocked ? A.blocked[row] : -1;
    const double T = A.temperature;
    for (int b = tid; b < kBuckets; b += kCT) hcount[b] = 0, hmass[b] = 0;
    if (A.repeat_penalty != 1.0) seen_bits(A, row, c0, (A.chunk_len + 31) / 32, seen, kCT);
    __syncthreads();
    const double scale0 = vmax > vmin ? (double)kBuckets / (vmax - vmin) : 0.0;
    unsigned long long total = 0;
    // each id's bucket (-1: no candidate) stays in registers for the listing
    int bk[kCE];
#pragma unroll
    for (int k = 0; k < kCE; ++k) {
        const int i = c0 + k * kCT + tid;
        bk[k] = -1;
        if (i >= c1 || i == blocked) continue;
        const double v = penalised(A, seen, c0, i, x[k]);
        const unsigned long long m = (unsigned long long)(exp((v - vmax) / T) * kFix + 0.5);
        total += m;
        const int b = bucket_of(v, vmin, scale0);
        bk[k] = b;
        atomicAdd(&hcount[b], 1u);
        atomicAdd(&hmass[b], m);
    }
    total = wg_reduce<kCT>(total, red.u, [](unsigned long long x, unsigned long long y) { return x + y; });
    const int64_t h = ((int64_t)row * A.chunks + c) * kBuckets;
    for (int b = tid; b < kBuckets; b += kCT) A.hcount[h + b] = hcount[b], A.hmass[h + b] = hmass[b];
    if (tid == 0) A.range[(int64_t)row * A.chunks + c].total = total;

    // Bucket offsets (exclusive running counts; thread t owns buckets
    // 8t .. 8t+7), then the chunk's candidate ids listed in bucket order
    // (within a bucket in any order: the cuts sort what they gather).
    constexpr int BPT = kBuckets / kCT;
    uint32_t own[BPT], sum = 0;
#pragma unroll
    for (int k = 0; k < BPT; ++k) own[k] = hcount[BPT * tid + k], sum += own[k];
    uint32_t inc = sum;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t t = __shfl_up(inc, o, 64);
        if ((tid & 63) >= o) inc += t;
    }
    if ((tid & 63) == 63) red.i[tid >> 6] = (int)inc;
    __syncthreads();
    uint32_t start = inc - sum;
    for (int w = 0; w < (tid >> 6); ++w) start += (uint32_t)red.i[w];
    int cnt_c = 0;  // candidates of the chunk
    for (int w = 0; w < kCT / 64; ++w) cnt_c += red.i[w];
#pragma unroll
    for (int k = 0; k < BPT; ++k) {
        hcount[BPT * tid + k] = start;  // now the bucket's next free slot
        A.hoff[h + BPT * tid + k] = start;
        start += own[k];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kCE; ++k)
        if (bk[k] >= 0) lorder[atomicAdd(&hcount[bk[k]], 1u)] = (uint16_t)(k * kCT + tid);
    __syncthreads();
    int32_t *order = A.order + ((int64_t)row * A.chunks + c) * A.chunk_len;
    for (int k = tid; k < cnt_c; k += kCT) order[k] = c0 + lorder[k];
}

__global__ __launch_bounds__(kST) void sample_kernel(const SampleArgs A) {
    extern __shared__ uint32_t seen[];  // history bitmap, (vocab + 31) / 32 words
    __shared__ SampleLds s;
    const int row = blockIdx.x, tid = threadIdx.x;
    const int vocab = A.vocab;
    const float *lg = row_logits(A, row);
    const int blocked = A.blocked ? A.blocked[row] : -1;
    const double T = A.temperature;
    if (A.repeat_penalty != 1.0) seen_bits(A, row, 0, (vocab + 31) / 32, seen, kST);
    auto value = [&](int i, float x) { return penalised(A, seen, 0, i, x); };

    // ---- the chunks' finiteness, range, first maximum and total mass --------
    // (what passes A and B over the whole row find), combined by wave 0: the
    // maxima and minima are order-free, the counts and masses exact sums.
    constexpr int U = 8;
    int bad = 0, cnt = 0;
    double vmax = -DBL_MAX, vmin = DBL_MAX;
    Cand best{-DBL_MAX, INT_MAX};
    unsigned long long total = 0;
    if (tid < 64) {
        for (int k = tid; k < A.chunks; k += 64) {
            const SampleRange &r = A.range[(int64_t)row * A.chunks + k];
            bad |= r.bad, cnt += r.cnt, vmax = fmax(vmax, r.vmax), vmin = fmin(vmin, r.vmin);
            if (before(r.best_v, r.best_id, best.v, best.id)) best.v = r.best_v, best.id = r.best_id;
            if (T != 0.0) total += r.total;
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            bad |= __shfl_xor(bad, o, 64);
            cnt += __shfl_xor(cnt, o, 64);
            vmax = fmax(vmax, __shfl_xor(vmax, o, 64));
            vmin = fmin(vmin, __shfl_xor(vmin, o, 64));
            total += __shfl_xor(total, o, 64);
            const double ov = __shfl_xor(best.v, o, 64);
            const int oi = __shfl_xor(best.id, o, 64);
            if (before(ov, oi, best.v, best.id)) best.v = ov, best.id = oi;
        }
        if (tid == 0) {
            s.red_d[0] = vmax, s.red_d[1] = vmin, s.red_d[2] = best.v;
            s.red_i[0] = bad, s.red_i[1] = cnt, s.red_i[2] = best.id;
            s.red_u[0] = total;
        }
    }
    __syncthreads();
    vmax = s.red_d[0], vmin = s.red_d[1], best.v = s.red_d[2];
    bad = s.red_i[0], cnt = s.red_i[1], best.id = s.red_i[2];
    total = s.red_u[0];
    __syncthreads();
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
                s.scan[tid] = block_scan(w0 + w1, s);  // inclusive
                __syncthreads();
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
                    s.scan[tid] = block_scan(w0 + w1, s);  // inclusive
                    __syncthreads();
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
            if (level == 0) {
                // The chunks list their ids in first-level bucket order: the
                // bucket's candidates are the chunks' shares of it.
                if (tid < 64) {
                    uint32_t nk = 0, ok = 0;
                    if (tid < A.chunks) {
                        const int64_t hk = ((int64_t)row * A.chunks + tid) * kBuckets + b;
                        nk = A.hcount[hk], ok = A.hoff[hk];
                    }
                    uint32_t inc = nk;
#pragma unroll
                    for (int o = 1; o < 64; o <<= 1) {
                        const uint32_t t = __shfl_up(inc, o, 64);
                        if (tid >= o) inc += t;
                    }
                    if (tid == 0) s.cstart[0] = 0;
                    if (tid < A.chunks) s.cstart[tid + 1] = inc, s.coff[tid] = ok;
                }
                __syncthreads();
                const uint32_t total_n = s.cstart[A.chunks];
                for (uint32_t j = tid; j < total_n; j += kST) {
                    int k = 0;  // the chunk whose share holds entry j
                    for (int w = kMaxChunks / 2; w > 0; w >>= 1)
                        if (k + w < A.chunks && s.cstart[k + w] <= j) k += w;
                    const int i = A.order[((int64_t)row * A.chunks + k) * A.chunk_len + s.coff[k] + (j - s.cstart[k])];
                    const double v = value(i, lg[i]);
                    if (!member(i, v)) continue;
                    const int q = atomicAdd(&s.list_n, 1);
                    s.lv[q] = v, s.li[q] = i, s.lp[q] = mass_of(v);
                }
            }
            __syncthreads();
            for (int base = level == 0 ? vocab : 0; base < vocab; base += kST * U) {
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
            if (ln <= kRankSort) {
                // Few candidates: each one's rank (the candidates before it,
                // counted by 8 threads over every 8th entry), then each is
                // stored at its rank.
                const int e = tid >> 3, q = tid & 7;
                double ev = 0.0;
                int eid = 0, rank = 0;
                unsigned long long ep = 0;
                if (e < ln) {
                    ev = s.lv[e], eid = s.li[e], ep = s.lp[e];
                    for (int j = q; j < ln; j += 8) rank += before(s.lv[j], s.li[j], ev, eid);
                }
                rank += __shfl_xor(rank, 1, 64);
                rank += __shfl_xor(rank, 2, 64);
                rank += __shfl_xor(rank, 4, 64);
                __syncthreads();
                if (e < ln && q == 0) s.lv[rank] = ev, s.li[rank] = eid, s.lp[rank] = ep;
                __syncthreads();
                pw = 1;  // sorted
            } else {
                for (int k = ln + tid; k < pw; k += kST) s.lv[k] = -DBL_MAX, s.li[k] = INT_MAX, s.lp[k] = 0;
                __syncthreads();
            }
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
                s.scan[tid] = block_scan(w0 + w1, s);  // inclusive
                __syncthreads();
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

    // ---- the chunks' total mass and first-level histograms (pass B) ---------
    // (buckets over [vmin, vmax], as locate's first level computes them)
    {
        uint32_t c0 = 0, c1 = 0;
        unsigned long long m0 = 0, m1 = 0;
        const int64_t h = (int64_t)row * A.chunks * kBuckets + 2 * tid;
        constexpr int KB = 16;  // chunks' loads in flight
        for (int k0 = 0; k0 < A.chunks; k0 += KB) {
            uint2 cc[KB];
            ulonglong2 mm[KB];
#pragma unroll
            for (int k = 0; k < KB; ++k) {
                const int64_t o = h + (int64_t)min(k0 + k, A.chunks - 1) * kBuckets;
                cc[k] = *(const uint2 *)(A.hcount + o);
                mm[k] = *(const ulonglong2 *)(A.hmass + o);
            }
#pragma unroll
            for (int k = 0; k < KB; ++k)
                if (k0 + k < A.chunks) c0 += cc[k].x, c1 += cc[k].y, m0 += mm[k].x, m1 += mm[k].y;
        }
        s.h0count[2 * tid] = c0, s.h0count[2 * tid + 1] = c1;
        s.h0mass[2 * tid] = m0, s.h0mass[2 * tid + 1] = m1;
    }
    __syncthreads();  // the cuts read every thread's buckets

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

void sample_plan(int32_t rows, int32_t vocab, int32_t &chunks, int32_t &chunk_len) {
    // About 512 chunk workgroups, chunks of at least 2048 ids.
    int c = (int)std::min<int64_t>(kMaxChunks, std::max<int64_t>(1, (512 + rows - 1) / rows));
    c = (int)std::min<int64_t>(c, (vocab + 2047) / 2048);
    c = (int)std::max<int64_t>({(int64_t)c, 1, ((int64_t)vocab + kChunkMax - 1) / kChunkMax});
    chunk_len = (vocab + c - 1) / c;
    chunks = (vocab + chunk_len - 1) / chunk_len;
}

// Scratch of one launch over `rows` rows.
static size_t plan_bytes(int32_t rows, int32_t vocab) {
    int32_t chunks, len;
    sample_plan(rows, vocab, chunks, len);
    return (size_t)rows * chunks *
           (sizeof(SampleRange) + kBuckets * (sizeof(unsigned long long) + 2 * sizeof(uint32_t)) +
            (size_t)len * sizeof(int32_t));
}

// Rows per launch group: the most (a power of two up to 1024) whose scratch
// fits kSampleScratchMax.  A row's draw is exact whatever the chunk plan, so
// grouping changes no result.
static int32_t group_rows(int32_t vocab) {
    int32_t g = 1024;
    while (g > 1 && plan_bytes(g, vocab) > kSampleScratchMax) g /= 2;
    return g;
}

size_t sample_scratch_bytes(int32_t rows, int32_t vocab) {
    const int32_t g = group_rows(vocab);
    if (rows <= g) return plan_bytes(rows, vocab);
    const int32_t tail = rows % g;
    return std::max(plan_bytes(g, vocab), tail ? plan_bytes(tail, vocab) : (size_t)0);
}

int launch_sample(hipStream_t s, const SampleArgs &a0, void *scratch) {
    if (a0.rows <= 0) return SRQ_OK;
    const size_t lds = (size_t)((a0.vocab + 31) / 32) * 4;
    if (lds > 48 * 1024) return fail(SRQ_EINVAL, "sample: vocabulary of %d ids exceeds the history bitmap", a0.vocab);
    const int32_t g = group_rows(a0.vocab);
    for (int32_t r0 = 0; r0 < a0.rows; r0 += g) {
        // Rows [r0, r0 + a.rows) of the call: every per-row pointer moves on.
        SampleArgs a = a0;
        a.rows = std::min(g, a0.rows - r0);
        if (a0.row_ids)
            a.row_ids = a0.row_ids + r0;
        else
            a.logits = a0.logits + (int64_t)r0 * a0.vocab;
        if (a0.history) a.history = a0.history + (int64_t)r0 * a0.history_stride;
        if (a0.history_len) a.history_len = a0.history_len + r0;
        if (a0.blocked) a.blocked = a0.blocked + r0;
        a.rng = a0.rng + r0;
        a.ids = a0.ids + r0;
        sample_plan(a.rows, a.vocab, a.chunks, a.chunk_len);
        if (a.chunks > kMaxChunks || a.chunk_len > kChunkMax)
            return fail(SRQ_EINVAL, "sample: vocabulary of %d ids exceeds the chunk plan", a.vocab);
        // [ranges: rows x chunks][masses: rows x chunks x 2048][counts: likewise]
        // [offsets: likewise][ids in bucket order: rows x chunks x chunk_len]
        const size_t nb = (size_t)a.rows * a.chunks * kBuckets;
        a.range = (SampleRange *)scratch;
        a.hmass = (unsigned long long *)(a.range + (size_t)a.rows * a.chunks);
        a.hcount = (uint32_t *)(a.hmass + nb);
        a.hoff = a.hcount + nb;
        a.order = (int32_t *)(a.hoff + nb);
        const size_t clds = (size_t)((a.chunk_len + 31) / 32) * 4;
        const dim3 grid(a.chunks, a.rows);
        sample_range_kernel<<<grid, kCT, a.repeat_penalty != 1.0 ? clds : 0, s>>>(a);
        SRQ_HIP(hipGetLastError());
        if (a.temperature != 0.0) {
            sample_mass_kernel<<<grid, kCT, a.repeat_penalty != 1.0 ? clds : 0, s>>>(a);
            SRQ_HIP(hipGetLastError());
        }
        sample_kernel<<<a.rows, kST, a.repeat_penalty != 1.0 ? lds : 0, s>>>(a);
        SRQ_HIP(hipGetLastError());
    }
    return SRQ_OK;
}

}  // namespace srq
