// Dequant-GEMM on FP32 MFMA for prefill chunks and batched steps (n > 16).
//
// Counterpart of linearQ8Into / linearQ4Into / linearFP32Range
// (cmd/monolith/monolith.go M:3942-4780) when many activation rows share
// each weight read.
//
// Tiling (gfx950, wave64, v_mfma_f32_16x16x4f32):
//  - Workgroup tile BMT (activation rows: 32 when n <= 32, else 64) x 128
//    (output features), K step 32 (half a scale block).  4 waves; each owns
//    32 rows x (128 / waves across N) features as 16x16 MFMA tiles with FP32
//    accumulators.
//  - Weights are read once per K step as int8 / packed int4 / f32,
//    dequantised in registers to f32(code)*scale (the copyRow rounding,
//    M:3900-3921) and stored to LDS; activations go to LDS unchanged.
//  - Within a K step, MFMA step s feeds lane group g (lane/16) the K index
//    8g+s, so every lane reads its 8 K values of a row as two ds_read_b128.
//  - Global loads for step k+1 are issued before the MFMAs of step k
//    (register double buffering); LDS is double buffered.
//  - Split K: when the (features x rows) tiles alone cannot fill the chip
//    (few rows per step, narrow outputs), blockIdx.z takes a slice of the
//    K steps and writes its partial sums to scratch; gemm_reduce_kernel adds
//    the slices in slice order, then the residual.  Results are
//    deterministic for a given (n, rows, cols).
//  - Rows holding any |x| > f32(MaxFloat32/(2*64*127)) (M:4346-4354) are
//    detected while staging x and recomputed in FP64 (linearQ8WideInto /
//    linearQ4WideInto, M:4356-4382, M:4754-4780): by the workgroup itself
//    when it saw all of K, else by the reduction from per-slice flags.
#include <algorithm>

#include "srq_internal.h"

namespace srq {
namespace {

constexpr int BN = 128, BK = 32, LDK = BK + 4;
constexpr int kFillWGs = 512;      // two resident workgroups on each of 256 CUs
constexpr int kMinSliceSteps = 8;  // K steps per split-K slice (256 inputs)
typedef float floatx4 __attribute__((ext_vector_type(4)));

template <int FMT>
__device__ __forceinline__ void load_b(const uint8_t *__restrict__ W, const float *__restrict__ S, int64_t rows,
                                       int64_t cols, int64_t n0, int64_t k0, int tid, uint4 (&raw)[4],
                                       float &scale) {
    const int r = tid >> 1, half = tid & 1;
    const int64_t row = n0 + r;
    if (row >= rows) {
        raw[0] = raw[1] = raw[2] = raw[3] = make_uint4(0, 0, 0, 0);
        scale = 0.0f;
        return;
    }
    if constexpr (FMT == SRQ_Q8) {
        raw[0] = ld_stream16(W + row * cols + k0 + 16 * half);
        scale = S[row * groups_of(cols) + k0 / kBlock];
    } else if constexpr (FMT == SRQ_Q4) {
        const uint2 v = ld_stream8(W + row * (cols / 2) + k0 / 2 + 8 * half);
        raw[0] = make_uint4(v.x, v.y, 0, 0);
        scale = S[row * groups_of(cols) + k0 / kBlock];
    } else {
        const uint4 *p = (const uint4 *)(W + (row * cols + k0 + 16 * half) * 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) raw[i] = ld_stream16(p + i);
        scale = 1.0f;
    }
}

template <int FMT>
__device__ __forceinline__ void store_b(float *Bs, int tid, const uint4 (&raw)[4], float scale) {
    const int r = tid >> 1, half = tid & 1;
    float *dst = Bs + r * LDK + 16 * half;
    float w[16];
    if constexpr (FMT == SRQ_Q8) {
        const uint32_t d[4] = {raw[0].x, raw[0].y, raw[0].z, raw[0].w};
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int b = 0; b < 4; ++b) w[4 * k + b] = (float)(int32_t)(int8_t)(d[k] >> (8 * b)) * scale;
    } else if constexpr (FMT == SRQ_Q4) {
        const uint32_t d[2] = {raw[0].x, raw[0].y};
#pragma unroll
        for (int k = 0; k < 2; ++k)
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const uint32_t byte = (d[k] >> (8 * b)) & 0xFFu;
                w[8 * k + 2 * b] = (float)(((int32_t)(byte << 28)) >> 28) * scale;
                w[8 * k + 2 * b + 1] = (float)(((int32_t)(byte << 24)) >> 28) * scale;
            }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            w[4 * i + 0] = __uint_as_float(raw[i].x);
            w[4 * i + 1] = __uint_as_float(raw[i].y);
            w[4 * i + 2] = __uint_as_float(raw[i].z);
            w[4 * i + 3] = __uint_as_float(raw[i].w);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) *(float4 *)(dst + 4 * i) = make_float4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
}

// Activation tile BMT x BK: each thread stages BMT*BK/256 floats of one row.
template <int BMT>
struct ATile {
    static constexpr int FPT = BMT * BK / 256;  // floats per thread (8 or 4)
    static constexpr int TPR = BK / FPT;        // threads per row
    static constexpr int NV = FPT / 4;          // float4 per thread
};

template <int BMT>
__device__ __forceinline__ void load_a(const float *__restrict__ X, int32_t n, int64_t cols, int64_t m0, int64_t k0,
                                       int tid, float4 (&a)[ATile<BMT>::NV]) {
    constexpr int FPT = ATile<BMT>::FPT, TPR = ATile<BMT>::TPR, NV = ATile<BMT>::NV;
    const int r = tid / TPR, kq = (tid % TPR) * FPT;
    const int64_t m = m0 + r;
    if (m < n) {
        const float4 *p = (const float4 *)(X + m * cols + k0 + kq);
#pragma unroll
        for (int i = 0; i < NV; ++i) a[i] = p[i];
    } else {
#pragma unroll
        for (int i = 0; i < NV; ++i) a[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

// Stores the staged floats; returns the largest |x| among them.
template <int BMT>
__device__ __forceinline__ float store_a(float *As, int tid, const float4 (&a)[ATile<BMT>::NV]) {
    constexpr int FPT = ATile<BMT>::FPT, TPR = ATile<BMT>::TPR, NV = ATile<BMT>::NV;
    const int r = tid / TPR, kq = (tid % TPR) * FPT;
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        *(float4 *)(As + r * LDK + kq + 4 * i) = a[i];
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(a[i].x), fabsf(a[i].y)), fmaxf(fabsf(a[i].z), fabsf(a[i].w))));
    }
    return amax;
}

// linearQ8WideInto / linearQ4WideInto (M:4356-4382, M:4754-4780): output o
// of row m in FP64, per-block partial sums scaled in FP64, plus residual.
__device__ __forceinline__ double wide_weight(int fmt, const uint8_t *wrow, int64_t c) {
    if (fmt == SRQ_Q8) return (double)((const int8_t *)wrow)[c];
    if (fmt == SRQ_Q4) {
        uint32_t b = wrow[c >> 1];
        uint32_t nib = (c & 1) ? (b >> 4) : (b & 15u);
        return (double)(((int32_t)(nib << 28)) >> 28);
    }
    return (double)((const float *)wrow)[c];
}

__device__ __forceinline__ float wide_output(const GemmArgs &G, int64_t m, int64_t o) {
    const uint8_t *wrow = (const uint8_t *)G.values + o * row_bytes(G.fmt, G.cols);
    const float *xr = G.x + m * G.cols;
    const int64_t groups = groups_of(G.cols);
    double sum = 0.0;
    for (int64_t g = 0; g < groups; ++g) {
        double part = 0.0;
        const int64_t end = (g + 1) * kBlock < G.cols ? (g + 1) * kBlock : G.cols;
        for (int64_t j = g * kBlock; j < end; ++j) part += (double)xr[j] * wide_weight(G.fmt, wrow, j);
        sum += part * (G.fmt == SRQ_F32 ? 1.0 : (double)G.scales[o * groups + g]);
    }
    float v = (float)sum;
    if (G.residual) v = G.residual[m * G.y_stride + o] + v;
    return v;
}

// partial == nullptr: one slice covers all K and the tile writes y.
// Otherwise slice blockIdx.z covers K steps [z*kper, (z+1)*kper) and
// writes partial[z][m][j] (n x rows per slice) and, from the first feature
// tile, wflags[z][m].
template <int FMT, int BMT>
__global__ __launch_bounds__(256) void gemm_kernel(const GemmArgs G, float *__restrict__ partial,
                                                   int32_t *__restrict__ wflags, const int kper) {
    constexpr int WM = BMT / 32, WN = 4 / WM, TN = BN / WN / 16, NV = ATile<BMT>::NV;
    __shared__ __attribute__((aligned(16))) float As[2][BMT * LDK];
    __shared__ __attribute__((aligned(16))) float Bs[2][BN * LDK];
    __shared__ int row_wide[BMT];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int64_t n0 = (int64_t)blockIdx.x * BN, m0 = (int64_t)blockIdx.y * BMT;
    const uint8_t *W = (const uint8_t *)G.values;
    const int64_t cols = G.cols;
    const int kbeg = (int)blockIdx.z * kper;
    const int kend = min(kbeg + kper, (int)(cols / BK));
    if (tid < BMT) row_wide[tid] = 0;

    floatx4 acc[2][TN];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    uint4 braw[4];
    float bscale;
    float4 areg[NV];
    load_b<FMT>(W, G.scales, G.rows, cols, n0, (int64_t)kbeg * BK, tid, braw, bscale);
    load_a<BMT>(G.x, G.n, cols, m0, (int64_t)kbeg * BK, tid, areg);
    store_b<FMT>(Bs[0], tid, braw, bscale);
    float amax = store_a<BMT>(As[0], tid, areg);
    __syncthreads();

    const int gq = lane >> 4, li = lane & 15;
    for (int ks = kbeg; ks < kend; ++ks) {
        const int cur = (ks - kbeg) & 1;
        if (ks + 1 < kend) {
            load_b<FMT>(W, G.scales, G.rows, cols, n0, (int64_t)(ks + 1) * BK, tid, braw, bscale);
            load_a<BMT>(G.x, G.n, cols, m0, (int64_t)(ks + 1) * BK, tid, areg);
        }
        const float *as = As[cur], *bs = Bs[cur];
        float af[2][8], bf[TN][8];
#pragma unroll
        for (int tm = 0; tm < 2; ++tm) {
            const float *p = as + (wm * 32 + tm * 16 + li) * LDK + 8 * gq;
            const float4 u = *(const float4 *)p, v = *(const float4 *)(p + 4);
            af[tm][0] = u.x, af[tm][1] = u.y, af[tm][2] = u.z, af[tm][3] = u.w;
            af[tm][4] = v.x, af[tm][5] = v.y, af[tm][6] = v.z, af[tm][7] = v.w;
        }
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
            const float *p = bs + (wn * TN * 16 + tn * 16 + li) * LDK + 8 * gq;
            const float4 u = *(const float4 *)p, v = *(const float4 *)(p + 4);
            bf[tn][0] = u.x, bf[tn][1] = u.y, bf[tn][2] = u.z, bf[tn][3] = u.w;
            bf[tn][4] = v.x, bf[tn][5] = v.y, bf[tn][6] = v.z, bf[tn][7] = v.w;
        }
#pragma unroll
        for (int s = 0; s < 8; ++s)
#pragma unroll
            for (int tm = 0; tm < 2; ++tm)
#pragma unroll
                for (int tn = 0; tn < TN; ++tn)
                    acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[tm][s], bf[tn][s], acc[tm][tn], 0, 0, 0);
        if (ks + 1 < kend) {
            store_b<FMT>(Bs[cur ^ 1], tid, braw, bscale);
            amax = fmaxf(amax, store_a<BMT>(As[cur ^ 1], tid, areg));
        }
        __syncthreads();
    }
    if (amax > kWideLimit) row_wide[tid / ATile<BMT>::TPR] = 1;
    __syncthreads();

    // D layout of 16x16x4: lane holds rows 4*(lane/16)+r, column lane%16.
    if (partial) {
        float *P = partial + (int64_t)blockIdx.z * G.n * G.rows;
        if (blockIdx.x == 0 && tid < BMT && m0 + tid < G.n) wflags[(int64_t)blockIdx.z * G.n + m0 + tid] = row_wide[tid];
#pragma unroll
        for (int tm = 0; tm < 2; ++tm)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t m = m0 + wm * 32 + tm * 16 + 4 * gq + r;
                if (m >= G.n) continue;
#pragma unroll
                for (int tn = 0; tn < TN; ++tn) {
                    const int64_t j = n0 + wn * TN * 16 + tn * 16 + li;
                    if (j < G.rows) P[m * G.rows + j] = acc[tm][tn][r];
                }
            }
        return;
    }
#pragma unroll
    for (int tm = 0; tm < 2; ++tm)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int mi = wm * 32 + tm * 16 + 4 * gq + r;
            const int64_t m = m0 + mi;
            if (m >= G.n || row_wide[mi]) continue;
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) {
                const int64_t j = n0 + wn * TN * 16 + tn * 16 + li;
                if (j >= G.rows) continue;
                float v = acc[tm][tn][r];
                if (G.residual) v = G.residual[m * G.y_stride + j] + v;
                G.y[m * G.y_stride + j] = v;
            }
        }
    // This workgroup saw all of K: it recomputes its wide rows itself.
    for (int mi = 0; mi < BMT; ++mi) {
        if (!row_wide[mi] || m0 + mi >= G.n) continue;
        const int64_t j = n0 + tid;
        if (tid < BN && j < G.rows) G.y[(m0 + mi) * G.y_stride + j] = wide_output(G, m0 + mi, j);
    }
}

// y[m][j] = residual + sum over slices z (in order) of partial[z][m][j];
// rows flagged wide by any slice take the FP64 path instead.
__global__ __launch_bounds__(256) void gemm_reduce_kernel(const GemmArgs G, const float *__restrict__ partial,
                                                          const int32_t *__restrict__ wflags, const int slices) {
    const int64_t m = blockIdx.y, j = (int64_t)blockIdx.x * 256 + threadIdx.x;
    int wide = 0;
    for (int z = 0; z < slices; ++z) wide |= wflags[(int64_t)z * G.n + m];
    if (j >= G.rows) return;
    float v;
    if (wide) {
        v = wide_output(G, m, j);
    } else {
        const int64_t plane = (int64_t)G.n * G.rows;
        const float *p = partial + m * G.rows + j;
        float s = p[0];
        for (int z = 1; z < slices; ++z) s += p[z * plane];
        v = G.residual ? G.residual[m * G.y_stride + j] + s : s;
    }
    G.y[m * G.y_stride + j] = v;
}

struct GemmPlan {
    int bm, slices, kper;
};

// Tile height from n; K slices so that tiles x slices reach kFillWGs
// workgroups, each slice at least kMinSliceSteps K steps.
GemmPlan plan_gemm(int32_t n, int64_t rows, int64_t cols) {
    GemmPlan p;
    p.bm = n <= 32 ? 32 : 64;
    const int64_t tiles = ((rows + BN - 1) / BN) * ((n + p.bm - 1) / p.bm);
    const int ksteps = (int)(cols / BK);
    int slices = 1;
    if (tiles < kFillWGs) {
        const int64_t want = (kFillWGs + tiles - 1) / tiles;
        slices = (int)std::max<int64_t>(1, std::min<int64_t>(want, ksteps / kMinSliceSteps));
    }
    p.kper = (ksteps + slices - 1) / slices;
    p.slices = (ksteps + p.kper - 1) / p.kper;
    return p;
}

template <int FMT, int BMT>
void launch_tiles(hipStream_t s, const GemmArgs &a, const GemmPlan &p, float *partial, int32_t *wflags) {
    dim3 grid((unsigned)((a.rows + BN - 1) / BN), (unsigned)((a.n + BMT - 1) / BMT), (unsigned)p.slices);
    gemm_kernel<FMT, BMT><<<grid, 256, 0, s>>>(a, partial, wflags, p.kper);
}

template <int BMT>
void launch_fmt(hipStream_t s, const GemmArgs &a, const GemmPlan &p, float *partial, int32_t *wflags) {
    switch (a.fmt) {
        case SRQ_Q8: launch_tiles<SRQ_Q8, BMT>(s, a, p, partial, wflags); break;
        case SRQ_Q4: launch_tiles<SRQ_Q4, BMT>(s, a, p, partial, wflags); break;
        default: launch_tiles<SRQ_F32, BMT>(s, a, p, partial, wflags); break;
    }
}

}  // namespace

bool gemm_ok(int fmt, int64_t cols) {
    (void)fmt;
    return cols % BK == 0 && cols >= BK;
}

size_t gemm_scratch_bytes(int32_t n, int64_t rows, int64_t cols) {
    if (n <= 0 || rows <= 0 || !gemm_ok(SRQ_F32, cols)) return 0;
    const GemmPlan p = plan_gemm(n, rows, cols);
    if (p.slices == 1) return 0;
    return (size_t)p.slices * (size_t)n * ((size_t)rows + 1) * 4;
}

int launch_gemm(hipStream_t s, const GemmArgs &a, void *scratch, size_t scratch_bytes) {
    if (a.n <= 0 || a.rows <= 0) return SRQ_OK;
    if (!gemm_ok(a.fmt, a.cols)) return fail(SRQ_EINVAL, "gemm: cols=%lld not a multiple of %d", (long long)a.cols, BK);
    const GemmPlan p = plan_gemm(a.n, a.rows, a.cols);
    float *partial = nullptr;
    int32_t *wflags = nullptr;
    if (p.slices > 1) {
        const size_t need = gemm_scratch_bytes(a.n, a.rows, a.cols);
        if (!scratch || scratch_bytes < need)
            return fail(SRQ_EINVAL, "gemm: scratch of %zu bytes, %zu needed", scratch_bytes, need);
        partial = (float *)scratch;
        wflags = (int32_t *)(partial + (size_t)p.slices * a.n * a.rows);
    }
    if (p.bm == 32)
        launch_fmt<32>(s, a, p, partial, wflags);
    else
        launch_fmt<64>(s, a, p, partial, wflags);
    SRQ_HIP(hipGetLastError());
    if (p.slices > 1) {
        dim3 grid((unsigned)((a.rows + 255) / 256), (unsigned)a.n);
        gemm_reduce_kernel<<<grid, 256, 0, s>>>(a, partial, wflags, p.slices);
        SRQ_HIP(hipGetLastError());
    }
    return SRQ_OK;
}

}  // namespace srq
