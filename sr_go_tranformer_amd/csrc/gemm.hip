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
//    the slices in slice order, then the residual.  The slice count depends
//    on (rows, cols) only, so a row's bits do not depend on n.
//  - Rows holding any |x| > f32(MaxFloat32/(2*64*127)) (M:4346-4354) are
//    detected while staging x and recomputed in FP64 (linearQ8WideInto /
//    linearQ4WideInto, M:4356-4382, M:4754-4780): by the workgroup itself
//    when it saw all of K, else by the reduction from per-slice flags.
#include <algorithm>
#include <utility>

#include "srq_internal.h"

namespace srq {
namespace {

constexpr int BN = 128, BK = 32, LDK = BK + 4;
constexpr int kCUs = 256;          // MI355X compute units
constexpr int kMinSliceInputs = 256;  // inputs per split-K slice, at least
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

// Sum over the K slices z of p[z * plane], added in slice order.  The loads
// go out eight slices at a time (a loop of one load per add would wait a
// full memory latency per slice).
template <typename V>
__device__ __forceinline__ V slice_sum(const float *__restrict__ p, int64_t plane, int slices) {
    V acc = *(const V *)p;
    for (int z = 1; z < slices; z += 8) {
        V a[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (z + i < slices) a[i] = *(const V *)(p + (int64_t)(z + i) * plane);
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (z + i < slices) acc += a[i];
    }
    return acc;
}

// Whether any K slice flagged row m wide.  Each thread reads a share of the
// flags, so the workgroup pays one memory latency (a loop over the slices in
// every thread would pay one per slice).  Every thread of the workgroup
// calls it.
__device__ __forceinline__ int any_wide(const int32_t *__restrict__ wflags, int64_t n, int64_t m, int slices) {
    int f = 0;
    for (int z = threadIdx.x; z < slices; z += blockDim.x) f |= wflags[(int64_t)z * n + m];
    return __syncthreads_or(f);
}

// y[m][j] = residual + sum over slices z (in order) of partial[z][m][j];
// rows flagged wide by any slice take the FP64 path instead.
__global__ __launch_bounds__(256) void gemm_reduce_kernel(const GemmArgs G, const float *__restrict__ partial,
                                                          const int32_t *__restrict__ wflags, const int slices) {
    const int64_t m = blockIdx.y, j = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int wide = any_wide(wflags, G.n, m, slices);
    if (j >= G.rows) return;
    float v;
    if (wide) {
        v = wide_output(G, m, j);
    } else {
        const float s = slice_sum<float>(partial + m * G.rows + j, (int64_t)G.n * G.rows, slices);
        v = G.residual ? G.residual[m * G.y_stride + j] + s : s;
    }
    G.y[m * G.y_stride + j] = v;
}

// ---------------------------------------------------------------------------
// Q8 / Q4 weights on bf16 MFMA (v_mfma_f32_16x16x32_bf16), FP32-exact terms.
//
// Every int8 / int4 code is an integer of at most 8 significant bits, so it
// is exact in bf16.  Every f32 activation x splits exactly into three bf16
// terms: hi = x with the low 16 bits cleared, mid = the same of x - hi, and
// lo = x - hi - mid (at most 8 significant bits left).  Each code x term
// product has at most 16 significant bits and is exact in the FP32
// accumulator, so sum_k x_k * c_k is formed from exact products with FP32
// additions -- the precision class of an FP32 dot product, at three bf16
// MFMA passes instead of the 16 FP32 ones per 16x16x64 block.
//
// Per 64-input scale block, a fresh FP32 block sum is scaled into the
// running sum: acc = fma(block, scale, acc) (the per-block form of
// linearQ8Into's dequantised dot, M:3942-4000).
//
// Tiling: 4 waves, each owning TM x TN tiles of 16x16 (TM*16 activation rows
// x TN*16 features); a workgroup covers TM*16 rows x 64*TN features.
//  - Weights go from HBM straight into MFMA operand registers: lane
//    (i = lane%16, q = lane/16) of feature tile tn loads the 16 codes
//    [16q, 16q+16) of its row's block (Q8: 16 bytes, Q4: 8 bytes); the
//    first 8 feed MFMA half 0, the rest half 1.  D blocks of weights and
//    activations are in flight.
//  - Activations are staged once per block into LDS as the three bf16
//    planes, row stride 72 bf16 (conflict-free 16-byte reads of 16 rows).
//    Lane (i, q) reads row i, inputs [16q + 8h, 16q + 8h + 8) for half h:
//    the same K map as the weights.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
constexpr int XLD = 72;

// Workgroup barrier over LDS only.  __syncthreads() also waits for every
// global load in flight (vmcnt(0)), which in the block loop below would
// drain the weight and activation loads issued blocks ahead at every block.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <int TM, int NT = 256>
struct XTile {
    static constexpr int BM = TM * 16;
    static constexpr int FPT = BM * 64 / NT;  // staged floats per thread (16, 8 or 4)
    static constexpr int TPR = 64 / FPT;      // threads per row
    static constexpr int NV = FPT / 4;
    static constexpr int PLANE = BM * XLD;    // bf16 per plane
    static_assert(FPT >= 4, "at least one float4 per thread");
};

__device__ __forceinline__ uint32_t pk_hi16(float lo, float hi) {
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// One lane's 16 codes of a block: Q8 16 bytes, Q4 8 bytes.
template <int FMT>
struct XRaw {
    typedef uint32_t type __attribute__((ext_vector_type(FMT == SRQ_Q8 ? 4 : 2)));
};

template <int FMT>
__device__ __forceinline__ void xload_b(const uint8_t *__restrict__ W, const float *__restrict__ S, int64_t rows,
                                        int64_t cols, int64_t groups, int64_t row, int64_t g, int q,
                                        typename XRaw<FMT>::type &raw, float &scale) {
    typedef typename XRaw<FMT>::type R;
    if (row < rows) {
        if constexpr (FMT == SRQ_Q8)
            raw = *(const R *)(W + row * cols + g * kBlock + 16 * q);
        else
            raw = *(const R *)(W + row * (cols / 2) + g * (kBlock / 2) + 8 * q);
        scale = S[row * groups + g];
    } else {
        raw = R{};
        scale = 0.0f;
    }
}

// Codes of one lane's block slice -> the two bf16x8 MFMA operands.
template <int FMT>
__device__ __forceinline__ void xcodes(const typename XRaw<FMT>::type raw, bf16x8 &h0, bf16x8 &h1) {
    u32x4v p0, p1;
    if constexpr (FMT == SRQ_Q8) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t d = raw[w];
            const float c0 = (float)(int32_t)(int8_t)d, c1 = (float)(int32_t)(int8_t)(d >> 8);
            const float c2 = (float)(int32_t)(int8_t)(d >> 16), c3 = (float)((int32_t)d >> 24);
            const uint32_t a = pk_hi16(c0, c1), b = pk_hi16(c2, c3);
            if (w < 2) {
                p0[2 * w] = a;
                p0[2 * w + 1] = b;
            } else {
                p1[2 * w - 4] = a;
                p1[2 * w - 3] = b;
            }
        }
    } else {
        // code/16 (exact in bf16), one SDWA convert per nibble; the block's
        // scale carries the factor 16 back (SRQ_CONVERT), so the product
        // block * scale is unchanged bit for bit
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            const uint32_t d = raw[w], h = d >> 4;
            u32x4v &p = w == 0 ? p0 : p1;
            p[0] = pk_hi16(nib16<0>(d), nib16<0>(h));
            p[1] = pk_hi16(nib16<1>(d), nib16<1>(h));
            p[2] = pk_hi16(nib16<2>(d), nib16<2>(h));
            p[3] = pk_hi16(nib16<3>(d), nib16<3>(h));
        }
    }
    h0 = __builtin_bit_cast(bf16x8, p0);
    h1 = __builtin_bit_cast(bf16x8, p1);
}

template <int TM>
__device__ __forceinline__ void xload_a(const float *__restrict__ X, int32_t n, int64_t cols, int64_t m0, int64_t g,
                                        int tid, float4 (&a)[XTile<TM>::NV]) {
    constexpr int FPT = XTile<TM>::FPT, TPR = XTile<TM>::TPR, NV = XTile<TM>::NV;
    const int r = tid / TPR, c = (tid % TPR) * FPT;
    const int64_t m = m0 + r;
    if (m < n) {
        const float4 *p = (const float4 *)(X + m * cols + g * kBlock + c);
#pragma unroll
        for (int i = 0; i < NV; ++i) a[i] = p[i];
    } else {
#pragma unroll
        for (int i = 0; i < NV; ++i) a[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

// Splits the staged floats into the hi / mid / lo planes; returns max |x|.
template <int TM, int NT = 256>
__device__ __forceinline__ float xstore_a(__bf16 *As, int tid, const float4 (&a)[XTile<TM, NT>::NV]) {
    typedef XTile<TM, NT> X;
    constexpr int FPT = X::FPT, TPR = X::TPR, NV = X::NV, PLANE = X::PLANE;
    const int r = tid / TPR, c = (tid % TPR) * FPT;
    float amax = 0.0f;
    uint32_t ph[FPT / 2], pm[FPT / 2], pl[FPT / 2];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const float v[4] = {a[i].x, a[i].y, a[i].z, a[i].w};
        float r1[4], r2[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            amax = fmaxf(amax, fabsf(v[e]));
            r1[e] = v[e] - __uint_as_float(__float_as_uint(v[e]) & 0xFFFF0000u);
            r2[e] = r1[e] - __uint_as_float(__float_as_uint(r1[e]) & 0xFFFF0000u);
        }
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            ph[2 * i + e] = pk_hi16(v[2 * e], v[2 * e + 1]);
            pm[2 * i + e] = pk_hi16(r1[2 * e], r1[2 * e + 1]);
            pl[2 * i + e] = pk_hi16(r2[2 * e], r2[2 * e + 1]);
        }
    }
    __bf16 *dst = As + r * XLD + c;
    if constexpr (FPT == 4) {
        *(uint2 *)dst = make_uint2(ph[0], ph[1]);
        *(uint2 *)(dst + PLANE) = make_uint2(pm[0], pm[1]);
        *(uint2 *)(dst + 2 * PLANE) = make_uint2(pl[0], pl[1]);
    } else {
#pragma unroll
        for (int i = 0; i < FPT / 8; ++i) {
            *(uint4 *)(dst + 8 * i) = make_uint4(ph[4 * i], ph[4 * i + 1], ph[4 * i + 2], ph[4 * i + 3]);
            *(uint4 *)(dst + PLANE + 8 * i) = make_uint4(pm[4 * i], pm[4 * i + 1], pm[4 * i + 2], pm[4 * i + 3]);
            *(uint4 *)(dst + 2 * PLANE + 8 * i) = make_uint4(pl[4 * i], pl[4 * i + 1], pl[4 * i + 2], pl[4 * i + 3]);
        }
    }
    return amax;
}

// Stores a tile's accumulators: partial sums of its K slice (partial !=
// nullptr), else y (+ residual), rows holding a |x| > kWideLimit recomputed
// in FP64.  D layout of 16x16x32: lane holds rows 4*(lane/16)+r, column
// lane%16.
// TN feature tiles per wave, XBN features and NT threads per workgroup.
template <int TM, int TN, int XBN = 64 * TN, int NT = 256>
__device__ __forceinline__ void x3_finish(const GemmArgs &G, float *__restrict__ partial, int32_t *__restrict__ wflags,
                                          const floatx4 (&acc)[TM][TN], const float amax, int *row_wide,
                                          const int64_t n0, const int64_t m0, const int tid) {
    constexpr int BM = XTile<TM>::BM;
    const int lane = tid & 63, li = lane & 15, q = lane >> 4;
    if (amax > kWideLimit) row_wide[tid / XTile<TM, NT>::TPR] = 1;
    lds_barrier();

    if (partial) {
        float *P = partial + (int64_t)blockIdx.z * G.n * G.rows;
        if (blockIdx.x == 0 && tid < BM && m0 + tid < G.n) wflags[(int64_t)blockIdx.z * G.n + m0 + tid] = row_wide[tid];
        const int64_t nw = (int64_t)blockIdx.x * XBN;  // the workgroup's first feature
        if (m0 + BM <= G.n && nw + XBN <= G.rows && G.rows * BM < (int64_t(1) << 30)) {
            // Every output of the workgroup is in bounds (a uniform test) and
            // its byte offsets from the corner fit 32 bits: no per-store checks.
            float *Pt = P + m0 * G.rows + nw;
            const uint32_t ld = (uint32_t)G.rows, c0 = (uint32_t)(n0 - nw) + (uint32_t)li;
#pragma unroll
            for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t mo = (uint32_t)(tm * 16 + 4 * q + r) * ld + c0;
#pragma unroll
                    for (int tn = 0; tn < TN; ++tn)
                        *(float *)((char *)Pt + (mo + (uint32_t)(tn * 16)) * 4u) = acc[tm][tn][r];
                }
            return;
        }
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t m = m0 + tm * 16 + 4 * q + r;
                if (m >= G.n) continue;
#pragma unroll
                for (int tn = 0; tn < TN; ++tn) {
                    const int64_t j = n0 + tn * 16 + li;
                    if (j < G.rows) P[m * G.rows + j] = acc[tm][tn][r];
                }
            }
        return;
    }
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int mi = tm * 16 + 4 * q + r;
            const int64_t m = m0 + mi;
            if (m >= G.n || row_wide[mi]) continue;
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) {
                const int64_t j = n0 + tn * 16 + li;
                if (j >= G.rows) continue;
                float v = acc[tm][tn][r];
                if (G.residual) v = G.residual[m * G.y_stride + j] + v;
                G.y[m * G.y_stride + j] = v;
            }
        }
    for (int mi = 0; mi < BM; ++mi) {
        if (!row_wide[mi] || m0 + mi >= G.n) continue;
        const int64_t j = (int64_t)blockIdx.x * XBN + tid;
        if (tid < XBN && j < G.rows) G.y[(m0 + mi) * G.y_stride + j] = wide_output(G, m0 + mi, j);
    }
}

// As gemm_kernel, for Q8 / Q4 weights and cols % 64 == 0; kper counts
// 64-input blocks.
//
// Software pipeline, two blocks deep: while the MFMAs of block g run, the
// wave converts block g+1's codes (loaded two blocks earlier) and splits
// block g+1's activations into the other LDS stage; blocks g+2 and g+3 are
// in flight.  Rows past the ends are clamped (weights: row rows-1;
// activations: row n-1) and their outputs are never stored, so the block
// body has no per-lane branches.
// MFMAs of one block for a wave's TM x TN tiles.  Each tile accumulates its
// six products (planes lo, mid, hi; halves 0, 1) from zero in that order,
// then acc += blk * scale (zero for a block past the slice's end).  The
// tiles of one row of tiles run interleaved -- product j of every tile
// before product j + 1 of any -- so that consecutive MFMAs do not depend
// on each other; each tile's own order, and so every bit, is unchanged.
template <int TM, int TN>
__device__ __forceinline__ void x3_block(const __bf16 *as, int li, int q, const bf16x8 (&b)[TN][2],
                                         const float (&s)[TN], bool live, floatx4 (&acc)[TM][TN]) {
    constexpr int PLANE = XTile<TM>::PLANE;
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
        bf16x8 a[3][2];
#pragma unroll
        for (int t = 2; t >= 0; --t)
#pragma unroll
            for (int h = 0; h < 2; ++h) a[t][h] = *(const bf16x8 *)(as + t * PLANE + (tm * 16 + li) * XLD + 16 * q + 8 * h);
        floatx4 blk[TN];
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) blk[tn] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 2; t >= 0; --t)
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int tn = 0; tn < TN; ++tn)
                    blk[tn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[t][h], b[tn][h], blk[tn], 0, 0, 0);
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
            const float sc_u = live ? s[tn] : 0.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[tm][tn][r] = __builtin_fmaf(blk[tn][r], sc_u, acc[tm][tn][r]);
        }
    }
}

// NW waves per workgroup share one staged activation block, so each wave
// splits BM * 64 / (64 * NW) of its floats per block.
template <int FMT, int TM, int TN, int KU, int NW = 4>
__global__ __launch_bounds__(64 * NW, 2) void gemm_x3_kernel(const GemmArgs G, float *__restrict__ partial,
                                                                       int32_t *__restrict__ wflags, const int kper) {
    constexpr int NT = 64 * NW;
    constexpr int BM = XTile<TM, NT>::BM, NV = XTile<TM, NT>::NV, PLANE = XTile<TM, NT>::PLANE, XBN = 16 * TN * NW;
    constexpr int FPT = XTile<TM, NT>::FPT, TPR = XTile<TM, NT>::TPR;
    constexpr int64_t BB = FMT == SRQ_Q8 ? kBlock : kBlock / 2;  // weight bytes per row and block
    typedef typename XRaw<FMT>::type R;
    __shared__ __attribute__((aligned(16))) __bf16 As[2][3 * PLANE];
    __shared__ int row_wide[BM];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, q = lane >> 4;
    const int64_t n0 = (int64_t)blockIdx.x * XBN + wave * 16 * TN, m0 = (int64_t)blockIdx.y * BM;
    const int64_t cols = G.cols, groups = cols / kBlock;
    const int gbeg = (int)blockIdx.z * kper;
    const int gend = min(gbeg + kper, (int)groups), glast = gend - 1;
    if (tid < BM) row_wide[tid] = 0;

    const uint8_t *wp[TN];
    const float *sp[TN];
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
        const int64_t row = n0 + tn * 16 + li;
        const int64_t rc = row < G.rows ? row : G.rows - 1;
        wp[tn] = (const uint8_t *)G.values + rc * (BB * groups) + (BB / 4) * q;
        sp[tn] = G.scales + rc * groups;
    }
    const int64_t am = min(m0 + tid / TPR, (int64_t)G.n - 1);
    const float *ap = G.x + am * cols + (tid % TPR) * FPT;

    floatx4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    // JIT (Q8, whose 16-byte code slices leave fewer registers): a block's
    // codes are converted just before its MFMAs, from weight loads issued
    // two blocks ahead; otherwise one block ahead, from loads issued three
    // blocks ahead.
    constexpr bool JIT = FMT == SRQ_Q8;
    constexpr int NB = JIT ? 1 : 2;
    R raw[2][TN];
    float sc[2][TN], s[NB][TN];
    float4 areg[2][NV];
    bf16x8 b[NB][TN][2];
// Loaded values are left untouched until the block is converted: an
// operation on them here would make the wave wait for the load at once.
// A clamped (out-of-range) feature row computes on row rows-1's data and is
// never stored.
#define SRQ_LOAD_B(g, slot)                                                         \
    _Pragma("unroll") for (int tn = 0; tn < TN; ++tn) {                              \
        raw[slot][tn] = *(const R *)(wp[tn] + (int64_t)(g) * BB);                    \
        sc[slot][tn] = sp[tn][(g)];                                                  \
    }
#define SRQ_LOAD_A(g, slot) \
    _Pragma("unroll") for (int i = 0; i < NV; ++i) areg[slot][i] = *(const float4 *)(ap + (int64_t)(g) * kBlock + 4 * i);
#define SRQ_CONVERT(slot, dst)                                                      \
    _Pragma("unroll") for (int tn = 0; tn < TN; ++tn) {                              \
        xcodes<FMT>(raw[slot][tn], b[dst][tn][0], b[dst][tn][1]);                    \
        s[dst][tn] = FMT == SRQ_Q4 ? 16.0f * sc[slot][tn] : sc[slot][tn];           \
    }

    SRQ_LOAD_B(gbeg, 0);
    SRQ_LOAD_A(gbeg, 0);
    SRQ_LOAD_B(min(gbeg + 1, glast), 1);
    SRQ_LOAD_A(min(gbeg + 1, glast), 1);
    if constexpr (!JIT) {
        SRQ_CONVERT(0, 0);
        SRQ_LOAD_B(min(gbeg + 2, glast), 0);
    }
    float amax = xstore_a<TM, NT>(As[0], tid, areg[0]);
    SRQ_LOAD_A(min(gbeg + 2, glast), 0);
    lds_barrier();

    if constexpr (KU > 0) {
        // One block: its MFMAs on the staged stage u, its codes converted (JIT:
        // its own; otherwise block g+1's), block g+1's activations split into the
        // other stage, and the refills of the slots so freed.  Block g runs on
        // the clamped data of the slice's last block with a zero scale (adding
        // exactly zero) when `live` is false.  Each slot's refill is kept
        // after its last use (sched_barrier), so that a refill never overlaps
        // the value it replaces.
        auto block = [&](const int g, const int u, const bool live) {
            const int v = u ^ 1;
            const int bu = JIT ? 0 : u;  // operand slot of block g
            if constexpr (JIT) {
                // block g: codes -> operands, then refill with block g+2
                SRQ_CONVERT(u, 0);
                __builtin_amdgcn_sched_barrier(0);
                SRQ_LOAD_B(min(g + 2, glast), u);
            } else {
                // block g+1: codes -> operands, then refill with block g+3
                SRQ_CONVERT(v, v);
                __builtin_amdgcn_sched_barrier(0);
                SRQ_LOAD_B(min(g + 3, glast), v);
            }
            x3_block<TM, TN>(As[u], li, q, b[bu], s[bu], live, acc);
            // block g+1's activations -> the other stage, then refill with block g+3
            amax = fmaxf(amax, xstore_a<TM, NT>(As[v], tid, areg[v]));
            __builtin_amdgcn_sched_barrier(0);
            SRQ_LOAD_A(min(g + 3, glast), v);
            lds_barrier();
        };
        // Slices of KU blocks (kper == KU), unrolled whole: straight-line
        // code, so no value is carried around a back edge.  (A loop carries
        // the ring slots in registers, and the copies the compiler makes of
        // them at the latch wait for the loads just issued; so does a branch
        // around a block.)  A shorter last slice runs its missing blocks with
        // a zero scale.
#pragma unroll
        for (int k = 0; k < KU; ++k) block(gbeg + k, k & 1, gbeg + k < gend);
    } else {
        // Blocks in pairs (the stage index is then a constant).  The second block
        // of a pair past the slice's end still runs, on the clamped block's data
        // with a zero scale (adding exactly zero), so that both halves of every
        // pair wait on the same loads and the loop has no early exit: an exit
        // after the first half makes the compiler drain every load in flight at
        // the end of each pair.
        for (int g0 = gbeg; g0 < gend; g0 += 2) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int g = g0 + u;
                const bool live = g < gend;
                const int v = u ^ 1;
                const int bu = JIT ? 0 : u;  // operand slot of block g
                if constexpr (JIT) {
                    // block g: codes -> operands, then refill with block g+2
                    SRQ_CONVERT(u, 0);
                    SRQ_LOAD_B(min(g + 2, glast), u);
                } else {
                    // block g+1: codes -> operands, then refill with block g+3
                    SRQ_CONVERT(v, v);
                    SRQ_LOAD_B(min(g + 3, glast), v);
                }
                x3_block<TM, TN>(As[u], li, q, b[bu], s[bu], live, acc);
                // block g+1's activations -> the other stage, then refill with block g+3
                amax = fmaxf(amax, xstore_a<TM, NT>(As[v], tid, areg[v]));
                SRQ_LOAD_A(min(g + 3, glast), v);
                lds_barrier();
            }
        }
    }
#undef SRQ_LOAD_B
#undef SRQ_LOAD_A
#undef SRQ_CONVERT
    x3_finish<TM, TN, XBN, NT>(G, partial, wflags, acc, amax, row_wide, n0, m0, tid);
}

// Q8 operands read as whole 128-byte row segments (steps of 9-32 rows).
//
// gemm_x3_kernel loads each lane's MFMA operand straight from memory: one
// wave instruction reads 16 bytes for each of 16 feature rows x 4 K
// quarters, i.e. one 64-byte block of 16 rows, half of each of 16 cache
// lines.  Streamed alone, that pattern moves 16384 x 3072 int8 in 15.0 us
// against 9.3 us for an instruction reading 4 rows x 256 bytes (loads-only
// kernel, 256 workgroups of 8 waves, 8 loads in flight per lane): the
// memory path is bound by cache lines per instruction, not bytes.  Here a
// wave reads a pair of blocks (two 64-input blocks, 128 bytes of a row) of
// its 16 feature rows as two instructions of 8 rows x 128 bytes, stages
// them in its own LDS region and reads each block back in the operand
// layout.  A slice starting or ending on an odd block loads that block
// alone, the old way.  Operands, MFMA order and the scale chain are those
// of gemm_x3_kernel, so every output has the same bits.
//
// Region layout per 16-row tile: row r (0..15) holds its eight 16-byte
// chunks at slots chunk ^ (r % 8) ^ (r / 8), so that both the stores (8
// lanes per row) and the operand reads (16 rows per K quarter) touch
// distinct banks.
template <int KU, int ODD>
struct PairRole {
    // Block k of a slice of KU blocks whose first block has the parity ODD:
    // first(k) loads blocks k and k + 1, single(k) loads block k alone.
    static constexpr bool first(int k) { return (k + ODD) % 2 == 0 && k + 1 < KU; }
    static constexpr bool single(int k) { return (k + ODD) % 2 == 0 ? k + 1 == KU : k == 0; }
};

// f(integral_constant<int, i>) for i = 0, 1, ... in order, as straight-line code.
template <typename F, int... I>
__device__ __forceinline__ void unroll_each(F &&f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}

template <int TM, int TN, int NW, int KU, int DIST, int ODD>
__device__ __forceinline__ void x3p_slice(const GemmArgs &G, const int64_t n0, const int64_t m0, const int gbeg,
                                          const int gend, const int tid, __bf16 (*As)[3 * XTile<TM>::PLANE],
                                          u32x4v *ws, float *ss, floatx4 (&acc)[TM][TN], float &amax) {
    typedef PairRole<KU, ODD> Role;
    typedef XTile<TM, 64 * NW> X;
    constexpr int NV = X::NV, PLANE = X::PLANE, FPT = X::FPT, TPR = X::TPR;
    // Activations run one block further ahead than weights and each
    // block issues them first.  The wave's load counter retires in issue
    // order, so a wait for block k+1's activations then never waits for
    // weights of a block beyond k, and the weight loads keep DIST blocks in
    // flight.
    constexpr int DA = DIST + 1;
    const int lane = tid & 63, li = lane & 15, q = lane >> 4;
    const int64_t cols = G.cols, groups = cols / kBlock;
    const int glast = gend - 1;
    // 32-bit offsets from the matrix base (rows * cols < 2^32): one
    // register per address instead of two
    const uint8_t *__restrict__ W = (const uint8_t *)G.values;
    uint32_t wo[TN], po[TN][2];
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
        const int64_t row = n0 + tn * 16 + li;
        const int64_t rc = row < G.rows ? row : G.rows - 1;
        wo[tn] = (uint32_t)(rc * cols + 16 * q);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int64_t prow = n0 + tn * 16 + 8 * i + (lane >> 3);
            const int64_t prc = prow < G.rows ? prow : G.rows - 1;
            po[tn][i] = (uint32_t)(prc * cols + 16 * (lane & 7));
        }
    }
    // region slots: stores of row 8i + lane/8, chunk lane%8; operand reads of row li
    const int wslot[2] = {(lane >> 3) * 8 + ((lane & 7) ^ (lane >> 3)), 64 + (lane >> 3) * 8 + ((lane & 7) ^ (lane >> 3) ^ 1)};
    const int rsw = (li & 7) ^ (li >> 3);
    const int64_t am = min(m0 + tid / TPR, (int64_t)G.n - 1);
    const float *ap = G.x + am * cols + (tid % TPR) * FPT;

    u32x4v praw[KU][TN][2], sraw[KU][TN];
    float4 areg[DA][NV];
    // The slice's scales of the workgroup's rows, loaded once in row order
    // (KU consecutive floats per row, the lanes of an instruction spanning
    // a few rows) into ss[row][block] (row stride KS, odd: the 16 rows of
    // an operand read hit distinct banks).  Per-block scale loads of 16
    // rows each would cost as many cache-line requests as the weights.
    constexpr int NT = 64 * NW, XBN = 16 * TN * NW, KS = KU | 1, SE = (XBN * KU + NT - 1) / NT;
    const int64_t wrow0 = n0 - (tid >> 6) * 16 * TN;  // the workgroup's first output
    float sreg[SE];
#pragma unroll
    for (int i = 0; i < SE; ++i) {
        const int e = tid + NT * i;
        const int r = e / KU, j = e - r * KU;
        const int64_t row = min(wrow0 + r, G.rows - 1);
        // a block past the slice's end (last slice) is added with a zero scale
        sreg[i] = e < XBN * KU && gbeg + j < gend ? G.scales[row * groups + min(gbeg + j, glast)] : 0.0f;
    }
    auto stage_s = [&]() {
#pragma unroll
        for (int i = 0; i < SE; ++i) {
            const int e = tid + NT * i;
            const int r = e / KU, j = e - r * KU;
            if (e < XBN * KU) ss[r * KS + j] = sreg[i];
        }
    };
    const float *sl = ss + ((tid >> 6) * 16 * TN + li) * KS;  // this lane's rows
    // Weight loads of block j (its scale, and its pair or its lone block).
    // A phantom block past the slice's end (last slice) reads clamped,
    // in-row data and is added with a zero scale.
    auto load_w = [&](auto J) {
        constexpr int j = decltype(J)::value;
        if constexpr (j < KU) {
            const int g = gbeg + j;
            if constexpr (Role::first(j)) {
                const uint32_t pg = (uint32_t)min((int64_t)g, groups - 2) * kBlock;
#pragma unroll
                for (int tn = 0; tn < TN; ++tn)
#pragma unroll
                    for (int i = 0; i < 2; ++i) praw[j][tn][i] = *(const u32x4v *)(W + (uint64_t)(po[tn][i] + pg));
            } else if constexpr (Role::single(j)) {
                const uint32_t sg = (uint32_t)min(g, glast) * kBlock;
#pragma unroll
                for (int tn = 0; tn < TN; ++tn) sraw[j][tn] = *(const u32x4v *)(W + (uint64_t)(wo[tn] + sg));
            }
        }
    };
    auto load_a = [&](auto J) {
        constexpr int j = decltype(J)::value;
        if constexpr (j < KU) {
            const int64_t g = min(gbeg + j, glast);
#pragma unroll
            for (int i = 0; i < NV; ++i) areg[j % DA][i] = *(const float4 *)(ap + g * kBlock + 4 * i);
        }
    };
    auto stage_w = [&](auto J) {
        constexpr int j = decltype(J)::value;
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
#pragma unroll
            for (int i = 0; i < 2; ++i) ws[tn * 128 + wslot[i]] = praw[j][tn][i];
    };

    // issue order A0, A1, W0, A2, W1, ..., A(DA-1), W(DIST-1): each
    // block's weights after the activations one block further on
    load_a(std::integral_constant<int, 0>{});
    unroll_each([&](auto J) {
        constexpr int j = decltype(J)::value;
        load_a(std::integral_constant<int, j + 1>{});
        load_w(J);
    }, std::make_integer_sequence<int, DIST>{});
    stage_s();
    if constexpr (Role::first(0)) stage_w(std::integral_constant<int, 0>{});
    amax = xstore_a<TM, NT>(As[0], tid, areg[0]);
    lds_barrier();

    unroll_each([&](auto K) {
        constexpr int k = decltype(K)::value;
        constexpr int u = k & 1, v = u ^ 1;
        bf16x8 b[TN][2];
        if constexpr (Role::single(k)) {
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) xcodes<SRQ_Q8>(sraw[k][tn], b[tn][0], b[tn][1]);
        } else {
            constexpr int half = Role::first(k) ? 0 : 1;
#pragma unroll
            for (int tn = 0; tn < TN; ++tn)
                xcodes<SRQ_Q8>(ws[tn * 128 + li * 8 + ((4 * half + q) ^ rsw)], b[tn][0], b[tn][1]);
        }
        __builtin_amdgcn_sched_barrier(0);
        load_a(std::integral_constant<int, k + DA>{});
        load_w(std::integral_constant<int, k + DIST>{});
        __builtin_amdgcn_sched_barrier(0);
        const __bf16 *as = As[u];
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) {
            bf16x8 a[3][2];
#pragma unroll
            for (int t = 0; t < 3; ++t)
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    a[t][h] = *(const bf16x8 *)(as + t * PLANE + (tm * 16 + li) * XLD + 16 * q + 8 * h);
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) {
                floatx4 blk = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int t = 2; t >= 0; --t)
#pragma unroll
                    for (int h = 0; h < 2; ++h)
                        blk = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[t][h], b[tn][h], blk, 0, 0, 0);
                const float sc_u = sl[tn * 16 * KS + k];
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[tm][tn][r] = __builtin_fmaf(blk[r], sc_u, acc[tm][tn][r]);
            }
        }
        if constexpr (k + 1 < KU) {
            // the next pair -> the region (after this block's reads of it),
            // block k+1's activations -> the other stage
            if constexpr (Role::first(k + 1)) stage_w(std::integral_constant<int, k + 1>{});
            amax = fmaxf(amax, xstore_a<TM, NT>(As[v], tid, areg[(k + 1) % DA]));
            lds_barrier();
        }
    }, std::make_integer_sequence<int, KU>{});
}

// Q8, 16- or 32-row tiles, cols % 128 == 0, rows * cols < 2^32, slices of exactly KU blocks
// (the last slice may be shorter).  DIST: blocks between a block's loads
// and its use.
// Q8, 16- or 32-row tiles, cols % 128 == 0, rows * cols < 2^32, slices of
// exactly KU blocks (the last slice may be shorter).  NW waves of TN
// feature tiles each; DIST: blocks between a block's loads and its use.
// Eight waves keep two per SIMD in the one workgroup a CU holds, so that
// one wave's MFMAs overlap another's conversions and LDS waits, while the
// activation stage stays shared by all the workgroup's features.  Up to
// eight tiles per workgroup, two workgroups fit a CU.
template <int TM, int TN, int NW, int KU, int DIST>
__global__ __launch_bounds__(64 * NW, TN * NW <= 8 ? 2 : 1) void gemm_x3p_kernel(
    const GemmArgs G, float *__restrict__ partial, int32_t *__restrict__ wflags, const int kper) {
    constexpr int BM = XTile<TM>::BM, PLANE = XTile<TM>::PLANE, XBN = 16 * TN * NW;
    __shared__ __attribute__((aligned(16))) __bf16 As[2][3 * PLANE];
    __shared__ u32x4v Ws[NW][TN * 128];
    __shared__ float Ss[XBN * (KU | 1)];
    __shared__ int row_wide[BM];
    const int tid = threadIdx.x, wave = tid >> 6;
    const int64_t n0 = (int64_t)blockIdx.x * XBN + wave * 16 * TN, m0 = (int64_t)blockIdx.y * BM;
    const int groups = (int)(G.cols / kBlock);
    const int gbeg = (int)blockIdx.z * kper;
    const int gend = min(gbeg + kper, groups);
    if (tid < BM) row_wide[tid] = 0;
    floatx4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
    float amax = 0.0f;
    if (gbeg & 1)
        x3p_slice<TM, TN, NW, KU, DIST, 1>(G, n0, m0, gbeg, gend, tid, As, Ws[wave], Ss, acc, amax);
    else
        x3p_slice<TM, TN, NW, KU, DIST, 0>(G, n0, m0, gbeg, gend, tid, As, Ws[wave], Ss, acc, amax);
    x3_finish<TM, TN, XBN, 64 * NW>(G, partial, wflags, acc, amax, row_wide, n0, m0, tid);
}

// The same for four consecutive outputs (rows, y_stride and the plane are
// multiples of 4): float4 loads, the sum still taken in slice order.
__global__ __launch_bounds__(256) void gemm_reduce4_kernel(const GemmArgs G, const float *__restrict__ partial,
                                                           const int32_t *__restrict__ wflags, const int slices) {
    const int64_t m = blockIdx.y, j = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    const int wide = any_wide(wflags, G.n, m, slices);
    if (j >= G.rows) return;
    float4 v;
    if (wide) {
        v = make_float4(wide_output(G, m, j), wide_output(G, m, j + 1), wide_output(G, m, j + 2),
                        wide_output(G, m, j + 3));
    } else {
        const floatx4 acc = slice_sum<floatx4>(partial + m * G.rows + j, (int64_t)G.n * G.rows, slices);
        v = make_float4(acc.x, acc.y, acc.z, acc.w);
        if (G.residual) {
            const float4 r = *(const float4 *)(G.residual + m * G.y_stride + j);
            v = make_float4(r.x + acc.x, r.y + acc.y, r.z + acc.z, r.w + acc.w);
        }
    }
    *(float4 *)(G.y + m * G.y_stride + j) = v;
}

__device__ __forceinline__ float4 slice_sum4(const float *__restrict__ p, int64_t plane, int slices) {
    const floatx4 a = slice_sum<floatx4>(p, plane, slices);
    return make_float4(a.x, a.y, a.z, a.w);
}

__device__ __forceinline__ float silu_mul(float g, float up) {
    const double gd = (double)g;
    return __fmul_rn((float)(gd / (1.0 + exp(-gd))), up);
}

// Split-K reduction fused with SwiGLU: W's rows are [gate; up] (hidden = rows
// / 2); thread -> row m, gate/up columns u..u+3.  Each column is the
// in-order slice sum (or the FP64 result for wide rows), then
// h = f32(g/(1+exp(-g))) * up as swiglu_kernel computes it.
__global__ __launch_bounds__(256) void gemm_reduce_swiglu4_kernel(const GemmArgs G, const float *__restrict__ partial,
                                                                  const int32_t *__restrict__ wflags,
                                                                  const int slices) {
    const int64_t hidden = G.rows / 2;
    const int64_t m = blockIdx.y, u = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    const int wide = any_wide(wflags, G.n, m, slices);
    if (u >= hidden) return;
    float4 g, up;
    if (wide) {
        g = make_float4(wide_output(G, m, u), wide_output(G, m, u + 1), wide_output(G, m, u + 2),
                        wide_output(G, m, u + 3));
        up = make_float4(wide_output(G, m, hidden + u), wide_output(G, m, hidden + u + 1),
                         wide_output(G, m, hidden + u + 2), wide_output(G, m, hidden + u + 3));
    } else {
        const int64_t plane = (int64_t)G.n * G.rows;
        g = slice_sum4(partial + m * G.rows + u, plane, slices);
        up = slice_sum4(partial + m * G.rows + hidden + u, plane, slices);
    }
    const float4 h = make_float4(silu_mul(g.x, up.x), silu_mul(g.y, up.y), silu_mul(g.z, up.z), silu_mul(g.w, up.w));
    *(float4 *)(G.swiglu_out + m * hidden + u) = h;
}

constexpr int kNormThreads = 1024;
constexpr int kNormVec = 2;  // float4 columns per thread of the norm reduction: rows <= 8192

// Split-K reduction fused with the next RMSNorm: one workgroup per
// activation row m.  y[m] is the in-order slice sum plus the residual (or
// the FP64 result for wide rows), as gemm_reduce4_kernel writes it; then
// norm_out[m] = (y*a)*w with a = f32(1/sqrt(Sum f64(y^2)/d + eps)) (rmsInto,
// M:6182-6194) from the values still in registers.
__global__ __launch_bounds__(kNormThreads) void gemm_reduce_norm4_kernel(const GemmArgs G,
                                                                         const float *__restrict__ partial,
                                                                         const int32_t *__restrict__ wflags,
                                                                         const int slices) {
    __shared__ double red[kNormThreads / 64];
    const int64_t m = blockIdx.x;
    const int tid = threadIdx.x;
    const int wide = any_wide(wflags, G.n, m, slices);
    const int64_t plane = (int64_t)G.n * G.rows;
    float4 v[kNormVec];
    double ss = 0.0;
#pragma unroll
    for (int k = 0; k < kNormVec; ++k) {
        const int64_t j = ((int64_t)k * kNormThreads + tid) * 4;
        if (j >= G.rows) break;
        float4 t;
        if (wide) {
            t = make_float4(wide_output(G, m, j), wide_output(G, m, j + 1), wide_output(G, m, j + 2),
                            wide_output(G, m, j + 3));
        } else {
            t = slice_sum4(partial + m * G.rows + j, plane, slices);
            if (G.residual) {
                const float4 r = *(const float4 *)(G.residual + m * G.y_stride + j);
                t = make_float4(r.x + t.x, r.y + t.y, r.z + t.z, r.w + t.w);
            }
        }
        *(float4 *)(G.y + m * G.y_stride + j) = t;
        v[k] = t;
        ss += (double)t.x * (double)t.x + (double)t.y * (double)t.y + (double)t.z * (double)t.z +
              (double)t.w * (double)t.w;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    double tot = 0.0;
    for (int w = 0; w < kNormThreads / 64; ++w) tot += red[w];
    const float a = (float)(1.0 / sqrt(tot / (double)G.rows + G.norm_eps));
#pragma unroll
    for (int k = 0; k < kNormVec; ++k) {
        const int64_t j = ((int64_t)k * kNormThreads + tid) * 4;
        if (j >= G.rows) break;
        const float4 w = *(const float4 *)(G.norm_w + j);
        const float4 t = v[k];
        *(float4 *)(G.norm_out + m * G.rows + j) =
            make_float4(__fmul_rn(__fmul_rn(t.x, a), w.x), __fmul_rn(__fmul_rn(t.y, a), w.y),
                        __fmul_rn(__fmul_rn(t.z, a), w.z), __fmul_rn(__fmul_rn(t.w, a), w.w));
    }
}

// Split-K reduction fused with RoPE and the KV write (the arithmetic of
// rope_kv_kernel): thread t of row m takes RoPE pair t (j, j + head_dim/2) of
// a q or k head, or past the pairs one v element.
__global__ __launch_bounds__(256) void gemm_reduce_rope_kernel(const GemmArgs G, const float *__restrict__ partial,
                                                               const int32_t *__restrict__ wflags, const int slices) {
    const GemmRope &R = G.rope;
    const int64_t m = blockIdx.y;
    const int dim = R.dim, kvdim = R.kvdim, half = R.head_dim / 2, pairs = (dim + kvdim) / 2;
    const int t = blockIdx.x * 256 + threadIdx.x;
    const int wide = any_wide(wflags, G.n, m, slices);
    if (t >= pairs + kvdim) return;
    const int64_t plane = (int64_t)G.n * G.rows;
    auto column = [&](int64_t j) {
        return wide ? wide_output(G, m, j) : slice_sum<float>(partial + m * G.rows + j, plane, slices);
    };
    const RowMeta &meta = R.meta;
    const int pos = meta.pos[m];
    const int page = meta.pages[(int64_t)meta.sess[m] * meta.pt_stride + pos / kPageTokens];
    float *kr = meta.kv_pool + (int64_t)page * meta.page_elems + (int64_t)meta.layer * 2 * kPageTokens * kvdim +
                (int64_t)(pos % kPageTokens) * kvdim;
    if (t < pairs) {
        const int h = t / half, j = t - h * half;
        const int i0 = h * R.head_dim + j, i1 = i0 + half;
        float a = column(i0), z = column(i1);
        if (R.bias) {
            a = __fadd_rn(a, R.bias[i0]);
            z = __fadd_rn(z, R.bias[i1]);
        }
        const float c = R.cos_t[(int64_t)pos * half + j], s = R.sin_t[(int64_t)pos * half + j];
        // x' = a*c - z*s ; z' = a*s + z*c  (M:5283-5285), unfused
        const float na = __fsub_rn(__fmul_rn(a, c), __fmul_rn(z, s));
        const float nz = __fadd_rn(__fmul_rn(a, s), __fmul_rn(z, c));
        if (i0 < dim) {
            R.q[m * dim + i0] = na;
            R.q[m * dim + i1] = nz;
        } else {
            kr[i0 - dim] = na;
            kr[i1 - dim] = nz;
        }
    } else {
        const int j = t - pairs;
        float v = column(dim + kvdim + j);
        if (R.bias) v = __fadd_rn(v, R.bias[dim + kvdim + j]);
        kr[(int64_t)kPageTokens * kvdim + j] = v;
    }
}

struct GemmPlan {
    bool x3;  // bf16 MFMA kernel (Q8 / Q4, cols % 64 == 0)
    int bm, tn, slices, kper;  // tn: 16-feature tiles per wave of the bf16 kernel
};

// Tile height and width from n; K slices from the matrix shape alone.
//
// A row's result is fixed by the K slices (each slice's chain of block
// sums, then the slices added in order); the tile height and width only
// decide which workgroup computes it.  The slice count therefore depends on
// (rows, cols) and never on n, so a row's bits are the same whatever other
// rows share the call (batch invariance, q8_test.go:88-92).  It is the count
// that fills the chip for one 32-row tile of outputs: with fewer feature
// tiles than CUs, slices of at least 256 inputs bring the grid to at most
// one workgroup per CU (each slice's partial sums cost as much traffic as a
// share of the weights, which outweighs a second resident workgroup).  The
// count rounds down: rounding up left a few CUs with two workgroups that
// finished last (3072 x 8192 at 32 rows: 24 x 11 = 264 workgroups, the
// slowest waves 4.6 us behind the median), and rounding down also halves
// some large-n partial traffic (Llama-3.2-3B continuous batching 1363 ->
// 1402 tokens/s, Mistral-7B q4-mixed prefill 15.30k -> 16.43k, 8.2k-token
// Q8 prefill 12.45k -> 12.74k).  Larger n adds row tiles to the same
// slices.
GemmPlan plan_gemm(int fmt, int32_t n, int64_t rows, int64_t cols) {
    GemmPlan p;
    p.x3 = (fmt == SRQ_Q8 || fmt == SRQ_Q4) && cols % kBlock == 0;
    // 16-row tiles (bf16 kernel) for at most 16 rows: the 32-row plan's
    // slices with half the MFMA, activation-split and scale work per block,
    // and features in tiles of half the width, so twice the workgroups
    // (Llama-3.2-3B continuous batching 1152 -> 1176 tokens/s with the
    // 32-row plan's feature tiles, 1186 with half-width ones).
    p.bm = p.x3 && n <= 16 ? 16 : n <= 32 ? 32 : 64;
    // 128-feature tiles for 32-row tiles of narrow outputs: twice the
    // tiles, so fewer K slices and half the partial-sum traffic per weight
    // byte (Llama-3.2-3B shapes at 24-32 rows: 3072 x 3072 17.2 -> 13.5 us,
    // 3072 x 8192 24.9 -> 23.3 us, 5120 x 3072 20.0 -> 18.9 us; at 16384
    // rows the 256-feature tile stays ahead, 30.4 against 33.5 us).
    p.tn = p.bm == 16 ? (rows <= 8192 ? 1 : 2) : p.bm == 32 && rows <= 8192 ? 2 : 4;  // 16-feature tiles per wave
    const int bk = p.x3 ? kBlock : BK;
    const int bn32 = p.x3 ? 64 * (rows <= 8192 ? 2 : 4) : BN;  // feature tile of a 32-row plan
    const int64_t tiles = (rows + bn32 - 1) / bn32;
    const int ksteps = (int)(cols / bk), min_steps = kMinSliceInputs / bk;
    int slices = 1;
    if (tiles < kCUs)
        slices = (int)std::max<int64_t>(1, std::min<int64_t>(kCUs / tiles, ksteps / min_steps));
    p.kper = (ksteps + slices - 1) / slices;
    p.slices = (ksteps + p.kper - 1) / p.kper;
    return p;
}

template <int TM, int TN, int KU = 4>
void launch_unrolled(hipStream_t s, dim3 grid, const GemmArgs &a, float *partial, int32_t *wflags, int kper) {
    if constexpr (KU <= 16) {
        if (kper == KU)
            gemm_x3_kernel<SRQ_Q8, TM, TN, KU><<<grid, 256, 0, s>>>(a, partial, wflags, kper);
        else
            launch_unrolled<TM, TN, KU + 1>(s, grid, a, partial, wflags, kper);
    }
}

// The same for any format and NW waves (the Q4 64-row tiles).
template <int FMT, int TM, int TN, int NW, int KU = 4>
void launch_unrolled_nw(hipStream_t s, dim3 grid, const GemmArgs &a, float *partial, int32_t *wflags, int kper) {
    if constexpr (KU <= 16) {
        if (kper == KU)
            gemm_x3_kernel<FMT, TM, TN, KU, NW><<<grid, 64 * NW, 0, s>>>(a, partial, wflags, kper);
        else
            launch_unrolled_nw<FMT, TM, TN, NW, KU + 1>(s, grid, a, partial, wflags, kper);
    }
}

// Pair-streamed Q8 tiles (gemm_x3p_kernel): blocks between a block's
// weight loads and its MFMAs.
template <int TN>
constexpr int kPairDist = 4;

template <int TM, int TN, int NW, int KU = 4>
void launch_pairs(hipStream_t s, dim3 grid, const GemmArgs &a, float *partial, int32_t *wflags, int kper) {
    if constexpr (KU <= 16) {
        if (kper == KU)
            gemm_x3p_kernel<TM, TN, NW, KU, kPairDist<TN>><<<grid, 64 * NW, 0, s>>>(a, partial, wflags, kper);
        else
            launch_pairs<TM, TN, NW, KU + 1>(s, grid, a, partial, wflags, kper);
    }
}

template <int FMT, int BMT>
void launch_tiles(hipStream_t s, const GemmArgs &a, const GemmPlan &p, float *partial, int32_t *wflags) {
    static_assert(BMT >= 32 || FMT != SRQ_F32, "16-row tiles are the bf16 kernel's");
    if constexpr (FMT == SRQ_F32) {
        dim3 grid((unsigned)((a.rows + BN - 1) / BN), (unsigned)((a.n + BMT - 1) / BMT), (unsigned)p.slices);
        gemm_kernel<FMT, BMT><<<grid, 256, 0, s>>>(a, partial, wflags, p.kper);
    } else {
        if (p.x3) {
            const int xbn = 64 * p.tn;
            dim3 grid((unsigned)((a.rows + xbn - 1) / xbn), (unsigned)((a.n + BMT - 1) / BMT), (unsigned)p.slices);
            // Q8 slices of 4..16 blocks run unrolled; at 16 and 32 rows with
            // whole 128-byte row segments (cols % 128 == 0), pair-streamed
            if constexpr (BMT <= 32) {
                if (FMT == SRQ_Q8 && p.kper >= 4 && p.kper <= 16 && a.cols % (2 * kBlock) == 0 &&
                    (uint64_t)a.rows * (uint64_t)a.cols <= UINT32_MAX) {
                    // the plan's feature tile (64 * tn); 256 features over 8 waves
                    // (gate/up 16384x3072 at 17-32 rows: 24.5 -> 22.6 us; 128
                    // features over 8 waves were slower)
                    if constexpr (BMT == 32) {
                        if (p.tn == 2)
                            launch_pairs<2, 2, 4>(s, grid, a, partial, wflags, p.kper);
                        else
                            launch_pairs<2, 2, 8>(s, grid, a, partial, wflags, p.kper);
                    } else if (p.tn == 1) {
                        launch_pairs<1, 1, 4>(s, grid, a, partial, wflags, p.kper);
                    } else {
                        launch_pairs<1, 2, 4>(s, grid, a, partial, wflags, p.kper);  // 16-row plans: tn <= 2
                    }
                    return;
                }
            }
            if constexpr (BMT == 16) {
                if (p.tn == 1) {
                    if (FMT == SRQ_Q8 && p.kper >= 4 && p.kper <= 16)
                        launch_unrolled<1, 1>(s, grid, a, partial, wflags, p.kper);
                    else
                        gemm_x3_kernel<FMT, 1, 1, 0><<<grid, 256, 0, s>>>(a, partial, wflags, p.kper);
                    return;
                }
            }
            if constexpr (BMT == 64 && FMT == SRQ_Q4) {
                // Q4 64-row tiles: 8 waves of 4 feature tiles (512 features)
                // share each staged activation block, which halves every
                // wave's share of the split (Mistral-7B q4-mixed prefill
                // 14.78k -> 15.23k tokens/s; its GEMM 101.8 -> 96.9 us a call).
                // Each tile's arithmetic is unchanged.  Q8, which converts its
                // codes just before their MFMAs, ran slower so (8.2k-token
                // prefill 12.15k -> 11.99k, continuous batching 1355 -> 1336).
                // Slices of 4..16 blocks run unrolled (prefill 16.49k ->
                // 16.60k tokens/s).
                if (p.tn == 4) {
                    const dim3 g8((unsigned)((a.rows + 511) / 512), grid.y, grid.z);
                    if (p.kper >= 4 && p.kper <= 16)
                        launch_unrolled_nw<FMT, 4, 4, 8>(s, g8, a, partial, wflags, p.kper);
                    else
                        gemm_x3_kernel<FMT, 4, 4, 0, 8><<<g8, 512, 0, s>>>(a, partial, wflags, p.kper);
                    return;
                }
            }
            if (FMT == SRQ_Q8 && p.kper >= 4 && p.kper <= 16) {
                if (p.tn == 2)
                    launch_unrolled<BMT / 16, 2>(s, grid, a, partial, wflags, p.kper);
                else
                    launch_unrolled<BMT / 16, 4>(s, grid, a, partial, wflags, p.kper);
            } else if (p.tn == 2) {
                gemm_x3_kernel<FMT, BMT / 16, 2, 0><<<grid, 256, 0, s>>>(a, partial, wflags, p.kper);
            } else {
                gemm_x3_kernel<FMT, BMT / 16, 4, 0><<<grid, 256, 0, s>>>(a, partial, wflags, p.kper);
            }
        } else {
            if constexpr (BMT >= 32) {
                dim3 grid((unsigned)((a.rows + BN - 1) / BN), (unsigned)((a.n + BMT - 1) / BMT), (unsigned)p.slices);
                gemm_kernel<FMT, BMT><<<grid, 256, 0, s>>>(a, partial, wflags, p.kper);
            }
        }
    }
}

template <int BMT>
void launch_fmt(hipStream_t s, const GemmArgs &a, const GemmPlan &p, float *partial, int32_t *wflags) {
    switch (a.fmt) {
        case SRQ_Q8: launch_tiles<SRQ_Q8, BMT>(s, a, p, partial, wflags); break;
        case SRQ_Q4: launch_tiles<SRQ_Q4, BMT>(s, a, p, partial, wflags); break;
        default:
            if constexpr (BMT >= 32) launch_tiles<SRQ_F32, BMT>(s, a, p, partial, wflags);
            break;
    }
}

}  // namespace

bool gemm_ok(int fmt, int64_t cols) {
    (void)fmt;
    return cols % BK == 0 && cols >= BK;
}

size_t gemm_scratch_bytes(int fmt, int32_t n, int64_t rows, int64_t cols) {
    if (n <= 0 || rows <= 0 || !gemm_ok(fmt, cols)) return 0;
    const GemmPlan p = plan_gemm(fmt, n, rows, cols);
    if (p.slices == 1) return 0;
    return (size_t)p.slices * (size_t)n * ((size_t)rows + 1) * 4;
}

int launch_gemm(hipStream_t s, const GemmArgs &a, void *scratch, size_t scratch_bytes) {
    if (a.n <= 0 || a.rows <= 0) return SRQ_OK;
    if (!gemm_ok(a.fmt, a.cols)) return fail(SRQ_EINVAL, "gemm: cols=%lld not a multiple of %d", (long long)a.cols, BK);
    const GemmPlan p = plan_gemm(a.fmt, a.n, a.rows, a.cols);
    float *partial = nullptr;
    int32_t *wflags = nullptr;
    if (p.slices > 1) {
        const size_t need = gemm_scratch_bytes(a.fmt, a.n, a.rows, a.cols);
        if (!scratch || scratch_bytes < need)
            return fail(SRQ_EINVAL, "gemm: scratch of %zu bytes, %zu needed", scratch_bytes, need);
        partial = (float *)scratch;
        wflags = (int32_t *)(partial + (size_t)p.slices * a.n * a.rows);
    }
    if (a.swiglu_out && (a.residual || a.rows % 8 || ((uintptr_t)a.swiglu_out & 15)))
        return fail(SRQ_EINVAL, "gemm: SwiGLU output needs an even row split, 16-byte alignment and no residual");
    if (a.norm_out && (!a.norm_w || a.y_stride != a.rows || a.rows > (int64_t)INT32_MAX))
        return fail(SRQ_EINVAL, "gemm: RMSNorm output needs a norm weight and y_stride == rows");
    if (a.rope.q && (a.residual || a.swiglu_out || a.norm_out || a.rope.head_dim < 2 || a.rope.head_dim % 2 ||
                     a.rope.dim % a.rope.head_dim || a.rope.kvdim % a.rope.head_dim ||
                     a.rows != (int64_t)a.rope.dim + 2 * (int64_t)a.rope.kvdim || a.y_stride != a.rows))
        return fail(SRQ_EINVAL, "gemm: RoPE/KV output needs rows = dim + 2*kvdim in whole heads and no other epilogue");
    if (p.bm == 16)
        launch_fmt<16>(s, a, p, partial, wflags);  // bf16 kernel only (plan_gemm)
    else if (p.bm == 32)
        launch_fmt<32>(s, a, p, partial, wflags);
    else
        launch_fmt<64>(s, a, p, partial, wflags);
    SRQ_HIP(hipGetLastError());
    if (a.rope.q) {
        if (p.slices > 1) {
            const int work = (a.rope.dim + a.rope.kvdim) / 2 + a.rope.kvdim;
            dim3 grid((unsigned)((work + 255) / 256), (unsigned)a.n);
            gemm_reduce_rope_kernel<<<grid, 256, 0, s>>>(a, partial, wflags, p.slices);
            SRQ_HIP(hipGetLastError());
            return SRQ_OK;
        }
        return launch_rope_kv(s, a.y, a.rope.bias, a.n, a.rope.dim, a.rope.kvdim, a.rope.head_dim, a.rope.cos_t,
                              a.rope.sin_t, a.rope.q, a.rope.meta);
    }
    if (a.norm_out) {
        const bool fused = p.slices > 1 && a.rows % 4 == 0 && a.rows <= 4 * kNormThreads * kNormVec &&
                           ((((uintptr_t)a.y) | ((uintptr_t)a.norm_w) | ((uintptr_t)a.norm_out) |
                             (a.residual ? (uintptr_t)a.residual : 0)) & 15) == 0;
        if (fused) {
            gemm_reduce_norm4_kernel<<<(unsigned)a.n, kNormThreads, 0, s>>>(a, partial, wflags, p.slices);
            SRQ_HIP(hipGetLastError());
            return SRQ_OK;
        }
        if (p.slices > 1) {
            dim3 grid((unsigned)((a.rows + 255) / 256), (unsigned)a.n);
            gemm_reduce_kernel<<<grid, 256, 0, s>>>(a, partial, wflags, p.slices);
            SRQ_HIP(hipGetLastError());
        }
        return launch_rmsnorm(s, a.y, a.norm_w, a.norm_out, a.n, (int32_t)a.rows, a.norm_eps);
    }
    if (a.swiglu_out) {
        if (p.slices > 1) {
            dim3 grid((unsigned)((a.rows / 8 + 255) / 256), (unsigned)a.n);
            gemm_reduce_swiglu4_kernel<<<grid, 256, 0, s>>>(a, partial, wflags, p.slices);
            SRQ_HIP(hipGetLastError());
            return SRQ_OK;
        }
        return launch_swiglu(s, a.y, a.n, (int32_t)(a.rows / 2), a.swiglu_out);
    }
    if (p.slices > 1) {
        const bool vec4 = a.rows % 4 == 0 && a.y_stride % 4 == 0 && ((uintptr_t)a.y & 15) == 0 &&
                          (!a.residual || ((uintptr_t)a.residual & 15) == 0);
        if (vec4) {
            dim3 grid((unsigned)((a.rows / 4 + 255) / 256), (unsigned)a.n);
            gemm_reduce4_kernel<<<grid, 256, 0, s>>>(a, partial, wflags, p.slices);
        } else {
            dim3 grid((unsigned)((a.rows + 255) / 256), (unsigned)a.n);
            gemm_reduce_kernel<<<grid, 256, 0, s>>>(a, partial, wflags, p.slices);
        }
        SRQ_HIP(hipGetLastError());
    }
    return SRQ_OK;
}

}  // namespace srq
