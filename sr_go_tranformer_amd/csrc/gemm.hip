// Dequant-GEMM on FP32 MFMA for prefill chunks and batched steps (n > 16).
//
// Counterpart of linearQ8Into / linearQ4Into / linearFP32Range
// (cmd/monolith/monolith.go M:3942-4780) when many activation rows share
// each weight read, which makes the contraction compute bound.
//
// Tiling (gfx950, wave64, v_mfma_f32_16x16x4_f32):
//  - Workgroup tile 64 (activation rows) x 128 (output features), K step 32
//    (half a scale block).  4 waves in a 2x2 grid, each owning 32x64 = 2x4
//    MFMA tiles of 16x16 with FP32 accumulators.
//  - Weights are read once per K step as int8 / packed int4 / f32,
//    dequantised in registers to f32(code)*scale (the copyRow rounding,
//    M:3900-3921) and stored to LDS; activations go to LDS unchanged.
//  - Within a K step, MFMA step s feeds lane group g (lane/16) the K index
//    8g+s, so every lane reads its 8 K values of a row as two ds_read_b128.
//  - Global loads for step k+1 are issued before the MFMAs of step k
//    (register double buffering); LDS is double buffered.
//  - Rows flagged wide (|x| > f32(MaxFloat32/(2*64*127)), M:4346-4354) are
//    skipped here and recomputed in FP64 by wide_fix_kernel.
#include "srq_internal.h"

namespace srq {
namespace {

constexpr int BM = 64, BN = 128, BK = 32, LDK = BK + 4;
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

__device__ __forceinline__ void load_a(const float *__restrict__ X, int32_t n, int64_t cols, int64_t m0, int64_t k0,
                                       int tid, float4 (&a)[2]) {
    const int r = tid >> 2, kq = (tid & 3) * 8;
    const int64_t m = m0 + r;
    if (m < n) {
        const float4 *p = (const float4 *)(X + m * cols + k0 + kq);
        a[0] = p[0];
        a[1] = p[1];
    } else {
        a[0] = a[1] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

__device__ __forceinline__ void store_a(float *As, int tid, const float4 (&a)[2]) {
    const int r = tid >> 2, kq = (tid & 3) * 8;
    *(float4 *)(As + r * LDK + kq) = a[0];
    *(float4 *)(As + r * LDK + kq + 4) = a[1];
}

template <int FMT>
__global__ __launch_bounds__(256) void gemm_kernel(const GemmArgs G, const int32_t *__restrict__ wide) {
    __shared__ __attribute__((aligned(16))) float As[2][BM * LDK];
    __shared__ __attribute__((aligned(16))) float Bs[2][BN * LDK];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int64_t n0 = (int64_t)blockIdx.x * BN, m0 = (int64_t)blockIdx.y * BM;
    const uint8_t *W = (const uint8_t *)G.values;
    const int64_t cols = G.cols;
    const int ksteps = (int)(cols / BK);

    floatx4 acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    uint4 braw[4];
    float bscale;
    float4 areg[2];
    load_b<FMT>(W, G.scales, G.rows, cols, n0, 0, tid, braw, bscale);
    load_a(G.x, G.n, cols, m0, 0, tid, areg);
    store_b<FMT>(Bs[0], tid, braw, bscale);
    store_a(As[0], tid, areg);
    __syncthreads();

    const int gq = lane >> 4, li = lane & 15;
    for (int ks = 0; ks < ksteps; ++ks) {
        const int cur = ks & 1;
        if (ks + 1 < ksteps) {
            load_b<FMT>(W, G.scales, G.rows, cols, n0, (int64_t)(ks + 1) * BK, tid, braw, bscale);
            load_a(G.x, G.n, cols, m0, (int64_t)(ks + 1) * BK, tid, areg);
        }
        const float *as = As[cur], *bs = Bs[cur];
        float af[2][8], bf[4][8];
#pragma unroll
        for (int tm = 0; tm < 2; ++tm) {
            const float *p = as + (wm * 32 + tm * 16 + li) * LDK + 8 * gq;
            const float4 u = *(const float4 *)p, v = *(const float4 *)(p + 4);
            af[tm][0] = u.x, af[tm][1] = u.y, af[tm][2] = u.z, af[tm][3] = u.w;
            af[tm][4] = v.x, af[tm][5] = v.y, af[tm][6] = v.z, af[tm][7] = v.w;
        }
#pragma unroll
        for (int tn = 0; tn < 4; ++tn) {
            const float *p = bs + (wn * 64 + tn * 16 + li) * LDK + 8 * gq;
            const float4 u = *(const float4 *)p, v = *(const float4 *)(p + 4);
            bf[tn][0] = u.x, bf[tn][1] = u.y, bf[tn][2] = u.z, bf[tn][3] = u.w;
            bf[tn][4] = v.x, bf[tn][5] = v.y, bf[tn][6] = v.z, bf[tn][7] = v.w;
        }
#pragma unroll
        for (int s = 0; s < 8; ++s)
#pragma unroll
            for (int tm = 0; tm < 2; ++tm)
#pragma unroll
                for (int tn = 0; tn < 4; ++tn)
                    acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[tm][s], bf[tn][s], acc[tm][tn], 0, 0, 0);
        if (ks + 1 < ksteps) {
            store_b<FMT>(Bs[cur ^ 1], tid, braw, bscale);
            store_a(As[cur ^ 1], tid, areg);
        }
        __syncthreads();
    }

    // D layout of 16x16x4: lane holds rows 4*(lane/16)+r, column lane%16.
#pragma unroll
    for (int tm = 0; tm < 2; ++tm)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t m = m0 + wm * 32 + tm * 16 + 4 * gq + r;
            if (m >= G.n || (wide && wide[m])) continue;
#pragma unroll
            for (int tn = 0; tn < 4; ++tn) {
                const int64_t j = n0 + wn * 64 + tn * 16 + li;
                if (j >= G.rows) continue;
                float v = acc[tm][tn][r];
                if (G.residual) v = G.residual[m * G.y_stride + j] + v;
                G.y[m * G.y_stride + j] = v;
            }
        }
}

__global__ __launch_bounds__(256) void wide_scan_kernel(const float *__restrict__ x, int64_t cols,
                                                        int32_t *__restrict__ flags) {
    __shared__ int any;
    if (threadIdx.x == 0) any = 0;
    __syncthreads();
    const float *xr = x + (int64_t)blockIdx.x * cols;
    int w = 0;
    for (int64_t c = threadIdx.x; c < cols; c += 256) w |= fabsf(xr[c]) > kWideLimit;
    if (w) any = 1;
    __syncthreads();
    if (threadIdx.x == 0) flags[blockIdx.x] = any;
}

// linearQ8WideInto / linearQ4WideInto (M:4356-4382, M:4754-4780).
__device__ __forceinline__ double wide_weight(int fmt, const uint8_t *wrow, int64_t c) {
    if (fmt == SRQ_Q8) return (double)((const int8_t *)wrow)[c];
    if (fmt == SRQ_Q4) {
        uint32_t b = wrow[c >> 1];
        uint32_t nib = (c & 1) ? (b >> 4) : (b & 15u);
        return (double)(((int32_t)(nib << 28)) >> 28);
    }
    return (double)((const float *)wrow)[c];
}

__global__ __launch_bounds__(256) void wide_fix_kernel(const GemmArgs G, const int32_t *__restrict__ flags) {
    const int64_t m = blockIdx.y;
    if (!flags[m]) return;
    const int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (o >= G.rows) return;
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
    G.y[m * G.y_stride + o] = v;
}

}  // namespace

bool gemm_ok(int fmt, int64_t cols) {
    (void)fmt;
    return cols % BK == 0 && cols >= BK;
}

int launch_gemm(hipStream_t s, const GemmArgs &a, const int32_t *wide) {
    if (a.n <= 0 || a.rows <= 0) return SRQ_OK;
    if (!gemm_ok(a.fmt, a.cols)) return fail(SRQ_EINVAL, "gemm: cols=%lld not a multiple of %d", (long long)a.cols, BK);
    dim3 grid((unsigned)((a.rows + BN - 1) / BN), (unsigned)((a.n + BM - 1) / BM));
    switch (a.fmt) {
        case SRQ_Q8: gemm_kernel<SRQ_Q8><<<grid, 256, 0, s>>>(a, wide); break;
        case SRQ_Q4: gemm_kernel<SRQ_Q4><<<grid, 256, 0, s>>>(a, wide); break;
        default: gemm_kernel<SRQ_F32><<<grid, 256, 0, s>>>(a, wide); break;
    }
    SRQ_HIP(hipGetLastError());
    return SRQ_OK;
}

int launch_wide_scan(hipStream_t s, const float *x, int32_t n, int64_t cols, int32_t *flags) {
    if (n <= 0) return SRQ_OK;
    wide_scan_kernel<<<n, 256, 0, s>>>(x, cols, flags);
    SRQ_HIP(hipGetLastError());
    return SRQ_OK;
}

int launch_wide_fix(hipStream_t s, const GemmArgs &a, const int32_t *flags) {
    if (a.n <= 0 || a.rows <= 0) return SRQ_OK;
    dim3 grid((unsigned)((a.rows + 255) / 256), (unsigned)a.n);
    wide_fix_kernel<<<grid, 256, 0, s>>>(a, flags);
    SRQ_HIP(hipGetLastError());
    return SRQ_OK;
}

}  // namespace srq
