// On-device Q8/Q4 packing and dequantization for gfx950.
//
// Packing restates the reference's streaming packer bit for bit
// (cmd/monolith/monolith.go: readParam M:857-880, lowBitScale M:3877-3891,
// q8Value M:3893-3898, putQuantized M:3840-3850, q4 put M:3819-3822,
// source decode M:884-920, halfFloat M:838-850).  One wavefront owns one
// 64-column block of one row: lanes load one value each (coalesced), the
// block amax is a wave max (exact in any order), every lane derives the same
// scale with the reference's FP64 divide / f32 round / nextafter steps, and
// each lane rounds its own code half away from zero in FP64.
#include "srq_internal.h"

namespace srq {
namespace {

// halfFloat (M:838-850): exact, including signed zero and subnormals.
__device__ inline float half_bits_to_float(uint32_t v) {
    uint32_t sign = (v & 0x8000u) << 16;
    uint32_t exp = (v >> 10) & 31u, frac = v & 1023u;
    if (exp == 0) {
        float x = (float)frac * 0x1p-24f;  // exact: frac < 2^10
        return __uint_as_float(__float_as_uint(x) | sign);
    }
    if (exp == 31) return __uint_as_float(sign | 0x7f800000u | (frac << 13));
    return __uint_as_float(sign | ((exp + 112u) << 23) | (frac << 13));
}

__device__ inline float load_src(const void *src, int64_t i, int dtype) {
    if (dtype == SRQ_SRC_F32) return ((const float *)src)[i];
    uint32_t w = ((const uint16_t *)src)[i];
    if (dtype == SRQ_SRC_BF16) return __uint_as_float(w << 16);
    return half_bits_to_float(w);
}

// lowBitScale (M:3877-3891).
__device__ inline float low_bit_scale(float amax, double levels) {
    if (amax == 0.0f) return 0.0f;
    float scale = (float)((double)amax / levels);
    const float tiny = __uint_as_float(1u);
    if (scale == 0.0f) return tiny;
    if (scale > tiny && (double)scale * levels > (double)amax) scale = __uint_as_float(__float_as_uint(scale) - 1u);
    return scale;
}

// q8Value / putQuantized: clamp(round_half_away(f64(v)/f64(scale))).
__device__ inline int quant_code(float v, float scale, double lim) {
    if (scale == 0.0f) return 0;
    double q = round((double)v / (double)scale);
    q = q > lim ? lim : q;
    q = q < -lim ? -lim : q;
    return (int)q;
}

__device__ inline float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

template <int FMT>
__global__ __launch_bounds__(256) void pack_kernel(int64_t rows, int64_t cols, const void *__restrict__ src,
                                                   int dtype, void *__restrict__ values,
                                                   float *__restrict__ scales, int *__restrict__ err_flag) {
    const int lane = threadIdx.x & 63;
    const int64_t groups = groups_of(cols);
    const int64_t block = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (block >= rows * groups) return;
    const int64_t row = block / groups, g = block % groups;
    const int64_t col = g * kBlock + lane;
    const bool valid = col < cols;
    float v = valid ? load_src(src, row * cols + col, dtype) : 0.0f;
    if (valid && !isfinite(v)) err_flag[0] = 1;
    float amax = wave_max(valid ? fabsf(v) : 0.0f);
    const double levels = FMT == SRQ_Q8 ? 127.0 : 7.0;
    float scale = low_bit_scale(amax, levels);
    if (lane == 0) scales[row * groups + g] = scale;
    int code = valid ? quant_code(v, scale, levels) : 0;
    if (FMT == SRQ_Q8) {
        if (valid) ((int8_t *)values)[row * cols + col] = (int8_t)code;
    } else {
        // Low nibble = even column, high nibble = odd column; an odd row
        // width leaves a zero high pad nibble (M:3819-3822).
        int hi = __shfl_down(code, 1, 64);
        if (valid && (col & 1) == 0) {
            uint32_t b = ((uint32_t)code & 15u) | ((col + 1 < cols ? ((uint32_t)hi & 15u) : 0u) << 4);
            ((uint8_t *)values)[row * ((cols + 1) / 2) + col / 2] = (uint8_t)b;
        }
    }
}

__global__ __launch_bounds__(256) void convert_kernel(int64_t count, const void *__restrict__ src, int dtype,
                                                      float *__restrict__ dst, int *__restrict__ err_flag) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < count; i += (int64_t)gridDim.x * 256) {
        float v = load_src(src, i, dtype);
        if (!isfinite(v)) err_flag[0] = 1;
        dst[i] = v;
    }
}

// copyRow (M:3900-3921): dst = f32(code) * scale, one rounding.
template <int FMT>
__global__ __launch_bounds__(256) void dequant_kernel(int64_t cols, const void *__restrict__ values,
                                                      const float *__restrict__ scales,
                                                      const int32_t *__restrict__ rows, float *__restrict__ dst) {
    const int64_t groups = groups_of(cols);
    const int64_t r = rows[blockIdx.y];
    float *out = dst + (int64_t)blockIdx.y * cols;
    for (int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x; j < cols; j += (int64_t)gridDim.x * 256) {
        float w;
        if (FMT == SRQ_F32) {
            out[j] = ((const float *)values)[r * cols + j];
            continue;
        } else if (FMT == SRQ_Q8) {
            w = (float)((const int8_t *)values)[r * cols + j];
        } else {
            uint32_t b = ((const uint8_t *)values)[r * ((cols + 1) / 2) + j / 2];
            uint32_t nib = (j & 1) ? (b >> 4) : (b & 15u);
            w = (float)(((int32_t)(nib << 28)) >> 28);
        }
        out[j] = w * scales[r * groups + j / kBlock];
    }
}

// SplitMix64 output number k (k >= 1) from state `seed` (M:1416-1422):
// the state after k calls is seed + k*gamma, so draws are independent.
__device__ inline uint64_t splitmix_at(uint64_t seed, uint64_t k) {
    uint64_t z = seed + k * 0x9e3779b97f4a7c15ULL;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

// dst[i] = f32(Normal() * scale) where Normal uses draws 2i+1 and 2i+2
// (RNG.Normal M:1437-1439, random init M:5218).
__global__ __launch_bounds__(256) void fill_normal_kernel(float *__restrict__ dst, int64_t count, uint64_t seed,
                                                          double scale) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < count; i += (int64_t)gridDim.x * 256) {
        const double u1 = (double)(splitmix_at(seed, 2 * (uint64_t)i + 1) >> 11) * (1.0 / 9007199254740992.0);
        const double u2 = (double)(splitmix_at(seed, 2 * (uint64_t)i + 2) >> 11) * (1.0 / 9007199254740992.0);
        const double nrm = sqrt(-2.0 * log(1.0 - u1)) * cos(2.0 * M_PI * u2);
        dst[i] = (float)(nrm * scale);
    }
}

}  // namespace

int launch_fill_normal(hipStream_t s, float *dst, int64_t count, uint64_t seed, double scale) {
    if (count <= 0) return SRQ_OK;
    int64_t blocks = (count + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    fill_normal_kernel<<<(unsigned)blocks, 256, 0, s>>>(dst, count, seed, scale);
    SRQ_HIP(hipGetLastError());
    return SRQ_OK;
}

int launch_pack(hipStream_t s, int fmt, int64_t rows, int64_t cols, const void *src, int dtype, void *values,
                float *scales, int *err_flag) {
    if (rows <= 0 || cols <= 0) return SRQ_OK;
    int64_t blocks = rows * groups_of(cols);
    dim3 grid((unsigned)((blocks + 3) / 4));
    if (fmt == SRQ_Q8)
        pack_kernel<SRQ_Q8><<<grid, 256, 0, s>>>(rows, cols, src, dtype, values, scales, err_flag);
    else
        pack_kernel<SRQ_Q4><<<grid, 256, 0, s>>>(rows, cols, src, dtype, values, scales, err_flag);
    SRQ_HIP(hipGetLastError());
    return SRQ_OK;
}

int launch_convert_f32(hipStream_t s, int64_t count, const void *src, int dtype, float *dst, int *err_flag) {
    if (count <= 0) return SRQ_OK;
    int64_t blocks = (count + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    convert_kernel<<<(unsigned)blocks, 256, 0, s>>>(count, src, dtype, dst, err_flag);
    SRQ_HIP(hipGetLastError());
    return SRQ_OK;
}

int launch_dequant_rows(hipStream_t s, int fmt, int64_t cols, const void *values, const float *scales,
                        const int32_t *rows, int32_t count, float *dst) {
    if (count <= 0 || cols <= 0) return SRQ_OK;
    int64_t bx = (cols + 255) / 256;
    if (bx > 64) bx = 64;
    dim3 grid((unsigned)bx, (unsigned)count);
    if (fmt == SRQ_Q8)
        dequant_kernel<SRQ_Q8><<<grid, 256, 0, s>>>(cols, values, scales, rows, dst);
    else if (fmt == SRQ_Q4)
        dequant_kernel<SRQ_Q4><<<grid, 256, 0, s>>>(cols, values, scales, rows, dst);
    else
        dequant_kernel<SRQ_F32><<<grid, 256, 0, s>>>(cols, values, scales, rows, dst);
    SRQ_HIP(hipGetLastError());
    return SRQ_OK;
}

}  // namespace srq
