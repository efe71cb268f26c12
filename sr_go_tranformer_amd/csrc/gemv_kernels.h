// Dequant-fused GEMV for decode and small batches (n <= 8 per launch):
// the kernels and their launch templates.  gemv_q8.hip, gemv_q4.hip and
// gemv_f32.hip instantiate them per weight format (compiled in parallel);
// gemv.hip dispatches.
//
// Counterpart of linearQ8Into / linearQ4Into / linearFP32Range
// (cmd/monolith/monolith.go M:3942-4780) for batch rows 1..8, with the
// step's neighbouring glue fused in: RMSNorm of the input (rmsInto,
// M:6182-6194) as a prologue; RoPE + KV page write (M:6386-6396), SwiGLU
// (M:6411-6413) or the residual add (M:6400, M:6417) as epilogues.
//
// Layout and mapping (HBM-bound; gfx950 wave64):
//  - A workgroup of 4 waves first stages its n activation rows into LDS
//    (one read of x per workgroup), optionally normalising them.
//  - Each wave owns whole output rows, two at a time ("row groups"): its
//    64 lanes sweep the row in chunks, each lane loading 16 contiguous bytes
//    per row per chunk (global_load_dwordx4), so a wave reads 1 KiB of a row
//    per instruction.  Q8: 16 weights / lane / chunk; Q4: 32; F32: 4.
//  - LDS holds x permuted so that the 16 B a lane reads for its columns are
//    consecutive across lanes (conflict-free ds_read_b128).
//  - Q8 codes convert with one SDWA sign-extending v_cvt_f32_i32 each, then
//    one FMA per weight and batch row.  Q4 nibbles convert with one SDWA
//    v_cvt_off_f32_i4 each (the low nibble of a selected byte, as code/16
//    exactly; the odd columns from the word shifted right by 4); the factor
//    1/16 is removed exactly after the block partial.
//  - Per lane: partial over its 16/32 weights of one 64-column block, then
//    acc = fma(partial, scale, acc); lanes are combined by a fixed xor tree.
//    The arithmetic of a (row, output) pair never depends on n or on the
//    row's slot, so results are batch invariant and deterministic.
//  - Rows holding any |x| > f32(MaxFloat32/(2*64*127)) are recomputed in
//    FP64 (Sum_g f64(scale_g) * Sum_j f64(x_j) f64(w_j), M:4356-4382).
#pragma once

#include <cstdlib>

#include "srq_internal.h"

namespace srq {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

template <int FMT, bool FAST>
struct Lay {
    static constexpr int E = 4;     // weights per lane per chunk
    static constexpr int CW = 256;  // columns per wave chunk
};
template <>
struct Lay<SRQ_Q8, true> {
    static constexpr int E = 16, CW = 1024;
};
template <>
struct Lay<SRQ_Q4, true> {
    static constexpr int E = 32, CW = 2048;
};
template <>
struct Lay<SRQ_F32, true> {
    static constexpr int E = 4, CW = 256;
};

// LDS word of column c: within a chunk, lane l's group q of 4 columns
// (columns E*l + 4q .. +3) lives at q*256 + 4*l.
template <int E, int CW>
__device__ __forceinline__ int xidx(int c) {
    int ch = c / CW, w = c - ch * CW;
    int l = w / E, rem = w - l * E;
    return ch * CW + (rem >> 2) * 256 + l * 4 + (rem & 3);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float sext8(uint32_t w, int byte) { return (float)(int32_t)(int8_t)(w >> (8 * byte)); }

// Decode one lane's weights of one chunk for the FAST layouts.  Q4 yields
// code/16 (see header comment).
template <int FMT>
__device__ __forceinline__ void decode16(const uint4 raw, float *w) {
    const uint32_t d[4] = {raw.x, raw.y, raw.z, raw.w};
    if constexpr (FMT == SRQ_Q8) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            w[4 * k + 0] = sext8(d[k], 0);
            w[4 * k + 1] = sext8(d[k], 1);
            w[4 * k + 2] = sext8(d[k], 2);
            w[4 * k + 3] = sext8(d[k], 3);
        }
    } else if constexpr (FMT == SRQ_Q4) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t hi = d[k] >> 4;  // odd columns in the low nibbles
            w[8 * k + 0] = nib16<0>(d[k]), w[8 * k + 1] = nib16<0>(hi);
            w[8 * k + 2] = nib16<1>(d[k]), w[8 * k + 3] = nib16<1>(hi);
            w[8 * k + 4] = nib16<2>(d[k]), w[8 * k + 5] = nib16<2>(hi);
            w[8 * k + 6] = nib16<3>(d[k]), w[8 * k + 7] = nib16<3>(hi);
        }
    } else {
        w[0] = __uint_as_float(raw.x);
        w[1] = __uint_as_float(raw.y);
        w[2] = __uint_as_float(raw.z);
        w[3] = __uint_as_float(raw.w);
    }
}

// One weight (generic layout, any width).
template <int FMT>
__device__ __forceinline__ float weight_at(const uint8_t *wrow, int64_t c) {
    if constexpr (FMT == SRQ_Q8) return (float)((const int8_t *)wrow)[c];
    if constexpr (FMT == SRQ_Q4) {
        uint32_t b = wrow[c >> 1];
        uint32_t nib = (c & 1) ? (b >> 4) : (b & 15u);
        return (float)(((int32_t)(nib << 28)) >> 28);
    }
    return ((const float *)wrow)[c];
}

struct Smem {
    double ss[8][kWaves];
    float a[8];
    int wide[8];
    int any_wide;
};

// Stage the n activation rows of x into LDS (permuted layout), apply the
// fused RMSNorm when NORM, and flag rows that need the FP64 path.  Ends with
// a barrier; every thread of the workgroup must call it.
template <int E, int CW, int NB, bool NORM>
__device__ __forceinline__ void stage_x(const GemvArgs &A, float *xs, Smem &sm, int ld) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t cols = A.cols;
    if (tid < NB) sm.wide[tid] = 0;
    if (tid == 0) sm.any_wide = 0;
    // Vector path: 4 consecutive columns share l and q, so they are 4
    // consecutive LDS words too.  Loads are issued 8 deep before the stores.
    const bool vec = (cols & 3) == 0 && (((uintptr_t)A.x) & 15) == 0 && (E & 3) == 0;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        double ss = 0.0;
        const float *xb = A.x + (int64_t)b * cols;
        if (vec) {
            constexpr int U = 8;
            for (int c0 = tid * 4; c0 < ld; c0 += kThreads * 4 * U) {
                float4 t[U];
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int c = c0 + u * kThreads * 4;
                    t[u] = (b < A.n && c < cols) ? *(const float4 *)(xb + c) : make_float4(0.f, 0.f, 0.f, 0.f);
                }
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int c = c0 + u * kThreads * 4;
                    if (c < ld) {
                        *(float4 *)(xs + b * ld + xidx<E, CW>(c)) = t[u];
                        if (NORM)
                            ss += (double)t[u].x * t[u].x + (double)t[u].y * t[u].y + (double)t[u].z * t[u].z +
                                  (double)t[u].w * t[u].w;
                    }
                }
            }
        } else {
            for (int c = tid; c < ld; c += kThreads) {
                float v = (b < A.n && c < cols) ? xb[c] : 0.0f;
                xs[b * ld + xidx<E, CW>(c)] = v;
                ss += (double)v * (double)v;
            }
        }
        if (NORM) {
            ss = wave_sum_d(ss);
            if (lane == 0) sm.ss[b][wave] = ss;
        }
    }
    __syncthreads();
    if (NORM) {
        if (tid < NB) {
            double ss = 0.0;
            for (int w = 0; w < kWaves; ++w) ss += sm.ss[tid][w];
            sm.a[tid] = (float)(1.0 / sqrt(ss / (double)cols + A.norm_eps));
        }
        __syncthreads();
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const float a = NORM ? sm.a[b] : 1.0f;
        int wide = 0;
        for (int c = tid; c < cols; c += kThreads) {
            const int i = b * ld + xidx<E, CW>(c);
            float v = xs[i];
            if (NORM) {
                v = __fmul_rn(__fmul_rn(v, a), A.norm_w[c]);  // (x*a)*w, M:6191
                xs[i] = v;
            }
            wide |= fabsf(v) > kWideLimit;
        }
        if (wide && b < A.n) {
            sm.wide[b] = 1;
            sm.any_wide = 1;
        }
    }
    __syncthreads();
}

template <int FMT, bool FAST, int NB, int EPI, bool NORM>
__global__ __launch_bounds__(kThreads) void gemv_kernel(const GemvArgs A) {
    using L = Lay<FMT, FAST>;
    constexpr int E = L::E, CW = L::CW;
    extern __shared__ __attribute__((aligned(16))) float xs[];  // 16 B: ds_read_b128
    __shared__ Smem sm;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t cols = A.cols;
    const int nch = (int)((cols + CW - 1) / CW);
    const int ld = nch * CW;  // LDS words per activation row

    stage_x<E, CW, NB, NORM>(A, xs, sm, ld);

    // ---- row groups ------------------------------------------------------
    const int64_t rows = A.rows;
    const int64_t rb = row_bytes(FMT, cols);
    const int64_t groups = groups_of(cols);
    int64_t ngroups;
    if constexpr (EPI == EPI_SWIGLU)
        ngroups = rows / 2;
    else
        ngroups = (rows + 1) / 2;
    const int64_t stride = (int64_t)gridDim.x * kWaves;
    const uint8_t *W = (const uint8_t *)A.values;

    for (int64_t g = (int64_t)blockIdx.x * kWaves + wave; g < ngroups; g += stride) {
        int64_t r0, r1;
        if constexpr (EPI == EPI_SWIGLU) {
            r0 = g;
            r1 = g + rows / 2;
        } else if constexpr (EPI == EPI_ROPE_KV) {
            const int half = A.head_dim / 2;
            const int64_t qk_pairs = (int64_t)(A.dim + A.kvdim) / 2;
            if (g < qk_pairs) {
                const int64_t h = g / half, j = g - h * half;
                r0 = h * A.head_dim + j;  // heads of q then k are contiguous
                r1 = r0 + half;
            } else {
                r0 = (int64_t)A.dim + A.kvdim + 2 * (g - qk_pairs);
                r1 = r0 + 1;
            }
        } else {
            r0 = 2 * g;
            r1 = 2 * g + 1;
        }
        const bool has1 = r1 < rows;
        const uint8_t *w0 = W + r0 * rb;
        const uint8_t *w1 = W + (has1 ? r1 : r0) * rb;
        const float *s0 = A.scales ? A.scales + r0 * groups : nullptr;
        const float *s1 = A.scales ? A.scales + (has1 ? r1 : r0) * groups : nullptr;

        float acc0[NB], acc1[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) acc0[b] = acc1[b] = 0.0f;

        for (int ch = 0; ch < nch; ++ch) {
            if constexpr (FAST) {
                const int64_t c0 = (int64_t)ch * CW + (int64_t)lane * E;
                if (c0 < cols) {
                    constexpr int BYTES = 16;
                    const int64_t boff = FMT == SRQ_Q8 ? c0 : FMT == SRQ_Q4 ? c0 / 2 : c0 * 4;
                    (void)BYTES;
                    const uint4 raw0 = ld_stream16(w0 + boff);
                    const uint4 raw1 = ld_stream16(w1 + boff);
                    float sc0 = 1.0f, sc1 = 1.0f;
                    if constexpr (FMT != SRQ_F32) {
                        sc0 = s0[c0 / kBlock];
                        sc1 = s1[c0 / kBlock];
                    }
                    float wv0[E], wv1[E];
                    if constexpr (FMT == SRQ_F32) {
                        decode16<FMT>(raw0, wv0);
                        decode16<FMT>(raw1, wv1);
                    } else {
                        // Q4 decodes 32 weights from its 16 bytes.
                        decode16<FMT>(raw0, wv0);
                        decode16<FMT>(raw1, wv1);
                    }
#pragma unroll
                    for (int b = 0; b < NB; ++b) {
                        const float *xb = xs + b * ld + ch * CW + lane * 4;
                        float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
                        for (int q = 0; q < E / 4; ++q) {
                            const float4 xv = *(const float4 *)(xb + q * 256);
                            p0 = __builtin_fmaf(xv.x, wv0[4 * q + 0], p0);
                            p0 = __builtin_fmaf(xv.y, wv0[4 * q + 1], p0);
                            p0 = __builtin_fmaf(xv.z, wv0[4 * q + 2], p0);
                            p0 = __builtin_fmaf(xv.w, wv0[4 * q + 3], p0);
                            p1 = __builtin_fmaf(xv.x, wv1[4 * q + 0], p1);
                            p1 = __builtin_fmaf(xv.y, wv1[4 * q + 1], p1);
                            p1 = __builtin_fmaf(xv.z, wv1[4 * q + 2], p1);
                            p1 = __builtin_fmaf(xv.w, wv1[4 * q + 3], p1);
                        }
                        if constexpr (FMT == SRQ_Q4) {
                            p0 *= 16.0f;  // exact: undo the /16 of the nibble decode
                            p1 *= 16.0f;
                        }
                        if constexpr (FMT == SRQ_F32) {
                            acc0[b] += p0;
                            acc1[b] += p1;
                        } else {
                            acc0[b] = __builtin_fmaf(p0, sc0, acc0[b]);
                            acc1[b] = __builtin_fmaf(p1, sc1, acc1[b]);
                        }
                    }
                }
            } else {
                // Generic: 4 columns per lane per chunk, any width/alignment.
                const int64_t c0 = (int64_t)ch * CW + (int64_t)lane * 4;
                if (c0 < cols) {
                    float wv0[4], wv1[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const bool ok = c0 + e < cols;
                        wv0[e] = ok ? weight_at<FMT>(w0, c0 + e) : 0.0f;
                        wv1[e] = ok ? weight_at<FMT>(w1, c0 + e) : 0.0f;
                    }
                    float sc0 = 1.0f, sc1 = 1.0f;
                    if constexpr (FMT != SRQ_F32) {
                        sc0 = s0[c0 / kBlock];
                        sc1 = s1[c0 / kBlock];
                    }
#pragma unroll
                    for (int b = 0; b < NB; ++b) {
                        const float4 xv = *(const float4 *)(xs + b * ld + c0);
                        float p0 = 0.0f, p1 = 0.0f;
                        p0 = __builtin_fmaf(xv.x, wv0[0], p0);
                        p0 = __builtin_fmaf(xv.y, wv0[1], p0);
                        p0 = __builtin_fmaf(xv.z, wv0[2], p0);
                        p0 = __builtin_fmaf(xv.w, wv0[3], p0);
                        p1 = __builtin_fmaf(xv.x, wv1[0], p1);
                        p1 = __builtin_fmaf(xv.y, wv1[1], p1);
                        p1 = __builtin_fmaf(xv.z, wv1[2], p1);
                        p1 = __builtin_fmaf(xv.w, wv1[3], p1);
                        if constexpr (FMT == SRQ_F32) {
                            acc0[b] += p0;
                            acc1[b] += p1;
                        } else {
                            acc0[b] = __builtin_fmaf(p0, sc0, acc0[b]);
                            acc1[b] = __builtin_fmaf(p1, sc1, acc1[b]);
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            acc0[b] = wave_sum(acc0[b]);
            acc1[b] = wave_sum(acc1[b]);
        }

        // ---- FP64 recomputation of wide rows (cold path) -----------------
        if (sm.any_wide) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                if (!sm.wide[b]) continue;
                double d0 = 0.0, d1 = 0.0;
                for (int64_t c = lane * 4; c < cols; c += 256) {
                    double p0 = 0.0, p1 = 0.0;
                    for (int e = 0; e < 4 && c + e < cols; ++e) {
                        const double xv = (double)xs[b * ld + xidx<E, CW>((int)(c + e))];
                        p0 += xv * (double)weight_at<FMT>(w0, c + e);
                        p1 += xv * (double)weight_at<FMT>(w1, c + e);
                    }
                    const double sc0 = FMT == SRQ_F32 ? 1.0 : (double)s0[c / kBlock];
                    const double sc1 = FMT == SRQ_F32 ? 1.0 : (double)s1[c / kBlock];
                    d0 += p0 * sc0;
                    d1 += p1 * sc1;
                }
                acc0[b] = (float)wave_sum_d(d0);
                acc1[b] = (float)wave_sum_d(d1);
            }
        }

        // ---- epilogues ---------------------------------------------------
        if (lane == 0) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                if (b >= A.n) break;
                float *yb = A.y + (int64_t)b * A.y_stride;
                if constexpr (EPI == EPI_PLAIN) {
                    yb[r0] = acc0[b];
                    if (has1) yb[r1] = acc1[b];
                } else if constexpr (EPI == EPI_RESID) {
                    const float *rs = A.residual + (int64_t)b * A.y_stride;
                    yb[r0] = rs[r0] + acc0[b];
                    if (has1) yb[r1] = rs[r1] + acc1[b];
                } else if constexpr (EPI == EPI_SWIGLU) {
                    // h = f32(g / (1 + exp(-g))) * u  (M:6411-6413)
                    const double gd = (double)acc0[b];
                    const float sg = (float)(gd / (1.0 + exp(-gd)));
                    yb[r0] = __fmul_rn(sg, acc1[b]);
                } else {  // EPI_ROPE_KV
                    float a = acc0[b], z = acc1[b];
                    if (A.bias) {
                        a = __fadd_rn(a, A.bias[r0]);
                        z = __fadd_rn(z, A.bias[r1]);
                    }
                    const int row = A.row0 + b;
                    const int pos = A.meta.pos[row];
                    const int64_t qk_rows = (int64_t)A.dim + A.kvdim;
                    if (r0 < qk_rows) {
                        const int half = A.head_dim / 2;
                        const int j = (int)((r0 % A.head_dim));
                        const float c = A.cos_t[(int64_t)pos * half + j];
                        const float s = A.sin_t[(int64_t)pos * half + j];
                        // x' = a*c - z*s ; z' = a*s + z*c  (M:5283-5285), unfused
                        const float na = __fsub_rn(__fmul_rn(a, c), __fmul_rn(z, s));
                        const float nz = __fadd_rn(__fmul_rn(a, s), __fmul_rn(z, c));
                        a = na;
                        z = nz;
                    }
                    if (r0 < A.dim) {
                        float *q = A.y + (int64_t)b * A.y_stride;
                        q[r0] = a;
                        q[r1] = z;
                    } else {
                        const int sess = A.meta.sess[row];
                        const int page = A.meta.pages[(int64_t)sess * A.meta.pt_stride + pos / kPageTokens];
                        float *kv = A.meta.kv_pool + (int64_t)page * A.meta.page_elems +
                                    (int64_t)A.meta.layer * 2 * kPageTokens * A.kvdim +
                                    (int64_t)(pos % kPageTokens) * A.kvdim;
                        if (r0 < qk_rows) {  // K plane
                            kv[r0 - A.dim] = a;
                            kv[r1 - A.dim] = z;
                        } else {  // V plane
                            float *v = kv + (int64_t)kPageTokens * A.kvdim;
                            v[r0 - qk_rows] = a;
                            if (has1) v[r1 - qk_rows] = z;
                        }
                    }
                }
            }
        }
    }
}



// ---------------------------------------------------------------------------
// Streaming GEMV (fast layouts).  The output rows are cut into "units" (one
// row; a gate/up or RoPE row pair for those epilogues) dealt round-robin to
// the waves.  A wave walks the steps (unit, chunk) of its units in order, keeping the loads of the next P steps in flight
// (16 loads of 16 B per lane) while it converts and accumulates the current
// step; cursors advance without divisions.
// ---------------------------------------------------------------------------

// Wave sum by DPP (quad swaps, half-row and row mirrors, then the GFX9 row
// broadcasts); fixed order, so every call gives the same bits.  The total
// is read from lane 63 and returned uniform.
__device__ __forceinline__ float dpp_sum(float v) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xA, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xC, 0xF, false));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// ------------------------------------------------------- streaming kernel
// Eight waves per workgroup, one workgroup per CU: two waves per SIMD, so one
// wave's convert/FMA work overlaps the other's memory waits.
constexpr int kStreamThreads = 512;
constexpr int kStreamWaves = kStreamThreads / 64;

// Rows per unit: SwiGLU pairs (gate_u, up_u) and RoPE pairs need two rows;
// plain and residual outputs take one row per unit.
template <int EPI>
constexpr int unit_rows_of() {
    return EPI == EPI_SWIGLU || EPI == EPI_ROPE_KV ? 2 : 1;
}

template <int EPI>
__host__ __device__ __forceinline__ int unit_count(const GemvArgs &A) {
    if (EPI == EPI_SWIGLU) return (int)(A.rows / 2);
    if (EPI == EPI_ROPE_KV) return (A.dim + 2 * A.kvdim) / 2;
    return (int)A.rows;
}

// Rows of one unit.  Row indices fit in 32 bits (checked at launch).
struct Unit {
    int r[2];
    int j;  // EPI_ROPE_KV: column within the half head (q/k rows), -1 for v rows
};

// Rows of unit u: gate/up (u, H+u); RoPE pairs (j, j+half) of q and k
// heads, then consecutive v row pairs; plain rows u.
template <int EPI>
__device__ __forceinline__ Unit unit_rows(const GemvArgs &A, int u) {
    Unit t;
    t.j = -1;
    if constexpr (EPI == EPI_SWIGLU) {
        t.r[0] = u;
        t.r[1] = (int)(A.rows / 2) + u;
    } else if constexpr (EPI == EPI_ROPE_KV) {
        const int qk = (A.dim + A.kvdim) / 2;
        if (u < qk) {
            const unsigned half = (unsigned)A.head_dim / 2;
            const unsigned h = (unsigned)u / half;
            t.j = u - (int)(h * half);
            t.r[0] = (int)h * A.head_dim + t.j;
            t.r[1] = t.r[0] + (int)half;
        } else {
            t.r[0] = A.dim + A.kvdim + 2 * (u - qk);
            t.r[1] = t.r[0] + 1;
        }
    } else {
        t.r[0] = u;
        t.r[1] = u;
    }
    return t;
}

// EPI_RESID with RS: a wave stages the residual values of at most this many
// units (its share of the rows) before its weight prefetch.
constexpr int kResidUnits = 16;

// Dynamic LDS of the streaming kernel, in floats: x rows [NB x ld], then the
// RMSNorm weight [ld] (NORM), then per batch row its RoPE {cos, sin} pairs
// [NB x head_dim] and the q/k/v bias [rows] (EPI_ROPE_KV), then with RS per
// wave the residual values of its units [kResidUnits x NB].
struct StreamLds {
    int ld, x, norm, rope, bias, rs, total;
};
template <int NB, int EPI, bool NORM, bool RS>
__host__ __device__ __forceinline__ StreamLds stream_lds(const GemvArgs &A, int ld) {
    StreamLds L;
    L.ld = ld;
    L.x = 0;
    L.norm = NB * ld;
    L.rope = L.norm + (NORM ? ld : 0);
    L.bias = L.rope + (EPI == EPI_ROPE_KV ? NB * A.head_dim : 0);
    const int bias_n = EPI == EPI_ROPE_KV && A.bias ? (int)A.rows : 0;
    L.rs = L.bias + ((bias_n + 3) & ~3);
    L.total = L.rs + (RS ? kStreamWaves * kResidUnits * NB : 0);
    return L;
}

struct StreamSmem {
    double ss[8][kStreamWaves];  // per batch row and wave: f64 sum of squares (RMSNorm)
    int wflag[kStreamWaves];     // per wave: bit b set if a |x| of batch row b exceeds kWideLimit
    int64_t kvoff[8];  // EPI_ROPE_KV: element offset of each batch row's K row (layer 0)
};

// EPI_ROPE_KV: each batch row's KV offset and its position's {cos, sin}
// pairs, loaded into registers ahead of the weight prefetch (loads complete
// in issue order, so loading them after it would make staging wait for the
// whole prefetch) and stored to LDS while staging.
template <int NB, int EPI>
struct RopeStage {
    static constexpr int K = EPI == EPI_ROPE_KV ? (NB * 256 + kStreamThreads - 1) / kStreamThreads : 0;  // head_dim <= 256
    float cs[K > 0 ? K : 1];
    int64_t kv;
};

template <int NB, int EPI>
__device__ __forceinline__ void rope_stage_load(const GemvArgs &A, RopeStage<NB, EPI> &r) {
    if constexpr (EPI == EPI_ROPE_KV) {
        const int tid = threadIdx.x, hd = A.head_dim;
        r.kv = tid < NB && tid < A.n ? A.meta.kvoff[A.row0 + tid] : 0;
#pragma unroll
        for (int k = 0; k < RopeStage<NB, EPI>::K; ++k) {
            const int i = tid + k * kStreamThreads, b = i / hd;
            r.cs[k] = i < NB * hd && b < A.n ? A.meta.rope_cs[(int64_t)(A.row0 + b) * hd + (i - b * hd)] : 0.0f;
        }
    }
}

// Stage the n activation rows of x into LDS (permuted, zero past cols), the
// norm weight, RoPE rows, KV offsets and bias; apply the fused RMSNorm
// (a = f32(1/sqrt(Sum f64(x^2)/d + eps)), y = (x*a)*w, M:6182-6194) and flag
// rows holding |x| > kWideLimit.  One batched pass of global loads, then
// LDS-only work.  Every thread of the workgroup calls it; ends with a barrier.
// Workgroup barrier over LDS only: it waits for this wave's LDS traffic but
// not for its global loads, so a weight prefetch issued before it keeps
// streaming across it (a __syncthreads() waits for every load in flight).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// One pass of the activation staging held in registers: float4 loads of 8
// rows' worth per thread, so one pass stages a 16384-column single row (the
// 14336-wide down input).  The first pass is issued before the weight
// prefetch, so staging waits only for its own loads (global loads complete
// in issue order).
template <int NB, bool NORM>
struct StagePass {
    static constexpr int U = NB >= 8 ? 1 : 8 / NB;
    float4 t[NB][U], w[U];
};

template <bool NORM>
__device__ __forceinline__ bool stage_vec(const GemvArgs &A) {
    return ((((uintptr_t)A.x) | (NORM ? (uintptr_t)A.norm_w : 0)) & 15) == 0 && (A.cols & 3) == 0;
}

template <int NB, bool NORM>
__device__ __forceinline__ void stage_pass_load(const GemvArgs &A, int c0, StagePass<NB, NORM> &s) {
    constexpr int U = StagePass<NB, NORM>::U;
    const int cols = (int)A.cols;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int c = c0 + u * kStreamThreads * 4;
#pragma unroll
        for (int b = 0; b < NB; ++b)
            s.t[b][u] = (b < A.n && c < cols) ? *(const float4 *)(A.x + (int64_t)b * cols + c)
                                              : make_float4(0.f, 0.f, 0.f, 0.f);
        if (NORM) s.w[u] = c < cols ? *(const float4 *)(A.norm_w + c) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

template <int E, int CW, int NB, int EPI, bool NORM>
__device__ __forceinline__ int stage_stream(const GemvArgs &A, float *lds, const StreamLds &L, StreamSmem &sm,
                                            bool vec, StagePass<NB, NORM> &sp, const RopeStage<NB, EPI> &rs) {
    constexpr int NT = kStreamThreads, NW = kStreamWaves;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int cols = (int)A.cols, ld = L.ld;
    float *xs = lds + L.x, *wn = lds + L.norm;
    if constexpr (EPI == EPI_ROPE_KV) {
        if (tid < NB) sm.kvoff[tid] = rs.kv;
        const int hd = A.head_dim;
#pragma unroll
        for (int k = 0; k < RopeStage<NB, EPI>::K; ++k) {
            const int i = tid + k * NT;
            if (i < NB * hd) lds[L.rope + i] = rs.cs[k];
        }
        if (A.bias)
            for (int i = tid; i < (int)A.rows; i += NT) lds[L.bias + i] = A.bias[i];
    }
    double ss[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) ss[b] = 0.0;
    int wide = 0;  // bit b: |x| > kWideLimit in a column of batch row b this thread staged
    auto flag4 = [](const float4 v) {
        return (int)(fabsf(v.x) > kWideLimit) | (int)(fabsf(v.y) > kWideLimit) | (int)(fabsf(v.z) > kWideLimit) |
               (int)(fabsf(v.w) > kWideLimit);
    };
    if (vec) {
        // The first pass (c0 = tid * 4) is already in sp.
        constexpr int U = StagePass<NB, NORM>::U;
        for (int c0 = tid * 4; c0 < ld; c0 += NT * 4 * U) {
            if (c0 != tid * 4) stage_pass_load<NB, NORM>(A, c0, sp);
            const auto &t = sp.t;
            const auto &w = sp.w;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int c = c0 + u * NT * 4;
                if (c >= ld) continue;
                const int i = xidx<E, CW>(c);
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    *(float4 *)(xs + b * ld + i) = t[b][u];
                    if (NORM)
                        ss[b] += (double)t[b][u].x * t[b][u].x + (double)t[b][u].y * t[b][u].y +
                                 (double)t[b][u].z * t[b][u].z + (double)t[b][u].w * t[b][u].w;
                    else
                        wide |= flag4(t[b][u]) << b;
                }
                if (NORM) *(float4 *)(wn + i) = w[u];
            }
        }
    } else {
        for (int c = tid; c < ld; c += NT) {
            const int i = xidx<E, CW>(c);
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const float v = (b < A.n && c < cols) ? A.x[(int64_t)b * cols + c] : 0.0f;
                xs[b * ld + i] = v;
                ss[b] += (double)v * (double)v;
                wide |= (int)(fabsf(v) > kWideLimit) << b;
            }
            if (NORM) wn[i] = c < cols ? A.norm_w[c] : 0.0f;
        }
    }
    if (NORM) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const double t = wave_sum_d(ss[b]);
            if (lane == 0) sm.ss[b][wave] = t;
        }
        lds_barrier();
        // Every thread forms a = f32(1/sqrt(Sum f64(x^2)/d + eps)) from the
        // waves' sums (the same order everywhere, so the same bits), then
        // normalises ((x*a)*w, unfused) the columns it staged itself -- its
        // own LDS writes, so no barrier is needed before reading them -- and
        // flags wide rows.
        wide = 0;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            double t = 0.0;
            for (int w = 0; w < NW; ++w) t += sm.ss[b][w];
            const float a = (float)(1.0 / sqrt(t / (double)cols + A.norm_eps));
            if (vec) {
                for (int c = tid * 4; c < cols; c += NT * 4) {
                    const int i = xidx<E, CW>(c);
                    float4 v = *(float4 *)(xs + b * ld + i);
                    const float4 w = *(const float4 *)(wn + i);
                    v.x = __fmul_rn(__fmul_rn(v.x, a), w.x);
                    v.y = __fmul_rn(__fmul_rn(v.y, a), w.y);
                    v.z = __fmul_rn(__fmul_rn(v.z, a), w.z);
                    v.w = __fmul_rn(__fmul_rn(v.w, a), w.w);
                    *(float4 *)(xs + b * ld + i) = v;
                    wide |= flag4(v) << b;
                }
            } else {
                for (int c = tid; c < cols; c += NT) {
                    const int i = xidx<E, CW>(c);
                    const float v = __fmul_rn(__fmul_rn(xs[b * ld + i], a), wn[i]);
                    xs[b * ld + i] = v;
                    wide |= (int)(fabsf(v) > kWideLimit) << b;
                }
            }
        }
    }
    // One flag word per wave (an OR over its lanes), then every thread ORs
    // the waves' words after the barrier: the workgroup-uniform mask of
    // batch rows that take the FP64 pass.
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) wide |= __shfl_xor(wide, o, 64);
    if (lane == 0) sm.wflag[wave] = wide;
    lds_barrier();
    int mask = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) mask |= sm.wflag[w];
    return mask & ((1 << A.n) - 1);
}

// Write one unit's results: lane b (b < NB, b < n, write) stores batch
// row b; values v[i][b] are wave-uniform.  resid: lane b's residual values
// of the unit's rows (EPI_RESID).  No global loads: operands come from LDS
// or the load stream.
template <int EPI, int NB, int R>
__device__ __forceinline__ void unit_epilogue(const GemvArgs &A, const Unit &t, const float (&v)[R][NB],
                                              const float *lds, const StreamLds &L, const StreamSmem &sm,
                                              float resid, int lane, bool write) {
    if (!(write && lane < NB && lane < A.n)) return;
    const int *r = t.r;
    const int b = lane;
    // vv[i] = v[i][b]: an OR of masked bit patterns (exactly one term is
    // nonzero), which stays in registers (an indexed pick would go through
    // scratch memory).
    float vv[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
        uint32_t bits = 0;
#pragma unroll
        for (int bb = 0; bb < NB; ++bb) bits |= b == bb ? __float_as_uint(v[i][bb]) : 0u;
        vv[i] = __uint_as_float(bits);
    }
    float *yb = A.y + (int64_t)b * A.y_stride;
    if constexpr (EPI == EPI_PLAIN) {
        yb[r[0]] = vv[0];
    } else if constexpr (EPI == EPI_RESID) {
        yb[r[0]] = resid + vv[0];
    } else if constexpr (EPI == EPI_SWIGLU) {
        // h = f32(g / (1 + exp(-g))) * u  (M:6411-6413)
        const double gd = (double)vv[0];
        const float sg = (float)(gd / (1.0 + exp(-gd)));
        yb[r[0]] = __fmul_rn(sg, vv[R - 1]);
    } else {  // EPI_ROPE_KV
        float a = vv[0], z = vv[R - 1];
        if (A.bias) {
            a = __fadd_rn(a, lds[L.bias + r[0]]);
            z = __fadd_rn(z, lds[L.bias + r[1]]);
        }
        if (t.j >= 0) {
            const float c = lds[L.rope + b * A.head_dim + 2 * t.j];
            const float sn = lds[L.rope + b * A.head_dim + 2 * t.j + 1];
            // x' = a*c - z*s ; z' = a*s + z*c  (M:5283-5285), unfused
            const float na = __fsub_rn(__fmul_rn(a, c), __fmul_rn(z, sn));
            const float nz = __fadd_rn(__fmul_rn(a, sn), __fmul_rn(z, c));
            a = na;
            z = nz;
        }
        const int qk_rows = A.dim + A.kvdim;
        if (r[0] < A.dim) {
            yb[r[0]] = a;
            yb[r[1]] = z;
        } else {
            float *kv = A.meta.kv_pool + sm.kvoff[b] + (int64_t)A.meta.layer * 2 * kPageTokens * A.kvdim;
            if (r[0] < qk_rows) {
                kv[r[0] - A.dim] = a;
                kv[r[1] - A.dim] = z;
            } else {
                float *vrow = kv + (int64_t)kPageTokens * A.kvdim;
                vrow[r[0] - qk_rows] = a;
                vrow[r[1] - qk_rows] = z;
            }
        }
    }
}

// G: chunks that share one load of block scales.  A step's lane needs the
// scale of its 64-column block; one dword load per lane covers 64
// consecutive scales, which are the blocks of G chunks (Q8: 4 x 16, Q4:
// 2 x 32).  With G > 1 the load is issued only at the first step of each
// group of G chunks -- a fixed slot of the unrolled prefetch ring, since
// every row holds a whole number of groups -- and each step takes its lane's
// scale from the group's register by a cross-lane permute.  A load per step
// instead (G = 1) doubles the vector memory instructions of the stream:
// 23.2 us against 22.3 us for the 28672 x 4096 GEMV.
//
// RS (EPI_RESID, at most kResidUnits units per wave): the residual values of
// the wave's units are loaded once, ahead of the prefetch, and kept in LDS,
// instead of one residual load per step riding in the weight stream.
//
// RG: units whose rows a step streams together (their chunks share one read
// of the activations from LDS: with 4 or 8 batch rows the per-unit LDS reads
// bound the kernel).  Waves are dealt groups of RG consecutive units; a
// group past the last unit repeats the last unit's rows and writes nothing.
// Every row's arithmetic is that of RG = 1.
template <int FMT, int NB, int EPI, bool NORM, bool WMAJOR, int G, bool RS, int RG = 1>
__global__ __launch_bounds__(kStreamThreads) void gemv_stream_kernel(const GemvArgs A) {
    using Ly = Lay<FMT, true>;
    constexpr int E = Ly::E, CW = Ly::CW, R1 = unit_rows_of<EPI>(), R = R1 * RG;  // R: rows per step
    // 8 row loads in flight per lane (two waves per SIMD, eight per CU).
    constexpr int P = 8 / R;
    static_assert(P % G == 0 && (G == 1 || (WMAJOR && FMT != SRQ_F32)), "scale groups fill the prefetch ring");
    static_assert(!RS || EPI == EPI_RESID, "staged residuals belong to the residual epilogue");
    static_assert(!RS || RG == 1, "staged residuals are per unit");
    extern __shared__ __attribute__((aligned(16))) float lds[];  // 16 B: ds_read_b128
    __shared__ StreamSmem sm;
    // The wave index is uniform: make it scalar so the step loop and its
    // branches are scalar control flow.
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t cols = A.cols;
    const int nch = (int)((cols + CW - 1) / CW);
    const StreamLds L = stream_lds<NB, EPI, NORM, RS>(A, nch * CW);
    const int ld = L.ld;
    float *xs = lds + L.x;

    const int64_t rb = row_bytes(FMT, cols), sgroups = groups_of(cols);
    const int UU = unit_count<EPI>(A);  // units
    const int U = RG == 1 ? UU : (UU + RG - 1) / RG;  // the groups dealt to waves
    if (U == 0) return;  // grid-uniform: no rows, nothing to load or write
    // Units are dealt round-robin (u = wid + k*nwaves): at any moment the
    // waves together sweep one contiguous band of rows, which spreads the
    // traffic over every HBM channel.  WMAJOR (rows of whole 1 KiB chunks):
    // waves are numbered wave-major (wid = wave * workgroups + workgroup),
    // so consecutive rows go to different CUs and XCDs, and when the units do
    // not divide evenly the extra ones land on every CU alike (q/k/v: 3072
    // units on 2048 waves give each CU 12, not 16 on half of them and 8 on
    // the rest).  Shorter rows share cache lines with their neighbours and
    // stay together on one CU (workgroup-major numbering).
    const int nwaves = (int)gridDim.x * kStreamWaves;
    const int wid = WMAJOR ? wave * (int)gridDim.x + (int)blockIdx.x : (int)blockIdx.x * kStreamWaves + wave;
    const int myunits = wid < U ? (U - 1 - wid) / nwaves + 1 : 0;
    const int steps = myunits * nch;
    const int ulast = wid + (myunits - 1) * nwaves;
    const uint8_t *W = (const uint8_t *)A.values;
    // Every chunk is 1 KiB of a row (Q8: 1024 codes, Q4: 2048 nibbles, F32:
    // 256 floats) and a lane reads its 16 bytes of it.  A lane past the row
    // end re-reads the row's first bytes: it meets zero activations (LDS is
    // zero past cols), so its finite weights contribute exactly nothing.
    constexpr int SPC = FMT == SRQ_Q8 ? 16 : FMT == SRQ_Q4 ? 32 : 0;  // scales per chunk
    const int lane_sc = FMT == SRQ_Q8 ? lane / 4 : FMT == SRQ_Q4 ? lane / 2 : 0;
    // EPI_RESID: lane b (< n) follows batch row b's residual; others row 0.
    const float *res_row = EPI == EPI_RESID ? A.residual + (lane < A.n ? lane : 0) * A.y_stride : nullptr;

    // Load cursor (unit lu, chunk lch) with its rows' base pointers.  Loads
    // are unconditional straight-line code, so the compiler waits for exactly
    // the oldest step; past the last step the cursor stays and re-reads it.
    int lu = wid;
    int lch = 0;
    const uint8_t *lw[R];
    const float *ls[R];
    const float *lres[RG] = {};
    auto set_rows = [&](int u) {
#pragma unroll
        for (int k = 0; k < RG; ++k) {
            const Unit t = unit_rows<EPI>(A, RG == 1 ? u : min(u * RG + k, UU - 1));
#pragma unroll
            for (int i = 0; i < R1; ++i) {
                lw[k * R1 + i] = W + (uint64_t)(uint32_t)t.r[i] * (uint64_t)rb;
                ls[k * R1 + i] = FMT == SRQ_F32 ? nullptr : A.scales + (uint64_t)(uint32_t)t.r[i] * (uint64_t)sgroups;
            }
            if constexpr (EPI == EPI_RESID) lres[k] = res_row + t.r[0];
        }
    };
    uint4 wb[P][R];
    float sb[P][R];
    float eb[P][RG];  // EPI_RESID: the units' residual values, carried with each step
    // group_start: constant once the ring is unrolled (slot % G == 0).
    auto load_next = [&](uint4(&w)[R], float(&sc)[R], float(&e)[RG], const bool group_start) {
        // Wave-major rows are whole 1 KiB chunks, so every lane is inside.
        // The offsets are 32-bit unsigned so that each load adds them to its
        // row's scalar base in the instruction (no 64-bit vector adds).
        const bool ok = WMAJOR || (int64_t)lch * CW + (int64_t)lane * E < cols;
        const uint32_t boff = ok ? (uint32_t)(lch * 1024 + lane * 16) : 0u;
        // G > 1: lane l loads scale l of the group (l mod G*SPC: Q8 with
        // G = 2 needs 32), in bounds since rows are whole groups of chunks.
        // The group is the one holding lch: a cursor parked on a wave's last
        // step (any chunk of the row) still reads inside its row.
        const uint32_t soff = G == 1 ? (ok ? (uint32_t)(lch * SPC + lane_sc) : 0u)
                                     : (uint32_t)((lch & ~(G - 1)) * SPC + (lane & (G * SPC - 1)));
#pragma unroll
        for (int i = 0; i < R; ++i) {
            w[i] = ld_stream16(lw[i] + boff);
            if constexpr (FMT != SRQ_F32) {
                if (group_start) sc[i] = *(const float *)((const uint8_t *)ls[i] + soff * 4u);
            } else {
                sc[i] = 1.0f;
            }
        }
        if constexpr (EPI == EPI_RESID && !RS) {
#pragma unroll
            for (int k = 0; k < RG; ++k) e[k] = *lres[k];
        }
        if (lch + 1 < nch) {
            ++lch;
        } else if (lu < ulast) {
            lu += nwaves;
            lch = 0;
            set_rows(lu);
        } else {
            // Past the wave's last step the cursor parks on the activations
            // (at least as many bytes as a row's chunks and its scales), which
            // every workgroup has just staged, so they sit in L2: re-reading
            // each wave's own last steps cost 11% extra HBM traffic at four
            // rows per step (Q4, 28672x4096).
            lch = 0;
#pragma unroll
            for (int i = 0; i < R; ++i) {
                lw[i] = (const uint8_t *)A.x;
                if constexpr (FMT != SRQ_F32) ls[i] = A.x;
            }
        }
    };
    // The first staging pass (and the q/k/v launch's RoPE rows and KV
    // offsets) is issued first; the weight prefetch, which does not depend
    // on x, follows and streams through the staging.
    const bool svec = stage_vec<NORM>(A);
    StagePass<NB, NORM> sp;
    RopeStage<NB, EPI> rs;
    if (svec) stage_pass_load<NB, NORM>(A, tid * 4, sp);
    rope_stage_load<NB, EPI>(A, rs);
    // RS: lane b (< n) loads batch row b's residual of each of the wave's
    // units (the host guarantees at most kResidUnits of them).
    constexpr int NR = RS ? kResidUnits : 1;
    float rsr[NR];
    if constexpr (RS) {
#pragma unroll
        for (int j = 0; j < NR; ++j) {
            rsr[j] = 0.0f;
            if (j < myunits && lane < NB && lane < A.n)
                rsr[j] = A.residual[(int64_t)lane * A.y_stride + unit_rows<EPI>(A, wid + j * nwaves).r[0]];
        }
    }
    // Every wave issues the prefetch, so it is straight-line code and the
    // compiler waits for the staging loads alone; a wave with no unit
    // re-reads unit 0's first chunks and discards them.
    set_rows(steps > 0 ? wid : 0);
#pragma unroll
    for (int p = 0; p < P; ++p) load_next(wb[p], sb[p], eb[p], p % G == 0);
    const int wmask = stage_stream<E, CW, NB, EPI, NORM>(A, lds, L, sm, svec, sp, rs);
    if (steps == 0) {  // wave-uniform; no barrier follows
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): no load outlives the wave
        return;
    }
    // This wave's slice of the staged residuals, written and read by this
    // wave only (its LDS operations complete in order): no barrier.
    float *rsl = lds + L.rs + wave * (kResidUnits * NB);
    if constexpr (RS) {
#pragma unroll
        for (int j = 0; j < NR; ++j)
            if (j < myunits && lane < NB) rsl[j * NB + lane] = rsr[j];
    }
    // Batch rows flagged wide are written by the FP64 pass below instead.
    const bool fast_row = !(lane < NB && ((wmask >> lane) & 1));

    float acc[R][NB];
#pragma unroll
    for (int i = 0; i < R; ++i)
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[i][b] = 0.0f;

    int cu = wid;  // compute cursor
    int kk = 0;    // its unit's index among the wave's units
    int ch = 0;
    float sg[R];  // G > 1: the scales of the current group, kept past the refill of its slot
#pragma unroll
    for (int i = 0; i < R; ++i) sg[i] = 0.0f;
    for (int base = 0; base < steps; base += P) {
#pragma unroll
        for (int k = 0; k < P; ++k) {
            const bool live = base + k < steps;  // wave-uniform
            float scale[R];
#pragma unroll
            for (int i = 0; i < R; ++i) {
                if constexpr (G == 1) {
                    scale[i] = sb[k][i];
                } else {
                    if (k % G == 0) sg[i] = sb[k][i];
                    scale[i] = __shfl(sg[i], (k % G) * SPC + lane_sc, 64);
                }
            }
            if (live) {
                float wv[R][E];
#pragma unroll
                for (int i = 0; i < R; ++i) decode16<FMT>(wb[k][i], wv[i]);
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    float xv[E];
                    const float *xb = xs + b * ld + ch * CW + lane * 4;
#pragma unroll
                    for (int q = 0; q < E / 4; ++q) {
                        const float4 t = *(const float4 *)(xb + q * 256);
                        xv[4 * q] = t.x, xv[4 * q + 1] = t.y, xv[4 * q + 2] = t.z, xv[4 * q + 3] = t.w;
                    }
#pragma unroll
                    for (int i = 0; i < R; ++i) {
                        float p = 0.0f;
#pragma unroll
                        for (int e = 0; e < E; ++e) p = __builtin_fmaf(xv[e], wv[i][e], p);
                        if constexpr (FMT == SRQ_Q4) p *= 16.0f;  // exact: undo the /16 decode
                        acc[i][b] = __builtin_fmaf(p, scale[i], acc[i][b]);
                    }
                }
            }
            // this step's residuals (RS: the unit's staged value), read before the slot is refilled
            float resid[RG];
#pragma unroll
            for (int gq = 0; gq < RG; ++gq) resid[gq] = RS ? (lane < NB ? rsl[kk * NB + lane] : 0.0f) : eb[k][gq];
            load_next(wb[k], sb[k], eb[k], k % G == 0);
            if (!live) continue;
            const bool done = ch == nch - 1;
            const int udone = cu;
            if (done) {
                ch = 0;
                cu += nwaves;
                ++kk;
            } else {
                ++ch;
            }
            if (!done) continue;

            // Units complete: reduce and write.
#pragma unroll
            for (int gq = 0; gq < RG; ++gq) {
                const int uq = RG == 1 ? udone : udone * RG + gq;
                const Unit t = unit_rows<EPI>(A, uq);
                float v[R1][NB];
#pragma unroll
                for (int i = 0; i < R1; ++i)
#pragma unroll
                    for (int b = 0; b < NB; ++b) {
                        v[i][b] = dpp_sum(acc[gq * R1 + i][b]);
                        acc[gq * R1 + i][b] = 0.0f;
                    }
                if (RG == 1 || uq < UU) unit_epilogue<EPI, NB, R1>(A, t, v, lds, L, sm, resid[gq], lane, fast_row);
            }
        }
    }

    // FP64 pass for batch rows holding |x| > kWideLimit (M:4356-4382):
    // Sum_g f64(scale_g) * Sum_j f64(x_j) * f64(w_j), then the epilogue.
    if (!wmask) return;
    for (int u = wid; u < UU; u += nwaves) {
        const Unit t = unit_rows<EPI>(A, u);
        float v[R1][NB] = {};
        for (int b = 0; b < NB; ++b) {
            if (!((wmask >> b) & 1)) continue;
#pragma unroll
            for (int i = 0; i < R1; ++i) {
                const uint8_t *wr = W + (int64_t)t.r[i] * rb;
                double d = 0.0;
                for (int64_t c = lane * 4; c < cols; c += 256) {
                    double pp = 0.0;
                    for (int e = 0; e < 4 && c + e < cols; ++e)
                        pp += (double)xs[b * ld + xidx<E, CW>((int)(c + e))] * (double)weight_at<FMT>(wr, c + e);
                    d += pp * (FMT == SRQ_F32 ? 1.0 : (double)A.scales[(int64_t)t.r[i] * sgroups + c / kBlock]);
                }
                const float f = (float)wave_sum_d(d);
#pragma unroll
                for (int bb = 0; bb < NB; ++bb)
                    if (bb == b) v[i][bb] = f;
            }
        }
        const float resid = EPI == EPI_RESID && lane < A.n ? A.residual[(int64_t)lane * A.y_stride + t.r[0]] : 0.0f;
        unit_epilogue<EPI, NB, R1>(A, t, v, lds, L, sm, resid, lane, !fast_row);
    }
}

// Host-side launch parameters.
int g_cus = 0;
int device_cus() {
    if (g_cus <= 0) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
            g_cus = n;
        else
            g_cus = 256;
    }
    return g_cus;
}

// Workgroups per CU of the streaming GEMV (tunable with SRQ_GEMV_WG_PER_CU).
int gemv_wg_per_cu() {
    static int v = [] {
        const char *e = getenv("SRQ_GEMV_WG_PER_CU");
        int x = e ? atoi(e) : 0;
        return x > 0 && x <= 4 ? x : 1;
    }();
    return v;
}

constexpr size_t kMaxLds = 150 * 1024;

// The streaming kernel variant for a row layout: wave-major dealing for rows
// of whole 1 KiB chunks, with as many chunks per scale load as divide the row
// (Q8 4 or 2, Q4 2; a chunk holds 16 or 32 blocks).
template <int FMT, int NB, int EPI, bool NORM, bool RS, int RG = 1>
int launch_grid(hipStream_t s, const GemvArgs &a, int nch, int64_t blocks) {
    const size_t lds = (size_t)stream_lds<NB, EPI, NORM, RS>(a, nch * Lay<FMT, true>::CW).total * sizeof(float);
    if (lds > kMaxLds)
        return fail(SRQ_EINVAL, "gemv: activation rows do not fit LDS (n=%d cols=%lld)", NB, (long long)a.cols);
    const dim3 grid((unsigned)blocks);
    // chunks per scale load, at most the prefetch ring's steps
    constexpr int P = 8 / (unit_rows_of<EPI>() * RG), GQ = FMT == SRQ_Q8 ? 4 : 2;
    if (row_bytes(FMT, a.cols) % 1024 != 0) {
        gemv_stream_kernel<FMT, NB, EPI, NORM, false, 1, RS, RG><<<grid, kStreamThreads, lds, s>>>(a);
    } else if constexpr (FMT == SRQ_F32) {
        gemv_stream_kernel<FMT, NB, EPI, NORM, true, 1, RS, RG><<<grid, kStreamThreads, lds, s>>>(a);
    } else {
        if constexpr (GQ == 4 && P % 4 == 0) {
            if (nch % 4 == 0) {
                gemv_stream_kernel<FMT, NB, EPI, NORM, true, 4, RS, RG><<<grid, kStreamThreads, lds, s>>>(a);
                SRQ_HIP(hipGetLastError());
                return SRQ_OK;
            }
        }
        if constexpr (P % 2 == 0) {
            if (nch % 2 == 0) {
                gemv_stream_kernel<FMT, NB, EPI, NORM, true, 2, RS, RG><<<grid, kStreamThreads, lds, s>>>(a);
                SRQ_HIP(hipGetLastError());
                return SRQ_OK;
            }
        }
        gemv_stream_kernel<FMT, NB, EPI, NORM, true, 1, RS, RG><<<grid, kStreamThreads, lds, s>>>(a);
    }
    SRQ_HIP(hipGetLastError());
    return SRQ_OK;
}

template <int FMT, bool FAST, int NB, int EPI, bool NORM>
int launch_t(hipStream_t s, const GemvArgs &a) {
    using Ly = Lay<FMT, FAST>;
    const int nch = (int)((a.cols + Ly::CW - 1) / Ly::CW);
    if constexpr (FAST) {
        // The kernel indexes rows, units and steps in 32 bits.
        if (a.rows >= (1LL << 30))
            return fail(SRQ_EINVAL, "gemv: %lld rows exceed the 2^30 row limit", (long long)a.rows);
        if (EPI == EPI_ROPE_KV && (a.head_dim < 2 || a.head_dim > 256))
            return fail(SRQ_EINVAL, "gemv: head_dim %d outside 2..256", a.head_dim);
        const int64_t units = unit_count<EPI>(a);
        int64_t blocks = (units + kStreamWaves - 1) / kStreamWaves;
        const int64_t cap = (int64_t)device_cus() * gemv_wg_per_cu();
        if (blocks > cap) blocks = cap;
        if (blocks < 1) blocks = 1;
        if ((units / (blocks * kStreamWaves) + 1) * nch >= (1LL << 31))
            return fail(SRQ_EINVAL, "gemv: %lld x %lld exceeds the per-wave step limit", (long long)a.rows,
                        (long long)a.cols);
        // One batch row: two units per step, so that their rows share each
        // read of the activations from LDS (Q4 reads 32 of them per 16
        // weight bytes).  Q8 pairs only one-row units: its two-row SwiGLU
        // units in groups of two ran slower (gate/up 22.5 -> 23.1 us).
        if constexpr (NB == 1 && (FMT == SRQ_Q4 || (FMT == SRQ_Q8 && unit_rows_of<EPI>() == 1))) {
            // four, for one-row Q4 units, where every wave gets two groups
            // (28672x4096: 50% -> 53% of peak; 14336x4096, 7 units a wave,
            // falls from 40.5% to 37%)
            if constexpr (FMT == SRQ_Q4 && unit_rows_of<EPI>() == 1) {
                if (units >= 8 * blocks * kStreamWaves)
                    return launch_grid<FMT, NB, EPI, NORM, false, 4>(s, a, nch, blocks);
            }
            if (units >= 2 * blocks * kStreamWaves) return launch_grid<FMT, NB, EPI, NORM, false, 2>(s, a, nch, blocks);
        }
        // Residuals staged when every wave has at most kResidUnits units and
        // their LDS slice fits.
        if constexpr (EPI == EPI_RESID) {
            const bool rs = (units + blocks * kStreamWaves - 1) / (blocks * kStreamWaves) <= kResidUnits &&
                            (size_t)stream_lds<NB, EPI, NORM, true>(a, nch * Ly::CW).total * sizeof(float) <= kMaxLds;
            if (rs) return launch_grid<FMT, NB, EPI, NORM, true>(s, a, nch, blocks);
        }
        // 4-8 batch rows: row groups when there are groups for every wave, as
        // large as the registers hold without spilling (4 batch rows: 4
        // one-row units or 2 pairs; 8 batch rows: 2 one-row units).
        if constexpr (NB >= 4 && FMT != SRQ_F32) {
            constexpr int RGM = NB == 4 ? 4 / unit_rows_of<EPI>() : unit_rows_of<EPI>() == 1 ? 2 : 1;
            const int64_t waves = blocks * kStreamWaves;
            if constexpr (RGM >= 4) {
                if (units >= 4 * waves) return launch_grid<FMT, NB, EPI, NORM, false, 4>(s, a, nch, blocks);
            }
            if constexpr (RGM >= 2) {
                if (units >= 2 * waves) return launch_grid<FMT, NB, EPI, NORM, false, 2>(s, a, nch, blocks);
            }
        }
        return launch_grid<FMT, NB, EPI, NORM, false>(s, a, nch, blocks);
    } else {
        const size_t lds = (size_t)NB * nch * Ly::CW * sizeof(float);
        if (lds > kMaxLds)
            return fail(SRQ_EINVAL, "gemv: activation rows do not fit LDS (n=%d cols=%lld)", NB, (long long)a.cols);
        int64_t ngroups = EPI == EPI_SWIGLU ? a.rows / 2 : (a.rows + 1) / 2;
        int64_t blocks = (ngroups + kWaves - 1) / kWaves;
        const int per_cu = lds > 72 * 1024 ? 1 : lds > 48 * 1024 ? 2 : 4;
        const int64_t cap = 256LL * per_cu * 2;
        if (blocks > cap) blocks = cap;
        if (blocks < 1) blocks = 1;
        gemv_kernel<FMT, false, NB, EPI, NORM><<<(unsigned)blocks, kThreads, lds, s>>>(a);
        SRQ_HIP(hipGetLastError());
        return SRQ_OK;
    }
}

// Widest streaming launch: 8 batch rows (Q4: 2, whose 32 codes per lane
// per chunk leave fewer registers); the generic kernel takes 8.
template <int FMT, bool FAST>
constexpr int max_nb() {
    return !FAST ? 8 : FMT == SRQ_Q4 ? 2 : 8;
}

template <int FMT, bool FAST, int EPI, bool NORM>
int launch_nb(hipStream_t s, const GemvArgs &a) {
    if (a.n > max_nb<FMT, FAST>())
        return fail(SRQ_EINVAL, "gemv: %d activation rows exceed one launch (%d)", a.n, max_nb<FMT, FAST>());
    if (a.n <= 1) return launch_t<FMT, FAST, 1, EPI, NORM>(s, a);
    if (a.n <= 2 || max_nb<FMT, FAST>() == 2) return launch_t<FMT, FAST, 2, EPI, NORM>(s, a);
    if constexpr (max_nb<FMT, FAST>() >= 4) {
        if (a.n <= 4 || max_nb<FMT, FAST>() == 4) return launch_t<FMT, FAST, 4, EPI, NORM>(s, a);
    }
    if constexpr (max_nb<FMT, FAST>() >= 8) return launch_t<FMT, FAST, 8, EPI, NORM>(s, a);
    return fail(SRQ_EINVAL, "gemv: unsupported batch");
}

template <int FMT, bool FAST, int EPI, bool NORM, int NB>
hipError_t prepare_one() {
    if constexpr (NB > max_nb<FMT, FAST>()) {
        return hipSuccess;
    } else {
        if constexpr (FAST) {
            const void *k[8] = {(const void *)gemv_stream_kernel<FMT, NB, EPI, NORM, false, 1, false>,
                                (const void *)gemv_stream_kernel<FMT, NB, EPI, NORM, true, 1, false>};
            if constexpr (FMT != SRQ_F32) {
                k[2] = (const void *)gemv_stream_kernel<FMT, NB, EPI, NORM, true, 2, false>;
                k[3] = (const void *)gemv_stream_kernel<FMT, NB, EPI, NORM, true, (FMT == SRQ_Q8 ? 4 : 2), false>;
            }
            if constexpr (EPI == EPI_RESID) {
                k[4] = (const void *)gemv_stream_kernel<FMT, NB, EPI, NORM, false, 1, true>;
                k[5] = (const void *)gemv_stream_kernel<FMT, NB, EPI, NORM, true, 1, true>;
                if constexpr (FMT != SRQ_F32) {
                    k[6] = (const void *)gemv_stream_kernel<FMT, NB, EPI, NORM, true, 2, true>;
                    k[7] = (const void *)gemv_stream_kernel<FMT, NB, EPI, NORM, true, (FMT == SRQ_Q8 ? 4 : 2), true>;
                }
            }
            for (const void *f : k) {
                if (!f) continue;
                const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxLds);
                if (e != hipSuccess) return e;
            }
            return hipSuccess;
        } else {
            return hipFuncSetAttribute((const void *)gemv_kernel<FMT, false, NB, EPI, NORM>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxLds);
        }
    }
}

template <int FMT, bool FAST, int EPI, bool NORM>
hipError_t prepare_nb() {
    // The fast layouts run only the streaming kernel, the generic one only
    // gemv_kernel; instantiate nothing else.
    const hipError_t errs[] = {prepare_one<FMT, FAST, EPI, NORM, 1>(), prepare_one<FMT, FAST, EPI, NORM, 2>(),
                               prepare_one<FMT, FAST, EPI, NORM, 4>(), prepare_one<FMT, FAST, EPI, NORM, 8>()};
    for (hipError_t e : errs)
        if (e != hipSuccess) return e;
    return hipSuccess;
}

// Instantiated variants: plain (linear), plain + norm (head), residual
// (o / down projections), SwiGLU + norm (gate/up), RoPE/KV + norm (q/k/v).
template <int FMT, bool FAST>
int launch_epi(hipStream_t s, const GemvArgs &a) {
    const bool norm = a.norm_w != nullptr;
    switch (a.epilogue) {
        case EPI_PLAIN:
            return norm ? launch_nb<FMT, FAST, EPI_PLAIN, true>(s, a) : launch_nb<FMT, FAST, EPI_PLAIN, false>(s, a);
        case EPI_RESID:
            if (norm) break;
            return launch_nb<FMT, FAST, EPI_RESID, false>(s, a);
        case EPI_SWIGLU:
            if (!norm) break;
            return launch_nb<FMT, FAST, EPI_SWIGLU, true>(s, a);
        case EPI_ROPE_KV:
            if (!norm) break;
            return launch_nb<FMT, FAST, EPI_ROPE_KV, true>(s, a);
    }
    return fail(SRQ_EINVAL, "gemv: unsupported epilogue/norm combination");
}
template <int FMT, bool FAST>
hipError_t prepare_epi() {
    hipError_t e[5] = {prepare_nb<FMT, FAST, EPI_PLAIN, false>(), prepare_nb<FMT, FAST, EPI_PLAIN, true>(),
                       prepare_nb<FMT, FAST, EPI_RESID, false>(), prepare_nb<FMT, FAST, EPI_SWIGLU, true>(),
                       prepare_nb<FMT, FAST, EPI_ROPE_KV, true>()};
    for (hipError_t x : e)
        if (x != hipSuccess) return x;
    return hipSuccess;
}

}  // namespace

// Per-format entry points (gemv_q8.hip, gemv_q4.hip, gemv_f32.hip).
int gemv_launch_q8(hipStream_t s, const GemvArgs &a, bool fast);
int gemv_launch_q4(hipStream_t s, const GemvArgs &a, bool fast);
int gemv_launch_f32(hipStream_t s, const GemvArgs &a, bool fast);
hipError_t gemv_prepare_q8();
hipError_t gemv_prepare_q4();
hipError_t gemv_prepare_f32();

}  // namespace srq
