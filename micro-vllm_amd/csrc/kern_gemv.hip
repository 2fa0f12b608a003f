// kern_gemv.hip -- decode-shaped (few rows per expert) GEMV kernels for gfx950.
//
// Phase 1 (dual):   H[j, o] = act( x_j . Wg[o], x_j . Wu[o] )   o < Iinter
// Phase 2 (single): Y[j, d] = H_j . Wd[d]                       d < D
// for every compact row j of every expert (src/gpu/metal_ops.cpp:301-327 does the
// same per expert with f32 accumulation; src/quant/quant.cpp:203-228, 298-321).
//
// Fast path (fmt 4/7, K % 32 == 0, 16-byte aligned rows): a group of L lanes owns
// one output row and strides over 16-byte chunks (32 weights) of it with 128-bit
// loads, so a wave streams 64/L rows at once.  Input rows are staged in LDS as
// 36-float records per 32 inputs (32 values, their sum, 3 pad floats: the 144-byte
// stride keeps ds_read_b128 conflict-free).
//   int4:  v_cvt_pk_f32_fp8 on a byte holding a nibble n yields n * 2^-9 exactly
//          (OCP e4m3: codes 0..7 are the subnormals m*2^-9, 8..15 are (8+m')*2^-9),
//          so  sum x*(n-8)*s = (s*2^9) * (sum x*n*2^-9 - 2^-6 * sum x).
//   MXFP4: v_cvt_scalef32_pk_f32_fp4 (scale 1.0) yields the e2m1 values exactly;
//          the ue8m0 scale multiplies the chunk partial.
// Any non-finite chunk contribution is recomputed with the reference's exact
// per-element formula, so Inf/NaN scales or activations propagate as they do there.
#include "moe_internal.h"

#include <cmath>

namespace mvllm_hip {

typedef float f2v __attribute__((ext_vector_type(2)));

// ---- scalar helpers shared with kern_misc.hip through inline definitions -------

__device__ __forceinline__ float dev_sigmoid(float x) {
    // split by sign like the reference (src/quant/quant.hpp:22-29)
    if (x >= 0.f)
        return 1.f / (1.f + expf(-x));
    const float z = expf(x);
    return z / (1.f + z);
}

__device__ __forceinline__ float dev_act(int act, float g, float u, float a, float b) {
    if (act == ACT_CLAMP_SWIGLU) {
        // src/quant/quant.hpp:37-50: gate clamped from above only; a <= 0 disables
        if (a > 0.f && g > a)
            g = a;
        const float s = g * dev_sigmoid(g);
        if (a > 0.f)
            u = fminf(fmaxf(u, -a), a);
        return s * u;
    }
    if (act == ACT_SITU)  // src/quant/quant.hpp:32-34
        return a * tanhf(g / a) * dev_sigmoid(g) * b * tanhf(u / b);
    return g * dev_sigmoid(g) * u;  // silu_mul, src/quant/quant.cpp:400-403
}

__device__ __forceinline__ float dev_mx4_lut(uint32_t n) {
    // e2m1: e = bits 2:1, m = bit 0; e == 0 -> m*0.5, else (1 + m/2) * 2^(e-1)
    const uint32_t e = (n >> 1) & 3u, m = n & 1u;
    const float mag = e == 0 ? 0.5f * (float)m : (1.f + 0.5f * (float)m) * (float)(1u << (e - 1));
    return (n & 8u) ? -mag : mag;
}

__device__ __forceinline__ float dev_mx4_scale(uint32_t e) { return __uint_as_float(e << 23); }

// 16 packed bytes -> 32 floats in natural element order.
// fmt 4: n * 2^-9 (n = raw nibble); fmt 7: exact e2m1 value.
template <int FMT>
__device__ __forceinline__ void decode_chunk(const uint4 &w, float (&v)[32]) {
    const uint32_t dw[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const uint32_t x = dw[d];
        if constexpr (FMT == 4) {
            const uint32_t lo = x & 0x0F0F0F0Fu;         // elements 0,2,4,6 of this dword
            const uint32_t hi = (x >> 4) & 0x0F0F0F0Fu;  // elements 1,3,5,7
            const f2v a = __builtin_amdgcn_cvt_pk_f32_fp8((int)lo, false);
            const f2v b = __builtin_amdgcn_cvt_pk_f32_fp8((int)lo, true);
            const f2v c = __builtin_amdgcn_cvt_pk_f32_fp8((int)hi, false);
            const f2v e = __builtin_amdgcn_cvt_pk_f32_fp8((int)hi, true);
            v[8 * d + 0] = a.x; v[8 * d + 2] = a.y; v[8 * d + 4] = b.x; v[8 * d + 6] = b.y;
            v[8 * d + 1] = c.x; v[8 * d + 3] = c.y; v[8 * d + 5] = e.x; v[8 * d + 7] = e.y;
        } else {
            const f2v p0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(x, 1.0f, 0);
            const f2v p1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(x, 1.0f, 1);
            const f2v p2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(x, 1.0f, 2);
            const f2v p3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(x, 1.0f, 3);
            v[8 * d + 0] = p0.x; v[8 * d + 1] = p0.y; v[8 * d + 2] = p1.x; v[8 * d + 3] = p1.y;
            v[8 * d + 4] = p2.x; v[8 * d + 5] = p2.y; v[8 * d + 6] = p3.x; v[8 * d + 7] = p3.y;
        }
    }
}

// Exact reference formula for one 32-element chunk (used for non-finite cases).
template <int FMT>
__device__ __noinline__ float chunk_exact(uint4 w, const float *x, float scale_raw) {
    float t = 0.f;
    for (int k = 0; k < 32; ++k) {
        const uint32_t word = (k < 8) ? w.x : (k < 16) ? w.y : (k < 24) ? w.z : w.w;
        const uint32_t n = (word >> (4 * (k & 7))) & 15u;
        const float wk = FMT == 4 ? (float)((int)n - 8) * scale_raw : dev_mx4_lut(n) * scale_raw;
        t += x[k] * wk;
    }
    return t;
}

// Scale of the chunk: fmt 4 returns the raw f32 scale; fmt 7 the ue8m0 value.
template <int FMT>
__device__ __forceinline__ float load_scale(const void *S, size_t row, int ngs, int cg) {
    if constexpr (FMT == 4)
        return static_cast<const float *>(S)[row * (size_t)ngs + (size_t)(cg >> 1)];
    else
        return dev_mx4_scale(static_cast<const uint8_t *>(S)[row * (size_t)ngs + (size_t)cg]);
}

template <int FMT, bool DUAL, int NR, int L>
__global__ __launch_bounds__(256) void k_gemv_fast(GemvArgs A, int passes, int kslice) {
    extern __shared__ float4 lds4[];
    float *lds = reinterpret_cast<float *>(lds4);
    constexpr int G = 64 / L;  // output rows per wave per pass
    constexpr int M = DUAL ? 2 : 1;
    const int a = blockIdx.x / A.tiles_per_expert;
    const int tile = blockIdx.x - a * A.tiles_per_expert;
    const ExpertWork &ew = A.ew[a];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int grp = lane / L, gl = lane % L;
    const int K = A.K, O = A.O;
    const size_t rowbytes = (size_t)(K >> 1);
    const int ngs = FMT == 4 ? (K + 63) / 64 : K / 32;
    const int NCH = kslice / 32;  // record stride per staged row
    const int nslices = (K + kslice - 1) / kslice;
    const uint8_t *W[M];
    const void *Sc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
        W[m] = static_cast<const uint8_t *>(ew.w[DUAL ? m : 2]);
        Sc[m] = ew.s[DUAL ? m : 2];
    }

    for (int rc = 0; rc < ew.nrows; rc += NR) {
        const int nrc = min(NR, ew.nrows - rc);
        for (int p = 0; p < passes; ++p) {
            const int o = tile * A.rows_per_tile + (p * 4 + wave) * G + grp;
            float acc[M][NR];
#pragma unroll
            for (int m = 0; m < M; ++m)
#pragma unroll
                for (int r = 0; r < NR; ++r)
                    acc[m][r] = 0.f;
            for (int sl = 0; sl < nslices; ++sl) {
                const int k0 = sl * kslice;
                const int ks = min(kslice, K - k0);
                const int nch = ks >> 5;
                if (nslices > 1 || p == 0) {
                    __syncthreads();
                    // stage nrc input rows [k0, k0+ks) as 36-float records; 8 threads
                    // cover one 32-float chunk and also produce its sum
                    const int q4 = ks >> 2;
                    for (int idx = threadIdx.x; idx < NR * q4; idx += 256) {
                        const int r = idx / q4, q = idx - r * q4;
                        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                        if (r < nrc) {
                            const int j = ew.row0 + rc + r;
                            const int ir = A.in_rows ? A.in_rows[j] : j;
                            v = reinterpret_cast<const float4 *>(A.in + (size_t)ir * (size_t)K +
                                                                 k0)[q];
                        }
                        const int c = q >> 3, pos = q & 7;
                        lds4[(r * NCH + c) * 9 + pos] = v;
                        float s = (v.x + v.y) + (v.z + v.w);
                        s += __shfl_xor(s, 1, 8);
                        s += __shfl_xor(s, 2, 8);
                        s += __shfl_xor(s, 4, 8);
                        if (pos == 0)
                            lds[(r * NCH + c) * 36 + 32] = s;
                    }
                    __syncthreads();
                }
                if (o < O) {
                    const int cg0 = k0 >> 5;
                    uint4 wv[M];
                    float sc[M];
                    int c = gl;
                    if (c < nch) {
#pragma unroll
                        for (int m = 0; m < M; ++m) {
                            wv[m] = *reinterpret_cast<const uint4 *>(W[m] + (size_t)o * rowbytes +
                                                                     (size_t)(cg0 + c) * 16);
                            sc[m] = load_scale<FMT>(Sc[m], (size_t)o, ngs, cg0 + c);
                        }
                    }
                    for (; c < nch; c += L) {
                        // prefetch the next chunk of every matrix before using this one
                        uint4 wn[M];
                        float sn[M];
                        const int cn = c + L;
                        if (cn < nch) {
#pragma unroll
                            for (int m = 0; m < M; ++m) {
                                wn[m] = *reinterpret_cast<const uint4 *>(
                                    W[m] + (size_t)o * rowbytes + (size_t)(cg0 + cn) * 16);
                                sn[m] = load_scale<FMT>(Sc[m], (size_t)o, ngs, cg0 + cn);
                            }
                        }
#pragma unroll
                        for (int m = 0; m < M; ++m) {
                            float wd[32];
                            decode_chunk<FMT>(wv[m], wd);
                            const float sm = FMT == 4 ? sc[m] * 512.f : sc[m];
#pragma unroll
                            for (int r = 0; r < NR; ++r) {
                                if (r < nrc) {
                                    const float4 *xr4 = lds4 + (r * NCH + c) * 9;
                                    float p0 = 0.f, p1 = 0.f;
#pragma unroll
                                    for (int i = 0; i < 8; ++i) {
                                        const float4 t = xr4[i];
                                        p0 = fmaf(t.x, wd[4 * i], p0);
                                        p1 = fmaf(t.y, wd[4 * i + 1], p1);
                                        p0 = fmaf(t.z, wd[4 * i + 2], p0);
                                        p1 = fmaf(t.w, wd[4 * i + 3], p1);
                                    }
                                    const float part = p0 + p1;
                                    float contrib;
                                    if constexpr (FMT == 4)
                                        contrib = fmaf(-xr4[8].x, 0.015625f, part) * sm;
                                    else
                                        contrib = part * sm;
                                    if (!isfinite(contrib))
                                        contrib = chunk_exact<FMT>(
                                            wv[m], reinterpret_cast<const float *>(xr4), sc[m]);
                                    acc[m][r] += contrib;
                                }
                            }
                        }
                        if (cn < nch) {
#pragma unroll
                            for (int m = 0; m < M; ++m) {
                                wv[m] = wn[m];
                                sc[m] = sn[m];
                            }
                        }
                    }
                }
            }
            // reduce over the L lanes of the group; lane gl == r writes row r
#pragma unroll
            for (int m = 0; m < M; ++m)
#pragma unroll
                for (int r = 0; r < NR; ++r) {
                    float v = acc[m][r];
#pragma unroll
                    for (int off = L / 2; off >= 1; off >>= 1)
                        v += __shfl_xor(v, off, L);
                    acc[m][r] = v;
                }
            if (o < O) {
#pragma unroll
                for (int r = 0; r < NR; ++r) {
                    if (r < nrc && gl == r) {
                        const size_t j = (size_t)(ew.row0 + rc + r);
                        float v;
                        if constexpr (DUAL)
                            v = dev_act(A.act, acc[0][r], acc[1][r], A.act_a, A.act_b);
                        else
                            v = acc[0][r];
                        A.out[j * (size_t)O + (size_t)o] = v;
                    }
                }
            }
        }
    }
}

// ---- generic path: any K / alignment / fmt, exact per-element reference formula ----

template <int FMT>
__device__ __forceinline__ float dequant_elem(const void *W, const void *S, int o, int k, int K) {
    if constexpr (FMT == 0) {
        return static_cast<const float *>(W)[(size_t)o * (size_t)K + (size_t)k];
    } else {
        const uint8_t *row = static_cast<const uint8_t *>(W) + (size_t)o * (size_t)((K + 1) / 2);
        const uint32_t b = row[k >> 1];
        const uint32_t n = (k & 1) ? (b >> 4) : (b & 15u);
        if constexpr (FMT == 4) {
            const int ngs = (K + 63) / 64;
            return (float)((int)n - 8) * static_cast<const float *>(S)[(size_t)o * ngs + k / 64];
        } else {
            const int ngs = (K + 31) / 32;
            return dev_mx4_lut(n) *
                   dev_mx4_scale(static_cast<const uint8_t *>(S)[(size_t)o * ngs + k / 32]);
        }
    }
}

// One wave per (expert, output row); 4 waves per block.
template <int FMT, bool DUAL>
__global__ __launch_bounds__(256) void k_gemv_generic(GemvArgs A) {
    const int a = blockIdx.x / A.tiles_per_expert;
    const int tile = blockIdx.x - a * A.tiles_per_expert;
    const ExpertWork &ew = A.ew[a];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int o = tile * 4 + wave;
    if (o >= A.O)
        return;
    const int K = A.K;
    for (int r = 0; r < ew.nrows; ++r) {
        const int j = ew.row0 + r;
        const int ir = A.in_rows ? A.in_rows[j] : j;
        const float *x = A.in + (size_t)ir * (size_t)K;
        float acc[2] = {0.f, 0.f};
        for (int m = 0; m < (DUAL ? 2 : 1); ++m) {
            const int mi = DUAL ? m : 2;
            float t = 0.f;
            for (int k = lane; k < K; k += 64)
                t += x[k] * dequant_elem<FMT>(ew.w[mi], ew.s[mi], o, k, K);
            for (int off = 32; off >= 1; off >>= 1)
                t += __shfl_xor(t, off, 64);
            acc[m] = t;
        }
        if (lane == 0)
            A.out[(size_t)j * (size_t)A.O + (size_t)o] =
                DUAL ? dev_act(A.act, acc[0], acc[1], A.act_a, A.act_b) : acc[0];
    }
}

// ---- launchers --------------------------------------------------------------------

template <int FMT, bool DUAL, int NR>
static hipError_t launch_fast_nr(int L, int passes, const GemvArgs &a, hipStream_t st) {
    const int ks = gemv_kslice(NR, a.K);
    const size_t lds = (size_t)NR * (size_t)(ks / 32) * 144;
    const dim3 grid((unsigned)(a.n_experts * a.tiles_per_expert)), block(256);
    switch (L) {
    case 8: hipLaunchKernelGGL((k_gemv_fast<FMT, DUAL, NR, 8>), grid, block, lds, st, a, passes, ks); break;
    case 16: hipLaunchKernelGGL((k_gemv_fast<FMT, DUAL, NR, 16>), grid, block, lds, st, a, passes, ks); break;
    case 32: hipLaunchKernelGGL((k_gemv_fast<FMT, DUAL, NR, 32>), grid, block, lds, st, a, passes, ks); break;
    default: hipLaunchKernelGGL((k_gemv_fast<FMT, DUAL, NR, 64>), grid, block, lds, st, a, passes, ks); break;
    }
    return hipGetLastError();
}

template <int FMT, bool DUAL>
static hipError_t launch_fast_fd(int nr_max, int L, int passes, const GemvArgs &a,
                                 hipStream_t st) {
    if (nr_max <= 1)
        return launch_fast_nr<FMT, DUAL, 1>(L, passes, a, st);
    if (nr_max <= 2)
        return launch_fast_nr<FMT, DUAL, 2>(L, passes, a, st);
    if (nr_max <= 4)
        return launch_fast_nr<FMT, DUAL, 4>(L, passes, a, st);
    return launch_fast_nr<FMT, DUAL, 8>(L, passes, a, st);
}

hipError_t launch_gemv_fast(int fmt, bool dual, int nr_max, int L, int passes, const GemvArgs &a,
                            hipStream_t st) {
    if (a.n_experts <= 0)
        return hipSuccess;
    if (fmt == 4)
        return dual ? launch_fast_fd<4, true>(nr_max, L, passes, a, st)
                    : launch_fast_fd<4, false>(nr_max, L, passes, a, st);
    if (fmt == 7)
        return dual ? launch_fast_fd<7, true>(nr_max, L, passes, a, st)
                    : launch_fast_fd<7, false>(nr_max, L, passes, a, st);
    return hipErrorInvalidValue;
}

hipError_t launch_gemv_generic(int fmt, bool dual, const GemvArgs &a, hipStream_t st) {
    if (a.n_experts <= 0)
        return hipSuccess;
    const dim3 grid((unsigned)(a.n_experts * a.tiles_per_expert)), block(256);
#define MVLLM_GEN(F, D_) hipLaunchKernelGGL((k_gemv_generic<F, D_>), grid, block, 0, st, a)
    if (fmt == 0) {
        if (dual) MVLLM_GEN(0, true); else MVLLM_GEN(0, false);
    } else if (fmt == 4) {
        if (dual) MVLLM_GEN(4, true); else MVLLM_GEN(4, false);
    } else {
        if (dual) MVLLM_GEN(7, true); else MVLLM_GEN(7, false);
    }
#undef MVLLM_GEN
    return hipGetLastError();
}

// ---- dequant export: the fast decode when the shape allows it, else elementwise ----

template <int FMT>
__global__ void k_dequant_fast(const uint8_t *P, const void *S, int O, int K, float *w) {
    const int nch = K / 32;
    const int ngs = FMT == 4 ? (K + 63) / 64 : K / 32;
    const size_t total = (size_t)O * (size_t)nch;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const int o = (int)(i / nch), c = (int)(i % nch);
        const uint4 wv = *reinterpret_cast<const uint4 *>(P + (size_t)o * (K / 2) + (size_t)c * 16);
        float v[32];
        decode_chunk<FMT>(wv, v);
        const float s = load_scale<FMT>(S, (size_t)o, ngs, c);
        float *dst = w + (size_t)o * K + (size_t)c * 32;
        for (int k = 0; k < 32; ++k) {
            // fmt 4: (n*2^-9)*2^9 = n exactly, then (n-8)*s as the reference rounds it
            dst[k] = FMT == 4 ? (v[k] * 512.f - 8.f) * s : v[k] * s;
        }
    }
}

template <int FMT>
__global__ void k_dequant_generic(const void *P, const void *S, int O, int K, float *w) {
    const size_t total = (size_t)O * (size_t)K;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x)
        w[i] = dequant_elem<FMT>(P, S, (int)(i / K), (int)(i % K), K);
}

hipError_t launch_dequant(int fmt, const void *packed, const void *scales, int O, int K, float *w,
                          hipStream_t st) {
    const bool fast = (K % 32 == 0) && ((uintptr_t)packed % 16 == 0) &&
                      (fmt == 7 || (uintptr_t)scales % 4 == 0);
    const dim3 grid(1024), block(256);
    if (fmt == 4) {
        if (fast)
            hipLaunchKernelGGL(k_dequant_fast<4>, grid, block, 0, st,
                               static_cast<const uint8_t *>(packed), scales, O, K, w);
        else
            hipLaunchKernelGGL(k_dequant_generic<4>, grid, block, 0, st, packed, scales, O, K, w);
    } else if (fmt == 7) {
        if (fast)
            hipLaunchKernelGGL(k_dequant_fast<7>, grid, block, 0, st,
                               static_cast<const uint8_t *>(packed), scales, O, K, w);
        else
            hipLaunchKernelGGL(k_dequant_generic<7>, grid, block, 0, st, packed, scales, O, K, w);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace mvllm_hip
