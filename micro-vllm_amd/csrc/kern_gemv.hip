// kern_gemv.hip -- the exact element-wise expert GEMV (any K, alignment or format) and
// the f32 dequantization export, for gfx950.
//
// Phase 1 (dual):   H[j, o] = act( x_j . Wg[o], x_j . Wu[o] )   o < Iinter
// Phase 2 (single): Y[j, d] = H_j . Wd[d]                       d < D
// for every compact row j of every expert, each weight formed as the reference forms
// it (src/quant/quant.cpp:203-228, 298-321).  Shapes the matrix-core path does not
// cover (K not a multiple of 1024, unaligned pointers, f32 weights) run here.
//
// The f32 decode used by the dequantization export:
//   int4:  v_cvt_pk_f32_fp8 on a byte holding a nibble n yields n * 2^-9 exactly
//          (OCP e4m3: codes 0..7 are the subnormals m*2^-9, 8..15 are (8+m')*2^-9).
//   MXFP4: v_cvt_scalef32_pk_f32_fp4 (scale 1.0) yields the e2m1 values exactly.
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
        if (a > 0.f) {  // comparisons, as the reference: a NaN up stays NaN
            if (u > a)
                u = a;
            if (u < -a)
                u = -a;
        }
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

// Scale of the chunk: fmt 4 returns the raw f32 scale; fmt 7 the ue8m0 value.
template <int FMT>
__device__ __forceinline__ float load_scale(const void *S, size_t row, int ngs, int cg) {
    if constexpr (FMT == 4)
        return static_cast<const float *>(S)[row * (size_t)ngs + (size_t)(cg >> 1)];
    else
        return dev_mx4_scale(static_cast<const uint8_t *>(S)[row * (size_t)ngs + (size_t)cg]);
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
