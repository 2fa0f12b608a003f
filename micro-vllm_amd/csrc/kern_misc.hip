// kern_misc.hip -- top-k combine and MXFP4 activation quantization for gfx950.
#include "moe_internal.h"

#include <algorithm>
#include <cmath>

namespace mvllm_hip {

// out[t] += w_e * Y[e] for the token's entries in reference order (expert order, then
// row order), each step rounded as `orow[i] += w * hr[i]` rounds on the host
// (src/gpu/metal_ops.cpp:328-339): a product, then a sum, no fused multiply-add.
// The entries' loads are issued in batches of 8 before the ordered accumulation.
// Contraction is off here, for the operators written in this function: clang would
// otherwise fuse the product and the sum into one v_fmac, which rounds once.
__global__ __launch_bounds__(64) void k_combine(CombineArgs A) {
#pragma clang fp contract(off)
    const int t = blockIdx.y;
    const int e0 = A.tok_ptr[t], e1 = A.tok_ptr[t + 1];
    float *orow = A.out + (size_t)(A.out_row ? A.out_row[t] : t) * (size_t)A.D;
    if ((A.D & 3) == 0 && ((uintptr_t)A.out & 15) == 0) {
        const int d4 = blockIdx.x * 64 + threadIdx.x;
        if (d4 * 4 >= A.D)
            return;
        float4 o = reinterpret_cast<float4 *>(orow)[d4];
        for (int eb = e0; eb < e1; eb += 8) {
            float4 y[8];
            float w[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (eb + i < e1) {
                    w[i] = A.ent_w[eb + i];
                    y[i] = reinterpret_cast<const float4 *>(
                        A.Y + (size_t)A.ent_row[eb + i] * (size_t)A.D)[d4];
                }
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (eb + i < e1) {
                    o.x = o.x + w[i] * y[i].x;
                    o.y = o.y + w[i] * y[i].y;
                    o.z = o.z + w[i] * y[i].z;
                    o.w = o.w + w[i] * y[i].w;
                }
            }
        }
        reinterpret_cast<float4 *>(orow)[d4] = o;
    } else {
        for (int d = blockIdx.x * 256 + threadIdx.x; d < A.D && d < (blockIdx.x + 1) * 256;
             d += 64) {
            float o = orow[d];
            for (int e = e0; e < e1; ++e)
                o = o + A.ent_w[e] * A.Y[(size_t)A.ent_row[e] * A.D + d];
            orow[d] = o;
        }
    }
}

hipError_t launch_combine(const CombineArgs &a, hipStream_t st) {
    if (a.n_tok <= 0)
        return hipSuccess;
    const dim3 grid((unsigned)((a.D + 255) / 256), (unsigned)a.n_tok), block(64);
    hipLaunchKernelGGL(k_combine, grid, block, 0, st, a);
    return hipGetLastError();
}

// n 8-byte words from pinned host memory (read over PCIe by the kernel) to device memory:
// a small host-to-device copy that stays a kernel in the stream's queue.
__global__ __launch_bounds__(256) void k_copy_words(const unsigned long long *src,
                                                    unsigned long long *dst, int n) {
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256)
        dst[i] = src[i];
}

// Up to kArgWords 8-byte words carried in the kernel arguments (which the runtime places
// in device memory): no host memory read at all.
__global__ __launch_bounds__(256) void k_fill_words(ArgWords w, unsigned long long *dst) {
    for (int i = threadIdx.x; i < w.n; i += 256)
        dst[i] = w.v[i];
}

hipError_t launch_fill_words(const ArgWords &w, void *dst, hipStream_t st) {
    if (w.n <= 0)
        return hipSuccess;
    if (w.n > kArgWords)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_fill_words, dim3(1), dim3(256), 0, st, w,
                       static_cast<unsigned long long *>(dst));
    return hipGetLastError();
}

hipError_t launch_copy_words(const void *host_src, void *dst, int n, hipStream_t st) {
    if (n <= 0)
        return hipSuccess;
    const unsigned grid = (unsigned)std::min(32, (n + 255) / 256);
    hipLaunchKernelGGL(k_copy_words, dim3(grid), dim3(256), 0, st,
                       static_cast<const unsigned long long *>(host_src),
                       static_cast<unsigned long long *>(dst), n);
    return hipGetLastError();
}

// ---- MXFP4 activation quantization (src/quant/native_act.cpp:159-179, block 32) ----

// Nearest e2m1 code to q in [-6, 6] with the reference's rule (scan of codes 0..15 with
// strict '<': the lowest index wins a tie).  The positive magnitudes are codes 0..7
// {0, .5, 1, 1.5, 2, 3, 4, 6}; a tie between two of them goes to the smaller one, and a
// result of zero is always code 0 (code 8, -0, comes later in the scan).  So: round |q|
// to the grid with ties toward zero, then set the sign bit for negative non-zero codes.
// NaN never gets here: clamping with fminf/fmaxf maps it to 6 first, as in the reference.
__device__ __forceinline__ int nearest_e2m1(float q) {
    const float m = fabsf(q);
    const int c = (m > 0.25f) + (m > 0.75f) + (m > 1.25f) + (m > 1.75f) + (m > 2.5f) +
                  (m > 3.5f) + (m > 5.f);
    return (q < 0.f && c > 0) ? (c | 8) : c;
}

// ceil(log2(v)) for v >= 2^-126 (frexp exponent, minus one at exact powers of two).
// An infinite v (a block holding +-Inf) gives 0: frexp leaves the exponent at 0 for
// non-finite input, which is what the reference's ceil_log2_positive then returns.
__device__ __forceinline__ int ceil_log2_normal(float v) {
    const uint32_t b = __float_as_uint(v);
    const int ef = (int)((b >> 23) & 0xffu);
    if (ef == 255)
        return 0;
    return (b & 0x7fffffu) == 0 ? ef - 127 : ef - 126;
}

// Eight lanes per 32-element block, four elements per lane (one 16-byte load), eight
// blocks per wave and QU blocks per lane in flight.  The block maximum is reduced
// across the 8 lanes; each lane packs its 4 codes into 2 bytes (low nibble = even
// element).  Output row j reads input row rows_map[j] (or j).  Indices are 32-bit: the
// launcher refuses more than 2^31 blocks.
constexpr int kQU = 4;

// e2m1 code -> value (0, 0.5, 1, 1.5, 2, 3, 4, 6; bit 3 the sign)
__device__ __forceinline__ float e2m1_value(uint32_t c) {
    const uint32_t m = c & 7u;
    const float v = m < 4u ? 0.5f * (float)m : (float)(2u << ((m - 4u) >> 1)) * (1.f + 0.5f * (float)(m & 1u));
    return (c & 8u) ? -v : v;
}

// planes (nullable): also the quantized values themselves as bf16 rows [n][K] (code value
// x 2^ex has at most two significant bits, so the bf16 holds it exactly; it is the f32
// value's upper half), for the rows j with pmask[j] != 0 (all rows when pmask is null).
__global__ __launch_bounds__(256) void k_quantize_mxfp4(const float *x, const int *rows_map,
                                                        int n, int K, uint8_t *codes,
                                                        uint8_t *scales, __bf16 *planes,
                                                        const uint8_t *pmask,
                                                        const int *n_live, int src_rows) {
    const uint32_t nb = (uint32_t)(K / 32);
    if (n_live)  // rows past the device count are left alone
        n = min(n, max(__builtin_amdgcn_readfirstlane(*n_live), 0));
    const uint32_t total = (uint32_t)n * nb;  // blocks
    const uint32_t lane = threadIdx.x & 63, e8 = lane & 7;
    const uint32_t wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const uint32_t nwaves = (gridDim.x * blockDim.x) >> 6;
    // wave-uniform loop bound: every shuffle below sees the whole wave
    for (uint32_t b0 = wave * 8 * kQU; b0 < total; b0 += nwaves * 8 * kQU) {
        float4 v[kQU];
        uint32_t row[kQU], blk[kQU];
#pragma unroll
        for (int u = 0; u < kQU; ++u) {
            const uint32_t bid = b0 + 8 * u + (lane >> 3);
            const bool ok = bid < total;
            row[u] = ok ? bid / nb : 0;
            blk[u] = ok ? bid - row[u] * nb : 0;
            const int srci = rows_map ? rows_map[row[u]] : (int)row[u];
            const bool live = ok && (src_rows < 0 || (srci >= 0 && srci < src_rows));
            const uint32_t src = live ? (uint32_t)srci : 0u;
            v[u] = live ? *reinterpret_cast<const float4 *>(x + (size_t)src * K + blk[u] * 32 +
                                                            4 * e8)
                        : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int u = 0; u < kQU; ++u) {
            const uint32_t bid = b0 + 8 * u + (lane >> 3);
            const float f[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
            float amax = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float a = fabsf(f[i]);
                if (a > amax)  // NaN never wins (the reference's '>' test)
                    amax = a;
            }
#pragma unroll
            for (int o = 4; o >= 1; o >>= 1)
                amax = fmaxf(amax, __shfl_xor(amax, o, 8));
            amax = fmaxf(amax, 6.f * 1.1754943508222875e-38f);  // 6 * 2^-126
            // amax / 6 lies in [2^-126, FLT_MAX / 6 < 2^126] or is +Inf (exponent 0), so
            // ex is within [-126, 126] and the reference's clamp to [-127, 127] never
            // binds; 2^-ex is then a normal float and x / 2^ex == x * 2^-ex exactly (both
            // round the same real number)
            const int ex = ceil_log2_normal(amax / 6.f);
            const float inv = __uint_as_float((uint32_t)(127 - ex) << 23);
            uint32_t packed = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float sc = f[i] * inv;
                const float q = fmaxf(-6.f, fminf(6.f, sc));
                packed |= (uint32_t)nearest_e2m1(q) << (4 * i);
            }
            if (bid < total) {
                *reinterpret_cast<uint16_t *>(codes + (size_t)row[u] * (size_t)(K / 2) +
                                              blk[u] * 16 + 2 * e8) = (uint16_t)packed;
                if (e8 == 0)
                    scales[bid] = (uint8_t)(ex + 127);
                if (planes && (!pmask || pmask[row[u]])) {
                    uint32_t h[2];
#pragma unroll
                    for (int i = 0; i < 2; ++i) {
                        const float lo = ldexpf(e2m1_value((packed >> (8 * i)) & 15u), ex);
                        const float hi = ldexpf(e2m1_value((packed >> (8 * i + 4)) & 15u), ex);
                        h[i] = (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xffff0000u);
                    }
                    *reinterpret_cast<uint2 *>(planes + (size_t)row[u] * (size_t)K +
                                               blk[u] * 32 + 4 * e8) = make_uint2(h[0], h[1]);
                }
            }
        }
    }
}

hipError_t launch_quantize_mxfp4(const float *x, int n, int K, uint8_t *codes, uint8_t *scales,
                                 hipStream_t st, const int *rows_map, void *planes,
                                 const uint8_t *pmask, const int *n_live, int src_rows) {
    if (n <= 0 || K <= 0 || K % 32 || (size_t)n * (K / 32) >= (size_t(1) << 31) ||
        (reinterpret_cast<uintptr_t>(x) & 15))
        return hipErrorInvalidValue;
    const size_t waves = ((size_t)n * (K / 32) + 8 * kQU - 1) / (8 * kQU);
    const size_t wgs = (waves + 3) / 4;
    const unsigned grid = (unsigned)(wgs < 4096 ? wgs : 4096);
    hipLaunchKernelGGL(k_quantize_mxfp4, dim3(grid), dim3(256), 0, st, x, rows_map, n, K, codes,
                       scales, static_cast<__bf16 *>(planes), pmask, n_live, src_rows);
    return hipGetLastError();
}

// ---- memory probes (roofline calibration) -------------------------------------------

// kind 0: coalesced 16-byte reads of n16 uint4 (grid-stride); the xor keeps them live.
// kind 2..: a wave walks a tile of rows (row16 uint4 per row) as the expert weights are
// walked; pattern = kind - 2 selects (bytes per lane, lanes per row):
//   0: (8, 4)  -> 16 rows x 32 B per load      1: (16, 2) -> 32 rows x 32 B
//   2: (16, 4) -> 16 rows x 64 B               3: (16, 16) -> 4 rows x 256 B
//   4: (16, 64) -> 1 row x 1 KB
template <int LB, int LPR>
__device__ __forceinline__ uint32_t walk_rows(const uint4 *src, size_t n16, int row16) {
    constexpr int RPI = 64 / LPR;  // rows per load instruction
    const int lane = threadIdx.x & 63;
    const size_t wave = (blockIdx.x * (size_t)blockDim.x + threadIdx.x) >> 6;
    const size_t nwaves = ((size_t)gridDim.x * blockDim.x) >> 6;
    const size_t tile16 = (size_t)RPI * row16;
    const size_t ntiles = n16 / tile16;
    const int step = LPR * LB;  // bytes per row per load
    uint32_t acc = 0;
    const uint8_t *s8 = reinterpret_cast<const uint8_t *>(src);
    for (size_t t = wave; t < ntiles; t += nwaves) {
        const uint8_t *row = s8 + (t * tile16 + (size_t)(lane / LPR) * row16) * 16 + (lane % LPR) * LB;
#pragma unroll 8
        for (int c = 0; c < row16 * 16; c += step) {
            if constexpr (LB == 8) {
                const uint2 v = *reinterpret_cast<const uint2 *>(row + c);
                acc ^= v.x ^ v.y;
            } else {
                const uint4 v = *reinterpret_cast<const uint4 *>(row + c);
                acc ^= v.x ^ v.y ^ v.z ^ v.w;
            }
        }
    }
    return acc;
}

__global__ __launch_bounds__(256) void k_stream_read(const uint4 *src, size_t n16, int kind,
                                                     int row16, uint32_t *sink) {
    uint32_t acc = 0;
    if (kind == 0) {
        for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n16;
             i += (size_t)gridDim.x * blockDim.x) {
            const uint4 v = src[i];
            acc ^= v.x ^ v.y ^ v.z ^ v.w;
        }
    } else if (kind == 2) {
        acc = walk_rows<8, 4>(src, n16, row16);
    } else if (kind == 3) {
        acc = walk_rows<16, 2>(src, n16, row16);
    } else if (kind == 4) {
        acc = walk_rows<16, 4>(src, n16, row16);
    } else if (kind == 5) {
        acc = walk_rows<16, 16>(src, n16, row16);
    } else {
        acc = walk_rows<16, 64>(src, n16, row16);
    }
    if (acc == 0x9e3779b9u)  // practically never; keeps the loads
        sink[0] = acc;
}

__global__ __launch_bounds__(256) void k_stream_copy(const uint4 *src, uint4 *dst, size_t n16) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n16;
         i += (size_t)gridDim.x * blockDim.x)
        dst[i] = src[i];
}

hipError_t launch_membench(int kind, const void *src, void *dst, size_t bytes, int row16,
                           hipStream_t st) {
    const size_t n16 = bytes / 16;
    const dim3 grid(256 * 16), block(256);
    if (kind == 1)
        hipLaunchKernelGGL(k_stream_copy, grid, block, 0, st, static_cast<const uint4 *>(src),
                           static_cast<uint4 *>(dst), n16);
    else
        hipLaunchKernelGGL(k_stream_read, grid, block, 0, st, static_cast<const uint4 *>(src), n16,
                           kind, row16, static_cast<uint32_t *>(dst));
    return hipGetLastError();
}

}  // namespace mvllm_hip
