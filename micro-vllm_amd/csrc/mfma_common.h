// mfma_common.h -- device helpers shared by the matrix-core kernels (kern_mfma.hip,
// kern_gemm.hip): weight decode into bf16 MFMA operands, the activation slot order of
// int4 operands, bf16 term splitting, activations and buffer resources.
#pragma once

#include "moe_internal.h"

#include <cmath>

namespace mvllm_hip {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f4v __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float mf_sigmoid(float x) {
    if (x >= 0.f)
        return 1.f / (1.f + expf(-x));
    const float z = expf(x);
    return z / (1.f + z);
}

__device__ __forceinline__ float mf_act(int act, float g, float u, float a, float b) {
    if (act == ACT_CLAMP_SWIGLU) {
        if (a > 0.f && g > a)
            g = a;
        const float s = g * mf_sigmoid(g);
        if (a > 0.f) {  // comparisons, as the reference: a NaN up stays NaN
            if (u > a)
                u = a;
            if (u < -a)
                u = -a;
        }
        return s * u;
    }
    if (act == ACT_SITU)
        return a * tanhf(g / a) * mf_sigmoid(g) * b * tanhf(u / b);
    return g * mf_sigmoid(g) * u;
}

__device__ __forceinline__ bf16x8 pack8(bf16x2 a, bf16x2 b, bf16x2 c, bf16x2 d) {
    bf16x8 r;
    r[0] = a[0]; r[1] = a[1]; r[2] = b[0]; r[3] = b[1];
    r[4] = c[0]; r[5] = c[1]; r[6] = d[0]; r[7] = d[1];
    return r;
}

// One dword = 8 weights (K order e0..e7) of one step -> B operand.
// fmt 4 yields slot order [e0 e2 e4 e6 e1 e3 e5 e7] (the A side is stored permuted to
// match); fmt 7 yields natural order with the block scale folded in, exact for scale
// bytes 2..252 (callers patch the others with decode_b7_exact, see b7_exceptional).
template <int FMT>
__device__ __forceinline__ bf16x8 decode_b(uint32_t w, float scale7) {
    if constexpr (FMT == 4) {
        const int lo = (int)(w & 0x0F0F0F0Fu), hi = (int)((w >> 4) & 0x0F0F0F0Fu);
        return pack8(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 512.f, false),
                     __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 512.f, true),
                     __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 512.f, false),
                     __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 512.f, true));
    } else {
        return pack8(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale7, 0),
                     __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale7, 1),
                     __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale7, 2),
                     __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale7, 3));
    }
}

// MXFP4 weights whose scale byte e would take v * 2^(e-127) out of bf16's normal range
// (e < 2 or e > 252; the reference's e = 0 means +0 and e = 255 means +inf): form the
// product in f32 as the reference does.  The e2m1 value v converts to bf16 exactly at
// scale 1; v has at most two significant bits, so v * scale is exact in f32 and in bf16
// (or is +-0 / +-inf / NaN), and its high half is the operand.
// v * s per element, formed in f32; exact in bf16 when v has at most 8 significant bits
// and the product is a power-of-two multiple of v, or +-0 / +-inf / NaN.
__device__ __forceinline__ bf16x8 mul_bf16x8_exact(bf16x8 v, float s) {
    bf16x8 r;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const float f = (float)v[k] * s;
        r[k] = __builtin_bit_cast(__bf16, (unsigned short)(__float_as_uint(f) >> 16));
    }
    return r;
}

__device__ __forceinline__ bf16x8 decode_b7_exact(uint32_t w, float scale7) {
    return mul_bf16x8_exact(decode_b<7>(w, 1.f), scale7);
}

// int4 nibbles n of one dword -> bf16(n - 8), in decode_b<4>'s slot order, exact: each
// byte becomes the e4m3 code of (n - 8) * 2^-9 (sign bit and 8 - n for n < 8), which the
// converter scales back by 2^9.
__device__ __forceinline__ uint32_t int4_signed_codes(uint32_t l) {  // bytes 0..15
    const uint32_t ge8 = ((l >> 3) & 0x01010101u) * 0xffu;
    const uint32_t neg = 0x80808080u | ((~l & 0x07070707u) + 0x01010101u);
    return (ge8 & (l & 0x07070707u)) | (~ge8 & neg);
}
__device__ __forceinline__ bf16x8 decode_b4_signed(uint32_t w) {
    const int lo = (int)int4_signed_codes(w & 0x0F0F0F0Fu);
    const int hi = (int)int4_signed_codes((w >> 4) & 0x0F0F0F0Fu);
    return pack8(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 512.f, false),
                 __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 512.f, true),
                 __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 512.f, false),
                 __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 512.f, true));
}

__device__ __forceinline__ bool nonfinite(float x) {
    return (__float_as_uint(x) & 0x7f800000u) == 0x7f800000u;
}

// Scale bytes the converter does not reproduce: e = 0 (+0 in the reference, 2^-127 in
// hardware), e = 1 (subnormal products) and e > 252 (overflow; e = 255 is +inf).
__device__ __forceinline__ bool b7_exceptional(float scale7) {
    const uint32_t e = __float_as_uint(scale7) >> 23;
    return e < 2u || e > 252u;
}

// ---- MXFP4 weight scale bytes the scaled matrix cores read differently --------------
// The matrix cores read an ue8m0 byte e as 2^(e-127) for 0..254 and 255 as NaN; the
// reference's mx4_scale gives +0 for e = 0 and +inf for e = 255 (src/quant/quant.hpp:12-20).
// Every other byte agrees.

// Bits of the first `valid` bytes of a 16-byte chunk of scale bytes: 1 = some byte is 0 or
// 255, 2 = some byte is 255 (bytes past `valid` belong to another row or lie past the
// buffer and are ignored).
__device__ __forceinline__ uint32_t ue8m0_special(u32x4 c, int valid) {
    uint32_t r = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int nv = min(max(valid - 4 * i, 0), 4);
        const uint32_t keep = nv >= 4 ? 0xffffffffu : (1u << (8 * nv)) - 1u;
        const uint32_t v = (c[i] & keep) | (0x7f7f7f7fu & ~keep);  // ignored bytes: 127
        const uint32_t nz = ~v;                                     // bytes 255 -> 0
        const uint32_t zero = (v - 0x01010101u) & ~v & 0x80808080u;
        const uint32_t full = (nz - 0x01010101u) & ~nz & 0x80808080u;
        r |= (zero | full) ? 1u : 0u;
        r |= full ? 2u : 0u;
    }
    return r;
}

// e2m1 code n -> its value (the reference's mx4_lut: code 8 is -0).
__device__ __forceinline__ float e2m1_val(uint32_t n) {
    const uint32_t e = (n >> 1) & 3u, m = n & 1u;
    const float mag = e == 0 ? 0.5f * (float)m : (1.f + 0.5f * (float)m) * (float)(1u << (e - 1));
    return (n & 8u) ? -mag : mag;
}

// ue8m0 byte -> the reference's scale bits(e << 23): e = 0 is +0, e = 255 is +inf.
__device__ __forceinline__ float ue8m0_ref(uint32_t e) { return __uint_as_float(e << 23); }

// Position of K element e (within its 8-block) in the stored A row.
template <int FMT>
__device__ __forceinline__ int a_slot(int e) {
    if constexpr (FMT == 4)
        return (e & 1) ? 4 + (e >> 1) : (e >> 1);
    else
        return e;
}

// f32 -> TERMS bf16 terms (hi, then successive remainders); returns the f32 value the
// terms represent (what the MFMA actually multiplies).
template <int TERMS>
__device__ __forceinline__ float split_terms(float x, __bf16 (&t)[3]) {
    t[0] = (__bf16)x;
    float rep = (float)t[0];
    if constexpr (TERMS >= 2) {
        // x = +-inf leaves inf - inf: the high term carries it alone
        const float r1 = nonfinite(rep) ? 0.f : x - rep;
        t[1] = (__bf16)r1;
        rep += (float)t[1];
        if constexpr (TERMS >= 3) {
            const float r2 = r1 - (float)t[1];
            t[2] = (__bf16)r2;
            rep += (float)t[2];
        }
    }
    return rep;
}

// Task of workgroup b out of n when the dispatcher hands workgroups to the 8 XCDs in
// turn (b % 8): XCD x runs the contiguous task range starting at x * n / 8 (the first
// n % 8 XCDs one task more), so consecutive tasks -- the column blocks of one item, and
// the row blocks of one expert -- share that XCD's L2 and are dispatched together.
__device__ __forceinline__ int xcd_task(int b, int n) {
    const int q = n >> 3, r = n & 7, x = b & 7, s = b >> 3;
    return x < r ? x * (q + 1) + s : r * (q + 1) + (x - r) * q + s;
}

// Raw buffer resource over [p, p + bytes) (gfx9 descriptor: stride 0, word 3 = 0x20000).
// Loads through it take a per-lane 32-bit offset plus a wave-uniform offset; offsets past
// `bytes` read as 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes,
                                             0x00020000);
}

}  // namespace mvllm_hip
