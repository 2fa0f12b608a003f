// kern_f32.hip -- f32-weight GEMMs on the gfx950 matrix cores (v_mfma_f32_16x16x4_f32):
// moe_block with fmt 0 experts (the shared experts, src/model/kimi_k3.cpp:192-209,
// src/model/glm53.cpp:2000-2027), the router scores (src/gpu/metal_ops.cpp:213-231) and
// fmt 0 dense linears (QuantMat::gemm, src/quant/weight.cpp:47-64).
//
// C[r, o] = sum_k X[r, k] * W[o, k] with f32 products and f32 sums (the reference's
// matmul_f32 in another summation order).  Work item = (expert, block of up to 16 * MT
// rows) x (block of columns).  Each wave computes MT row tiles x 2 column tiles of 16
// (dual: the gate and the up rows of the same 16 columns, then the activation; single:
// two adjacent tiles) and streams K in blocks of 16: lane (t, q) loads 16 bytes of row t
// of each operand at K offset 4 q, and MFMA step s takes element s of them, so the four
// steps of a block cover its 16 K indices once.  Waves are independent (no LDS, no
// barrier); loads of the next block are issued before the current one is multiplied.
// I8: a linear on QuantMat's int8 rows (fmt 8; quant::matmul_int8_row,
// src/quant/quant.cpp:255-268): lane (t, q) loads the 4 codes of row t at K offset 4 q,
// each converts exactly to f32, and the row's f32 scale multiplies the finished sum once,
// as the reference does.
#include "mfma_common.h"

#include <algorithm>

namespace mvllm_hip {

constexpr int kF32Waves = 4;

struct F32Item {
    int a, r0, nrow, pad;
};

struct F32Args {
    const ExpertWork *ew;   // per expert: w[0..2] = gate, up, down f32 [O][K]
                            // (I8: w[mi] int8 [O][K], s[mi] f32 [O])
    const F32Item *items;   // null: one expert (ew1), items of 16 * MT rows over nrows_all
    ExpertWork ew1;
    int nrows_all;
    const float *in;        // input rows [*][K]
    const int *in_rows;     // compact row -> input row (null: identity)
    float *out;             // output rows [rcap][O]
    int mi;                 // single: which matrix of the expert (2 = down; 0 = a linear)
    int nbn, K, O;
    int act;
    float act_a, act_b;
};

template <bool DUAL, int MT, bool I8 = false>
__global__ __launch_bounds__(64 * kF32Waves) void k_f32mm(F32Args A) {
    static_assert(!(I8 && DUAL), "int8 rows: single projections only");
    const int item = blockIdx.x / A.nbn;
    const int nb = blockIdx.x - item * A.nbn;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63, t = lane & 15, q = lane >> 4;
    const int K = A.K, O = A.O;
    const int col0 = DUAL ? (nb * kF32Waves + wave) * 16 : (nb * kF32Waves + wave) * 32;
    if (col0 >= O)
        return;  // past the last column tile (waves share nothing: no barrier below)
    F32Item it;
    if (A.items) {
        it = A.items[item];
    } else {
        it.a = 0;
        it.r0 = item * 16 * MT;
        it.nrow = min(16 * MT, A.nrows_all - it.r0);
    }
    const ExpertWork &ew = A.items ? A.ew[it.a] : A.ew1;
    const int jbase = ew.row0 + it.r0;
    // operand row pointers of this lane: MT input rows, two weight rows
    const float4 *xr[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int r = min(mt * 16 + t, it.nrow - 1);  // rows past the item repeat the last
        const int src = A.in_rows ? A.in_rows[jbase + r] : jbase + r;
        xr[mt] = reinterpret_cast<const float4 *>(A.in + (size_t)src * K) + q;
    }
    const float4 *wr[2];
    const int *wr8[2];  // I8: 4 codes of row t at K offset 4 q of each 16-wide block
#pragma unroll
    for (int m = 0; m < 2; ++m) {
        const int row = DUAL ? col0 + t : col0 + 16 * m + t;
        if constexpr (I8) {
            const int8_t *w = static_cast<const int8_t *>(ew.w[A.mi]);
            wr8[m] = reinterpret_cast<const int *>(w + (size_t)row * K) + q;
        } else {
            const float *w = static_cast<const float *>(ew.w[DUAL ? m : A.mi]);
            wr[m] = reinterpret_cast<const float4 *>(w + (size_t)row * K) + q;
        }
    }
    f4v acc[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
        acc[mt][0] = acc[mt][1] = f4v{0.f, 0.f, 0.f, 0.f};
    const int nkb = K >> 4;  // 16-wide K blocks; a block is 4 float4 per row
    float4 xa[2][MT], wb[2][2];
    int wq[2][2];  // I8: raw codes
    auto load = [&](int kb, int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
            xa[buf][mt] = xr[mt][4 * kb];
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            if constexpr (I8)
                wq[buf][m] = wr8[m][4 * kb];
            else
                wb[buf][m] = wr[m][4 * kb];
        }
    };
    auto mma = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                float4 b;
                if constexpr (I8) {
                    const int v = wq[buf][m];
                    b = float4{(float)(int8_t)(v & 0xff), (float)(int8_t)((v >> 8) & 0xff),
                               (float)(int8_t)((v >> 16) & 0xff), (float)(int8_t)(v >> 24)};
                } else {
                    b = wb[buf][m];
                }
                const float4 a = xa[buf][mt];
                acc[mt][m] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, b.x, acc[mt][m], 0, 0, 0);
                acc[mt][m] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, b.y, acc[mt][m], 0, 0, 0);
                acc[mt][m] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, b.z, acc[mt][m], 0, 0, 0);
                acc[mt][m] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, b.w, acc[mt][m], 0, 0, 0);
            }
    };
    // two blocks in flight: block kb + 1 loads while block kb multiplies (past the end:
    // the last block again, never consumed)
    load(0, 0);
    for (int kb = 0; kb < nkb; kb += 2) {
        load(min(kb + 1, nkb - 1), 1);
        mma(0);
        if (kb + 1 >= nkb)
            break;
        load(min(kb + 2, nkb - 1), 0);
        mma(1);
    }
    // C[4 q + i][t] of row tile mt and column tile m
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = mt * 16 + 4 * q + i;
            if (r >= it.nrow)
                continue;
            float *dst = A.out + (size_t)(jbase + r) * O;
            if constexpr (DUAL) {
                dst[col0 + t] = mf_act(A.act, acc[mt][0][i], acc[mt][1][i], A.act_a, A.act_b);
            } else if constexpr (I8) {
                const float *sc = static_cast<const float *>(ew.s[A.mi]);
                dst[col0 + t] = acc[mt][0][i] * sc[col0 + t];
                dst[col0 + 16 + t] = acc[mt][1][i] * sc[col0 + 16 + t];
            } else {
                dst[col0 + t] = acc[mt][0][i];
                dst[col0 + 16 + t] = acc[mt][1][i];
            }
        }
}

bool f32mm_fits(bool dual, int K, int O) {
    return K >= 16 && K % 16 == 0 && O % (dual ? 16 : 32) == 0;
}

hipError_t launch_f32mm(bool dual, int mt, const ExpertWork *ew, const void *items, int n_items,
                        const ExpertWork *ew1, int nrows_all, const float *in,
                        const int *in_rows, float *out, int mi, int K, int O, int act,
                        float act_a, float act_b, hipStream_t st, bool i8) {
    if (!f32mm_fits(dual, K, O) || (mt != 1 && mt != 2 && mt != 4) || (!items && !ew1) ||
        (i8 && dual))
        return hipErrorInvalidValue;
    F32Args a{};
    a.ew = ew;
    a.items = static_cast<const F32Item *>(items);
    if (ew1)
        a.ew1 = *ew1;
    a.nrows_all = nrows_all;
    a.in = in;
    a.in_rows = in_rows;
    a.out = out;
    a.mi = mi;
    a.K = K;
    a.O = O;
    a.act = act;
    a.act_a = act_a;
    a.act_b = act_b;
    const int cols_wg = (dual ? 16 : 32) * kF32Waves;
    a.nbn = (O + cols_wg - 1) / cols_wg;
    if (!items)
        n_items = (nrows_all + 16 * mt - 1) / (16 * mt);
    if (n_items <= 0)
        return hipSuccess;
    const dim3 grid((unsigned)(n_items * a.nbn)), block(64 * kF32Waves);
#define MVLLM_F32(D, M) hipLaunchKernelGGL((k_f32mm<D, M>), grid, block, 0, st, a)
#define MVLLM_I8(M) hipLaunchKernelGGL((k_f32mm<false, M, true>), grid, block, 0, st, a)
    if (i8) {
        if (mt == 1) MVLLM_I8(1); else if (mt == 2) MVLLM_I8(2); else MVLLM_I8(4);
    } else if (dual) {
        if (mt == 1) MVLLM_F32(true, 1); else if (mt == 2) MVLLM_F32(true, 2); else MVLLM_F32(true, 4);
    } else {
        if (mt == 1) MVLLM_F32(false, 1); else if (mt == 2) MVLLM_F32(false, 2); else MVLLM_F32(false, 4);
    }
#undef MVLLM_F32
#undef MVLLM_I8
    return hipGetLastError();
}

// ---- the router's elementwise tail (src/gpu/metal_ops.cpp:218-231) ------------------

// scores [n][E] (the router GEMM) -> mix = sigmoid(score) and choice = mix + bias[e],
// written in place of scores (mix) and into choice.  Sigmoid split by sign as the
// reference's (src/quant/quant.hpp:22-29).
__global__ void k_route_tail(float *scores, const float *bias, float *choice, int n, int E) {
    const size_t total = (size_t)n * E;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const float s = mf_sigmoid(scores[i]);
        scores[i] = s;
        choice[i] = s + (bias ? bias[i % E] : 0.f);
    }
}

// w[n][k] *= rscale (after moe_topk normalized them)
__global__ void k_scale(float *w, size_t count, float rscale) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < count;
         i += (size_t)gridDim.x * blockDim.x)
        w[i] *= rscale;
}

hipError_t launch_route_tail(float *scores, const float *bias, float *choice, int n, int E,
                             hipStream_t st) {
    const size_t total = (size_t)n * E;
    const unsigned grid = (unsigned)std::min<size_t>((total + 255) / 256, 4096);
    hipLaunchKernelGGL(k_route_tail, dim3(grid), dim3(256), 0, st, scores, bias, choice, n, E);
    return hipGetLastError();
}

hipError_t launch_scale(float *w, size_t count, float rscale, hipStream_t st) {
    const unsigned grid = (unsigned)std::min<size_t>((count + 255) / 256, 1024);
    hipLaunchKernelGGL(k_scale, dim3(grid), dim3(256), 0, st, w, count, rscale);
    return hipGetLastError();
}

// ---- RMSNorm (src/quant/quant.cpp:384-398), one workgroup per row -------------------

__global__ __launch_bounds__(256) void k_rmsnorm(const float *x, const float *w, float *y,
                                                 int n, float eps) {
    const float *xr = x + (size_t)blockIdx.x * n;
    float *yr = y + (size_t)blockIdx.x * n;
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += 256)
        ss = fmaf(xr[i], xr[i], ss);
    // wave sums, then across the four waves in fixed order
    for (int o = 32; o > 0; o >>= 1)
        ss += __shfl_xor(ss, o);
    __shared__ float part[4];
    if ((threadIdx.x & 63) == 0)
        part[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float tot = ((part[0] + part[1]) + part[2]) + part[3];
    const float inv = 1.f / sqrtf(tot / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += 256)
        yr[i] = w ? xr[i] * inv * w[i] : xr[i] * inv;
}

hipError_t launch_rmsnorm(const float *x, const float *w, float *y, int rows, int n, float eps,
                          hipStream_t st) {
    hipLaunchKernelGGL(k_rmsnorm, dim3((unsigned)rows), dim3(256), 0, st, x, w, y, n, eps);
    return hipGetLastError();
}

}  // namespace mvllm_hip
