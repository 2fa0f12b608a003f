// kern_fp4.hip -- native MXFP4 expert GEMMs on the gfx950 scaled matrix cores
// (v_mfma_scale_f32_16x16x128_f8f6f4, both operands e2m1 with one ue8m0 scale per 32).
//
// The weights feed the matrix cores exactly as stored (no decode); the activations are
// the reference's MXFP4 quantization of the GEMM inputs (fp4_activation_qdq, block 32),
// made by k_quantize_mxfp4.  Every product of two e2m1 values times two powers of two
// is exact, so the result differs from the composed reference (QDQ, then the f32
// moe_block maths) only by summation order.
//
// Operand layout of the 16x16x128 step (lane l, t = l % 16, q = l / 16): A row t and B
// column t hold K elements [32 q, 32 q + 32) -- 16 bytes of packed codes, low nibble
// first -- and the lane's scale operand is the ue8m0 byte of that 32-block; the result
// is C[4 q + i][t], i = 0..3, as for the bf16 16x16 MFMAs.
//
// Tiling as the bf16 grouped GEMM (row tiles MT = 4, 8 or 16; the 16- and 32-row classes
// take the bf16 GEMM on exact bf16 copies of the quantized activations): a workgroup of 8
// waves serves (item, column block), each wave two 16-column tiles (gate and up at the same
// columns for the dual projection, two adjacent tiles of the down matrix otherwise) over
// MT row tiles; K advances 256 per step.  The item's activation codes of a step go
// straight into LDS (buffer_load ... lds, double buffered, one step ahead), their scales
// through registers; the weights of a step are loaded two steps ahead into registers (per
// tile and lane two 16-byte loads: row t, bytes 32 q + 16 s), their scales in 64-byte
// chunks per 8 steps.  MFMA step s takes 32-block 2 q + s of the 256-K step in lane
// (t, q) (A and B agree on the order, which only permutes the summation).
#include "mfma_common.h"

namespace mvllm_hip {

typedef int i32x8 __attribute__((ext_vector_type(8)));

struct F4Item {
    int a, r0, nrow, pad;
};

struct F4Args {
    const ExpertWork *ew;
    const F4Item *items;
    const uint8_t *acode;   // [rcap][K/2]
    const uint8_t *ascale;  // [rcap][K/32]
    float *hout;            // dual: H f32 [rcap][O]
    float *out;             // single: Y f32 [rcap][O]
    int nbn, K, O, rcap;
    int xcd;  // 1: tasks ordered per XCD (xcd_task)
    const int *n_items_dev;  // non-null: item count in device memory (grid sized for a bound)
    int act;
    float act_a, act_b;
};

constexpr int kF4Threads = 512;
constexpr int kF4Row = 128;  // LDS bytes per A row of codes (a step of 256 K)

__host__ __device__ constexpr int f4_stage_bytes(int mt) {
    return 16 * mt * kF4Row + 16 * mt * 8;
}

size_t fp4_lds_bytes(int mt) { return 2 * (size_t)f4_stage_bytes(mt); }

struct F4Step {
    u32x4 w[2][2];  // tile m, MFMA step s: row t, bytes 32 q + 16 s of the 128-byte step
};
// Weight scales in 64-byte chunks of each row (8 steps): lane (t, q) holds bytes 16 q ..
// 16 q + 15 of row t's chunk, i.e. steps 2 q and 2 q + 1 of it.  One load per 8 steps:
// per-step 8-byte loads made a third of the kernel's L2 requests.
struct F4Scl {
    u32x4 c[2];
};

template <bool DUAL, int MT>
__global__ __launch_bounds__(kF4Threads) void k_gemm_fp4(F4Args A) {
    constexpr int BM = 16 * MT;
    constexpr int STAGE = f4_stage_bytes(MT);
    // steps of weights in flight (128 and 256 rows: three, faster than two or four) and
    // the loop unroll, a multiple of NB and of 2
    constexpr int NB = MT >= 8 ? 3 : 2;
    constexpr int UN = NB % 2 ? 2 * NB : NB;
    extern __shared__ __attribute__((aligned(16))) char smem[];

    const int n_tasks = A.n_items_dev
                            ? __builtin_amdgcn_readfirstlane(*A.n_items_dev) * A.nbn
                            : (int)gridDim.x;
    if ((int)blockIdx.x >= n_tasks)
        return;
    const int task = A.xcd ? xcd_task(blockIdx.x, n_tasks) : (int)blockIdx.x;
    // An expert's run of nblk items owns tasks [g0 nbn, (g0 + nblk) nbn); they go column
    // block by column block, its row blocks adjacent, so that the row blocks running side
    // by side on one XCD read that column block's weights through its L2 together.
    int item = task / A.nbn;
    const int grp = A.items[item].pad;  // index in the run << 16 | run length (0: alone)
    const int nblk = max(grp & 0xffff, 1);
    const int g0 = item - (grp >> 16);
    const int local = task - g0 * A.nbn;
    const int nb = local / nblk;
    item = g0 + (local - nb * nblk);
    const F4Item it = A.items[item];
    const ExpertWork &ew = A.ew[it.a];
    const int K = A.K, O = A.O, nrow = it.nrow;
    const int jbase = ew.row0 + it.r0;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, t = lane & 15, q = lane >> 4;
    const int col0 = DUAL ? nb * 128 + wave * 16 : nb * 256 + wave * 32;
    const uint32_t rowb = (uint32_t)(K >> 1), srow = (uint32_t)(K >> 5);

    __amdgpu_buffer_rsrc_t rw[2], rs[2];
    uint32_t vw[2], vs[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
        const int mi = DUAL ? m : 2;
        const int trow = DUAL ? col0 : col0 + 16 * m;
        rw[m] = buf_rsrc(ew.w[mi], (uint32_t)O * rowb);
        rs[m] = buf_rsrc(ew.s[mi], (uint32_t)O * srow);
        vw[m] = (uint32_t)(trow + t) * rowb + 32u * (uint32_t)q;
        vs[m] = (uint32_t)(trow + t) * srow + 16u * (uint32_t)q;
    }
    auto load_b = [&] __attribute__((always_inline)) (F4Step &b, int k) {
#pragma unroll
        for (int m = 0; m < 2; ++m) {
#pragma unroll
            for (int s = 0; s < 2; ++s)
                b.w[m][s] = __builtin_bit_cast(
                    u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw[m], vw[m] + 16 * s,
                                                                 (uint32_t)k * 128u, 0));
        }
    };
    // the scale chunk holding step k, loaded only when step k opens it (otherwise the
    // offset lies past the buffer: zeros, no memory access, no branch around the load)
    auto load_s = [&] __attribute__((always_inline)) (F4Scl &sc, int k) {
        const bool open = (k & 7) == 0;
#pragma unroll
        for (int m = 0; m < 2; ++m)
            sc.c[m] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                           rs[m], open ? vs[m] + (uint32_t)(k >> 3) * 64u : 0xffffff00u, 0, 0));
    };

    // A codes of step k into LDS buffer buf straight from memory (buffer_load ... lds), no
    // staging registers.  DMA load i of wave w fills rows 8 (w BM / 64 + i) .. + 7 (lane l:
    // row + l / 8, physical chunk l % 8, which holds logical chunk (l % 8) ^ ((row / 2) %
    // 8)): the fragment reads of 16 rows then hit 16 distinct bank groups.  The item's
    // rows are one buffer resource: rows past nrow load as zeros (never stored).
    const __amdgpu_buffer_rsrc_t rac =
        buf_rsrc(A.acode + (size_t)jbase * rowb, (uint32_t)nrow * rowb);
    auto dma_a = [&] __attribute__((always_inline)) (int k, int buf) {
#pragma unroll
        for (int i = 0; i < BM / 64; ++i) {
            const int g = wave * (BM / 64) + i;
            const int r = 8 * g + (lane >> 3);
            const int lc = (lane & 7) ^ ((r >> 1) & 7);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rac, (__attribute__((address_space(3))) void *)(smem + buf * STAGE + g * 1024),
                16, (uint32_t)r * rowb + 16u * (uint32_t)lc, (uint32_t)k * 128u, 0, 0);
        }
    };
    // A scales: thread r < BM takes row r's 8 bytes of the step (the other threads'
    // offsets lie past the buffer: no memory access)
    const __amdgpu_buffer_rsrc_t ras =
        buf_rsrc(A.ascale + (size_t)jbase * srow, (uint32_t)nrow * srow);
    const uint32_t vas = tid < BM ? (uint32_t)tid * srow : 0xffffff00u;
    auto load_as = [&] __attribute__((always_inline)) (int k) {
        return __builtin_bit_cast(
            u32x2, __builtin_amdgcn_raw_buffer_load_b64(ras, vas, (uint32_t)k * 8u, 0));
    };
    auto store_as = [&] __attribute__((always_inline)) (u32x2 v, int buf) {
        if (tid < BM)
            *reinterpret_cast<u32x2 *>(smem + buf * STAGE + BM * kF4Row + 8 * tid) = v;
    };

    f4v acc[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
        acc[mt][0] = acc[mt][1] = f4v{0.f, 0.f, 0.f, 0.f};

    // this lane's LDS offsets in a stage: row t's chunk 2 q + s of the codes (swizzled; rows
    // 16 mt + t add 16 mt rows, which keep the swizzle), and its scale byte 2 q
    const int ao0 = t * kF4Row + 16 * ((2 * q) ^ ((t >> 1) & 7));
    const int ao1 = t * kF4Row + 16 * ((2 * q + 1) ^ ((t >> 1) & 7));
    const int so = BM * kF4Row + 8 * t + 2 * q;
    // step k (parity P = k % 2) on LDS buffer P: step k's 8 scale bytes of row t sit in
    // lane (t, (k % 8) / 2), words 2 P and 2 P + 1
    auto compute = [&] __attribute__((always_inline)) (const F4Step &b, const F4Scl &sc, int k,
                                                        auto par) {
        constexpr int P = decltype(par)::value;
        const char *base = smem + P * STAGE;
        const int src = 4 * (t + 16 * ((k & 7) >> 1));
        uint32_t sw[2][2];
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            sw[m][0] = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)sc.c[m][2 * P]);
            sw[m][1] = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)sc.c[m][2 * P + 1]);
        }
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            i32x8 bv[2];
            int sb[2];
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                const u32x4 w = b.w[m][s];
                bv[m] = i32x8{(int)w.x, (int)w.y, (int)w.z, (int)w.w, 0, 0, 0, 0};
                const int blk = 2 * q + s;  // this lane's 32-block among the step's 8
                const uint32_t word = q < 2 ? sw[m][0] : sw[m][1];
                sb[m] = (int)((word >> (8 * (blk & 3))) & 0xffu);
            }
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                // row tile mt: constant offsets from this lane's addresses (ds immediates)
                const u32x4 av = *reinterpret_cast<const u32x4 *>(base + (s ? ao1 : ao0) +
                                                                  mt * 16 * kF4Row);
                const i32x8 a8 = i32x8{(int)av.x, (int)av.y, (int)av.z, (int)av.w, 0, 0, 0, 0};
                const int sa = (int)(uint8_t)base[so + mt * 16 * 8 + s];
#pragma unroll
                for (int m = 0; m < 2; ++m)
                    acc[mt][m] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                        a8, bv[m], acc[mt][m], 4, 4, 0, sa, 0, sb[m]);
            }
        }
    };

    // pipeline as the bf16 grouped GEMM: weights NB steps ahead, activation codes one
    // step ahead (issued first: the barrier waits for them only), activation scales
    // staged one step ahead from registers loaded two steps ahead, weight-scale chunks two
    // steps ahead of the step that opens them; no branches around the loads; prefetches
    // past the last step read that step again
    // The step's MFMAs complete before the next loads of its weight registers are issued:
    // left free, the compiler sank them below the loads and the barrier and held three
    // sets of weight registers (the 128-row form then spilled).
    auto pin_acc = [&] __attribute__((always_inline)) () {
        if constexpr (MT >= 8)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int m = 0; m < 2; ++m)
                asm volatile("" : "+v"(acc[mt][m]));
    };
    const int nk = K / 256;
    F4Step b[NB];
    F4Scl sc, sn;  // scale chunk of this step / the next chunk
    u32x2 as[2];
    // Weight scale bytes the matrix cores read differently from the reference (0 and 255,
    // ue8m0_special), noted as each chunk opens: a wave that met one recomputes its
    // outputs element by element instead (below).
    uint32_t exc = 0;
    dma_a(0, 0);
    as[0] = load_as(0);
    load_b(b[0], 0);
    load_s(sn, 0);
    as[1] = load_as(min(1, nk - 1));
#pragma unroll
    for (int j = 1; j < NB; ++j)
        load_b(b[j], min(j, nk - 1));
    store_as(as[0], 0);
    __syncthreads();
    for (int k = 0; k < nk; k += UN) {
#pragma unroll
        for (int j = 0; j < UN; ++j) {  // step k + j: LDS buffer j % 2, weights b[j % NB]
            const int kk = k + j;
            if (j > 0 && kk >= nk)
                break;
            if (j % 2 == 0 && (kk & 7) == 0) {
                sc = sn;
                // this lane's 16 bytes of the chunk that lie in its row
                const int valid = (int)srow - 64 * (kk >> 3) - 16 * q;
#pragma unroll
                for (int m = 0; m < 2; ++m)
                    exc |= ue8m0_special(sc.c[m], valid);
            }
            dma_a(min(kk + 1, nk - 1), (j & 1) ^ 1);
            as[j & 1] = load_as(min(kk + 2, nk - 1));
            if (j & 1)
                compute(b[j % NB], sc, kk, std::integral_constant<int, 1>{});
            else
                compute(b[j % NB], sc, kk, std::integral_constant<int, 0>{});
            pin_acc();
            __builtin_amdgcn_sched_barrier(0);
            load_b(b[j % NB], min(kk + NB, nk - 1));
            if (j % 2 == 0)
                load_s(sn, min(kk + 2, nk - 1));
            store_as(as[(j & 1) ^ 1], (j & 1) ^ 1);
            __syncthreads();
        }
    }

    // Rare: a weight scale byte 0 or 255 among the wave's columns.  The wave computes its
    // outputs again element by element, as the composed reference does: x * (lut[n] *
    // scale) with the reference's scales (+0, +inf), products exact in f32, summed in K
    // order, so +-inf and NaN land where the reference puts them.  No barrier: the wave
    // reads the activation codes and the weights from memory.
    if (__builtin_amdgcn_ballot_w64(exc != 0) != 0) {
        const uint8_t *wc[2], *ws[2];
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            const int mi = DUAL ? m : 2;
            const size_t wrow = (size_t)((DUAL ? col0 : col0 + 16 * m) + t);
            wc[m] = static_cast<const uint8_t *>(ew.w[mi]) + wrow * rowb;
            ws[m] = static_cast<const uint8_t *>(ew.s[mi]) + wrow * srow;
        }
        for (int mt = 0; mt < MT; ++mt) {
            float sum[2][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
            for (int blk = 0; blk < (int)srow; ++blk) {
                u32x4 wv[2];
                float wsc[2];
#pragma unroll
                for (int m = 0; m < 2; ++m) {
                    wv[m] = *reinterpret_cast<const u32x4 *>(wc[m] + 16 * blk);
                    wsc[m] = ue8m0_ref(ws[m][blk]);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = min(mt * 16 + 4 * q + i, nrow - 1);
                    const u32x4 av = *reinterpret_cast<const u32x4 *>(
                        A.acode + (size_t)(jbase + r) * rowb + 16 * blk);
                    const float asc = ue8m0_ref(A.ascale[(size_t)(jbase + r) * srow + blk]);
                    for (int e = 0; e < 32; ++e) {
                        const float x = e2m1_val((av[e >> 3] >> (4 * (e & 7))) & 15u) * asc;
#pragma unroll
                        for (int m = 0; m < 2; ++m) {
                            const float w =
                                e2m1_val((wv[m][e >> 3] >> (4 * (e & 7))) & 15u) * wsc[m];
                            sum[m][i] += x * w;
                        }
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = mt * 16 + 4 * q + i;
                if (r >= nrow)
                    continue;
                const size_t j = (size_t)(jbase + r);
                if constexpr (DUAL) {
                    A.hout[j * O + col0 + t] = mf_act(A.act, sum[0][i], sum[1][i], A.act_a, A.act_b);
                } else {
                    A.out[j * O + col0 + t] = sum[0][i];
                    A.out[j * O + col0 + 16 + t] = sum[1][i];
                }
            }
        }
        return;
    }

#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = mt * 16 + 4 * q + i;
            if (r >= nrow)
                continue;
            const size_t j = (size_t)(jbase + r);
            if constexpr (DUAL) {
                A.hout[j * O + col0 + t] =
                    mf_act(A.act, acc[mt][0][i], acc[mt][1][i], A.act_a, A.act_b);
            } else {
                A.out[j * O + col0 + t] = acc[mt][0][i];
                A.out[j * O + col0 + 16 + t] = acc[mt][1][i];
            }
        }
    }
}

template <bool DUAL, int MT>
static hipError_t launch_f4_t(const F4Args &a, int n_items, hipStream_t st) {
    const size_t lds = fp4_lds_bytes(MT);
    auto kern = k_gemm_fp4<DUAL, MT>;
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess)
        return e;
    hipLaunchKernelGGL(kern, dim3((unsigned)(n_items * a.nbn)), dim3(kF4Threads), lds, st, a);
    return hipGetLastError();
}

hipError_t launch_gemm_fp4(bool dual, int mt, const ExpertWork *ew, const void *items,
                           int n_items, const uint8_t *acode, const uint8_t *ascale, float *hout,
                           float *out, int K, int O, int rcap, int act, float act_a, float act_b,
                           hipStream_t st, const int *n_items_dev) {
    if (n_items <= 0)
        return hipSuccess;
    if (K % 256 || O % (dual ? 128 : 256))
        return hipErrorInvalidValue;
    F4Args a{};
    a.n_items_dev = n_items_dev;
    a.ew = ew;
    a.items = static_cast<const F4Item *>(items);
    a.acode = acode;
    a.ascale = ascale;
    a.hout = hout;
    a.out = out;
    a.nbn = O / (dual ? 128 : 256);
    a.xcd = gemm_xcd() ? 1 : 0;
    a.K = K;
    a.O = O;
    a.rcap = rcap;
    a.act = act;
    a.act_a = act_a;
    a.act_b = act_b;
#define MVLLM_F4(D_)                                                                          \
    switch (mt) {                                                                             \
    case 4: return launch_f4_t<D_, 4>(a, n_items, st);                                        \
    case 8: return launch_f4_t<D_, 8>(a, n_items, st);                                        \
    case 16: return launch_f4_t<D_, 16>(a, n_items, st);                                      \
    default: return hipErrorInvalidValue;                                                     \
    }
    if (dual) {
        MVLLM_F4(true)
    }
    MVLLM_F4(false)
#undef MVLLM_F4
}

}  // namespace mvllm_hip
