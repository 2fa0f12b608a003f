// kern_wide.hip -- the heavy experts' grouped GEMM for MXFP4 weights and bf16
// activations (the 128-row class of the prefill path) with wide wave tiles: each wave
// accumulates 16 * MT rows x 16 * NT weight columns, so that every A fragment read from
// LDS feeds NT matrix-core products (v_mfma_f32_16x16x32_bf16) and every decoded B
// fragment MT of them.
//
// Task = (item: expert, block of <= 16 MT of its rows) x (column block: WAVES waves of
// NT weight tiles of 16 rows; the dual projection takes gate and up tiles at the same
// output columns, NT / 2 of each).  K advances 256 per step:
//   * A: the item's rows of the bf16 input planes go straight into LDS (buffer_load ...
//     lds, double buffered, one step ahead); rows are 512 bytes apart and a row's 16-byte
//     chunks are XOR-swizzled by a mask of the row's low four bits (wide_swz: conflict-free
//     fragment reads);
//   * weight scales: the step's 8 ue8m0 bytes of each of the workgroup's weight rows go
//     into LDS the same way (4-byte loads), next to the A tile;
//   * weights: each wave's tiles two steps ahead in registers.  Lane (t, q) of a tile
//     holds its row t's bytes [16 q, 16 q + 16) and [64 + 16 q, 64 + 16 q + 16) of the
//     step's 128: K elements [32 q, 32 q + 32) and [128 + 32 q, 160 + 32 q), the
//     32-blocks q and 4 + q.  MFMA step s (0..7) takes the lane's dword s, and the A
//     fragment is read at the same K elements (the K order only permutes the summation),
//     so no cross-lane shuffles are needed.
//   * decode: v_cvt_scalef32_pk_bf16_fp4 with the block's ue8m0 scale, exact for scale
//     bytes 2..252 (bf16(lut[n] * 2^(e-127))).  A wave that meets another byte computes
//     its outputs again element by element with the reference's scales (rare; below).
// The dual epilogue applies the activation and writes H as one bf16 plane (or f32), the
// format the down GEMMs read; the down form writes Y f32.
#include "mfma_common.h"

namespace mvllm_hip {

struct WideItem {
    int a, r0, nrow, pad;
};

struct WideArgs {
    const ExpertWork *ew;
    const WideItem *items;
    const int *n_items_dev;  // non-null: item count in device memory (grid sized for a bound)
    const __bf16 *pin;       // A plane [rcap][K] (one bf16 term, natural K order)
    __bf16 *pout;            // dual: H plane [rcap][O]
    float *out;              // single: Y [rcap][O]; dual: H f32 instead of the plane when set
    int n_tasks, nbn, K, O, rcap, xcd, act;
    float act_a, act_b;
};

constexpr int kWideBK = 256;

__host__ __device__ constexpr int wide_stage_bytes(int mt, int nt, int waves) {
    return 16 * mt * kWideBK * 2 + waves * nt * 16 * 8;
}

// XOR mask of a row's 16-byte chunks in LDS (t = the row's low four bits): 2 (t mod 8) +
// t / 8.  With it the fragment reads (lane 16 q + t reads row t's chunk 4 q + s) run at
// the LDS's full read rate in a microbenchmark of this access pattern; XOR by t itself
// ran them 1.7 x slower (the kernel's time did not change: its LDS reads are not what
// bounds it).
__device__ __forceinline__ uint32_t wide_swz(uint32_t t) { return ((t & 7u) << 1) | (t >> 3); }

template <bool DUAL, int MT, int NT, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void k_gemm_wide(WideArgs A) {
    // A fragments read this many row tiles ahead (2: 1 % slower; the compiler's
    // interleaving of reads, MFMAs and decode by sched_group_barrier: no faster)
    constexpr int PD = 4;
    constexpr int BM = 16 * MT;
    constexpr int HT = DUAL ? NT / 2 : NT;  // output tiles of 16 columns per wave
    constexpr int ABYTES = BM * kWideBK * 2;
    constexpr int STAGE = wide_stage_bytes(MT, NT, WAVES);
    constexpr int ADMA = BM / 2 / WAVES;  // A DMA loads per wave and step (two rows each)
    static_assert(BM % (2 * WAVES) == 0 && NT % 2 == 0 && HT % 2 == 0, "tile split");
    extern __shared__ __attribute__((aligned(16))) char smem[];

    const int n_tasks =
        A.n_items_dev ? __builtin_amdgcn_readfirstlane(*A.n_items_dev) * A.nbn : A.n_tasks;
    if ((int)blockIdx.x >= n_tasks)
        return;
    const int task = A.xcd ? xcd_task(blockIdx.x, n_tasks) : (int)blockIdx.x;
    // (row block by row block: ordering an expert's tasks column block by column block, so
    // that its row blocks share each column block's weights in L2, measured no faster)
    const int item = task / A.nbn, nb = task - item * A.nbn;
    const WideItem it = A.items[item];
    const ExpertWork &ew = A.ew[it.a];
    const int K = A.K, O = A.O, nrow = it.nrow, jbase = ew.row0 + it.r0;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, t = lane & 15, q = lane >> 4;
    const uint32_t rowb = (uint32_t)(K >> 1), srow = (uint32_t)(K >> 5);
    const int nk = K / kWideBK;
    const int col0 = (nb * WAVES + wave) * 16 * HT;  // the wave's first output column
    // tile m: matrix (gate / up for the dual form, down otherwise) and its first row
    auto tmat = [](int m) { return DUAL ? m / HT : 0; };
    auto trow = [](int m) { return 16 * (DUAL ? m % HT : m); };  // + col0

    constexpr int NMAT = DUAL ? 2 : 1;
    __amdgpu_buffer_rsrc_t rw[NMAT], rs[NMAT];
#pragma unroll
    for (int mi = 0; mi < NMAT; ++mi) {
        rw[mi] = buf_rsrc(ew.w[DUAL ? mi : 2], (uint32_t)O * rowb);
        rs[mi] = buf_rsrc(ew.s[DUAL ? mi : 2], (uint32_t)O * srow);
    }
    // lane's weight bytes of tile 0 (other tiles: + 16 rows each, in the scalar offset)
    const uint32_t vw = (uint32_t)(col0 + t) * rowb + 16u * (uint32_t)q;

    struct WB {
        u32x4 w[NT][2];
    };
    // half h (bytes [64 h + 16 q, 64 h + 16 q + 16) of each tile row's 128) of step k
    auto load_bh = [&] __attribute__((always_inline)) (WB &b, int k, int h) {
#pragma unroll
        for (int m = 0; m < NT; ++m)
            b.w[m][h] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                           rw[tmat(m)], vw + 64u * (uint32_t)h,
                           (uint32_t)k * 128u + (uint32_t)trow(m) * rowb, 0));
    };

    // A of step k into LDS buffer buf.  DMA load i of wave w fills the two rows
    // r0 = 16 (i / R) + 2 w + 2 WAVES (i % R) and r0 + 1 (R = 8 / WAVES; lane l: row r0 + l / 32,
    // physical chunk l % 32, which holds logical chunk (l % 32) ^ wide_swz(row % 16)).  A lane's
    // rows then share row % 16 across its loads, so its offsets differ by scalars only.
    // Rows past nrow lie beyond the buffer: zeros.
    constexpr int R = 8 / WAVES;
    static_assert(ADMA % R == 0, "A DMA residues");
    const __amdgpu_buffer_rsrc_t ra =
        buf_rsrc(A.pin + (size_t)jbase * (size_t)K, (uint32_t)nrow * (uint32_t)K * 2u);
    // (two scalars, not an array: the host pass drops the kernel's stub when the builtin's
    // offset comes from a captured array)
    auto va_of = [&](int j) {
        const int r = 2 * wave + 2 * WAVES * j + (lane >> 5);
        return (uint32_t)r * (uint32_t)K * 2u +
               16u * ((uint32_t)(lane & 31) ^ wide_swz((uint32_t)(r & 15)));
    };
    const uint32_t va0 = va_of(0), va1 = R > 1 ? va_of(1) : 0u;
    auto dma_a = [&] __attribute__((always_inline)) (int k, int buf) {
#pragma unroll
        for (int i = 0; i < ADMA; ++i) {
            const int r0 = 16 * (i / R) + 2 * wave + 2 * WAVES * (i % R);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                ra, (__attribute__((address_space(3))) void *)(smem + buf * STAGE + r0 * 512), 16,
                (i % R) ? va1 : va0,
                (uint32_t)k * (uint32_t)(kWideBK * 2) + (uint32_t)(16 * (i / R)) * (uint32_t)K * 2u,
                0, 0);
        }
    };
    // weight scales of step k into LDS after the A tile: (wave, tile m, row t) at
    // ((wave NT + m) 16 + t) 8, the step's 8 bytes.  DMA load i covers tiles 2 i and 2 i + 1
    // (lane l: tile 2 i + l / 32, row (l / 2) % 16, dword l % 2); both lie in one matrix.
    const uint32_t vs = (uint32_t)(col0 + 16 * (lane >> 5) + ((lane >> 1) & 15)) * srow +
                        4u * (uint32_t)(lane & 1);
    auto dma_s = [&] __attribute__((always_inline)) (int k, int buf) {
#pragma unroll
        for (int i = 0; i < NT / 2; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rs[tmat(2 * i)],
                (__attribute__((address_space(3))) void *)(smem + buf * STAGE + ABYTES +
                                                          (wave * NT + 2 * i) * 128),
                4, vs + (uint32_t)trow(2 * i) * srow, (uint32_t)k * 8u, 0, 0);
    };

    f4v acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int m = 0; m < NT; ++m)
            acc[mt][m] = f4v{0.f, 0.f, 0.f, 0.f};
    // a scale byte the folded bf16 decode does not reproduce (b7_exceptional)
    uint32_t exc = 0;

    // LDS byte offsets of this lane: A row t's chunk for MFMA step s is
    // abase ^ (256 (s / 4) + 16 (s % 4)) (row tile mt: + mt 8192), its scales sbase (+ 128 m)
    const uint32_t abase = (uint32_t)t * 512u + 16u * ((uint32_t)(4 * q) ^ wide_swz((uint32_t)t));
    const uint32_t sbase = (uint32_t)ABYTES + ((uint32_t)wave * NT * 16u + (uint32_t)t) * 8u;
    // scales of the lane's block (q for h = 0, 4 + q for h = 1) of every tile
    auto read_sc = [&] __attribute__((always_inline)) (const char *base, int h, float (&sc)[NT]) {
#pragma unroll
        for (int m = 0; m < NT; ++m) {
            const uint32_t w = *reinterpret_cast<const uint32_t *>(base + sbase + 128 * m + 4 * h);
            sc[m] = __uint_as_float(((w >> (8 * q)) & 0xffu) << 23);
            exc |= (uint32_t)b7_exceptional(sc[m]);
        }
    };
    auto read_a = [&] __attribute__((always_inline)) (const char *base, int s, int mt) {
        const uint32_t off = abase ^ (uint32_t)(256 * (s >> 2) + 16 * (s & 3));
        return *reinterpret_cast<const bf16x8 *>(base + off + mt * 8192);
    };
    // Step k from LDS buffer buf and the weights in b; the weights of step k + 1 are loaded
    // into b half by half as soon as the decode has consumed a half (kn = its step index).
    // Each MFMA step decodes the next step's weights and reads the A fragment two row tiles
    // ahead, so that the LDS latency and the decode run under the matrix-core work.
    auto compute = [&] __attribute__((always_inline)) (WB &b, int buf, int kn) {
        const char *base = smem + buf * STAGE;
        float sc[NT];
        read_sc(base, 0, sc);
        bf16x8 bd[NT];
#pragma unroll
        for (int m = 0; m < NT; ++m)
            bd[m] = decode_b<7>(b.w[m][0][0], sc[m]);
        bf16x8 ap[PD];
#pragma unroll
        for (int i = 0; i < PD; ++i)
            ap[i] = read_a(base, 0, i);
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            bf16x8 bn[NT];
            if (s == 3)
                read_sc(base, 1, sc);  // blocks 4 + q from MFMA step 4 on
            if (s < 7) {
#pragma unroll
                for (int m = 0; m < NT; ++m)
                    bn[m] = decode_b<7>(b.w[m][(s + 1) >> 2][(s + 1) & 3], sc[m]);
            }
            if (s == 3)
                load_bh(b, kn, 0);  // half 0 fully decoded
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                // the A fragment PD positions ahead in (s, mt) order
                const int mt2 = mt + PD < MT ? mt + PD : mt + PD - MT;
                const int s2 = mt + PD < MT ? s : s + 1;
                bf16x8 an = ap[0];
                if (s2 < 8)
                    an = read_a(base, s2, mt2);
#pragma unroll
                for (int m = 0; m < NT; ++m)
                    acc[mt][m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ap[0], bd[m], acc[mt][m],
                                                                         0, 0, 0);
#pragma unroll
                for (int i = 0; i + 1 < PD; ++i)
                    ap[i] = ap[i + 1];
                ap[PD - 1] = an;
            }
            if (s < 7) {
#pragma unroll
                for (int m = 0; m < NT; ++m)
                    bd[m] = bn[m];
            }
            // keep each MFMA step's work in its place (register pressure)
            __builtin_amdgcn_sched_barrier(0);
        }
        load_bh(b, kn, 1);  // half 1 fully decoded
    };

    // A and the scales one step ahead into the other LDS buffer, issued first so that the
    // barrier ending the step waits for them and not for the weights behind them.
    // Prefetches past the last step read that step again (never consumed).
    WB b;
    dma_a(0, 0);
    dma_s(0, 0);
    load_bh(b, 0, 0);
    load_bh(b, 0, 1);
    __syncthreads();
    auto step = [&] __attribute__((always_inline)) (int k, int buf) {
        dma_a(min(k + 1, nk - 1), buf ^ 1);
        dma_s(min(k + 1, nk - 1), buf ^ 1);
        compute(b, buf, min(k + 1, nk - 1));
        __syncthreads();
    };
    for (int k = 0; k + 2 <= nk; k += 2) {
        step(k, 0);
        step(k + 1, 1);
    }
    if (nk & 1)
        step(nk - 1, 0);

    // Rare: a scale byte outside 2..252 among the wave's weights.  The wave computes its
    // outputs again element by element: the bf16 activation times lut[n] * scale with the
    // reference's scales (e = 0: +0, e = 255: +inf), products exact in f32, summed in K
    // order.  No barrier: everything is read from memory.
    if (__builtin_amdgcn_ballot_w64(exc != 0) != 0) {
        for (int mt = 0; mt < MT; ++mt) {
            float sum[NT][4];
#pragma unroll
            for (int m = 0; m < NT; ++m)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    sum[m][i] = 0.f;
            for (int blk = 0; blk < (int)srow; ++blk) {
                u32x4 wv[NT];
                float wsc[NT];
#pragma unroll
                for (int m = 0; m < NT; ++m) {
                    const size_t wr = (size_t)(col0 + trow(m) + t);
                    wv[m] = *reinterpret_cast<const u32x4 *>(
                        static_cast<const uint8_t *>(ew.w[DUAL ? tmat(m) : 2]) + wr * rowb +
                        16 * blk);
                    wsc[m] = ue8m0_ref(static_cast<const uint8_t *>(
                        ew.s[DUAL ? tmat(m) : 2])[wr * srow + blk]);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = min(mt * 16 + 4 * q + i, nrow - 1);
                    const __bf16 *xr = A.pin + (size_t)(jbase + r) * (size_t)K + 32 * blk;
                    for (int e = 0; e < 32; ++e) {
                        const float x = (float)xr[e];
#pragma unroll
                        for (int m = 0; m < NT; ++m)
                            sum[m][i] +=
                                x * (e2m1_val((wv[m][e >> 3] >> (4 * (e & 7))) & 15u) * wsc[m]);
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = mt * 16 + 4 * q + i;
                if (r >= nrow)
                    continue;
                const size_t j = (size_t)(jbase + r);
#pragma unroll
                for (int m = 0; m < HT; ++m) {
                    const int col = col0 + 16 * m + t;
                    if constexpr (DUAL) {
                        const float h = mf_act(A.act, sum[m][i], sum[m + HT][i], A.act_a, A.act_b);
                        if (A.out)
                            A.out[j * O + col] = h;
                        else
                            A.pout[j * O + col] = (__bf16)h;
                    } else {
                        A.out[j * O + col] = sum[m][i];
                    }
                }
            }
        }
        return;
    }

    // C[4 q + i][t] of row tile mt and tile m
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = mt * 16 + 4 * q + i;
            if (r >= nrow)
                continue;
            const size_t j = (size_t)(jbase + r);
#pragma unroll
            for (int m = 0; m < HT; ++m) {
                const int col = col0 + 16 * m + t;
                if constexpr (DUAL) {
                    const float h = mf_act(A.act, acc[mt][m][i], acc[mt][m + HT][i], A.act_a,
                                           A.act_b);
                    if (A.out)
                        A.out[j * O + col] = h;
                    else
                        A.pout[j * O + col] = (__bf16)h;
                } else {
                    A.out[j * O + col] = acc[mt][m][i];
                }
            }
        }
}

// ---- launcher -----------------------------------------------------------------------

static int g_wide = 1;  // option "gemm_wide": 1 on, 0 off (the grouped GEMM's 128-row class)
void gemm_set_wide(int v) { g_wide = v; }
int gemm_wide() { return g_wide; }

template <bool DUAL, int MT, int NT, int WAVES>
static hipError_t launch_wide_t(WideArgs a, int n_items, hipStream_t st) {
    const size_t lds = 2 * (size_t)wide_stage_bytes(MT, NT, WAVES);
    auto kern = k_gemm_wide<DUAL, MT, NT, WAVES>;
    static bool attr = false;  // the dynamic LDS limit, raised once per process
    if (!attr) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess)
            return e;
        attr = true;
    }
    a.nbn = a.O / (16 * (DUAL ? NT / 2 : NT) * WAVES);
    a.n_tasks = n_items * a.nbn;
    hipLaunchKernelGGL(kern, dim3((unsigned)a.n_tasks), dim3(64 * WAVES), lds, st, a);
    return hipGetLastError();
}

// Column block of one task: 256 output columns of the dual form, 512 of the down form.
bool gemm_wide_fits(bool dual, int K, int O) {
    return g_wide != 0 && K % kWideBK == 0 && O % (dual ? 256 : 512) == 0;
}

hipError_t launch_gemm_wide(bool dual, const ExpertWork *ew, const void *items, int n_items,
                            const void *pin, void *pout, float *out, int K, int O, int rcap,
                            int act, float act_a, float act_b, hipStream_t st,
                            const int *n_items_dev) {
    if (n_items <= 0)
        return hipSuccess;
    if (!gemm_wide_fits(dual, K, O))
        return hipErrorInvalidValue;
    WideArgs a{};
    a.ew = ew;
    a.items = static_cast<const WideItem *>(items);
    a.n_items_dev = n_items_dev;
    a.pin = static_cast<const __bf16 *>(pin);
    a.pout = static_cast<__bf16 *>(pout);
    a.out = out;
    a.K = K;
    a.O = O;
    a.rcap = rcap;
    a.xcd = gemm_xcd() ? 1 : 0;
    a.act = act;
    a.act_a = act_a;
    a.act_b = act_b;
    // eight waves of 128 rows x 4 tiles (two per SIMD); four waves of 128 x 8 tiles, one
    // per SIMD with 256 accumulators each, measured 10 % slower (c4 3.05 -> 3.37 ms)
    return dual ? launch_wide_t<true, 8, 4, 8>(a, n_items, st)
                : launch_wide_t<false, 8, 4, 8>(a, n_items, st);
}

}  // namespace mvllm_hip
