// kern_gemm.hip -- prefill-shaped expert GEMMs on the gfx950 matrix cores: a grouped
// GEMM over token-sorted expert segments (v_mfma_f32_16x16x32_bf16).
//
// Work item = (expert, block of up to 16 * MT of its rows) x (block of output columns).
// A workgroup of 8 waves streams K in steps of 256:
//   * activations (A): the item's rows of the bf16 input planes [TERMS][rcap][K] are
//     staged into LDS, double buffered, by all 512 threads (16-byte loads);
//   * weights (B): each wave owns two 16-column tiles (gate and up at the same columns
//     for the dual projection, two adjacent tiles of the down matrix otherwise) and
//     reads their packed rows with coalesced 8-byte loads (lane l -> row l / 4, 32 B
//     per row per load) two steps ahead, moves them into the operand layout with
//     ds_bpermute and decodes them exactly in registers; the tiles' scales come once per
//     pair of steps and are handed out the same way;
//   * each decoded B fragment feeds MT row tiles (one A fragment read per two MFMAs).
// int4: nibble n decodes to bf16(n - 8) exactly (signed e4m3 codes through the
// converter), every 64-wide group is its own chain from 0, and one f32 FMA applies the
// group's f32 scale (exact (n - 8) * scale, no rounding of the product to bf16).
// MXFP4: the ue8m0 scale is folded into the bf16 decode (exact for bytes 2..252).  Other
// operands (MXFP4 bytes outside that range, non-finite int4 scales) send the task
// through a second pass with the per-element exact decode.
// The dual epilogue applies the activation and writes H in the same plane format that
// the down kernel reads.
#include "mfma_common.h"

#include <algorithm>
#include <type_traits>

namespace mvllm_hip {


struct GemmItem {
    int a;     // expert index into ExpertWork
    int r0;    // first row within the expert's compact rows
    int nrow;  // rows in this item (<= 16 * MT)
    int pad;
};

struct GemmArgs {
    const ExpertWork *ew;
    const GemmItem *items;  // per item (UNI kernels: none; one expert ew1 over nrows_all rows)
    ExpertWork ew1;
    int nrows_all;
    const __bf16 *pin;  // A planes [TERMS][rcap][K] (int4: 8-blocks in slot order)
    __bf16 *pout;       // dual: H planes [TERMS][rcap][O]
    float *out;         // single: Y [rcap][O] f32; dual: H [rcap][O] f32 instead of planes
                        // when set (the native-MXFP4 call quantizes H afterwards)
    int nbn;            // column blocks per item
    int n_tasks;        // items * nbn
    const int *n_items_dev;  // non-null: the item count is in device memory (a grid sized
                             // for its bound; workgroups past items * nbn exit)
    int xcd;            // 1: tasks ordered per XCD (xcd_task), 0: task = workgroup index
    int K, O, rcap;
    int act;
    float act_a, act_b;
};

constexpr int kGemmThreads = 512;
constexpr int kGemmBK = 256;
constexpr int kGemmPitch = kGemmBK * 2 + 16;  // LDS bytes per A row and plane (+16: banks)

__host__ __device__ constexpr int gemm_stage_bytes(int fmt, int terms, int mt) {
    return (void)fmt, terms * 16 * mt * kGemmPitch;
}

size_t gemm_lds_bytes(int fmt, int terms, int mt) {
    return 2 * (size_t)gemm_stage_bytes(fmt, terms, mt);
}

// Packed weights of one K step for the wave's two tiles, as loaded.
template <int FMT>
struct GStep {
    u32x2 w[2][4];
};

// Scales of one pair of K steps (p = k / 2) for the wave's two tiles, as loaded, each
// scale once: lane 4 r + c holds row r's int4 group scales 8 p + 2 c and 8 p + 2 c + 1,
// or its MXFP4 block scale bytes 16 p + 4 c .. 16 p + 4 c + 3.  The compute hands them
// to the lanes of row r with ds_bpermute.  (Loading each step's scales into every lane of
// the row took two more 16-row loads per step and their registers; the loop ran 20 %
// slower for it.)
template <int FMT>
struct GScale {
    u32x2 s4[FMT == 4 ? 2 : 1];
    uint32_t s7[FMT == 7 ? 2 : 1];
};

// Scales in chunks of 64 bytes of each row (MXFP4: four pairs of steps, int4: two): lane
// 4 r + c holds bytes 64 C + 16 c .. + 15 of row r, i.e. MXFP4 pair 4 C + c whole, or
// int4 groups 16 C + 4 c .. + 3.  One load per chunk instead of per pair: a row's scale
// line is fetched from HBM about twice, where per-pair loads far apart in time fetched it
// again after each L2 eviction (the small-expert classes read ~25 % more than their
// weights and scales).
struct GScaleC {
    u32x4 c[2];
};
// pairs of K steps per scale chunk
template <int FMT>
__host__ __device__ constexpr int gscale_ppc() { return FMT == 7 ? 4 : 2; }

// Where one task's operands live: its two weight tiles (buffer resources + this lane's
// offsets), its activation rows and its output columns.
template <int FMT>
struct TaskD {
    __amdgpu_buffer_rsrc_t rw[2], rs[2];
    uint32_t vw[2], vs[2];
    int jbase, nrow, col0;
};

// One workgroup per task.  UNI: one expert (A.ew1) over rows [0, A.nrows_all) in blocks of
// BM, no item list (dense linears; a template parameter so that the selection costs the
// grouped form no registers).  The 32-row class with one term is held to 128 VGPRs (4 waves
// per SIMD), so two workgroups share a CU: the grouped form needs 110-120 (its A tiles go
// straight into LDS), the dense-linear form 126-131, where the cap costs at most a few
// spilled registers (c3 with register-staged A tiles: 1.60 -> 1.53 ms per call).
template <int FMT, bool DUAL, int TERMS, int MT, bool UNI>
__global__ __launch_bounds__(kGemmThreads)
__attribute__((amdgpu_waves_per_eu(MT == 2 && TERMS == 1 ? 4 : 1, 8))) void k_gemm(GemmArgs A) {
    // scales in 64-byte chunks (GScaleC) where the registers allow (not the MXFP4 down
    // kernel of the 32-row class: it would pass its 128-VGPR cap and spill)
    constexpr bool kChunkS = !UNI && TERMS == 1 && MT <= 4 && !(FMT == 7 && !DUAL && MT == 2);
    constexpr int PPC = gscale_ppc<FMT>();
    using Scl = std::conditional_t<kChunkS, GScaleC, GScale<FMT>>;
    constexpr int BM = 16 * MT;
    constexpr int PA = MT >= 8 ? 1 : 2;  // activation prefetch distance in K steps
    // The one-term classes load their A tiles straight into LDS (buffer_load ... lds): no
    // staging registers.  Rows are then 512 bytes apart without padding, and a row's
    // 16-byte chunks are XOR-swizzled by the row's low four bits, which keeps the fragment
    // reads free of bank conflicts (the padded layout staged through registers spent
    // 14-20 % of the 16/32/64-row classes' CU cycles in LDS bank conflicts).
    constexpr bool kDmaA = TERMS == 1 && !UNI;
    constexpr int APITCH = kDmaA ? kGemmBK * 2 : kGemmPitch;  // LDS bytes per A row
    constexpr int PL = BM * APITCH;                  // bytes per plane per stage
    constexpr int STAGE = kDmaA ? TERMS * PL : gemm_stage_bytes(FMT, TERMS, MT);
    constexpr int ACH = TERMS * BM * (kGemmBK / 8) / kGemmThreads;  // 16-byte chunks/thread
    // Row tiles' A fragments read one tile ahead where registers allow (the one-workgroup
    // classes: their MFMAs otherwise wait out each tile's LDS latency)
    constexpr bool kPipeA = MT >= 4 && TERMS == 1;
    // the next group's weight shuffles ahead of this group's MFMAs (same classes)
    constexpr bool kPipeB = MT >= 4 && TERMS == 1;
    static_assert(ACH * kGemmThreads == TERMS * BM * (kGemmBK / 8), "A staging split");
    extern __shared__ __attribute__((aligned(16))) char smem[];

    const int K = A.K, O = A.O, rcap = A.rcap;
    const int n_tasks =
        A.n_items_dev ? __builtin_amdgcn_readfirstlane(*A.n_items_dev) * A.nbn : A.n_tasks;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, t = lane & 15, q = lane >> 4;
    const uint32_t rowb = (uint32_t)(K >> 1);
    const uint32_t srow = (uint32_t)(FMT == 4 ? (K / 64) * 4 : K / 32);
    const int nk = K / kGemmBK;

    auto make_task = [&] __attribute__((always_inline)) (int task) {
        TaskD<FMT> d;
        int item = task / A.nbn;
        int nb = task - item * A.nbn;
        if constexpr (!UNI && MT <= 2) {
            // An expert's run of nblk items owns tasks [g0 nbn, (g0 + nblk) nbn); they go
            // column block by column block, its row blocks adjacent, so that the row blocks
            // running side by side on one XCD read that column block's weights through its
            // L2 together (item word 3: index in the run << 16 | run length, 0: alone).
            const int grp = A.items[item].pad;
            const int nblk = max(grp & 0xffff, 1);
            const int g0 = item - (grp >> 16);
            const int local = task - g0 * A.nbn;
            nb = local / nblk;
            item = g0 + (local - nb * nblk);
        }
        GemmItem it;
        if constexpr (UNI) {
            it.a = 0;
            it.r0 = item * BM;
            it.nrow = min(BM, A.nrows_all - it.r0);
        } else {
            it = A.items[item];
        }
        const ExpertWork &ew = UNI ? A.ew1 : A.ew[it.a];
        d.jbase = ew.row0 + it.r0;
        d.nrow = it.nrow;
        d.col0 = DUAL ? nb * 128 + wave * 16 : nb * 256 + wave * 32;
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            const int mi = DUAL ? m : 2;
            const int trow = DUAL ? d.col0 : d.col0 + 16 * m;  // first weight row of tile m
            d.rw[m] = buf_rsrc(ew.w[mi], (uint32_t)O * rowb);
            d.rs[m] = buf_rsrc(ew.s[mi], (uint32_t)O * srow);
            d.vw[m] = (uint32_t)(trow + (lane >> 2)) * rowb + 8u * (uint32_t)(lane & 3);
            d.vs[m] = (uint32_t)(trow + (lane >> 2)) * srow +
                      (kChunkS ? 16u : FMT == 4 ? 8u : 4u) * (uint32_t)(lane & 3);
        }
        return d;
    };

    auto load_b = [&] __attribute__((always_inline)) (GStep<FMT> &b, const TaskD<FMT> &d, int k) {
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
            for (int g = 0; g < 4; ++g)
                b.w[m][g] = __builtin_bit_cast(
                    u32x2, __builtin_amdgcn_raw_buffer_load_b64(d.rw[m], d.vw[m] + 32 * g,
                                                                (uint32_t)k * 128u, 0));
    };
    // scales of the pair holding step k; chunked: the chunk holding step k, loaded only
    // when step k opens the chunk (otherwise the offset lies past the buffer, which loads
    // zeros without touching memory and keeps the body free of branches)
    auto load_s = [&] __attribute__((always_inline)) (Scl &s, const TaskD<FMT> &d, int k) {
        if constexpr (kChunkS) {
            const bool open = ((k >> 1) % PPC) == 0;
            const uint32_t off = (uint32_t)((k >> 1) / PPC) * 64u;
#pragma unroll
            for (int m = 0; m < 2; ++m)
                s.c[m] = __builtin_bit_cast(
                    u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                               d.rs[m], open ? d.vs[m] + off : 0xffffff00u, 0, 0));
        } else {
            const uint32_t off = (uint32_t)(k >> 1) * (FMT == 4 ? 32u : 16u);
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                if constexpr (FMT == 4)
                    s.s4[m] = __builtin_bit_cast(
                        u32x2, __builtin_amdgcn_raw_buffer_load_b64(d.rs[m], d.vs[m], off, 0));
                else
                    s.s7[m] = __builtin_amdgcn_raw_buffer_load_b32(d.rs[m], d.vs[m], off, 0);
            }
        }
    };

    // Set when the fast decode would not reproduce the reference for this task: an MXFP4
    // scale byte outside the range where the folded bf16 decode is exact
    // (b7_exceptional), or a non-finite int4 scale (applied to the whole group's sum, where
    // the reference forms each product (n - 8) * scale).  The task is then computed again
    // with the exact decode.
    uint32_t exc = 0;

    // A staging: chunk c = u * 512 + tid -> plane c / (BM * 32), row (c / 32) % BM,
    // 16-byte column c % 32 of the step.  Two register sets let the loads of step k + 2
    // be issued while step k computes (PA = 2), so their latency spans two steps.
    struct AStage {
        u32x4 v[ACH];  // native vectors: copies of HIP's uint4 struct go through scratch
    };
    auto load_a = [&] __attribute__((always_inline)) (AStage &ra, const TaskD<FMT> &d, int k) {
        // unconditional loads (rows past nrow re-read the last row; their results are
        // never stored) keep the loop body free of branches
#pragma unroll
        for (int u = 0; u < ACH; ++u) {
            const int c = u * kGemmThreads + tid;
            const int tm = c / (BM * 32), r = min((c >> 5) % BM, d.nrow - 1), cc = c & 31;
            ra.v[u] = *reinterpret_cast<const u32x4 *>(
                A.pin + ((size_t)tm * rcap + d.jbase + r) * (size_t)K + (size_t)k * kGemmBK +
                8 * cc);
        }
    };
    auto store_a = [&] __attribute__((always_inline)) (const AStage &ra, int buf) {
        char *base = smem + buf * STAGE;
#pragma unroll
        for (int u = 0; u < ACH; ++u) {
            const int c = u * kGemmThreads + tid;
            const int tm = c / (BM * 32), r = (c >> 5) % BM, cc = c & 31;
            *reinterpret_cast<u32x4 *>(base + tm * PL + r * kGemmPitch + cc * 16) = ra.v[u];
        }
    };

    // kDmaA: the A tile of step k into LDS buffer buf.  DMA load i of wave w fills LDS rows
    // (BM / 8) w + 2 i and + 1 (lane l: row + l / 32, physical chunk l % 32, which holds
    // logical chunk (l % 32) ^ (row % 16)).  The item's rows are one buffer resource: rows past
    // nrow lie beyond it and load as zeros (their results are never stored).
    auto dma_a = [&] __attribute__((always_inline)) (const TaskD<FMT> &d, int k, int buf) {
        if constexpr (kDmaA) {
            const __amdgpu_buffer_rsrc_t ra =
                buf_rsrc(A.pin + (size_t)d.jbase * (size_t)K, (uint32_t)d.nrow * (uint32_t)K * 2u);
            const int dr = lane >> 5, pc = lane & 31;
#pragma unroll
            for (int i = 0; i < BM * APITCH / 1024 / 8; ++i) {
                const int r = (BM / 8) * wave + 2 * i + dr;
                const int lc = pc ^ (r & 15);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    ra,
                    (__attribute__((address_space(3))) void *)(smem + buf * STAGE +
                                                              ((BM / 16) * wave + i) * 1024),
                    16, (uint32_t)r * (uint32_t)K * 2u + 16u * (uint32_t)lc,
                    (uint32_t)k * (uint32_t)(kGemmBK * 2), 0, 0);
            }
        }
    };

    f4v acc[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
        acc[mt][0] = acc[mt][1] = f4v{0.f, 0.f, 0.f, 0.f};
    const int src4 = 4 * (4 * t + q);  // ds_bpermute address of lane 4 t + q


    // step j (0 or 1) of pair p, whose scales are in sc
    auto compute1 = [&] __attribute__((always_inline)) (const GStep<FMT> &b, int buf,
                                                         const Scl &sc, int p, int j, auto exact) {
        constexpr bool EXACT = decltype(exact)::value;
        const char *base = smem + buf * STAGE;
        // scale words of step j, groups 0-1 / 2-3, sit in lanes 4 t + 2 j and 4 t + 2 j + 1;
        // chunked: MXFP4 pair p in lane 4 t + p % 4 (word 2 j + g / 2), int4 groups of step
        // j in lane 4 t + 2 (p % 2) + j (component g)
        const int ssrc = kChunkS ? (FMT == 7 ? 4 * (4 * t + p % PPC) : 4 * (4 * t + 2 * (p % PPC) + j))
                                 : 4 * (4 * t + 2 * j);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            bf16x8 bf[2][2];
            float sg[2];
            bool spec[2] = {false, false};  // EXACT int4: this lane's column scale is not finite
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                const uint32_t wx = (uint32_t)__builtin_amdgcn_ds_bpermute(src4, (int)b.w[m][g].x);
                const uint32_t wy = (uint32_t)__builtin_amdgcn_ds_bpermute(src4, (int)b.w[m][g].y);
                if constexpr (kChunkS && FMT == 4) {
                    sg[m] = __uint_as_float(
                        (uint32_t)__builtin_amdgcn_ds_bpermute(ssrc, (int)sc.c[m][g]));
                } else if constexpr (kChunkS) {
                    const uint32_t word = (uint32_t)__builtin_amdgcn_ds_bpermute(
                        ssrc, (int)sc.c[m][2 * j + (g >> 1)]);
                    const int byte = 2 * (g & 1) + (q >> 1);
                    sg[m] = __uint_as_float(((word >> (8 * byte)) & 0xffu) << 23);
                } else if constexpr (FMT == 4) {
                    sg[m] = __uint_as_float((uint32_t)__builtin_amdgcn_ds_bpermute(
                        ssrc + 4 * (g >> 1), (int)((g & 1) ? sc.s4[m].y : sc.s4[m].x)));
                } else {  // lanes q < 2 take 32-block 2 g, q >= 2 block 2 g + 1
                    const uint32_t word =
                        (uint32_t)__builtin_amdgcn_ds_bpermute(ssrc + 4 * (g >> 1), (int)sc.s7[m]);
                    const int byte = 2 * (g & 1) + (q >> 1);
                    sg[m] = __uint_as_float(((word >> (8 * byte)) & 0xffu) << 23);
                }
                if constexpr (FMT == 7 && EXACT) {
                    bf[m][0] = decode_b7_exact(wx, sg[m]);
                    bf[m][1] = decode_b7_exact(wy, sg[m]);
                } else if constexpr (FMT == 4) {
                    bf[m][0] = decode_b4_signed(wx);
                    bf[m][1] = decode_b4_signed(wy);
                    if constexpr (EXACT) {
                        // the reference's x * ((n - 8) * scale): a non-finite scale enters
                        // each product, which then takes the high term of x alone (its
                        // low terms would turn inf * 0 into NaN)
                        spec[m] = nonfinite(sg[m]);
                        if (spec[m]) {
                            bf[m][0] = mul_bf16x8_exact(bf[m][0], sg[m]);
                            bf[m][1] = mul_bf16x8_exact(bf[m][1], sg[m]);
                        }
                    } else {
                        exc |= (uint32_t)nonfinite(sg[m]);
                    }
                } else {
                    bf[m][0] = decode_b<FMT>(wx, sg[m]);
                    bf[m][1] = decode_b<FMT>(wy, sg[m]);
                    exc |= (uint32_t)b7_exceptional(sg[m]);
                }
            }
            // A fragments of row tile mt (two 32-wide halves of group g, per term)
            auto read_a = [&] __attribute__((always_inline)) (int mt, bf16x8 (&a)[TERMS][2]) {
                const char *rp = base + (mt * 16 + t) * APITCH;
#pragma unroll
                for (int tm = 0; tm < TERMS; ++tm)
#pragma unroll
                    for (int s = 0; s < 2; ++s) {
                        const int off = kDmaA ? ((8 * g + 2 * q + s) ^ t) * 16
                                              : (64 * g + 16 * q) * 2 + 16 * s;
                        a[tm][s] = *reinterpret_cast<const bf16x8 *>(rp + tm * PL + off);
                    }
            };
            bf16x8 an[TERMS][2];
            if constexpr (kPipeA)
                read_a(0, an);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                bf16x8 a[TERMS][2];
                if constexpr (kPipeA) {
                    // the next row tile's fragments are read before this tile's MFMAs, so
                    // their LDS latency runs under the MFMAs
#pragma unroll
                    for (int tm = 0; tm < TERMS; ++tm)
                        a[tm][0] = an[tm][0], a[tm][1] = an[tm][1];
                    if (mt + 1 < MT)
                        read_a(mt + 1, an);
                    __builtin_amdgcn_sched_barrier(0);
                } else {
                    read_a(mt, a);
                }
                if constexpr (FMT == 4) {
                    // each 64-wide group is its own chain over n - 8, then one f32 FMA
                    // applies the group's scale
#pragma unroll
                    for (int m = 0; m < 2; ++m) {
                        f4v c = f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                        for (int tm = 0; tm < TERMS; ++tm) {
                            bf16x8 b0 = bf[m][0], b1 = bf[m][1];
                            if (EXACT && tm > 0 && spec[m])
                                b0 = b1 = bf16x8{};
                            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[tm][0], b0, c, 0, 0, 0);
                            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[tm][1], b1, c, 0, 0, 0);
                        }
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            acc[mt][m][i] = EXACT && spec[m] ? acc[mt][m][i] + c[i]
                                                             : fmaf(sg[m], c[i], acc[mt][m][i]);
                        // keep the scaling here: sunk below the next step's loads, it
                        // drags a wait for those loads in with it
                        asm volatile("" : "+v"(acc[mt][m]));
                    }
                } else {
#pragma unroll
                    for (int m = 0; m < 2; ++m)
#pragma unroll
                        for (int tm = 0; tm < TERMS; ++tm) {
                            acc[mt][m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[tm][0], bf[m][0],
                                                                                 acc[mt][m], 0, 0, 0);
                            acc[mt][m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[tm][1], bf[m][1],
                                                                                 acc[mt][m], 0, 0, 0);
                        }
                }
                // one row tile's A fragments live at a time, or two with kPipeA
                // (register pressure)
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };

    // One group g (64 K) of step j of pair p: the operand shuffles of the two weight tiles
    // and their scale words (LDS crossbar), the decode (VALU), then the MFMAs of every
    // row tile.
    struct GRaw {
        uint32_t wx[2], wy[2], sw[2];
    };
    struct GDec {
        bf16x8 bf[2][2];
        float sg[2];
        bool spec[2];  // EXACT int4: this lane's column scale is not finite
    };
    auto shuffle = [&] __attribute__((always_inline)) (const GStep<FMT> &b, const Scl &sc, int p,
                                                         int j, int g, GRaw &r) {
        // scale words of step j, groups 0-1 / 2-3, sit in lanes 4 t + 2 j and 4 t + 2 j + 1;
        // chunked: MXFP4 pair p in lane 4 t + p % 4 (word 2 j + g / 2), int4 groups of step
        // j in lane 4 t + 2 (p % 2) + j (component g)
        const int ssrc = kChunkS ? (FMT == 7 ? 4 * (4 * t + p % PPC) : 4 * (4 * t + 2 * (p % PPC) + j))
                                 : 4 * (4 * t + 2 * j);
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            r.wx[m] = (uint32_t)__builtin_amdgcn_ds_bpermute(src4, (int)b.w[m][g].x);
            r.wy[m] = (uint32_t)__builtin_amdgcn_ds_bpermute(src4, (int)b.w[m][g].y);
            if constexpr (kChunkS && FMT == 4)
                r.sw[m] = (uint32_t)__builtin_amdgcn_ds_bpermute(ssrc, (int)sc.c[m][g]);
            else if constexpr (kChunkS)
                r.sw[m] = (uint32_t)__builtin_amdgcn_ds_bpermute(ssrc, (int)sc.c[m][2 * j + (g >> 1)]);
            else if constexpr (FMT == 4)
                r.sw[m] = (uint32_t)__builtin_amdgcn_ds_bpermute(
                    ssrc + 4 * (g >> 1), (int)((g & 1) ? sc.s4[m].y : sc.s4[m].x));
            else
                r.sw[m] = (uint32_t)__builtin_amdgcn_ds_bpermute(ssrc + 4 * (g >> 1), (int)sc.s7[m]);
        }
    };
    auto decode = [&] __attribute__((always_inline)) (const GRaw &r, int g, GDec &d, auto exact) {
        constexpr bool EXACT = decltype(exact)::value;
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            d.spec[m] = false;
            if constexpr (FMT == 4) {
                d.sg[m] = __uint_as_float(r.sw[m]);
            } else {  // lanes q < 2 take 32-block 2 g, q >= 2 block 2 g + 1
                const int byte = 2 * (g & 1) + (q >> 1);
                d.sg[m] = __uint_as_float(((r.sw[m] >> (8 * byte)) & 0xffu) << 23);
            }
            if constexpr (FMT == 7 && EXACT) {
                d.bf[m][0] = decode_b7_exact(r.wx[m], d.sg[m]);
                d.bf[m][1] = decode_b7_exact(r.wy[m], d.sg[m]);
            } else if constexpr (FMT == 4) {
                d.bf[m][0] = decode_b4_signed(r.wx[m]);
                d.bf[m][1] = decode_b4_signed(r.wy[m]);
                if constexpr (EXACT) {
                    // the reference's x * ((n - 8) * scale): a non-finite scale enters each
                    // product, which then takes the high term of x alone (its low terms
                    // would turn inf * 0 into NaN)
                    d.spec[m] = nonfinite(d.sg[m]);
                    if (d.spec[m]) {
                        d.bf[m][0] = mul_bf16x8_exact(d.bf[m][0], d.sg[m]);
                        d.bf[m][1] = mul_bf16x8_exact(d.bf[m][1], d.sg[m]);
                    }
                } else {
                    exc |= (uint32_t)nonfinite(d.sg[m]);
                }
            } else {
                d.bf[m][0] = decode_b<FMT>(r.wx[m], d.sg[m]);
                d.bf[m][1] = decode_b<FMT>(r.wy[m], d.sg[m]);
                exc |= (uint32_t)b7_exceptional(d.sg[m]);
            }
        }
    };
    auto mfmas = [&] __attribute__((always_inline)) (const char *base, int g, const GDec &d,
                                                       auto exact) {
        constexpr bool EXACT = decltype(exact)::value;
        // A fragments of row tile mt (two 32-wide halves of group g, per term)
        auto read_a = [&] __attribute__((always_inline)) (int mt, bf16x8 (&a)[TERMS][2]) {
            const char *rp = base + (mt * 16 + t) * APITCH;
#pragma unroll
            for (int tm = 0; tm < TERMS; ++tm)
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    const int off = kDmaA ? ((8 * g + 2 * q + s) ^ t) * 16
                                          : (64 * g + 16 * q) * 2 + 16 * s;
                    a[tm][s] = *reinterpret_cast<const bf16x8 *>(rp + tm * PL + off);
                }
        };
        bf16x8 an[TERMS][2];
        if constexpr (kPipeA)
            read_a(0, an);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            bf16x8 a[TERMS][2];
            if constexpr (kPipeA) {
                // the next row tile's fragments are read before this tile's MFMAs, so
                // their LDS latency runs under the MFMAs
#pragma unroll
                for (int tm = 0; tm < TERMS; ++tm)
                    a[tm][0] = an[tm][0], a[tm][1] = an[tm][1];
                if (mt + 1 < MT)
                    read_a(mt + 1, an);
                __builtin_amdgcn_sched_barrier(0);
            } else {
                read_a(mt, a);
            }
            if constexpr (FMT == 4) {
                // each 64-wide group is its own chain over n - 8, then one f32 FMA applies
                // the group's scale
#pragma unroll
                for (int m = 0; m < 2; ++m) {
                    f4v c = f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int tm = 0; tm < TERMS; ++tm) {
                        bf16x8 b0 = d.bf[m][0], b1 = d.bf[m][1];
                        if (EXACT && tm > 0 && d.spec[m])
                            b0 = b1 = bf16x8{};
                        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[tm][0], b0, c, 0, 0, 0);
                        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[tm][1], b1, c, 0, 0, 0);
                    }
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        acc[mt][m][i] = EXACT && d.spec[m] ? acc[mt][m][i] + c[i]
                                                           : fmaf(d.sg[m], c[i], acc[mt][m][i]);
                    // keep the scaling here: sunk below the next step's loads, it drags a
                    // wait for those loads in with it
                    asm volatile("" : "+v"(acc[mt][m]));
                }
            } else {
#pragma unroll
                for (int m = 0; m < 2; ++m)
#pragma unroll
                    for (int tm = 0; tm < TERMS; ++tm) {
                        acc[mt][m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[tm][0], d.bf[m][0],
                                                                             acc[mt][m], 0, 0, 0);
                        acc[mt][m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[tm][1], d.bf[m][1],
                                                                             acc[mt][m], 0, 0, 0);
                    }
            }
            // one row tile's A fragments live at a time, or two with kPipeA (register
            // pressure)
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // step j (0 or 1) of pair p, whose scales are in sc.  kPipeB: group g + 1's operand
    // shuffles are issued before group g's MFMAs and decoded after them, so the shuffles'
    // LDS latency runs under the MFMAs instead of ahead of every group.
    auto compute = [&] __attribute__((always_inline)) (const GStep<FMT> &b, int buf,
                                                         const Scl &sc, int p, int j, auto exact) {
        const char *base = smem + buf * STAGE;
        if constexpr (kPipeB) {
            GRaw r;
            GDec d;
            shuffle(b, sc, p, j, 0, r);
            decode(r, 0, d, exact);
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                if (g < 3)
                    shuffle(b, sc, p, j, g + 1, r);
                __builtin_amdgcn_sched_barrier(0);
                mfmas(base, g, d, exact);
                if (g < 3)
                    decode(r, g + 1, d, exact);
            }
        } else {
            compute1(b, buf, sc, p, j, exact);
        }
    };

    // epilogue of one task: C[4 q + i][t] of row tile mt and tile m
    auto epilogue = [&] __attribute__((always_inline)) (const TaskD<FMT> &d) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = mt * 16 + 4 * q + i;
                const int j = d.jbase + r;
                if constexpr (DUAL) {
                    const float h = mf_act(A.act, acc[mt][0][i], acc[mt][1][i], A.act_a, A.act_b);
                    __bf16 tt[3];
                    split_terms<TERMS>(h, tt);
                    const int col = d.col0 + t;
                    const int pos = (col & ~7) + a_slot<FMT>(col & 7);
                    if (r < d.nrow) {
                        if (A.out) {
                            A.out[(size_t)j * O + col] = h;
                        } else {
#pragma unroll
                            for (int tm = 0; tm < TERMS; ++tm)
                                A.pout[((size_t)tm * rcap + j) * O + pos] = tt[tm];
                        }
                    }
                } else {
                    if (r < d.nrow) {
                        A.out[(size_t)j * O + d.col0 + t] = acc[mt][0][i];
                        A.out[(size_t)j * O + d.col0 + 16 + t] = acc[mt][1][i];
                    }
                }
            }
            acc[mt][0] = acc[mt][1] = f4v{0.f, 0.f, 0.f, 0.f};
        }
    };

    // software pipeline: B two steps ahead in registers; A staged into LDS one step
    // ahead from registers loaded PA steps ahead (PA = 1 for the compute-bound 128-row
    // class, whose registers are full).  Prefetches past the task's last step re-read
    // harmless bytes that are never consumed, so the body has no branches around its
    // loads; the scheduling barriers keep each step's uses of a register set ahead of the
    // loads that refill it.
    if ((int)blockIdx.x >= n_tasks)
        return;
    const int task = A.xcd ? xcd_task(blockIdx.x, n_tasks) : (int)blockIdx.x;
    const TaskD<FMT> cur = make_task(task);
    GStep<FMT> b0, b1;
    Scl sc, sn;  // scales of this pair of steps (chunk) / of the next pair (chunk)
    AStage ra0, ra1;
    // The prologue issues its loads in the loop's own order (A, B of step 0, A, B of
    // step 1): the wait counts at the loop head are merged from both ways in, and a
    // different order here would make the loop wait for step k + 1's weights too.
    auto prologue = [&] __attribute__((always_inline)) () {
        if constexpr (kDmaA)
            dma_a(cur, 0, 0);
        else
            load_a(ra0, cur, 0);
        load_b(b0, cur, 0);
        load_s(sn, cur, 0);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (PA == 2)
            load_a(ra1, cur, min(1, nk - 1));
        load_b(b1, cur, min(1, nk - 1));
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (!kDmaA)
            store_a(ra0, 0);
        __syncthreads();
    };
    // Even step k: LDS buffer 0, weights b0; stages A(k + 1) into buffer 1.  Prefetches
    // past the task's last step read its last step again (L2 hits, never consumed):
    // wrapping to the first steps instead re-read two steps of weights from HBM per task,
    // a quarter of the bytes at K = 2048.
    auto step_even = [&] __attribute__((always_inline)) (int k, auto exact) {
        const int k2 = min(k + 2, nk - 1);
        if constexpr (kChunkS) {
            // a new chunk opens at this pair: the chunk loaded two steps ago
            if (((k >> 1) % PPC) == 0)
                sc = sn;
        } else {
            sc = sn;
        }
        if constexpr (kDmaA)
            dma_a(cur, min(k + 1, nk - 1), 1);  // first: the barrier below waits for it only
        else if constexpr (PA == 2)
            load_a(ra0, cur, k2);
        else
            load_a(ra1, cur, min(k + 1, nk - 1));
        compute(b0, 0, sc, k >> 1, 0, exact);
        __builtin_amdgcn_sched_barrier(0);
        load_b(b0, cur, k2);
        load_s(sn, cur, k2);
        if constexpr (!kDmaA)
            store_a(ra1, 1);
        __syncthreads();
    };
    // odd step k + 1: LDS buffer 1, weights b1; stages A(k + 2) into buffer 0
    auto step_odd = [&] __attribute__((always_inline)) (int k, auto exact) {
        const int k3 = min(k + 3, nk - 1);
        if constexpr (kDmaA)
            dma_a(cur, min(k + 2, nk - 1), 0);
        else if constexpr (PA == 2)
            load_a(ra1, cur, k3);
        else
            load_a(ra0, cur, min(k + 2, nk - 1));
        compute(b1, 1, sc, k >> 1, 1, exact);
        __builtin_amdgcn_sched_barrier(0);
        load_b(b1, cur, k3);
        if constexpr (!kDmaA)
            store_a(ra0, 0);
        __syncthreads();
    };
    // The pair loop has no exit between its two steps: an exit there, merged by the
    // compiler with the loop test, gives a path from the even step straight back to the
    // loop head, on which the wait counts would also wait for step k + 1's weights.  An
    // odd last step runs after the loop.
    auto k_loop = [&] __attribute__((always_inline)) (auto exact) {
        for (int k = 0; k + 2 <= nk; k += 2) {
            step_even(k, exact);
            step_odd(k, exact);
        }
        if (nk & 1)
            step_even(nk - 1, exact);
    };
    prologue();
    k_loop(std::false_type{});
    // Rare second pass: some operand of the task needs the exact decode.  The whole
    // workgroup runs the task again (the A staging is shared).  (The same loop with a
    // uniform branch per step instead of this second copy raised the register count of
    // the common pass.)
    if (__syncthreads_or((int)exc)) {
        exc = 0;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
            acc[mt][0] = acc[mt][1] = f4v{0.f, 0.f, 0.f, 0.f};
        prologue();
        k_loop(std::true_type{});
    }
    epilogue(cur);
}

// ---- input planes for the GEMM: gather, split into bf16 terms ------------------------

// One workgroup per row j of the planes: the source row is one scalar load, and each
// thread converts up to 4 of the row's 8-element chunks per pass with all their loads
// issued first (clamped to the row, so they stay unconditional; only the stores are).
constexpr int kPrepThreads = 256, kPrepUnroll = 4;

// n_live (device, may be null): rows j >= *n_live are left alone (a grid sized for a
// bound).  src_rows >= 0: a source row outside [0, src_rows) gives a zero row.
template <int FMT, int TERMS>
__global__ __launch_bounds__(kPrepThreads) void k_prep_planes(const float *x,
                                                              const int *rows_map, int K,
                                                              int rcap, __bf16 *planes,
                                                              const int *n_live, int src_rows) {
    const int j = blockIdx.x;
    if (n_live && j >= *n_live)
        return;
    int src = rows_map ? rows_map[j] : j;
    const bool zero = src_rows >= 0 && (src < 0 || src >= src_rows);
    if (zero)
        src = 0;
    const int per_row = K >> 3;
    const float4 *p = reinterpret_cast<const float4 *>(x + (size_t)src * K);
    for (int c0 = 0; c0 < per_row; c0 += kPrepUnroll * kPrepThreads) {
        float4 v[kPrepUnroll][2];
#pragma unroll
        for (int u = 0; u < kPrepUnroll; ++u) {
            const int c = min(c0 + u * kPrepThreads + (int)threadIdx.x, per_row - 1);
            v[u][0] = p[2 * c];
            v[u][1] = p[2 * c + 1];
            if (zero)
                v[u][0] = v[u][1] = float4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int u = 0; u < kPrepUnroll; ++u) {
            const int c = c0 + u * kPrepThreads + (int)threadIdx.x;
            const float e8[8] = {v[u][0].x, v[u][0].y, v[u][0].z, v[u][0].w,
                                 v[u][1].x, v[u][1].y, v[u][1].z, v[u][1].w};
            bf16x8 o[3];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                __bf16 tt[3];
                split_terms<TERMS>(e8[e], tt);
#pragma unroll
                for (int tm = 0; tm < TERMS; ++tm)
                    o[tm][a_slot<FMT>(e)] = tt[tm];
            }
            if (c < per_row) {
#pragma unroll
                for (int tm = 0; tm < TERMS; ++tm)
                    *reinterpret_cast<bf16x8 *>(planes + ((size_t)tm * rcap + j) * K + 8 * c) =
                        o[tm];
            }
        }
    }
}

// ---- launchers ----------------------------------------------------------------------

static bool g_gemm_xcd = true;  // option "gemm_xcd"
void gemm_set_xcd(bool on) { g_gemm_xcd = on; }
bool gemm_xcd() { return g_gemm_xcd; }

template <int FMT, bool DUAL, int TERMS, int MT, bool UNI = false>
static hipError_t launch_gemm_t(GemmArgs a, int n_items, hipStream_t st) {
    const size_t lds = gemm_lds_bytes(FMT, TERMS, MT);
    auto kern = k_gemm<FMT, DUAL, TERMS, MT, UNI>;
    static bool attr = false;  // the dynamic LDS limit, raised once per process
    if (!attr) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess)
            return e;
        attr = true;
    }
    a.n_tasks = n_items * a.nbn;
    a.xcd = g_gemm_xcd ? 1 : 0;
    hipLaunchKernelGGL(kern, dim3((unsigned)a.n_tasks), dim3(kGemmThreads), lds, st, a);
    return hipGetLastError();
}

template <int FMT, bool DUAL>
static hipError_t launch_gemm_fd(const GemmArgs &a, int n_items, int terms, int mt,
                                 hipStream_t st) {
    if (mt > gemm_max_mt(FMT, terms))
        return hipErrorInvalidValue;
    if (terms == 1) {
        switch (mt) {
        case 1: return launch_gemm_t<FMT, DUAL, 1, 1>(a, n_items, st);
        case 2: return launch_gemm_t<FMT, DUAL, 1, 2>(a, n_items, st);
        }
        if (mt == 4)
            return launch_gemm_t<FMT, DUAL, 1, 4>(a, n_items, st);
        if (mt == 8)
            return launch_gemm_t<FMT, DUAL, 1, 8>(a, n_items, st);
        return hipErrorInvalidValue;
    }
    if (terms == 2) {
        switch (mt) {
        case 1: return launch_gemm_t<FMT, DUAL, 2, 1>(a, n_items, st);
        case 2: return launch_gemm_t<FMT, DUAL, 2, 2>(a, n_items, st);
        }
        if (mt == 4)
            return launch_gemm_t<FMT, DUAL, 2, 4>(a, n_items, st);
        return hipErrorInvalidValue;
    }
    return hipErrorInvalidValue;
}

hipError_t launch_gemm(int fmt, bool dual, int terms, int mt, const ExpertWork *ew,
                       const void *items, int n_items, const void *pin, void *pout, float *out,
                       int K, int O, int rcap, int act,
                       float act_a, float act_b, hipStream_t st, const int *n_items_dev) {
    if (n_items <= 0)
        return hipSuccess;
    if (K % kGemmBK || O % (dual ? 128 : 256) || gemm_lds_bytes(fmt, terms, mt) > 163840)
        return hipErrorInvalidValue;
    GemmArgs a{};
    a.ew = ew;
    a.items = static_cast<const GemmItem *>(items);
    a.pin = static_cast<const __bf16 *>(pin);
    a.pout = static_cast<__bf16 *>(pout);
    a.out = out;
    a.nbn = O / (dual ? 128 : 256);
    a.K = K;
    a.O = O;
    a.rcap = rcap;
    a.act = act;
    a.act_a = act_a;
    a.act_b = act_b;
    a.n_items_dev = n_items_dev;
    if (fmt == 4)
        return dual ? launch_gemm_fd<4, true>(a, n_items, terms, mt, st)
                    : launch_gemm_fd<4, false>(a, n_items, terms, mt, st);
    if (fmt == 7)
        return dual ? launch_gemm_fd<7, true>(a, n_items, terms, mt, st)
                    : launch_gemm_fd<7, false>(a, n_items, terms, mt, st);
    return hipErrorInvalidValue;
}

hipError_t launch_gemm_rows(int fmt, int terms, int mt, const ExpertWork *ew1, int nrows,
                            const void *pin, float *out, int K, int O, hipStream_t st) {
    if (nrows <= 0)
        return hipSuccess;
    if (K % kGemmBK || O % 256 || gemm_lds_bytes(fmt, terms, mt) > 163840 || !ew1)
        return hipErrorInvalidValue;
    GemmArgs a{};
    a.ew1 = *ew1;
    a.nrows_all = nrows;
    a.pin = static_cast<const __bf16 *>(pin);
    a.out = out;
    a.nbn = O / 256;
    a.K = K;
    a.O = O;
    a.rcap = nrows;
    const int n_items = (nrows + 16 * mt - 1) / (16 * mt);
    if (terms != 2)
        return hipErrorInvalidValue;
#define MVLLM_ROWS(F)                                                                          \
    return mt == 1 ? launch_gemm_t<F, false, 2, 1, true>(a, n_items, st)                      \
         : mt == 2 ? launch_gemm_t<F, false, 2, 2, true>(a, n_items, st)                      \
         : mt == 4 ? launch_gemm_t<F, false, 2, 4, true>(a, n_items, st)                      \
                   : hipErrorInvalidValue
    if (fmt == 4)
        MVLLM_ROWS(4);
    if (fmt == 7)
        MVLLM_ROWS(7);
#undef MVLLM_ROWS
    return hipErrorInvalidValue;
}

hipError_t launch_prep_planes(int fmt, int terms, const float *x, const int *rows_map, int R,
                              int K, int rcap, void *planes, hipStream_t st, const int *n_live,
                              int src_rows) {
    if (R <= 0)
        return hipSuccess;
    if (K % 8)
        return hipErrorInvalidValue;
    __bf16 *pl = static_cast<__bf16 *>(planes);
#define MVLLM_PREP(F, T)                                                                      \
    hipLaunchKernelGGL((k_prep_planes<F, T>), dim3((unsigned)R), dim3(kPrepThreads), 0, st, x, \
                       rows_map, K, rcap, pl, n_live, src_rows)
    if (fmt == 4) {
        if (terms == 1) MVLLM_PREP(4, 1); else if (terms == 2) MVLLM_PREP(4, 2); else MVLLM_PREP(4, 3);
    } else if (fmt == 7) {
        if (terms == 1) MVLLM_PREP(7, 1); else if (terms == 2) MVLLM_PREP(7, 2); else MVLLM_PREP(7, 3);
    } else {
        return hipErrorInvalidValue;
    }
#undef MVLLM_PREP
    return hipGetLastError();
}

}  // namespace mvllm_hip
