// kern_gemm.hip -- prefill-shaped expert GEMMs on the gfx950 matrix cores: a grouped
// GEMM over token-sorted expert segments (v_mfma_f32_16x16x32_bf16).
//
// Work item = (expert, block of up to 16 * MT of its rows) x (block of output columns).
// A workgroup of 8 waves streams K in steps of 256:
//   * activations (A): the item's rows of the bf16 input planes [TERMS][rcap][K] are
//     staged into LDS, double buffered, by all 512 threads (16-byte loads); for int4
//     the per-64 sums of each row (the -8 offset correction) come along;
//   * weights (B): each wave owns two 16-column tiles (gate and up at the same columns
//     for the dual projection, two adjacent tiles of the down matrix otherwise) and
//     reads their packed rows with coalesced 8-byte loads (lane l -> row l / 4, 32 B
//     per row per load) two steps ahead, moves them into the operand layout with
//     ds_bpermute and decodes them exactly in registers, as the decode kernel does;
//   * each decoded B fragment feeds MT row tiles (one A fragment read per two MFMAs).
// int4: every 64-wide group is its own chain started from -8 * (group sum of the row),
// then one f32 FMA applies the group's f32 scale (exact (n - 8) * scale, no rounding of
// the product to bf16).  MXFP4: the ue8m0 scale is folded into the bf16 decode (exact).
// The dual epilogue applies the activation and writes H in the same plane format (with
// per-16-column partial sums for int4) that both down kernels read.
#include "mfma_common.h"

#include <algorithm>

namespace mvllm_hip {


struct GemmItem {
    int a;     // expert index into ExpertWork
    int r0;    // first row within the expert's compact rows
    int nrow;  // rows in this item (<= 16 * MT)
    int pad;
};

struct GemmArgs {
    const ExpertWork *ew;
    const GemmItem *items;
    const __bf16 *pin;  // A planes [TERMS][rcap][K] (int4: 8-blocks in slot order)
    const float *xs;    // int4: A partial sums [K/64][4][rcap]
    __bf16 *pout;       // dual: H planes [TERMS][rcap][O]
    float *hp;          // dual, int4: H partial sums [O/64][4][rcap]
    float *out;         // single: Y [rcap][O] f32
    int nbn;            // column blocks per item
    int n_tasks;        // items * nbn
    int K, O, rcap;
    int act;
    float act_a, act_b;
};

constexpr int kGemmThreads = 512;
constexpr int kGemmBK = 256;
constexpr int kGemmPitch = kGemmBK * 2 + 16;  // LDS bytes per A row and plane (+16: banks)

__host__ __device__ constexpr int gemm_stage_bytes(int fmt, int terms, int mt) {
    return terms * 16 * mt * kGemmPitch + (fmt == 4 ? 4 * 16 * mt * 4 : 0);
}

size_t gemm_lds_bytes(int fmt, int terms, int mt) {
    return 2 * (size_t)gemm_stage_bytes(fmt, terms, mt);
}

// Packed weights and scales of one K step for the wave's two tiles, as loaded.
template <int FMT>
struct GStep {
    u32x2 w[2][4];
    u32x4 s4[FMT == 4 ? 2 : 1];  // int4: scales of the step's 4 groups, row t
    u32x2 s7[FMT == 7 ? 2 : 1];  // MXFP4: scale bytes of the step's 8 blocks, row t
};

// Where one task's operands live: its two weight tiles (buffer resources + this lane's
// offsets), its activation rows and its output columns.
template <int FMT>
struct TaskD {
    __amdgpu_buffer_rsrc_t rw[2], rs[2];
    uint32_t vw[2], vs[2];
    int jbase, nrow, col0;
};

// Persistent over tasks (PERSIST): workgroup b runs tasks b, b + G, b + 2G, ...
// (G = gridDim.x) as one stream of K steps.  The loads of the first two steps of task i + 1 are issued
// during the last two steps of task i (its descriptor is fetched a whole task earlier),
// so a task's prologue latency and epilogue stores overlap the neighbouring task's
// streaming.  Without PERSIST (the compute-bound row classes, whose registers are full),
// or with an odd number of K steps, the host launches one task per workgroup.
template <int FMT, bool DUAL, int TERMS, int MT, bool PERSIST>
__global__ __launch_bounds__(kGemmThreads) void k_gemm(GemmArgs A) {
    constexpr int BM = 16 * MT;
    constexpr int PA = MT >= 8 ? 1 : 2;  // activation prefetch distance in K steps
    constexpr int PL = BM * kGemmPitch;                  // bytes per plane per stage
    constexpr int STAGE = gemm_stage_bytes(FMT, TERMS, MT);
    constexpr int ACH = TERMS * BM * (kGemmBK / 8) / kGemmThreads;  // 16-byte chunks/thread
    static_assert(ACH * kGemmThreads == TERMS * BM * (kGemmBK / 8), "A staging split");
    extern __shared__ __attribute__((aligned(16))) char smem[];

    const int K = A.K, O = A.O, rcap = A.rcap;
    const int n_tasks = A.n_tasks;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, t = lane & 15, q = lane >> 4;
    const uint32_t rowb = (uint32_t)(K >> 1);
    const uint32_t srow = (uint32_t)(FMT == 4 ? (K / 64) * 4 : K / 32);
    const int nk = K / kGemmBK;

    auto make_task = [&] __attribute__((always_inline)) (int task) {
        TaskD<FMT> d;
        const int item = task / A.nbn;
        const int nb = task - item * A.nbn;
        const GemmItem it = A.items[item];
        const ExpertWork &ew = A.ew[it.a];
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
            d.vs[m] = (uint32_t)(trow + t) * srow;
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
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            if constexpr (FMT == 4)
                b.s4[m] = __builtin_bit_cast(
                    u32x4, __builtin_amdgcn_raw_buffer_load_b128(d.rs[m], d.vs[m], (uint32_t)k * 16u, 0));
            else
                b.s7[m] = __builtin_bit_cast(
                    u32x2, __builtin_amdgcn_raw_buffer_load_b64(d.rs[m], d.vs[m], (uint32_t)k * 8u, 0));
        }
    };

    // A staging: chunk c = u * 512 + tid -> plane c / (BM * 32), row (c / 32) % BM,
    // 16-byte column c % 32 of the step.  Two register sets let the loads of step k + 2
    // be issued while step k computes (PA = 2), so their latency spans two steps.
    struct AStage {
        u32x4 v[ACH];  // native vectors: copies of HIP's uint4 struct go through scratch
        float p[4];  // int4: the four partial sums of this thread's (group, row)
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
        if constexpr (FMT == 4) {
            // the four partial sums of (group, row) are added only when stored: adding
            // here would wait for these loads, and with them for every load issued
            // before (loads complete in order)
            const int i4 = tid < 4 * BM ? tid : 0;
            const int g = i4 / BM, r = min(i4 - g * BM, d.nrow - 1);
            const float *p = A.xs + (size_t)(4 * k + g) * 4 * rcap + d.jbase + r;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                ra.p[i] = p[i * rcap];
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
        if constexpr (FMT == 4) {
            if (tid < 4 * BM) {
                const int g = tid / BM, r = tid - g * BM;
                reinterpret_cast<float *>(base + TERMS * PL)[g * BM + r] =
                    -8.f * (((ra.p[0] + ra.p[1]) + ra.p[2]) + ra.p[3]);
            }
        }
    };

    f4v acc[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
        acc[mt][0] = acc[mt][1] = f4v{0.f, 0.f, 0.f, 0.f};
    const int src4 = 4 * (4 * t + q);  // ds_bpermute address of lane 4 t + q

    auto compute = [&] __attribute__((always_inline)) (const GStep<FMT> &b, int buf) {
        const char *base = smem + buf * STAGE;
        const float *lsum = reinterpret_cast<const float *>(base + TERMS * PL);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            bf16x8 bf[2][2];
            float sg[2];
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                const uint32_t wx = (uint32_t)__builtin_amdgcn_ds_bpermute(src4, (int)b.w[m][g].x);
                const uint32_t wy = (uint32_t)__builtin_amdgcn_ds_bpermute(src4, (int)b.w[m][g].y);
                if constexpr (FMT == 4) {
                    sg[m] = __uint_as_float(b.s4[m][g]);
                } else {  // lanes q < 2 take 32-block 2 g, q >= 2 block 2 g + 1
                    const int blk = 2 * g + (q >> 1);
                    const uint32_t word = blk < 4 ? b.s7[m].x : b.s7[m].y;
                    sg[m] = __uint_as_float(((word >> (8 * (blk & 3))) & 0xffu) << 23);
                }
                bf[m][0] = decode_b<FMT>(wx, sg[m]);
                bf[m][1] = decode_b<FMT>(wy, sg[m]);
                if constexpr (FMT == 7) {
                    const bool exc = b7_exceptional(sg[m]);
                    if (__builtin_expect(__builtin_amdgcn_ballot_w64(exc) != 0, 0)) {
                        if (exc) {
                            bf[m][0] = decode_b7_exact(wx, sg[m]);
                            bf[m][1] = decode_b7_exact(wy, sg[m]);
                        }
                    }
                }
            }
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const char *ap = base + (mt * 16 + t) * kGemmPitch + (64 * g + 16 * q) * 2;
                bf16x8 a[TERMS][2];
#pragma unroll
                for (int tm = 0; tm < TERMS; ++tm)
#pragma unroll
                    for (int s = 0; s < 2; ++s)
                        a[tm][s] = *reinterpret_cast<const bf16x8 *>(ap + tm * PL + 16 * s);
                if constexpr (FMT == 4) {
                    const f4v init = *reinterpret_cast<const f4v *>(lsum + g * BM + mt * 16 + 4 * q);
#pragma unroll
                    for (int m = 0; m < 2; ++m) {
                        f4v c = init;
#pragma unroll
                        for (int tm = 0; tm < TERMS; ++tm) {
                            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[tm][0], bf[m][0], c, 0, 0, 0);
                            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[tm][1], bf[m][1], c, 0, 0, 0);
                        }
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            acc[mt][m][i] = fmaf(sg[m], c[i], acc[mt][m][i]);
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
                // one row tile's A fragments live at a time (register pressure)
                __builtin_amdgcn_sched_barrier(0);
            }
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
                    float rep = split_terms<TERMS>(h, tt);
                    const int col = d.col0 + t;
                    const int pos = (col & ~7) + a_slot<FMT>(col & 7);
                    if (r < d.nrow) {
#pragma unroll
                        for (int tm = 0; tm < TERMS; ++tm)
                            A.pout[((size_t)tm * rcap + j) * O + pos] = tt[tm];
                    }
                    if constexpr (FMT == 4) {
                        rep += __shfl_xor(rep, 1, 16);
                        rep += __shfl_xor(rep, 2, 16);
                        rep += __shfl_xor(rep, 4, 16);
                        rep += __shfl_xor(rep, 8, 16);
                        const int tile = d.col0 >> 4;
                        if (t == 0 && r < d.nrow)
                            A.hp[((size_t)(tile >> 2) * 4 + (tile & 3)) * rcap + j] = rep;
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
    // class, whose registers are full).  Prefetches past a task's last step go to the
    // next task (or, after the last task, re-read harmless bytes that are never
    // consumed), so the body has no branches around its loads; the scheduling barriers
    // keep each step's uses of a register set ahead of the loads that refill it.
    int task = blockIdx.x;
    if (task >= n_tasks)
        return;
    TaskD<FMT> cur = make_task(task);
    bool has_next = PERSIST && task + (int)gridDim.x < n_tasks;
    TaskD<FMT> nxt = cur;
    if (PERSIST && has_next)
        nxt = make_task(task + (int)gridDim.x);
    GStep<FMT> b0, b1;
    AStage ra0, ra1;
    load_a(ra0, cur, 0);
    if constexpr (PA == 2)
        load_a(ra1, cur, min(1, nk - 1));
    load_b(b0, cur, 0);
    load_b(b1, cur, 1);
    store_a(ra0, 0);
    __syncthreads();
    for (;;) {
        for (int k = 0; k < nk; k += 2) {
            const bool tail = k + 2 >= nk;  // this pair's prefetches belong to the next task
            const TaskD<FMT> &pd = PERSIST && tail ? nxt : cur;
            const int k2 = tail ? k + 2 - nk : k + 2;
            // even step: LDS buffer 0, weights b0; stage A(k + 1) into buffer 1
            if constexpr (PA == 2)
                load_a(ra0, pd, min(k2, nk - 1));
            else
                load_a(ra1, cur, min(k + 1, nk - 1));
            compute(b0, 0);
            __builtin_amdgcn_sched_barrier(0);
            load_b(b0, pd, k2);
            store_a(ra1, 1);
            __syncthreads();
            if (k + 1 >= nk)
                break;  // odd step count: one task per workgroup
            // odd step: LDS buffer 1, weights b1; stage A(k + 2) into buffer 0
            if constexpr (PA == 2)
                load_a(ra1, pd, min(k2 + 1, nk - 1));
            else
                load_a(ra0, pd, min(k2, nk - 1));
            compute(b1, 1);
            __builtin_amdgcn_sched_barrier(0);
            load_b(b1, pd, k2 + 1);
            store_a(ra0, 0);
            __syncthreads();
        }
        epilogue(cur);
        if (!PERSIST || !has_next)
            break;
        task += (int)gridDim.x;
        cur = nxt;
        has_next = task + (int)gridDim.x < n_tasks;
        if (has_next)
            nxt = make_task(task + (int)gridDim.x);
    }
}

// ---- input planes for the GEMM: gather, split into bf16 terms, per-16 partial sums ----

// One thread per 8-element chunk of a row; for int4 the two chunks of a 16-column
// partial sit in adjacent lanes (K / 8 is even).
template <int FMT, int TERMS>
__global__ __launch_bounds__(256) void k_prep_planes(const float *x, const int *rows_map, int R,
                                                     int K, int rcap, __bf16 *planes, float *xs) {
    const int per_row = K >> 3;
    const size_t total = (size_t)R * per_row;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t base = (size_t)blockIdx.x * blockDim.x; base < total; base += stride) {
        const size_t idx = base + threadIdx.x;
        const bool ok = idx < total;
        const int j = ok ? (int)(idx / per_row) : 0;
        const int c = ok ? (int)(idx - (size_t)j * per_row) : 0;
        float rs8 = 0.f;
        if (ok) {
            const int src = rows_map ? rows_map[j] : j;
            const float4 *p = reinterpret_cast<const float4 *>(x + (size_t)src * K + 8 * c);
            const float4 v0 = p[0], v1 = p[1];
            const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
            bf16x8 o[3];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                __bf16 tt[3];
                rs8 += split_terms<TERMS>(v[e], tt);
#pragma unroll
                for (int tm = 0; tm < TERMS; ++tm)
                    o[tm][a_slot<FMT>(e)] = tt[tm];
            }
#pragma unroll
            for (int tm = 0; tm < TERMS; ++tm)
                *reinterpret_cast<bf16x8 *>(planes + ((size_t)tm * rcap + j) * K + 8 * c) = o[tm];
        }
        if constexpr (FMT == 4) {
            rs8 += __shfl_xor(rs8, 1, 64);
            if (ok && (c & 1) == 0)
                xs[((size_t)(c >> 3) * 4 + ((c >> 1) & 3)) * rcap + j] = rs8;
        }
    }
}

// ---- launchers ----------------------------------------------------------------------

template <int FMT, bool DUAL, int TERMS, int MT, bool PERSIST>
static hipError_t launch_gemm_p(GemmArgs a, int n_items, hipStream_t st) {
    const size_t lds = gemm_lds_bytes(FMT, TERMS, MT);
    auto kern = k_gemm<FMT, DUAL, TERMS, MT, PERSIST>;
    // resident workgroups of this instantiation (queried once per process)
    static int resident = 0;
    if (resident == 0) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess)
            return e;
        int dev = 0, cus = 0, per_cu = 0;
        if ((e = hipGetDevice(&dev)) != hipSuccess ||
            (e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev)) !=
                hipSuccess ||
            (e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
                 &per_cu, reinterpret_cast<const void *>(kern), kGemmThreads, lds)) != hipSuccess)
            return e;
        resident = std::max(1, cus * std::max(1, per_cu));
    }
    a.n_tasks = n_items * a.nbn;
    // persistent (cross-task prefetch) only with an even number of K steps
    const int grid = PERSIST && (a.K / kGemmBK) % 2 == 0 ? std::min(a.n_tasks, resident)
                                                         : a.n_tasks;
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(kGemmThreads), lds, st, a);
    return hipGetLastError();
}

static bool g_gemm_persist = false;  // measured slower than independent workgroups

template <int FMT, bool DUAL, int TERMS, int MT>
static hipError_t launch_gemm_t(GemmArgs a, int n_items, hipStream_t st) {
    if constexpr (MT <= 2 && !(TERMS == 2 && MT == 2)) {  // (that one spills)
        if (g_gemm_persist && (a.K / kGemmBK) % 2 == 0)
            return launch_gemm_p<FMT, DUAL, TERMS, MT, true>(a, n_items, st);
    }
    return launch_gemm_p<FMT, DUAL, TERMS, MT, false>(a, n_items, st);
}

void gemm_set_persistent(bool on) { g_gemm_persist = on; }

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
        if constexpr (FMT == 7) {
            if (mt == 4)
                return launch_gemm_t<FMT, DUAL, 1, 4>(a, n_items, st);
            if (mt == 8)
                return launch_gemm_t<FMT, DUAL, 1, 8>(a, n_items, st);
        }
        return hipErrorInvalidValue;
    }
    if (terms == 2) {
        switch (mt) {
        case 1: return launch_gemm_t<FMT, DUAL, 2, 1>(a, n_items, st);
        case 2: return launch_gemm_t<FMT, DUAL, 2, 2>(a, n_items, st);
        }
        if constexpr (FMT == 7) {
            if (mt == 4)
                return launch_gemm_t<FMT, DUAL, 2, 4>(a, n_items, st);
        }
        return hipErrorInvalidValue;
    }
    return hipErrorInvalidValue;
}

hipError_t launch_gemm(int fmt, bool dual, int terms, int mt, const ExpertWork *ew,
                       const void *items, int n_items, const void *pin, const float *xs,
                       void *pout, float *hp, float *out, int K, int O, int rcap, int act,
                       float act_a, float act_b, hipStream_t st) {
    if (n_items <= 0)
        return hipSuccess;
    if (K % kGemmBK || O % (dual ? 128 : 256) || gemm_lds_bytes(fmt, terms, mt) > 163840)
        return hipErrorInvalidValue;
    GemmArgs a{};
    a.ew = ew;
    a.items = static_cast<const GemmItem *>(items);
    a.pin = static_cast<const __bf16 *>(pin);
    a.xs = xs;
    a.pout = static_cast<__bf16 *>(pout);
    a.hp = hp;
    a.out = out;
    a.nbn = O / (dual ? 128 : 256);
    a.K = K;
    a.O = O;
    a.rcap = rcap;
    a.act = act;
    a.act_a = act_a;
    a.act_b = act_b;
    if (fmt == 4)
        return dual ? launch_gemm_fd<4, true>(a, n_items, terms, mt, st)
                    : launch_gemm_fd<4, false>(a, n_items, terms, mt, st);
    if (fmt == 7)
        return dual ? launch_gemm_fd<7, true>(a, n_items, terms, mt, st)
                    : launch_gemm_fd<7, false>(a, n_items, terms, mt, st);
    return hipErrorInvalidValue;
}

hipError_t launch_prep_planes(int fmt, int terms, const float *x, const int *rows_map, int R,
                              int K, int rcap, void *planes, float *xs, hipStream_t st) {
    if (R <= 0)
        return hipSuccess;
    if (K % 16)
        return hipErrorInvalidValue;
    const size_t total = (size_t)R * (K / 8);
    const unsigned blocks = (unsigned)std::min<size_t>((total + 255) / 256, 8192);
    __bf16 *pl = static_cast<__bf16 *>(planes);
#define MVLLM_PREP(F, T)                                                                      \
    hipLaunchKernelGGL((k_prep_planes<F, T>), dim3(blocks), dim3(256), 0, st, x, rows_map, R, \
                       K, rcap, pl, xs)
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
