// kern_fused.hip -- both decode projections of a moe_block call in one cooperative launch.
//
// Tasks 0 .. n_gu-1 are the gate/up column blocks (dual), the rest the down column
// blocks.  Workgroup b runs tasks b, b + grid, b + 2 grid, ... in order, so every
// workgroup finishes all its gate/up tasks before it starts a down task.  A down task
// issues its first weight loads and then waits for its expert's gate/up tasks (done
// counter, see DecSync).  The launch is cooperative -- all workgroups are resident at
// once -- so each awaited task belongs to a running workgroup that never waits before
// finishing it: the waits end.  The down weights stream while the last gate/up tasks
// finish, and the launch gap between the projections is gone.
#include "mfma_dec.h"

#include <algorithm>

namespace mvllm_hip {

struct FusedArgs {
    DecArgs gu, dn;  // as the two launches would take them (wgs set)
    int n_gu;        // gate/up tasks = gate/up items x gu.wgs
    int n_tasks;     // + down items x dn.wgs
    DecSync sy;
};

template <int FMT, int TERMS, int KSG, int SRG, int KSD, int NTD, int SRD>
__global__ __launch_bounds__(kDecThreads) __attribute__((amdgpu_waves_per_eu(4)))
void k_mfma_fused(FusedArgs F) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    for (int task = blockIdx.x; task < F.n_tasks; task += gridDim.x) {
        // the thread index through an opaque move: per-lane values are then recomputed per
        // task instead of held (spilled) across the task loop
        int tid = (int)threadIdx.x;
        asm volatile("" : "+v"(tid));
        if (task < F.n_gu) {
            const int item = task / F.gu.wgs;
            dec_task<FMT, true, TERMS, KSG, 2, SRG, true>(F.gu, item, task - item * F.gu.wgs,
                                                          tid, smem, F.sy);
        } else {
            const int t2 = task - F.n_gu, item = t2 / F.dn.wgs;
            dec_task<FMT, false, TERMS, KSD, NTD, SRD, true>(F.dn, item, t2 - item * F.dn.wgs,
                                                             tid, smem, F.sy);
        }
        __syncthreads();  // the next task reuses the LDS
    }
}

namespace {

int device_cus() {
    static int n = 0;
    if (!n) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            n = 0;
    }
    return n;
}

template <int FMT, int TERMS, int KSG, int SRG, int KSD, int NTD, int SRD>
hipError_t launch_fused_t(FusedArgs f, size_t lds, hipStream_t st) {
    auto kern = k_mfma_fused<FMT, TERMS, KSG, SRG, KSD, NTD, SRD>;
    // resident workgroups per CU for this LDS size (queried once per size)
    static size_t c_lds = 0;
    static int c_occ = 0;
    if (lds != c_lds) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess)
            return e;
        int occ = 0;
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kern, kDecThreads, lds);
        if (e != hipSuccess)
            return e;
        c_lds = lds;
        c_occ = occ;
    }
    const int cap = c_occ * device_cus();
    if (cap <= 0)
        return hipErrorInvalidConfiguration;
    const int grid = std::min(f.n_tasks, cap);
    void *args[] = {&f};
    return hipLaunchCooperativeKernel(reinterpret_cast<const void *>(kern), dim3(grid),
                                      dim3(kDecThreads), args, (unsigned)lds, st);
}

// staging-register variants of the gate/up task (as launch_dec_t picks them); the down
// task stages at most 4 chunks per thread here (more would spill in the fused kernel)
template <int FMT, int TERMS, int KSG, int KSD, int NTD>
hipError_t launch_fused_sr(const FusedArgs &f, bool sr_gu_big, size_t lds, hipStream_t st) {
    return sr_gu_big ? launch_fused_t<FMT, TERMS, KSG, kDecStageDual, KSD, NTD, 4>(f, lds, st)
                     : launch_fused_t<FMT, TERMS, KSG, 2, KSD, NTD, 4>(f, lds, st);
}

template <int FMT, int TERMS, int KSG>
hipError_t launch_fused_dn(const FusedArgs &f, int ksd, int ntd, bool sg, size_t lds,
                           hipStream_t st) {
    if (ntd == 2)
        return ksd == 1 ? launch_fused_sr<FMT, TERMS, KSG, 1, 2>(f, sg, lds, st)
                        : hipErrorInvalidValue;
    switch (ksd) {
    case 1: return launch_fused_sr<FMT, TERMS, KSG, 1, 1>(f, sg, lds, st);
    case 2: return launch_fused_sr<FMT, TERMS, KSG, 2, 1>(f, sg, lds, st);
    case 4: return launch_fused_sr<FMT, TERMS, KSG, 4, 1>(f, sg, lds, st);
    default: return hipErrorInvalidValue;
    }
}

template <int FMT>
hipError_t launch_fused_f(const FusedArgs &f, int ksg, int ksd, int ntd, bool sg, size_t lds,
                          hipStream_t st) {
    switch (ksg) {
    case 1: return launch_fused_dn<FMT, 2, 1>(f, ksd, ntd, sg, lds, st);
    case 2: return launch_fused_dn<FMT, 2, 2>(f, ksd, ntd, sg, lds, st);
    case 4: return launch_fused_dn<FMT, 2, 4>(f, ksd, ntd, sg, lds, st);
    case 8: return launch_fused_dn<FMT, 2, 8>(f, ksd, ntd, sg, lds, st);
    default: return hipErrorInvalidValue;
    }
}

// Staging registers per thread (dual: 8-float chunks; single: uint4 of the planes).
int stage_regs(bool dual, int terms, int rmax, int K) {
    const size_t need = dual ? (size_t)rmax * (K / 8) : (size_t)terms * rmax * (K / 8);
    return (int)((need + kDecThreads - 1) / kDecThreads);
}

}  // namespace

bool fused_supported(int fmt, int terms, int ks_gu, int ks_dn, int nt_dn, int rmax_dn, int I) {
    return (fmt == 4 || fmt == 7) && terms == 2 &&
           (ks_gu == 1 || ks_gu == 2 || ks_gu == 4 || ks_gu == 8) &&
           ((nt_dn == 2 && ks_dn == 1) ||
            (nt_dn == 1 && (ks_dn == 1 || ks_dn == 2 || ks_dn == 4))) &&
           stage_regs(false, terms, rmax_dn, I) <= 4;
}

hipError_t launch_mfma_fused(int fmt, int terms, int ks_gu, int ks_dn, int nt_dn,
                             const DecDesc *gu_desc, int n_gu_items, const DecDesc *dn_desc,
                             int n_dn_items, const float *xin, void *planes, float *hp,
                             float *out, int D, int I, int rcap, int rmax_gu, int rmax_dn,
                             int act, float act_a, float act_b, unsigned *done, int *err,
                             hipStream_t st) {
    if (!fused_supported(fmt, terms, ks_gu, ks_dn, nt_dn, rmax_dn, I) || n_gu_items <= 0 ||
        n_dn_items <= 0)
        return hipErrorInvalidValue;
    const int tw_gu = kDecWaves / ks_gu, tw_dn = (kDecWaves / ks_dn) * nt_dn;
    if (D % 512 || I % 512 || D % (256 * ks_gu) || I % (256 * ks_dn) ||
        D / ks_gu > dec_max_kr(fmt) || I / ks_dn > dec_max_kr(fmt) || I % (16 * tw_gu) ||
        D % (16 * tw_dn) || rmax_gu < 1 || rmax_gu > 16 || rmax_dn < 1 || rmax_dn > 16)
        return hipErrorInvalidValue;
    const int sg = stage_regs(true, terms, rmax_gu, D);
    if (sg > kDecStageDual)
        return hipErrorInvalidValue;
    const size_t lds = std::max(dec_lds_plan(fmt, D, rmax_gu, terms, ks_gu, 2, nullptr),
                                dec_lds_plan(fmt, I, rmax_dn, terms, ks_dn, nt_dn, nullptr));
    if (lds > kDecLdsBudget)
        return hipErrorInvalidValue;
    FusedArgs f{};
    DecArgs &g = f.gu;
    g.desc = gu_desc;
    g.xin = xin;
    g.pout = static_cast<__bf16 *>(planes);
    g.hp = hp;
    g.K = D;
    g.O = I;
    g.rcap = rcap;
    g.rmax = rmax_gu;
    g.act = act;
    g.act_a = act_a;
    g.act_b = act_b;
    g.wgs = I / (16 * tw_gu);
    DecArgs &d = f.dn;
    d.desc = dn_desc;
    d.pin = static_cast<const __bf16 *>(planes);
    d.xs = hp;
    d.out = out;
    d.fold = 1;
    d.K = I;
    d.O = D;
    d.rcap = rcap;
    d.rmax = rmax_dn;
    d.wgs = D / (16 * tw_dn);
    f.n_gu = n_gu_items * g.wgs;
    f.n_tasks = f.n_gu + n_dn_items * d.wgs;
    f.sy.done = done;
    f.sy.err = err;
    const bool bg = sg > 2;
    return fmt == 4 ? launch_fused_f<4>(f, ks_gu, ks_dn, nt_dn, bg, lds, st)
                    : launch_fused_f<7>(f, ks_gu, ks_dn, nt_dn, bg, lds, st);
}

}  // namespace mvllm_hip
