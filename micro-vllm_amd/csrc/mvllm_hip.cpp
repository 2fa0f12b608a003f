// mvllm_hip.cpp -- C ABI of the MI355X routed-expert moe_block backend (host side).
//
// Per call: validate exactly as metal_ops::moe_block does (src/gpu/metal_ops.cpp:448-460),
// walk the experts with cpu_moe_block's skip rules (src/gpu/metal_ops.cpp:283-297) to
// build a plan -- active experts, their compact rows (rows whose destination reaches
// `out`), and per destination token the ordered list of (row, weight) it receives --
// then run three stream-ordered phases: gate/up/act GEMV -> H, down GEMV -> Y, combine
// Y into out in the reference's expert order.
#include "../../include/mvllm_hip.h"
#include "moe_internal.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <list>
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

namespace mvllm_hip {
void set_error(const std::string &s);
}

using namespace mvllm_hip;

namespace {

thread_local std::string g_err;

// A miss expert whose six pieces lie in one block from mvllm_hip_host_alloc and span at
// most their own bytes plus this much (the ExpertStore's blob padding) is staged with one
// host-to-device copy of the span.
constexpr size_t kSpanSlack = 4096;

// Pinned blocks handed out by mvllm_hip_host_alloc: base -> bytes.
std::mutex g_host_mu;
std::map<uintptr_t, size_t> g_host_blocks;

// True when [lo, hi) lies inside one block of g_host_blocks.
bool in_one_host_block(const uint8_t *lo, const uint8_t *hi) {
    std::lock_guard<std::mutex> lk(g_host_mu);
    auto it = g_host_blocks.upper_bound(reinterpret_cast<uintptr_t>(lo));
    if (it == g_host_blocks.begin())
        return false;
    --it;
    return reinterpret_cast<uintptr_t>(hi) <= it->first + it->second;
}

void set_err(const std::string &s) { g_err = s; }

}  // namespace

// the library's other host files report through the same thread's error text
void mvllm_hip::set_error(const std::string &s) { set_err(s); }

namespace {

#define HIP_TRY(expr)                                                                         \
    do {                                                                                      \
        hipError_t e_ = (expr);                                                               \
        if (e_ != hipSuccess) {                                                               \
            set_err(std::string(#expr) + ": " + hipGetErrorString(e_));                       \
            return 0;                                                                         \
        }                                                                                     \
    } while (0)

// Buffers a grow-only device buffer has outgrown.  Work already enqueued may still read
// them, so they are not freed when replaced (a free would have to drain the device first,
// in the middle of a call); they are kept until shutdown.  Growth is geometric, so what is
// kept stays below the live buffers' own size.
std::vector<void *> g_retired;

// grow-only device buffer
struct DevBuf {
    void *p = nullptr;
    size_t cap = 0;
    hipError_t ensure(size_t bytes) {
        if (bytes <= cap)
            return hipSuccess;
        size_t want = std::max(bytes, cap + cap / 2);
        want = (want + 255) & ~size_t(255);
        void *np = nullptr;
        hipError_t e = hipMalloc(&np, want);
        if (e != hipSuccess)
            return e;
        if (p)
            g_retired.push_back(p);
        p = np;
        cap = want;
        return hipSuccess;
    }
    void release() {
        if (p)
            (void)hipFree(p);
        p = nullptr;
        cap = 0;
    }
};

// grow-only pinned host buffer
struct HostBuf {
    void *p = nullptr;
    size_t cap = 0;
    hipError_t ensure(size_t bytes) {
        if (bytes <= cap)
            return hipSuccess;
        size_t want = std::max(bytes, cap + cap / 2);
        if (p)
            (void)hipHostFree(p);
        p = nullptr;
        cap = 0;
        hipError_t e = hipHostMalloc(&p, want, hipHostMallocDefault);
        if (e == hipSuccess)
            cap = want;
        return e;
    }
    void release() {
        if (p)
            (void)hipHostFree(p);
        p = nullptr;
        cap = 0;
    }
};

// One plan slot: pinned staging of the plan, its device copy, and an event that marks
// the end of the call that last used the slot.
struct PlanSlot {
    HostBuf host;
    DevBuf dev;
};

struct Resident {
    int layer = 0, eid = 0;
    const uint8_t *host = nullptr;
    size_t bytes = 0;
    void *dev = nullptr;
    hipEvent_t ready = nullptr;    // copy finished (copy stream)
    hipEvent_t last_use = nullptr; // last compute that read it
    bool used = false;
    std::list<long long>::iterator lru;
};

// Per-phase events of one call: start, after the input preparation (bf16 planes or MXFP4
// quantization of x), after the gate/up kernels, after the preparation of H (MXFP4
// quantization), after the down kernels, after the combine.  Phases a path does not have
// are empty spans.
struct TimedCall {
    hipEvent_t ev[6];
};

// ---- plan -------------------------------------------------------------------------

struct Plan {
    std::vector<ExpertWork> ew;     // active experts
    std::vector<int> src_expert;    // ew index -> caller's expert index e
    std::vector<int> xrow;          // compact row -> row of xg
    std::vector<int> dest;          // compact row -> destination row of out
    std::vector<float> w;           // compact row -> combine weight
    std::vector<int> tok_ptr, ent_row, out_row;
    std::vector<float> ent_w;
    int nr_max = 0;
    int D = 0, I = 0;
    std::vector<int> pos, order;  // build_plan's sort scratch
    // empties the plan, keeping every vector's storage (no heap traffic per call)
    void reset() {
        for (auto *v : {&src_expert, &xrow, &dest, &tok_ptr, &ent_row, &out_row})
            v->clear();
        ew.clear();
        w.clear();
        ent_w.clear();
        nr_max = D = I = 0;
    }
};

// How one call runs: the matrix-core path for both projections (activation planes,
// items of up to rmax rows), or the exact element-wise kernels.
struct PhaseCfg {
    int rmax = 0, ks = 1, nt = 1;  // rows per item, K split, tiles per wave
    size_t it0 = 0, it_split = 0, it1 = 0;  // item range; [it0, it_split) = experts < split
};

// Row-block class of the grouped GEMM: items of 16 * mt rows at most, in
// [it0, it1) of CallCfg::items; items of experts < split come first, up to it_split.
struct GemmCls {
    int mt = 0;
    size_t it0 = 0, it_split = 0, it1 = 0;
};

struct CallCfg {
    bool mfma = false;        // decode-shaped matrix-core kernels
    bool gemm = false;        // grouped GEMM (prefill-shaped)
    bool fp4 = false;         // grouped GEMM on native MXFP4 activations (option fp4act)
    bool f32 = false;         // fmt 0: the f32 matrix-core GEMM (kern_f32.hip)
    bool atomic_combine = false;  // decode kernels: combine folded into down (float atomics)
    bool w16 = false;         // every weight pointer 16-byte aligned (the wide-tile GEMM)
    int terms = 2;            // bf16 terms per activation (3: exact, 2: 2^-17, 1: bf16)
    PhaseCfg gu, dn;
    std::vector<int> items;   // {expert, r0, nrow, 0} records of both phases
    GemmCls gcls[kGemmClasses];
    int n_gcls = 0;
    std::vector<int> per[kGemmClasses];  // plan_gemm's per-class scratch
    // the default configuration, keeping the vectors' storage
    void reset() {
        mfma = gemm = fp4 = f32 = atomic_combine = w16 = false;
        terms = 2;
        gu = dn = PhaseCfg();
        items.clear();
        n_gcls = 0;
    }
};

struct Ctx {
    std::mutex mu;
    bool ready = false;
    int device = -1;
    hipStream_t own = nullptr;   // compute stream for the host-pointer entry
    hipStream_t copy = nullptr;  // promotions / misses
    hipStream_t last_stream = nullptr;
    // Ordering after the previous call (another stream, the miss copies): recorded on the
    // previous call's stream when such a call comes, not after every call.  Every event
    // recorded is a queue packet that idles the GPU between two calls' kernels (~4.6 us).
    hipEvent_t prev_done = nullptr;
    hipEvent_t miss_done = nullptr;  // the staged path's miss copies (copy stream)
    void *scratch_ptr = nullptr;     // device address of `scratch` on `device`
    bool have_last = false;
    DevBuf H, Y, Xc, Oc, miss, Ph, HP, Xp;
    DevBuf Lp;  // planes of mvllm_hip_linear_dev's input rows
    DevBuf Rp;  // device plan of mvllm_hip_moe_block_routed_dev
    HostBuf hx, ho;
    // the plan and configuration of the current call (every entry holds mu), reused
    Plan plan;
    CallCfg cfg;
    // Plan slots, reused in groups of kGroup: one event after a group's last call guards
    // the reuse of all its slots.  A group whose last call did not reach finish_call is
    // drained before its slots are reused (open_last).
    static constexpr int kSlots = 8, kGroup = 4;
    PlanSlot slots[kSlots];
    hipEvent_t grp_done[kSlots / kGroup] = {};
    bool grp_used[kSlots / kGroup] = {};
    int slot_next = 0, open_last = -1;
    // options
    int mode = 0;
    int timing = 0;
    int dequant_path = 0;    // mvllm_hip_dequant: 0 f32 decode, 1 matrix-core bf16 decode
    int dec_ks = 0;          // K split of the decode GEMM: 0 auto, 1, 2, 4 or 8
    int gemm = 0;            // grouped GEMM: 0 auto, 1 whenever it applies, 2 never
    int fp4act = 0;          // MXFP4 experts: 1 = quantize activations, native FP4 GEMMs
    int combine_ordered = 0;  // 1 = separate combine in the reference's order (decode too)
    int dec_inline = 1;      // decode: gate/up descriptors in the kernel arguments when they fit
    // residency
    size_t budget = size_t(64) << 30;
    size_t used_bytes = 0;
    size_t parked_bytes = 0;  // blocks of dropped blobs held until their layer's tables close
    std::unordered_map<long long, Resident> res;  // key = (layer << 32) | eid
    std::map<const uint8_t *, long long> by_host;  // host blob start -> key
    std::list<long long> lru;                      // front = most recent
    std::multimap<size_t, void *> free_blocks;     // recycled device blocks by size
    // per layer: the end of the last compute that read a tier table of it
    // (mvllm_hip_tier_table_done); a blob of the layer is recycled only after it
    std::unordered_map<int, hipEvent_t> layer_use;
    // per layer: tables handed out and not yet closed by mvllm_hip_tier_table_done, and
    // the blocks of the layer's blobs dropped meanwhile (their readers may still be
    // unrecorded: the blocks are recycled when the last open table is closed)
    std::unordered_map<int, int> layer_open;
    std::unordered_map<int, std::vector<std::pair<size_t, void *>>> layer_parked;
    // pinned staging of tier tables of more than kArgWords entries, a ring guarded by one
    // event per entry
    static constexpr int kTabSlots = 8, kTabMax = 8192;
    HostBuf tab_host[kTabSlots];
    hipEvent_t tab_done[kTabSlots] = {};
    bool tab_used[kTabSlots] = {};
    int tab_next = 0;
    hipEvent_t tier_ready = nullptr;  // copy stream: every promotion enqueued so far
    // copies enqueued on the copy stream so far, and as of tier_ready's last record
    unsigned long long copy_epoch = 0, tier_epoch = 0;
    std::vector<std::pair<size_t, void *>> pending_free;
    // stats
    double stats[20] = {0};
    std::vector<TimedCall> timed;
};

Ctx &ctx() {
    static Ctx c;
    return c;
}

// ---- device memory of the no-allocation entry (mvllm_hip_moe_block_dev_noalloc) -----
// One array per device, held until the process ends: the plan's device copy in the first
// kScratchPlan bytes, then the call's buffers.  Host code must not pass `scratch` itself
// to a kernel or a copy (in host code it names a host-side stand-in): mvllm_hip_init
// looks up its device address with hipGetSymbolAddress and keeps it in Ctx::scratch_ptr.
constexpr size_t kScratchBytes = size_t(48) << 20;
constexpr size_t kScratchPlan = size_t(256) << 10;
static __device__ __attribute__((aligned(256))) char scratch[kScratchBytes];

// Host time spent inside an entry point, added to stats[15] (ms) when the scope ends.
struct HostClock {
    double *acc;
    std::chrono::steady_clock::time_point t0 = std::chrono::steady_clock::now();
    explicit HostClock(double *a) : acc(a) {}
    ~HostClock() {
        *acc += std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0)
                    .count();
    }
};

long long res_key(int layer, int eid) {
    return (static_cast<long long>(layer) << 32) | static_cast<unsigned>(eid);
}

size_t piece_bytes(int fmt, int piece, int D, int I) {
    // piece: 0 gate/up packed, 1 gate/up scales, 2 down packed, 3 down scales
    const size_t O = piece < 2 ? (size_t)I : (size_t)D;
    const size_t K = piece < 2 ? (size_t)D : (size_t)I;
    if (fmt == 0)
        return (piece & 1) ? 0 : O * K * 4;
    if (piece & 1)
        return fmt == 4 ? O * ((K + 63) / 64) * 4 : O * ((K + 31) / 32);
    return O * ((K + 1) / 2);
}

// Reference skip rules and row filtering (src/gpu/metal_ops.cpp:283-339).
void build_plan(Plan &P, int nb, int D, int Iinter, int fmt, const void *const *g,
                const void *const *u, const void *const *d, const float *const *gs,
                const float *const *us, const float *const *ds, const int *xoff, const int *nr,
                const int *rows, const float *rw, int S) {
    P.reset();
    P.D = D;
    P.I = Iinter;
    size_t total = 0;
    for (int e = 0; e < nb; ++e)
        total += nr[e] > 0 ? (size_t)nr[e] : 0;
    P.xrow.reserve(total);
    P.dest.reserve(total);
    P.w.reserve(total);
    P.ew.reserve(nb);
    P.src_expert.reserve(nb);
    int base = 0, max_dest = -1;
    for (int e = 0; e < nb; ++e) {
        const int nre = nr[e];
        if (nre <= 0)
            continue;
        bool ok = Iinter >= 1 && g && u && d && g[e] && u[e] && d[e];
        if (ok && (fmt == 4 || fmt == 7))
            ok = gs && us && ds && gs[e] && us[e] && ds[e];
        if (ok && rows && rw) {
            ExpertWork w{};
            w.w[0] = g[e];
            w.w[1] = u[e];
            w.w[2] = d[e];
            if (fmt != 0) {
                w.s[0] = gs[e];
                w.s[1] = us[e];
                w.s[2] = ds[e];
            }
            w.row0 = static_cast<int>(P.xrow.size());
            for (int r = 0; r < nre; ++r) {
                const int dst = rows[base + r];
                if (dst < 0 || (S > 0 && dst >= S))
                    continue;
                P.xrow.push_back(xoff[e] + r);
                P.dest.push_back(dst);
                P.w.push_back(rw[base + r]);
                max_dest = std::max(max_dest, dst);
            }
            w.nrows = static_cast<int>(P.xrow.size()) - w.row0;
            if (w.nrows > 0) {
                P.ew.push_back(w);
                P.src_expert.push_back(e);
                P.nr_max = std::max(P.nr_max, w.nrows);
            }
        }
        base += nre;
    }
    // Combine CSR over destination rows (ascending), each row's entries in compact-row
    // (= expert) order: a stable counting sort by destination (a comparison sort of the
    // rows took 1.2 ms per call at 16,384 rows); destinations spread far beyond the row
    // count (host entry with S <= 0) take the comparison sort.
    const int R = static_cast<int>(P.dest.size());
    P.ent_row.resize(R);
    P.ent_w.resize(R);
    if ((size_t)max_dest + 1 <= 4 * (size_t)R + 4096) {
        std::vector<int> &pos = P.pos;
        pos.assign((size_t)max_dest + 2, 0);
        for (int j = 0; j < R; ++j)
            ++pos[(size_t)P.dest[j] + 1];
        for (int t = 0; t <= max_dest; ++t) {
            if (pos[(size_t)t + 1]) {
                P.tok_ptr.push_back(pos[t]);
                P.out_row.push_back(t);
            }
            pos[(size_t)t + 1] += pos[t];
        }
        for (int j = 0; j < R; ++j) {
            const int at = pos[P.dest[j]]++;
            P.ent_row[at] = j;
            P.ent_w[at] = P.w[j];
        }
    } else {
        std::vector<int> &order = P.order;
        order.resize(R);
        for (int j = 0; j < R; ++j)
            order[j] = j;
        std::stable_sort(order.begin(), order.end(),
                         [&](int a, int b) { return P.dest[a] < P.dest[b]; });
        for (int i = 0; i < R; ++i) {
            const int j = order[i];
            if (i == 0 || P.dest[j] != P.dest[order[i - 1]]) {
                P.tok_ptr.push_back(i);
                P.out_row.push_back(P.dest[j]);
            }
            P.ent_row[i] = j;
            P.ent_w[i] = P.w[j];
        }
    }
    P.tok_ptr.push_back(R);
}

bool aligned(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Does the decode kernel take this phase shape (K split ks, nt tiles per wave)?
bool dec_fits(int fmt, int K, int O, int rmax, int terms, bool dual, int ks, int nt) {
    const int tiles_wg = (kDecWaves / ks) * (dual ? 1 : nt);
    if (K % 512 || K % (256 * ks) || K / ks > dec_max_kr(fmt) || O % (16 * tiles_wg) ||
        (dual && nt != 2) || (nt == 2 && !dual && ks != 1))
        return false;
    const size_t stage = dual ? (size_t)rmax * (K / 8)
                              : (size_t)terms * rmax * (K / 8);
    const size_t cap = (size_t)(dual ? kDecStageDual : kDecStageSingle) * kDecThreads;
    return stage <= cap && mfma_dec_lds_bytes(fmt, K, rmax, terms, dual, ks, nt) <= kDecLdsBudget;
}

// (ks, nt) choices of a phase: dual waves always carry a gate and an up tile.
constexpr int kDecOpts[2][5][2] = {
    {{1, 2}, {1, 1}, {2, 1}, {4, 1}, {8, 1}},   // single (down)
    {{1, 2}, {2, 2}, {4, 2}, {8, 2}, {0, 0}}};  // dual (gate/up)

// Largest rows-per-item (<= want) that fits with some (ks, nt); 0 if none.
int pick_rmax(int fmt, int K, int O, int terms, bool dual, int want) {
    for (int r = std::min(16, want); r > 0; --r)
        for (const auto &kt : kDecOpts[dual ? 1 : 0])
            if (kt[0] && dec_fits(fmt, K, O, r, terms, dual, kt[0], kt[1]))
                return r;
    return 0;
}

// The (ks, nt) of a decode phase of n_items items of up to rmax rows; false if none fits.
// Each wave streams nt tiles x K/ks.  Cost of an admissible (ks, nt): the busiest of
// the 256 CUs runs n = ceil(workgroups / 256) workgroups, each its waves' blocks plus a
// ramp of ~4 blocks; two workgroups sharing a CU overlap by ~15 %.  Ties keep the
// smaller split.  This picks the fastest choice measured on MI355X at c1 T = 1, 2, 4, 8
// and 16 and at c2, for both projections.
bool pick_kt(const Ctx &C, int fmt, int K, int O, int rmax, int terms, bool dual,
             size_t n_items, PhaseCfg &ph) {
    const size_t tiles = n_items * (size_t)(O / 16) * (dual ? 2 : 1);  // 16-row weight tiles
    double best = 1e30;
    for (const auto &kt : kDecOpts[dual ? 1 : 0]) {
        if (!kt[0] || !dec_fits(fmt, K, O, rmax, terms, dual, kt[0], kt[1]))
            continue;
        if (C.dec_ks && kt[0] != C.dec_ks)
            continue;
        const size_t wgs = tiles * (size_t)kt[0] / ((size_t)kDecWaves * (size_t)kt[1]);
        const double per_cu = (double)((wgs + 255) / 256);
        const double cost = per_cu * ((double)(K / 256) * kt[1] / kt[0] + 4.0) /
                            (per_cu >= 2 ? 1.15 : 1.0);
        if (cost < best - 1e-9) {
            best = cost;
            ph.ks = kt[0];
            ph.nt = kt[1];
        }
    }
    ph.rmax = rmax;
    return best < 1e30;
}

bool add_phase(const Ctx &C, CallCfg &cc, PhaseCfg &ph, const Plan &P, size_t split, int fmt,
               int K, int O, bool dual) {
    // LDS holds activations for the largest item actually present, within the limits
    int most = 1;
    for (const ExpertWork &w : P.ew)
        most = std::max(most, w.nrows);
    const int rmax = pick_rmax(fmt, K, O, cc.terms, dual, most);
    if (rmax < 1)
        return false;
    size_t n_items = 0;
    for (const ExpertWork &w : P.ew)
        n_items += (size_t)((w.nrows + rmax - 1) / rmax);
    if (!pick_kt(C, fmt, K, O, rmax, cc.terms, dual, n_items, ph))
        return false;
    ph.it0 = cc.items.size() / 4;
    ph.it_split = ph.it0;
    for (size_t i = 0; i < P.ew.size(); ++i) {
        if (i == split)
            ph.it_split = cc.items.size() / 4;
        for (int r0 = 0; r0 < P.ew[i].nrows; r0 += ph.rmax) {
            cc.items.push_back(static_cast<int>(i));
            cc.items.push_back(r0);
            cc.items.push_back(std::min(ph.rmax, P.ew[i].nrows - r0));
            cc.items.push_back(0);
        }
    }
    ph.it1 = cc.items.size() / 4;
    if (split >= P.ew.size())
        ph.it_split = ph.it1;
    return true;
}

// Grouped-GEMM items: each expert's rows in blocks of 16 * max_mt, the remainder in the
// smallest class that holds it; classes ordered by mt, experts ascending within each.
void plan_gemm(CallCfg &cc, const Plan &P, size_t split, int fmt) {
    cc.terms = cc.terms >= 2 ? 2 : 1;
    const int max_mt = cc.f32 ? 4 : cc.fp4 ? kFp4MaxMt : gemm_max_mt(fmt, cc.terms);
    const int bm = 16 * max_mt;
    // bf16 one-term GEMM: an expert of 33-64 rows (a last block of that size) runs as two
    // 32-row items of the two-workgroups-per-CU class, which read its weights together
    const bool split64 = !cc.f32 && !cc.fp4 && cc.terms == 1 && max_mt >= 4;
    std::vector<int> *per = cc.per;  // class index = log2(mt)
    for (int c = 0; c < kGemmClasses; ++c)
        per[c].clear();
    size_t split_at[kGemmClasses] = {};
    for (size_t i = 0; i < P.ew.size(); ++i) {
        if (i == split)
            for (int c = 0; c < kGemmClasses; ++c)
                split_at[c] = per[c].size();
        const int n = P.ew[i].nrows;
        for (int r0 = 0; r0 < n; r0 += bm) {
            const int nrow = std::min(bm, n - r0);
            if (split64 && nrow > 32 && nrow <= 64) {
                per[1].insert(per[1].end(), {static_cast<int>(i), r0, 32, 0,
                                             static_cast<int>(i), r0 + 32, nrow - 32, 0});
                continue;
            }
            int c = 0;  // smallest class of 16 * 2^c rows that holds the block
            while ((16 << c) < nrow)
                ++c;
            per[c].insert(per[c].end(), {static_cast<int>(i), r0, nrow, 0});
        }
    }
    if (split >= P.ew.size())
        for (int c = 0; c < kGemmClasses; ++c)
            split_at[c] = per[c].size();
    // 4th word: (block index within the expert's run of items in this class) << 16 | run
    // length; the scaled-FP4 kernels and the 16/32-row bf16 kernels order an expert's
    // tasks column block by column block with these (runs of 2^15 blocks or more stay one
    // item per run)
    for (int c = 0; c < kGemmClasses; ++c) {
        std::vector<int> &v = per[c];
        for (size_t j = 0; j < v.size();) {
            size_t e = j;
            while (e < v.size() && v[e] == v[j])
                e += 4;
            const int n = static_cast<int>((e - j) / 4);
            for (int r = 0; r < n; ++r)
                v[j + 4 * r + 3] = n < 0x8000 ? (r << 16) | n : 1;
            j = e;
        }
    }
    cc.items.clear();
    cc.n_gcls = 0;
    for (int c = 0; c < kGemmClasses; ++c) {
        if (per[c].empty())
            continue;
        GemmCls &g = cc.gcls[cc.n_gcls++];
        g.mt = 1 << c;
        g.it0 = cc.items.size() / 4;
        g.it_split = g.it0 + split_at[c] / 4;
        cc.items.insert(cc.items.end(), per[c].begin(), per[c].end());
        g.it1 = cc.items.size() / 4;
    }
    cc.gemm = !cc.f32;
}

// ordered: the combine keeps the reference's expert order even for decode-shaped calls
// (no float-atomic fold into the down kernel).
void plan_call(const Ctx &C, CallCfg &cc, const Plan &P, int fmt, int D, int I, size_t split,
               const void *in, bool ordered) {
    cc.reset();
    // bf16 terms per activation: 2 (default) represents each f32 activation to 2^-17
    // relative, 3 exactly (mode 1), 1 is plain bf16 (mode 2).  The grouped GEMM takes
    // 1 term by default (bf16 activations, the prefill arithmetic) and 2 in mode 1.
    cc.terms = C.mode == 1 ? 3 : C.mode == 2 ? 1 : 2;
    bool ok = (fmt == 4 || fmt == 7) && D % 256 == 0 && I % 256 == 0 && D <= kDecMaxK &&
              I <= kDecMaxK && aligned(in, 16);
    bool gok = (fmt == 4 || fmt == 7) && D % 256 == 0 && I % 256 == 0 && aligned(in, 16);
    // fmt 0 (f32 weights, the shared experts): the f32 matrix-core GEMM for every row count
    if (fmt == 0 && f32mm_fits(true, D, I) && f32mm_fits(false, I, D) && aligned(in, 16)) {
        bool al = true;
        for (const ExpertWork &w : P.ew)
            for (int m = 0; m < 3; ++m)
                al = al && aligned(w.w[m], 16);
        if (al) {
            cc.f32 = true;
            plan_gemm(cc, P, split, fmt);
            return;
        }
    }
    const size_t walign = fmt == 7 && C.fp4act ? 16 : 8;  // the FP4 GEMM loads 16-byte rows
    int most = 0;
    bool w16 = true;
    for (const ExpertWork &w : P.ew) {
        most = std::max(most, w.nrows);
        for (int m = 0; m < 3; ++m)
            w16 = w16 && aligned(w.w[m], 16);
        for (int m = 0; m < 3; ++m) {
            ok = ok && aligned(w.w[m], 16) && aligned(w.s[m], fmt == 4 ? 16 : 8);
            gok = gok && aligned(w.w[m], walign) && aligned(w.s[m], fmt == 4 ? 16 : 8);
        }
    }
    // native MXFP4 activations (opt-in): the scaled FP4 GEMM for every row count
    if (fmt == 7 && C.fp4act && gok) {
        cc.fp4 = true;
        plan_gemm(cc, P, split, fmt);
        return;
    }
    // grouped GEMM when forced, or when some expert has more rows than one decode item
    if (gok && C.gemm != 2 && (C.gemm == 1 || most > 16)) {
        cc.terms = C.mode == 1 ? 2 : 1;
        plan_gemm(cc, P, split, fmt);
        cc.w16 = w16;
        return;
    }
    if (ok && pick_rmax(fmt, D, I, cc.terms, true, 1) >= 1 &&
        pick_rmax(fmt, I, D, cc.terms, false, 1) >= 1) {
        cc.mfma = add_phase(C, cc, cc.gu, P, split, fmt, D, I, true) &&
                  add_phase(C, cc, cc.dn, P, P.ew.size(), fmt, I, D, false);
        if (cc.mfma) {
            // decode-sized outputs: fold the combine into the down kernel (one launch less);
            // an ordered call keeps the reference's summation order instead
            cc.atomic_combine = !ordered;
            return;
        }
        cc.items.clear();
    }
    if (gok && C.gemm != 2) {  // decode-shaped call the decode kernels do not fit: keep
        cc.terms = C.mode == 2 ? 1 : 2;  // the decode accuracy (2 terms) unless mode 2
        plan_gemm(cc, P, split, fmt);
    }
}

// Device scratch of one call: the exact path's f32 H; the matrix-core paths' H planes
// Ph (+ int4 partial sums HP); the down output Y (not written when the decode kernels fold
// the combine into out); the grouped GEMM's input planes (or MXFP4 codes) Xp.
struct Bufs {
    void *H = nullptr, *Y = nullptr, *Ph = nullptr, *HP = nullptr, *Xp = nullptr;
};

// Bytes of each buffer of Bufs that a call of R compact rows uses (0 = unused).
void buf_sizes(const CallCfg &cc, size_t R, int D, int I, size_t sz[5]) {
    const size_t tb = (size_t)cc.terms * 2;
    for (int i = 0; i < 5; ++i)
        sz[i] = 0;
    if (cc.f32) {
        sz[0] = R * I * 4;
        sz[1] = R * D * 4;
    } else if (cc.fp4) {
        sz[0] = R * I * 4;
        sz[1] = R * D * 4;
        sz[2] = R * (I / 2 + I / 32);
        bool bf = false;  // bf16 planes of the quantized x and H (kFp4BfMaxMt)
        for (int c = 0; c < cc.n_gcls; ++c)
            bf = bf || cc.gcls[c].mt <= kFp4BfMaxMt;
        sz[3] = bf ? R * (D + I) * 2 : 0;
        sz[4] = R * (D / 2 + D / 32);
    } else if (cc.gemm) {
        sz[1] = R * D * 4;
        sz[2] = tb * R * I;
        sz[4] = tb * R * D;
    } else if (cc.mfma) {
        sz[1] = cc.atomic_combine ? 0 : R * D * 4;
        sz[2] = tb * R * I;
        sz[3] = (size_t)(I / 64) * 4 * R * 4;
    } else {
        sz[0] = R * I * 4;
        sz[1] = R * D * 4;
    }
}

// The call's buffers from the library's grow-only device buffers.
hipError_t get_bufs(Ctx &C, const CallCfg &cc, size_t R, int D, int I, Bufs &B) {
    size_t sz[5];
    buf_sizes(cc, R, D, I, sz);
    DevBuf *db[5] = {&C.H, &C.Y, &C.Ph, &C.HP, &C.Xp};
    void **dst[5] = {&B.H, &B.Y, &B.Ph, &B.HP, &B.Xp};
    for (int i = 0; i < 5; ++i) {
        if (!sz[i])
            continue;
        hipError_t e = db[i]->ensure(sz[i]);
        if (e != hipSuccess)
            return e;
        *dst[i] = db[i]->p;
    }
    return hipSuccess;
}

// Upload the plan (experts, xrow, combine CSR, items) through a pinned slot; returns
// device pointers into the slot's device buffer, or into dev_dst (dev_cap bytes) when
// given, in which case nothing is allocated: the slot's pinned buffer must already hold
// the plan.
struct DevPlan {
    ExpertWork *ew;
    int *xrow, *tok_ptr, *ent_row, *out_row, *items, *rdest;
    float *ent_w, *rw;
    DecDesc *gu_desc, *dn_desc;  // decode kernels: one descriptor per item of each phase
    DecDesc *dn_desc_dev;        // dn_desc in device memory (a copy the gate/up kernel makes)
    uint8_t *pmask;              // native FP4: 1 for the compact rows that get bf16 planes
    const DecDesc *gu_host;      // gu_desc's copy in the pinned slot (host memory)
    int slot;  // plan slot index
};

// Decode descriptors of items [i0, i1) of cc.items.  Dual: the expert's gate and up, and
// the input row of each item row (x row through the compact-row map, or the compact row
// itself); single: the down matrix and, with the folded combine, each row's out row and
// weight.
void build_desc(const Plan &P, const CallCfg &cc, size_t i0, size_t i1, bool dual,
                bool rows_identity, const int *rdest, DecDesc *d) {
    for (size_t it = i0; it < i1; ++it, ++d) {
        std::memset(d, 0, sizeof(DecDesc));
        const ExpertWork &w = P.ew[cc.items[4 * it]];
        const int r0 = cc.items[4 * it + 1], nrow = cc.items[4 * it + 2];
        d->w[0] = dual ? w.w[0] : w.w[2];
        d->w[1] = dual ? w.w[1] : w.w[2];
        d->s[0] = dual ? w.s[0] : w.s[2];
        d->s[1] = dual ? w.s[1] : w.s[2];
        d->jbase = w.row0 + r0;
        d->nrow = nrow;
        for (int r = 0; r < nrow; ++r) {
            const int j = d->jbase + r;
            if (dual) {
                d->rows[r] = rows_identity ? j : P.xrow[j];
            } else {
                d->rows[r] = rdest[j];
                d->wts[r] = P.w[j];
            }
        }
    }
}

// The compact (kernel-argument) form of gate/up descriptors d[0, n); false when some
// descriptor does not fit it (more than kDecInline, an offset beyond 32 bits, a row index
// beyond 16 bits).
bool compact_desc(const DecDesc *d, int n, DecDescK *k) {
    if (n > kDecInline)
        return false;
    for (int i = 0; i < n; ++i) {
        const uintptr_t w0 = reinterpret_cast<uintptr_t>(d[i].w[0]);
        const uintptr_t p[3] = {reinterpret_cast<uintptr_t>(d[i].w[1]),
                                reinterpret_cast<uintptr_t>(d[i].s[0]),
                                reinterpret_cast<uintptr_t>(d[i].s[1])};
        k[i].w0 = d[i].w[0];
        for (int m = 0; m < 3; ++m) {
            const long long off = static_cast<long long>(p[m] - w0);
            if (off < INT32_MIN || off > INT32_MAX)
                return false;
            k[i].off[m] = static_cast<int>(off);
        }
        if (d[i].jbase < 0 || d[i].jbase > 65535 || d[i].nrow < 0 || d[i].nrow > 16)
            return false;
        k[i].jbase = static_cast<unsigned short>(d[i].jbase);
        k[i].nrow = static_cast<unsigned short>(d[i].nrow);
        for (int r = 0; r < 16; ++r) {
            if (d[i].rows[r] < 0 || d[i].rows[r] > 65535)
                return false;
            k[i].rows[r] = static_cast<unsigned short>(d[i].rows[r]);
        }
    }
    return true;
}

int upload_plan(Ctx &C, const Plan &P, const CallCfg &cc, hipStream_t st, DevPlan &dp,
                bool rows_identity, void *dev_dst = nullptr, size_t dev_cap = 0) {
    if (C.open_last >= 0) {  // a group's last call stopped early: its event is stale
        HIP_TRY(hipDeviceSynchronize());
        C.grp_used[C.open_last / Ctx::kGroup] = false;
        C.open_last = -1;
    }
    const int si = C.slot_next;
    PlanSlot &s = C.slots[si];
    C.slot_next = (si + 1) % Ctx::kSlots;
    const int gi = si / Ctx::kGroup;
    if (si % Ctx::kGroup == 0 && C.grp_used[gi]) {
        // the group's previous calls are done (time blocked here: stats[16])
        const auto t0 = std::chrono::steady_clock::now();
        HIP_TRY(hipEventSynchronize(C.grp_done[gi]));
        C.stats[16] += std::chrono::duration<double, std::milli>(
                           std::chrono::steady_clock::now() - t0).count();
    }
    if (si % Ctx::kGroup == Ctx::kGroup - 1)
        C.open_last = si;
    auto al = [](size_t n) { return (n + 255) & ~size_t(255); };
    const size_t b_ew = al(P.ew.size() * sizeof(ExpertWork));
    const size_t b_x = al(P.xrow.size() * 4), b_tp = al(P.tok_ptr.size() * 4);
    const size_t b_er = al(P.ent_row.size() * 4), b_or = al(P.out_row.size() * 4);
    const size_t b_ew2 = al(P.ent_w.size() * 4), b_it = al(cc.items.size() * 4);
    const size_t R = P.xrow.size();
    const size_t b_rd = al(R * 4), b_rw = al(R * 4);
    const size_t n_gu = cc.mfma ? cc.gu.it1 - cc.gu.it0 : 0;
    const size_t n_dn = cc.mfma ? cc.dn.it1 - cc.dn.it0 : 0;
    const size_t b_dg = n_gu * sizeof(DecDesc), b_dd = n_dn * sizeof(DecDesc);
    const size_t b_pm = cc.fp4 ? al(R) : 0;  // native FP4: rows with bf16 planes
    const size_t total =
        b_ew + b_x + b_tp + b_er + b_or + b_ew2 + b_it + b_rd + b_rw + b_dg + b_dd + b_pm;
    if (dev_dst) {
        if (total > s.host.cap || total > dev_cap) {
            set_err("plan of " + std::to_string(total) + " bytes exceeds the preallocated " +
                    std::to_string(std::min(s.host.cap, dev_cap)) + "-byte plan buffers");
            if (si % Ctx::kGroup == Ctx::kGroup - 1)
                C.open_last = -1;  // nothing of this call was enqueued
            C.slot_next = si;
            return 0;
        }
    } else if (total > s.host.cap || total > s.dev.cap) {
        // Every slot grows together, once per new plan size: freeing pinned memory drains
        // the device, and slots growing one by one on their first use at a size would
        // drain it once per slot, in the middle of a stream of calls.
        HIP_TRY(hipDeviceSynchronize());
        for (auto &g : C.grp_used)
            g = false;  // every earlier call is done
        const size_t want = std::max(total, std::max(s.host.cap, s.dev.cap) * 3 / 2);
        for (PlanSlot &t : C.slots) {
            HIP_TRY(t.host.ensure(want));
            HIP_TRY(t.dev.ensure(want));
        }
    }
    char *dbase = dev_dst ? static_cast<char *>(dev_dst) : static_cast<char *>(s.dev.p);
    char *h = static_cast<char *>(s.host.p);
    size_t o = 0;
    auto put = [&](const void *src, size_t n, size_t b) {
        if (n)
            std::memcpy(h + o, src, n);
        const size_t at = o;
        o += b;
        return at;
    };
    const size_t o_ew = put(P.ew.data(), P.ew.size() * sizeof(ExpertWork), b_ew);
    const size_t o_x = put(P.xrow.data(), P.xrow.size() * 4, b_x);
    const size_t o_tp = put(P.tok_ptr.data(), P.tok_ptr.size() * 4, b_tp);
    const size_t o_er = put(P.ent_row.data(), P.ent_row.size() * 4, b_er);
    const size_t o_or = put(P.out_row.data(), P.out_row.size() * 4, b_or);
    const size_t o_w = put(P.ent_w.data(), P.ent_w.size() * 4, b_ew2);
    const size_t o_it = put(cc.items.data(), cc.items.size() * 4, b_it);
    // per compact row: its row of out (through the combine CSR) and its weight
    int *rdest = reinterpret_cast<int *>(h + o);
    for (size_t t = 0; t + 1 < P.tok_ptr.size(); ++t)
        for (int e = P.tok_ptr[t]; e < P.tok_ptr[t + 1]; ++e)
            rdest[P.ent_row[e]] = P.out_row[t];
    const size_t o_rd = o;
    o += b_rd;
    const size_t o_rw = put(P.w.data(), R * 4, b_rw);
    const size_t o_dg = o, o_dd = o + b_dg;
    if (cc.mfma) {
        build_desc(P, cc, cc.gu.it0, cc.gu.it1, true, rows_identity, rdest,
                   reinterpret_cast<DecDesc *>(h + o_dg));
        build_desc(P, cc, cc.dn.it0, cc.dn.it1, false, rows_identity, rdest,
                   reinterpret_cast<DecDesc *>(h + o_dd));
    }
    o += b_dg + b_dd;
    // native FP4: the compact rows of the classes that run the bf16 GEMM
    const size_t o_pm = o;
    if (b_pm) {
        uint8_t *pm = reinterpret_cast<uint8_t *>(h + o_pm);
        std::memset(pm, 0, R);
        for (int c = 0; c < cc.n_gcls; ++c) {
            const GemmCls &g = cc.gcls[c];
            if (g.mt > kFp4BfMaxMt)
                continue;
            for (size_t i = g.it0; i < g.it1; ++i) {
                const int *it = &cc.items[4 * i];
                std::memset(pm + P.ew[it[0]].row0 + it[1], 1, (size_t)it[2]);
            }
        }
        o += b_pm;
    }
    // The decode kernels with the folded combine read nothing of the plan but their
    // descriptors, and those straight from this pinned slot (no copy, no copy launch):
    // the slot is rewritten only after the call that read it has finished (above).
    const bool zero_copy = cc.mfma && cc.atomic_combine;
    char *d = static_cast<char *>(s.host.p);
    if (!zero_copy) {
        HIP_TRY(hipMemcpyAsync(dbase, s.host.p, total, hipMemcpyHostToDevice, st));
        d = dbase;
    }
    dp.ew = reinterpret_cast<ExpertWork *>(d + o_ew);
    dp.xrow = reinterpret_cast<int *>(d + o_x);
    dp.tok_ptr = reinterpret_cast<int *>(d + o_tp);
    dp.ent_row = reinterpret_cast<int *>(d + o_er);
    dp.out_row = reinterpret_cast<int *>(d + o_or);
    dp.ent_w = reinterpret_cast<float *>(d + o_w);
    dp.items = reinterpret_cast<int *>(d + o_it);
    dp.rdest = reinterpret_cast<int *>(d + o_rd);
    dp.rw = reinterpret_cast<float *>(d + o_rw);
    dp.gu_desc = reinterpret_cast<DecDesc *>(d + o_dg);
    dp.gu_host = reinterpret_cast<const DecDesc *>(h + o_dg);
    dp.dn_desc = reinterpret_cast<DecDesc *>(d + o_dd);
    dp.dn_desc_dev = reinterpret_cast<DecDesc *>(dbase + o_dd);
    dp.pmask = b_pm ? reinterpret_cast<uint8_t *>(d + o_pm) : nullptr;
    if (!zero_copy)
        dp.dn_desc_dev = dp.dn_desc;  // already there
    dp.slot = si;
    return 1;
}

// Scratch H/Y are shared by all calls: order this call after the previous one if it
// came on another stream.
// Makes `waiter` wait for everything enqueued so far on the previous call's stream.
int wait_previous(Ctx &C, hipStream_t waiter) {
    if (!C.have_last || C.last_stream == waiter)
        return 1;
    if (hipEventRecord(C.prev_done, C.last_stream) != hipSuccess) {
        // that stream is gone (destroyed after its call): drain the device instead
        (void)hipGetLastError();
        HIP_TRY(hipDeviceSynchronize());
        C.have_last = false;
        return 1;
    }
    HIP_TRY(hipStreamWaitEvent(waiter, C.prev_done, 0));
    return 1;
}

int order_after_previous(Ctx &C, hipStream_t st) { return wait_previous(C, st); }

int finish_call(Ctx &C, hipStream_t st, int si) {
    if (si % Ctx::kGroup == Ctx::kGroup - 1) {
        const int gi = si / Ctx::kGroup;
        HIP_TRY(hipEventRecord(C.grp_done[gi], st));
        C.grp_used[gi] = true;
        C.open_last = -1;
    }
    C.last_stream = st;
    C.have_last = true;
    return 1;
}

// One row class of the grouped GEMM: the 128-row blocks of MXFP4 experts in one-term
// bf16 arithmetic take the wide-tile kernel when the shapes and alignment allow.
hipError_t launch_gemm_cls(bool w16, int fmt, bool dual, int terms, int mt, const ExpertWork *ew,
                           const void *items, int n_items, const void *pin, void *pout,
                           float *out, int K, int O, int rcap, int act, float act_a, float act_b,
                           hipStream_t st, const int *n_items_dev = nullptr) {
    if (w16 && fmt == 7 && terms == 1 && mt == 8 && gemm_wide_fits(dual, K, O))
        return launch_gemm_wide(dual, ew, items, n_items, pin, pout, out, K, O, rcap, act, act_a,
                                act_b, st, n_items_dev);
    return launch_gemm(fmt, dual, terms, mt, ew, items, n_items, pin, pout, out, K, O, rcap, act,
                       act_a, act_b, st, n_items_dev);
}

GemvArgs generic_args(const DevPlan &dp, size_t first, size_t count, const int *in_rows,
                      const float *in, float *out, int K, int O, int act, float a, float b) {
    GemvArgs g{};
    g.ew = dp.ew + first;
    g.n_experts = static_cast<int>(count);
    g.in_rows = in_rows;
    g.in = in;
    g.out = out;
    g.K = K;
    g.O = O;
    g.act = act;
    g.act_a = a;
    g.act_b = b;
    g.rows_per_tile = 4;
    g.tiles_per_expert = (O + 3) / 4;
    return g;
}

// The phases of one call.  Experts [0, split) run gate/up first; a wait on `gate_event`
// (may be null) precedes gate/up of [split, n).
int run_phases(Ctx &C, const Plan &P, const CallCfg &cc, const DevPlan &dp, const Bufs &B,
               int fmt, int D, int I, int act, float a, float b, const float *in,
               const int *in_rows, float *out, hipStream_t st, size_t split,
               hipEvent_t gate_event, bool timed = true) {
    const bool timing = C.timing && timed;  // per-phase events (created per call)
    const size_t n = P.ew.size(), R = P.xrow.size();
    const int rcap = static_cast<int>(R);
    TimedCall tc{};
    if (timing) {
        // no system-scope release: its L2 write-back would sit inside the timed spans
        for (auto &e : tc.ev)
            HIP_TRY(hipEventCreateWithFlags(&e, hipEventDisableSystemFence));
    }
    // records the event that ends phase i (TimedCall), when timing
    auto mark = [&](int i) { return timing ? hipEventRecord(tc.ev[i], st) : hipSuccess; };
    HIP_TRY(mark(0));
    if (cc.fp4) {
        // activations quantized to MXFP4 (bit-exact with fp4_activation_qdq), the gate/up
        // GEMM writes H f32, H is quantized, the down GEMM writes Y.  The 16- and 32-row
        // classes run the bf16 grouped GEMM on the quantized values as bf16 planes (exact
        // copies of them, written by the quantizer): it streams those classes' weights
        // faster than the scaled-FP4 kernel, with the same exact products.
        uint8_t *xq = static_cast<uint8_t *>(B.Xp), *xsc = xq + R * (D / 2);
        uint8_t *hq = static_cast<uint8_t *>(B.Ph), *hsc = hq + R * (I / 2);
        float *H = static_cast<float *>(B.H);
        bool bf = false;
        for (int c = 0; c < cc.n_gcls; ++c)
            bf = bf || cc.gcls[c].mt <= kFp4BfMaxMt;
        __bf16 *xb = bf ? static_cast<__bf16 *>(B.HP) : nullptr;
        __bf16 *hb = bf ? xb + R * (size_t)D : nullptr;
        HIP_TRY(launch_quantize_mxfp4(in, rcap, D, xq, xsc, st, in_rows, xb, dp.pmask));
        HIP_TRY(mark(1));
        for (int part = 0; part < 2; ++part) {
            if (part == 1 && gate_event)
                HIP_TRY(hipStreamWaitEvent(st, gate_event, 0));
            for (int c = 0; c < cc.n_gcls; ++c) {
                const GemmCls &g = cc.gcls[c];
                const size_t i0 = part ? g.it_split : g.it0, i1 = part ? g.it1 : g.it_split;
                if (i1 <= i0)
                    continue;
                if (g.mt <= kFp4BfMaxMt)
                    HIP_TRY(launch_gemm(fmt, true, 1, g.mt, dp.ew, dp.items + 4 * i0,
                                        static_cast<int>(i1 - i0), xb, nullptr, H, D, I, rcap,
                                        act, a, b, st));
                else
                    HIP_TRY(launch_gemm_fp4(true, g.mt, dp.ew, dp.items + 4 * i0,
                                            static_cast<int>(i1 - i0), xq, xsc, H, nullptr, D,
                                            I, rcap, act, a, b, st));
                C.stats[13] += 1;
            }
        }
        HIP_TRY(mark(2));
        HIP_TRY(launch_quantize_mxfp4(H, rcap, I, hq, hsc, st, nullptr, hb, dp.pmask));
        HIP_TRY(mark(3));
        for (int c = 0; c < cc.n_gcls; ++c) {
            const GemmCls &g = cc.gcls[c];
            if (g.mt <= kFp4BfMaxMt)
                HIP_TRY(launch_gemm(fmt, false, 1, g.mt, dp.ew, dp.items + 4 * g.it0,
                                    static_cast<int>(g.it1 - g.it0), hb, nullptr,
                                    static_cast<float *>(B.Y), I, D, rcap, 0, 0.f, 0.f, st));
            else
                HIP_TRY(launch_gemm_fp4(false, g.mt, dp.ew, dp.items + 4 * g.it0,
                                        static_cast<int>(g.it1 - g.it0), hq, hsc, nullptr,
                                        static_cast<float *>(B.Y), I, D, rcap, 0, 0.f, 0.f,
                                        st));
            C.stats[14] += 1;
        }
    } else if (cc.f32) {
        // f32 matrix cores on the f32 rows themselves (no planes): gate/up + act -> H f32,
        // down -> Y
        HIP_TRY(mark(1));
        for (int part = 0; part < 2; ++part) {
            if (part == 1 && gate_event)
                HIP_TRY(hipStreamWaitEvent(st, gate_event, 0));
            for (int c = 0; c < cc.n_gcls; ++c) {
                const GemmCls &g = cc.gcls[c];
                const size_t i0 = part ? g.it_split : g.it0, i1 = part ? g.it1 : g.it_split;
                if (i1 <= i0)
                    continue;
                HIP_TRY(launch_f32mm(true, g.mt, dp.ew, dp.items + 4 * i0,
                                     static_cast<int>(i1 - i0), nullptr, 0, in, in_rows,
                                     static_cast<float *>(B.H), 0, D, I, act, a, b, st));
                C.stats[13] += 1;
            }
        }
        HIP_TRY(mark(2));
        HIP_TRY(mark(3));
        for (int c = 0; c < cc.n_gcls; ++c) {
            const GemmCls &g = cc.gcls[c];
            HIP_TRY(launch_f32mm(false, g.mt, dp.ew, dp.items + 4 * g.it0,
                                 static_cast<int>(g.it1 - g.it0), nullptr, 0,
                                 static_cast<const float *>(B.H), nullptr,
                                 static_cast<float *>(B.Y), 2, I, D, 0, 0.f, 0.f, st));
            C.stats[14] += 1;
        }
    } else if (cc.gemm) {
        HIP_TRY(launch_prep_planes(fmt, cc.terms, in, in_rows, rcap, D, rcap, B.Xp, st));
        HIP_TRY(mark(1));
        for (int part = 0; part < 2; ++part) {
            if (part == 1 && gate_event)
                HIP_TRY(hipStreamWaitEvent(st, gate_event, 0));
            for (int c = 0; c < cc.n_gcls; ++c) {
                const GemmCls &g = cc.gcls[c];
                const size_t i0 = part ? g.it_split : g.it0, i1 = part ? g.it1 : g.it_split;
                if (i1 <= i0)
                    continue;
                HIP_TRY(launch_gemm_cls(cc.w16, fmt, true, cc.terms, g.mt, dp.ew,
                                        dp.items + 4 * i0, static_cast<int>(i1 - i0), B.Xp, B.Ph,
                                        nullptr, D, I, rcap, act, a, b, st));
                C.stats[13] += 1;
            }
        }
        HIP_TRY(mark(2));
        HIP_TRY(mark(3));
        for (int c = 0; c < cc.n_gcls; ++c) {
            const GemmCls &g = cc.gcls[c];
            HIP_TRY(launch_gemm_cls(cc.w16, fmt, false, cc.terms, g.mt, dp.ew,
                                    dp.items + 4 * g.it0, static_cast<int>(g.it1 - g.it0), B.Ph,
                                    nullptr, static_cast<float *>(B.Y), I, D, rcap, 0, 0.f, 0.f,
                                    st));
            C.stats[14] += 1;
        }
    } else if (cc.mfma) {
        // the gate/up workgroups copy the down descriptors from the pinned plan slot to
        // device memory (when they are not there already), a descriptor a workgroup
        const int n_dn = static_cast<int>(cc.dn.it1 - cc.dn.it0);
        const int wgs_gu = I / (16 * (kDecWaves / cc.gu.ks));
        // Items of <= 8 rows with two terms: the packed kernels (both terms in one MFMA),
        // launched with that row capacity.
        auto max_rows = [&](size_t i0, size_t i1) {
            int m = 1;
            for (size_t i = i0; i < i1; ++i)
                m = std::max(m, cc.items[4 * i + 2]);
            return m;
        };
        const int mr_gu = max_rows(cc.gu.it0, cc.gu.it1), mr_dn = max_rows(cc.dn.it0, cc.dn.it1);
        const bool pk_gu = cc.terms == 2 && mr_gu <= 8, pk_dn = cc.terms == 2 && mr_dn <= 8;
        const int rmax_gu = pk_gu ? mr_gu : cc.gu.rmax, rmax_dn = pk_dn ? mr_dn : cc.dn.rmax;
        int copied = dp.dn_desc_dev == dp.dn_desc ? n_dn : 0;
        HIP_TRY(mark(1));
        for (int part = 0; part < 2; ++part) {
            const size_t i0 = part ? cc.gu.it_split : cc.gu.it0;
            const size_t i1 = part ? cc.gu.it1 : cc.gu.it_split;
            if (part == 1 && gate_event)
                HIP_TRY(hipStreamWaitEvent(st, gate_event, 0));
            if (i1 <= i0)
                continue;
            const int ncp = std::min(n_dn - copied, static_cast<int>(i1 - i0) * wgs_gu);
            const int ni = static_cast<int>(i1 - i0);
            DecDescK kd[kDecInline];
            const bool inl = C.dec_inline && compact_desc(dp.gu_host + (i0 - cc.gu.it0), ni, kd);
            HIP_TRY(launch_mfma_dec(fmt, true, cc.terms, cc.gu.ks, cc.gu.nt,
                                    dp.gu_desc + (i0 - cc.gu.it0), ni, in, nullptr, nullptr,
                                    B.Ph, static_cast<float *>(B.HP), nullptr, D, I, rcap,
                                    rmax_gu, act, a, b, false, pk_gu, dp.dn_desc + copied,
                                    dp.dn_desc_dev + copied, ncp, st, inl ? kd : nullptr));
            copied += ncp;
            C.stats[13] += 1;
        }
        if (copied < n_dn)  // more down items than gate/up workgroups
            HIP_TRY(hipMemcpyAsync(dp.dn_desc_dev + copied, dp.dn_desc + copied,
                                   (size_t)(n_dn - copied) * sizeof(DecDesc),
                                   hipMemcpyHostToDevice, st));
        HIP_TRY(mark(2));
        HIP_TRY(mark(3));
        HIP_TRY(launch_mfma_dec(fmt, false, cc.terms, cc.dn.ks, cc.dn.nt, dp.dn_desc_dev,
                                static_cast<int>(cc.dn.it1 - cc.dn.it0), nullptr, B.Ph,
                                static_cast<const float *>(B.HP), nullptr, nullptr,
                                cc.atomic_combine ? out : static_cast<float *>(B.Y), I, D,
                                rcap, rmax_dn, 0, 0.f, 0.f, cc.atomic_combine, pk_dn, nullptr,
                                nullptr, 0, st));
        C.stats[14] += 1;
    } else {
        HIP_TRY(mark(1));
        for (int part = 0; part < 2; ++part) {
            const size_t first = part == 0 ? 0 : split, cnt = part == 0 ? split : n - split;
            if (part == 1 && gate_event)
                HIP_TRY(hipStreamWaitEvent(st, gate_event, 0));
            if (!cnt)
                continue;
            HIP_TRY(launch_gemv_generic(fmt, true,
                                        generic_args(dp, first, cnt, in_rows, in,
                                                     static_cast<float *>(B.H), D, I, act, a, b),
                                        st));
            C.stats[13] += 1;
        }
        HIP_TRY(mark(2));
        HIP_TRY(mark(3));
        HIP_TRY(launch_gemv_generic(fmt, false,
                                    generic_args(dp, 0, n, nullptr,
                                                 static_cast<const float *>(B.H),
                                                 static_cast<float *>(B.Y), I, D, 0, 0.f, 0.f),
                                    st));
        C.stats[14] += 1;
    }
    HIP_TRY(mark(4));
    if (cc.atomic_combine) {  // already folded into the down kernel
        if (timing) {
            HIP_TRY(mark(5));
            C.timed.push_back(tc);
        }
        C.stats[1] += static_cast<double>(R);
        return 1;
    }
    CombineArgs cb{};
    cb.Y = static_cast<const float *>(B.Y);
    cb.tok_ptr = dp.tok_ptr;
    cb.ent_row = dp.ent_row;
    cb.ent_w = dp.ent_w;
    cb.out_row = dp.out_row;
    cb.out = out;
    cb.n_tok = static_cast<int>(P.out_row.size());
    cb.D = D;
    HIP_TRY(launch_combine(cb, st));
    if (timing) {
        HIP_TRY(mark(5));
        C.timed.push_back(tc);
    }
    C.stats[1] += static_cast<double>(R);
    return 1;
}

// One mvllm_hip_moe_block_dev call (arguments validated).  noalloc: every device buffer
// comes from the scratch array (the plan's copy first, then the call's Bufs), nothing is
// allocated, calls that do not fit are refused, and option "timing" is ignored.
int dev_call(Ctx &C, int nb, int D, int Iinter, int fmt, const void *const *g,
             const void *const *u, const void *const *d, const float *const *gs,
             const float *const *us, const float *const *ds, const float *xg, const int *xoff,
             const int *nr, const int *rows, const float *rw, float *out, int S, int act,
             float act_a, float act_b, hipStream_t st, bool noalloc) {
    HostClock hc(&C.stats[15]);
    Plan &P = C.plan;
    build_plan(P, nb, D, Iinter, fmt, g, u, d, gs, us, ds, xoff, nr, rows, rw, S);
    C.stats[0] += 1;
    if (P.ew.empty())
        return 1;
    const size_t R = P.xrow.size();
    CallCfg &cc = C.cfg;
    plan_call(C, cc, P, fmt, D, Iinter, P.ew.size(), xg, C.combine_ordered != 0);
    Bufs B;
    if (noalloc) {  // carve the buffers out of the scratch array, after the plan region
        size_t sz[5], off = kScratchPlan;
        buf_sizes(cc, R, D, Iinter, sz);
        void **dst[5] = {&B.H, &B.Y, &B.Ph, &B.HP, &B.Xp};
        for (int i = 0; i < 5; ++i) {
            if (!sz[i])
                continue;
            *dst[i] = static_cast<char *>(C.scratch_ptr) + off;
            off += (sz[i] + 255) & ~size_t(255);
        }
        if (off > kScratchBytes) {
            set_err("call needs " + std::to_string(off - kScratchPlan) +
                    " bytes of scratch; the no-allocation entry holds " +
                    std::to_string(kScratchBytes - kScratchPlan));
            return 0;
        }
    }
    if (!order_after_previous(C, st))
        return 0;
    if (!noalloc)
        HIP_TRY(get_bufs(C, cc, R, D, Iinter, B));
    DevPlan dp{};
    if (!upload_plan(C, P, cc, st, dp, false, noalloc ? C.scratch_ptr : nullptr,
                     noalloc ? kScratchPlan : 0))
        return 0;
    C.stats[19] += std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() -
                                                             hc.t0).count();
    if (!run_phases(C, P, cc, dp, B, fmt, D, Iinter, act, act_a, act_b, xg, dp.xrow, out, st,
                    P.ew.size(), nullptr, !noalloc))
        return 0;
    return finish_call(C, st, dp.slot);
}

bool args_ok(int nb, int D, int fmt, const float *xg, const int *xoff, const int *nr,
             const float *out) {
    // src/gpu/metal_ops.cpp:452-455
    if (nb < 1 || D < 1 || !out || !xg || (fmt != 0 && fmt != 4 && fmt != 7)) {
        set_err("invalid arguments (nb, D, out, xg or fmt)");
        return false;
    }
    if (!xoff || !nr) {
        set_err("xoff and nr are required");
        return false;
    }
    return true;
}

// ---- residency --------------------------------------------------------------------

void *res_alloc(Ctx &C, size_t bytes) {
    auto it = C.free_blocks.find(bytes);
    if (it != C.free_blocks.end()) {
        void *p = it->second;
        C.free_blocks.erase(it);
        return p;
    }
    void *p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess)
        return nullptr;
    return p;
}

void res_drop(Ctx &C, long long key) {
    auto it = C.res.find(key);
    if (it == C.res.end())
        return;
    Resident &r = it->second;
    // the block is recycled only after readers and the copy are done: the copy
    // stream waits for the last reader before writing into a recycled block
    if (r.used)
        (void)hipStreamWaitEvent(C.copy, r.last_use, 0);
    auto lu = C.layer_use.find(r.layer);
    if (lu != C.layer_use.end())
        (void)hipStreamWaitEvent(C.copy, lu->second, 0);
    auto lo = C.layer_open.find(r.layer);
    if (lo != C.layer_open.end() && lo->second > 0) {
        C.layer_parked[r.layer].emplace_back(r.bytes, r.dev);
        C.parked_bytes += r.bytes;  // still device memory of the tier: counted in the budget
    } else
        C.free_blocks.emplace(r.bytes, r.dev);
    C.used_bytes -= r.bytes;
    if (r.host)
        C.by_host.erase(r.host);
    C.lru.erase(r.lru);
    (void)hipEventDestroy(r.ready);
    (void)hipEventDestroy(r.last_use);
    C.res.erase(it);
    C.stats[8] += 1;
}

// device address for host pointer p (inside a resident blob), or nullptr
Resident *res_lookup(Ctx &C, const void *p) {
    const uint8_t *q = static_cast<const uint8_t *>(p);
    auto it = C.by_host.upper_bound(q);
    if (it == C.by_host.begin())
        return nullptr;
    --it;
    Resident &r = C.res[it->second];
    if (q >= r.host + r.bytes)
        return nullptr;
    return &r;
}

}  // namespace

// ====================================================================================

extern "C" {

int mvllm_hip_init(int device) {
    Ctx &C = ctx();
    std::lock_guard<std::mutex> lk(C.mu);
    set_err("");
    if (C.ready)
        return C.device == device ? 1 : 0;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= device || device < 0) {
        set_err("no HIP device " + std::to_string(device));
        return 0;
    }
    HIP_TRY(hipSetDevice(device));
    // the no-allocation entry's device array, and its pinned plan slots, sized up front
    HIP_TRY(hipGetSymbolAddress(&C.scratch_ptr, HIP_SYMBOL(scratch)));
    for (auto &s : C.slots)
        HIP_TRY(s.host.ensure(kScratchPlan));
    HIP_TRY(hipStreamCreateWithFlags(&C.own, hipStreamNonBlocking));
    HIP_TRY(hipStreamCreateWithFlags(&C.copy, hipStreamNonBlocking));
    // The plan-slot and ordering events order the host's reuse of a slot and other streams
    // after a call.  Neither needs the call's device writes visible to the host, so they
    // skip the system-scope release (an L2 write-back between two calls' kernels).
    constexpr unsigned kEvFlags = hipEventDisableTiming | hipEventDisableSystemFence;
    for (auto &e : C.grp_done)
        HIP_TRY(hipEventCreateWithFlags(&e, kEvFlags));
    HIP_TRY(hipEventCreateWithFlags(&C.prev_done, kEvFlags));
    HIP_TRY(hipEventCreateWithFlags(&C.miss_done, hipEventDisableTiming));
    HIP_TRY(hipEventCreateWithFlags(&C.tier_ready, kEvFlags));
    for (int i = 0; i < Ctx::kTabSlots; ++i) {
        HIP_TRY(C.tab_host[i].ensure(Ctx::kTabMax * sizeof(void *)));
        HIP_TRY(hipEventCreateWithFlags(&C.tab_done[i], kEvFlags));
        C.tab_used[i] = false;
    }
    C.tab_next = 0;
    C.device = device;
    C.ready = true;
    return 1;
}

void mvllm_hip_shutdown(void) {
    Ctx &C = ctx();
    std::lock_guard<std::mutex> lk(C.mu);
    if (!C.ready)
        return;
    (void)hipDeviceSynchronize();
    while (!C.res.empty())
        res_drop(C, C.res.begin()->first);
    for (auto &fb : C.free_blocks)
        (void)hipFree(fb.second);
    C.free_blocks.clear();
    for (auto &lp : C.layer_parked)
        for (auto &fb : lp.second)
            (void)hipFree(fb.second);
    C.layer_parked.clear();
    C.parked_bytes = 0;
    C.layer_open.clear();
    C.H.release();
    C.Y.release();
    C.Ph.release();
    C.HP.release();
    C.Xp.release();
    C.Lp.release();
    C.Rp.release();
    C.Xc.release();
    C.Oc.release();
    C.miss.release();
    C.hx.release();
    C.ho.release();
    for (auto &s : C.slots) {
        s.host.release();
        s.dev.release();
    }
    for (int g = 0; g < Ctx::kSlots / Ctx::kGroup; ++g) {
        (void)hipEventDestroy(C.grp_done[g]);
        C.grp_done[g] = nullptr;
        C.grp_used[g] = false;
    }
    C.open_last = -1;
    C.slot_next = 0;
    for (auto &t : C.timed)
        for (auto &e : t.ev)
            (void)hipEventDestroy(e);
    C.timed.clear();
    (void)hipEventDestroy(C.prev_done);
    C.prev_done = nullptr;
    (void)hipEventDestroy(C.miss_done);
    C.miss_done = nullptr;
    (void)hipEventDestroy(C.tier_ready);
    C.tier_ready = nullptr;
    for (auto &lu : C.layer_use)
        (void)hipEventDestroy(lu.second);
    C.layer_use.clear();
    for (int i = 0; i < Ctx::kTabSlots; ++i) {
        C.tab_host[i].release();
        (void)hipEventDestroy(C.tab_done[i]);
        C.tab_done[i] = nullptr;
    }
    for (void *p : g_retired)
        (void)hipFree(p);
    g_retired.clear();
    C.scratch_ptr = nullptr;
    (void)hipStreamDestroy(C.own);
    (void)hipStreamDestroy(C.copy);
    C.have_last = false;
    C.ready = false;
    C.device = -1;
}

int mvllm_hip_available(void) { return ctx().ready ? 1 : 0; }

const char *mvllm_hip_name(void) { return "hip"; }

const char *mvllm_hip_last_error(void) { return g_err.c_str(); }

int mvllm_hip_set_option(const char *key, long long value) {
    Ctx &C = ctx();
    std::lock_guard<std::mutex> lk(C.mu);
    if (!key)
        return 0;
    const std::string k(key);
    if (k == "mode") {
        if (value < 0 || value > 2)
            return 0;
        C.mode = static_cast<int>(value);
    } else if (k == "timing") {
        C.timing = value ? 1 : 0;
    } else if (k == "dec_ks") {
        if (value != 0 && value != 1 && value != 2 && value != 4 && value != 8)
            return 0;
        C.dec_ks = static_cast<int>(value);
    } else if (k == "gemm_xcd") {
        gemm_set_xcd(value != 0);
    } else if (k == "gemm_wide") {
        if (value < 0 || value > 1)
            return 0;
        gemm_set_wide(static_cast<int>(value));

    } else if (k == "dec_inline") {
        C.dec_inline = value ? 1 : 0;
    } else if (k == "combine_ordered") {
        C.combine_ordered = value ? 1 : 0;
    } else if (k == "fp4act") {
        C.fp4act = value ? 1 : 0;
    } else if (k == "gemm") {
        if (value < 0 || value > 2)
            return 0;
        C.gemm = static_cast<int>(value);
    } else if (k == "dequant_path") {
        C.dequant_path = value ? 1 : 0;
    } else {
        return 0;
    }
    return 1;
}

int mvllm_hip_moe_block_dev(int nb, int D, int Iinter, int fmt, int qgs, const void *const *g,
                            const void *const *u, const void *const *d, const float *const *gs,
                            const float *const *us, const float *const *ds, const float *xg,
                            const int *xoff, const int *nr, const int *rows, const float *rw,
                            float *out, int S, int act, float act_a, float act_b,
                            void *stream) {
    (void)qgs;  // the reference ignores it too: 64 for fmt 4, 32 for fmt 7
    Ctx &C = ctx();
    std::lock_guard<std::mutex> lk(C.mu);
    set_err("");
    if (!C.ready) {
        set_err("mvllm_hip_init not called");
        return 0;
    }
    if (!args_ok(nb, D, fmt, xg, xoff, nr, out))
        return 0;
    if (S <= 0) {
        set_err("the device entry needs S > 0 (row count of out)");
        return 0;
    }
    return dev_call(C, nb, D, Iinter, fmt, g, u, d, gs, us, ds, xg, xoff, nr, rows, rw, out, S,
                    act, act_a, act_b, static_cast<hipStream_t>(stream), false);
}

int mvllm_hip_moe_block_dev_noalloc(int nb, int D, int Iinter, int fmt, int qgs,
                                    const void *const *g, const void *const *u,
                                    const void *const *d, const float *const *gs,
                                    const float *const *us, const float *const *ds,
                                    const float *xg, const int *xoff, const int *nr,
                                    const int *rows, const float *rw, float *out, int S, int act,
                                    float act_a, float act_b, void *stream) {
    (void)qgs;
    Ctx &C = ctx();
    std::lock_guard<std::mutex> lk(C.mu);
    set_err("");
    if (!C.ready || !C.scratch_ptr) {
        set_err("mvllm_hip_init not called");
        return 0;
    }
    if (!args_ok(nb, D, fmt, xg, xoff, nr, out))
        return 0;
    if (S <= 0) {
        set_err("the device entry needs S > 0 (row count of out)");
        return 0;
    }
    return dev_call(C, nb, D, Iinter, fmt, g, u, d, gs, us, ds, xg, xoff, nr, rows, rw, out, S,
                    act, act_a, act_b, static_cast<hipStream_t>(stream), true);
}

int mvllm_hip_moe_block(int nb, int D, int Iinter, int fmt, int qgs, const void *const *g,
                        const void *const *u, const void *const *d, const float *const *gs,
                        const float *const *us, const float *const *ds, const float *xg,
                        const int *xoff, const int *nr, const int *rows, const float *rw,
                        float *out, int S, int act, float act_a, float act_b) {
    (void)qgs;
    Ctx &C = ctx();
    std::lock_guard<std::mutex> lk(C.mu);
    set_err("");
    if (!C.ready) {
        set_err("mvllm_hip_init not called");
        return 0;
    }
    if (!args_ok(nb, D, fmt, xg, xoff, nr, out))
        return 0;
    HostClock hc(&C.stats[15]);
    Plan &P = C.plan;
    build_plan(P, nb, D, Iinter, fmt, g, u, d, gs, us, ds, xoff, nr, rows, rw, S);
    C.stats[0] += 1;
    if (P.ew.empty())
        return 1;
    hipStream_t st = C.own;
    if (!order_after_previous(C, st))
        return 0;

    // 1) resolve expert pieces: resident blobs first, misses copied into the arena
    const size_t pb[4] = {piece_bytes(fmt, 0, D, Iinter), piece_bytes(fmt, 1, D, Iinter),
                          piece_bytes(fmt, 2, D, Iinter), piece_bytes(fmt, 3, D, Iinter)};
    std::vector<ExpertWork> hit, miss;
    std::vector<std::vector<int>> hit_rows;  // unused; order kept by row0
    std::vector<Resident *> touched;
    std::vector<std::pair<const void *, size_t>> miss_src;  // per miss expert: 6 pieces
    for (const ExpertWork &w0 : P.ew) {
        ExpertWork w = w0;
        bool all = true;
        Resident *rs[6] = {};
        for (int m = 0; m < 3 && all; ++m) {
            rs[2 * m] = res_lookup(C, w.w[m]);
            rs[2 * m + 1] = fmt ? res_lookup(C, w.s[m]) : rs[2 * m];
            const size_t bw = pb[m == 2 ? 2 : 0], bs = pb[m == 2 ? 3 : 1];
            all = rs[2 * m] &&
                  static_cast<const uint8_t *>(w.w[m]) + bw <= rs[2 * m]->host + rs[2 * m]->bytes &&
                  (!fmt || (rs[2 * m + 1] && static_cast<const uint8_t *>(w.s[m]) + bs <=
                                                 rs[2 * m + 1]->host + rs[2 * m + 1]->bytes));
        }
        if (all) {
            for (int m = 0; m < 3; ++m) {
                w.w[m] = static_cast<uint8_t *>(rs[2 * m]->dev) +
                         (static_cast<const uint8_t *>(w.w[m]) - rs[2 * m]->host);
                if (fmt)
                    w.s[m] = static_cast<uint8_t *>(rs[2 * m + 1]->dev) +
                             (static_cast<const uint8_t *>(w.s[m]) - rs[2 * m + 1]->host);
            }
            for (auto *r : rs)
                if (r) {
                    HIP_TRY(hipStreamWaitEvent(st, r->ready, 0));
                    touched.push_back(r);
                    C.lru.splice(C.lru.begin(), C.lru, r->lru);
                }
            hit.push_back(w);
            C.stats[6] += 1;
        } else {
            miss.push_back(w);
            C.stats[7] += 1;
        }
    }
    // 2) misses: copy their pieces on the copy stream into the arena
    size_t per_expert = 0;  // arena bytes per miss: six padded pieces, or one span
    for (int m = 0; m < 3; ++m)
        per_expert += ((pb[m == 2 ? 2 : 0] + 255) & ~size_t(255)) +
                      (fmt ? ((pb[m == 2 ? 3 : 1] + 255) & ~size_t(255)) : 0);
    per_expert += kSpanSlack + 512;  // a single-span copy may carry slot padding
    hipEvent_t miss_ev = nullptr;
    if (!miss.empty()) {
        HIP_TRY(C.miss.ensure(per_expert * miss.size()));
        uint8_t *arena = static_cast<uint8_t *>(C.miss.p);
        size_t off = 0;
        // the arena is reused per call: the copy stream waits for the previous call
        if (!wait_previous(C, C.copy))
            return 0;
        for (ExpertWork &w : miss) {
            // the six pieces of an ExpertStore blob are one contiguous host range: one copy
            // (whole-blob DMA runs closer to the PCIe rate than six small ones)
            const uint8_t *lo = nullptr, *hi = nullptr;
            for (int m = 0; m < 3; ++m) {
                const uint8_t *pw = static_cast<const uint8_t *>(w.w[m]);
                const size_t bw = pb[m == 2 ? 2 : 0], bs = pb[m == 2 ? 3 : 1];
                lo = (!lo || pw < lo) ? pw : lo;
                hi = (!hi || pw + bw > hi) ? pw + bw : hi;
                if (fmt) {
                    const uint8_t *ps = static_cast<const uint8_t *>(w.s[m]);
                    lo = ps < lo ? ps : lo;
                    hi = ps + bs > hi ? ps + bs : hi;
                }
            }
            size_t pieces = 0;
            for (int m = 0; m < 3; ++m)
                pieces += pb[m == 2 ? 2 : 0] + (fmt ? pb[m == 2 ? 3 : 1] : 0);
            // start at the 256-byte boundary below (blocks are page aligned): the device copy
            // then keeps every piece's alignment
            lo = reinterpret_cast<const uint8_t *>(reinterpret_cast<uintptr_t>(lo) & ~uintptr_t(255));
            if ((size_t)(hi - lo) <= pieces + kSpanSlack && in_one_host_block(lo, hi)) {
                const size_t span = (size_t)(hi - lo);
                HIP_TRY(hipMemcpyAsync(arena + off, lo, span, hipMemcpyHostToDevice, C.copy));
                for (int m = 0; m < 3; ++m) {
                    w.w[m] = arena + off + (static_cast<const uint8_t *>(w.w[m]) - lo);
                    if (fmt)
                        w.s[m] = arena + off + (static_cast<const uint8_t *>(w.s[m]) - lo);
                }
                off += (span + 255) & ~size_t(255);
                C.stats[2] += static_cast<double>(span);
                continue;
            }
            for (int m = 0; m < 3; ++m) {
                const size_t bw = pb[m == 2 ? 2 : 0], bs = pb[m == 2 ? 3 : 1];
                HIP_TRY(hipMemcpyAsync(arena + off, w.w[m], bw, hipMemcpyHostToDevice, C.copy));
                w.w[m] = arena + off;
                off += (bw + 255) & ~size_t(255);
                C.stats[2] += static_cast<double>(bw);
                if (fmt) {
                    HIP_TRY(hipMemcpyAsync(arena + off, w.s[m], bs, hipMemcpyHostToDevice, C.copy));
                    w.s[m] = arena + off;
                    off += (bs + 255) & ~size_t(255);
                    C.stats[2] += static_cast<double>(bs);
                }
            }
        }
        C.copy_epoch += 1;
        // one event for every call: a wait takes the record current when it is enqueued
        miss_ev = C.miss_done;
        HIP_TRY(hipEventRecord(miss_ev, C.copy));
    }
    // resident experts first, so their gate/up overlaps the miss copies
    P.ew.clear();
    P.ew.insert(P.ew.end(), hit.begin(), hit.end());
    P.ew.insert(P.ew.end(), miss.begin(), miss.end());

    // 3) activations: gather the compact rows into pinned memory, one H2D copy
    const size_t R = P.xrow.size();
    HIP_TRY(C.hx.ensure(R * D * 4));
    HIP_TRY(C.Xc.ensure(R * D * 4));
    for (size_t j = 0; j < R; ++j)
        std::memcpy(static_cast<float *>(C.hx.p) + j * D, xg + (size_t)P.xrow[j] * D,
                    (size_t)D * 4);
    HIP_TRY(hipMemcpyAsync(C.Xc.p, C.hx.p, R * D * 4, hipMemcpyHostToDevice, st));
    // 4) the destination rows of out, compacted (combine writes out_row = t)
    const size_t T = P.out_row.size();
    HIP_TRY(C.ho.ensure(T * D * 4));
    HIP_TRY(C.Oc.ensure(T * D * 4));
    for (size_t t = 0; t < T; ++t)
        std::memcpy(static_cast<float *>(C.ho.p) + t * D, out + (size_t)P.out_row[t] * D,
                    (size_t)D * 4);
    HIP_TRY(hipMemcpyAsync(C.Oc.p, C.ho.p, T * D * 4, hipMemcpyHostToDevice, st));
    C.stats[3] += static_cast<double>((R + T) * D * 4);
    std::vector<int> dest_rows = P.out_row;
    for (size_t t = 0; t < T; ++t)
        P.out_row[t] = static_cast<int>(t);
    CallCfg &cc = C.cfg;
    plan_call(C, cc, P, fmt, D, Iinter, hit.size(), C.Xc.p, true);
    Bufs B;
    HIP_TRY(get_bufs(C, cc, R, D, Iinter, B));
    DevPlan dp{};
    if (!upload_plan(C, P, cc, st, dp, true))
        return 0;
    const int ok = run_phases(C, P, cc, dp, B, fmt, D, Iinter, act, act_a, act_b,
                              static_cast<const float *>(C.Xc.p), nullptr,
                              static_cast<float *>(C.Oc.p), st, hit.size(), miss_ev);
    if (!ok)
        return 0;
    for (Resident *r : touched) {
        HIP_TRY(hipEventRecord(r->last_use, st));
        r->used = true;
    }
    HIP_TRY(hipMemcpyAsync(C.ho.p, C.Oc.p, T * D * 4, hipMemcpyDeviceToHost, st));
    C.stats[4] += static_cast<double>(T * D * 4);
    if (!finish_call(C, st, dp.slot))
        return 0;
    HIP_TRY(hipStreamSynchronize(st));
    for (size_t t = 0; t < T; ++t)
        std::memcpy(out + (size_t)dest_rows[t] * D, static_cast<float *>(C.ho.p) + t * D,
                    (size_t)D * 4);
    return 1;
}

void *mvllm_hip_host_alloc(size_t bytes) {
    void *p = nullptr;
    if (hipHostMalloc(&p, bytes, hipHostMallocDefault) != hipSuccess) {
        set_err("hipHostMalloc failed");
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_host_mu);
    g_host_blocks[reinterpret_cast<uintptr_t>(p)] = bytes;
    return p;
}

int mvllm_hip_host_free(void *p) {
    if (!p)
        return 0;
    {
        std::lock_guard<std::mutex> lk(g_host_mu);
        if (g_host_blocks.erase(reinterpret_cast<uintptr_t>(p)) == 0)
            return 0;  // not ours: the caller's own allocator frees it
    }
    (void)hipHostFree(p);
    return 1;
}

int mvllm_hip_set_expert_budget(size_t bytes) {
    Ctx &C = ctx();
    std::lock_guard<std::mutex> lk(C.mu);
    C.budget = bytes;
    while (C.used_bytes + C.parked_bytes > C.budget && !C.lru.empty())
        res_drop(C, C.lru.back());
    return 1;
}

}  // extern "C"

namespace {

// One promotion (mvllm_hip_promote / mvllm_hip_prefetch); *staged = 1 when a copy was
// enqueued, 0 when the blob was resident already.  Caller holds C.mu.
int promote_locked(Ctx &C, const void *host_blob, size_t bytes, int layer, int eid,
                   int *staged) {
    *staged = 0;
    if (!C.ready || !host_blob || bytes == 0) {
        set_err("promote: not initialised or empty blob");
        return 0;
    }
    const long long key = res_key(layer, eid);
    auto it = C.res.find(key);
    if (it != C.res.end()) {
        if (it->second.host == host_blob && it->second.bytes == bytes) {
            C.lru.splice(C.lru.begin(), C.lru, it->second.lru);
            return 1;
        }
        res_drop(C, key);  // the store moved this expert to another slot
    }
    // a different expert previously promoted from an overlapping host range is stale
    for (auto h = C.by_host.begin(); h != C.by_host.end();) {
        const Resident &r = C.res[h->second];
        const uint8_t *a = static_cast<const uint8_t *>(host_blob);
        if (r.host < a + bytes && a < r.host + r.bytes) {
            const long long k2 = h->second;
            ++h;
            res_drop(C, k2);
        } else {
            ++h;
        }
    }
    // parked blocks (blobs dropped while their layer's tables are open) count against the
    // budget until mvllm_hip_tier_table_done recycles them
    while (C.used_bytes + C.parked_bytes + bytes > C.budget && !C.lru.empty())
        res_drop(C, C.lru.back());
    if (C.used_bytes + C.parked_bytes + bytes > C.budget) {
        set_err(C.parked_bytes ? "promote: expert budget held by blobs of open tier tables"
                               : "promote: blob larger than the expert budget");
        return 0;
    }
    void *dev = res_alloc(C, bytes);
    if (!dev) {
        set_err("promote: hipMalloc failed");
        return 0;
    }
    Resident r;
    r.layer = layer;
    r.eid = eid;
    r.host = static_cast<const uint8_t *>(host_blob);
    r.bytes = bytes;
    r.dev = dev;
    HIP_TRY(hipEventCreateWithFlags(&r.ready, hipEventDisableTiming));
    HIP_TRY(hipEventCreateWithFlags(&r.last_use, hipEventDisableTiming));
    HIP_TRY(hipMemcpyAsync(dev, host_blob, bytes, hipMemcpyHostToDevice, C.copy));
    C.copy_epoch += 1;
    HIP_TRY(hipEventRecord(r.ready, C.copy));
    C.lru.push_front(key);
    r.lru = C.lru.begin();
    C.res[key] = r;
    C.by_host[r.host] = key;
    C.used_bytes += bytes;
    C.stats[5] += 1;
    C.stats[2] += static_cast<double>(bytes);
    *staged = 1;
    return 1;
}

// mvllm_hip_moe_block_routed_dev at decode shapes (S <= 16 out rows): the decode kernels,
// the top-k combine folded into the down kernel as in the host-planned decode call, the
// gate/up kernel planning its own item from the segments and writing the down
// descriptors (k_mfma_dec_seg); or, with option combine_ordered, on descriptors the
// device planner writes (k_dplan_dec) with the ordered combine on device-built lists.
// Two launches (six ordered) where the grouped-GEMM path takes fifteen.  Returns -1 when the shapes do not take this path (the
// caller runs the grouped GEMM), else the entry's result.  Arguments validated by the
// caller, which holds C.mu.
int routed_dec(Ctx &C, int D, int I, int fmt, const void *const *table, int n_table,
               const int *counts, const int *eids, const int *xoff, const int *nr,
               int cap_experts, const int *rows, const float *rw, int cap_rows, const float *x,
               float *out, int S, int act, float act_a, float act_b, int *status,
               hipStream_t st, const long long off6[6]) {
    const int terms = C.mode == 1 ? 3 : C.mode == 2 ? 1 : 2;
    if (C.gemm == 1 || S > 16 || D > kDecMaxK || I > kDecMaxK || (fmt == 7 && C.fp4act))
        return -1;
    for (int k = 0; k < 6; ++k)  // weights 16-byte aligned, scales 16 (int4) or 8 (MXFP4)
        if (off6[k] % ((k & 1) && fmt == 7 ? 8 : 16))
            return -1;
    // rows per item: S (a token picks an expert at most once, so no segment of routing
    // output holds more rows), or fewer where the activations of S rows do not fit the
    // kernels' staging; longer segments split into items of rmax rows.  Items at most: M
    // segments of one item, plus one more per further rmax rows of the call
    const int rmax = std::min(pick_rmax(fmt, D, I, terms, true, S),
                              pick_rmax(fmt, I, D, terms, false, S));
    if (rmax < 1)
        return -1;
    const int M = std::min(cap_experts, cap_rows);
    const int cap_items = M + (cap_rows - M) / rmax;
    if (cap_items > 8192)  // caps far beyond a decode call's rows: the grouped path
        return -1;
    PhaseCfg gu, dn;
    if (!pick_kt(C, fmt, D, I, rmax, terms, true, (size_t)cap_items, gu) ||
        !pick_kt(C, fmt, I, D, rmax, terms, false, (size_t)cap_items, dn))
        return -1;
    const bool fold = !C.combine_ordered;
    const bool pk = terms == 2 && rmax <= 8;  // the packed kernels (both terms in one MFMA)
    auto al = [](size_t n) { return (n + 255) & ~size_t(255); };
    const size_t b_desc = al((size_t)cap_items * sizeof(DecDesc));
    const size_t b_misc = 256, b_ok = al((size_t)cap_rows), b_cnt = al(((size_t)S + 1) * 4);
    const size_t b_cur = al((size_t)S * 4), b_er = al((size_t)cap_rows * 4);
    if (!order_after_previous(C, st))
        return 0;
    HIP_TRY(C.Rp.ensure(2 * b_desc + b_misc + b_ok + b_cnt + b_cur + 2 * b_er));
    HIP_TRY(C.Ph.ensure((size_t)terms * cap_rows * I * 2));
    if (fmt == 4)
        HIP_TRY(C.HP.ensure((size_t)(I / 64) * 4 * cap_rows * 4));
    if (!fold)
        HIP_TRY(C.Y.ensure((size_t)cap_rows * D * 4));
    char *p = static_cast<char *>(C.Rp.p);
    DPlanDecArgs a{};
    a.table = table;
    a.n_table = n_table;
    for (int k = 0; k < 6; ++k)
        a.off[k] = off6[k];
    a.counts = counts;
    a.eids = eids;
    a.xoff = xoff;
    a.nr = nr;
    a.rows = rows;
    a.rw = rw;
    a.cap_e = cap_experts;
    a.cap_rows = cap_rows;
    a.S = S;
    a.rmax = rmax;
    a.cap_items = cap_items;
    a.gu = reinterpret_cast<DecDesc *>(p);
    a.dn = reinterpret_cast<DecDesc *>(p + b_desc);
    char *misc = p + 2 * b_desc;
    a.n_items = reinterpret_cast<int *>(misc);
    a.err = status ? status : reinterpret_cast<int *>(misc + 64);
    a.row_ok = reinterpret_cast<unsigned char *>(misc + b_misc);
    float *hp = fmt == 4 ? static_cast<float *>(C.HP.p) : nullptr;
    // with the combine folded into the down kernel, the gate/up kernel plans its own items
    // (the compact descriptor: 16-bit compact rows, 32-bit piece offsets); the ordered
    // combine needs the planner's row flags
    bool self_plan = fold && cap_rows <= 65535;
    for (int k = 1; k < 4; ++k)
        self_plan = self_plan && std::llabs(off6[k] - off6[0]) < (1ll << 31);
    if (self_plan) {
        DecSegArgs sg{};
        sg.table = table;
        sg.n_table = n_table;
        for (int k = 0; k < 6; ++k)
            sg.off[k] = off6[k];
        sg.counts = counts;
        sg.eids = eids;
        sg.xoff = xoff;
        sg.nr = nr;
        sg.rows = rows;
        sg.rw = rw;
        sg.cap_e = cap_experts;
        sg.cap_rows = cap_rows;
        sg.S = S;
        sg.rmax = rmax;
        sg.cap_items = cap_items;
        sg.dn = a.dn;
        sg.n_items = a.n_items;
        sg.err = a.err;
        HIP_TRY(launch_mfma_dec(fmt, true, terms, gu.ks, gu.nt, nullptr, cap_items, x, nullptr,
                                nullptr, C.Ph.p, hp, nullptr, D, I, cap_rows, rmax, act, act_a,
                                act_b, false, pk, nullptr, nullptr, 0, st, nullptr, nullptr,
                                &sg));
    } else {
        HIP_TRY(launch_dplan_dec(a, st));
        HIP_TRY(launch_mfma_dec(fmt, true, terms, gu.ks, gu.nt, a.gu, cap_items, x, nullptr,
                                nullptr, C.Ph.p, hp, nullptr, D, I, cap_rows, rmax, act, act_a,
                                act_b, false, pk, nullptr, nullptr, 0, st, nullptr, a.n_items));
    }
    HIP_TRY(launch_mfma_dec(fmt, false, terms, dn.ks, dn.nt, a.dn, cap_items, nullptr, C.Ph.p, hp,
                            nullptr, nullptr, fold ? out : static_cast<float *>(C.Y.p), I, D,
                            cap_rows, rmax, 0, 0.f, 0.f, fold, pk, nullptr, nullptr, 0, st,
                            nullptr, a.n_items));
    if (!fold) {
        CsrArgs cs{};
        cs.counts = counts;
        cs.cap_rows = cap_rows;
        cs.S = S;
        cs.rows = rows;
        cs.rw = rw;
        cs.row_ok = a.row_ok;
        cs.cnt = reinterpret_cast<int *>(misc + b_misc + b_ok);
        cs.cursor = reinterpret_cast<int *>(misc + b_misc + b_ok + b_cnt);
        cs.ent_row = reinterpret_cast<int *>(misc + b_misc + b_ok + b_cnt + b_cur);
        cs.ent_w = reinterpret_cast<float *>(misc + b_misc + b_ok + b_cnt + b_cur + b_er);
        HIP_TRY(launch_dcsr(cs, st));
        CombineArgs cb{};
        cb.Y = static_cast<const float *>(C.Y.p);
        cb.tok_ptr = cs.cnt;
        cb.ent_row = cs.ent_row;
        cb.ent_w = cs.ent_w;
        cb.out_row = nullptr;
        cb.out = out;
        cb.n_tok = S;
        cb.D = D;
        HIP_TRY(launch_combine(cb, st));
    }
    C.stats[0] += 1;
    C.stats[13] += 1;
    C.stats[14] += 1;
    C.last_stream = st;
    C.have_last = true;
    return 1;
}

}  // namespace

extern "C" {

int mvllm_hip_promote(const void *host_blob, size_t bytes, int layer, int eid) {
    Ctx &C = ctx();
    std::lock_guard<std::mutex> lk(C.mu);
    set_err("");
    int staged;
    return promote_locked(C, host_blob, bytes, layer, eid, &staged);
}

int mvllm_hip_prefetch(int n, const int *layers, const int *eids, const void *const *host_blobs,
                       const size_t *bytes) {
    Ctx &C = ctx();
    std::lock_guard<std::mutex> lk(C.mu);
    set_err("");
    if (n < 0 || (n > 0 && (!layers || !eids || !host_blobs || !bytes))) {
        set_err("prefetch: bad arguments");
        return -1;
    }
    int count = 0;
    for (int i = 0; i < n; ++i) {
        int staged;
        if (!promote_locked(C, host_blobs[i], bytes[i], layers[i], eids[i], &staged))
            return -1;
        count += staged;
    }
    return count;
}

int mvllm_hip_repin(int n, const int *layer_eid) {
    Ctx &C = ctx();
    std::lock_guard<std::mutex> lk(C.mu);
    set_err("");
    if (n < 0 || (n > 0 && !layer_eid)) {
        set_err("repin: bad arguments");
        return -1;
    }
    int count = 0;
    for (int i = 0; i < n; ++i) {
        auto it = C.res.find(res_key(layer_eid[2 * i], layer_eid[2 * i + 1]));
        if (it == C.res.end() || !it->second.host)
            continue;
        // the host slot now belongs to another expert: the HBM copy stays, addressable by
        // (layer, eid), but no host pointer maps to it any more
        C.by_host.erase(it->second.host);
        it->second.host = nullptr;
        ++count;
    }
    return count;
}

int mvllm_hip_host_reuse(const void *host_lo, size_t bytes) {
    Ctx &C = ctx();
    std::lock_guard<std::mutex> lk(C.mu);
    set_err("");
    if (!C.ready || !host_lo || bytes == 0) {
        set_err("host_reuse: bad arguments");
        return -1;
    }
    const uint8_t *lo = static_cast<const uint8_t *>(host_lo), *hi = lo + bytes;
    int count = 0;
    for (auto h = C.by_host.begin(); h != C.by_host.end();) {
        Resident &r = C.res[h->second];
        if (r.host < hi && lo < r.host + r.bytes) {
            // the copy from the old contents must be complete before the slot is rewritten
            if (hipEventSynchronize(r.ready) != hipSuccess) {
                set_err("host_reuse: hipEventSynchronize failed");
                return -1;
            }
            r.host = nullptr;
            h = C.by_host.erase(h);
            ++count;
        } else {
            ++h;
        }
    }
    return count;
}

int mvllm_hip_tier_table(int layer, int n_experts, void **table_dev, int *n_resident,
                         void *stream) {
    Ctx &C = ctx();
    std::lock_guard<std::mutex> lk(C.mu);
    set_err("");
    if (!C.ready || !table_dev || n_experts < 1 || n_experts > Ctx::kTabMax) {
        set_err("tier_table: bad arguments (1 <= n_experts <= 8192)");
        return 0;
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    // tables of up to kArgWords entries travel in a kernel's arguments; larger ones through
    // a ring of pinned slots that a kernel reads, each slot guarded by an event
    const bool in_args = n_experts <= kArgWords;
    ArgWords aw;
    const int si = C.tab_next;
    if (!in_args) {
        C.tab_next = (si + 1) % Ctx::kTabSlots;
        if (C.tab_used[si])
            HIP_TRY(hipEventSynchronize(C.tab_done[si]));
    }
    void **h = in_args ? reinterpret_cast<void **>(aw.v) : static_cast<void **>(C.tab_host[si].p);
    int count = 0;
    for (int e = 0; e < n_experts; ++e) {
        auto it = C.res.find(res_key(layer, e));
        h[e] = it == C.res.end() ? nullptr : it->second.dev;
        if (h[e]) {
            C.lru.splice(C.lru.begin(), C.lru, it->second.lru);
            ++count;
        }
    }
    // the compute that reads the table runs after every promotion enqueued so far: a wait
    // unless those copies have all finished (a wait is a queue packet that idles the GPU)
    if (C.tier_epoch != C.copy_epoch) {
        HIP_TRY(hipEventRecord(C.tier_ready, C.copy));
        C.tier_epoch = C.copy_epoch;
    }
    const hipError_t q = hipEventQuery(C.tier_ready);
    if (q == hipErrorNotReady)
        HIP_TRY(hipStreamWaitEvent(st, C.tier_ready, 0));
    else
        HIP_TRY(q);
    // the table by a kernel (an asynchronous copy of a few KB idled the stream ~15 us per
    // table; a kernel reading a pinned slot takes ~3.6 us, plus the slot's event)
    if (in_args) {
        aw.n = n_experts;
        HIP_TRY(launch_fill_words(aw, table_dev, st));
    } else {
        HIP_TRY(launch_copy_words(h, table_dev, n_experts, st));
        HIP_TRY(hipEventRecord(C.tab_done[si], st));
        C.tab_used[si] = true;
    }
    C.layer_open[layer] += 1;
    if (n_resident)
        *n_resident = count;
    return 1;
}

int mvllm_hip_tier_table_done(int layer, void *stream) {
    Ctx &C = ctx();
    std::lock_guard<std::mutex> lk(C.mu);
    set_err("");
    if (!C.ready) {
        set_err("tier_table_done: not initialised");
        return 0;
    }
    hipEvent_t &ev = C.layer_use[layer];
    if (!ev)
        HIP_TRY(hipEventCreateWithFlags(&ev, hipEventDisableTiming | hipEventDisableSystemFence));
    HIP_TRY(hipEventRecord(ev, static_cast<hipStream_t>(stream)));
    int &open = C.layer_open[layer];
    open = open > 0 ? open - 1 : 0;
    auto lp = C.layer_parked.find(layer);
    if (open == 0 && lp != C.layer_parked.end() && !lp->second.empty()) {
        // blobs of the layer dropped while its tables were open: copies into their
        // blocks wait for the readers recorded just now
        HIP_TRY(hipStreamWaitEvent(C.copy, ev, 0));
        for (auto &fb : lp->second) {
            C.free_blocks.emplace(fb.first, fb.second);
            C.parked_bytes -= fb.first;
        }
        lp->second.clear();
    }
    return 1;
}

int mvllm_hip_evict(int layer, int eid) {
    Ctx &C = ctx();
    std::lock_guard<std::mutex> lk(C.mu);
    const long long key = res_key(layer, eid);
    if (C.res.find(key) == C.res.end())
        return 0;
    res_drop(C, key);
    return 1;
}

void *mvllm_hip_resident_ptr(int layer, int eid) {
    Ctx &C = ctx();
    std::lock_guard<std::mutex> lk(C.mu);
    auto it = C.res.find(res_key(layer, eid));
    if (it == C.res.end())
        return nullptr;
    (void)hipEventSynchronize(it->second.ready);
    return it->second.dev;
}

int mvllm_hip_stats(double *vals, int n) {
    Ctx &C = ctx();
    std::lock_guard<std::mutex> lk(C.mu);
    for (auto &t : C.timed) {
        float ms[5] = {0, 0, 0, 0, 0};
        (void)hipEventSynchronize(t.ev[5]);
        for (int i = 0; i < 5; ++i)
            (void)hipEventElapsedTime(&ms[i], t.ev[i], t.ev[i + 1]);
        C.stats[12] += ms[0] + ms[2];
        C.stats[9] += ms[1];
        C.stats[10] += ms[3];
        C.stats[11] += ms[4];
        for (auto &e : t.ev)
            (void)hipEventDestroy(e);
    }
    C.timed.clear();
    C.stats[17] = static_cast<double>(C.used_bytes + C.parked_bytes);
    C.stats[18] = static_cast<double>(C.parked_bytes);
    const int m = std::min(n, 20);
    for (int i = 0; i < m; ++i)
        vals[i] = C.stats[i];
    return m;
}

void mvllm_hip_stats_reset(void) {
    Ctx &C = ctx();
    std::lock_guard<std::mutex> lk(C.mu);
    for (auto &t : C.timed) {
        (void)hipEventSynchronize(t.ev[5]);
        for (auto &e : t.ev)
            (void)hipEventDestroy(e);
    }
    C.timed.clear();
    for (double &v : C.stats)
        v = 0;
}

int mvllm_hip_dequant(int fmt, const void *packed_dev, const void *scales_dev, int O, int K,
                      float *w_dev) {
    Ctx &C = ctx();
    std::lock_guard<std::mutex> lk(C.mu);
    set_err("");
    if (!C.ready || (fmt != 4 && fmt != 7) || O < 1 || K < 1 || !packed_dev || !scales_dev ||
        !w_dev) {
        set_err("dequant: bad arguments");
        return 0;
    }
    if (C.dequant_path)
        HIP_TRY(launch_dequant_bf16path(fmt, packed_dev, scales_dev, O, K, w_dev, C.own));
    else
        HIP_TRY(launch_dequant(fmt, packed_dev, scales_dev, O, K, w_dev, C.own));
    HIP_TRY(hipStreamSynchronize(C.own));
    return 1;
}

int mvllm_hip_moe_topk_dev(const float *choice, const float *mix, int n_tok, int n_exp, int k,
                           int *idx, float *wt, void *stream) {
    Ctx &C = ctx();
    set_err("");
    if (!C.ready || !choice || !idx || !wt || n_tok < 1 || n_exp < 1 ||
        n_exp > kRouteMaxExperts || k < 1 || k > 64 || k > n_exp) {
        set_err("moe_topk_dev: bad arguments");
        return 0;
    }
    HIP_TRY(launch_moe_topk(choice, mix, n_tok, n_exp, k, idx, wt,
                            static_cast<hipStream_t>(stream)));
    return 1;
}

int mvllm_hip_moe_segments_dev(const int *idx, const float *wt, int n_tok, int topk, int n_exp,
                               int *work, int *eids, int *xoff, int *nr, int *rows, float *rw,
                               int cap_experts, int cap_rows, int *counts, void *stream) {
    Ctx &C = ctx();
    set_err("");
    if (!C.ready || !idx || !wt || !work || !eids || !xoff || !nr || !rows || !rw || !counts ||
        n_tok < 1 || topk < 1 || n_exp < 1 || cap_experts < 1 || cap_rows < 1 ||
        (long long)n_tok * topk > (1ll << 30)) {
        set_err("moe_segments_dev: bad arguments");
        return 0;
    }
    HIP_TRY(launch_moe_segments(idx, wt, n_tok, topk, n_exp, work, eids, xoff, nr, rows, rw,
                                cap_experts, cap_rows, counts, static_cast<hipStream_t>(stream)));
    return 1;
}

int mvllm_hip_moe_route_dev(const float *choice, const float *mix, int n_tok, int n_exp, int k,
                            int *idx, float *wt, int *work, int *eids, int *xoff, int *nr,
                            int *rows, float *rw, int cap_experts, int cap_rows, int *counts,
                            void *stream) {
    Ctx &C = ctx();
    set_err("");
    if (!C.ready || !choice || !idx || !wt || !work || !eids || !xoff || !nr || !rows || !rw ||
        !counts || n_tok < 1 || n_exp < 1 || n_exp > kRouteMaxExperts || k < 1 || k > 64 ||
        k > n_exp || cap_experts < 1 || cap_rows < 1 || (long long)n_tok * k > (1ll << 30)) {
        set_err("moe_route_dev: bad arguments");
        return 0;
    }
    HIP_TRY(launch_moe_route(choice, mix, n_tok, n_exp, k, idx, wt, work, eids, xoff, nr, rows, rw,
                             cap_experts, cap_rows, counts, static_cast<hipStream_t>(stream)));
    return 1;
}

int mvllm_hip_moe_block_routed_dev(int D, int Iinter, int fmt, const void *const *table,
                                   int n_table, const int *counts, const int *eids,
                                   const int *xoff, const int *nr, int cap_experts,
                                   const int *rows, const float *rw, int cap_rows,
                                   const float *x, float *out, int S, int act, float act_a,
                                   float act_b, int *status, void *stream) {
    Ctx &C = ctx();
    std::lock_guard<std::mutex> lk(C.mu);
    HostClock hc(&C.stats[15]);
    set_err("");
    if (!C.ready || !table || n_table < 1 || !counts || !eids || !xoff || !nr || !rows || !rw ||
        !x || !out || cap_experts < 1 || cap_rows < 1 || S < 1 || S > 65535 ||
        (fmt != 4 && fmt != 7) || D < 256 || D % 256 || Iinter < 256 || Iinter % 256 ||
        !aligned(x, 16) || (long long)cap_rows * D > (1ll << 31)) {
        set_err("moe_block_routed_dev: bad arguments (fmt 4/7, D and Iinter multiples of 256, "
                "1 <= S <= 65535, caps >= 1, x 16-byte aligned)");
        return 0;
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    long long off6[6];
    (void)mvllm_expert_geom(fmt, D, Iinter, off6);
    const int rd = routed_dec(C, D, Iinter, fmt, table, n_table, counts, eids, xoff, nr,
                              cap_experts, rows, rw, cap_rows, x, out, S, act, act_a, act_b,
                              status, st, off6);
    if (rd >= 0)
        return rd;
    // blobs are 256-byte aligned (k_dplan skips others): the pieces are 16-byte aligned
    // when their offsets are
    bool w16 = true;
    for (int k = 0; k < 6; k += 2)
        w16 = w16 && off6[k] % 16 == 0;
    // native MXFP4 activations (option fp4act), as the host-planned call runs them: the
    // scaled-FP4 GEMM's classes of up to 256 rows (its 16-byte weight rows), the 16- and
    // 32-row classes on bf16 copies of the quantized activations
    const bool fp4 = fmt == 7 && C.fp4act && w16;
    // bf16 terms per activation: two (2^-17 relative, the decode accuracy) for calls of at
    // most 256 rows, one (the prefill arithmetic) above; mode 1 always two, mode 2 one
    const int terms = fp4 ? 1 : C.mode == 1 ? 2 : C.mode == 2 ? 1 : (cap_rows <= 256 ? 2 : 1);
    const int max_mt = fp4 ? kFp4MaxMt : gemm_max_mt(fmt, terms);
    const int top = max_mt == 16 ? 4 : max_mt == 8 ? 3 : 2, bm = 16 * max_mt;
    // remainders of 33-64 rows as two 32-row items, as the host planner does (plan_gemm)
    const bool split64 = !fp4 && terms == 1 && max_mt >= 4;
    // items per class at most: one remainder per expert of >= lo rows; the top class's
    // items (full blocks and remainders above bm / 2) hold >= lo[top] rows each; with
    // split64 the 32-row class holds up to two items per expert, >= 16 rows per item
    static const int lo[kGemmClasses] = {1, 17, 33, 65, 129};
    int cap[kGemmClasses] = {}, base[kGemmClasses] = {}, n_it = 0;
    for (int c = 0; c <= top; ++c) {
        if (cap_rows >= lo[c])
            cap[c] = c == top ? cap_rows / lo[c] : std::min(cap_experts, cap_rows / lo[c]);
        if (split64 && c == 1)
            cap[c] = std::min(2 * cap_experts, cap_rows / 16);
        if (split64 && c == 2)
            cap[c] = 0;
        base[c] = n_it;
        n_it += cap[c];
    }
    auto al = [](size_t n) { return (n + 255) & ~size_t(255); };
    const size_t b_ew = al((size_t)cap_experts * sizeof(ExpertWork)), b_it = al((size_t)n_it * 16);
    const size_t b_misc = 256, b_ok = al((size_t)cap_rows), b_cnt = al(((size_t)S + 1) * 4);
    const size_t b_cur = al((size_t)S * 4), b_er = al((size_t)cap_rows * 4);
    const size_t total = b_ew + b_it + b_misc + b_ok + b_cnt + b_cur + 2 * b_er;
    if (!order_after_previous(C, st))
        return 0;
    HIP_TRY(C.Rp.ensure(total));
    const size_t R = (size_t)cap_rows;
    const bool bf = fp4 && (cap[0] || cap[1]);  // bf16 copies for the 16- and 32-row classes
    if (fp4) {
        HIP_TRY(C.Xp.ensure(R * (D / 2 + D / 32)));           // x codes + scales
        HIP_TRY(C.Ph.ensure(R * (Iinter / 2 + Iinter / 32)));  // H codes + scales
        HIP_TRY(C.H.ensure(R * Iinter * 4));
        if (bf)
            HIP_TRY(C.HP.ensure(R * (D + Iinter) * 2));
    } else {
        HIP_TRY(C.Xp.ensure((size_t)terms * R * D * 2));
        HIP_TRY(C.Ph.ensure((size_t)terms * R * Iinter * 2));
    }
    HIP_TRY(C.Y.ensure(R * D * 4));
    char *p = static_cast<char *>(C.Rp.p);
    DPlanArgs a{};
    a.table = table;
    a.n_table = n_table;
    for (int k = 0; k < 6; ++k)
        a.off[k] = off6[k];
    a.counts = counts;
    a.eids = eids;
    a.xoff = xoff;
    a.nr = nr;
    a.cap_e = cap_experts;
    a.cap_rows = cap_rows;
    a.bm = bm;
    a.top = top;
    a.split64 = split64 ? 1 : 0;
    a.ew = reinterpret_cast<ExpertWork *>(p);
    a.items = reinterpret_cast<int4 *>(p + b_ew);
    for (int c = 0; c < kGemmClasses; ++c) {
        a.item_base[c] = base[c];
        a.item_cap[c] = cap[c];
    }
    char *misc = p + b_ew + b_it;
    a.n_items = reinterpret_cast<int *>(misc);
    a.err = status ? status : reinterpret_cast<int *>(misc + 64);
    a.row_ok = reinterpret_cast<unsigned char *>(misc + b_misc);
    CsrArgs cs{};
    cs.counts = counts;
    cs.cap_rows = cap_rows;
    cs.S = S;
    cs.rows = rows;
    cs.rw = rw;
    cs.row_ok = a.row_ok;
    cs.cnt = reinterpret_cast<int *>(misc + b_misc + b_ok);
    cs.cursor = reinterpret_cast<int *>(misc + b_misc + b_ok + b_cnt);
    cs.ent_row = reinterpret_cast<int *>(misc + b_misc + b_ok + b_cnt + b_cur);
    cs.ent_w = reinterpret_cast<float *>(misc + b_misc + b_ok + b_cnt + b_cur + b_er);
    HIP_TRY(launch_dplan(a, st));
    float *Y = static_cast<float *>(C.Y.p);
    if (fp4) {
        // x rows quantized (gathered through rows; rows past the device count untouched,
        // out-of-range tokens as zero rows), gate/up into H f32, H quantized, down into Y
        uint8_t *xq = static_cast<uint8_t *>(C.Xp.p), *xsc = xq + R * (D / 2);
        uint8_t *hq = static_cast<uint8_t *>(C.Ph.p), *hsc = hq + R * (Iinter / 2);
        float *Hf = static_cast<float *>(C.H.p);
        __bf16 *xb = bf ? static_cast<__bf16 *>(C.HP.p) : nullptr;
        __bf16 *hb = bf ? xb + R * (size_t)D : nullptr;
        HIP_TRY(launch_quantize_mxfp4(x, cap_rows, D, xq, xsc, st, rows, xb, nullptr,
                                      counts + 1, S));
        for (int c = 0; c <= top; ++c) {
            if (!cap[c])
                continue;
            if ((1 << c) <= kFp4BfMaxMt)
                HIP_TRY(launch_gemm(fmt, true, 1, 1 << c, a.ew, a.items + base[c], cap[c], xb,
                                    nullptr, Hf, D, Iinter, cap_rows, act, act_a, act_b, st,
                                    a.n_items + c));
            else
                HIP_TRY(launch_gemm_fp4(true, 1 << c, a.ew, a.items + base[c], cap[c], xq, xsc,
                                        Hf, nullptr, D, Iinter, cap_rows, act, act_a, act_b, st,
                                        a.n_items + c));
        }
        HIP_TRY(launch_quantize_mxfp4(Hf, cap_rows, Iinter, hq, hsc, st, nullptr, hb, nullptr,
                                      counts + 1));
        for (int c = 0; c <= top; ++c) {
            if (!cap[c])
                continue;
            if ((1 << c) <= kFp4BfMaxMt)
                HIP_TRY(launch_gemm(fmt, false, 1, 1 << c, a.ew, a.items + base[c], cap[c], hb,
                                    nullptr, Y, Iinter, D, cap_rows, 0, 0.f, 0.f, st,
                                    a.n_items + c));
            else
                HIP_TRY(launch_gemm_fp4(false, 1 << c, a.ew, a.items + base[c], cap[c], hq, hsc,
                                        nullptr, Y, Iinter, D, cap_rows, 0, 0.f, 0.f, st,
                                        a.n_items + c));
        }
    } else {
        HIP_TRY(launch_prep_planes(fmt, terms, x, rows, cap_rows, D, cap_rows, C.Xp.p, st,
                                   counts + 1, S));
        for (int c = 0; c <= top; ++c)
            if (cap[c])
                HIP_TRY(launch_gemm_cls(w16, fmt, true, terms, 1 << c, a.ew, a.items + base[c],
                                        cap[c], C.Xp.p, C.Ph.p, nullptr, D, Iinter, cap_rows, act,
                                        act_a, act_b, st, a.n_items + c));
        for (int c = 0; c <= top; ++c)
            if (cap[c])
                HIP_TRY(launch_gemm_cls(w16, fmt, false, terms, 1 << c, a.ew, a.items + base[c],
                                        cap[c], C.Ph.p, nullptr, Y, Iinter, D, cap_rows, 0, 0.f,
                                        0.f, st, a.n_items + c));
    }
    HIP_TRY(launch_dcsr(cs, st));
    CombineArgs cb{};
    cb.Y = Y;
    cb.tok_ptr = cs.cnt;
    cb.ent_row = cs.ent_row;
    cb.ent_w = cs.ent_w;
    cb.out_row = nullptr;
    cb.out = out;
    cb.n_tok = S;
    cb.D = D;
    HIP_TRY(launch_combine(cb, st));
    C.stats[0] += 1;
    C.last_stream = st;
    C.have_last = true;
    return 1;
}

int mvllm_hip_router_dev(const float *x, const float *w, const float *bias, int n_tok, int D,
                         int n_exp, int k, float rscale, float *scores, float *choice,
                         int *idx, float *wt, void *stream) {
    Ctx &C = ctx();
    std::lock_guard<std::mutex> lk(C.mu);
    set_err("");
    if (!C.ready || !x || !w || !scores || !choice || !idx || !wt || n_tok < 1 || D < 1 ||
        n_exp < 1 || n_exp > kRouteMaxExperts || k < 1 || k > 64 || k > n_exp ||
        !f32mm_fits(false, D, n_exp) || !aligned(x, 16) || !aligned(w, 16)) {
        set_err("router_dev: bad arguments (D % 16, n_exp % 32, 16-byte aligned rows, "
                "1 <= k <= min(64, n_exp), n_exp <= 4096)");
        return 0;
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    ExpertWork ew{};
    ew.w[0] = w;
    const int mt = n_tok <= 16 ? 1 : n_tok <= 32 ? 2 : 4;
    HIP_TRY(launch_f32mm(false, mt, nullptr, nullptr, 0, &ew, n_tok, x, nullptr, scores, 0, D,
                         n_exp, 0, 0.f, 0.f, st));
    HIP_TRY(launch_route_tail(scores, bias, choice, n_tok, n_exp, st));
    HIP_TRY(launch_moe_topk(choice, scores, n_tok, n_exp, k, idx, wt, st));
    if (rscale != 1.f)
        HIP_TRY(launch_scale(wt, (size_t)n_tok * k, rscale, st));
    return 1;
}

int mvllm_hip_linear_dev(int fmt, const void *w, const void *scales, int O, int K,
                         const float *x, int n, float *y, void *stream) {
    Ctx &C = ctx();
    std::lock_guard<std::mutex> lk(C.mu);
    set_err("");
    const bool q = fmt == 4 || fmt == 7;
    if (!C.ready || !w || !x || !y || n < 1 || (fmt != 0 && fmt != 8 && !q) ||
        ((q || fmt == 8) && !scales) ||
        (fmt == 0 && (!f32mm_fits(false, K, O) || !aligned(w, 16) || !aligned(x, 16))) ||
        (fmt == 8 && (!f32mm_fits(false, K, O) || !aligned(w, 4) || !aligned(x, 16) ||
                      !aligned(scales, 4))) ||
        (q && (K % 256 || O % 256 || !aligned(w, 8) || !aligned(scales, fmt == 4 ? 16 : 8)))) {
        set_err("linear_dev: bad arguments (fmt 0: K % 16, O % 32, 16-byte aligned rows; "
                "fmt 8: K % 16, O % 32, 4-byte aligned codes and scales, 16-byte aligned x; "
                "fmt 4/7: K % 256, O % 256, 8-byte aligned codes, aligned scales)");
        return 0;
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    ExpertWork ew{};
    if (fmt == 0 || fmt == 8) {
        // f32 matrix cores on the f32 rows; int8 codes convert exactly and the row scale
        // applies once per output (quant::matmul_int8_row, src/quant/quant.cpp:255-268)
        ew.w[0] = w;
        ew.s[0] = scales;
        const int mt = n <= 16 ? 1 : n <= 32 ? 2 : 4;
        HIP_TRY(launch_f32mm(false, mt, nullptr, nullptr, 0, &ew, n, x, nullptr, y, 0, K, O, 0,
                             0.f, 0.f, st, fmt == 8));
        return 1;
    }
    // quantized: the input rows as two bf16 terms (2^-17 relative), then the grouped GEMM.
    // The planes buffer is shared by every call: a call on another stream than the
    // previous one waits for it first, as the block entry points do.
    ew.w[2] = w;
    ew.s[2] = scales;
    const int terms = 2;
    HIP_TRY(C.Lp.ensure((size_t)terms * 2 * n * K));
    if (!order_after_previous(C, st))
        return 0;
    HIP_TRY(launch_prep_planes(fmt, terms, x, nullptr, n, K, n, C.Lp.p, st));
    const int mt = n <= 16 ? 1 : n <= 32 ? 2 : 4;
    HIP_TRY(launch_gemm_rows(fmt, terms, mt, &ew, n, C.Lp.p, y, K, O, st));
    C.last_stream = st;
    C.have_last = true;
    return 1;
}

int mvllm_hip_rmsnorm_dev(const float *x, const float *w, float *y, int rows, int n, float eps,
                          void *stream) {
    Ctx &C = ctx();
    set_err("");
    if (!C.ready || !x || !y || rows < 1 || n < 1) {
        set_err("rmsnorm_dev: bad arguments");
        return 0;
    }
    HIP_TRY(launch_rmsnorm(x, w, y, rows, n, eps, static_cast<hipStream_t>(stream)));
    return 1;
}

int mvllm_hip_bf16_planes(int fmt, int terms, const float *x_dev, int n, int K,
                          uint16_t *planes_dev) {
    Ctx &C = ctx();
    std::lock_guard<std::mutex> lk(C.mu);
    set_err("");
    if (!C.ready || !x_dev || !planes_dev || (fmt != 4 && fmt != 7) || terms < 1 ||
        terms > 3 || n < 1 || K < 8 || K % 8) {
        set_err("bf16_planes: bad arguments");
        return 0;
    }
    HIP_TRY(launch_prep_planes(fmt, terms, x_dev, nullptr, n, K, n, planes_dev, C.own));
    HIP_TRY(hipStreamSynchronize(C.own));
    return 1;
}

int mvllm_hip_quantize_mxfp4(const float *x_dev, int n, int K, uint8_t *codes_dev,
                             uint8_t *scales_dev, uint16_t *planes_dev) {
    Ctx &C = ctx();
    std::lock_guard<std::mutex> lk(C.mu);
    set_err("");
    if (!C.ready || !x_dev || !codes_dev || !scales_dev || n < 1 || K < 32 || K % 32) {
        set_err("quantize_mxfp4: bad arguments");
        return 0;
    }
    HIP_TRY(launch_quantize_mxfp4(x_dev, n, K, codes_dev, scales_dev, C.own, nullptr,
                                  planes_dev));
    HIP_TRY(hipStreamSynchronize(C.own));
    return 1;
}

int mvllm_hip_membench(int kind, const void *src_dev, void *dst_dev, size_t bytes, int row_bytes,
                       int reps, double *ms_per_rep) {
    Ctx &C = ctx();
    std::lock_guard<std::mutex> lk(C.mu);
    set_err("");
    if (!C.ready || !src_dev || !dst_dev || bytes < 4096 || reps < 1 || kind < 0 || kind > 6 ||
        (kind >= 2 && (row_bytes < 1024 || row_bytes % 1024))) {
        set_err("membench: bad arguments");
        return 0;
    }
    hipEvent_t e0, e1;
    HIP_TRY(hipEventCreate(&e0));
    HIP_TRY(hipEventCreate(&e1));
    if (reps > 1)  // untimed warm-up pass (a single repetition is timed cold)
        HIP_TRY(launch_membench(kind, src_dev, dst_dev, bytes, row_bytes / 16, C.own));
    HIP_TRY(hipEventRecord(e0, C.own));
    for (int r = 0; r < reps; ++r)
        HIP_TRY(launch_membench(kind, src_dev, dst_dev, bytes, row_bytes / 16, C.own));
    HIP_TRY(hipEventRecord(e1, C.own));
    HIP_TRY(hipEventSynchronize(e1));
    float ms = 0.f;
    HIP_TRY(hipEventElapsedTime(&ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (ms_per_rep)
        *ms_per_rep = ms / reps;
    return 1;
}

}  // extern "C"
