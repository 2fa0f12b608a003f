// kern_mfma.hip -- decode-shaped expert GEMMs on the gfx950 matrix cores, one launch per
// projection (the task itself is in mfma_dec.h), and the matrix-core decode restated
// element by element for checking.
#include "mfma_dec.h"

#include <algorithm>
#include <cmath>
#include <type_traits>
#include <utility>
#include <vector>

namespace mvllm_hip {


template <int FMT, bool DUAL, int TERMS, int KS, int NT, int SR, bool PACK>
__global__ __launch_bounds__(kDecThreads) __attribute__((amdgpu_waves_per_eu(4)))
void k_mfma_dec(DecArgs A) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const int item = blockIdx.x / A.wgs;
    if (A.n_items_dev && item >= *A.n_items_dev)
        return;  // past the device planner's item count (the whole workgroup)
    dec_task<FMT, DUAL, TERMS, KS, NT, SR, PACK>(A, item, blockIdx.x - item * A.wgs,
                                                 (int)threadIdx.x, smem);
}

// Gate/up with its descriptors in the kernel arguments (device memory at launch).
template <int FMT, int TERMS, int KS, int SR, bool PACK>
__global__ __launch_bounds__(kDecThreads) __attribute__((amdgpu_waves_per_eu(4)))
void k_mfma_dec_inl(DecArgs A, DecInline I) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const int item = blockIdx.x / A.wgs;
    dec_task<FMT, true, TERMS, KS, 2, SR, PACK, true>(A, item, blockIdx.x - item * A.wgs,
                                                      (int)threadIdx.x, smem, I.d);
}

// Wave 0 of a k_mfma_dec_seg workgroup (lane 0..63): the descriptor of item `item` in kd
// (kd->nrow = 0 when the call has no such item).  Items are the rmax-row pieces of the live
// segments in segment order, k_dplan_dec's numbering: a segment whose expert id is outside
// the table, or whose blob is null or not 256-byte aligned, or that has no rows, has none.
// Column block 0 of each item also writes the item's down descriptor; workgroup 0 the
// item count and the status.
__device__ __forceinline__ void seg_plan(const DecSegArgs &G, int item, int wg, int lane,
                                         DecDescK *kd) {
    // the first 64 segments' fields loaded with the counts, before they are known
    int e_l = -1, x_l = 0, nr_l = 0;
    if (lane < G.cap_e) {
        e_l = G.eids[lane];
        x_l = G.xoff[lane];
        nr_l = G.nr[lane];
    }
    const int nb = min(max(G.counts[0], 0), G.cap_e);
    const int nrows = min(max(G.counts[1], 0), G.cap_rows);
    int base = 0, err = 0;
    bool mine = false;
    const char *my_blob = nullptr;
    int my_x0 = 0, my_n = 0, my_r0 = 0;
    // Up to 64 segments (one lane each): the item's owner is found on the assumption that
    // every segment with rows has a usable blob, and its rows are read together with the
    // blob table; the general scan below runs only if some blob is not usable.
    bool fast = nb <= 64;
    int sp_rows[16];
    float sp_w[16];
    if (fast) {
        const bool in = lane < nb;
        const int n = !in || x_l < 0 || x_l > nrows ? 0 : max(0, min(nr_l, nrows - max(x_l, 0)));
        const int cnt = n ? (n + G.rmax - 1) / G.rmax : 0;
        int incl = cnt;
        for (int o = 1; o < 64; o <<= 1) {
            const int v = __shfl_up(incl, o);
            if (lane >= o)
                incl += v;
        }
        const int excl = incl - cnt;
        const bool own = cnt && item >= excl && item < incl;
        const char *blob =
            in && e_l >= 0 && e_l < G.n_table ? static_cast<const char *>(G.table[e_l]) : nullptr;
        if (own) {
            const int r0 = (item - excl) * G.rmax, jb = x_l + r0, nrow = min(G.rmax, n - r0);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                sp_rows[r] = r < nrow ? G.rows[jb + r] : 0;
                sp_w[r] = r < nrow ? G.rw[jb + r] : 0.f;
            }
            my_x0 = x_l;
            my_n = n;
            my_r0 = r0;
        }
        const bool bad = n && (!blob || (reinterpret_cast<uintptr_t>(blob) & 255));
        err = in && (reinterpret_cast<uintptr_t>(blob) & 255) ? 2 : 0;
        if (__builtin_amdgcn_ballot_w64(bad) == 0) {
            mine = own;
            my_blob = blob;
            base = __shfl(incl, 63);
        } else {
            fast = false;  // the general scan, with the blobs' validity
            err = 0;
            my_x0 = my_n = my_r0 = 0;
        }
    }
    for (int c0 = 0; !fast && c0 < nb; c0 += 64) {  // uniform trip count
        const int i = c0 + lane;
        int cnt = 0, x0 = 0, n = 0;
        const char *blob = nullptr;
        if (i < nb) {
            const int e = G.eids[i];
            x0 = G.xoff[i];
            const int nri = G.nr[i];
            n = (x0 < 0 || x0 > nrows) ? 0 : max(0, min(nri, nrows - max(x0, 0)));
            blob = (e >= 0 && e < G.n_table) ? static_cast<const char *>(G.table[e]) : nullptr;
            if (reinterpret_cast<uintptr_t>(blob) & 255) {
                err = 2;
                blob = nullptr;
            }
            cnt = (blob && n) ? (n + G.rmax - 1) / G.rmax : 0;
        }
        int incl = cnt;
        for (int o = 1; o < 64; o <<= 1) {
            const int v = __shfl_up(incl, o);
            if (lane >= o)
                incl += v;
        }
        const int excl = incl - cnt;
        if (cnt && item >= base + excl && item < base + incl) {
            mine = true;
            my_blob = blob;
            my_x0 = x0;
            my_n = n;
            my_r0 = (item - base - excl) * G.rmax;
        }
        base += __shfl(incl, 63);
    }
    if (item == 0 && wg == 0) {
        const bool any_err = __builtin_amdgcn_ballot_w64(err != 0) != 0;
        if (lane == 0) {
            *G.n_items = min(base, G.cap_items);
            // 1: more items than the capacity (segments whose rows overlap; the items past
            // it are dropped), as the planner kernel reports it
            *G.err = any_err ? 2 : base > G.cap_items ? 1 : 0;
        }
    }
    if (__builtin_amdgcn_ballot_w64(mine) == 0 || item >= G.cap_items) {
        if (lane == 0)
            kd->nrow = 0;
        return;
    }
    if (!mine)
        return;
    const int jb = my_x0 + my_r0, nrow = min(G.rmax, my_n - my_r0);
    if (!fast) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            sp_rows[r] = r < nrow ? G.rows[jb + r] : 0;
            sp_w[r] = r < nrow ? G.rw[jb + r] : 0.f;
        }
    }
    DecDescK k;
    k.w0 = my_blob + G.off[0];
    k.off[0] = (int)(G.off[2] - G.off[0]);
    k.off[1] = (int)(G.off[1] - G.off[0]);
    k.off[2] = (int)(G.off[3] - G.off[0]);
    k.jbase = (unsigned short)jb;
    k.nrow = (unsigned short)nrow;
    DecDesc d{};
    d.w[0] = d.w[1] = my_blob + G.off[4];
    d.s[0] = d.s[1] = my_blob + G.off[5];
    d.jbase = jb;
    d.nrow = nrow;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int t = sp_rows[r];
        const bool ok = r < nrow && t >= 0 && t < G.S;
        k.rows[r] = (unsigned short)(ok ? t : 0);
        d.rows[r] = ok ? t : -1;
        d.wts[r] = r < nrow ? sp_w[r] : 0.f;
    }
    *kd = k;
    if (wg == 0)
        G.dn[item] = d;
}

// Gate/up of the device-resident block at decode shapes, planning its own item from the
// segments (no planner launch): wave 0 builds the descriptor in LDS, then the workgroup
// runs the task as the compact-descriptor kernel does.
template <int FMT, int TERMS, int KS, int SR, bool PACK>
__global__ __launch_bounds__(kDecThreads) __attribute__((amdgpu_waves_per_eu(4)))
void k_mfma_dec_seg(DecArgs A, DecSegArgs G) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const int item = blockIdx.x / A.wgs, wg = blockIdx.x - item * A.wgs;
    DecDescK *kd = reinterpret_cast<DecDescK *>(smem + G.kd_off);
    if (threadIdx.x < 64)
        seg_plan(G, item, wg, (int)threadIdx.x, kd);
    __syncthreads();
    if (__builtin_amdgcn_readfirstlane((int)kd->nrow) == 0)
        return;  // past the call's items (the whole workgroup)
    dec_task<FMT, true, TERMS, KS, 2, SR, PACK, true>(A, 0, wg, (int)threadIdx.x, smem, kd);
}

size_t mfma_dec_lds_bytes(int fmt, int K, int rmax, int terms, int dual, int ks, int nt) {
    (void)dual;
    return dec_lds_plan(fmt, K, rmax, terms, ks, nt, nullptr);
}

// Raises kernel f's dynamic LDS limit to `lds` bytes once per process: up to 64 KiB needs
// no attribute, and a limit already raised that far is not set again (the attribute call
// costs host time on every decode launch otherwise).  The library's entry points hold its
// lock around every launch, which guards this table.
static hipError_t lds_limit(const void *f, size_t lds) {
    static std::vector<std::pair<const void *, size_t>> set;
    if (lds <= 65536)
        return hipSuccess;
    for (auto &p : set)
        if (p.first == f && p.second >= lds)
            return hipSuccess;
    hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess)
        return e;
    for (auto &p : set)
        if (p.first == f) {
            p.second = lds;
            return e;
        }
    set.emplace_back(f, lds);
    return e;
}

template <int FMT, bool DUAL, int TERMS, int KS, int NT>
static hipError_t launch_dec_t(DecArgs a, int n_items, hipStream_t st, const DecDescK *inl,
                               const DecSegArgs *seg) {
    const size_t lds = mfma_dec_lds_bytes(FMT, a.K, a.rmax, TERMS, DUAL, KS, NT);
    // the self-planning kernel keeps its descriptor past the task's LDS
    const size_t kd_off = (lds + 15) & ~(size_t)15;
    const size_t lds_seg = kd_off + sizeof(DecDescK);
    const int tiles_wg = (kDecWaves / KS) * (DUAL ? 1 : NT);  // column tiles per workgroup
    if (a.K % 512 || a.K % (256 * KS) || a.K / KS > dec_max_kr(FMT) || a.O % (16 * tiles_wg) ||
        a.rmax < 1 || a.rmax > 16 ||
        lds > kDecLdsBudget)
        return hipErrorInvalidValue;
    a.wgs = a.O / (16 * tiles_wg);
    if (a.n_cp < 0 || a.n_cp > n_items * a.wgs || (a.n_cp > 0 && !DUAL))
        return hipErrorInvalidValue;  // every descriptor to copy needs a workgroup
    const dim3 grid((unsigned)(n_items * a.wgs)), block(kDecThreads);
    // staging registers per thread: dual = 8-float chunks of rmax rows, single = uint4 of
    // TERMS planes of rmax rows
    const size_t need = DUAL ? (size_t)a.rmax * (a.K / 8) : (size_t)TERMS * a.rmax * (a.K / 8);
    const int sr = (int)((need + kDecThreads - 1) / kDecThreads);
    if (inl && (!DUAL || n_items > kDecInline))
        return hipErrorInvalidValue;
    if (seg && (!DUAL || inl || a.n_cp || a.n_items_dev || lds_seg > kDecLdsBudget))
        return hipErrorInvalidValue;
    DecSegArgs sg{};
    if (seg) {
        sg = *seg;
        sg.kd_off = (int)kd_off;
    }
    DecInline di;
    if (inl)
        std::copy(inl, inl + n_items, di.d);
    auto go = [&](auto kern, auto kern_inl, auto kern_seg, auto has_inl) {
        constexpr bool HI = decltype(has_inl)::value;
        if constexpr (HI) {
            if (seg) {
                hipError_t e = lds_limit(reinterpret_cast<const void *>(kern_seg), lds_seg);
                if (e == hipSuccess)
                    hipLaunchKernelGGL(kern_seg, grid, block, lds_seg, st, a, sg);
                return e;
            }
        }
        const void *f = HI && inl ? reinterpret_cast<const void *>(kern_inl)
                                  : reinterpret_cast<const void *>(kern);
        hipError_t e = lds_limit(f, lds);
        if (e != hipSuccess)
            return e;
        if constexpr (HI) {
            if (inl) {
                hipLaunchKernelGGL(kern_inl, grid, block, lds, st, a, di);
                return e;
            }
        }
        hipLaunchKernelGGL(kern, grid, block, lds, st, a);
        return e;
    };
    // the compact-descriptor kernel of the same configuration (gate/up only)
    auto with_inl = [&](auto kern, auto sr_c, auto pack_c) {
        constexpr int SRv = decltype(sr_c)::value;
        constexpr bool PKv = decltype(pack_c)::value;
        if constexpr (DUAL && NT == 2)
            return go(kern, k_mfma_dec_inl<FMT, TERMS, KS, SRv, PKv>,
                      k_mfma_dec_seg<FMT, TERMS, KS, SRv, PKv>, std::true_type{});
        else
            return go(kern, kern, kern, std::false_type{});
    };
    hipError_t e;
    constexpr int SR1 = DUAL ? 2 : 4, SR2 = DUAL ? kDecStageDual : kDecStageSingle;
    using S1 = std::integral_constant<int, SR1>;
    using S2 = std::integral_constant<int, SR2>;
    using PT = std::true_type;
    using PF = std::false_type;
    if (a.pack && (TERMS != 2 || a.rmax > 8))
        return hipErrorInvalidValue;
    if (DUAL ? sr <= 2 : sr <= 4) {
        if constexpr (TERMS == 2)
            e = a.pack ? with_inl(k_mfma_dec<FMT, DUAL, TERMS, KS, NT, SR1, true>, S1{}, PT{})
                       : with_inl(k_mfma_dec<FMT, DUAL, TERMS, KS, NT, SR1, false>, S1{}, PF{});
        else
            e = with_inl(k_mfma_dec<FMT, DUAL, TERMS, KS, NT, SR1, false>, S1{}, PF{});
    } else if (DUAL ? sr <= kDecStageDual : sr <= kDecStageSingle) {
        if constexpr (TERMS == 2)
            e = a.pack ? with_inl(k_mfma_dec<FMT, DUAL, TERMS, KS, NT, SR2, true>, S2{}, PT{})
                       : with_inl(k_mfma_dec<FMT, DUAL, TERMS, KS, NT, SR2, false>, S2{}, PF{});
        else
            e = with_inl(k_mfma_dec<FMT, DUAL, TERMS, KS, NT, SR2, false>, S2{}, PF{});
    } else {
        return hipErrorInvalidValue;
    }
    if (e != hipSuccess)
        return e;
    return hipGetLastError();
}

template <int FMT, bool DUAL, int TERMS>
static hipError_t launch_dec_k(const DecArgs &a, int n_items, int ks, int nt, hipStream_t st,
                               const DecDescK *inl, const DecSegArgs *seg) {
    if constexpr (DUAL) {
        if (nt != 2)
            return hipErrorInvalidValue;
        switch (ks) {
        case 1: return launch_dec_t<FMT, true, TERMS, 1, 2>(a, n_items, st, inl, seg);
        case 2: return launch_dec_t<FMT, true, TERMS, 2, 2>(a, n_items, st, inl, seg);
        case 4: return launch_dec_t<FMT, true, TERMS, 4, 2>(a, n_items, st, inl, seg);
        case 8: return launch_dec_t<FMT, true, TERMS, 8, 2>(a, n_items, st, inl, seg);
        default: return hipErrorInvalidValue;
        }
    } else {
        if (nt == 2)
            return ks == 1 ? launch_dec_t<FMT, false, TERMS, 1, 2>(a, n_items, st, inl, seg)
                           : hipErrorInvalidValue;
        switch (ks) {
        case 1: return launch_dec_t<FMT, false, TERMS, 1, 1>(a, n_items, st, inl, seg);
        case 2: return launch_dec_t<FMT, false, TERMS, 2, 1>(a, n_items, st, inl, seg);
        case 4: return launch_dec_t<FMT, false, TERMS, 4, 1>(a, n_items, st, inl, seg);
        case 8: return launch_dec_t<FMT, false, TERMS, 8, 1>(a, n_items, st, inl, seg);
        default: return hipErrorInvalidValue;
        }
    }
}

template <int FMT, bool DUAL>
static hipError_t launch_dec_fd(const DecArgs &a, int n_items, int terms, int ks, int nt,
                                hipStream_t st, const DecDescK *inl,
                                const DecSegArgs *seg) {
    if (terms <= 1)
        return launch_dec_k<FMT, DUAL, 1>(a, n_items, ks, nt, st, inl, seg);
    if (terms == 2)
        return launch_dec_k<FMT, DUAL, 2>(a, n_items, ks, nt, st, inl, seg);
    return launch_dec_k<FMT, DUAL, 3>(a, n_items, ks, nt, st, inl, seg);
}

hipError_t launch_mfma_dec(int fmt, bool dual, int terms, int ks, int nt, const DecDesc *desc,
                           int n_items, const float *xin, const void *pin, const float *xs,
                           void *pout, float *hp, float *out, int K, int O, int rcap, int rmax,
                           int act, float act_a, float act_b, bool fold, bool pack,
                           const DecDesc *cp_src, DecDesc *cp_dst, int n_cp, hipStream_t st,
                           const DecDescK *inl, const int *n_items_dev, const DecSegArgs *seg) {
    if (n_items <= 0)
        return n_cp > 0 ? hipErrorInvalidValue : hipSuccess;
    if (K > kDecMaxK || (n_items_dev && (inl || n_cp > 0)))
        return hipErrorInvalidValue;
    if (seg && (seg->rmax != rmax || seg->cap_items != n_items || seg->cap_rows > 65535 ||
                seg->cap_rows > rcap || seg->S > 65535 || seg->cap_e < 0 || !seg->dn ||
                !seg->n_items || !seg->err))
        return hipErrorInvalidValue;
    DecArgs a{};
    a.n_items_dev = n_items_dev;
    a.desc = desc;
    a.xin = xin;
    a.pin = static_cast<const __bf16 *>(pin);
    a.xs = xs;
    a.pout = static_cast<__bf16 *>(pout);
    a.hp = hp;
    a.out = out;
    a.fold = fold ? 1 : 0;
    a.K = K;
    a.O = O;
    a.rcap = rcap;
    a.rmax = rmax;
    a.act = act;
    a.act_a = act_a;
    a.act_b = act_b;
    a.cp_src = cp_src;
    a.cp_dst = cp_dst;
    a.n_cp = n_cp;
    a.pack = pack ? 1 : 0;
    if (fmt == 4)
        return dual ? launch_dec_fd<4, true>(a, n_items, terms, ks, nt, st, inl, seg)
                    : launch_dec_fd<4, false>(a, n_items, terms, ks, nt, st, inl, seg);
    if (fmt == 7)
        return dual ? launch_dec_fd<7, true>(a, n_items, terms, ks, nt, st, inl, seg)
                    : launch_dec_fd<7, false>(a, n_items, terms, ks, nt, st, inl, seg);
    return hipErrorInvalidValue;
}

// ---- checking aid: the weights exactly as the MFMA path decodes them --------------

template <int FMT>
__global__ void k_dequant_bf16path(const uint8_t *P, const void *S, int O, int K, float *w) {
    // lane-free restatement: each thread decodes one dword (8 weights) like decode_b
    const int ngs = FMT == 4 ? K / 64 : K / 32;
    const size_t total = (size_t)O * (size_t)(K / 8);
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const int o = (int)(i / (K / 8)), d = (int)(i % (K / 8));
        const uint32_t word = reinterpret_cast<const uint32_t *>(P + (size_t)o * (K / 2))[d];
        const int k0 = 8 * d;
        float s7 = 0.f;
        if constexpr (FMT == 7)
            s7 = __uint_as_float((uint32_t)static_cast<const uint8_t *>(S)[(size_t)o * ngs + k0 / 32]
                                 << 23);
        bf16x8 b = decode_b<FMT>(word, s7);
        if constexpr (FMT == 7) {
            if (b7_exceptional(s7))
                b = decode_b7_exact(word, s7);
        }
        float *dst = w + (size_t)o * K + k0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float v = (float)b[a_slot<FMT>(e)];
            if constexpr (FMT == 4)
                dst[e] = (v - 8.f) * static_cast<const float *>(S)[(size_t)o * ngs + k0 / 64];
            else
                dst[e] = v;
        }
    }
}

hipError_t launch_dequant_bf16path(int fmt, const void *packed, const void *scales, int O, int K,
                                   float *w, hipStream_t st) {
    if (K % 64 || ((uintptr_t)packed & 3))
        return hipErrorInvalidValue;
    if (fmt == 4)
        hipLaunchKernelGGL(k_dequant_bf16path<4>, dim3(1024), dim3(256), 0, st,
                           static_cast<const uint8_t *>(packed), scales, O, K, w);
    else if (fmt == 7)
        hipLaunchKernelGGL(k_dequant_bf16path<7>, dim3(1024), dim3(256), 0, st,
                           static_cast<const uint8_t *>(packed), scales, O, K, w);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace mvllm_hip
