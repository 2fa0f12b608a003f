// kern_dplan.hip -- the plan of a moe_block call whose segments live in device memory
// (as mvllm_hip_moe_segments_dev writes them), built on the device: no host round trip
// between routing and the block.
//
// The host-planned call (build_plan / plan_gemm in mvllm_hip.cpp) turns the segments
// into per-expert work, grouped-GEMM items in row classes, and the combine's per-token
// lists.  Here the same three come from kernels:
//   k_dplan   one workgroup: per segment i, expert work from the blob table (blob address
//             of expert eids[i] + the blob geometry's piece offsets), its rows'
//             liveness, and its grouped-GEMM items (full blocks of BM rows in the top
//             class, the remainder in the smallest class that holds it), written per
//             class in expert order by a workgroup scan, with the class item counts;
//   k_dplan_dec  the same for decode-shaped calls: the decode kernels' descriptors (items
//             of up to rmax rows, a gate/up and a down descriptor each) and their count;
//   k_csr_*   the combine lists: per out row t, the compact rows j with rows[j] == t of
//             experts that are present, in ascending j (= the reference's expert order,
//             src/gpu/metal_ops.cpp:328-339): count, scan, place, then a per-row sort.
// A segment whose expert id is outside the table, or whose table entry is null, consumes
// its rows without writing (the reference's null-expert rule, metal_ops.cpp:291-296).
#include "mfma_common.h"

#include <algorithm>

namespace mvllm_hip {

constexpr int kPlanThreads = 1024;

// smallest class of 16 * 2^c rows that holds n rows
__device__ __forceinline__ int dplan_class(int n) {
    return n <= 16 ? 0 : n <= 32 ? 1 : n <= 64 ? 2 : n <= 128 ? 3 : 4;
}

// Items per class of a segment of n live rows, the host planner's rule (plan_gemm): full
// blocks of bm rows in the top class, the remainder in the smallest class that holds it,
// or with split64 a remainder of 33-64 rows as two items of the 32-row class.
__device__ __forceinline__ void dplan_counts(const DPlanArgs &A, int n, int (&k)[kGemmClasses]) {
#pragma unroll
    for (int c = 0; c < kGemmClasses; ++c)
        k[c] = 0;
    k[A.top] = n / A.bm;
    const int rem = n % A.bm;
    if (rem && A.split64 && rem > 32 && rem <= 64)
        k[1] += 2;
    else if (rem)
        k[dplan_class(rem)] += 1;
}

// The blob of expert e (null when e is outside the table, its entry is null or not
// 256-byte aligned: err = 2 for the last) and the live row count of a segment at compact
// row x0 with nr rows (out of nrows).
template <class Args>
__device__ __forceinline__ const char *dplan_blob(const Args &A, int e, int nrows, int x0,
                                                  int nr, int &n) {
    n = (x0 < 0 || x0 > nrows) ? 0 : max(0, min(nr, nrows - max(x0, 0)));
    const char *blob = (e >= 0 && e < A.n_table) ? static_cast<const char *>(A.table[e])
                                                 : nullptr;
    if (reinterpret_cast<uintptr_t>(blob) & 255) {  // not a slab / tier blob address
        *A.err = 2;
        blob = nullptr;
    }
    return blob;
}

// Segment i's blob, first compact row x0 and live row count n (dplan_blob).
template <class Args>
__device__ __forceinline__ const char *dplan_segment(const Args &A, int i, int nrows, int &x0,
                                                     int &n) {
    // the three independent loads first, then the table read that depends on one
    const int e = A.eids[i];
    x0 = A.xoff[i];
    const int nr = A.nr[i];
    return dplan_blob(A, e, nrows, x0, nr, n);
}

__global__ __launch_bounds__(kPlanThreads) void k_dplan(DPlanArgs A) {
    __shared__ int part[kPlanThreads][kGemmClasses];
    __shared__ int tot[kGemmClasses];
    const int tid = threadIdx.x;
    const int nb = min(max(A.counts[0], 0), A.cap_e);
    const int nrows = min(max(A.counts[1], 0), A.cap_rows);
    for (int j = tid; j < nrows; j += kPlanThreads)
        A.row_ok[j] = 0;
    if (tid == 0)
        *A.err = 0;
    __syncthreads();
    // segments [s0, s1) of this thread, in order
    const int per = (nb + kPlanThreads - 1) / kPlanThreads;
    const int s0 = min(nb, tid * per), s1 = min(nb, s0 + per);
    int cnt[kGemmClasses] = {};
    for (int i = s0; i < s1; ++i) {
        int x0, n;
        const char *blob = dplan_segment(A, i, nrows, x0, n);
        ExpertWork w{};
        if (blob) {
            w.w[0] = blob + A.off[0];
            w.s[0] = blob + A.off[1];
            w.w[1] = blob + A.off[2];
            w.s[1] = blob + A.off[3];
            w.w[2] = blob + A.off[4];
            w.s[2] = blob + A.off[5];
        }
        w.row0 = max(x0, 0);
        w.nrows = blob ? n : 0;
        A.ew[i] = w;
        if (!blob || n == 0)
            continue;
        for (int j = x0; j < x0 + n; ++j)
            A.row_ok[j] = 1;
        int k[kGemmClasses];
        dplan_counts(A, n, k);
#pragma unroll
        for (int c = 0; c < kGemmClasses; ++c)
            cnt[c] += k[c];
    }
#pragma unroll
    for (int c = 0; c < kGemmClasses; ++c)
        part[tid][c] = cnt[c];
    __syncthreads();
    // exclusive scan over threads, one class per wave of the first kGemmClasses
    if (tid < kGemmClasses * 64) {
        const int c = tid >> 6, l = tid & 63;
        constexpr int kPer = kPlanThreads / 64;  // 16 consecutive threads per lane
        int run = 0;
        for (int k = 0; k < kPer; ++k) {
            const int v = part[l * kPer + k][c];
            part[l * kPer + k][c] = run;
            run += v;
        }
        // exclusive scan of the lanes' sums
        int incl = run;
        for (int o = 1; o < 64; o <<= 1) {
            const int v = __shfl_up(incl, o);
            if (l >= o)
                incl += v;
        }
        const int base = incl - run;
        for (int k = 0; k < kPer; ++k)
            part[l * kPer + k][c] += base;
        if (l == 63)
            tot[c] = incl;
    }
    __syncthreads();
    int pos[kGemmClasses];
#pragma unroll
    for (int c = 0; c < kGemmClasses; ++c)
        pos[c] = part[tid][c];
    for (int i = s0; i < s1; ++i) {
        const ExpertWork &w = A.ew[i];
        const int n = w.nrows;
        // word 3: (index in the segment's run of items of the class << 16) | run length,
        // as the host writes it (the 16- and 32-row kernels order a run's tasks column
        // block by column block).  A run that would pass the class's capacity (inputs whose
        // segments overlap) is written as items alone: a run's tasks index all its items,
        // and those past the capacity are never written.
        int k[kGemmClasses], idx[kGemmClasses] = {};
        dplan_counts(A, n, k);
        auto put = [&](int c, int r0, int nrow) {
            const bool fits = pos[c] - idx[c] + k[c] <= A.item_cap[c];
            const int word = k[c] < 0x8000 && fits ? (idx[c] << 16) | k[c] : 1;
            ++idx[c];
            if (pos[c] < A.item_cap[c])
                A.items[A.item_base[c] + pos[c]] = int4{i, r0, nrow, word};
            else
                *A.err = 1;
            ++pos[c];
        };
        for (int r0 = 0; r0 < n; r0 += A.bm) {
            const int nrow = min(A.bm, n - r0);
            if (nrow == A.bm) {
                put(A.top, r0, nrow);
            } else if (A.split64 && nrow > 32 && nrow <= 64) {
                put(1, r0, 32);
                put(1, r0 + 32, nrow - 32);
            } else {
                put(dplan_class(nrow), r0, nrow);
            }
        }
    }
    if (tid < kGemmClasses)
        A.n_items[tid] = min(tot[tid], A.item_cap[tid]);
}

// Decode-shaped calls: items of up to rmax rows of each live segment, in segment order,
// each with the gate/up descriptor (the input row of each item row: its out row, x being
// [S][D]; 0 for a row whose out row is out of range, whose H is then never used) and the
// down descriptor (out row and combine weight of each item row, -1 for such a row: the
// folded combine skips it).  One workgroup: the item counts of each thread's segments,
// a workgroup scan, then the descriptors.
__global__ __launch_bounds__(kPlanThreads) void k_dplan_dec(DPlanDecArgs A) {
    __shared__ int wsum[kPlanThreads / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // segment tid's fields, loaded with the counts before they are known (calls of at most
    // kPlanThreads segments have one a thread: the plan's dependent reads are then the
    // counts and these, the blob table, the rows, nothing more)
    int e_t = -1, x_t = 0, nr_t = 0;
    if (tid < A.cap_e) {
        e_t = A.eids[tid];
        x_t = A.xoff[tid];
        nr_t = A.nr[tid];
    }
    const int nb = min(max(A.counts[0], 0), A.cap_e);
    const int nrows = min(max(A.counts[1], 0), A.cap_rows);
    for (int j = tid; j < nrows; j += kPlanThreads)
        A.row_ok[j] = 0;
    if (tid == 0)
        *A.err = 0;
    __syncthreads();
    const int per = (nb + kPlanThreads - 1) / kPlanThreads;
    const int s0 = min(nb, tid * per), s1 = min(nb, s0 + per);
    // segment tid's blob, read once (the second pass reuses it)
    const char *b_t = nullptr;
    int n_t = 0;
    if (s0 <= tid && tid < s1)
        b_t = dplan_blob(A, e_t, nrows, x_t, nr_t, n_t);
    auto segment = [&](int i, int &x0, int &n) -> const char * {
        if (i == tid) {
            x0 = x_t;
            n = n_t;
            return b_t;
        }
        return dplan_segment(A, i, nrows, x0, n);
    };
    int cnt = 0;
    for (int i = s0; i < s1; ++i) {
        int x0, n;
        if (!segment(i, x0, n) || n == 0)
            continue;
        for (int j = x0; j < x0 + n; ++j)
            A.row_ok[j] = 1;
        cnt += (n + A.rmax - 1) / A.rmax;
    }
    int incl = cnt;  // inclusive scan within the wave, then over the waves' sums
    for (int o = 1; o < 64; o <<= 1) {
        const int v = __shfl_up(incl, o);
        if (lane >= o)
            incl += v;
    }
    if (lane == 63)
        wsum[wave] = incl;
    __syncthreads();
    int pos = incl - cnt, tot = 0;
    for (int w = 0; w < kPlanThreads / 64; ++w) {
        pos += w < wave ? wsum[w] : 0;
        tot += wsum[w];
    }
    for (int i = s0; i < s1; ++i) {
        int x0, n;
        const char *blob = segment(i, x0, n);
        if (!blob || n == 0)
            continue;
        for (int r0 = 0; r0 < n; r0 += A.rmax, ++pos) {
            if (pos >= A.cap_items) {
                *A.err = 1;
                continue;
            }
            const int nrow = min(A.rmax, n - r0), jb = x0 + r0;
            DecDesc g{}, d{};
            g.w[0] = blob + A.off[0];
            g.s[0] = blob + A.off[1];
            g.w[1] = blob + A.off[2];
            g.s[1] = blob + A.off[3];
            d.w[0] = d.w[1] = blob + A.off[4];
            d.s[0] = d.s[1] = blob + A.off[5];
            g.jbase = d.jbase = jb;
            g.nrow = d.nrow = nrow;
            for (int r = 0; r < nrow; ++r) {
                const int t = A.rows[jb + r];
                const bool ok = t >= 0 && t < A.S;
                g.rows[r] = ok ? t : 0;
                d.rows[r] = ok ? t : -1;
                d.wts[r] = A.rw[jb + r];
            }
            A.gu[pos] = g;
            A.dn[pos] = d;
        }
    }
    if (tid == 0)
        *A.n_items = min(tot, A.cap_items);
}

// ---- the combine lists -----------------------------------------------------------

__device__ __forceinline__ int csr_live(const CsrArgs &A, int j) {
    const int t = A.rows[j];
    return (A.row_ok[j] && t >= 0 && t < A.S) ? t : -1;
}

__global__ void k_csr_zero(CsrArgs A) {
    for (int t = blockIdx.x * blockDim.x + threadIdx.x; t <= A.S; t += gridDim.x * blockDim.x)
        A.cnt[t] = 0;
}

__global__ void k_csr_count(CsrArgs A) {
    const int n = min(max(A.counts[1], 0), A.cap_rows);
    for (int j = blockIdx.x * blockDim.x + threadIdx.x; j < n; j += gridDim.x * blockDim.x) {
        const int t = csr_live(A, j);
        if (t >= 0)
            atomicAdd(&A.cnt[t], 1);
    }
}

// exclusive scan of cnt[0..S) into cnt[0..S] (tok_ptr) and cursor, one workgroup
__global__ __launch_bounds__(kPlanThreads) void k_csr_scan(CsrArgs A) {
    __shared__ int wsum[kPlanThreads / 64];
    __shared__ int carry;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid == 0)
        carry = 0;
    __syncthreads();
    for (int b = 0; b < A.S; b += kPlanThreads) {
        const int t = b + tid;
        const int v = t < A.S ? A.cnt[t] : 0;
        int incl = v;
        for (int o = 1; o < 64; o <<= 1) {
            const int u = __shfl_up(incl, o);
            if (lane >= o)
                incl += u;
        }
        if (lane == 63)
            wsum[wave] = incl;
        __syncthreads();
        int before = carry;
        for (int w = 0; w < wave; ++w)
            before += wsum[w];
        const int excl = before + incl - v;
        __syncthreads();  // every thread has read carry and wsum
        if (t < A.S) {
            A.cnt[t] = excl;
            A.cursor[t] = excl;
        }
        if (tid == kPlanThreads - 1)
            carry = excl + v;
        __syncthreads();
    }
    if (tid == 0)
        A.cnt[A.S] = carry;
}

__global__ void k_csr_place(CsrArgs A) {
    const int n = min(max(A.counts[1], 0), A.cap_rows);
    for (int j = blockIdx.x * blockDim.x + threadIdx.x; j < n; j += gridDim.x * blockDim.x) {
        const int t = csr_live(A, j);
        if (t < 0)
            continue;
        const int p = atomicAdd(&A.cursor[t], 1);
        A.ent_row[p] = j;
        A.ent_w[p] = A.rw[j];
    }
}

// each out row's entries in ascending compact row (insertion sort: a row has about top-k
// entries)
__global__ void k_csr_sort(CsrArgs A) {
    for (int t = blockIdx.x * blockDim.x + threadIdx.x; t < A.S; t += gridDim.x * blockDim.x) {
        const int e0 = A.cnt[t], e1 = A.cnt[t + 1];
        for (int i = e0 + 1; i < e1; ++i) {
            const int r = A.ent_row[i];
            const float w = A.ent_w[i];
            int k = i - 1;
            while (k >= e0 && A.ent_row[k] > r) {
                A.ent_row[k + 1] = A.ent_row[k];
                A.ent_w[k + 1] = A.ent_w[k];
                --k;
            }
            A.ent_row[k + 1] = r;
            A.ent_w[k + 1] = w;
        }
    }
}

hipError_t launch_dplan(const DPlanArgs &a, hipStream_t st) {
    hipLaunchKernelGGL(k_dplan, dim3(1), dim3(kPlanThreads), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_dplan_dec(const DPlanDecArgs &a, hipStream_t st) {
    if (a.rmax < 1 || a.rmax > 16 || a.cap_items < 1)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_dplan_dec, dim3(1), dim3(kPlanThreads), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_dcsr(const CsrArgs &a, hipStream_t st) {
    const unsigned gs = (unsigned)std::min(1024, (a.S + 255) / 256 + 1);
    const unsigned gr = (unsigned)std::min(1024, (a.cap_rows + 255) / 256);
    hipLaunchKernelGGL(k_csr_zero, dim3(gs), dim3(256), 0, st, a);
    hipLaunchKernelGGL(k_csr_count, dim3(gr), dim3(256), 0, st, a);
    hipLaunchKernelGGL(k_csr_scan, dim3(1), dim3(kPlanThreads), 0, st, a);
    hipLaunchKernelGGL(k_csr_place, dim3(gr), dim3(256), 0, st, a);
    hipLaunchKernelGGL(k_csr_sort, dim3(gs), dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // namespace mvllm_hip
