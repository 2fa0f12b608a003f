// kern_route.hip -- the routing in front of the expert block, on the device: moe_topk of
// every token (src/model/ops.cpp:860-889), then the moe_block segments of one batched
// call (the union of src/model/ops.cpp:1082-1099 and the per-expert gather of
// src/model/glm53.cpp:1938-1971 / src/model/kimi_k3.cpp:2009-2050).  Integer work and a
// few f32 additions and divisions in the reference's order: bit-exact.
//
//   k_moe_topk      one wave per token: k rounds of a wave-wide argmax under the
//                   reference's order (larger score first, lower index on ties), then the
//                   weights summed in pick order by every lane alike;
//   k_seg_count     per (token, slot): the expert's count of tokens whose summed weight
//                   is non-zero, and its presence (union membership: any slot);
//   k_seg_scan      one workgroup: experts in ascending id -> positions, row offsets,
//                   the capacity checks;
//   k_seg_rows      one workgroup per kept expert: its tokens in ascending order by a
//                   ballot per 256 tokens (two chunks a pass), written at the expert's
//                   row offset.
#include "moe_internal.h"

#include <algorithm>

namespace mvllm_hip {

// a ranks before b: larger score first, lower index on ties (the reference comparator;
// -0 and +0 tie).  Scores are not NaN (the reference's sort has no order for NaN).
__device__ __forceinline__ bool rank_before(float va, int a, float vb, int b) {
    return va == vb ? a < b : va > vb;
}

constexpr int kTopkWaves = 4;

// NV > 0: the lane's scores (elements lane + 64 s, s < NV) stay in registers for all k
// rounds (n_exp <= 64 NV); NV = 0 reads them again each round (up to 4096 experts).
template <int NV>
__global__ __launch_bounds__(64 * kTopkWaves) void k_moe_topk(const float *choice,
                                                                const float *mix, int n_tok,
                                                                int n_exp, int k, int *idx,
                                                                float *wt) {
    const int tok = blockIdx.x * kTopkWaves + (int)(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (tok >= n_tok)  // wave-uniform
        return;
    const float *row = choice + (size_t)tok * n_exp;
    float cv[NV > 0 ? NV : 1];
#pragma unroll
    for (int s = 0; s < NV; ++s)
        cv[s] = lane + 64 * s < n_exp ? row[lane + 64 * s] : 0.f;
    uint64_t taken = 0;  // bit s: element lane + 64 s is picked (n_exp <= 4096)
    int mine = -1;       // lane i < k: the i-th pick
    for (int i = 0; i < k; ++i) {
        float bv = 0.f;
        int bi = -1;
        if constexpr (NV > 0) {
#pragma unroll
            for (int s = 0; s < NV; ++s) {
                const int j = lane + 64 * s;
                if (j < n_exp && !((taken >> s) & 1u) && (bi < 0 || rank_before(cv[s], j, bv, bi))) {
                    bv = cv[s];
                    bi = j;
                }
            }
        } else {
            for (int s = 0; lane + 64 * s < n_exp; ++s) {
                const int j = lane + 64 * s;
                if ((taken >> s) & 1u)
                    continue;
                const float v = row[j];
                if (bi < 0 || rank_before(v, j, bv, bi)) {
                    bv = v;
                    bi = j;
                }
            }
        }
        // the order is total on the candidates, so any reduction tree finds the same one
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(bv, off);
            const int oi = __shfl_xor(bi, off);
            if (oi >= 0 && (bi < 0 || rank_before(ov, oi, bv, bi))) {
                bv = ov;
                bi = oi;
            }
        }
        if ((bi & 63) == lane)
            taken |= 1ull << (bi >> 6);
        if (lane == i)
            mine = bi;
    }
    // weights: clipped at 0, summed in pick order (every lane adds the same sequence)
    float w = 0.f;
    if (lane < k) {
        w = mix ? mix[(size_t)tok * n_exp + mine] : row[mine];
        if (w < 0.f)
            w = 0.f;
    }
    float sum = 0.f;
    for (int i = 0; i < k; ++i)
        sum += __shfl(w, i);
    if (lane < k) {
        idx[(size_t)tok * k + lane] = mine;
        wt[(size_t)tok * k + lane] = sum > 0.f ? w / sum : 1.f / (float)k;
    }
}

// work layout (ints): cnt[n_exp] | pos[n_exp] (0 = absent, 1 = present; the scan turns
// it into the expert's position or -1) | flag (1: an id >= n_exp was seen)
__global__ __launch_bounds__(256) void k_seg_zero(int *work, int n) {
    for (int i = blockIdx.x * 256 + (int)threadIdx.x; i < n; i += (int)gridDim.x * 256)
        work[i] = 0;
}

// Summed weight of token c for expert e over its slots, in slot order from +0 (the
// reference's wsum).  Slots naming another expert add +0, which leaves the sum as it is:
// a sum started at +0 never becomes -0, and x + 0 = x otherwise (inf and NaN included).
// So every slot is loaded unconditionally and the loads issue together.
__device__ __forceinline__ float slot_wsum(const int *idx, const float *wt, int c, int topk,
                                           int e) {
    float ws = 0.f;
    for (int t = 0; t < topk; ++t) {
        const int id = idx[(size_t)c * topk + t];
        const float w = wt[(size_t)c * topk + t];
        ws += id == e ? w : 0.f;
    }
    return ws;
}

// One thread per (token, slot): the token's first slot naming an expert counts the token
// for it when the summed weight is non-zero; every named expert is present.
__global__ __launch_bounds__(256) void k_seg_count(const int *idx, const float *wt, int n_tok,
                                                   int topk, int n_exp, int *work) {
    const int i = blockIdx.x * 256 + (int)threadIdx.x;
    if (i >= n_tok * topk)
        return;
    const int c = i / topk, t = i - c * topk;
    const int e = idx[i];
    if (e < 0)
        return;
    if (e >= n_exp) {
        work[2 * n_exp] = 1;
        return;
    }
    bool first = true;
    for (int u = 0; u < t; ++u)
        first = first && idx[(size_t)c * topk + u] != e;
    if (!first)
        return;
    const float ws = slot_wsum(idx, wt, c, topk, e);
    work[n_exp + e] = 1;
    if (ws != 0.f)
        atomicAdd(work + e, 1);
}

// One workgroup of 1024: experts in ascending id.  counts = {nb, rows}, or {-1, -1} when
// cap_rows is short or an id is out of range.  The union keeps its cap_experts smallest
// ids, as the reference's union does.
__global__ __launch_bounds__(1024) void k_seg_scan(int n_exp, int *work, int cap_experts,
                                                   int cap_rows, int *eids, int *xoff, int *nr,
                                                   int *counts) {
    __shared__ int wsum_p[16], wsum_r[16];
    __shared__ int base_p, base_r;
    const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid == 0) {
        base_p = 0;
        base_r = 0;
    }
    __syncthreads();
    for (int e0 = 0; e0 < n_exp; e0 += 1024) {
        const int e = e0 + tid;
        const int p = e < n_exp ? work[n_exp + e] : 0;
        const int r = e < n_exp && p ? work[e] : 0;
        // inclusive scans within the wave
        int sp = p, sr = r;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int up = __shfl_up(sp, off), ur = __shfl_up(sr, off);
            if (lane >= off) {
                sp += up;
                sr += ur;
            }
        }
        if (lane == 63) {
            wsum_p[wave] = sp;
            wsum_r[wave] = sr;
        }
        __syncthreads();
        int bp = base_p, br = base_r;
        for (int w = 0; w < wave; ++w) {
            bp += wsum_p[w];
            br += wsum_r[w];
        }
        const int ui = bp + sp - p;  // exclusive: position among present experts
        const int ro = br + sr - r;  // rows before this expert
        if (e < n_exp) {
            const bool kept = p && ui < cap_experts;
            work[n_exp + e] = kept ? ui : -1;
            if (kept) {
                eids[ui] = e;
                xoff[ui] = ro;
                nr[ui] = r;
            }
        }
        __syncthreads();
        if (tid == 1023) {
            base_p = bp + sp;
            base_r = br + sr;
        }
        __syncthreads();
    }
    if (tid == 0) {
        // rows of the kept experts only: the dropped ones have the larger ids
        int nb = base_p < cap_experts ? base_p : cap_experts;
        int rows = 0;
        if (base_p <= cap_experts) {
            rows = base_r;
        } else {
            for (int e = 0; e < n_exp; ++e)  // truncated union (rare): count again
                if (work[n_exp + e] >= 0)
                    rows += work[e];
        }
        const bool bad = work[2 * n_exp] != 0 || rows > cap_rows;
        counts[0] = bad ? -1 : nb;
        counts[1] = bad ? -1 : rows;
    }
}

// One workgroup per expert id: the kept ones write their tokens (ascending) and sums.
// A pass covers kRowsChunks chunks of 256 tokens (token base + 256 r + thread), their
// id loads issued together, placed by one ballot per chunk and one barrier pair per
// pass.  Weights are loaded only for the slots that name the expert (loading every
// slot's weight measured 50 % slower here).
constexpr int kRowsChunks = 2;

__global__ __launch_bounds__(256) void k_seg_rows(const int *idx, const float *wt, int n_tok,
                                                  int topk, int n_exp, const int *work,
                                                  const int *xoff, const int *counts,
                                                  int *rows, float *rw) {
    __shared__ int wcnt[kRowsChunks][4];
    const int e = blockIdx.x;
    const int ui = work[n_exp + e];
    if (ui < 0 || counts[0] < 0)  // workgroup-uniform
        return;
    const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint64_t below = (1ull << lane) - 1ull;
    int j = xoff[ui];
    for (int base = 0; base < n_tok; base += 256 * kRowsChunks) {
        float ws[kRowsChunks];
        uint64_t m[kRowsChunks];
#pragma unroll
        for (int r = 0; r < kRowsChunks; ++r) {
            const int c = base + 256 * r + tid;
            ws[r] = 0.f;  // the reference's wsum: matching slots in slot order from +0
            if (c < n_tok)
                for (int t = 0; t < topk; ++t)
                    if (idx[(size_t)c * topk + t] == e)
                        ws[r] += wt[(size_t)c * topk + t];
            m[r] = __ballot(c < n_tok && ws[r] != 0.f);
            if (lane == 0)
                wcnt[r][wave] = __popcll(m[r]);
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < kRowsChunks; ++r) {
            int before = 0, total = 0;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const int v = wcnt[r][w];
                total += v;
                before += w < wave ? v : 0;
            }
            if ((m[r] >> lane) & 1u) {
                const int pos = j + before + __popcll(m[r] & below);
                rows[pos] = base + 256 * r + tid;
                rw[pos] = ws[r];
            }
            j += total;
        }
        __syncthreads();  // wcnt is rewritten by the next pass
    }
}

hipError_t launch_moe_topk(const float *choice, const float *mix, int n_tok, int n_exp, int k,
                           int *idx, float *wt, hipStream_t st) {
    if (n_tok < 1 || n_exp < 1 || n_exp > kRouteMaxExperts || k < 1 || k > 64 || k > n_exp)
        return hipErrorInvalidValue;
    const dim3 grid((unsigned)((n_tok + kTopkWaves - 1) / kTopkWaves)), block(64 * kTopkWaves);
    const int nv = (n_exp + 63) / 64;
    if (nv <= 2)
        hipLaunchKernelGGL(k_moe_topk<2>, grid, block, 0, st, choice, mix, n_tok, n_exp, k, idx, wt);
    else if (nv <= 8)
        hipLaunchKernelGGL(k_moe_topk<8>, grid, block, 0, st, choice, mix, n_tok, n_exp, k, idx, wt);
    else
        hipLaunchKernelGGL(k_moe_topk<0>, grid, block, 0, st, choice, mix, n_tok, n_exp, k, idx, wt);
    return hipGetLastError();
}

hipError_t launch_moe_segments(const int *idx, const float *wt, int n_tok, int topk, int n_exp,
                               int *work, int *eids, int *xoff, int *nr, int *rows, float *rw,
                               int cap_experts, int cap_rows, int *counts, hipStream_t st) {
    if (n_tok < 1 || topk < 1 || n_exp < 1 || cap_experts < 1 || cap_rows < 1 ||
        (long long)n_tok * topk > (1ll << 30))
        return hipErrorInvalidValue;
    const int nw = 2 * n_exp + 1;
    hipLaunchKernelGGL(k_seg_zero, dim3((unsigned)std::min((nw + 255) / 256, 1024)), dim3(256), 0,
                       st, work, nw);
    const int pairs = n_tok * topk;
    hipLaunchKernelGGL(k_seg_count, dim3((unsigned)((pairs + 255) / 256)), dim3(256), 0, st, idx,
                       wt, n_tok, topk, n_exp, work);
    hipLaunchKernelGGL(k_seg_scan, dim3(1), dim3(1024), 0, st, n_exp, work, cap_experts, cap_rows,
                       eids, xoff, nr, counts);
    hipLaunchKernelGGL(k_seg_rows, dim3((unsigned)n_exp), dim3(256), 0, st, idx, wt, n_tok, topk,
                       n_exp, work, xoff, counts, rows, rw);
    return hipGetLastError();
}

hipError_t launch_moe_route(const float *choice, const float *mix, int n_tok, int n_exp, int k,
                            int *idx, float *wt, int *work, int *eids, int *xoff, int *nr,
                            int *rows, float *rw, int cap_experts, int cap_rows, int *counts,
                            hipStream_t st) {
    hipError_t e = launch_moe_topk(choice, mix, n_tok, n_exp, k, idx, wt, st);
    if (e != hipSuccess)
        return e;
    return launch_moe_segments(idx, wt, n_tok, k, n_exp, work, eids, xoff, nr, rows, rw,
                               cap_experts, cap_rows, counts, st);
}

}  // namespace mvllm_hip
