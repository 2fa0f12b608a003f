// kern_mfma.hip -- expert GEMMs on the gfx950 matrix cores (v_mfma_f32_16x16x32_bf16).
//
// Both moe_block projections, H = act(X Wg^T, X Wu^T) and Y = H Wd^T, run as
// C[token, o] = sum_k A[token, k] * B[k, o] with A = activations (16 tokens per tile),
// B = quantized weights decoded in registers (16 output rows per tile):
//   fmt 4 (int4-g64): byte n -> v_cvt_scalef32_pk_bf16_fp8(scale 2^9) -> bf16(n) exactly
//                     (an e4m3 byte 0..15 is n * 2^-9); each 64-wide group is its own MFMA
//                     chain C_g, then acc += s * (C_g - 8 * sum_k A[., k]) in f32, which is
//                     sum_k A * (n - 8) * s with the reference's f32 scale.
//   fmt 7 (MXFP4):    v_cvt_scalef32_pk_bf16_fp4 with the ue8m0 scale 2^(e-127) passed as
//                     an f32 gives bf16(lut[n] * scale) -- exact (a power-of-two scaling of
//                     a 2-bit mantissa); the chain accumulates straight into acc.
// Activations are split into TERMS bf16 terms (x = hi + mid + lo for TERMS = 3): every
// product with a decoded weight is then exact in f32 and the result differs from the
// f32 reference only by summation order.  TERMS = 1 is plain bf16 activations.
//
// MFMA 16x16x32 operand layout (lane l = 0..63, t = l % 16, q = l / 16): A row t and B
// column t take K elements [8q, 8q+8) of the 32-wide step; C[4q + i][t], i = 0..3.
// Within a 64-wide group, step s in {0,1} takes K offsets 16q + 8s .. +8, so a lane's
// 16 weights of the group are 8 contiguous bytes and one scale serves the whole chain.
#include "mfma_common.h"

#include <algorithm>
#include <cmath>

namespace mvllm_hip {


// ---------------------------------------------------------------------------------
// Activation planes.  A GEMM input row is held as TERMS bf16 planes P[tm][j][K] (fmt 4:
// each 8-block in slot order, see a_slot) plus, for fmt 4, the per-64 sums of what the
// terms represent (the -8 correction).  The gate/up kernel builds them in LDS from the
// f32 input rows; its epilogue writes H in this form to HBM for the down kernel, the
// per-64 sums as four per-16-column partials hp[g][p][j], p = 0..3, summed in that
// order by the reader.
// ---------------------------------------------------------------------------------

// ---------------------------------------------------------------------------------
// Decode-shaped GEMM.  A workgroup of kDecWaves waves serves one item (up to rmax rows of
// one expert).  Each wave computes TPW 16-row output tiles of one weight matrix over one of
// KS equal K ranges: wave w -> tile slot w % TW, matrix (w / TW) % MS, K range
// w / (TW * MS), with MS = 2 matrices (gate, up) for the dual projection and
// TW = kDecWaves / (KS * MS) tile slots per workgroup.
//
// Memory access.  The weights of a 256-wide K block of a tile (16 rows x 128 bytes) are
// read with coalesced 8-byte loads -- lane l takes row l / 4, bytes 8 (l % 4) + 32 g of
// load g -- and moved into the matrix-core layout (lane 16 q + t holds row t, bytes
// 8 q + 32 g) with ds_bpermute.  A tile's scales over the wave's K range are read once,
// coalesced, into wave-private LDS.  The item's activations are copied into LDS once for
// all waves (the dual projection splits the f32 rows into bf16 terms on the way);
// those loads are issued before any weight load (vector loads complete in order).  NB
// blocks per wave stay in flight.  Partial tiles are combined through LDS in fixed order.
// ---------------------------------------------------------------------------------

struct DecItem {
    int a;     // expert index into ExpertWork
    int r0;    // first row (within the expert's compact rows)
    int nrow;  // rows in this item (<= rmax)
    int pad;
};

struct DecArgs {
    const ExpertWork *ew;
    const DecItem *items;
    const float *xin;     // dual: f32 input rows (row of compact row j: in_rows[j] or j)
    const int *in_rows;   // dual: compact row -> input row (null = identity)
    const __bf16 *pin;    // single: input planes [TERMS][rcap][K]
    const float *xs;      // single, fmt 4: H partial sums [K/64][4][rcap]
    __bf16 *pout;         // dual: H planes [TERMS][rcap][O]
    float *hp;            // dual, fmt 4: H partial sums [O/64][4][rcap]
    float *out;           // single: Y [rcap][O] f32, or the caller's out [S][O] when dest
    const int *dest;      // single, optional: compact row -> row of out; the epilogue then
    const float *wrow;    // adds wrow[j] * y into out (float atomics) instead of writing Y
    int wgs;              // workgroups per item = O / (16 * TW * TPW)
    int K, O, rcap, rmax;
    int act;
    float act_a, act_b;
};

#ifndef MVLLM_DEC_NB_EXTRA
#define MVLLM_DEC_NB_EXTRA 0  // extra weight blocks in flight per wave (tuning)
#endif


constexpr int kScaleDw = 8;  // scale dwords per lane and tile (<= 128 scale bytes per row)


// Weights of one 256-wide K block of a tile, as loaded (lane l: row l / 4).
struct WBlock {
    u32x2 w[4];
};

__device__ __forceinline__ void load_block(WBlock &b, __amdgpu_buffer_rsrc_t rw, uint32_t voff,
                                           uint32_t soff) {
#pragma unroll
    for (int g = 0; g < 4; ++g)
        b.w[g] = __builtin_bit_cast(
            u32x2, __builtin_amdgcn_raw_buffer_load_b64(rw, voff + 32 * g, soff, 0));
}

// One block through the matrix cores.  A rows live in LDS as [rmax][K/8][TERMS][8] bf16
// (a row's terms of each 8-block side by side; tb = this lane's row t at the block's
// first 8-block plus 2 q; `a` holds zeros for rows t >= nrow); fmt 4 keeps
// -8 * the per-64 sums of each row as [K/64][16] f32; the tile's scales sit in
// wave-private LDS (ls = row t's bytes over the wave's K range; gb = first group of the
// block within that range).
template <int FMT, int TERMS>
__device__ __forceinline__ void compute_block(f4v &acc, bf16x8 (&a)[TERMS][2], const WBlock &b,
                                              const char *tb, int t, int nrow, const float *lxs,
                                              const uint8_t *ls, int kb, int gb, int q,
                                              int src4) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const int kg = kb + 64 * g;
        // Only the lanes of live rows (t < nrow) read LDS: its bandwidth is shared by the
        // waves and scales with the active lanes.  `a` is carried across groups and
        // blocks, so the rows past nrow keep the zeros they started with.  The row count
        // goes through an empty asm per group so that the compiler keeps one small masked
        // region per group instead of merging them (register pressure).
        int nr = nrow;
        asm volatile("" : "+v"(nr));
        if (t < nr) {
#pragma unroll
            for (int tm = 0; tm < TERMS; ++tm)
#pragma unroll
                for (int s = 0; s < 2; ++s)
                    a[tm][s] = *reinterpret_cast<const bf16x8 *>(
                        tb + (8 * g + s) * TERMS * 16 + tm * 16);
        }
        // row t's 8 bytes of this group: held by lane 4 t + q of the coalesced load
        const uint32_t wx = (uint32_t)__builtin_amdgcn_ds_bpermute(src4, (int)b.w[g].x);
        const uint32_t wy = (uint32_t)__builtin_amdgcn_ds_bpermute(src4, (int)b.w[g].y);
        float sg;
        if constexpr (FMT == 4) {
            sg = *reinterpret_cast<const float *>(ls + 4 * (gb + g));
        } else {  // lanes q < 2 take 32-block 2 g, q >= 2 block 2 g + 1
            sg = __uint_as_float((uint32_t)ls[2 * (gb + g) + (q >> 1)] << 23);
        }
        bf16x8 B0 = decode_b<FMT>(wx, sg);
        bf16x8 B1 = decode_b<FMT>(wy, sg);
        if constexpr (FMT == 7) {
            // rare exceptional scale bytes: a wave-uniform branch keeps the exact decode
            // out of the common path
            const bool exc = b7_exceptional(sg);
            if (__builtin_expect(__builtin_amdgcn_ballot_w64(exc) != 0, 0)) {
                if (exc) {
                    B0 = decode_b7_exact(wx, sg);
                    B1 = decode_b7_exact(wy, sg);
                }
            }
        }
        if constexpr (FMT == 4) {
            // the chain starts from -8 * (sum of the group's activations) of each row, so
            // it ends at sum_k a_k (n_k - 8); one scale per (row, group) then applies
            f4v c = *reinterpret_cast<const f4v *>(lxs + (kg >> 6) * 16 + 4 * q);
#pragma unroll
            for (int tm = 0; tm < TERMS; ++tm) {
                c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[tm][0], B0, c, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[tm][1], B1, c, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
                acc[i] = fmaf(sg, c[i], acc[i]);
            // materialise acc here: otherwise the chain is sunk past the masked regions
            // and every group's C and sums stay live to the end of the block
            asm volatile("" : "+v"(acc));
        } else {
#pragma unroll
            for (int tm = 0; tm < TERMS; ++tm) {
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[tm][0], B0, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[tm][1], B1, acc, 0, 0, 0);
            }
        }
        // keep the next group's LDS reads from being hoisted over this one (register
        // pressure: two workgroups share a CU, so each wave has 128 VGPRs)
        __builtin_amdgcn_sched_barrier(0);
    }
}

// LDS layout of the decode kernel: A rows [rmax][K/8][terms][8] bf16 (+ 16 bytes per
// row), fmt 4 sums [K/64][16] f32, then the wave-private scales [waves][tpw][16][rbw];
// the combine buffer [waves][tpw][4][64] f32 reuses the start.  Returns the total bytes.
__host__ __device__ inline int dec_row_bytes(int K, int terms) {
    return K * terms * 2 + 16;  // + 16: consecutive rows start in different LDS banks
}

__host__ __device__ inline size_t dec_lds_plan(int fmt, int K, int rmax, int terms, bool dual,
                                               int ks, int tpw, size_t *off_xs, size_t *off_sc) {
    const size_t planes = (size_t)rmax * dec_row_bytes(K, terms);
    const size_t xs = fmt == 4 ? (size_t)(K / 64) * 16 * 4 : 0;
    const size_t rbw = (size_t)(K / ks) / (fmt == 4 ? 16 : 32);  // scale bytes per tile row
    const size_t sc = (size_t)kDecWaves * tpw * 16 * rbw;
    const size_t red = (ks > 1 || dual) ? (size_t)kDecWaves * tpw * 4 * 64 * 4 : 0;
    if (off_xs)
        *off_xs = planes;
    if (off_sc)
        *off_sc = planes + xs;
    const size_t tot = planes + xs + sc;
    return tot > red ? tot : red;
}

template <int FMT, bool DUAL, int TERMS, int KS, int TPW, int SR>
__global__ __launch_bounds__(kDecThreads) __attribute__((amdgpu_waves_per_eu(4)))
void k_mfma_dec(DecArgs A) {
    constexpr int MS = DUAL ? 2 : 1;
    constexpr int TW = kDecWaves / (KS * MS);  // tile slots per workgroup
    constexpr int NB = ((TERMS == 1 && TPW == 1) ? 4 : 3) + MVLLM_DEC_NB_EXTRA;  // blocks in flight (VGPR budget)
    constexpr int XSR = 2;              // single, fmt 4: sums per thread (K / 4 <= 2048)
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const int item = blockIdx.x / A.wgs;
    const int wg = blockIdx.x - item * A.wgs;
    const DecItem it = A.items[item];
    const ExpertWork &ew = A.ew[it.a];
    const int K = A.K, O = A.O, nrow = it.nrow;
    const int jbase = ew.row0 + it.r0;
    // wave index as a scalar: tiles, matrix and K range are then wave-uniform (SGPRs)
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const int t = lane & 15, q = lane >> 4;
    const int tl = wave % TW, mat = (wave / TW) % MS, ks = wave / (TW * MS);
    const int tile0 = wg * TW * TPW + tl;  // this wave's tiles: tile0 + r * TW, r < TPW
    const int ngs = FMT == 4 ? K / 64 : K / 32;
    const uint32_t rowb = (uint32_t)(K >> 1);
    const uint32_t srow = (uint32_t)ngs * (FMT == 4 ? 4u : 1u);  // scale bytes per row
    const int mi = DUAL ? mat : 2;
    const __amdgpu_buffer_rsrc_t rw = buf_rsrc(ew.w[mi], (uint32_t)O * rowb);
    const __amdgpu_buffer_rsrc_t rs = buf_rsrc(ew.s[mi], (uint32_t)O * srow);
    const int Kr = K / KS, kw0 = ks * Kr;
    const int nblk = Kr >> 8;
    const int nbt = TPW * nblk;            // blocks of this wave over all its tiles
    const int rbw = Kr / (FMT == 4 ? 16 : 32);  // scale bytes per tile row (<= 128)
    const int rsb = dec_row_bytes(K, TERMS);  // bytes per A row in LDS
    size_t off_xs = 0, off_sc = 0;
    dec_lds_plan(FMT, K, A.rmax, TERMS, DUAL, KS, TPW, &off_xs, &off_sc);
    __bf16 *lp = reinterpret_cast<__bf16 *>(smem);
    float *lxs = reinterpret_cast<float *>(smem + off_xs);  // [K/64][16]
    uint8_t *lsc = reinterpret_cast<uint8_t *>(smem + off_sc) +
                   (size_t)wave * TPW * 16 * rbw;           // this wave's [TPW][16][rbw]
    float *red = reinterpret_cast<float *>(smem);  // [waves][TPW][4][64], reuses the planes

    // coalesced weight loads: lane l -> row l / 4 of the tile, bytes 8 (l % 4) (+ 32 g)
    const uint32_t voff_w =
        (uint32_t)(tile0 * 16 + (lane >> 2)) * rowb + 8u * (uint32_t)(lane & 3);
    const uint32_t tstep_w = (uint32_t)(TW * 16) * rowb;
    auto soff_i = [&](int i) {  // block i: tile r = i / nblk, K offset kw0 + 256 (i % nblk)
        const bool hi = TPW > 1 && i >= nblk;
        return (uint32_t)((kw0 + 256 * (hi ? i - nblk : i)) >> 1) + (hi ? tstep_w : 0u);
    };

    // 1) activation loads of this thread (issued first; unconditional loads, clamped to
    // valid addresses, keep the arrays in registers) ...
    const int per_row = K >> 3;  // 8-element chunks per row
    const int total = DUAL ? nrow * per_row : TERMS * nrow * per_row;
    float4 xv[DUAL ? SR : 1][2];
    uint4 st[DUAL ? 1 : SR];
    float xsr[XSR];
    if constexpr (DUAL) {
#pragma unroll
        for (int u = 0; u < SR; ++u) {
            const int idx0 = u * kDecThreads + (int)threadIdx.x;
            const int idx = idx0 < total ? idx0 : 0;
            const int r = idx / per_row, c = idx - r * per_row;
            const int j = jbase + r;
            const int src = A.in_rows ? A.in_rows[j] : j;
            const float4 *p = reinterpret_cast<const float4 *>(A.xin + (size_t)src * K + 8 * c);
            xv[u][0] = p[0];
            xv[u][1] = p[1];
        }
    } else {
#pragma unroll
        for (int u = 0; u < SR; ++u) {
            const int idx0 = u * kDecThreads + (int)threadIdx.x;
            const int idx = idx0 < total ? idx0 : 0;
            const int row = idx / per_row, c = idx - row * per_row;  // row = tm * nrow + r
            const int tm = row / nrow, r = row - tm * nrow;
            st[u] = reinterpret_cast<const uint4 *>(A.pin + ((size_t)tm * A.rcap + jbase + r) *
                                                                (size_t)K)[c];
        }
        if constexpr (FMT == 4) {
#pragma unroll
            for (int u = 0; u < XSR; ++u) {
                const int i = u * kDecThreads + (int)threadIdx.x;
                const int g = i >> 4, r = i & 15;
                const bool ok = i < (K >> 2) && r < nrow;
                const float *pp =
                    A.xs + (size_t)(ok ? g : 0) * 4 * A.rcap + jbase + (ok ? r : 0);
                const float v = ((pp[0] + pp[A.rcap]) + pp[2 * A.rcap]) + pp[3 * A.rcap];
                xsr[u] = ok ? v : 0.f;
            }
        }
    }
    // 2) ... the scales of this wave's tiles (coalesced dwords: dword p of a tile's
    // [16][rbw] block is row p / (rbw / 4), dword p % (rbw / 4)) ...
    const int dpr = rbw >> 2;  // dwords per tile row
    const int ndw = 16 * dpr;  // dwords per tile
    uint32_t scv[TPW][kScaleDw];
#pragma unroll
    for (int r = 0; r < TPW; ++r)
#pragma unroll
        for (int d = 0; d < kScaleDw; ++d) {
            const int p0 = d * 64 + lane;
            const int pp = p0 < ndw ? p0 : 0;
            const int row = pp / dpr, col = pp - row * dpr;
            const uint32_t off = (uint32_t)((tile0 + r * TW) * 16 + row) * srow +
                                 (uint32_t)(kw0 / (FMT == 4 ? 16 : 32) + 4 * col);
            scv[r][d] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0);
        }
    // 3) ... then the first weight blocks of this wave
    WBlock b[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u)
        if (u < nbt)
            load_block(b[u], rw, voff_w, soff_i(u));
    // 4) activations, sums and scales into LDS
    if constexpr (DUAL) {
#pragma unroll
        for (int u = 0; u < SR; ++u) {
            const int idx = u * kDecThreads + (int)threadIdx.x;
            const bool ok = idx < total;
            const int r = ok ? idx / per_row : 0, c = ok ? idx - r * per_row : 0;
            const float v[8] = {xv[u][0].x, xv[u][0].y, xv[u][0].z, xv[u][0].w,
                                xv[u][1].x, xv[u][1].y, xv[u][1].z, xv[u][1].w};
            bf16x8 o[3];
            float rs8 = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                __bf16 tt[3];
                rs8 += split_terms<TERMS>(v[e], tt);
#pragma unroll
                for (int tm = 0; tm < TERMS; ++tm)
                    o[tm][a_slot<FMT>(e)] = tt[tm];
            }
            if (ok) {
                char *dst = reinterpret_cast<char *>(lp) + (size_t)r * rsb + (size_t)c * TERMS * 16;
#pragma unroll
                for (int tm = 0; tm < TERMS; ++tm)
                    *reinterpret_cast<bf16x8 *>(dst + tm * 16) = o[tm];
            }
            if constexpr (FMT == 4) {
                // per-64 sums of what the terms represent: 8 consecutive threads hold one
                // group of one row (per_row and kDecThreads are multiples of 8)
                rs8 += __shfl_xor(rs8, 1, 8);
                rs8 += __shfl_xor(rs8, 2, 8);
                rs8 += __shfl_xor(rs8, 4, 8);
                if (ok && (c & 7) == 0)
                    lxs[(c >> 3) * 16 + r] = -8.f * rs8;
            }
        }
        if constexpr (FMT == 4) {  // rows nrow..15 of the sums read as 0
            for (int i = threadIdx.x; i < (K / 64) * 16; i += kDecThreads)
                if ((i & 15) >= nrow)
                    lxs[i] = 0.f;
        }
    } else {
#pragma unroll
        for (int u = 0; u < SR; ++u) {
            const int idx = u * kDecThreads + (int)threadIdx.x;
            if (idx < total) {
                const int row = idx / per_row, c = idx - row * per_row;
                const int tm = row / nrow, r = row - tm * nrow;
                *reinterpret_cast<uint4 *>(reinterpret_cast<char *>(lp) + (size_t)r * rsb +
                                           (size_t)c * TERMS * 16 + tm * 16) = st[u];
            }
        }
        if constexpr (FMT == 4) {
#pragma unroll
            for (int u = 0; u < XSR; ++u) {
                const int i = u * kDecThreads + (int)threadIdx.x;
                if (i < (K >> 2))
                    lxs[i] = -8.f * xsr[u];
            }
        }
    }
#pragma unroll
    for (int r = 0; r < TPW; ++r)
#pragma unroll
        for (int d = 0; d < kScaleDw; ++d) {
            const int p = d * 64 + lane;
            if (p < ndw)
                reinterpret_cast<uint32_t *>(lsc + (size_t)r * 16 * rbw)[p] = scv[r][d];
        }
    __syncthreads();

    // 5) MFMA over this wave's blocks with NB in flight: b[u] holds block i0 + u; the
    // steady-state loop reloads each slot right after consuming it.  Tile 0's result
    // moves to res[0] when its last block is done (TPW = 2).
    f4v acc = {0.f, 0.f, 0.f, 0.f};
    f4v res[TPW];
    const char *ta = reinterpret_cast<const char *>(lp) + (size_t)(t < nrow ? t : 0) * rsb +
                     (size_t)(2 * q) * TERMS * 16;
    const int src4 = 4 * (4 * t + q);  // ds_bpermute byte address of lane 4 t + q
    bf16x8 a[TERMS][2] = {};           // A fragments; stay zero in rows t >= nrow
    auto consume = [&](const WBlock &bb, int i) {
        const bool hi = TPW > 1 && i >= nblk;
        const int kl = hi ? i - nblk : i;  // block within the tile's K range
        const uint8_t *ls = lsc + (size_t)((hi ? 16 : 0) + t) * rbw;
        const int kb = kw0 + 256 * kl;
        compute_block<FMT, TERMS>(acc, a, bb, ta + (size_t)(kb >> 3) * TERMS * 16, t, nrow, lxs,
                                  ls, kb, 4 * kl, q, src4);
        if constexpr (TPW > 1) {
            if (i == nblk - 1) {
                res[0] = acc;
                acc = f4v{0.f, 0.f, 0.f, 0.f};
            }
        }
    };
    int i0 = 0;
    for (; i0 + 2 * NB <= nbt; i0 += NB) {
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            consume(b[u], i0 + u);
            load_block(b[u], rw, voff_w, soff_i(i0 + u + NB));
        }
    }
#pragma unroll
    for (int u = 0; u < NB; ++u) {
        if (i0 + u < nbt) {
            consume(b[u], i0 + u);
            if (i0 + u + NB < nbt)
                load_block(b[u], rw, voff_w, soff_i(i0 + u + NB));
        }
    }
#pragma unroll
    for (int u = 0; u < NB; ++u)
        if (i0 + NB + u < nbt)
            consume(b[u], i0 + NB + u);
    res[TPW - 1] = acc;

    // 6) combine: sum the K ranges of each (matrix, tile) in fixed order; the waves of
    // matrix 0, range 0 finish their tiles
    f4v fin[TPW][MS];
#pragma unroll
    for (int r = 0; r < TPW; ++r)
        fin[r][0] = res[r];
    if constexpr (KS * MS > 1) {
        __syncthreads();  // every wave is done reading the planes that `red` overwrites
#pragma unroll
        for (int r = 0; r < TPW; ++r)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                red[((wave * TPW + r) * 4 + i) * 64 + lane] = res[r][i];
        __syncthreads();
        if (ks != 0 || mat != 0)
            return;
#pragma unroll
        for (int r = 0; r < TPW; ++r)
#pragma unroll
            for (int m = 0; m < MS; ++m)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float sm = red[(((m * TW + tl) * TPW + r) * 4 + i) * 64 + lane];
#pragma unroll
                    for (int k2 = 1; k2 < KS; ++k2)
                        sm += red[((((k2 * MS + m) * TW + tl) * TPW + r) * 4 + i) * 64 + lane];
                    fin[r][m][i] = sm;
                }
    }
#pragma unroll
    for (int r = 0; r < TPW; ++r) {
        const int tile = tile0 + r * TW;
        const int o = tile * 16 + t;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int tok = 4 * q + i;  // C row of this lane
            const int j = jbase + tok;
            if constexpr (DUAL) {
                // H = act(gate, up) -> planes of the down projection (+ 16-column partials)
                const float h = mf_act(A.act, fin[r][0][i], fin[r][MS - 1][i], A.act_a, A.act_b);
                __bf16 tt[3];
                float rep = split_terms<TERMS>(h, tt);
                if (tok < nrow) {
                    const int pos = (o & ~7) + a_slot<FMT>(o & 7);
#pragma unroll
                    for (int tm = 0; tm < TERMS; ++tm)
                        A.pout[((size_t)tm * A.rcap + j) * O + pos] = tt[tm];
                }
                if constexpr (FMT == 4) {
                    rep += __shfl_xor(rep, 1, 16);
                    rep += __shfl_xor(rep, 2, 16);
                    rep += __shfl_xor(rep, 4, 16);
                    rep += __shfl_xor(rep, 8, 16);
                    if (t == 0 && tok < nrow)
                        A.hp[((size_t)(tile >> 2) * 4 + (tile & 3)) * A.rcap + j] = rep;
                }
            } else {
                if (tok < nrow) {
                    if (A.dest)  // top-k combine folded in: out[dest] += w * y
                        unsafeAtomicAdd(A.out + (size_t)A.dest[j] * O + o,
                                        __fmul_rn(A.wrow[j], fin[r][0][i]));
                    else
                        A.out[(size_t)j * O + o] = fin[r][0][i];
                }
            }
        }
    }
}

size_t mfma_dec_lds_bytes(int fmt, int K, int rmax, int terms, int dual, int ks, int tpw) {
    return dec_lds_plan(fmt, K, rmax, terms, dual != 0, ks, tpw, nullptr, nullptr);
}

template <int FMT, bool DUAL, int TERMS, int KS, int TPW>
static hipError_t launch_dec_t(DecArgs a, int n_items, hipStream_t st) {
    const size_t lds = mfma_dec_lds_bytes(FMT, a.K, a.rmax, TERMS, DUAL, KS, TPW);
    a.wgs = a.O / (16 * TPW * (kDecWaves / (KS * (DUAL ? 2 : 1))));
    const dim3 grid((unsigned)(n_items * a.wgs)), block(kDecThreads);
    // staging registers per thread: dual = 8-float chunks of rmax rows, single = uint4 of
    // TERMS planes of rmax rows
    const size_t need = DUAL ? (size_t)a.rmax * (a.K / 8) : (size_t)TERMS * a.rmax * (a.K / 8);
    const int sr = (int)((need + kDecThreads - 1) / kDecThreads);
    auto go = [&](auto kern) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e == hipSuccess)
            hipLaunchKernelGGL(kern, grid, block, lds, st, a);
        return e;
    };
    hipError_t e;
    if (DUAL ? sr <= 2 : sr <= 4)
        e = go(k_mfma_dec<FMT, DUAL, TERMS, KS, TPW, DUAL ? 2 : 4>);
    else if (DUAL ? sr <= kDecStageDual : sr <= kDecStageSingle)
        e = go(k_mfma_dec<FMT, DUAL, TERMS, KS, TPW, DUAL ? kDecStageDual : kDecStageSingle>);
    else
        return hipErrorInvalidValue;
    if (e != hipSuccess)
        return e;
    return hipGetLastError();
}

template <int FMT, bool DUAL>
static hipError_t launch_dec_fd(const DecArgs &a, int n_items, int terms, int ks, int tpw,
                                hipStream_t st) {
#define MVLLM_DEC_T(TM)                                                                      \
    return tpw == 2    ? launch_dec_t<FMT, DUAL, TM, 1, 2>(a, n_items, st)                   \
           : ks == 4   ? launch_dec_t<FMT, DUAL, TM, 4, 1>(a, n_items, st)                   \
           : ks == 2   ? launch_dec_t<FMT, DUAL, TM, 2, 1>(a, n_items, st)                   \
                       : launch_dec_t<FMT, DUAL, TM, 1, 1>(a, n_items, st)
    if (terms <= 1) {
        MVLLM_DEC_T(1);
    }
    if (terms == 2) {
        MVLLM_DEC_T(2);
    }
    MVLLM_DEC_T(3);
#undef MVLLM_DEC_T
}

hipError_t launch_mfma_dec(int fmt, bool dual, int terms, int ks, int tpw, const ExpertWork *ew,
                           const void *items, int n_items, const float *xin, const int *in_rows,
                           const void *pin, const float *xs, void *pout, float *hp, float *out,
                           int K, int O, int rcap, int rmax, int act, float act_a, float act_b,
                           hipStream_t st, const int *dest, const float *wrow) {
    if (n_items <= 0)
        return hipSuccess;
    if ((tpw == 2 && ks != 1) || (tpw != 1 && tpw != 2) || K > kDecMaxK ||
        K / ks / (fmt == 4 ? 16 : 32) > 4 * kScaleDw * 64 / 16)
        return hipErrorInvalidValue;
    DecArgs a{};
    a.ew = ew;
    a.items = static_cast<const DecItem *>(items);
    a.xin = xin;
    a.in_rows = in_rows;
    a.pin = static_cast<const __bf16 *>(pin);
    a.xs = xs;
    a.pout = static_cast<__bf16 *>(pout);
    a.hp = hp;
    a.out = out;
    a.dest = dest;
    a.wrow = wrow;
    a.K = K;
    a.O = O;
    a.rcap = rcap;
    a.rmax = rmax;
    a.act = act;
    a.act_a = act_a;
    a.act_b = act_b;
    if (fmt == 4)
        return dual ? launch_dec_fd<4, true>(a, n_items, terms, ks, tpw, st)
                    : launch_dec_fd<4, false>(a, n_items, terms, ks, tpw, st);
    if (fmt == 7)
        return dual ? launch_dec_fd<7, true>(a, n_items, terms, ks, tpw, st)
                    : launch_dec_fd<7, false>(a, n_items, terms, ks, tpw, st);
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
