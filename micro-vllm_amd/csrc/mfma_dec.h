// mfma_dec.h -- the decode-shaped matrix-core task of the decode kernels (kern_mfma.hip).
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
#pragma once

#include "mfma_common.h"

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
// one expert).  Wave w streams NT tiles of 16 output rows over one of KS equal K ranges:
// slot w % TW, K range w / TW (TW = kDecWaves / KS).  Dual: the two tiles are the gate
// and the up rows of the same 16 columns (column tile wg * TW + slot), so the activation
// is applied in registers; single: tiles wg * TW * NT + slot + n * TW.  The tiles advance
// together one 256-wide K block at a time and share the activation fragments.
//
// Memory access.  The weights of a 256-wide K block of a tile (16 rows x 128 bytes) come
// in through coalesced 8-byte loads -- lane l takes row l / 4, bytes 8 (l % 4) + 32 g of
// load g -- and move into the matrix-core layout (lane 16 q + t holds row t, bytes
// 8 q + 32 g) with ds_bpermute.  A tile's scales over the wave's K range are loaded once
// (load_scales) and handed out per group by ds_bpermute.  The item's
// activations are copied into LDS once for all waves (dual: split into bf16 terms on
// the way).  Their loads are issued first, then the weight loads (vector loads complete
// in order), both right after the one descriptor read they depend on.  NU K blocks per
// tile stay in flight.  Partial sums of K ranges meet in LDS in fixed order.
// ---------------------------------------------------------------------------------

struct DecArgs {
    const DecDesc *desc;
    const float *xin;     // dual: f32 input rows [*][K]
    const __bf16 *pin;    // single: input planes [TERMS][rcap][K]
    const float *xs;      // single, fmt 4: input partial sums [K/64][4][rcap]
    __bf16 *pout;         // dual: H planes [TERMS][rcap][O]
    float *hp;            // dual, fmt 4: H partial sums [O/64][4][rcap]
    float *out;           // single: Y [rcap][O] f32, or the caller's out [S][O] with fold
    int fold;             // single: add wts[r] * y into out[rows[r]] (float atomics); rows
                          // with rows[r] < 0 are skipped
    // dual: workgroups [0, n_cp) copy descriptor i of cp_src (the down launch's, in host
    // memory) to cp_dst (device memory): the down kernel then starts from an HBM/L2 read
    // instead of a PCIe round trip (measured 20.6 -> 18.4 us at c1 T=16)
    const DecDesc *cp_src;
    DecDesc *cp_dst;
    int n_cp;
    int pack;  // every item has <= 8 rows and TERMS == 2: the packed kernel is launched
    // item count in device memory (a device planner's), or null: the grid then covers a
    // capacity of items and the workgroups of items at or past the count return at once
    const int *n_items_dev;
    int wgs;              // workgroups per item
    int K, O, rcap, rmax;
    int act;
    float act_a, act_b;
};

// One 256-wide K block of one tile as loaded: lane l holds row l / 4's weight bytes
// 8 (l % 4) + 32 g, g = 0..3.
template <int FMT> struct DBlock {
    u32x2 w[4];
};

template <int FMT>
__device__ __forceinline__ void load_dblock(DBlock<FMT> &b, __amdgpu_buffer_rsrc_t rw,
                                            uint32_t vw, int kb) {
    const uint32_t sw = (uint32_t)(kb >> 1);
#pragma unroll
    for (int g = 0; g < 4; ++g)
        b.w[g] = __builtin_bit_cast(
            u32x2, __builtin_amdgcn_raw_buffer_load_b64(rw, vw + 32 * g, sw, 0));
}

// A tile's scales over the wave's whole K range, loaded once: lane (t, q) holds bytes
// [32 q, 32 q + 32) of row t's scales from the range's start (int4: f32 groups 8 q ..
// 8 q + 7; MXFP4: ue8m0 bytes of 32-blocks 32 q .. 32 q + 31).  128 bytes a row, hence
// K / ks <= dec_max_kr.  Reading them per K block instead re-fetched each row's scale
// line from HBM whenever the L2 had dropped it in between.

template <int FMT>
__device__ __forceinline__ void load_scales(u32x4 (&sc)[2], __amdgpu_buffer_rsrc_t rs,
                                            uint32_t vs) {
    if constexpr (FMT == 4) {  // 16-byte aligned: rows of K / 16 bytes, ranges of 16 * nblk
        sc[0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, vs, 0, 0));
        sc[1] = __builtin_bit_cast(u32x4,
                                   __builtin_amdgcn_raw_buffer_load_b128(rs, vs + 16, 0, 0));
    } else {  // 8-byte aligned: rows of K / 32 bytes, ranges of 8 * nblk
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const u32x2 lo = __builtin_bit_cast(
                u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs, vs + 16 * h, 0, 0));
            const u32x2 hi = __builtin_bit_cast(
                u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs, vs + 16 * h + 8, 0, 0));
            sc[h] = u32x4{lo.x, lo.y, hi.x, hi.y};
        }
    }
}

// One K block of NT tiles through the matrix cores.  A rows live in LDS as
// [rmax][K/8][TERMS][8] bf16 (a row's terms of each 8-block side by side; tb = this
// lane's row t at the block's first 8-block plus 2 q; `a` holds zeros for rows
// t >= nrow); fmt 4 keeps -8 * the per-64 sums of each row as [K/64][16] f32.
// EXACT is the redo of a wave's tiles whose operands the common path does not reproduce
// (see dec_needs_exact): it decodes per element, MXFP4 through decode_b7_exact, int4 as
// n - 8 with chains from 0 and a non-finite scale inside each product.
// PACK (two terms, items of <= 8 rows): A row t holds term t / 8 of row t % 8, so one
// MFMA takes both terms (tb already points at this lane's term) and C rows r and r + 8
// are added after the loop: half the matrix-core work and A reads per block.
template <int FMT, int TERMS, int NT, bool EXACT, bool PACK = false>
__device__ __forceinline__ void compute_dblock(f4v (&acc)[NT], bf16x8 (&a)[PACK ? 1 : TERMS][2],
                                               const DBlock<FMT> (&b)[NT],
                                               const u32x4 (&sc)[NT][2], int kl, const char *tb,
                                               int t, int nrow, const float *lxs, int kb, int q,
                                               int src4) {
    // this block's scale words sit in lane (t, kl / 2) (int4) or (t, kl / 4) (MXFP4)
    const int ssrc = 4 * (t + 16 * (FMT == 4 ? (kl >> 1) : (kl >> 2)));
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        // Only the lanes of live rows (t < nrow) read LDS: its bandwidth is shared by the
        // waves and scales with the active lanes.  `a` is carried across groups and
        // blocks, so the rows past nrow keep the zeros they started with.  The row count
        // goes through an empty asm per group so that the compiler keeps one small masked
        // region per group instead of merging them (register pressure).
        int nr = nrow;
        asm volatile("" : "+v"(nr));
        if ((PACK ? (t & 7) : t) < nr) {
#pragma unroll
            for (int tm = 0; tm < (PACK ? 1 : TERMS); ++tm)
#pragma unroll
                for (int s = 0; s < 2; ++s)
                    a[tm][s] = *reinterpret_cast<const bf16x8 *>(
                        tb + (8 * g + s) * TERMS * 16 + tm * 16);
        }
        f4v c0 = {0.f, 0.f, 0.f, 0.f};
        if constexpr (FMT == 4 && !EXACT)
            c0 = *reinterpret_cast<const f4v *>(lxs + ((kb >> 6) + g) * 16 + 4 * q);
#pragma unroll
        for (int n = 0; n < NT; ++n) {
            // row t's 8 bytes of this group: held by lane 4 t + q of the coalesced load
            const uint32_t wx = (uint32_t)__builtin_amdgcn_ds_bpermute(src4, (int)b[n].w[g].x);
            const uint32_t wy = (uint32_t)__builtin_amdgcn_ds_bpermute(src4, (int)b[n].w[g].y);
            // the word of row t holding group g's scale (int4: group 4 kl + g; MXFP4:
            // 32-blocks 8 kl + 2 g + {0, 1}), picked by a wave-uniform select
            uint32_t w;
            if constexpr (FMT == 4) {
                w = (kl & 1) ? sc[n][1][g] : sc[n][0][g];
            } else {
                const int k3 = kl & 3;  // values selected, not references (no stack copy)
                const uint32_t lo = (k3 & 2) ? sc[n][1][g >> 1] : sc[n][0][g >> 1];
                const uint32_t hi = (k3 & 2) ? sc[n][1][2 + (g >> 1)] : sc[n][0][2 + (g >> 1)];
                w = (k3 & 1) ? hi : lo;
            }
            const uint32_t sv = (uint32_t)__builtin_amdgcn_ds_bpermute(ssrc, (int)w);
            float sg;
            if constexpr (FMT == 4) {
                sg = __uint_as_float(sv);
            } else {  // lanes q < 2 take 32-block 2 g, q >= 2 block 2 g + 1
                sg = __uint_as_float(((sv >> (8 * (2 * (g & 1) + (q >> 1)))) & 0xffu) << 23);
            }
            bf16x8 B0, B1;
            bool spec = false;  // EXACT int4: this lane's column scale is not finite
            if constexpr (FMT == 4 && EXACT) {
                // the reference's x * ((n - 8) * scale): a non-finite scale enters each
                // product, which then takes the high term of x alone (its low terms would
                // turn inf * 0 into NaN)
                B0 = decode_b4_signed(wx);
                B1 = decode_b4_signed(wy);
                spec = nonfinite(sg);
                if (spec) {
                    B0 = mul_bf16x8_exact(B0, sg);
                    B1 = mul_bf16x8_exact(B1, sg);
                }
            } else {
                B0 = decode_b<FMT>(wx, sg);
                B1 = decode_b<FMT>(wy, sg);
                if constexpr (FMT == 7 && EXACT) {
                    if (b7_exceptional(sg)) {
                        B0 = decode_b7_exact(wx, sg);
                        B1 = decode_b7_exact(wy, sg);
                    }
                }
            }
            if constexpr (FMT == 4) {
                // the chain starts from -8 * (sum of the group's activations) of each row,
                // so it ends at sum_k a_k (n_k - 8) (EXACT: n - 8 decoded, from 0); one
                // scale per (row, group) then applies
                f4v c = c0;
#pragma unroll
                for (int tm = 0; tm < (PACK ? 1 : TERMS); ++tm) {
                    bf16x8 b0 = B0, b1 = B1;
                    if (EXACT && tm > 0 && spec)
                        b0 = b1 = bf16x8{};
                    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[tm][0], b0, c, 0, 0, 0);
                    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[tm][1], b1, c, 0, 0, 0);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    acc[n][i] = EXACT && spec ? acc[n][i] + c[i] : fmaf(sg, c[i], acc[n][i]);
                // materialise acc here: otherwise the chain is sunk past the masked
                // regions and every group's C and sums stay live to the end of the block
                asm volatile("" : "+v"(acc[n]));
            } else {
#pragma unroll
                for (int tm = 0; tm < (PACK ? 1 : TERMS); ++tm) {
                    acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[tm][0], B0, acc[n], 0, 0, 0);
                    acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[tm][1], B1, acc[n], 0, 0, 0);
                }
            }
            // one tile's operands at a time (register pressure)
            __builtin_amdgcn_sched_barrier(0);
        }
        // keep the next group's LDS reads from being hoisted over this one (register
        // pressure: two workgroups share a CU, so each wave has 128 VGPRs)
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Whether a wave's tiles need the exact redo, checked once after the streaming loop on
// what the wave holds: its tiles' scales over its K range (sc, this lane's 32 bytes of
// each row's range; only the nblk blocks' bytes count, as bytes past the scale buffer
// read as 0) and, for int4, the item's activation sums over the range (xr, [4 nblk][16]
// f32 in LDS; rows past the item hold 0).  Reasons: an MXFP4 scale byte outside the
// converter's exact range (b7_exceptional); a non-finite int4 scale (the common path
// applies it to the group's sum, where the reference forms each product (n - 8) *
// scale); a non-finite activation (-8 * sum + inf * n is NaN where the reference has
// +-inf).
template <int FMT, int NT>
__device__ __forceinline__ bool dec_needs_exact(const u32x4 (&sc)[NT][2], int q, int nblk,
                                                const float *xr, int lane) {
    const int used = (FMT == 4 ? 16 : 8) * nblk;  // scale bytes of a row's range
    bool r = false;
#pragma unroll
    for (int n = 0; n < NT; ++n)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (32 * q + 16 * h + 4 * e >= used)
                    continue;
                const uint32_t w = sc[n][h][e];
                if constexpr (FMT == 4) {
                    r |= nonfinite(__uint_as_float(w));
                } else {
#pragma unroll
                    for (int b = 0; b < 4; ++b)
                        r |= b7_exceptional(__uint_as_float(((w >> (8 * b)) & 0xffu) << 23));
                }
            }
    if constexpr (FMT == 4) {
        for (int i = lane; i < 64 * nblk; i += 64)
            r |= nonfinite(xr[i]);
    }
    return r;
}

// LDS layout of the decode kernel: A rows [rmax][K/8][terms][8] bf16 (+ 16 bytes per
// row), then fmt 4 sums [K/64][16] f32; the K-range combine buffer [waves][nt][4][64] f32
// reuses the start; after all of them the item's 16 out rows and 16 combine weights
// (the descriptor's, read once in the prologue).  Returns the total bytes.
__host__ __device__ inline int dec_row_bytes(int K, int terms) {
    return K * terms * 2 + 16;  // + 16: consecutive rows start in different LDS banks
}

__host__ __device__ inline size_t dec_lds_plan(int fmt, int K, int rmax, int terms, int ks,
                                               int nt, size_t *off_xs,
                                               size_t *off_comb = nullptr) {
    const size_t planes = (size_t)rmax * dec_row_bytes(K, terms);
    const size_t xs = fmt == 4 ? (size_t)(K / 64) * 16 * 4 : 0;
    const size_t red = ks > 1 ? (size_t)kDecWaves * nt * 4 * 64 * 4 : 0;
    if (off_xs)
        *off_xs = planes;
    const size_t tot = planes + xs > red ? planes + xs : red;
    if (off_comb)
        *off_comb = tot;
    return tot + 128;
}

// A pointer every lane holds the same value of, made visibly uniform (SGPRs): a buffer
// resource the compiler cannot prove uniform makes each load a loop over the lanes.
__device__ __forceinline__ const void *uniform_ptr(const void *p) {
    const unsigned long long v = reinterpret_cast<unsigned long long>(p);
    const unsigned lo = (unsigned)__builtin_amdgcn_readfirstlane((int)(unsigned)v);
    const unsigned hi = (unsigned)__builtin_amdgcn_readfirstlane((int)(unsigned)(v >> 32));
    return reinterpret_cast<const void *>(((unsigned long long)hi << 32) | lo);
}

// One task: item `item`, column block `wg` of one projection.
// INL: the descriptor comes from `kd` (compact, in the kernel arguments), not A.desc.
template <int FMT, bool DUAL, int TERMS, int KS, int NT, int SR, bool PACK = false,
          bool INL = false>
__device__ __forceinline__ void dec_task(const DecArgs &A, int item, int wg, int tid,
                                         char *smem, const DecDescK *kd = nullptr) {
    constexpr int TW = kDecWaves / KS;   // wave slots per K range
    constexpr int NU = NT == 2 ? 2 : 4;  // K blocks per tile in flight (VGPR budget)
    constexpr int XSR = 2;               // single, fmt 4: sums per thread (K / 4 <= 2048)
    static_assert(!DUAL || NT == 2, "dual waves carry a gate and an up tile");
    item = __builtin_amdgcn_readfirstlane(item);
    wg = __builtin_amdgcn_readfirstlane(wg);
    // the down descriptor this workgroup copies (wave 0): 16 bytes a lane, lanes l and
    // l + 16 k reading the same bytes (four requests; one 4-byte request a lane slowed
    // every workgroup's descriptor read over PCIe).  Issued first, stored with the staging
    // below: vector loads complete in order, so nothing waits for it early.
    const int cpi = item * A.wgs + wg;
    const bool cp =
        DUAL && cpi < A.n_cp && __builtin_amdgcn_readfirstlane(tid >> 6) == 0;
    u32x4 cpv = {0u, 0u, 0u, 0u};
    if (cp)
        cpv = reinterpret_cast<const u32x4 *>(A.cp_src + cpi)[tid & 15];
    static_assert(!INL || DUAL, "compact descriptors are gate/up only");
    const DecDesc &dd = A.desc[INL ? 0 : item];  // not read when INL
    const int K = A.K, O = A.O;
    const void *wp[2], *sp[2];
    int nrow, jbase;
    if constexpr (INL) {
        const DecDescK &k = kd[item];
        const char *w0 = static_cast<const char *>(k.w0);
        wp[0] = w0;
        wp[1] = w0 + k.off[0];
        sp[0] = w0 + k.off[1];
        sp[1] = w0 + k.off[2];
        nrow = k.nrow;
        jbase = k.jbase;
    } else {
        wp[0] = dd.w[0];
        wp[1] = dd.w[1];
        sp[0] = dd.s[0];
        sp[1] = dd.s[1];
        nrow = dd.nrow;
        jbase = dd.jbase;
    }
    // wave index as a scalar: tiles and K range are then wave-uniform (SGPRs)
    const int wave = __builtin_amdgcn_readfirstlane((tid >> 6));
    const int lane = tid & 63;
    const int t = lane & 15, q = lane >> 4;
    const int slot = wave % TW, ks = wave / TW;
    const int Kr = K / KS, kw0 = ks * Kr;
    const int nblk = Kr >> 8;
    const uint32_t rowb = (uint32_t)(K >> 1);
    const uint32_t srow = FMT == 4 ? (uint32_t)(K >> 4) : (uint32_t)(K >> 5);  // scale bytes
    int tile[NT];
    __amdgpu_buffer_rsrc_t rw[NT], rs[NT];
    uint32_t vw[NT], vs[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) {
        tile[n] = DUAL ? wg * TW + slot : wg * TW * NT + slot + n * TW;
        rw[n] = buf_rsrc(uniform_ptr(wp[DUAL ? n : 0]), (uint32_t)O * rowb);
        rs[n] = buf_rsrc(uniform_ptr(sp[DUAL ? n : 0]), (uint32_t)O * srow);
        vw[n] = (uint32_t)(tile[n] * 16 + (lane >> 2)) * rowb + 8u * (uint32_t)(lane & 3);
        vs[n] = (uint32_t)(tile[n] * 16 + t) * srow +
                (uint32_t)(FMT == 4 ? (kw0 >> 4) : (kw0 >> 5)) + 32u * (uint32_t)q;
    }
    const int rsb = dec_row_bytes(K, TERMS);  // bytes per A row in LDS
    size_t off_xs = 0, off_comb = 0;
    dec_lds_plan(FMT, K, A.rmax, TERMS, KS, NT, &off_xs, &off_comb);
    unsigned *lcomb = reinterpret_cast<unsigned *>(smem + off_comb);  // rows[16], wts[16]
    __bf16 *lp = reinterpret_cast<__bf16 *>(smem);
    float *lxs = reinterpret_cast<float *>(smem + off_xs);  // [K/64][16]
    float *red = reinterpret_cast<float *>(smem);           // [waves][NT][4][64]

    // 1) activation loads of this thread, issued first.  Chunk u * threads + thread of 8
    // elements; a row has per_row chunks, a multiple of 64 (K % 512 == 0), so the row of
    // a wave's chunks is wave-uniform (scalar loads of the descriptor's row map).  Chunks
    // past the item load and later store what chunk `lane` of row 0 does: loads and
    // stores stay unconditional, so the compiler neither sinks the loads into branches
    // nor waits for the weight loads issued after them.
    const int per_row = K >> 3;  // 8-element chunks per row
    const int total = DUAL ? nrow * per_row : TERMS * nrow * per_row;
    float4 xv[DUAL ? SR : 1][2];
    u32x4 st[DUAL ? 1 : SR];
    float xsr[XSR];
    unsigned comb = 0;  // single: word tid % 32 of the descriptor's rows[16] + wts[16]
    auto stage_loads = [&]() __attribute__((always_inline)) {
    if constexpr (!DUAL)  // unconditional: every lane loads, lanes < 32 keep it
        comb = reinterpret_cast<const unsigned *>(dd.rows)[tid & 31];
    if constexpr (DUAL) {
        int rr[16];  // the row map, one scalar load; picked below by uniform selects
#pragma unroll
        for (int i = 0; i < 16; ++i)
            rr[i] = INL ? (int)kd[item].rows[i] : dd.rows[i];
#pragma unroll
        for (int u = 0; u < SR; ++u) {
            // (divisions outside the selects: a division under a condition is not
            // speculated, and the branch it needs would pull loads into it)
            const int w0 = u * kDecThreads + wave * 64;  // first chunk of this wave
            const bool in = w0 < total;
            const int q0 = w0 / per_row;
            const int r = in ? q0 : 0;
            const int c = (in ? w0 - q0 * per_row : 0) + lane;
            int src = rr[0];
#pragma unroll
            for (int i = 1; i < 16; ++i)
                src = r == i ? rr[i] : src;
            const float4 *p = reinterpret_cast<const float4 *>(A.xin + (size_t)src * K + 8 * c);
            xv[u][0] = p[0];
            xv[u][1] = p[1];
        }
    } else {
#pragma unroll
        for (int u = 0; u < SR; ++u) {
            const int w0 = u * kDecThreads + wave * 64;
            const bool in = w0 < total;
            const int q0 = w0 / per_row;
            const int row = in ? q0 : 0;  // row = tm * nrow + r
            const int c = (in ? w0 - q0 * per_row : 0) + lane;
            const int tm = row / nrow, r = row - tm * nrow;
            const u32x4 *src = reinterpret_cast<const u32x4 *>(
                                   A.pin + ((size_t)tm * A.rcap + jbase + r) * (size_t)K) + c;
            st[u] = *src;
        }
        if constexpr (FMT == 4) {
#pragma unroll
            for (int u = 0; u < XSR; ++u) {
                const int i = u * kDecThreads + tid;
                const int g = i >> 4, r = i & 15;
                const bool ok = i < (K >> 2) && r < nrow;
                const float *pp =
                    A.xs + (size_t)(ok ? g : 0) * 4 * A.rcap + jbase + (ok ? r : 0);
                float p4[4];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    p4[e] = pp[e * A.rcap];
                xsr[u] = ok ? ((p4[0] + p4[1]) + p4[2]) + p4[3] : 0.f;
            }
        }
    }
    };
    // 2) ... then the first NU K blocks of every tile.  Unconditional (a range shorter
    // than NU blocks repeats its last block, never consumed): loads under a branch would
    // make the compiler's wait counts assume none were issued, and the staging below
    // would wait for the weights as well.
    DBlock<FMT> b[NU][NT];
    u32x4 sc[NT][2];
    auto prefetch = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int n = 0; n < NT; ++n)
            load_scales<FMT>(sc[n], rs[n], vs[n]);
        // the scales ahead of the weight blocks: the check before the loop waits for the
        // scales only, so no wave drains its weight prefetch before the loop starts
        asm volatile("" ::: "memory");
#pragma unroll
        for (int u = 0; u < NU; ++u)
#pragma unroll
            for (int n = 0; n < NT; ++n)
                load_dblock<FMT>(b[u][n], rw[n], vw[n], kw0 + 256 * (u < nblk ? u : nblk - 1));
    };
    stage_loads();
    prefetch();
    // every load above stays above (the compiler would otherwise sink the staging loads
    // into the stores' branches, behind a full wait); emits no instruction
    asm volatile("" ::: "memory");
    // 3) activations and sums into LDS
    if constexpr (DUAL) {
#pragma unroll
        for (int u = 0; u < SR; ++u) {
            const int w0 = u * kDecThreads + wave * 64;
            const bool in = w0 < total;
            const int q0 = w0 / per_row;
            const int r = in ? q0 : 0;
            const int c = (in ? w0 - q0 * per_row : 0) + lane;
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
            char *dst = reinterpret_cast<char *>(lp) + (size_t)r * rsb + (size_t)c * TERMS * 16;
#pragma unroll
            for (int tm = 0; tm < TERMS; ++tm)
                *reinterpret_cast<bf16x8 *>(dst + tm * 16) = o[tm];
            if constexpr (FMT == 4) {
                // per-64 sums of what the terms represent: 8 consecutive threads hold one
                // group of one row (per_row and kDecThreads are multiples of 8)
                rs8 += __shfl_xor(rs8, 1, 8);
                rs8 += __shfl_xor(rs8, 2, 8);
                rs8 += __shfl_xor(rs8, 4, 8);
                if ((c & 7) == 0)
                    lxs[(c >> 3) * 16 + r] = -8.f * rs8;
            }
        }
        if constexpr (FMT == 4) {  // rows nrow..15 of the sums read as 0
            for (int i = tid; i < (K / 64) * 16; i += kDecThreads)
                if ((i & 15) >= nrow)
                    lxs[i] = 0.f;
        }
    } else {
#pragma unroll
        for (int u = 0; u < SR; ++u) {
            const int w0 = u * kDecThreads + wave * 64;
            const bool in = w0 < total;
            const int q0 = w0 / per_row;
            const int row = in ? q0 : 0;
            const int c = (in ? w0 - q0 * per_row : 0) + lane;
            const int tm = row / nrow, r = row - tm * nrow;
            *reinterpret_cast<u32x4 *>(reinterpret_cast<char *>(lp) + (size_t)r * rsb +
                                       (size_t)c * TERMS * 16 + tm * 16) = st[u];
        }
        if constexpr (FMT == 4) {
#pragma unroll
            for (int u = 0; u < XSR; ++u) {
                const int i = u * kDecThreads + tid;
                if (i < (K >> 2))
                    lxs[i] = -8.f * xsr[u];
            }
        }
        if (tid < 32)
            lcomb[tid] = comb;
    }
    if (cp)
        reinterpret_cast<u32x4 *>(A.cp_dst + cpi)[tid & 15] = cpv;
    __syncthreads();

    // 4) MFMA over this wave's K blocks with NU in flight: b[u] holds block k0 + u; the
    // steady-state loop reloads each slot right after consuming it.
    f4v acc[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n)
        acc[n] = f4v{0.f, 0.f, 0.f, 0.f};
    static_assert(!PACK || TERMS == 2, "packing puts two terms into one MFMA");
    // this lane's A row (PACK: row t % 8, term t / 8)
    const int ar = PACK ? (t & 7) : t;
    const char *ta = reinterpret_cast<const char *>(lp) + (size_t)(ar < nrow ? ar : 0) * rsb +
                     (size_t)(2 * q) * TERMS * 16 + (PACK ? (t >> 3) * 16 : 0);
    const int src4 = 4 * (4 * t + q);  // ds_bpermute byte address of lane 4 t + q
    bf16x8 a[PACK ? 1 : TERMS][2] = {};  // A fragments; stay zero in rows past nrow
    // checked before the loop, while its first weight loads are in flight (the first
    // block needs the scales anyway); at the end it would lengthen every wave's tail
    const bool exc = __builtin_amdgcn_ballot_w64(
                         dec_needs_exact<FMT>(sc, q, nblk, lxs + (kw0 >> 6) * 16, lane)) != 0;
    auto consume = [&](const DBlock<FMT>(&bb)[NT], int kl) {
        const int kb = kw0 + 256 * kl;
        compute_dblock<FMT, TERMS, NT, false, PACK>(acc, a, bb, sc, kl,
                                                    ta + (size_t)(kb >> 3) * TERMS * 16, t, nrow,
                                                    lxs, kb, q, src4);
    };
    auto reload = [&](DBlock<FMT>(&bb)[NT], int kl) {
#pragma unroll
        for (int n = 0; n < NT; ++n)
            load_dblock<FMT>(bb[n], rw[n], vw[n], kw0 + 256 * kl);
    };
    int k0 = 0;
    for (; k0 + 2 * NU <= nblk; k0 += NU) {
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            consume(b[u], k0 + u);
            reload(b[u], k0 + u + NU);
        }
    }
#pragma unroll
    for (int u = 0; u < NU; ++u) {
        if (k0 + u < nblk) {
            consume(b[u], k0 + u);
            if (k0 + u + NU < nblk)
                reload(b[u], k0 + u + NU);
        }
    }
#pragma unroll
    for (int u = 0; u < NU; ++u)
        if (k0 + NU + u < nblk)
            consume(b[u], k0 + NU + u);
    if constexpr (PACK) {  // C row r + 8 holds the low term's part of row r
#pragma unroll
        for (int n = 0; n < NT; ++n)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                acc[n][i] += __shfl_xor(acc[n][i], 32);
    }
    {
        // Rare: operands the common path does not reproduce in this wave's tiles.  Redo
        // the tiles block by block with the exact decode; the streaming loop above then
        // carries no exact-path registers or checks.
        if (__builtin_expect(exc, 0)) {
#pragma unroll
            for (int n = 0; n < NT; ++n)
                acc[n] = f4v{0.f, 0.f, 0.f, 0.f};
            // unpacked: the exact int4 path keeps the low terms out of non-finite products
            const char *tu = reinterpret_cast<const char *>(lp) +
                             (size_t)(t < nrow ? t : 0) * rsb + (size_t)(2 * q) * TERMS * 16;
            bf16x8 au[TERMS][2] = {};
#pragma unroll 1
            for (int kl = 0; kl < nblk; ++kl) {
                DBlock<FMT> bb[NT];
                reload(bb, kl);
                const int kb = kw0 + 256 * kl;
                compute_dblock<FMT, TERMS, NT, true>(acc, au, bb, sc, kl,
                                                     tu + (size_t)(kb >> 3) * TERMS * 16, t, nrow,
                                                     lxs, kb, q, src4);
            }
        }
    }

    // 5) K ranges meet in LDS, summed in fixed order by the waves of range 0
    f4v fin[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n)
        fin[n] = acc[n];
    if constexpr (KS > 1) {
        __syncthreads();  // every wave is done reading the planes that `red` overwrites
#pragma unroll
        for (int n = 0; n < NT; ++n)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                red[((wave * NT + n) * 4 + i) * 64 + lane] = acc[n][i];
        __syncthreads();
#pragma unroll
        for (int n = 0; n < NT; ++n)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float sm = red[((slot * NT + n) * 4 + i) * 64 + lane];
#pragma unroll
                for (int k2 = 1; k2 < KS; ++k2)
                    sm += red[(((k2 * TW + slot) * NT + n) * 4 + i) * 64 + lane];
                fin[n][i] = sm;
            }
    }

    // 6) results, written by the waves of K range 0
    if (ks != 0) {
    } else if constexpr (DUAL) {
        // H = act(gate, up) -> planes of the down projection (+ 16-column partial sums)
        const int tl = tile[0];
        const int o = tl * 16 + t;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int tok = 4 * q + i;  // C row of this lane
            const int j = jbase + tok;
            const float h = mf_act(A.act, fin[0][i], fin[1][i], A.act_a, A.act_b);
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
                    A.hp[((size_t)(tl >> 2) * 4 + (tl & 3)) * A.rcap + j] = rep;
            }
        }
    } else {
        // this lane's rows 4 q + i of out and their weights (staged in LDS by the
        // prologue: the descriptor may live in host memory, too far to read at the end)
        u32x4 drow4 = {0u, 0u, 0u, 0u};
        f4v dwt4 = {0.f, 0.f, 0.f, 0.f};
        if (A.fold) {
            drow4 = *reinterpret_cast<const u32x4 *>(lcomb + 4 * q);
            dwt4 = *reinterpret_cast<const f4v *>(lcomb + 16 + 4 * q);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int tok = 4 * q + i;
            const int drow = (int)drow4[i];
            const float dwt = dwt4[i];
            if (tok < nrow && (!A.fold || drow >= 0)) {
#pragma unroll
                for (int n = 0; n < NT; ++n) {
                    const int o = tile[n] * 16 + t;
                    if (A.fold)  // top-k combine folded in: out[row] += w * y
                        unsafeAtomicAdd(A.out + (size_t)drow * O + o, __fmul_rn(dwt, fin[n][i]));
                    else
                        A.out[(size_t)(jbase + tok) * O + o] = fin[n][i];
                }
            }
        }
    }
}

}  // namespace mvllm_hip
