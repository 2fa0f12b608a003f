/*
 * moe_oracle.c -- CPU restatement of micro-vllm's routed-expert moe_block path.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker and CPU-baseline timer); the HIP
 * product never links or falls back to it.  Build: oracle/Makefile, which uses
 * -O2 -ffp-contract=off so float expressions round exactly as written, matching
 * the reference's -O2 x86-64 build (no FMA contraction there either).
 *
 * Each function names the reference file:line it restates.  Float expressions
 * keep the reference's association order; that is what makes the outputs
 * bit-identical to oracle/_ref (checked in tests/test_oracle.py).
 */
#include "moe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static float bits_to_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

static uint32_t f32_to_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    return u;
}

/* ---- bf16 (src/quant/bf16.cpp:9-33) -------------------------------------- */

float orc_bf16_round(float v) {
    uint32_t u = f32_to_bits(v);
    /* finite: round-to-nearest-even on the discarded 16 bits; Inf/NaN: truncate */
    if ((u & 0x7f800000u) != 0x7f800000u)
        u += 0x7fffu + ((u >> 16) & 1u);
    return bits_to_f32(u & 0xffff0000u);
}

uint16_t orc_bf16_encode(float v) { return (uint16_t)(f32_to_bits(orc_bf16_round(v)) >> 16); }

float orc_bf16_decode(uint16_t h) { return bits_to_f32((uint32_t)h << 16); }

/* ---- MXFP4 codecs (src/quant/quant.cpp:16-17, src/quant/quant.hpp:13-20) --- */

/* e2m1: bit 3 = sign, bits 0..2 index {0, .5, 1, 1.5, 2, 3, 4, 6}; code 8 is -0. */
float orc_mx4_lut(int nibble) {
    static const float mag[8] = {0.f, 0.5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f};
    const float m = mag[nibble & 7];
    return (nibble & 8) ? -m : m;
}

/* ue8m0 -> float by placing the byte in the exponent field: 0 -> +0, 255 -> +inf. */
float orc_mx4_scale(uint8_t s) { return bits_to_f32((uint32_t)s << 23); }

/* ---- activations (src/quant/quant.hpp:22-50, src/quant/quant.cpp:400-403) -- */

float orc_sigmoid(float x) {
    if (x >= 0.f)
        return 1.f / (1.f + expf(-x));
    const float z = expf(x);
    return z / (1.f + z);
}

float orc_clamped_swiglu(float gate, float up, float limit) {
    float g = gate, u = up;
    if (limit > 0.f && g > limit)
        g = limit; /* the gate is clamped from above only */
    const float s = g * orc_sigmoid(g);
    if (limit > 0.f) {
        if (u > limit)
            u = limit;
        if (u < -limit)
            u = -limit;
    }
    return s * u;
}

float orc_situ_glu(float g, float u, float b1, float b2) {
    /* left-to-right: ((((b1*tanh(g/b1)) * sig(g)) * b2) * tanh(u/b2)) */
    return b1 * tanhf(g / b1) * orc_sigmoid(g) * b2 * tanhf(u / b2);
}

void orc_apply_act(float *g, const float *u, int n, int act, float a, float b) {
    if (!g || !u || n < 1)
        return;
    for (int i = 0; i < n; ++i) {
        if (act == ORC_ACT_CLAMP_SWIGLU)
            g[i] = orc_clamped_swiglu(g[i], u[i], a);
        else if (act == ORC_ACT_SITU)
            g[i] = orc_situ_glu(g[i], u[i], a, b);
        else
            g[i] = g[i] * orc_sigmoid(g[i]) * u[i]; /* silu_mul: (g*sig(g))*u */
    }
}

/* ---- GEMMs (src/quant/quant.cpp:156-168, 203-228, 298-321) --------------- */

void orc_matmul_f32(float *y, const float *x, const float *w, int S, int I, int O) {
    for (int s = 0; s < S; ++s) {
        const float *xr = x + (size_t)s * (size_t)I;
        for (int o = 0; o < O; ++o) {
            const float *wr = w + (size_t)o * (size_t)I;
            float acc = 0.f;
            for (int i = 0; i < I; ++i)
                acc += xr[i] * wr[i];
            y[(size_t)s * (size_t)O + (size_t)o] = acc;
        }
    }
}

static int nib(const uint8_t *row, int i) {
    const uint8_t b = row[i >> 1];
    return (i & 1) ? (b >> 4) : (b & 0x0f); /* low nibble holds the even index */
}

void orc_matmul_int4_g64(float *y, const float *x, const uint8_t *packed, const float *scales,
                         int S, int I, int O) {
    const size_t stride = (size_t)((I + 1) / 2);
    const int ng = (I + 63) / 64;
    for (int s = 0; s < S; ++s) {
        const float *xr = x + (size_t)s * (size_t)I;
        for (int o = 0; o < O; ++o) {
            const uint8_t *prow = packed + (size_t)o * stride;
            const float *srow = scales + (size_t)o * (size_t)ng;
            float acc = 0.f; /* one running accumulator across all groups */
            for (int gi = 0; gi < ng; ++gi) {
                const float sc = srow[gi];
                const int hi = (gi * 64 + 64 < I) ? gi * 64 + 64 : I;
                for (int i = gi * 64; i < hi; ++i)
                    acc += xr[i] * ((float)(nib(prow, i) - 8) * sc);
            }
            y[(size_t)s * (size_t)O + (size_t)o] = acc;
        }
    }
}

void orc_matmul_int8_row(float *y, const float *x, const int8_t *q, const float *scales, int S,
                         int I, int O) {
    for (int s = 0; s < S; ++s) {
        const float *xr = x + (size_t)s * (size_t)I;
        for (int o = 0; o < O; ++o) {
            const int8_t *qr = q + (size_t)o * (size_t)I;
            float acc = 0.f;
            for (int i = 0; i < I; ++i)
                acc += xr[i] * (float)qr[i];
            y[(size_t)s * (size_t)O + (size_t)o] = acc * scales[o];
        }
    }
}

void orc_matmul_mxfp4(float *y, const float *x, const uint8_t *packed, const uint8_t *scales,
                      int S, int I, int O) {
    const size_t stride = (size_t)((I + 1) / 2);
    const int ng = (I + 31) / 32;
    for (int s = 0; s < S; ++s) {
        const float *xr = x + (size_t)s * (size_t)I;
        for (int o = 0; o < O; ++o) {
            const uint8_t *prow = packed + (size_t)o * stride;
            const uint8_t *srow = scales + (size_t)o * (size_t)ng;
            float acc = 0.f;
            for (int gi = 0; gi < ng; ++gi) {
                const float sc = orc_mx4_scale(srow[gi]);
                const int hi = (gi * 32 + 32 < I) ? gi * 32 + 32 : I;
                for (int i = gi * 32; i < hi; ++i)
                    acc += xr[i] * (orc_mx4_lut(nib(prow, i)) * sc);
            }
            y[(size_t)s * (size_t)O + (size_t)o] = acc;
        }
    }
}

void orc_dequant_int4_g64(float *w, const uint8_t *packed, const float *scales, int O, int I) {
    const size_t stride = (size_t)((I + 1) / 2);
    const int ng = (I + 63) / 64;
    for (int o = 0; o < O; ++o)
        for (int i = 0; i < I; ++i)
            w[(size_t)o * (size_t)I + (size_t)i] =
                (float)(nib(packed + (size_t)o * stride, i) - 8) * scales[(size_t)o * ng + i / 64];
}

void orc_dequant_mxfp4(float *w, const uint8_t *packed, const uint8_t *scales, int O, int I) {
    const size_t stride = (size_t)((I + 1) / 2);
    const int ng = (I + 31) / 32;
    for (int o = 0; o < O; ++o)
        for (int i = 0; i < I; ++i)
            w[(size_t)o * (size_t)I + (size_t)i] =
                orc_mx4_lut(nib(packed + (size_t)o * stride, i)) *
                orc_mx4_scale(scales[(size_t)o * ng + i / 32]);
}

/* ---- moe_block (src/gpu/metal_ops.cpp:278-342, 448-460) ------------------ */

static void expert_mlp(int fmt, int nre, int D, int Iinter, const void *gw, const void *uw,
                       const void *dw, const void *gsc, const void *usc, const void *dsc,
                       const float *xe, float *gate, float *up, float *hh, int act, float a,
                       float b) {
    if (fmt == 0) {
        orc_matmul_f32(gate, xe, (const float *)gw, nre, D, Iinter);
        orc_matmul_f32(up, xe, (const float *)uw, nre, D, Iinter);
        orc_apply_act(gate, up, nre * Iinter, act, a, b);
        orc_matmul_f32(hh, gate, (const float *)dw, nre, Iinter, D);
    } else if (fmt == 7) {
        orc_matmul_mxfp4(gate, xe, (const uint8_t *)gw, (const uint8_t *)gsc, nre, D, Iinter);
        orc_matmul_mxfp4(up, xe, (const uint8_t *)uw, (const uint8_t *)usc, nre, D, Iinter);
        orc_apply_act(gate, up, nre * Iinter, act, a, b);
        orc_matmul_mxfp4(hh, gate, (const uint8_t *)dw, (const uint8_t *)dsc, nre, Iinter, D);
    } else {
        orc_matmul_int4_g64(gate, xe, (const uint8_t *)gw, (const float *)gsc, nre, D, Iinter);
        orc_matmul_int4_g64(up, xe, (const uint8_t *)uw, (const float *)usc, nre, D, Iinter);
        orc_apply_act(gate, up, nre * Iinter, act, a, b);
        orc_matmul_int4_g64(hh, gate, (const uint8_t *)dw, (const float *)dsc, nre, Iinter, D);
    }
}

int orc_moe_block(int nb, int D, int Iinter, int fmt, int qgs, const void *const *g,
                  const void *const *u, const void *const *d, const float *const *gs,
                  const float *const *us, const float *const *ds, const float *xg,
                  const int *xoff, const int *nr, const int *rows, const float *rw, float *out,
                  int S, int act, float act_a, float act_b) {
    (void)qgs; /* the reference ignores qgs: 64 for fmt 4, 32 for fmt 7 */
    if (nb < 1 || D < 1 || !out || !xg || (fmt != 0 && fmt != 4 && fmt != 7))
        return 0;
    if (!xoff || !nr)
        return 0;
    int base = 0;
    for (int e = 0; e < nb; ++e) {
        const int nre = nr[e];
        if (nre <= 0)
            continue;
        /* experts that cannot run still consume their rows */
        if (Iinter < 1 || !g || !u || !d || !g[e] || !u[e] || !d[e]) {
            base += nre;
            continue;
        }
        if ((fmt == 4 || fmt == 7) && (!gs || !us || !ds || !gs[e] || !us[e] || !ds[e])) {
            base += nre;
            continue;
        }
        const size_t ni = (size_t)nre * (size_t)Iinter, nd = (size_t)nre * (size_t)D;
        float *gate = (float *)calloc(ni, sizeof(float));
        float *up = (float *)calloc(ni, sizeof(float));
        float *hh = (float *)calloc(nd, sizeof(float));
        if (!gate || !up || !hh) {
            free(gate);
            free(up);
            free(hh);
            return 0;
        }
        const float *xe = xg + (size_t)xoff[e] * (size_t)D;
        expert_mlp(fmt, nre, D, Iinter, g[e], u[e], d[e], fmt ? (const void *)gs[e] : NULL,
                   fmt ? (const void *)us[e] : NULL, fmt ? (const void *)ds[e] : NULL, xe, gate,
                   up, hh, act, act_a, act_b);
        if (rows && rw) {
            for (int r = 0; r < nre; ++r) {
                const int dest = rows[base + r];
                if (dest < 0 || (S > 0 && dest >= S))
                    continue;
                const float wgt = rw[base + r];
                float *orow = out + (size_t)dest * (size_t)D;
                const float *hrow = hh + (size_t)r * (size_t)D;
                for (int i = 0; i < D; ++i)
                    orow[i] += wgt * hrow[i];
            }
        }
        free(gate);
        free(up);
        free(hh);
        base += nre;
    }
    return 1;
}

/* ---- routing / segments -------------------------------------------------- */

/* a ranks before b: larger choice first, lower index on ties (src/model/ops.cpp:866-871) */
static int ranks_before(const float *choice, int a, int b) {
    if (choice[a] == choice[b])
        return a < b;
    return choice[a] > choice[b];
}

/* src/model/ops.cpp:860-889.  Selection instead of partial_sort; both yield the k
 * first elements of the same strict weak order, sorted. */
int orc_moe_topk(const float *choice, int n, int k, int *idx, float *w, const float *mix) {
    if (k > n)
        k = n;
    if (k <= 0)
        return k < 0 ? k : 0;
    char *taken = (char *)calloc((size_t)n, 1);
    if (!taken)
        return 0;
    for (int i = 0; i < k; ++i) {
        int best = -1;
        for (int j = 0; j < n; ++j)
            if (!taken[j] && (best < 0 || ranks_before(choice, j, best)))
                best = j;
        taken[best] = 1;
        idx[i] = best;
    }
    free(taken);
    float sum = 0.f;
    for (int i = 0; i < k; ++i) {
        w[i] = mix ? mix[idx[i]] : choice[idx[i]];
        if (w[i] < 0.f)
            w[i] = 0.f;
        sum += w[i];
    }
    for (int i = 0; i < k; ++i)
        w[i] = (sum > 0.f) ? w[i] / sum : 1.f / (float)k;
    return k;
}

/* moe_topk over n_tok tokens in one call (choice/mix rows of n floats, idx/w rows of k):
 * the per-token loop of the reference's prefill router, so a host timing of it carries
 * no per-token call overhead.  Returns the per-token k. */
int orc_moe_topk_batch(const float *choice, int n_tok, int n, int k, int *idx, float *w,
                       const float *mix) {
    int kk = 0;
    for (int t = 0; t < n_tok; ++t)
        kk = orc_moe_topk(choice + (size_t)t * n, n, k, idx + (size_t)t * k, w + (size_t)t * k,
                          mix ? mix + (size_t)t * n : NULL);
    return kk;
}

static int cmp_int(const void *a, const void *b) {
    const int x = *(const int *)a, y = *(const int *)b;
    return (x > y) - (x < y);
}

/* src/model/ops.cpp:1082-1099: sorted unique non-negative ids, at most out_cap. */
int orc_moe_union_ids(const int *idx, int n_tok, int topk, int *out, int out_cap) {
    if (!idx || !out || n_tok <= 0 || topk <= 0 || out_cap <= 0)
        return 0;
    const size_t total = (size_t)n_tok * (size_t)topk;
    int *all = (int *)malloc(total * sizeof(int));
    if (!all)
        return 0;
    int n = 0;
    for (size_t i = 0; i < total; ++i)
        if (idx[i] >= 0)
            all[n++] = idx[i];
    qsort(all, (size_t)n, sizeof(int), cmp_int);
    int cnt = 0;
    for (int i = 0; i < n && cnt < out_cap; ++i)
        if (cnt == 0 || all[i] != out[cnt - 1])
            out[cnt++] = all[i];
    free(all);
    return cnt;
}

/* src/model/glm53.cpp:1938-1971 (and the identical src/model/kimi_k3.cpp:2009-2050):
 * for each unique expert in ascending order, its rows are the tokens c in ascending
 * order whose summed weight wsum (adds in top-k slot order, from 0.f) is non-zero. */
int orc_moe_segments(const int *idx, const float *wt, int n_tok, int topk, int *eids, int *xoff,
                     int *nr, int *rows, float *rw, int cap_experts, int cap_rows,
                     int *n_rows_out) {
    if (n_rows_out)
        *n_rows_out = 0;
    if (!idx || !wt || n_tok <= 0 || topk <= 0 || cap_experts <= 0)
        return 0;
    int *uniq = (int *)malloc((size_t)cap_experts * sizeof(int));
    if (!uniq)
        return -1;
    const int nu = orc_moe_union_ids(idx, n_tok, topk, uniq, cap_experts);
    int j = 0;
    for (int ui = 0; ui < nu; ++ui) {
        const int eid = uniq[ui];
        eids[ui] = eid;
        xoff[ui] = j;
        int cnt = 0;
        for (int c = 0; c < n_tok; ++c) {
            float wsum = 0.f;
            for (int t = 0; t < topk; ++t)
                if (idx[(size_t)c * topk + t] == eid)
                    wsum += wt[(size_t)c * topk + t];
            if (wsum == 0.f)
                continue;
            if (j >= cap_rows) {
                free(uniq);
                return -1;
            }
            rows[j] = c;
            rw[j] = wsum;
            ++j;
            ++cnt;
        }
        nr[ui] = cnt;
    }
    free(uniq);
    if (n_rows_out)
        *n_rows_out = j;
    return nu;
}

/* ---- native activation codecs (src/quant/native_act.cpp:24-88, 159-179) --- */

float orc_e8m0_decode(uint8_t v) {
    if (v == 0xff)
        return NAN;
    return ldexpf(1.f, (int)v - 127);
}

float orc_e2m1_decode(uint8_t nibble) {
    /* unlike orc_mx4_lut, code 8 decodes to +0 here (src/quant/native_act.cpp:82-88) */
    const int n = nibble & 15;
    return n == 8 ? 0.f : orc_mx4_lut(n);
}

/* ceil(log2(v)) for v > 0: frexp gives v = f * 2^e with f in [0.5, 1). */
static int ceil_log2_pos(float v) {
    int e = 0;
    const float f = frexpf(v, &e);
    return f == 0.5f ? e - 1 : e;
}

/* nearest e2m1 code; strict '<' keeps the lowest code index on ties */
static int nearest_code(float v) {
    int best = 0;
    float dist = fabsf(v - orc_e2m1_decode(0));
    for (int c = 1; c < 16; ++c) {
        const float dd = fabsf(v - orc_e2m1_decode((uint8_t)c));
        if (dd < dist) {
            dist = dd;
            best = c;
        }
    }
    return best;
}

int orc_fp4_activation_qdq(float *output, uint8_t *scales, const float *input, int length,
                           int block_size, uint8_t *codes) {
    if (!output || !scales || !input || length <= 0 || block_size <= 0)
        return -1;
    const float floor_amax = 6.f * ldexpf(1.f, -126);
    for (int base = 0; base < length; base += block_size) {
        const int n = (length - base < block_size) ? length - base : block_size;
        float amax = 0.f;
        for (int i = 0; i < n; ++i) {
            const float a = fabsf(input[base + i]);
            if (a > amax) /* NaN never wins */
                amax = a;
        }
        amax = fmaxf(amax, floor_amax);
        int ex = ceil_log2_pos(amax / 6.f);
        ex = ex < -127 ? -127 : (ex > 127 ? 127 : ex);
        const uint8_t sc = (uint8_t)(ex + 127);
        scales[base / block_size] = sc;
        const float scale = orc_e8m0_decode(sc);
        for (int i = 0; i < n; ++i) {
            const float q = fmaxf(-6.f, fminf(6.f, input[base + i] / scale));
            const int c = nearest_code(q);
            if (codes)
                codes[base + i] = (uint8_t)c;
            output[base + i] = orc_e2m1_decode((uint8_t)c) * scale;
        }
    }
    return 0;
}


/* ---- native-FP4 composition (the checker of the MXFP4-activation path) -------
 * The reference moe_block (src/gpu/metal_ops.cpp:278-342) with the input of each GEMM
 * passed through the reference's MXFP4 activation quantize-dequantize
 * (fp4_activation_qdq, block 32, src/quant/native_act.cpp:159-179) row by row: x rows
 * before gate/up, h rows before down.  fmt must be 7; validation and skip rules are
 * moe_block's. */
static void qdq_rows(float *dst, const float *src, int n, int len, uint8_t *sc) {
    for (int r = 0; r < n; ++r)
        orc_fp4_activation_qdq(dst + (size_t)r * len, sc, src + (size_t)r * len, len, 32, NULL);
}

int orc_moe_block_fp4act(int nb, int D, int Iinter, int fmt, int qgs, const void *const *g,
                         const void *const *u, const void *const *d, const float *const *gs,
                         const float *const *us, const float *const *ds, const float *xg,
                         const int *xoff, const int *nr, const int *rows, const float *rw,
                         float *out, int S, int act, float act_a, float act_b) {
    (void)qgs;
    if (nb < 1 || D < 1 || !out || !xg || fmt != 7 || !xoff || !nr)
        return 0;
    int base = 0;
    for (int e = 0; e < nb; ++e) {
        const int nre = nr[e];
        if (nre <= 0)
            continue;
        if (Iinter < 1 || !g || !u || !d || !g[e] || !u[e] || !d[e] || !gs || !us || !ds ||
            !gs[e] || !us[e] || !ds[e]) {
            base += nre;
            continue;
        }
        const size_t ni = (size_t)nre * (size_t)Iinter, nd = (size_t)nre * (size_t)D;
        float *xq = (float *)calloc(nd, sizeof(float));
        float *gate = (float *)calloc(ni, sizeof(float));
        float *up = (float *)calloc(ni, sizeof(float));
        float *hq = (float *)calloc(ni, sizeof(float));
        float *hh = (float *)calloc(nd, sizeof(float));
        uint8_t *sc = (uint8_t *)calloc((size_t)(D > Iinter ? D : Iinter) / 32 + 1, 1);
        if (!xq || !gate || !up || !hq || !hh || !sc) {
            free(xq); free(gate); free(up); free(hq); free(hh); free(sc);
            return 0;
        }
        qdq_rows(xq, xg + (size_t)xoff[e] * (size_t)D, nre, D, sc);
        orc_matmul_mxfp4(gate, xq, (const uint8_t *)g[e], (const uint8_t *)gs[e], nre, D, Iinter);
        orc_matmul_mxfp4(up, xq, (const uint8_t *)u[e], (const uint8_t *)us[e], nre, D, Iinter);
        orc_apply_act(gate, up, nre * Iinter, act, act_a, act_b);
        qdq_rows(hq, gate, nre, Iinter, sc);
        orc_matmul_mxfp4(hh, hq, (const uint8_t *)d[e], (const uint8_t *)ds[e], nre, Iinter, D);
        if (rows && rw) {
            for (int r = 0; r < nre; ++r) {
                const int dest = rows[base + r];
                if (dest < 0 || (S > 0 && dest >= S))
                    continue;
                const float wgt = rw[base + r];
                float *orow = out + (size_t)dest * (size_t)D;
                const float *hrow = hh + (size_t)r * (size_t)D;
                for (int i = 0; i < D; ++i)
                    orow[i] += wgt * hrow[i];
            }
        }
        free(xq); free(gate); free(up); free(hq); free(hh); free(sc);
        base += nre;
    }
    return 1;
}

/* ---- the steps either side of the block --------------------------------------- */

/* quant::rmsnorm (src/quant/quant.cpp:384-398): sequential f32 sum of squares, one
 * reciprocal square root, then x * inv * w in that order. */
void orc_rmsnorm(const float *x, const float *w, float *y, int n, float eps) {
    if (n <= 0)
        return;
    float ss = 0.f;
    for (int i = 0; i < n; ++i)
        ss += x[i] * x[i];
    const float inv = 1.f / sqrtf(ss / (float)n + eps);
    if (w) {
        for (int i = 0; i < n; ++i)
            y[i] = x[i] * inv * w[i];
    } else {
        for (int i = 0; i < n; ++i)
            y[i] = x[i] * inv;
    }
}

/* cpu_route (src/gpu/metal_ops.cpp:213-231) for one row: scores = matmul_f32(x, w),
 * mix = sigmoid(scores), choice = mix + bias (0 without), moe_topk(choice, mix), then the
 * first min(k, E) weights times rscale when rscale != 1. */
void orc_route(const float *x, const float *w, const float *bias, int D, int E, int k,
               float rscale, int *idx, float *wt) {
    if (!x || !w || !idx || !wt || D < 1 || E < 1 || k < 1)
        return;
    float *scores = (float *)calloc((size_t)E, sizeof(float));
    float *choice = (float *)calloc((size_t)E, sizeof(float));
    if (!scores || !choice) {
        free(scores);
        free(choice);
        return;
    }
    orc_matmul_f32(scores, x, w, 1, D, E);
    for (int i = 0; i < E; ++i) {
        scores[i] = orc_sigmoid(scores[i]);
        choice[i] = scores[i] + (bias ? bias[i] : 0.f);
    }
    orc_moe_topk(choice, E, k, idx, wt, scores);
    if (rscale != 1.f) {
        const int kk = k > E ? E : k;
        for (int i = 0; i < kk; ++i)
            wt[i] *= rscale;
    }
    free(scores);
    free(choice);
}
