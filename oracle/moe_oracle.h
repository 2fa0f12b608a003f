/*
 * moe_oracle.h -- CPU restatement of micro-vllm's routed-expert moe_block path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * implementation in micro-vllm_amd/csrc.  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load it, and only to check or to time the
 * CPU baseline.  The product never links, loads or falls back to it.
 *
 * Every function restates one reference function (file:line under the
 * reference tree) with the same loop order and the same float evaluation order,
 * so that on x86-64 built with -O2 -ffp-contract=off it is bit-identical to the
 * reference build in oracle/_ref.  How each function is pinned (reference KATs,
 * bit-exact comparison against oracle/_ref, f64 closed forms) is listed in
 * tests/test_oracle.py; no function here is "parity unpinned".
 */
#ifndef MVLLM_MOE_ORACLE_H
#define MVLLM_MOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Activation selector; same numbering as metal_ops::Act (src/gpu/metal_ops.hpp:41-44). */
enum { ORC_ACT_SILU = 0, ORC_ACT_CLAMP_SWIGLU = 1, ORC_ACT_SITU = 2 };

/* bf16 helpers: src/quant/bf16.cpp:9-33 */
float orc_bf16_round(float v);
uint16_t orc_bf16_encode(float v);
float orc_bf16_decode(uint16_t h);

/* MXFP4 codecs: src/quant/quant.cpp:16-17 (LUT), src/quant/quant.hpp:13-20 (ue8m0 scale). */
float orc_mx4_lut(int nibble);
float orc_mx4_scale(uint8_t s);

/* Activations: src/quant/quant.hpp:22-50, src/quant/quant.cpp:400-403. */
float orc_sigmoid(float x);
float orc_clamped_swiglu(float gate, float up, float limit);
float orc_situ_glu(float g, float u, float b1, float b2);
/* src/gpu/metal_ops.cpp:197-211 */
void orc_apply_act(float *g, const float *u, int n, int act, float a, float b);

/* GEMMs, y[S,O] = x[S,I] . W[O,I]^T: src/quant/quant.cpp:156-168, 203-228, 298-321. */
void orc_matmul_f32(float *y, const float *x, const float *w, int S, int I, int O);
void orc_matmul_int4_g64(float *y, const float *x, const uint8_t *packed, const float *scales,
                         int S, int I, int O);
/* quant::matmul_int8_row (src/quant/quant.cpp:255-268): y[s,o] = (sum_i x[s,i] * q[o,i]) *
 * scales[o], one sequential f32 sum per output, the row scale applied once after it.  q is
 * int8 [O][I] (QuantMat fmt 8, src/quant/weight.cpp:38-41,57-61). */
void orc_matmul_int8_row(float *y, const float *x, const int8_t *q, const float *scales, int S,
                         int I, int O);
void orc_matmul_mxfp4(float *y, const float *x, const uint8_t *packed, const uint8_t *scales,
                      int S, int I, int O);

/* Dequantized weight matrices w[O,I] exactly as the GEMM inner loops form them:
 * int4: (nib-8)*scale (src/quant/quant.cpp:220-222); mxfp4: lut[nib]*scale
 * (src/quant/quant.cpp:313-316). */
void orc_dequant_int4_g64(float *w, const uint8_t *packed, const float *scales, int O, int I);
void orc_dequant_mxfp4(float *w, const uint8_t *packed, const uint8_t *scales, int O, int I);

/* metal_ops::moe_block validation + cpu_moe_block
 * (src/gpu/metal_ops.cpp:278-342, 448-460).  Returns 1 ("ran"), 0 ("fall back"). */
int orc_moe_block(int nb, int D, int Iinter, int fmt, int qgs, const void *const *g,
                  const void *const *u, const void *const *d, const float *const *gs,
                  const float *const *us, const float *const *ds, const float *xg,
                  const int *xoff, const int *nr, const int *rows, const float *rw, float *out,
                  int S, int act, float act_a, float act_b);

/* Routing and segment construction: src/model/ops.cpp:860-889 (moe_topk),
 * src/model/ops.cpp:1082-1099 (moe_union_ids), src/model/glm53.cpp:1938-1971
 * (per-expert gather loop). */
int orc_moe_topk(const float *choice, int n, int k, int *idx, float *w, const float *mix);
int orc_moe_topk_batch(const float *choice, int n_tok, int n, int k, int *idx, float *w,
                       const float *mix);
int orc_moe_union_ids(const int *idx, int n_tok, int topk, int *out, int out_cap);
/* Segments for one batched moe_block call that reproduces moe_layer_n's
 * per-expert loop: eids[nb] (ascending), xoff/nr[nb], and per routed row j:
 * rows[j] = token, rw[j] = wsum, which is also the gather index into x.
 * Returns nb, or -1 if a capacity is too small. */
int orc_moe_segments(const int *idx, const float *wt, int n_tok, int topk, int *eids, int *xoff,
                     int *nr, int *rows, float *rw, int cap_experts, int cap_rows,
                     int *n_rows_out);

/* moe_block with MXFP4-quantized GEMM inputs: fp4_activation_qdq (block 32) on the x rows
 * before gate/up and on the h rows before down, fmt 7 only -- the checker of the native
 * scaled-FP4 matrix-core path (src/gpu/metal_ops.cpp:278-342 composed with
 * src/quant/native_act.cpp:159-179). */
int orc_moe_block_fp4act(int nb, int D, int Iinter, int fmt, int qgs, const void *const *g,
                         const void *const *u, const void *const *d, const float *const *gs,
                         const float *const *us, const float *const *ds, const float *xg,
                         const int *xoff, const int *nr, const int *rows, const float *rw,
                         float *out, int S, int act, float act_a, float act_b);

/* Native activation codecs: src/quant/native_act.cpp:24-88, 159-179.
 * codes (nullable) receives the chosen e2m1 code per element. */
float orc_e8m0_decode(uint8_t v);
float orc_e2m1_decode(uint8_t nib);
int orc_fp4_activation_qdq(float *output, uint8_t *scales, const float *input, int length,
                           int block_size, uint8_t *codes);

/* The steps either side of the block: quant::rmsnorm (src/quant/quant.cpp:384-398) and
 * cpu_route (src/gpu/metal_ops.cpp:213-231) of one row. */
void orc_rmsnorm(const float *x, const float *w, float *y, int n, float eps);
void orc_route(const float *x, const float *w, const float *bias, int D, int E, int k,
               float rscale, int *idx, float *wt);

#ifdef __cplusplus
}
#endif

#endif
