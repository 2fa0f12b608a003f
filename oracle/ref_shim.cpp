// ref_shim.cpp -- extern "C" entry points over the reference's own hot-path functions.
//
// TEST INFRASTRUCTURE ONLY.  oracle/Makefile compiles this file together with the
// reference sources where they lie under /root/reference/src (nothing is copied)
// into oracle/_ref/libmvllm_ref.so.  Tests use it to check the C restatement in
// oracle/moe_oracle.c bit for bit; bench.py may time it as the CPU baseline.
#include "gpu/metal_ops.hpp"
#include "model/family.hpp"
#include "quant/bf16.hpp"
#include "quant/native_act.hpp"
#include "quant/quant.hpp"

#include <cstdint>

using namespace mvllm;

extern "C" {

int ref_moe_block(int nb, int D, int Iinter, int fmt, int qgs, const void *const *g,
                  const void *const *u, const void *const *d, const float *const *gs,
                  const float *const *us, const float *const *ds, const float *xg,
                  const int *xoff, const int *nr, const int *rows, const float *rw, float *out,
                  int S, int act, float act_a, float act_b) {
    return metal_ops::moe_block(nb, D, Iinter, fmt, qgs, g, u, d, gs, us, ds, xg, xoff, nr, rows,
                                rw, out, S, static_cast<metal_ops::Act>(act), act_a, act_b)
               ? 1
               : 0;
}

void ref_matmul_f32(float *y, const float *x, const float *w, int S, int I, int O) {
    quant::matmul_f32(y, x, w, S, I, O);
}
void ref_matmul_int4_g64(float *y, const float *x, const uint8_t *p, const float *s, int S, int I,
                         int O) {
    quant::matmul_int4_g64(y, x, p, s, S, I, O);
}
void ref_matmul_mxfp4(float *y, const float *x, const uint8_t *p, const uint8_t *s, int S, int I,
                      int O) {
    quant::matmul_mxfp4(y, x, p, s, S, I, O);
}
void ref_matmul_int8_row(float *y, const float *x, const int8_t *q, const float *s, int S, int I,
                         int O) {
    quant::matmul_int8_row(y, x, q, s, S, I, O);
}
void ref_quantize_int8_row(const float *w, int O, int I, int8_t *q, float *s) {
    quant::quantize_int8_row(w, O, I, q, s);
}
void ref_quantize_int4_g64(const float *w, int O, int I, uint8_t *p, float *s) {
    quant::quantize_int4_g64(w, O, I, p, s);
}
void ref_pack_mxfp4(const float *w, int O, int I, uint8_t *p, uint8_t *s) {
    quant::pack_mxfp4(w, O, I, p, s);
}
float ref_mx4_lut(int n) { return quant::mx4_lut[n & 15]; }
float ref_mx4_scale(uint8_t s) { return quant::mx4_scale(s); }
float ref_sigmoid(float x) { return quant::sigmoid(x); }
float ref_clamped_swiglu(float g, float u, float a) { return quant::clamped_swiglu(g, u, a); }
float ref_situ_glu(float g, float u, float a, float b) { return quant::situ_glu(g, u, a, b); }
void ref_silu_mul(float *g, const float *u, int n) { quant::silu_mul(g, u, n); }

int ref_moe_topk(const float *choice, int n, int k, int *idx, float *w, const float *mix) {
    return moe_topk(choice, n, k, idx, w, mix);
}
// The reference's moe_topk for n_tok tokens in one call (rows of n scores, rows of k out).
int ref_moe_topk_batch(const float *choice, int n_tok, int n, int k, int *idx, float *w,
                       const float *mix) {
    int kk = 0;
    for (int t = 0; t < n_tok; ++t)
        kk = moe_topk(choice + (size_t)t * n, n, k, idx + (size_t)t * k, w + (size_t)t * k,
                      mix ? mix + (size_t)t * n : nullptr);
    return kk;
}
int ref_moe_union_ids(const int *idx, int n_tok, int topk, int *out, int cap) {
    return moe_union_ids(idx, n_tok, topk, out, cap);
}

float ref_bf16_round(float v) { return bf16_round(v); }
void ref_rmsnorm(const float *x, const float *w, float *y, int n, float eps) {
    quant::rmsnorm(x, w, y, n, eps);
}
// The reference's own router (cpu_route, file-local in metal_ops.cpp) through its public
// host path: metal_ops::layer_decode_full with no attention, no shared expert and the
// library never initialised runs rmsnorm(x, post_ln) -> nrm, then cpu_route(nrm).
void ref_norm_route(float *x, const float *post_ln, int D, float eps, const float *w,
                    const float *bias, int E, int K, float rscale, float *nrm, int *idx,
                    float *wt) {
    metal_ops::layer_decode_full(x, nullptr, nullptr, post_ln, nullptr, nullptr, nullptr, D, 0,
                                 eps, metal_ops::Act::Silu, 0.f, 0.f, w, bias, E, K, rscale,
                                 nullptr, nrm, nullptr, idx, wt);
}
void ref_bf16_round_array(float *v, int n) { bf16_round_array(v, n); }
float ref_e8m0_decode(uint8_t v) { return e8m0_decode(v); }
float ref_e2m1_decode(uint8_t v) { return e2m1_decode(v); }
int ref_fp4_activation_qdq(float *o, uint8_t *s, const float *in, int len, int bs) {
    return fp4_activation_qdq(o, s, in, len, bs);
}

} // extern "C"
