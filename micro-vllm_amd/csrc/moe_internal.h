// moe_internal.h -- structures shared by the C-ABI host code and the HIP kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace mvllm_hip {

// One expert with at least one row that reaches `out`.  Matrix m: 0 gate, 1 up, 2 down.
struct ExpertWork {
    const void *w[3];  // packed nibbles (fmt 4/7) or f32 rows (fmt 0), device
    const void *s[3];  // f32 scales (fmt 4) or ue8m0 bytes (fmt 7); unused for fmt 0
    int row0;          // first compact row of this expert (index into H / Y)
    int nrows;         // compact rows of this expert
    int pad[2];
};
static_assert(sizeof(ExpertWork) == 64, "ExpertWork layout");

// Arguments of one GEMV phase (gate/up/act, or down).
struct GemvArgs {
    const ExpertWork *ew;  // [n_experts]
    const int *in_rows;    // compact row -> input row (nullptr: identity)
    const float *in;       // input rows [*, K] f32
    float *out;            // output rows [R, O] f32 (H for gate/up, Y for down)
    int n_experts;
    int tiles_per_expert;
    int rows_per_tile;     // output rows one workgroup covers
    int K, O;
    int act;
    float act_a, act_b;
};

// Combine: out[out_row[t]] += sum_{e in [tok_ptr[t], tok_ptr[t+1])} ent_w[e] * Y[ent_row[e]]
struct CombineArgs {
    const float *Y;
    const int *tok_ptr;
    const int *ent_row;
    const float *ent_w;
    const int *out_row;
    float *out;
    int n_tok, D;
};

enum : int { ACT_SILU = 0, ACT_CLAMP_SWIGLU = 1, ACT_SITU = 2 };

// Launchers (kern_gemv.hip / kern_misc.hip).  All return hipSuccess or the launch error.
// Fast GEMV: fmt 4 or 7, K % 32 == 0, 16-byte aligned packed rows.
hipError_t launch_gemv_fast(int fmt, bool dual, int nr_max, int lanes_per_row, int passes,
                            const GemvArgs &a, hipStream_t st);
// Generic GEMV: any K, any alignment, fmt 0/4/7 (exact reference per-element formula).
hipError_t launch_gemv_generic(int fmt, bool dual, const GemvArgs &a, hipStream_t st);
hipError_t launch_combine(const CombineArgs &a, hipStream_t st);
hipError_t launch_dequant(int fmt, const void *packed, const void *scales, int O, int K,
                          float *w, hipStream_t st);
hipError_t launch_quantize_mxfp4(const float *x, int n, int K, uint8_t *codes, uint8_t *scales,
                                 hipStream_t st);

// Output rows one fast-GEMV workgroup covers for the given lanes_per_row / passes.
inline int gemv_rows_per_tile(int lanes_per_row, int passes) {
    return 4 * (64 / lanes_per_row) * passes;
}
// LDS bytes the fast GEMV stages per K-slice (one row: 36 floats per 32 inputs).
constexpr int kGemvLdsBytes = 36864;
inline int gemv_kslice(int nr_max, int K) {
    int chunks = kGemvLdsBytes / (nr_max * 144);
    int ks = chunks * 32;
    return ks >= K ? K : ks;
}

}  // namespace mvllm_hip
