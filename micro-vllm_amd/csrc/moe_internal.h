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
    const int *out_row;  // null: out row t
    float *out;
    int n_tok, D;
};

enum : int { ACT_SILU = 0, ACT_CLAMP_SWIGLU = 1, ACT_SITU = 2 };

// Launchers (kern_gemv.hip / kern_misc.hip / kern_mfma.hip).  All return hipSuccess or
// the launch error.
// Generic GEMV: any K, any alignment, fmt 0/4/7 (exact reference per-element formula).
hipError_t launch_gemv_generic(int fmt, bool dual, const GemvArgs &a, hipStream_t st);
hipError_t launch_combine(const CombineArgs &a, hipStream_t st);
// n 8-byte words from pinned host memory to device memory by a kernel on st.
hipError_t launch_copy_words(const void *host_src, void *dst, int n, hipStream_t st);
// n <= kArgWords words in the kernel arguments, written to dst by a kernel on st.
constexpr int kArgWords = 448;
struct ArgWords {
    unsigned long long v[kArgWords];
    int n;
};
hipError_t launch_fill_words(const ArgWords &w, void *dst, hipStream_t st);
hipError_t launch_dequant(int fmt, const void *packed, const void *scales, int O, int K,
                          float *w, hipStream_t st);
hipError_t launch_dequant_bf16path(int fmt, const void *packed, const void *scales, int O,
                                   int K, float *w, hipStream_t st);
hipError_t launch_membench(int kind, const void *src, void *dst, size_t bytes, int row16,
                           hipStream_t st);
// MXFP4 activation quantization of n rows of K (row j = x row rows_map[j], or j); planes
// (optional, 8-byte aligned): the quantized values as bf16 rows [n][K] as well, for the
// rows j with pmask[j] != 0 (every row when pmask is null).  n_live (device, optional):
// rows j >= *n_live are left alone (a launch sized for a bound); src_rows >= 0: a source
// row outside [0, src_rows) quantizes as a zero row.
hipError_t launch_quantize_mxfp4(const float *x, int n, int K, uint8_t *codes, uint8_t *scales,
                                 hipStream_t st, const int *rows_map = nullptr,
                                 void *planes = nullptr, const uint8_t *pmask = nullptr,
                                 const int *n_live = nullptr, int src_rows = -1);

// Routing on the device (kern_route.hip): moe_topk per token, and the segments of one
// batched moe_block call.  Bit-exact with the host versions.
constexpr int kRouteMaxExperts = 4096;
hipError_t launch_moe_topk(const float *choice, const float *mix, int n_tok, int n_exp, int k,
                           int *idx, float *wt, hipStream_t st);
hipError_t launch_moe_segments(const int *idx, const float *wt, int n_tok, int topk, int n_exp,
                               int *work, int *eids, int *xoff, int *nr, int *rows, float *rw,
                               int cap_experts, int cap_rows, int *counts, hipStream_t st);
// moe_topk then the segments, on one stream.
hipError_t launch_moe_route(const float *choice, const float *mix, int n_tok, int n_exp, int k,
                            int *idx, float *wt, int *work, int *eids, int *xoff, int *nr,
                            int *rows, float *rw, int cap_experts, int cap_rows, int *counts,
                            hipStream_t st);

// Matrix-core decode path (kern_mfma.hip).  One descriptor per item (up to rmax <= 16
// rows of one expert), built by the host: everything a workgroup needs before its first
// weight load, so one dependent read starts both the weight stream and the activation
// staging.
struct DecDesc {
    const void *w[2];  // the wave's two weight streams: gate and up (dual), down twice
    const void *s[2];  // their scales (int4: f32 [O][K/64]; MXFP4: ue8m0 [O][K/32])
    int jbase;         // first compact row of the item (row of H / Y)
    int nrow;          // rows in the item
    int pad0[2];
    int rows[16];      // dual: input row of item row r; single + fold: row of out
    float wts[16];     // single + fold: combine weight of item row r
    int pad1[20];
};
static_assert(sizeof(DecDesc) == 256, "DecDesc layout");

// A gate/up descriptor compact enough to travel in the kernel arguments, which the
// runtime places in device memory: the workgroups' first read is then an HBM read
// instead of a PCIe round trip to the pinned plan slot.  Used when a launch has at most
// kDecInline items, every offset fits 32 bits and every row index 16 bits.
struct DecDescK {
    const void *w0;          // gate weights
    int off[3];              // up weights, gate scales, up scales: byte offsets from w0
    unsigned short jbase;    // first compact row of the item
    unsigned short nrow;     // rows in the item
    unsigned short rows[16]; // input row of item row r
};
static_assert(sizeof(DecDescK) == 56, "DecDescK layout");
constexpr int kDecInline = 64;
struct DecInline {
    DecDescK d[kDecInline];
};

// Segments of a call on device-resident segments for the gate/up decode kernel that plans
// its own item (k_mfma_dec_seg, the device-resident block at decode shapes): wave 0 of each
// workgroup finds item blockIdx / wgs among the live segments (items of rmax rows in
// segment order, as k_dplan_dec numbers them) and builds its descriptor in LDS at byte
// kd_off; column block 0 of each item writes the item's down descriptor to dn, and
// workgroup 0 the item count and the status.
struct DecSegArgs {
    const void *const *table;  // blob address per expert id (device)
    int n_table;
    long long off[6];          // piece offsets: gate_p gate_s up_p up_s down_p down_s
    const int *counts, *eids, *xoff, *nr, *rows;
    const float *rw;
    int cap_e, cap_rows, S, rmax, cap_items;
    int kd_off;                // LDS byte offset of the descriptor (past the task's LDS)
    DecDesc *dn;               // [cap_items]
    int *n_items;              // [1]
    int *err;                  // 0, or 2: a blob address not 256-byte aligned (skipped)
};

// The gate/up kernel (dual) reads the f32 input rows and splits them into `terms` bf16
// terms in LDS; each wave computes the gate and the up tile of the same 16 columns over
// K / ks and applies the activation in registers (ks > 1: partial sums meet in LDS).  It
// writes H as terms planes [terms][rcap][I] (+ fmt 4 per-16-column partial sums
// hp[I/64][4][rcap]) for the down kernel (single), whose waves compute nt (1 or 2) tiles
// each and write Y [rcap][D] f32 or, with fold, add wts[r] * y into out[rows[r]] by float
// atomics (the top-k combine; out has row stride O).  A workgroup of kDecWaves waves covers
// one item and (kDecWaves / ks) * (dual ? 1 : nt) column tiles of 16.
// Requires fmt 4/7, K % 512 == 0, K % (256 ks) == 0, K / ks <= dec_max_kr(fmt),
// O % (16 * that tile count) == 0, K <= kDecMaxK,
// 16-byte aligned weights and scales (int4) / 8-byte aligned scales (MXFP4), 16-byte
// aligned input rows and LDS (mfma_dec_lds_bytes) <= kDecLdsBudget.
// Waves per decode workgroup.  Eight waves at <= 128 VGPRs let two workgroups share a CU.
constexpr int kDecWaves = 8;
constexpr int kDecThreads = 64 * kDecWaves;
constexpr size_t kDecLdsBudget = 163840 / 2;  // two workgroups per CU
constexpr int kDecStageDual = 4;     // 8-float chunks per thread (rmax * K / 8 <= 4 * threads)
constexpr int kDecStageSingle = 12;  // uint4 per thread (terms * rmax * K / 8 <= 12 * threads)
constexpr int kDecMaxK = 8192;
// Longest K range of one wave: its tiles' scales over the range are held in registers,
// 128 bytes a row (int4: 32 groups of 64; MXFP4: 128 blocks of 32).
inline int dec_max_kr(int fmt) { return fmt == 4 ? 2048 : 4096; }
size_t mfma_dec_lds_bytes(int fmt, int K, int rmax, int terms, int dual, int ks, int nt);
// inl (dual only, optional): the n_items (<= kDecInline) descriptors in the compact form,
// in host memory; copied into the kernel arguments, and desc is not read.
// n_items_dev (optional, not with inl or n_cp): the item count in device memory; n_items
// is then the capacity the grid covers.  seg (dual only, not with inl, n_cp or
// n_items_dev): the gate/up kernel plans its items from the segments (DecSegArgs); desc
// is not read and n_items is the capacity.
hipError_t launch_mfma_dec(int fmt, bool dual, int terms, int ks, int nt, const DecDesc *desc,
                           int n_items, const float *xin, const void *pin, const float *xs,
                           void *pout, float *hp, float *out, int K, int O, int rcap, int rmax,
                           int act, float act_a, float act_b, bool fold, bool pack,
                           const DecDesc *cp_src, DecDesc *cp_dst, int n_cp, hipStream_t st,
                           const DecDescK *inl = nullptr, const int *n_items_dev = nullptr,
                           const DecSegArgs *seg = nullptr);

// Grouped GEMM (kern_gemm.hip), the prefill path: items {expert, r0, nrow, 0} with
// nrow <= 16 * mt (mt in 1, 2, 4, 8, up to gemm_max_mt); one workgroup of 8 waves per
// (item, block of 128 columns of each of gate/up, or 256 columns of down).  Requires
// fmt 4/7, K % 256 == 0, O % 128 (dual) / % 256 (single) == 0, 8-byte aligned weights,
// 16-byte (int4) / 8-byte (MXFP4) aligned scales and 16-byte aligned planes.  Inputs are
// bf16 planes [terms][rcap][K] (int4: K in the 8-block slot order of the decode
// kernel); launch_prep_planes builds them from f32 rows.
// Largest row-tile count per workgroup: 8 (128 rows) with one term, 4 with two, for both
// formats (int4 decodes n - 8 directly and needs no per-row sums).  Larger blocks read an
// expert's weights fewer times; MT = 8 spills at most 5 registers.
inline int gemm_max_mt(int fmt, int terms) { return (void)fmt, terms == 1 ? 8 : 4; }
size_t gemm_lds_bytes(int fmt, int terms, int mt);
// Grouped-GEMM task order (option "gemm_xcd"): 1 (default) = each XCD runs a contiguous
// range of tasks (an item's column blocks share one L2), 0 = task = workgroup index.
void gemm_set_xcd(bool on);
bool gemm_xcd();
// dual with out set: H is written to out as f32 rows [rcap][O] instead of planes to pout.
hipError_t launch_gemm(int fmt, bool dual, int terms, int mt, const ExpertWork *ew,
                       const void *items, int n_items, const void *pin, void *pout, float *out,
                       int K, int O, int rcap, int act, float act_a, float act_b,
                       hipStream_t st, const int *n_items_dev = nullptr);
// The 128-row class of MXFP4 weights with one bf16 term (kern_wide.hip): wide wave tiles
// (option "gemm_wide": 1 = eight waves of 128 rows x 4 tiles of 16 weight rows, 0 = the
// grouped GEMM above).  Same items, planes and outputs as launch_gemm at mt 8; requires
// K % 256 == 0 and O % 256 (dual) / % 512 (single) == 0 (gemm_wide_fits), 16-byte aligned
// weights.  launch_gemm takes this path itself when it fits.
void gemm_set_wide(int v);
int gemm_wide();
bool gemm_wide_fits(bool dual, int K, int O);
hipError_t launch_gemm_wide(bool dual, const ExpertWork *ew, const void *items, int n_items,
                            const void *pin, void *pout, float *out, int K, int O, int rcap,
                            int act, float act_a, float act_b, hipStream_t st,
                            const int *n_items_dev);
// One matrix (w[2], s[2] of *ew1) over input rows [0, nrows) of the planes, in items of
// 16 * mt rows computed in the kernel (a dense linear): out [nrows][O] f32.
hipError_t launch_gemm_rows(int fmt, int terms, int mt, const ExpertWork *ew1, int nrows,
                            const void *pin, float *out, int K, int O, hipStream_t st);
hipError_t launch_prep_planes(int fmt, int terms, const float *x, const int *rows_map, int R,
                              int K, int rcap, void *planes, hipStream_t st,
                              const int *n_live = nullptr, int src_rows = -1);

// f32-weight GEMMs on the matrix cores (kern_f32.hip): fmt 0 moe_block, router scores,
// fmt 0 linears.  Items {expert, r0, nrow, 0} of <= 16 * mt rows (mt 1, 2, 4), or, with
// items null, one expert *ew1 over rows [0, nrows_all) in blocks of 16 * mt.  dual: gate
// w[0] and up w[1] -> act -> out [rcap][O]; single: w[mi] -> out.  Input row of compact
// row j: in_rows[j] (or j).  Requires K % 16 == 0, O % 16 (dual) / % 32 (single) == 0,
// 16-byte aligned weight and input rows.
bool f32mm_fits(bool dual, int K, int O);
// i8 (single only): w[mi] holds int8 rows [O][K] and s[mi] their f32 row scales (QuantMat
// fmt 8); 4-byte aligned rows.
hipError_t launch_f32mm(bool dual, int mt, const ExpertWork *ew, const void *items, int n_items,
                        const ExpertWork *ew1, int nrows_all, const float *in,
                        const int *in_rows, float *out, int mi, int K, int O, int act,
                        float act_a, float act_b, hipStream_t st, bool i8 = false);
// Router tail: scores -> sigmoid in place (the mix), choice = mix + bias; then w *= rscale.
hipError_t launch_route_tail(float *scores, const float *bias, float *choice, int n, int E,
                             hipStream_t st);
hipError_t launch_scale(float *w, size_t count, float rscale, hipStream_t st);
// y[r] = rmsnorm(x[r]) * w (w may be null), rows of n.
hipError_t launch_rmsnorm(const float *x, const float *w, float *y, int rows, int n, float eps,
                          hipStream_t st);

// Native MXFP4 GEMM (kern_fp4.hip): v_mfma_scale_f32_16x16x128_f8f6f4 with e2m1 activations
// (codes [rcap][K/2] + ue8m0 scales [rcap][K/32], from launch_quantize_mxfp4) against the
// MXFP4 weights as stored.  Items and workgroup tiling as launch_gemm (mt 4, 8 and 16; an
// expert's row blocks run column block by column block);
// the dual projection writes H = act(gate, up) as f32 [rcap][O], the single one Y.
// Requires K % 256 == 0, O % 128 (dual) / % 256 (single) == 0, 16-byte aligned weights,
// 8-byte aligned scales.
constexpr int kFp4MaxMt = 16;
// row classes of a grouped-GEMM call: 16, 32, 64, 128 and (native FP4 only) 256 rows
constexpr int kGemmClasses = 5;
// Row classes of a native-MXFP4 call (option fp4act) up to this one take the bf16 grouped
// GEMM on bf16 copies of the quantized activations instead (launch_quantize_mxfp4's
// planes): the same exact products, streamed faster (c4: gate/up 16-row class 794 ->
// ~680 us, 32-row 347 -> ~270 us).
constexpr int kFp4BfMaxMt = 2;
size_t fp4_lds_bytes(int mt);
// n_items_dev (optional): the item count in device memory, n_items the bound the grid
// covers (workgroups past the count exit).
hipError_t launch_gemm_fp4(bool dual, int mt, const ExpertWork *ew, const void *items,
                           int n_items, const uint8_t *acode, const uint8_t *ascale, float *hout,
                           float *out, int K, int O, int rcap, int act, float act_a, float act_b,
                           hipStream_t st, const int *n_items_dev = nullptr);

// ---- device-planned calls (kern_dplan.hip) ---------------------------------------

// k_dplan: expert work, row liveness and grouped-GEMM items of a call whose segments are
// in device memory.
struct DPlanArgs {
    const void *const *table;  // blob address per expert id (device)
    int n_table;
    long long off[6];  // piece offsets: gate_p gate_s up_p up_s down_p down_s
    const int *counts;  // [0] segments, [1] compact rows
    const int *eids, *xoff, *nr;
    int cap_e, cap_rows;
    int bm;            // rows per full block (16 * top class)
    int top;           // index of the top class (log2 of its MT)
    int split64;       // remainders of 33-64 rows as two items of the 32-row class
    ExpertWork *ew;    // [cap_e]
    int4 *items;       // class c at items + item_base[c] ({expert, r0, nrow, 0})
    int item_base[kGemmClasses], item_cap[kGemmClasses];
    int *n_items;      // [kGemmClasses]
    unsigned char *row_ok;  // [cap_rows]
    int *err;          // 0; 1 = a class overflowed its capacity (the bounds exclude it),
                       // 2 = a blob address not 256-byte aligned (that expert skipped)
};

// The combine's per-out-row lists of such a call (tok_ptr in cnt after the scan).
struct CsrArgs {
    const int *counts;  // [1] compact rows
    int cap_rows, S;
    const int *rows;
    const float *rw;
    const unsigned char *row_ok;
    int *cnt;      // [S + 1]: per out row, then (after the scan) tok_ptr
    int *cursor;   // [S]
    int *ent_row;  // [cap_rows]
    float *ent_w;  // [cap_rows]
};

// The decode-kernel plan of such a call (k_dplan_dec): per segment of live expert, items
// of up to rmax rows with a gate/up and a down descriptor each.
struct DPlanDecArgs {
    const void *const *table;
    int n_table;
    long long off[6];
    const int *counts, *eids, *xoff, *nr;
    const int *rows;     // [cap_rows] out row of each compact row
    const float *rw;     // [cap_rows] combine weights
    int cap_e, cap_rows, S;
    int rmax;            // rows per item (1..16)
    int cap_items;       // descriptors the buffers hold (a bound for any valid input)
    DecDesc *gu, *dn;    // [cap_items] each
    int *n_items;        // [1]
    unsigned char *row_ok;  // [cap_rows] (for the ordered combine's lists)
    int *err;            // as DPlanArgs::err
};

hipError_t launch_dplan(const DPlanArgs &a, hipStream_t st);
hipError_t launch_dplan_dec(const DPlanDecArgs &a, hipStream_t st);
hipError_t launch_dcsr(const CsrArgs &a, hipStream_t st);

}  // namespace mvllm_hip
