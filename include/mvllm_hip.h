/*
 * mvllm_hip.h -- C ABI of the MI355X (gfx950) routed-expert moe_block backend.
 *
 * This is the drop-in boundary.  Every entry point takes plain pointers and sizes
 * (no torch or C++ types) and names the reference interface it replaces.  The
 * reference is micro-vllm; paths below are relative to its tree.
 *
 * Return convention (same as the reference's device ops, src/gpu/metal_ops.hpp:9-10):
 * 1 = ran, 0 = "use the host kernel" (bad arguments, no device, or a HIP error;
 * mvllm_hip_last_error() then says which).  No entry point throws.
 *
 * Weight formats (fmt), byte-identical to src/quant:
 *   0  f32 row-major [O, K]                                  (src/quant/quant.cpp:156-168)
 *   4  int4-g64: nibbles [O, (K+1)/2], low nibble = even k, value (n-8)*scale;
 *      f32 scales [O, ceil(K/64)]                            (src/quant/quant.cpp:203-228)
 *   7  MXFP4: e2m1 nibbles [O, (K+1)/2]; ue8m0 scale bytes [O, ceil(K/32)], passed
 *      through the const float* slots                        (src/quant/quant.cpp:298-321)
 * For gate/up O = Iinter, K = D; for down O = D, K = Iinter.
 */
#ifndef MVLLM_HIP_H
#define MVLLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- lifecycle: metal_ops::init / shutdown / available / backend_name
 *      (src/gpu/metal_ops.hpp:15-18); device selection gpu::select
 *      (src/gpu/backend.cpp:92-113) for Device::Hip. ------------------------- */

/* Selects HIP device `device` and creates the backend's streams.  1 ok, 0 no device. */
int mvllm_hip_init(int device);
/* Waits for outstanding work, frees device memory the backend owns. */
void mvllm_hip_shutdown(void);
/* 1 after a successful init. */
int mvllm_hip_available(void);
/* "hip" -- the string the engine's info tag shows as coli=hip
 * (src/model/glm53.cpp:407-413, src/model/kimi_k3.cpp:740-746). */
const char *mvllm_hip_name(void);
/* Text of the last failure on this thread's most recent call ("" if none). */
const char *mvllm_hip_last_error(void);

/* ---- the hot path ---------------------------------------------------------- */

/* Drop-in for metal_ops::moe_block (src/gpu/metal_ops.hpp:99-108,
 * src/gpu/metal_ops.cpp:448-460).  All pointers are caller-owned HOST memory,
 * exactly as in the reference: per expert e, nr[e] rows of xg starting at row
 * xoff[e] go through gate/up -> act -> down, and out[rows[j]] += rw[j] * y[j]
 * in expert order (always: this entry never uses the unordered atomic combine, so
 * equal inputs give bit-identical out from run to run).
 * act: 0 Silu, 1 ClampSwiGLU(act_a), 2 SiTU(act_a, act_b).
 * Validation and skip rules are the reference's (nb<1, D<1, !out, !xg, fmt not in
 * {0,4,7}, !xoff, !nr -> 0; null expert pointers or Iinter<1 consume rows without
 * writing; rows outside [0,S) (S>0) are skipped).  Expert weights that were
 * promoted with mvllm_hip_promote are read from HBM; others are copied in.
 * Synchronous: out holds the result on return. */
int mvllm_hip_moe_block(int nb, int D, int Iinter, int fmt, int qgs, const void *const *g,
                        const void *const *u, const void *const *d, const float *const *gs,
                        const float *const *us, const float *const *ds, const float *xg,
                        const int *xoff, const int *nr, const int *rows, const float *rw,
                        float *out, int S, int act, float act_a, float act_b);

/* Same contract for GPU-resident callers (no reference counterpart beyond
 * moe_block itself, src/gpu/metal_ops.hpp:104-108): the six pointer arrays and
 * xoff/nr/rows/rw are HOST arrays; the weights and scales they point to, xg
 * ([rows, D] f32) and out ([S, D] f32, accumulated) are DEVICE pointers.
 * Summation order of out: decode-shaped calls (every expert <= 16 rows, matrix-core
 * decode kernels) fold the combine into the down kernel with float atomics by default,
 * so out's rows are summed in an arbitrary order and may differ in the last bits from
 * run to run; option "combine_ordered" = 1 applies the reference's expert order
 * instead.  Every other call uses the reference's order.
 * Work is enqueued on `stream` (a hipStream_t; NULL = the null stream) and the
 * call returns without waiting.  Requires S > 0 (out's row count).  Calls are ordered
 * after each other across streams (they share scratch): a call on another stream than
 * the previous one first marks the previous stream's end, so keep that stream alive
 * until then (if it is gone, the call drains the device instead). */
int mvllm_hip_moe_block_dev(int nb, int D, int Iinter, int fmt, int qgs, const void *const *g,
                            const void *const *u, const void *const *d,
                            const float *const *gs, const float *const *us,
                            const float *const *ds, const float *xg, const int *xoff,
                            const int *nr, const int *rows, const float *rw, float *out, int S,
                            int act, float act_a, float act_b, void *stream);

/* No counterpart in the reference.  For callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc):
 * mvllm_hip_moe_block_dev with the same arguments, results and ordering rules, except
 * that it allocates no device or pinned memory (hipMalloc, hipHostMalloc, hipFree or
 * the like; host-side planning still uses the C++ heap).  Its device scratch is one
 * 48 MiB array per device, held from mvllm_hip_init until the process ends: the plan's
 * device copy (at most 256 KiB, about 450 decode items) and the call's buffers (at most
 * 47.75 MiB; decode calls need about R * Iinter * 4.1 bytes with the default
 * arithmetic, or R * (Iinter * 4.1 + D * 4) with combine_ordered, grouped-GEMM calls
 * R * (2 * D + 2 * Iinter + 4 * D), for R routed rows).  A call beyond either limit
 * returns 0 with a message in mvllm_hip_last_error and enqueues nothing.  Every call on
 * a device shares that device's array and the array keeps the last call's contents:
 * calls ordered by this library (one stream, or the library's own ordering across
 * streams) are safe; calls that overlap on one device from outside that ordering race.
 * Option "timing" is ignored by this entry. */
int mvllm_hip_moe_block_dev_noalloc(int nb, int D, int Iinter, int fmt, int qgs,
                                    const void *const *g, const void *const *u,
                                    const void *const *d, const float *const *gs,
                                    const float *const *us, const float *const *ds,
                                    const float *xg, const int *xoff, const int *nr,
                                    const int *rows, const float *rw, float *out, int S, int act,
                                    float act_a, float act_b, void *stream);

/* Options (key, value), process-wide; returns 1 if the key and value are accepted.
 *   "mode"   how activations enter the bf16 matrix cores (weights are always decoded
 *            exactly; products and sums are f32):
 *            0  default: decode-shaped calls split each f32 activation into 2 bf16 terms
 *               (hi + lo; 2^-17 relative); the prefill grouped GEMM uses 1 term (bf16)
 *            1  3 terms in the decode kernels (the activation exactly), 2 in the GEMM
 *            2  1 bf16 term everywhere
 *   "gemm"   0 = automatic (the grouped GEMM when some expert has more than 16 rows, or
 *            the decode kernels do not fit the shape), 1 = grouped GEMM whenever it
 *            applies, 2 = never.
 *   "fp4act" 1 = MXFP4 experts (fmt 7) run on native MXFP4 activations: the GEMM inputs
 *            (x, then h) are quantized exactly as fp4_activation_qdq with block 32
 *            (src/quant/native_act.cpp:159-179) and fed with the weights as stored to the
 *            scaled FP4 matrix cores.  Changes the numbers (activation quantization).
 *            Weight scale bytes 0 and 255 keep the reference's +0 and +inf: a wave of the
 *            scaled-FP4 kernel that meets one computes its outputs element by element.
 *   "gemm_wide" 1 (default) = the 128-row blocks of MXFP4 experts in the one-term grouped
 *            GEMM run a kernel with wide wave tiles (8 waves of 128 rows x 64 weight
 *            columns), 0 = the grouped GEMM's own 128-row class.  Same products; sums in
 *            another order.
 *   "combine_ordered" 1 = decode calls of mvllm_hip_moe_block_dev also run the separate
 *            combine kernel, which applies out[t] += w * y in the reference's expert order
 *            (bit-exact given the same expert outputs); by default they fold the combine
 *            into the down kernel with float atomics (same products, any summation
 *            order).  mvllm_hip_moe_block always uses the ordered combine.
 *   "timing" 1 = record per-phase HIP events; read them with mvllm_hip_stats.
 *   "dec_ks" 0 = automatic; 1, 2, 4 or 8 forces the split of K across waves.
 *   "dec_inline" 1 (default) = the decode gate/up launch carries its descriptors in
 *            its kernel arguments (at most 64 items; same results); 0 = it reads them
 *            from the pinned plan slot.
 *   "dequant_path" 1 = mvllm_hip_dequant decodes through the matrix-core operand path.
 * fmt 0 experts (f32 weights, the shared experts) run on the f32 matrix cores when
 * D % 16 == 0, Iinter % 32 == 0, D % 32 == 0 and rows are 16-byte aligned.  Shapes the
 * matrix-core kernels do not take (D or Iinter not a multiple of 256 for fmt 4/7, odd
 * fmt 0 shapes, misaligned pointers) run an exact element-wise f32 kernel instead. */
int mvllm_hip_set_option(const char *key, long long value);

/* ---- segment construction: moe_union_ids (src/model/ops.cpp:1082-1099) and the
 *      per-expert gather of moe_layer_n (src/model/glm53.cpp:1938-1971,
 *      src/model/kimi_k3.cpp:2009-2050).  Host integer work, bit-exact. ------- */

/* Sorted unique non-negative ids of idx[n_tok*topk], at most out_cap. */
int mvllm_moe_union_ids(const int *idx, int n_tok, int topk, int *out, int out_cap);

/* Arguments for ONE batched moe_block call that reproduces moe_layer_n's
 * per-expert loop: eids[nb] ascending; expert i owns rows [xoff[i], xoff[i]+nr[i]);
 * row j is token rows[j] (also its gather index into the token matrix) with weight
 * rw[j] = sum of that token's top-k weights for the expert (rows whose sum is 0
 * are dropped, as the reference does).  Returns nb, or -1 if a capacity is short;
 * *n_rows receives the total row count. */
int mvllm_moe_segments(const int *idx, const float *wt, int n_tok, int topk, int *eids,
                       int *xoff, int *nr, int *rows, float *rw, int cap_experts, int cap_rows,
                       int *n_rows);

/* ---- the same routing on the device, for callers that keep the router output in HBM:
 *      moe_topk (src/model/ops.cpp:860-889) of every token, and mvllm_moe_segments.
 *      Bit-exact with the host functions.  Enqueued on `stream` (NULL: the null stream);
 *      both return 1 when enqueued, 0 on bad arguments (mvllm_hip_last_error). ---- */

/* choice, mix (or NULL: weights from choice): device f32 [n_tok][n_exp]; idx int32 and
 * wt f32 [n_tok][k] on the device, row t equal to moe_topk(choice + t*n_exp, n_exp, k,
 * ..., mix ? mix + t*n_exp : NULL).  1 <= k <= 64, k <= n_exp <= 4096; scores must not
 * be NaN (the reference's sort has no order for them). */
int mvllm_hip_moe_topk_dev(const float *choice, const float *mix, int n_tok, int n_exp, int k,
                           int *idx, float *wt, void *stream);

/* mvllm_moe_segments of device idx/wt [n_tok][topk] (ids < n_exp; negative ids are
 * skipped as the reference does).  Device outputs eids/xoff/nr [cap_experts], rows/rw
 * [cap_rows] and counts int32[2] = {nb, n_rows}, or {-1, -1} when cap_rows is short or
 * an id >= n_exp (the other outputs are then undefined).  The union keeps its
 * cap_experts smallest ids, as mvllm_moe_union_ids does.  work: device int32 scratch of
 * 2 * n_exp + 1 entries; calls that share a work buffer must not overlap. */
int mvllm_hip_moe_segments_dev(const int *idx, const float *wt, int n_tok, int topk, int n_exp,
                               int *work, int *eids, int *xoff, int *nr, int *rows, float *rw,
                               int cap_experts, int cap_rows, int *counts, void *stream);

/* Both in one call: mvllm_hip_moe_topk_dev, then mvllm_hip_moe_segments_dev of its
 * idx / wt (same arguments, same results; five launches). */
int mvllm_hip_moe_route_dev(const float *choice, const float *mix, int n_tok, int n_exp, int k,
                            int *idx, float *wt, int *work, int *eids, int *xoff, int *nr,
                            int *rows, float *rw, int cap_experts, int cap_rows, int *counts,
                            void *stream);

/* moe_block on segments that are already in device memory, with no host round trip:
 * the per-expert loop of the engines' batched MoE (src/model/glm53.cpp:1938-1992) fed by
 * mvllm_hip_moe_route_dev / mvllm_hip_moe_segments_dev, whose outputs it reads as they
 * are: counts[0] = segments, counts[1] = compact rows; segment i is expert eids[i] with
 * compact rows [xoff[i], xoff[i] + nr[i]); compact row j is token rows[j] of x with
 * weight rw[j].  Expert e's weights are the blob at table[e] (device array of n_table
 * blob addresses in the reference blob layout, 256-byte aligned: a slab's table, or the
 * HBM tier's blobs); an id outside [0, n_table), a null entry or a misaligned one
 * consumes its rows without writing (the reference's null-expert rule,
 * src/gpu/metal_ops.cpp:291-296).  x [S][D] token rows, out [S][D] accumulated with
 * += in expert order (src/gpu/metal_ops.cpp:328-339).  The plan is built by kernels;
 * launches are sized for the caps (cap_experts segments, cap_rows compact rows) and their
 * surplus workgroups exit.  Two paths:
 *   S <= 16 (decode): the decode kernels of mvllm_hip_moe_block_dev's decode-shaped calls
 *     (two bf16 terms per activation; mode 1 three, mode 2 one) on items of up to S rows
 *     of one expert (fewer where the activations of S rows do not fit the kernels), and, as there, the combine folded into the down kernel as float
 *     atomics (out row sums in any expert order) unless option combine_ordered is 1;
 *     two launches (the gate/up kernel plans its own items).  Option gemm=1 takes the grouped path instead.
 *   otherwise: the grouped GEMM with two bf16 terms per activation (2^-17) when cap_rows
 *     <= 256, one above (mode option 1: always two, 2: always one), and the ordered
 *     combine on lists built by kernels.
 * With option fp4act, MXFP4 experts (fmt 7) take the native-MXFP4 grouped path at every
 * size, as mvllm_hip_moe_block_dev does (x and H quantized as fp4_activation_qdq; blocks
 * of up to 256 rows; the same results as that call on the same segments).
 * fmt 4 / 7, D and Iinter multiples of 256, 1 <= S <= 65535.  status (device int, may be
 * NULL) receives 0; 2 when a blob address was not 256-byte aligned (that expert skipped);
 * 1 when segments whose rows overlap made more work items than the caps bound (the
 * surplus dropped; routing output never does).  Enqueued on `stream`; 1 enqueued. */
int mvllm_hip_moe_block_routed_dev(int D, int Iinter, int fmt, const void *const *table,
                                   int n_table, const int *counts, const int *eids,
                                   const int *xoff, const int *nr, int cap_experts,
                                   const int *rows, const float *rw, int cap_rows,
                                   const float *x, float *out, int S, int act, float act_a,
                                   float act_b, int *status, void *stream);

/* ---- the steps either side of the block (device, enqueued on `stream`; 1 = enqueued,
 *      0 = bad arguments, see mvllm_hip_last_error) --------------------------------- */

/* The router of one MoE layer for n_tok token rows: cpu_route (src/gpu/metal_ops.cpp:
 * 213-231) of every row -- scores = x . w^T (f32 [n_exp][D] weights, f32 matrix cores),
 * mix = sigmoid(scores), choice = mix + bias (bias NULL: none), moe_topk(choice, mix),
 * weights * rscale.  x [n_tok][D], workspaces scores and choice [n_tok][n_exp] f32 (scores
 * returns the mix), idx / wt [n_tok][k] as mvllm_hip_moe_topk_dev writes them; they feed
 * mvllm_hip_moe_segments_dev.  The dot products are f32 in another order than the
 * reference's sequential sum and the sigmoid uses the device's expf, so a score may
 * differ from the host's by a few ulp: picks agree except where the k-th and (k+1)-th
 * choices are that close.  D % 16 == 0, n_exp % 32 == 0 (<= 4096), 1 <= k <= min(64,
 * n_exp), x and w 16-byte aligned. */
int mvllm_hip_router_dev(const float *x, const float *w, const float *bias, int n_tok, int D,
                         int n_exp, int k, float rscale, float *scores, float *choice,
                         int *idx, float *wt, void *stream);

/* A dense linear y[n][O] = x[n][K] . W^T, as QuantMat::gemm (src/quant/weight.cpp:47-64):
 * K3's latent down / up projections around the routed block (src/model/kimi_k3.cpp:
 * 2003-2006, 2074-2090).  fmt 0: f32 W [O][K] on the f32 matrix cores (K % 16, O % 32,
 * 16-byte aligned rows); fmt 4 / 7: W codes [O][K/2] with scales as in moe_block, the
 * input rows as two bf16 terms (2^-17 relative) on the bf16 matrix cores (K % 256,
 * O % 256); fmt 8: QuantMat's int8 rows W [O][K] with f32 row scales [O]
 * (quant::matmul_int8_row, src/quant/quant.cpp:255-268; MVLLM_DENSE_BITS=8), each code
 * exact in f32 on the f32 matrix cores and the row scale applied once to the finished
 * sum (K % 16, O % 32, 4-byte aligned codes and scales, 16-byte aligned x).  Calls on
 * one stream, or ordered by the caller: the int4 / MXFP4 forms share one input buffer
 * (a call on another stream than the previous one waits for it). */
int mvllm_hip_linear_dev(int fmt, const void *w, const void *scales, int O, int K,
                         const float *x, int n, float *y, void *stream);

/* y[r] = rmsnorm(x[r]) with weight w (NULL: none), rows of n: quant::rmsnorm
 * (src/quant/quant.cpp:384-398), the lat_n norm of K3's routed output
 * (src/model/kimi_k3.cpp:2074-2079).  The sum of squares is f32 in another order. */
int mvllm_hip_rmsnorm_dev(const float *x, const float *w, float *y, int rows, int n, float eps,
                          void *stream);

/* Expert blob geometry (byte offsets of the six pieces inside one expert blob):
 * fmt 4 = GLM gate_p|gate_s|up_p|up_s|down_p|down_s (src/model/glm53.cpp:56-78,
 * 116-132); fmt 7 = K3 w1p|w1s|w2p|w2s|w3p|w3s with gate=w1, down=w2, up=w3
 * (src/model/kimi_k3.cpp:83-102, 132-159).  off[6] = gate_p, gate_s, up_p, up_s,
 * down_p, down_s.  Returns the blob size in bytes, or -1 for a bad fmt/shape. */
long long mvllm_expert_geom(int fmt, int D, int Iinter, long long off[6]);

/* ---- expert containers -> device slabs --------------------------------------- */

/* Where each routed expert's six pieces lie in the safetensors containers of `dir`
 * (host only, no device).  Replaces the expert registration of the engines' loaders:
 * src/model/glm53.cpp:1829-1871 (fmt 4: "<prefix>layers.<L>.mlp.experts.<e>.
 * {gate,up,down}_proj.weight" U8/I8 codes + ".qs" f32 scales) and
 * src/model/kimi_k3.cpp:1881-1934 (fmt 7: "<prefix>model.layers.<L>.block_sparse_moe.
 * experts.<e>.w{1,2,3}.weight_{packed,scale}"), over the container reader of
 * src/io/safetensors.cpp (st_open_dir: every "*.safetensors" file in name order, a name
 * resolving to the first file that holds it).  Each piece's byte count must equal the blob
 * geometry's (mvllm_expert_geom for D, Iinter), as the reference requires.  For layers
 * [layer0, layer1) and experts [0, n_experts), piece k of blob b = (L - layer0) *
 * n_experts + e (k in blob order: GLM gate_p gate_s up_p up_s down_p down_s, K3 w1p w1s
 * w2p w2s w3p w3s) is file[6b+k] (index into the sorted file list, written to `paths`
 * one path a line when paths is not NULL), absolute byte offset[6b+k], bytes[6b+k].
 * Returns the number of files, or -1 with the reference's message in err
 * ("glm53 expert pieces missing or wrong size at L<L> E<e>", ...). */
int mvllm_st_expert_pieces(const char *dir, const char *prefix, int fmt, int D, int Iinter,
                           int layer0, int layer1, int n_experts, int *file, long long *offset,
                           long long *bytes, char *paths, long long paths_cap, char *err,
                           long long err_cap);

/* Reads those pieces into one device allocation: blob b at base + b * stride (stride =
 * the blob size rounded up to 256 bytes), its six pieces back to back in the blob
 * layout (so the blob address plus mvllm_expert_geom's offsets give the six pointers of
 * moe_block), and a device table of the blob addresses (const void *[n_blobs], indexed
 * (L - layer0) * n_experts + e).  The ExpertStore reads the same pieces into pinned host
 * slots on demand (src/store/expert_store.cpp); this places a layer range in HBM at
 * once.  File reads overlap the host-to-device copies (two pinned staging buffers);
 * synchronous.  Returns a handle > 0, or 0 (see mvllm_hip_last_error). */
long long mvllm_hip_slab_load(const char *dir, const char *prefix, int fmt, int D, int Iinter,
                              int layer0, int layer1, int n_experts);
/* The slab's device base, device table, blob stride and size, and blob count.  1 ok. */
int mvllm_hip_slab_info(long long slab, void **base, void **table, long long *stride,
                        long long *blob_bytes, int *n_blobs);
/* Waits for the device, frees the slab.  1 ok, 0 unknown handle. */
int mvllm_hip_slab_free(long long slab);

/* ---- HBM expert residency (the LRU tier in front of ExpertStore,
 *      src/store/expert_store.hpp:71-175).  Blobs are keyed by (layer, eid). -- */

/* Page-locked host memory for ExpertStore slots (replaces aligned_alloc_pages,
 * src/io/file_io.cpp:95, so promotion copies are truly asynchronous).  NULL (with the
 * error text set) when the runtime refuses, e.g. without a device: the caller keeps its
 * own allocator then. */
void *mvllm_hip_host_alloc(size_t bytes);
/* Frees a block from mvllm_hip_host_alloc: 1.  Any other pointer (NULL included) is left
 * alone: 0, so a caller with a fallback allocator frees it with that one. */
int mvllm_hip_host_free(void *p);

/* Sets the HBM budget of the expert tier (bytes; default 64 GiB). */
int mvllm_hip_set_expert_budget(size_t bytes);

/* Starts an asynchronous copy of one expert blob (host_blob, bytes) into HBM on
 * the backend's copy stream, evicting least-recently-used blobs when the budget
 * is full.  Later moe_block calls whose expert pointers fall inside
 * [host_blob, host_blob+bytes) read the HBM copy once the copy's event has
 * completed (the compute stream waits on it).  Already resident: only bumps LRU.
 * 1 ok, 0 failure. */
int mvllm_hip_promote(const void *host_blob, size_t bytes, int layer, int eid);

/* Drops the HBM copy of (layer, eid); call it when ExpertStore reuses the slot
 * (its REPIN / evict path, src/store/expert_store.cpp:350-405).  1 if found. */
int mvllm_hip_evict(int layer, int eid);

/* Device address of a resident blob (NULL if absent); waits for its copy. */
void *mvllm_hip_resident_ptr(int layer, int eid);

/* The store's prefetch path (ExpertStore::prefetch / prefetch_one_async,
 * src/store/expert_store.cpp:73-91, 416-456): n blobs (layers[i], eids[i]) that the RAM
 * tier holds at host_blobs[i] (bytes[i]) start their copies into HBM on the copy stream,
 * as mvllm_hip_promote, without waiting; resident ones only move up the LRU.  A layer's
 * experts prefetched while the previous layer computes are in HBM when its block runs.
 * Returns the number of copies enqueued, or -1 (see mvllm_hip_last_error). */
int mvllm_hip_prefetch(int n, const int *layers, const int *eids, const void *const *host_blobs,
                       const size_t *bytes);

/* The store's REPIN path (ExpertStore::take_repin, src/store/expert_store.cpp:305-316,
 * 524-538): the RAM tier evicted these experts (layer_eid = n pairs layer, eid), so their
 * host slots now hold other experts.  Their HBM copies stay resident (reachable by
 * (layer, eid): mvllm_hip_resident_ptr, mvllm_hip_tier_table) but host pointers no longer
 * map to them.  Returns how many resident blobs were unlinked, or -1. */
int mvllm_hip_repin(int n, const int *layer_eid);

/* The store's slot reuse (ExpertStore::load_into evicting a slot for another expert,
 * src/store/expert_store.cpp:300-318): call before the slot [host_lo, host_lo + bytes)
 * is rewritten.  Waits until every promotion copy from that range has finished, then
 * unlinks the HBM blobs mapped to it as mvllm_hip_repin does.  Returns the number
 * unlinked, or -1.  (The moe_block host entry's own miss copies finish before it
 * returns.) */
int mvllm_hip_host_reuse(const void *host_lo, size_t bytes);

/* A layer's blob table for mvllm_hip_moe_block_routed_dev: table_dev[e] (device array of
 * n_experts entries) = the HBM address of resident (layer, e) or NULL, written on
 * `stream`, which first waits for every promotion enqueued so far (so prefetched experts
 * are complete when the block reads them).  *n_resident (may be NULL) = entries that are
 * not NULL.  Each table is closed by one mvllm_hip_tier_table_done(layer, stream) after
 * the compute that reads it: until the layer's last open table is closed, a blob of the
 * layer that is dropped meanwhile (evicted by a concurrent promotion) keeps its device
 * block, and a later copy into the block waits for those readers.  n_experts <= 8192.
 * 1 ok. */
int mvllm_hip_tier_table(int layer, int n_experts, void **table_dev, int *n_resident,
                         void *stream);
/* Marks the end of the layer's table readers on `stream` (see above).  1 ok. */
int mvllm_hip_tier_table_done(int layer, void *stream);

/* Counters since init (or the last reset): index
 *  0 moe_block calls      1 rows computed        2 H2D bytes (weights)
 *  3 H2D bytes (acts/out) 4 D2H bytes            5 promotions
 *  6 resident hits        7 misses (copied in)   8 evictions
 *  9 kernel ms gate/up    10 kernel ms down      11 kernel ms combine
 *  12 kernel ms preparing GEMM inputs (the grouped GEMM's bf16 planes of x, or the
 *     MXFP4 quantization of x and of H)
 *  13 launches gate/up    14 launches down
 *  15 host ms spent inside the moe_block entry points (plan building, argument
 *     marshalling and launches; for mvllm_hip_moe_block also the copies and the wait),
 *     including 16
 *  16 host ms of 15 spent blocked until the device finished earlier calls whose pinned
 *     plan slots are reused (a host running ahead of the device waits there)
 *  17 (gauge) device bytes the HBM tier holds for blobs: resident plus parked; kept
 *     within mvllm_hip_set_expert_budget
 *  18 (gauge) of 17, the blocks of blobs dropped while their layer's tier tables are
 *     open, held until mvllm_hip_tier_table_done recycles them
 *  19 host ms of 15 spent in mvllm_hip_moe_block_dev(_noalloc) before its first kernel
 *     launch: the plan, the call's configuration, buffers and the plan's upload (the
 *     rest of 15 is the launches)
 * Kernel times are filled only with option "timing"=1.  Returns the count written
 * (<= n). */
int mvllm_hip_stats(double *vals, int n);
void mvllm_hip_stats_reset(void);

/* ---- checking aids (no reference counterpart: they expose the device's view
 *      of the quantized formats so tests can pin it bit for bit) ------------ */

/* Dequantizes one device matrix to f32 [O, K] on the device exactly as the
 * kernels see it: fmt 4 (n-8)*scale, fmt 7 lut[n]*2^(e-127) with e=0 -> +0 and
 * e=255 -> +inf (src/quant/quant.hpp:13-20).  Synchronous.  1 ok. */
int mvllm_hip_dequant(int fmt, const void *packed_dev, const void *scales_dev, int O, int K,
                      float *w_dev);

/* The bf16 planes the matrix-core paths feed from f32 rows, exactly as the device forms
 * them (the same conversion, split_terms, serves the decode kernels' activations and H):
 * x_dev [n, K] f32 -> planes_dev [terms][n][K] bf16 bit patterns (uint16), plane 0 =
 * bf16_round(x) (src/quant/bf16.cpp:9-20, round to nearest even), plane 1 = bf16_round of
 * x - plane 0 (0 when plane 0 is not finite), plane 2 = the next remainder.  fmt 4 stores
 * each 8-element block in the int4 operand order (elements 0 2 4 6 1 3 5 7), fmt 7 in
 * natural order.  terms 1..3, K a multiple of 8.  Synchronous.  1 ok. */
int mvllm_hip_bf16_planes(int fmt, int terms, const float *x_dev, int n, int K,
                          uint16_t *planes_dev);

/* MXFP4 activation quantization on the device, bit-exact with fp4_activation_qdq
 * (src/quant/native_act.cpp:159-179) for block 32: rows x [n, K] f32 ->
 * codes [n, K/2] packed e2m1 (low nibble = even k) + scales [n, K/32] ue8m0, and,
 * when planes_dev is not NULL, the quantized values themselves as bf16 [n, K] (each is
 * exact in bf16: the reference's QDQ output rounded to nothing).  K must be a multiple
 * of 32.  Synchronous.  1 ok. */
int mvllm_hip_quantize_mxfp4(const float *x_dev, int n, int K, uint8_t *codes_dev,
                             uint8_t *scales_dev, uint16_t *planes_dev);

/* Memory-system probe used to calibrate the roofline (no reference counterpart):
 * kind 0 streams `bytes` of src_dev with coalesced 16-byte reads, kind 1 copies them to
 * dst_dev, kinds 2..6 walk rows of row_bytes (a multiple of 1024) the way a wave walks
 * expert weight rows: 2 = 16 rows x 32 B per load (8-byte lanes), 3 = 32 rows x 32 B,
 * 4 = 16 rows x 64 B, 5 = 4 rows x 256 B, 6 = 1 row x 1 KB (16-byte lanes); dst_dev
 * receives a sink word.
 * Runs `reps` times on the backend's stream, after one untimed warm-up pass when
 * reps > 1 (reps == 1 times a single cold pass); *ms_per_rep gets the mean time.  1 ok. */
int mvllm_hip_membench(int kind, const void *src_dev, void *dst_dev, size_t bytes, int row_bytes,
                       int reps, double *ms_per_rep);

#ifdef __cplusplus
}
#endif

#endif /* MVLLM_HIP_H */
