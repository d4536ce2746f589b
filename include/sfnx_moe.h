/*
 * sfnx_amd: the quantized mixture-of-experts hot path for MI355X (gfx950), behind a C ABI.
 *
 * Every entry point is stream-asynchronous on `st` (a hipStream_t passed as void*, null = the default stream), takes
 * device pointers only, allocates nothing, never synchronises the host and is safe to capture into a HIP graph
 * (unless its comment says otherwise).  Each returns 0 on success or a negative status; sfnx_last_error() then holds
 * the message (thread-local).  The C++ header sfnx_amd/include/sfnx/kernels.hpp wraps these under the reference
 * engine's own names, throwing std::runtime_error as the reference's wrappers do (src/kernels.cu:31-34).
 *
 * Citations are johnfink8/sfnx paths; each entry point names the reference interface it replaces.
 *
 * Weight matrices are the "planar" store (sfnx_store_pack): per matrix of R rows x C columns,
 *   Q4_K: a nibble plane of R x C/2 bytes, then a header plane of R x C/256 x 16 bytes (f16 d, f16 dmin, 12 scale
 *         bytes, byte-identical to the GGUF super-block's first 16 bytes).  Within each 256-byte run of a row's nibble
 *         plane (the quants of two super-blocks), the 16-byte pieces are ordered [half][group of 64 values].
 *   Q5_K: as Q4_K, with a fifth-bit plane of R x C/8 bytes (each super-block's 32 qh bytes) between the nibble and
 *         header planes.
 *   Q8_0: an int8 plane of R x C bytes (16-byte halves of each 512-byte run ordered [half][block]), then an f16 scale
 *         plane of R x C/32.
 *   Q4_0: a nibble plane of R x C/2 (a block's 16 quant bytes as one piece), then an f16 d plane of R x C/16.
 *   Q5_1: a nibble plane of R x C/2, then a (f16 d, f16 m) plane of R x C/8, then a qh plane of R x C/8.
 * Every plane is tiled by rows (32 for the K-quants, 4 for the 32-value block types): piece p of a row lies one tile's pieces after piece
 * p - 1, so a wavefront's 16-byte loads over a tile's rows cover whole 128-byte lines.  The planar matrix has exactly
 * the GGUF matrix's size; experts sit at base + e * stride.  C % 512 == 0, R % 32 == 0.
 * Every expert store argument (A with its stride sa, and the gu/dn fields of sfnx_moe_layer_w) may instead be a device
 * table of expert pointers, signalled by a stride of 0: expert e's matrix is ((const void* const*) A)[e], wherever
 * it lives (src/moe_w.cuh:9 moe_expert over DW::ep, src/model.hpp:85-86).
 */
#ifndef SFNX_MOE_H
#define SFNX_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SFNX_MAXT 16     /* rows of a decode window (src/model.hpp:48 MAXT) */
#define SFNX_PF_JOB 64   /* rows of a prompt-path job (src/kernels.hpp:26 PF_JOB) */

enum { SFNX_Q4_0 = 2, SFNX_Q5_1 = 7, SFNX_Q8_0 = 8, SFNX_Q4_K = 12, SFNX_Q5_K = 13 }; /* GgmlType ids (src/gguf.hpp:22-25; the others ggml's) */

/* src/kernels.hpp:18-23: one expert's matrix applied to up to SFNX_MAXT activation rows */
typedef struct sfnx_job {
    int w;                    /* expert */
    int n;                    /* rows */
    int y[SFNX_MAXT];         /* activation rows */
    int out[SFNX_MAXT];       /* output rows */
} sfnx_job;

/* src/kernels.hpp:25-32 */
typedef struct sfnx_bigjob {
    int w;
    int n;
    int y[SFNX_PF_JOB];
    int out[SFNX_PF_JOB];
} sfnx_bigjob;

/* src/model.hpp:71-74 Q8S: a dense Q8_0 matrix [rows][cols] in the reference's split layout (src/model.cpp:384-440
 * q8split): int8 values q [rows][cols] row-major and the f16 scale bits d [rows][cols / 32] of each 32-value block.
 * The shared expert's dense matrices cross the boundary in it (DW::s). */
typedef struct sfnx_q8s {
    int8_t* q;
    uint16_t* d;
} sfnx_q8s;

/* ---------------------------------------------------------------------------------------------- errors */
const char* sfnx_last_error(void);
int sfnx_abi_version(void);

/* ---------------------------------------------------------------------------------------------- weight store */
/* bytes of one row of `cols` values (src/gguf.cpp:19-37 type_info: Q4_K 256/144, Q8_0 32/34) */
size_t sfnx_row_bytes(uint32_t type, int cols);
/* seeded synthetic values: out[i] = std * IrwinHall12(seed, offset + i) (splitmix64 draws) */
int sfnx_synth_normal(float* out, size_t n, uint64_t seed, uint64_t offset, float std, void* st);
/* fp32 rows -> GGUF blocks (Q4_K: the library's quantizer; Q8_0: tools/mtp_experts.py:44-55) */
int sfnx_quantize_weights(uint32_t type, const float* x, void* gguf, int64_t rows, int cols, void* st);
/* GGUF blocks of n_mat matrices [rows][cols] <-> the planar store (replaces the loader's slicing into DW,
 * src/model.cpp:554-606; the store keeps every block's bytes, only their places change) */
int sfnx_store_pack(uint32_t type, const void* gguf, void* planar, int64_t n_mat, int rows, int cols, void* st);
int sfnx_store_unpack(uint32_t type, const void* planar, void* gguf, int64_t n_mat, int rows, int cols, void* st);
/* planar -> fp32 (d sc q - dmin m; d q) and -> f16 bits as the tensor-core path makes them (src/moe_mma.cuh:67-216) */
int sfnx_dequantize(uint32_t type, const void* planar, float* y, int64_t n_mat, int rows, int cols, void* st);
int sfnx_dequantize_f16(uint32_t type, const void* planar, uint16_t* y, int64_t n_mat, int rows, int cols, void* st);

/* ---------------------------------------------------------------------------------------------- activations */
/* src/kernels.hpp:36 quantize_q8_1: fp32 rows of n -> q8_1 blocks (36 bytes per 32 values) */
int sfnx_quantize_q8_1(const float* x, void* q, int n, int rows, void* st);

/* ---------------------------------------------------------------------------------------------- routing */
/* src/kernels.hpp:269-278 router_route (decode window, 1 <= T <= 16).  logits [T][E + 1] = W [E + 1][H] . x[t] (row E
 * gates the shared expert); top-K per token among the first E by logit, ties to the lower index; weights the selected
 * softmax renormalised; jobs: one per distinct expert in first-pick order, rows in pair order (pair p = t K + k:
 * gu.y = t, gu.out = dn.y = dn.out = p).  shared != 0: one more job, expert E, rows t -> T K + t.  njobs[0] = job
 * count; njobs[1] is the launch's block counter and must be 0 before the first call (every call leaves it 0).
 * H % 256 == 0, H <= 4096; E % 64 == 0, E <= 1024; 1 <= K <= 16.  Pick rounds with nothing left (NaN / -inf logits)
 * write topi -1, topw 0 and leave the pair out of the jobs. */
int sfnx_router_route(const float* W, const float* x, float* logits, int T, int H, int E, int K, int* topi, float* topw,
                      sfnx_job* jobs_gu, sfnx_job* jobs_dn, int* njobs, int shared, void* st);
/* the router's logits alone, [T][L] = W [L][H] . x[t], any T (the prompt path's sgemm, src/prefill.cu:1163).  From
 * 512 tokens on the fp32 matrix cores: each of 8 slices of H / 8 columns one fmaf chain, the slices added in order;
 * fewer tokens in sfnx_router_route's order.  H % 256 == 0. */
int sfnx_router_logits(const float* W, const float* x, float* logits, int T, int H, int L, void* st);
/* No counterpart in the reference: sfnx_router_logits that also writes xh = f16(x) (sfnx_to_f16's values, bit for bit)
 * from the router's own reads of x, for a prompt path that needs both (from 512 tokens it saves the conversion's
 * launch and its second read of x). */
int sfnx_router_logits_xh(const float* W, const float* x, float* logits, uint16_t* xh, int T, int H, int L, void* st);
/* src/prefill.cu:189-279 (k_pf_top10, k_pf_count, k_pf_jobbase, k_pf_fill): top-K of rows of E + 1 logits, cnt[E],
 * jbase[E] (exclusive scan of ceil(cnt / 64)), BigJobs of each expert's pairs in pair order.  shared != 0: ceil(C/64)
 * more jobs of expert E, rows t -> C K + t.  Job capacity needed: C K / 64 + E + ceil(C / 64). */
int sfnx_pf_route(const float* logits, int C, int E, int K, int* topi, float* topw, int* cnt, int* jbase,
                  sfnx_bigjob* jobs_gu, sfnx_bigjob* jobs_dn, int* njobs, int shared, void* st);

/* ---------------------------------------------------------------------------------------------- routed experts */
/* src/kernels.hpp:281-282 moe_gate_up: gu[job.out[j]][r] = A_e[r] . xq[job.y[j]] for r < n_out, jobs [0, *njobs);
 * A: planar experts (n_out rows of n_in, stride sa bytes); xq: q8_1 rows of n_in; T: the most rows a job holds */
int sfnx_moe_gate_up(const void* A, size_t sa, uint32_t type, int n_in, int n_out, const sfnx_job* jobs,
                     const int* njobs, int njobs_max, int T, const void* xq, float* gu, void* st);
/* src/kernels.hpp:305 moe_down: h = silu(gate) * up of gu rows job.y[j] ([gate (n_in) | up (n_in)]) as q8_1, then
 * part[job.out[j]][r] = A_e[r] . h (the Q4_K down the reference refuses, src/moe.cuh:473-474, included) */
int sfnx_moe_down(const void* A, size_t sa, uint32_t type, int n_in, int n_out, const sfnx_job* jobs, const int* njobs,
                  int njobs_max, int T, const float* gu, float* part, void* st);
/* src/kernels.hpp:286-287 moe_gate_up_big / moe_down_big: the same arithmetic over BigJobs (the q8 prompt path) */
int sfnx_moe_gate_up_big(const void* A, size_t sa, uint32_t type, int n_in, int n_out, const sfnx_bigjob* jobs,
                         const int* njobs, int njobs_cap, const void* xq, float* gu, void* st);
int sfnx_moe_down_big(const void* A, size_t sa, uint32_t type, int n_in, int n_out, const sfnx_bigjob* jobs,
                      const int* njobs, int njobs_cap, const float* gu, float* part, void* st);
/* the weighted sum (src/kernels.cu:797-803 ring_x, src/prefill.cu:476-484 k_pfr_addend):
 * y[t][i] = fmaf(sigmoid(logits[t][E]), part[T K + t][i], sum_k fmaf(topw[t K + k], part[t K + k][i], .)) in k order;
 * shared == 0 drops the shared term; pairs with topi < 0 are skipped */
int sfnx_moe_combine(const float* part, const float* topw, const int* topi, const float* logits, float* y, int T, int H,
                     int E, int K, int shared, void* st);

/* ---------------------------------------------------------------------------------------------- matrix cores */
/* src/kernels.hpp:290-292 moe_gate_up_mma / swiglu_h16 / moe_down_mma: the prompt path's experts as f16 x f16 products
 * with fp32 accumulation on MFMA (src/moe_mma.cuh): weights dequantized to f16 as the reference does (Q4_K:
 * hfma2(q, f16(d sc), f16(-(dmin m))); Q8_0: hmul2(q, d)), activations f16 rows (xh: [tokens][n_in]; h16: [pairs][ff]).
 * out[job.out[m]][r] for r < n_out (a multiple of 256), jobs [0, *njobs) of at most njobs_cap. */
int sfnx_moe_gate_up_mma(const void* A, size_t sa, uint32_t type, int n_in, int n_out, const sfnx_bigjob* jobs,
                         const int* njobs, int njobs_cap, const uint16_t* xh, float* gu, void* st);
int sfnx_swiglu_h16(const float* gu, int ffs, int P, uint16_t* h16, void* st);
/* moe_gate_up_mma and swiglu_h16 in one launch (src/kernels.hpp:290-291 called back to back, as the prompt path does,
 * src/prefill.cu:1167-1169): h16[job.out[m]][f] = f16(silu(gate) * up) for the job's rows, without writing the fp32
 * gate|up rows; equal bit for bit to the two calls.  ff a multiple of 256; the experts' rows are [gate (ff) | up (ff)]. */
int sfnx_moe_gate_up_swiglu_mma(const void* A, size_t sa, uint32_t type, int n_in, int ff, const sfnx_bigjob* jobs,
                                const int* njobs, int njobs_cap, const uint16_t* xh, uint16_t* h16, void* st);
int sfnx_moe_down_mma(const void* A, size_t sa, uint32_t type, int n_in, int n_out, const sfnx_bigjob* jobs,
                      const int* njobs, int njobs_cap, const uint16_t* h16, float* part, void* st);
/* fp32 -> f16 (round to nearest even), n values: the activations the matrix-core path reads (the reference's hc read
 * writes them, src/prefill.cu:1160) */
int sfnx_to_f16(const float* x, uint16_t* y, size_t n, void* st);

/* ---------------------------------------------------------------------------------------------- dense Q8_0 */
/* src/kernels.hpp:47 q8s_gemv (kernel src/dense.cuh:24-154): out[t][r] (row stride out_stride) for t < T = row r of the
 * dense Q8_0 matrix W [rows][cols] (sfnx_q8s split layout; rows % 32 == 0, cols % 512 == 0) dotted with q8_1 row t of
 * y ([T][cols / 32] blocks): 32 lanes a row, lane l the 16-column halves 16 l + 512 i in order, each
 * acc = fmaf(d_w d_a, sum, acc), then the xor butterfly 16 .. 1. */
int sfnx_q8s_gemv(const sfnx_q8s* W, int rows, int cols, const void* y, float* out, int out_stride, int T, void* st);
/* src/model.cpp:384-440 q8split: GGUF Q8_0 blocks [rows][cols / 32] (34 bytes: f16 d, 32 int8) into the split planes
 * of W (cols % 32 == 0).  The loader's conversion, done on the device. */
int sfnx_q8s_split(const void* blocks, int rows, int cols, const sfnx_q8s* W, void* st);
/* src/kernels.cu:1948-2024 swiglu_stacked_q8_1: hq row t ([T][ffs / 32] q8_1 blocks) = silu(gu[t][c]) * gu[t][ffs + c]
 * quantized per 32 values (d = amax / 127, q = round(v / d), ds = (f16 d, f16 sum)); gu is [T][2 ffs], ffs % 32 == 0 */
int sfnx_swiglu_stacked_q8_1(const float* gu, void* hq, int ffs, int T, void* st);
/* The shared expert's SwiGLU and dense Q8_0 down in one launch, as the reference fuses them into its routed gate|up
 * launch (src/kernels.hpp:281-282 moe_gate_up's sh_down / sh_ffs / sh_gu / sh_out; src/dense.cuh:156-198): out[t][r] =
 * W[r] . q8_1(silu(gu[t][0..ffs)) * gu[t][ffs..2 ffs)) for r < rows, t < T.  h never leaves the workgroup, so no
 * buffer is needed for it; the values equal sfnx_swiglu_stacked_q8_1 followed by sfnx_q8s_gemv, bit for bit. */
int sfnx_q8s_swiglu_gemv(const sfnx_q8s* W, int rows, int ffs, const float* gu, float* out, int out_stride, int T,
                         void* st);

/* src/prefill.cu:407-417 pf_dense_xh (the prompt path's dense matrices, the shared expert's among them): out[c][r]
 * (row stride ldo) = sum_k f16(W[r][k]) xh[c][k] for C f16 rows xh [C][cols], fp32 accumulation.  W is a dense Q8_0
 * matrix (sfnx_q8s).  As the reference first converts W into its staging buffer wk (k_q8s_f16 into p.wh), W is first
 * repacked into wk here, into the planar Q8_0 layout of one matrix (rows * cols * 34 / 32 bytes; the reference sizes
 * wk for f16, twice that), and then run as one expert of the matrix-core kernels (sfnx_moe_down_mma's): its f16
 * weights are the reference's k_q8s_f16 values (f16(q d)), made in registers, and the products are summed in fp32 where
 * the reference calls cublasGemmEx; the C rows are taken 64 at a time.  rows % 256 == 0, cols % 512 == 0. */
int sfnx_pf_dense(const sfnx_q8s* W, int rows, int cols, const uint16_t* xh, int C, float* out, int ldo, void* wk,
                  size_t wk_bytes, void* st);

/* ---------------------------------------------------------------------------------------------- fused decode */
/* one layer's weights: router W [E + 1][H] fp32 (row E gates the shared expert), planar gate|up experts (E + 1 of
 * [2 ff][H], the shared expert last) and planar down experts (E + 1 of [H][ff]) */
typedef struct sfnx_moe_layer_w {
    const float* W;
    const void* gu;
    size_t gu_stride;
    const void* dn;
    size_t dn_stride;
} sfnx_moe_layer_w;

/* bytes of the workspace sfnx_moe_decode needs (1 <= T <= 16 is only checked: every piece is laid out for 16 rows, so
 * one workspace serves windows of any size and the offsets do not depend on T); offsets (may be null) receives the byte
 * offsets of its pieces, each with room for 16 rows (M = 16): logits [M][E+1] f32, xq [M][H/32] q8_1, topi [M][K] i32,
 * topw [M][K] f32, jobs_gu and jobs_dn [M K + 1] sfnx_job, njobs [2] i32, gu [M K + M][2 ff] f32, hq_q [M K + M][ff]
 * i8, hq_d and hq_s [M K + M][ff / 32] (f32 scale, i32 sum), y [M][H] f32, then the total (13 values).  After a
 * window of T rows, row t of a piece holds that window's row t (pairs p = t K + k, the shared expert's at T K + t). */
size_t sfnx_moe_decode_workspace(int T, int H, int E, int K, int ff, size_t* offsets);

/* A decode window (1 <= T <= 16 rows) through n_layers stacked MoE layers, replacing the engine's per-layer calls
 * router_route + moe_gate_up + moe_down + the combine (src/engine.cu:933-978, src/kernels.hpp:269-313).  x [T][H] is
 * the residual stream, updated in place: per layer x += MoE(norm ? rmsnorm(x) : x) (rmsnorm as
 * sfnx_residual_rmsnorm).  The workspace keeps the last layer's routing and intermediates (see
 * sfnx_moe_decode_workspace).  Same arithmetic, value for value, as the unfused entry points.  H in {1024, 2048,
 * 2560, 4096}, ff in {512, 1024}.
 * Three launches a layer (four for T > 1: the routing once, in a launch of its own, before gate|up).
 * phases: 0 runs everything; otherwise a mask of the launches to issue per layer (1 router, 2 routing (T > 1) and
 * gate|up, 4 down + combine), for timing each one alone. */
int sfnx_moe_decode(const sfnx_moe_layer_w* layers, int n_layers, uint32_t type, int H, int E, int K, int ff, int shared,
                    float* x, int T, int norm, float eps, void* ws, size_t ws_bytes, int phases, void* st);
/* sfnx_moe_decode with the gate|up and down matrices of different types, as the reference keeps a type per matrix
 * (src/model.cpp:540-606: gate and up stack into one DW, down is its own): gu_type for every layer's gu store, dn_type
 * for its dn store. */
int sfnx_moe_decode2(const sfnx_moe_layer_w* layers, int n_layers, uint32_t gu_type, uint32_t dn_type, int H, int E,
                     int K, int ff, int shared, float* x, int T, int norm, float eps, void* ws, size_t ws_bytes, int phases,
                     void* st);

/* No counterpart in the reference: sfnx_moe_decode2 for callers that cannot allocate (code under HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc).  The workspace is the library's own file-scope device array of
 * 4 MiB, one per GPU, held until the process ends; the call allocates nothing and refuses a shape whose workspace
 * (sfnx_moe_decode_workspace) is larger.  Every call on one GPU shares that array, and the array keeps the last call's
 * routing and intermediates (nothing in it needs to start at zero).  Calls that overlap on one GPU would race on it:
 * a call on another stream than the previous (uncaptured) call's is refused ("a call on another stream still runs")
 * while that call has not finished; calls on one stream are ordered by it.  Under HIP graph capture the check is the
 * caller's: captured calls run at replay.  Same arguments and values as sfnx_moe_decode2 without ws / ws_bytes /
 * phases. */
int sfnx_moe_decode_noalloc(const sfnx_moe_layer_w* layers, int n_layers, uint32_t gu_type, uint32_t dn_type, int H, int E,
                            int K, int ff, int shared, float* x, int T, int norm, float eps, void* st);

/* A layer's shared expert as its own dense Q8_0 matrices, as the reference holds it (src/model.hpp:71-83 Q8S,
 * src/model.cpp:384-440 q8split: LayerW::sh_gu.s, sh_down.s): gu [2 ff][H] and dn [H][ff], each in the split layout. */
typedef struct sfnx_moe_shared_q8s {
    sfnx_q8s gu;
    sfnx_q8s dn;
} sfnx_moe_shared_q8s;
/* sfnx_moe_decode2 with every layer's shared expert from shared_w[l] in the reference's dense q8s arithmetic
 * (src/dense.cuh:24-154; 32 lanes over 16-column halves, fmaf, xor butterfly), as src/engine.cu:936-945 runs it
 * (q8s_gemv gate|up, swiglu_stacked_q8_1, q8s_gemv down into part rows P + t); the shared gate is still router row E.
 * The routed stores need only E experts.  Same values, bit for bit, as sfnx_q8s_gemv + sfnx_swiglu_stacked_q8_1. */
int sfnx_moe_decode_q8s(const sfnx_moe_layer_w* layers, const sfnx_moe_shared_q8s* shared_w, int n_layers,
                        uint32_t gu_type, uint32_t dn_type, int H, int E, int K, int ff, float* x, int T, int norm,
                        float eps, void* ws, size_t ws_bytes, int phases, void* st);

/* ---------------------------------------------------------------------------------------------- hc read */
/* bytes of the workspace sfnx_hc_read needs (windows of up to 16 rows); offsets (may be null, else 6 values) receives
 * the byte offsets of its pieces, each laid out for 16 rows (row t at t times a row's size): part [16][HC N / 512]
 * [LR + HC] f32 (the slices' partial down and inject dots), ssp [16][HC N / 512] f32 (the slices' square sums), lo
 * [16][LR] int8, its scales [16][LR / 32] f32, rs [16][HC] f32, then the total. */
size_t sfnx_hc_workspace(int N, int HC, int LR, size_t* offsets);
/* The hyper-connection read that produces the MoE half's input, src/kernels.cu:1054 hc_read (kernel src/hc.cuh:13-380):
 * R [T][HC N] (HC residual streams, updated to R' when bo is given), bo [T][N] (the last half's output, or null) with
 * inj_prev [T][HC] (its inject logits), w_norm [HC N] f32, the down Q8S matrix (down_q int8 [LR][HC N], down_d f16
 * [LR][HC N / 32]), the up Q8S matrix (up_q int8 [HC N][LR], up_d f16 [HC N][LR / 32]) and w_inj bf16 [HC][HC N] (or
 * null: no inject rows).  Writes mixed [T][N] (the MoE input), inject [T][HC] (when w_inj and inject are given) and,
 * when xq is given, mixed as q8_1 [T][N / 32] (the expert dots' activations).  1 <= T <= 16, N % 512 == 0,
 * HC <= 8, LR % 32 == 0 and LR <= 512.  The reference's grid barriers and its err word have no counterpart: three
 * launches, no waits. */
int sfnx_hc_read(float* R, const float* bo, const float* inj_prev, const float* w_norm, const void* down_q,
                 const void* down_d, const void* up_q, const void* up_d, const void* w_inj, float eps, float* mixed,
                 float* inject, void* xq, int T, int N, int HC, int LR, void* ws, size_t ws_bytes, void* st);

/* the stacked-layer driver's glue between layers (no reference counterpart on the MoE path: the engine's
 * hyper-connection read, src/hc.cuh, normalises the MoE input): x += y (y may be null), then
 * xn = x / sqrt(mean(x^2) + eps) per row of H */
int sfnx_residual_rmsnorm(float* x, const float* y, float* xn, int T, int H, float eps, void* st);

/* Measurement hook (no reference counterpart: for benchmarks that need each kernel's own duration).  While enabled,
 * sfnx_moe_decode launches its three kernels with start/stop events that the runtime stamps at the dispatch's
 * begin and end; sfnx_kernel_clock_read waits for the last such launches and writes their durations in us
 * (router, gate|up, down + combine) to us[3].  Windows of T > 1 rows add a fourth launch per layer, the routing
 * (k_dec_route, one workgroup) between the router and gate|up: the clock does not cover it, so a window's per-kernel
 * figures leave it out (the window's whole time comes from timing the layers' launches together).  Process-wide; not
 * for concurrent callers. */
int sfnx_kernel_clock(int enable);
int sfnx_kernel_clock_read(float* us);

/* ---------------------------------------------------------------------------------------------- GGUF files
 * A read-only mapping of a GGUF model (every shard of a split "<stem>-0000N-of-0000M.gguf" model), its tensor index
 * and the first shard's metadata (src/gguf.hpp:20-88 Gguf, TypeInfo, Tensor; src/gguf.cpp).  Lookups return 1 when
 * found, 0 when missing and a negative status on error. */
typedef struct sfnx_gguf sfnx_gguf;
typedef struct sfnx_gguf_tensor {
    uint32_t type;      /* ggml type id */
    int n_dims;
    int64_t ne[4];      /* ne[0]: elements a row */
    const void* data;   /* in the mapping (host memory) */
    size_t nbytes;
    int shard;
} sfnx_gguf_tensor;
int sfnx_gguf_type_info(uint32_t type, int* block, int* bytes);                       /* src/gguf.hpp:29 type_info */
int sfnx_gguf_open(const char* path, sfnx_gguf** g);                                   /* src/gguf.hpp:49 Gguf::Gguf */
void sfnx_gguf_close(sfnx_gguf* g);                                                    /* src/gguf.hpp:50 ~Gguf */
int sfnx_gguf_n_tensors(const sfnx_gguf* g);                                           /* src/gguf.hpp:66 tensors() */
int sfnx_gguf_tensor_at(const sfnx_gguf* g, int i, const char** name, sfnx_gguf_tensor* t);
int sfnx_gguf_find(const sfnx_gguf* g, const char* name, sfnx_gguf_tensor* t);          /* src/gguf.hpp:52 find */
int sfnx_gguf_int(const sfnx_gguf* g, const char* key, int64_t* v);                    /* src/gguf.hpp:57 i */
int sfnx_gguf_float(const sfnx_gguf* g, const char* key, double* v);                   /* src/gguf.hpp:61 num */
int sfnx_gguf_str(const sfnx_gguf* g, const char* key, const char** v);                /* src/gguf.hpp:59 s */

/* One layer's MoE weights from a GGUF into the device store (src/model.cpp:554-606 expert_rows2 / expert_cols,
 * 766-809): blk.<layer>.ffn_{gate,up}_exps rows ff0..ff1 stacked [gate ; up] per expert into gu (planar, gu_stride a
 * matrix), ffn_down_exps columns ff0..ff1 into dn (dn_stride a matrix), the shared expert ffn_*_shexp (when present,
 * of the same type and FF) as expert E, and the router W = [ffn_gate_inp rows ; ffn_gate_inp_shexp] (f32 [E+1][H]).
 * Q4_0, Q5_1, Q8_0, Q4_K or Q5_K experts, gate and up of one type, down of that or another; ff0 on a block of the
 * down type (32 or 256 columns), ff1 - ff0 and H multiples of 512.  info (may be null, else 6 ints) receives the
 * gate|up type, H, E, ff1 - ff0, shared and the down type.  A loader, not a hot-path call: it allocates a staging
 * buffer and synchronises the stream.  E comes from the file (ne[2] of blk.<layer>.ffn_gate_exps, sfnx_gguf_find):
 * gu_bytes and dn_bytes are the sizes of the caller's gu and dn buffers, and w_rows the rows W holds; the call refuses
 * a layer whose experts (E + 1 with a shared expert that joins the stores, E otherwise) or router rows (E + 1) do not
 * fit, before it writes anything. */
int sfnx_gguf_moe_layer(const sfnx_gguf* g, int layer, int ff0, int ff1, void* gu, size_t gu_stride, size_t gu_bytes,
                        void* dn, size_t dn_stride, size_t dn_bytes, float* W, int w_rows, int* info, void* st);
/* sfnx_gguf_moe_layer for the model as the reference loads it (src/model.cpp:807-809): the shared expert must be
 * present and Q8_0 ("the shared expert is not Q8_0" otherwise) and goes, as dense matrices in the split layout
 * (src/model.cpp:384-440 q8split), to sh_gu ([2 ffs][H]) and sh_dn ([H][ffs], columns ff0..ff1), for
 * sfnx_moe_decode_q8s, sfnx_q8s_gemv and sfnx_pf_dense; gu and dn then receive the E routed experts only.  W, the
 * buffer sizes and info as sfnx_gguf_moe_layer. */
int sfnx_gguf_moe_layer_q8s(const sfnx_gguf* g, int layer, int ff0, int ff1, void* gu, size_t gu_stride, size_t gu_bytes,
                            void* dn, size_t dn_stride, size_t dn_bytes, float* W, int w_rows, const sfnx_q8s* sh_gu,
                            const sfnx_q8s* sh_dn, int* info, void* st);

/* ---------------------------------------------------------------------------------------------- expert cache */
/* src/model.hpp:95-116 ExpertCache, src/moe.cuh:19-71 cache_plan, src/kernels.cu:1636-1668: routed experts kept in
 * page-locked host memory (device-visible, sfnx_host_alloc), with VRAM slots for the ones in use.  A pool's slots hold
 * whole experts of one size (gate|up at 0, down at dn_off); layers whose experts have that size share the pool.  The
 * tables ep_gu / ep_dn ([n_layers * n_experts] device pointers) say where each expert's matrices are now, a slot or
 * its host copy; a layer's rows of them are the expert stores the calls above take with stride 0.  The arena fields
 * of the reference (slots lent to its K/V pool) have no counterpart: no pool here lends its slots. */
#define SFNX_EC_POOLS 4
#define SFNX_EC_LAYERS 128
typedef struct sfnx_expert_cache {
    int n_slots;                          /* all pools' */
    int n_pools;
    int n_layers, n_experts;              /* the tables' shape (the reference's NL, NEXP) */
    int pool_of[SFNX_EC_LAYERS];          /* each layer's pool */
    int s0[SFNX_EC_POOLS], n[SFNX_EC_POOLS];   /* a pool's slots: [s0, s0 + n) of the slot numbers */
    size_t slot_bytes[SFNX_EC_POOLS], dn_off[SFNX_EC_POOLS];
    void* pool[SFNX_EC_POOLS];            /* device: a pool's slots, slot_bytes apart */
    const void** ep_gu;                   /* device [n_layers * n_experts]: where each expert's gate|up is now */
    const void** ep_dn;
    const void* const* host_gu;           /* device [n_layers * n_experts]: its host copy (device-visible address) */
    const void* const* host_dn;
    int* slot_of;                         /* device [n_layers * n_experts]: its slot, or -1 */
    int* owner;                           /* device [n_slots]: the expert in it (layer * n_experts + e), or -1 */
    unsigned char* ref;                   /* device [n_slots]: 0 free to take, 1 used since the hand passed, 2 the layer's */
    int* hand;                            /* device [SFNX_EC_POOLS]: each pool's CLOCK hand, a slot number in it */
    int* status;                          /* device [2] or null: [0] the misses the last plan left on their host copies
                                             (0 when every job got a slot), [1] their running total (no counterpart in
                                             the reference, whose plan spins until a slot frees) */
} sfnx_expert_cache;

/* page-locked host memory the GPU reads directly (the reference's mapped host copies): *host and *dev receive the host
 * and device addresses of `bytes` bytes; sfnx_host_free releases them */
int sfnx_host_alloc(size_t bytes, void** host, void** dev);
int sfnx_host_free(void* host);
/* src/moe.cuh:22-71 cache_plan (k_cache_plan, src/kernels.cu:1637): one wavefront plans the window's slots for layer
 * `layer`: every job whose expert is in a slot keeps it; each other one takes the slot of the layer's pool that the
 * pool's CLOCK hand reaches first with ref 0, a ref 1 it passes dropping to 0, 32 slots a sweep step as the reference's
 * warp; the slot's old expert points back at its host copy.  list (1 + njobs ints) receives the number of experts
 * that took a slot, then their ids (layer * n_experts + e), in job order.  When every slot of the pool is held by the
 * window, a miss finds no victim: it and the misses after it stay on their host copies (their table entries point
 * there, so the expert calls read them over the bus and compute the same values), the misses planned before it keep
 * their slots, and status[0] receives the count (the reference's plan would spin).  Every slot the window holds ends
 * at ref 1 either way. */
int sfnx_cache_plan(const sfnx_job* jobs, const int* njobs, int layer, const sfnx_expert_cache* ec, int* list, void* st);
/* src/kernels.hpp:269-278 router_route with an ExpertCache (src/moe.cuh:128-198): sfnx_router_route, and then, in
 * the same launch, its last block's first wavefront plans the window's slots for `layer` as sfnx_cache_plan does (the
 * same slots, list, tables, refs, hand and status), so a cached layer's plan takes no launch of its own.  With shared
 * != 0 the shared job (expert E) is planned like the others, so the cache's tables need E + 1 experts a layer. */
int sfnx_router_route_plan(const float* W, const float* x, float* logits, int T, int H, int E, int K, int* topi,
                           float* topw, sfnx_job* jobs_gu, sfnx_job* jobs_dn, int* njobs, int shared,
                           const sfnx_expert_cache* ec, int layer, int* list, void* st);
/* src/kernels.cu:1642-1658 k_cache_copy / cache_copy: the listed experts' matrices from their host copies into their
 * slots of pool p */
int sfnx_cache_copy(const sfnx_expert_cache* ec, int p, const int* list, void* st);
/* src/kernels.cu:1659-1668 moe_cache: the plan (when jobs is given) and the copy for `layer`, after checking that the
 * layer's expert strides are its pool's */
int sfnx_moe_cache(int layer, size_t gu_stride, size_t dn_stride, const sfnx_expert_cache* ec, int* list,
                   const sfnx_job* jobs, const int* njobs, void* st);

#ifdef __cplusplus
}
#endif
#endif
