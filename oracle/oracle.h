/*
 * CPU oracle for the quantized MoE layer.  TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg call it as the checker; the product library never links, loads or calls it.
 *
 * A plain-C restatement of the reference's arithmetic (johnfink8/sfnx, citations are paths under its src/ and tools/).
 * Every function names the reference lines it follows.  Formats are GGUF's: Q4_K super-blocks of 256 values in
 * 144 bytes, Q8_0 blocks of 32 in 34 bytes, activation q8_1 blocks of 32 in 36 bytes.
 *
 * Parity status per function (how each is pinned lives in tests/test_oracle_*.py):
 *   f16 conversion, Q4_K / Q8_0 dequant, q8_1, top-k, jobs, permutation, Q4_K dot, combine: pinned by closed forms,
 *   hand-built known answers, brute force and float64 products.
 *   Q4_K quantizer: the reference has none; pinned by round-trip bounds only (its bytes are not llama.cpp's).
 *   Q8_0 x q8_1 dot (ggml vec_dot_q8_0_q8_1, not vendored in the reference): pinned by its closed form in float64.
 *   exp in silu / sigmoid / softmax weights: the reference uses fast-math __expf; the oracle uses libm expf, so values
 *   downstream of exp are compared within tolerance, never bit for bit.
 */
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_Q4_0 = 2, ORC_Q5_1 = 7, ORC_Q8_0 = 8, ORC_Q4_K = 12, ORC_Q5_K = 13 };   /* GgmlType ids (src/gguf.hpp:22-25; the others ggml's) */
#define ORC_QK_K 256
#define ORC_Q4K_BYTES 144
#define ORC_Q5K_BYTES 176
#define ORC_Q40_BYTES 18
#define ORC_Q51_BYTES 24
#define ORC_Q80_BYTES 34
#define ORC_Q81_BYTES 36
#define ORC_MAXT 16
#define ORC_PF_JOB 64

/* src/kernels.hpp:18-32 */
typedef struct { int w, n, y[ORC_MAXT], out[ORC_MAXT]; } orc_job;
typedef struct { int w, n, y[ORC_PF_JOB], out[ORC_PF_JOB]; } orc_bigjob;

float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
/* round_f16(a * b + c) with a single rounding: __hfma2 of src/moe_mma.cuh:82-95 on exact f16 operands */
uint16_t orc_f16_fma(uint16_t a, uint16_t b, uint16_t c);
uint16_t orc_f16_mul(uint16_t a, uint16_t b);

/* Seeded synthetic data: value i = std * (sum of 12 uniform 24-bit draws - 6), an Irwin-Hall(12) normal; the draws
 * come from splitmix64(seed, counter), so any slice [offset, offset + n) is reproducible on its own. */
void orc_synth_normal(float* out, size_t n, uint64_t seed, uint64_t offset, float std);

/* Q4_K quantizer (the reference ships none: src comments and tools/mtp_experts.py:1-8 cover Q4_0/Q8_0 only).
 * Per 32-value sub-block: min' = min(0, min x), scale = (max x - min') / 15; per super-block d = max scale / 63 and
 * dmin = max(-min') / 63 stored as f16; 6-bit sc, m = round(scale / d), round(-min' / dmin) against the stored f16;
 * q = round((x + dmin m) / (d sc)) clamped to 0..15.  rows x cols, cols % 256 == 0. */
void orc_quantize_q4_k(const float* x, void* dst, int64_t rows, int cols);
/* tools/mtp_experts.py:44-55: d = amax / 127, q = round-half-away(x * (1 / d)), f16 d */
void orc_quantize_q8_0(const float* x, void* dst, int64_t rows, int cols);
/* Q5_K (ggml block_q5_K, 176 bytes: f16 d, f16 dmin, 12 scale bytes, qh[32], qs[128]; value l of sub-block j is
 * (qs[32 (j / 2) + l] >> 4 (j % 2)) & 15 | ((qh[l] >> j) & 1) << 4, src/moe_mma.cuh:84-92,123-136).  The library's
 * quantizer as for Q4_K with 31 levels: scale = (max - min') / 31, q clamped to 0..31. */
void orc_quantize_q5_k(const float* x, void* dst, int64_t rows, int cols);
void orc_dequant_q5_k(const void* src, float* y, int64_t rows, int cols);
void orc_dequant_q5_k_f16(const void* src, uint16_t* y, int64_t rows, int cols);
/* Q4_0 (18 bytes: f16 d, value l in the low nibble of byte l, l + 16 in its high nibble; (q - 8) d), quantizer
 * tools/mtp_experts.py:29-41.  Q5_1 (24 bytes: f16 d, f16 m, u32 qh, 16 nibble bytes; d q + m, the fifth bit of value
 * l is qh bit l), the library's quantizer in ggml's closed form. */
void orc_quantize_q4_0(const float* x, void* dst, int64_t rows, int cols);
void orc_quantize_q5_1(const float* x, void* dst, int64_t rows, int cols);
void orc_dequant_q4_0(const void* src, float* y, int64_t rows, int cols);
void orc_dequant_q4_0_f16(const void* src, uint16_t* y, int64_t rows, int cols);
void orc_dequant_q5_1(const void* src, float* y, int64_t rows, int cols);
void orc_dequant_q5_1_f16(const void* src, uint16_t* y, int64_t rows, int cols);

/* get_scale_min_k4: src/moe_q4k.cuh:15-23, tools/moe_mma_bench.cu:44-52 */
void orc_q4k_scale_min(const uint8_t* scales12, int j, int* sc, int* m);
/* fp32 dequant, tools/moe_mma_bench.cu:54-69 (before its f16 rounding): (d sc) q - dmin m */
void orc_dequant_q4_k(const void* src, float* y, int64_t rows, int cols);
/* the f16 weights of the tensor-core path, src/moe_mma.cuh:67-104: hfma2(q, f16(d sc), f16(-(dmin m))) */
void orc_dequant_q4_k_f16(const void* src, uint16_t* y, int64_t rows, int cols);
void orc_dequant_q8_0(const void* src, float* y, int64_t rows, int cols);
/* src/moe_mma.cuh:196-215: hmul2(q, d) */
void orc_dequant_q8_0_f16(const void* src, uint16_t* y, int64_t rows, int cols);

/* k_quantize, src/kernels.cu:99-113: per 32 values d = amax / 127, q = roundf(x / d), ds = {f16(d), f16(sum)},
 * the sum in the warp butterfly's order (xor 16, 8, 4, 2, 1) */
void orc_quantize_q8_1(const float* x, void* q, int n, int rows);

/* Router logits [T][L] = W [L][H] . x[t], H % 256 == 0.  Summation order of the HIP kernel (the reference's own order
 * under fast-math contraction cannot be recovered, src/moe.cuh:80-120): 64 lanes, lane l takes the float4 chunks
 * l, l + 64, ... as an fmaf chain, then a xor butterfly 32, 16, 8, 4, 2, 1. */
void orc_router_logits(const float* W, const float* x, float* logits, int T, int H, int L);
/* The prompt path's router logits (src/prefill.cu:1163, the engine's sgemm) in the order of the HIP matrix-core
 * kernel, H % 128 == 0: the hidden dimension in 8 slices of H / 8; slice s is one fmaf chain from 0 over
 * k = s H / 8 + 16 j + 4 g + i in the order j, i, g (j the step of 16 columns, i = 0..3, g = 0..3: a chain of
 * v_mfma_f32_16x16x4_f32, which sums its 4 k-slots as fmaf in slot order g); the logit is
 * ((((((p0 + p1) + p2) + p3) + p4) + p5) + p6) + p7. */
void orc_router_logits_mm(const float* W, const float* x, float* logits, int T, int H, int L);
/* sfnx_router_logits: chunks of ORC_ROUTER_MM_MIN_T tokens or more in the matrix-core order, fewer in the VALU
 * kernel's (orc_router_logits) */
#define ORC_ROUTER_MM_MIN_T 512
void orc_router_logits_prompt(const float* W, const float* x, float* logits, int T, int H, int L);

/* Top-k per row, src/moe.cuh:128-162 / src/prefill.cu:191-221: k rounds of the largest untaken logit among the first
 * E of each row (stride ld), ties to the lower index, NaN and -inf never taken; weight exp(l - l_top1) / sum.
 * A round with nothing left to take writes topi -1, topw 0.  Returns how many rounds found nothing. */
int orc_topk(const float* logits, int T, int E, int ld, int K, int* topi, float* topw);

/* Decode jobs, src/moe.cuh:164-198 and tools/kbench.cu:77-95: one job per distinct expert in first-pick order over
 * pairs p = t K + k, rows in pair order; gu.y = token, gu.out = dn.y = dn.out = p.  shared: one more job, expert E,
 * rows t with out T K + t.  Pairs with topi < 0 are left out.  Returns the job count. */
int orc_jobs_decode(const int* topi, int T, int K, int E, int shared, orc_job* gu, orc_job* dn);
/* Prefill permutation, src/prefill.cu:223-279: cnt[e]; jbase = exclusive scan of ceil(cnt / 64) in expert order; each
 * expert's pairs in pair-index order, 64 a job.  shared: ceil(C / 64) more jobs of expert E, rows t -> C K + t.
 * Returns the job count. */
int orc_jobs_prefill(const int* topi, int C, int K, int E, int shared, int* cnt, int* jbase, orc_bigjob* gu,
                     orc_bigjob* dn);

/* Q4_K row (K columns, K % 512 == 0) . one q8_1 activation row: the per-64-group term and summation order of
 * q4k_groups / q4k_row / job_store, src/moe_q4k.cuh:30-86 and src/moe.cuh:224-235 (8 lanes a row, a lane's groups in
 * order, then xor 4, 2, 1). */
float orc_dot_q4_k(const uint8_t* wrow, const uint8_t* yq, int K);
/* Q8_0 row . q8_1 row: per 32-block (d_w d_a) * sum q_w q_a (ggml vec_dot_q8_0_q8_1's closed form); 16 lanes a row,
 * lane l the blocks l, l + 16, ... in order, then xor 8, 4, 2, 1. */
float orc_dot_q8_0(const uint8_t* wrow, const uint8_t* yq, int K);
/* Q5_K x q8_1: the Q4_K lane order and combine on 5-bit values (the reference's Q5_K decode dot is ggml's
 * vec_dot_q5_K_q8_1, not vendored: its order is parity unpinned; this form is pinned by float64 products) */
float orc_dot_q5_k(const uint8_t* wrow, const uint8_t* yq, int K);
/* Q4_0 / Q5_1 x q8_1: the Q8_0 lanes; per block (d_w d_a) sum (q - 8) a, or (d_w d_a) sum q a + (m_w d_a) sum a */
/* the shared expert's dense Q8_0 rows, src/dense.cuh:24-154 (32 lanes over 16-column halves, fmaf, butterfly) */
float orc_dot_q8s(const uint8_t* wrow, const uint8_t* yq, int K);
float orc_dot_q4_0(const uint8_t* wrow, const uint8_t* yq, int K);
float orc_dot_q5_1(const uint8_t* wrow, const uint8_t* yq, int K);
float orc_dot(int type, const uint8_t* wrow, const uint8_t* yq, int K);

/* k_moe_h, src/moe.cuh:284-295: h = silu(gate) * up of one [gate (ff) | up (ff)] row, as q8_1 */
void orc_swiglu_q8_1(const float* gu, int ff, void* hq);

/* The routed + shared layer, T tokens (pairs computed one by one: the result of a pair does not depend on which job
 * carries it).  Experts: gate|up matrices [2 ff][H] at gu_w + e * gu_stride, down [H][ff] at dn_w + e * dn_stride, in
 * GGUF block layout, the shared expert at index E.  Router W [E + 1][H] (row E: the shared expert's gate).
 * y[t] = sum_k fmaf(topw, part) + sigmoid(l[t][E]) part_shared (src/kernels.cu:797-803).  Optional outputs may be
 * null.  nthreads > 1 splits the rows over threads (same arithmetic, same result). */
typedef struct {
    const float* W;
    const uint8_t* gu_w;
    size_t gu_stride;
    const uint8_t* dn_w;
    size_t dn_stride;
    int type;          /* the gate|up matrices' type (ORC_*) */
    int H, E, K, ff, shared;
    int dn_type;       /* the down matrices' type */
    const uint8_t* sh_gu;   /* when set: the shared expert's gate|up [2 ff][H] as Q8_0 blocks, computed as the reference's */
    const uint8_t* sh_dn;   /* dense q8s rows (orc_dot_q8s); its down [H][ff] likewise.  Else it is expert E of gu_w / dn_w */
} orc_layer;
void orc_layer_decode(const orc_layer* L, const float* x, int T, float* y, float* logits, int* topi, float* topw,
                      float* gu, float* part, int nthreads);
/* orc_layer_decode with the prompt path's router order (orc_router_logits_prompt): a chunk through the layer as the
 * prompt-path kernels route it */
void orc_layer_prompt(const orc_layer* L, const float* x, int T, float* y, float* logits, int* topi, float* topw,
                      float* gu, float* part, int nthreads);

/* The f16 tensor-core path (src/moe_mma.cuh, src/prefill.cu:1164-1168) in float64: out[r] = sum_k w16[r][k] x16[k]
 * with the f16 weights of orc_dequant_*_f16 (tools/moe_mma_bench.cu:197-220 checks the same way) */
void orc_mma_matvec(const uint8_t* w, int type, int n_in, int n_out, const uint16_t* x16, double* out);
/* k_swiglu_h16, src/moe_mma.cuh:382-388: h16 = f16(silu(gate) * up) of one [gate (ff) | up (ff)] row */
void orc_swiglu_h16(const float* gu, int ff, uint16_t* h16);
/* the hyper-connection read, src/hc.cuh:13-380 (k_hc), for T rows: R [T][HC N] (updated to R' when bo), bo [T][N] or
 * null, inj_prev [T][HC], w_norm [HC N], down Q8S (dq int8 [LR][HC N], dd f16 [LR][HC N / 32]), up Q8S (uq [HC N][LR],
 * ud [HC N][LR / 32]), w_inj bf16 [HC][HC N] or null; out: mixed [T][N], inject [T][HC] (or null), xq [T][N / 32]
 * q8_1 (or null), part [T][HC N / 512][LR + HC] and ssp [T][HC N / 512] (or null): the slices' partial dots and
 * square sums.  N % 512 == 0, LR % 32 == 0, LR <= 512, HC <= 64. */
void orc_hc_read(float* R, const float* bo, const float* inj_prev, const float* w_norm, const int8_t* dq,
                 const uint16_t* dd, const int8_t* uq, const uint16_t* ud, const uint16_t* w_inj, float eps, int T, int N,
                 int HC, int LR, float* mixed, float* inject, uint8_t* xq, float* part, float* ssp);

/* one token through the layer with nthreads threads, median of reps wall times in microseconds (cache swept between
 * runs through a buffer of sweep_bytes) */
double orc_time_layer_decode(const orc_layer* L, const float* x, int nthreads, int reps, size_t sweep_bytes, float* y);

#ifdef __cplusplus
}
#endif
