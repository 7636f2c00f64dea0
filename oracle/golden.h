/* golden.h -- CPU golden models for the SGEMM / batch-1 GEMV hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the oracle: the C restatement of the
 * reference's own CPU golden models.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it, and only to check results against (or, in
 * the bench, as the timed CPU baseline).  The product path never calls into it.
 *
 * Every function cites the reference lines it restates.  All arithmetic is plain
 * fp32 in the reference's serial k-ascending order; the library is compiled with
 * -O2 -ffp-contract=off so a*b+c is never fused (bit-reproducible on x86-64 SSE).
 *
 * Pinning (what fixes each function independently of this restatement):
 *   og_h2f            exhaustive 65,536-entry check against the closed form and numpy
 *   og_sgemm*         small-integer inputs (exact in fp32) vs int64 matmul; identity;
 *                     fp64 brute force within the fp32 rounding bound
 *   og_gemv*          same integer trick, bias/NULL-bias, N != K argument order
 *   og_gemv_hh        integer fp16 W and x vs int64; equals og_gemv_h_fbias on numpy's IEEE
 *                     decode of normal x codes; x subnormals read +0, exponent-31 x finite
 *   og_gemv_multi     reduces to og_gemv row by row (T = 1 and T > 1)
 *   og_rms            torch.nn.functional.rms_norm
 *   og_rope_tables    closed form cos/sin(pos * theta^(-2d/HD)) in float64
 *   og_qwen_forward   transformers' Qwen2 model (library forward) on the same
 *                     h2f-decoded weights; attention at pos 0 returns v exactly
 */
#ifndef SWITCH_GPU_ORACLE_GOLDEN_H
#define SWITCH_GPU_ORACLE_GOLDEN_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* fp16 bits -> fp32 with the reference's contract (qwen_engine.c:90-98,
 * qwen_kernels.cu:6-14): exponent 0 -> +0.0 (subnormals and -0 flushed),
 * exponent 31 -> finite +-2^16 * (1 + m/1024), otherwise exact IEEE. */
float og_h2f(uint16_t h);

/* C = A*B, fp32 row-major, serial k-ascending (gpu_workload.c:97-98).
 * A is MxK (stride K), B is KxN (stride N), C is MxN (stride N). */
void og_sgemm(const float *A, const float *B, float *C, int M, int N, int K);
/* Same sum for rows [row0, row1) only, spread over nthreads OpenMP threads.
 * Each element keeps its serial k order, so results equal og_sgemm bit for bit. */
void og_sgemm_rows(const float *A, const float *B, float *C, int M, int N, int K,
                   int row0, int row1, int nthreads);
/* The reference verdict (gpu_workload.c:95-112): counts cells with
 * |got-ref| > 0.05*|ref| + 1e-3, stopping at 5 bad rows (one per row).  Returns the count. */
int og_sgemm_verdict_bad(const float *got, const float *ref, int M, int N);

/* y[n] = sum_k W[n*K+k]*x[k] (+ bias[n] if bias), fp32, serial k-ascending
 * (gemv_test.c:85-90; gpt2_engine.c:342-349 for the nullable bias). */
void og_gemv(const float *W, const float *x, const float *bias, float *y, int K, int N,
             int nthreads);

/* fp16-weight GEMV, cpu_gemv_h (qwen_engine.c:276-284): bias is fp16 bits, nullable. */
void og_gemv_h(const uint16_t *W, const float *x, const uint16_t *bias, float *y,
               int K, int N, int nthreads);
/* The device-side contract of gemv_h (qwen_kernels.cu:34-70 with the host bias
 * decode of qwen_engine.c:170-175): bias is fp32 (already h2f-decoded), nullable. */
void og_gemv_h_fbias(const uint16_t *W, const float *x, const float *bias, float *y,
                     int K, int N, int nthreads);

/* The fp16-x form of gemv_h: x as fp16 bits too, decoded with og_h2f like W (the same
 * contract, qwen_kernels.cu:6-14), then og_gemv_h_fbias's serial dot product; bias fp32,
 * nullable.  No reference counterpart (the reference gemv_h reads fp32 x only). */
void og_gemv_hh(const uint16_t *W, const uint16_t *x, const float *bias, float *y,
                int K, int N, int nthreads);

/* Batched GEMV, Y[t*N+n] = sum_k W[n*K+k]*X[t*K+k] + (bias ? bias[n] : 0)
 * (gpt2_kernels.cu:110-155 semantics; serial k order per output). */
void og_gemv_multi(const float *W, const float *X, const float *bias, float *Y,
                   int K, int N, int T, int nthreads);

/* RMSNorm with fp16 weight, cpu_rms (qwen_engine.c:285-290). */
void og_rms(const float *x, const uint16_t *w, float *y, int n, float eps);

/* ---- Qwen2.5 decode (qwen_engine.c:43-75 dims/layout, :292-358 cpu_forward) ---- */
typedef struct {
    int V, C, NL, NH, NKV, HD, FC, CTX;
    float eps;     /* RMSNorm eps, 1e-6 (qwen_engine.c:55) */
    float theta;   /* RoPE base, 1e6 (conv_qwen.py:27); tables live in the blob */
} og_qwen_cfg;

/* Byte size of the flat weight file for cfg (qwen_engine.c:61-67). */
size_t og_qwen_file_bytes(const og_qwen_cfg *cfg);
/* RoPE tables as conv_qwen.py:75-80 writes them: float64 angles, stored fp32. */
void og_rope_tables(int ctx, int hd, double theta, float *cos_out, float *sin_out);

/* One decode position through the CPU golden (cpu_forward, qwen_engine.c:292-358).
 * blob: the whole weight file.  kc/vc: NL*CTX*KVD fp32 caches (position pos is
 * written).  logits (V floats) written only if want_logits.  trace, if non-NULL,
 * receives the residual after each layer (NL*C floats).  nthreads row-parallelises
 * the GEMVs (bit-identical to serial).  Returns 0, or -1 on a bad argument. */
int og_qwen_forward(const og_qwen_cfg *cfg, const void *blob, float *kc, float *vc,
                    int token, int pos, int want_logits, float *logits, float *trace,
                    int nthreads);

/* ---- GPT-2 124M fp32 decode (gpt2_engine.c:40-70 dims/layout, :333-349 cpu_ln/cpu_gemv,
 * :363-421 cpu_forward) ---- */
typedef struct {
    int V, C, NL, NH, HD, FC, CTX;
    float eps;     /* LayerNorm eps, 1e-5 (gpt2_engine.c:339) */
} og_gpt2_cfg;
/* Float count of the flat fp32 weight file (gpt2_engine.c:50-58). */
size_t og_gpt2_file_floats(const og_gpt2_cfg *cfg);
/* LayerNorm with two-pass mean/variance, cpu_ln (gpt2_engine.c:333-341). */
void og_layernorm(const float *x, const float *w, const float *b, float *y, int n, float eps);
/* One decode position (cpu_forward).  kc/vc: NL*CTX*C fp32 caches.  Returns 0 or -1. */
int og_gpt2_forward(const og_gpt2_cfg *cfg, const float *w, float *kc, float *vc, int token, int pos,
                    int want_logits, float *logits, float *trace, int nthreads);

/* First-max argmax (qwen_engine.c:360-364). */
int og_argmax(const float *v, int n);

#ifdef __cplusplus
}
#endif
#endif
