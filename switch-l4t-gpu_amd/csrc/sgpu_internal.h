/* sgpu_internal.h -- functions shared between the library's own C files (not exported). */
#ifndef SGPU_INTERNAL_H
#define SGPU_INTERNAL_H
#include <stdint.h>

#include "switch_gpu.h"

#ifdef __cplusplus
extern "C" {
#endif

#define SGPU_MAX_DEVICES 16

/* x[i] = h2f(emb[token*C + i]) on the device (sgpu_embed_h in the tuned code object). */
__attribute__((visibility("hidden"))) int sgpu_internal_embed_h(const uint16_t *emb, int token, float *x, int C,
                                                                void *stream);
/* Fused decode kernels (sgpu_decode.hip); see qwen.c for the call sequence. */
#define SGPU_HIDDEN __attribute__((visibility("hidden")))
SGPU_HIDDEN int sgpu_internal_dec_qkv(const uint16_t *W, int K, int nrows, const float *x, const uint16_t *lnw,
                                      float eps, const float *bias, float *q, float *kc, float *vc,
                                      const float *cosT, const float *sinT, const int *step, int NH, int NKV,
                                      int HD, void *stream);
SGPU_HIDDEN int sgpu_internal_dec_gateup(const uint16_t *W, int K, int FC, const float *x, const uint16_t *lnw,
                                         float eps, float *y, void *stream);
SGPU_HIDDEN int sgpu_internal_dec_res(const uint16_t *W, int K, int N, const float *a, const float *bias, float *x,
                                      void *stream);
SGPU_HIDDEN int sgpu_internal_dec_lmhead(const uint16_t *W, int K, int N, const float *x, const uint16_t *lnw,
                                         float eps, float *y, void *stream);
/* Attention runs NH * SGPU_ATTN_SPLITS blocks (position chunks of one head each); ws holds
 * SGPU_ATTN_WS_FLOATS(NH, HD) floats of chunk partials and cnt NH zero-initialised counters
 * (each kernel leaves them at zero).  SGPU_ATTN_SPLITS matches kAttnSplits in sgpu_decode.hip. */
#define SGPU_ATTN_SPLITS 32
#define SGPU_ATTN_WS_FLOATS(NH, HD) ((size_t)(NH) * SGPU_ATTN_SPLITS * ((HD) + 2))
SGPU_HIDDEN int sgpu_internal_dec_attn(const float *q, const float *kc, const float *vc, float *out,
                                       const int *step, int NH, int NKV, int HD, float scale, float *ws,
                                       unsigned *cnt, void *stream);
SGPU_HIDDEN int sgpu_internal_dec_embed(const uint16_t *emb, int token, int pos, float *x, int C, int *step,
                                        void *stream);
/* Greedy step tail: two-stage argmax of v (SGPU_ARGMAX_PARTS partial (value, index) pairs in
 * part_v / part_i); the second stage writes the token to step[0] (and out[step[1] + 1] if out
 * != NULL), advances step[1] and writes the next position's input x: h2f(emb[token]) when emb
 * != NULL, else wte[token] + wpe[step[1]] while step[1] < ctx. */
#define SGPU_ARGMAX_PARTS 256
SGPU_HIDDEN int sgpu_internal_dec_argmax_next(const float *v, int n, float *part_v, int *part_i, int *step, int *out,
                                              const uint16_t *emb, const float *wte, const float *wpe, float *x,
                                              int C, int ctx, void *stream);
/* Batched prompt prefill of the Qwen engine (qwen.c sgpu_qwen_prefill): row embedding, the
 * fp16-weight matrix-core GEMM Y[T][N] = X[T][K] W[N][K]^T + bias, RoPE of q in place and
 * of k into the key cache with v into the value cache, causal attention of T prompt rows
 * (positions pos0..pos0+T-1, pos0 + T <= 8192), and row SwiGLU over gate|up rows of 2*FC. */
SGPU_HIDDEN int sgpu_internal_pf_embed(const uint16_t *emb, const int *ids, int T, float *x, int C, void *stream);
/* accum != 0: Y += X W^T (+ bias), the residual add fused into the GEMM. */
SGPU_HIDDEN int sgpu_internal_pf_gemm(const uint16_t *W, const float *X, const float *bias, float *Y, int K, int N,
                                      int T, float *ws, unsigned *cnt, int accum, void *stream);
/* gemv_multi with an explicit split-K workspace (NULL: never split). */
SGPU_HIDDEN int sgpu_internal_gemv_multi(const float *W, const float *X, const float *bias, float *Y, int K, int N,
                                         int T, float *ws, unsigned *cnt, void *stream);
/* Split-K workspace of the batched matrix-core GEMMs (sgpu_internal_pf_gemm,
 * sgpu_internal_gemv_multi): SGPU_NT_WS_FLOATS floats of partial tiles and SGPU_NT_CNT
 * counters, zeroed once (every launch leaves them at zero). */
#define SGPU_NT_WS_FLOATS (1u << 20)
#define SGPU_NT_CNT 1024u
SGPU_HIDDEN int sgpu_internal_pf_qkv_post(float *qkv, int T, int pos0, const float *cosT, const float *sinT,
                                          float *kc, float *vc, int NH, int NKV, int HD, void *stream);
SGPU_HIDDEN int sgpu_internal_pf_attn(const float *qkv, const float *kc, const float *vc, float *out, int T,
                                      int pos0, int NH, int NKV, int HD, float scale, void *stream);
SGPU_HIDDEN int sgpu_internal_pf_swiglu(const float *Y, float *G, int FC, int T, void *stream);
/* GPT-2 fused decode (fp32 weights), see gpt2.c. */
SGPU_HIDDEN int sgpu_internal_g2_qkv(const float *W, int K, int N, const float *x, const float *lnw,
                                     const float *lnb, float eps, const float *bias, float *q, float *kc,
                                     float *vc, const int *step, void *stream);
SGPU_HIDDEN int sgpu_internal_g2_res(const float *W, int K, int N, const float *a, const float *bias, float *x,
                                     void *stream);
SGPU_HIDDEN int sgpu_internal_g2_fc(const float *W, int K, int N, const float *x, const float *lnw,
                                    const float *lnb, float eps, const float *bias, float *y, void *stream);
SGPU_HIDDEN int sgpu_internal_g2_lmhead(const float *W, int K, int N, const float *x, const float *lnw,
                                        const float *lnb, float eps, float *y, void *stream);
SGPU_HIDDEN int sgpu_internal_g2_embed(const float *wte, const float *wpe, int token, int pos, float *x, int C,
                                       int *step, void *stream);
/* The allocation-free split-K entry point's fixed device scratch (sgpu_scratch.hip): room for
 * SGPU_SCRATCH_FLOATS floats of partial tiles (32 MiB: S x tiles x 4096 <= 8 Mi) and
 * SGPU_SCRATCH_TILES tile counters, one copy per device.  setup resolves the current device's
 * copy and zeroes its counters (once per device, from the library's device set-up); scratch
 * returns the device's pointers, SGPU_ERR_NOT_INITIALIZED before setup. */
#define SGPU_SCRATCH_FLOATS (8u << 20)
#define SGPU_SCRATCH_TILES 16384u
SGPU_HIDDEN int sgpu_internal_scratch_setup(int dev);
SGPU_HIDDEN int sgpu_internal_scratch(int dev, float **ws, unsigned **cnt);

/* A stage vector of a traced forward: the stream's work so far waited for, the n floats at
 * dev (at most cap) copied to host and handed to fn. */
typedef struct {
    sgpu_stage_fn fn;
    void *ctx;
    float *host;                  /* scratch of cap floats */
    int cap;
} sgpu_stage_sink;
SGPU_HIDDEN int sgpu_internal_stage_out(void *stream, sgpu_stage_sink *k, const char *tag, const float *dev, int n);

#ifdef __cplusplus
}
#endif
#endif
