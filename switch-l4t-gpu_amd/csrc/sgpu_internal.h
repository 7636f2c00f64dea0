/* sgpu_internal.h -- functions shared between the library's own C files (not exported). */
#ifndef SGPU_INTERNAL_H
#define SGPU_INTERNAL_H
#include <stdint.h>

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
SGPU_HIDDEN int sgpu_internal_dec_embed_next(const uint16_t *emb, float *x, int C, int *step, void *stream);
/* Two-stage argmax: SGPU_ARGMAX_PARTS partial (value, index) pairs in part_v / part_i. */
#define SGPU_ARGMAX_PARTS 256
SGPU_HIDDEN int sgpu_internal_dec_argmax(const float *v, int n, float *part_v, int *part_i, int *step, int *out,
                                         void *stream);
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
SGPU_HIDDEN int sgpu_internal_g2_embed_next(const float *wte, const float *wpe, float *x, int C, int *step,
                                            void *stream);
#endif
