/* sgpu_internal.h -- functions shared between the library's own C files (not exported). */
#ifndef SGPU_INTERNAL_H
#define SGPU_INTERNAL_H
#include <stdint.h>

/* x[i] = h2f(emb[token*C + i]) on the device (sgpu_embed_h in the tuned code object). */
__attribute__((visibility("hidden"))) int sgpu_internal_embed_h(const uint16_t *emb, int token, float *x, int C,
                                                                void *stream);
#endif
