/* gpt2.c -- GPT-2 124M fp32 decode engine over the C-ABI launchers (part of libswitchgpu.so).
 *
 * The device side of gpt2_engine.c: weight upload and buffers (gpu_setup, :108-166), the
 * per-position forward (gpu_forward, :174-264) with its --fused variant (gemv_warp_b instead
 * of gemv_warp + add_bias), and the batched prompt prefill (gpu_prefill, :269-326) that runs
 * every projection through the weight-stationary gemv_multi.
 * Weight layout (gpt2_engine.c:10-13,50-70; writer conv_gpt2.py:37-52), fp32:
 *   wte[V*C] wpe[CTX*C] { ln1_w ln1_b qkv_w[3C*C] qkv_b[3C] ao_w[C*C] ao_b ln2_w ln2_b
 *   fc_w[FC*C] fc_b[FC] proj_w[C*FC] proj_b } x NL, ln_f_w[C] ln_f_b[C]
 */
#define __HIP_PLATFORM_AMD__ 1
#include <hip/hip_runtime_api.h>

#include <stdlib.h>
#include <string.h>

#include "sgpu_internal.h"
#include "switch_gpu.h"

typedef struct {
    size_t wte, wpe, l_base, lstride, lnfw, lnfb, total;                       /* floats */
    size_t ln1w, ln1b, qkvw, qkvb, aow, aob, ln2w, ln2b, fcw, fcb, projw, projb;  /* in-layer */
} g2layout;

static void g2_layout(const sgpu_gpt2_cfg *c, g2layout *L) {
    const size_t C = (size_t)c->C, FC = (size_t)c->FC;
    L->wte = 0;
    L->wpe = (size_t)c->V * C;
    L->l_base = L->wpe + (size_t)c->CTX * C;
    L->lstride = 2 * C + 3 * C * C + 3 * C + C * C + C + 2 * C + FC * C + FC + FC * C + C;
    L->lnfw = L->l_base + (size_t)c->NL * L->lstride;
    L->lnfb = L->lnfw + C;
    L->total = L->lnfb + C;
    L->ln1w = 0; L->ln1b = C; L->qkvw = 2 * C; L->qkvb = L->qkvw + 3 * C * C; L->aow = L->qkvb + 3 * C;
    L->aob = L->aow + C * C; L->ln2w = L->aob + C; L->ln2b = L->ln2w + C; L->fcw = L->ln2b + C;
    L->fcb = L->fcw + FC * C; L->projw = L->fcb + FC; L->projb = L->projw + FC * C;
}

static int cfg_ok(const sgpu_gpt2_cfg *c) {
    /* the attention kernels fix 12 heads of 64 in rows of 768 (gpt2_kernels.cu:5) */
    return c && c->C == 768 && c->NH == 12 && c->HD == 64 && c->V > 0 && c->NL > 0 && c->FC > 0 &&
           c->CTX > 0 && (long long)c->CTX * c->FC < 0x7fffffffLL;
}

void sgpu_gpt2_default_cfg(sgpu_gpt2_cfg *c) {
    c->V = 50257; c->C = 768; c->NL = 12; c->NH = 12; c->HD = 64; c->FC = 3072; c->CTX = 1024; c->eps = 1e-5f;
}

size_t sgpu_gpt2_file_floats(const sgpu_gpt2_cfg *c) {
    if (!cfg_ok(c)) return 0;
    g2layout L;
    g2_layout(c, &L);
    return L.total;
}

int sgpu_gpt2_fill_random(float *blob, const sgpu_gpt2_cfg *c, uint64_t seed, float amp) {
    if (!blob || !cfg_ok(c)) return SGPU_ERR_INVALID_ARG;
    g2layout L;
    g2_layout(c, &L);
    uint64_t s = seed;
    sgpu_gen_uniform(blob, L.total, &s, -0.5f);
    for (size_t i = 0; i < L.total; i++) blob[i] *= 2.0f * amp;
    return SGPU_OK;
}

struct sgpu_gpt2 {
    sgpu_gpt2_cfg cfg;
    g2layout L;
    int path;                                       /* SGPU_GPT2_PATH_* */
    hipStream_t stream;
    float *w;                                       /* the whole weight file on the device */
    float **kc, **vc;
    float *x, *ln1, *qkv, *att, *y, *ln2, *fc, *scores, *probs, *logits, *x2;
    float *xT, *ln1T, *qkvT, *attT, *yT, *ln2T, *fcT;     /* batched prefill */
    float *d_q;                                     /* q of the fused path */
    int *d_step;                                    /* {token, pos} read by the fused kernels */
    int *d_tokens;                                  /* CTX + 1 greedy ids, by position */
    float *d_amax_v;                                /* argmax partials */
    int *d_amax_i;
    float *d_attn_ws;                               /* attention chunk partials */
    unsigned *d_attn_cnt;                           /* per-head chunk counters (kept at zero) */
    float *d_split_ws;                              /* prefill GEMM k-split partials */
    unsigned *d_split_cnt;                          /* ... and per-tile counters (kept at zero) */
    hipGraph_t g_layers, g_step;
    hipGraphExec_t ge_layers, ge_step;
};

void sgpu_gpt2_destroy(sgpu_gpt2 *e) {
    if (!e) return;
    /* the stream's work finishes, then the graphs that reference the buffers go, then the
     * buffers, then the stream */
    if (e->stream) hipStreamSynchronize(e->stream);
    if (e->ge_layers) hipGraphExecDestroy(e->ge_layers);
    if (e->g_layers) hipGraphDestroy(e->g_layers);
    if (e->ge_step) hipGraphExecDestroy(e->ge_step);
    if (e->g_step) hipGraphDestroy(e->g_step);
    float *bufs[] = {e->w, e->x, e->ln1, e->qkv, e->att, e->y, e->ln2, e->fc, e->scores, e->probs, e->logits,
                     e->x2, e->xT, e->ln1T, e->qkvT, e->attT, e->yT, e->ln2T, e->fcT, e->d_q, e->d_amax_v,
                     e->d_attn_ws, e->d_split_ws};
    for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; i++) sgpu_free(bufs[i]);
    sgpu_free(e->d_step);
    sgpu_free(e->d_tokens);
    sgpu_free(e->d_amax_i);
    sgpu_free(e->d_attn_cnt);
    sgpu_free(e->d_split_cnt);
    for (int l = 0; l < e->cfg.NL; l++) {
        if (e->kc) sgpu_free(e->kc[l]);
        if (e->vc) sgpu_free(e->vc[l]);
    }
    free(e->kc);
    free(e->vc);
    if (e->stream) hipStreamDestroy(e->stream);
    free(e);
}

static int zalloc(float **p, size_t floats) {
    int rc = sgpu_malloc((void **)p, floats * 4);
    if (rc) return rc;
    return sgpu_memset_d8(*p, 0, floats * 4);
}

int sgpu_gpt2_create(sgpu_gpt2 **out, const sgpu_gpt2_cfg *c, const float *blob) {
    if (!out || !blob || !cfg_ok(c)) return SGPU_ERR_INVALID_ARG;
    *out = NULL;
    int dev = 0, rc;
    if (hipGetDevice(&dev) != hipSuccess) return SGPU_ERR_NO_DEVICE;
    if ((rc = sgpu_init(dev))) return rc;
    sgpu_gpt2 *e = calloc(1, sizeof *e);
    if (!e) return SGPU_ERR_HOST_ALLOC;
    e->cfg = *c;
    g2_layout(c, &e->L);
    const size_t C = (size_t)c->C, FC = (size_t)c->FC, CTX = (size_t)c->CTX;
#define TRY(x) do { if ((rc = (x))) goto fail; } while (0)
    if (hipStreamCreate(&e->stream) != hipSuccess) { rc = SGPU_ERR_NO_DEVICE; goto fail; }
    e->kc = calloc((size_t)c->NL, sizeof(float *));
    e->vc = calloc((size_t)c->NL, sizeof(float *));
    if (!e->kc || !e->vc) { rc = SGPU_ERR_HOST_ALLOC; goto fail; }
    TRY(sgpu_malloc((void **)&e->w, e->L.total * 4));
    TRY(sgpu_memcpy_htod(e->w, blob, e->L.total * 4));
    for (int l = 0; l < c->NL; l++) {
        TRY(zalloc(&e->kc[l], CTX * C));
        TRY(zalloc(&e->vc[l], CTX * C));
    }
    TRY(zalloc(&e->x, C)); TRY(zalloc(&e->ln1, C)); TRY(zalloc(&e->qkv, 3 * C)); TRY(zalloc(&e->att, C));
    TRY(zalloc(&e->y, C)); TRY(zalloc(&e->ln2, C)); TRY(zalloc(&e->fc, FC)); TRY(zalloc(&e->x2, C));
    TRY(zalloc(&e->scores, CTX * 12)); TRY(zalloc(&e->probs, CTX * 12)); TRY(zalloc(&e->logits, (size_t)c->V));
    TRY(zalloc(&e->xT, CTX * C)); TRY(zalloc(&e->ln1T, CTX * C)); TRY(zalloc(&e->qkvT, CTX * 3 * C));
    TRY(zalloc(&e->attT, CTX * C)); TRY(zalloc(&e->yT, CTX * C)); TRY(zalloc(&e->ln2T, CTX * C));
    TRY(zalloc(&e->fcT, CTX * FC));
    TRY(zalloc(&e->d_q, C));
    TRY(zalloc(&e->d_amax_v, SGPU_ARGMAX_PARTS));
    TRY(sgpu_malloc((void **)&e->d_amax_i, SGPU_ARGMAX_PARTS * sizeof(int)));
    TRY(sgpu_malloc((void **)&e->d_step, 4 * sizeof(int)));
    TRY(sgpu_memset_d8(e->d_step, 0, 4 * sizeof(int)));
    TRY(sgpu_malloc((void **)&e->d_tokens, (CTX + 1) * sizeof(int)));
    TRY(zalloc(&e->d_attn_ws, SGPU_ATTN_WS_FLOATS(c->NH, c->HD)));
    TRY(sgpu_malloc((void **)&e->d_attn_cnt, (size_t)c->NH * sizeof(unsigned)));
    TRY(sgpu_memset_d8(e->d_attn_cnt, 0, (size_t)c->NH * sizeof(unsigned)));
    TRY(zalloc(&e->d_split_ws, SGPU_NT_WS_FLOATS));
    TRY(sgpu_malloc((void **)&e->d_split_cnt, SGPU_NT_CNT * sizeof(unsigned)));
    TRY(sgpu_memset_d8(e->d_split_cnt, 0, SGPU_NT_CNT * sizeof(unsigned)));
#undef TRY
    *out = e;
    return SGPU_OK;
fail:
    sgpu_gpt2_destroy(e);
    return rc;
}

static int logits_out(sgpu_gpt2 *e, const float *xrow, float *logits_host) {
    const int C = e->cfg.C;
    void *s = (void *)e->stream;
    const float *W = e->w;
    int rc;
    if ((rc = sgpu_layernorm(xrow, W + e->L.lnfw, W + e->L.lnfb, e->x2, C, e->cfg.eps, 1, s))) return rc;
    if ((rc = sgpu_gemv_warp(W + e->L.wte, e->x2, e->logits, C, e->cfg.V, s))) return rc;   /* tied lm_head */
    if (logits_host) {
        hipError_t he = hipMemcpyAsync(logits_host, e->logits, (size_t)e->cfg.V * 4, hipMemcpyDeviceToHost, e->stream);
        if (he != hipSuccess) return (int)he;
        return sgpu_stream_synchronize(s);
    }
    return SGPU_OK;
}

/* One projection y = W x + b, fused (gemv_warp_b) or as the reference's two launches. */
static int proj(const float *W, const float *x, const float *b, float *y, int K, int N, int fused, void *s) {
    if (fused) return sgpu_gemv_warp_b(W, x, b, y, K, N, s);
    int rc = sgpu_gemv_warp(W, x, y, K, N, s);
    return rc ? rc : sgpu_add_bias(y, b, N, s);
}

/* ---- fused path: five kernels per layer (sgpu_decode.hip g2 families) ----
 * LayerNorm + qkv + bias + K/V cache write; attention (one block per head); o + bias +
 * residual; LayerNorm + fc + bias + GELU; proj + bias + residual.  Same arithmetic as the
 * reference sequence below, grouped so each kernel streams one weight matrix. */
static int fused_layers(sgpu_gpt2 *e) {
    const sgpu_gpt2_cfg *c = &e->cfg;
    const int C = c->C, FC = c->FC;
    const float eps = c->eps;
    void *s = (void *)e->stream;
    const float *W = e->w;
    int rc;
#define TRY(x) do { if ((rc = (x))) return rc; } while (0)
    for (int l = 0; l < c->NL; l++) {
        const float *b = W + e->L.l_base + (size_t)l * e->L.lstride;
        TRY(sgpu_internal_g2_qkv(b + e->L.qkvw, C, 3 * C, e->x, b + e->L.ln1w, b + e->L.ln1b, eps, b + e->L.qkvb,
                                 e->d_q, e->kc[l], e->vc[l], e->d_step, s));
        TRY(sgpu_internal_dec_attn(e->d_q, e->kc[l], e->vc[l], e->att, e->d_step, c->NH, c->NH, c->HD, 0.125f,
                                   e->d_attn_ws, e->d_attn_cnt, s));
        TRY(sgpu_internal_g2_res(b + e->L.aow, C, C, e->att, b + e->L.aob, e->x, s));
        TRY(sgpu_internal_g2_fc(b + e->L.fcw, C, FC, e->x, b + e->L.ln2w, b + e->L.ln2b, eps, b + e->L.fcb, e->fc, s));
        TRY(sgpu_internal_g2_res(b + e->L.projw, FC, C, e->fc, b + e->L.projb, e->x, s));
    }
#undef TRY
    return SGPU_OK;
}

static int fused_lm_head(sgpu_gpt2 *e) {
    const float *W = e->w;
    return sgpu_internal_g2_lmhead(W + e->L.wte, e->cfg.C, e->cfg.V, e->x, W + e->L.lnfw, W + e->L.lnfb, e->cfg.eps,
                                   e->logits, (void *)e->stream);
}

/* Greedy argmax of the logits into step[0] and the token list, then the next position's
 * input: x = wte[token] + wpe[step[1] + 1], step[1] + 1. */
static int argmax_next(sgpu_gpt2 *e) {
    const float *W = e->w;
    return sgpu_internal_dec_argmax_next(e->logits, e->cfg.V, e->d_amax_v, e->d_amax_i, e->d_step, e->d_tokens, NULL,
                                         W + e->L.wte, W + e->L.wpe, e->x, e->cfg.C, e->cfg.CTX, (void *)e->stream);
}

/* One greedy step on the device, x and step already set for its position. */
static int device_step(sgpu_gpt2 *e) {
    int rc = fused_layers(e);
    if (!rc) rc = fused_lm_head(e);
    if (!rc) rc = argmax_next(e);
    return rc;
}

static int capture(sgpu_gpt2 *e, int (*fn)(sgpu_gpt2 *), hipGraph_t *g, hipGraphExec_t *ge) {
    hipError_t he = hipStreamBeginCapture(e->stream, hipStreamCaptureModeRelaxed);
    if (he != hipSuccess) return (int)he;
    int rc = fn(e);
    hipGraph_t graph = NULL;
    he = hipStreamEndCapture(e->stream, &graph);
    if (rc || he != hipSuccess) {
        if (graph) hipGraphDestroy(graph);
        return rc ? rc : (int)he;
    }
    he = hipGraphInstantiate(ge, graph, NULL, NULL, 0);
    if (he != hipSuccess) {
        hipGraphDestroy(graph);
        return (int)he;
    }
    *g = graph;
    return SGPU_OK;
}

static int run_layers(sgpu_gpt2 *e) {
    if (e->path != SGPU_GPT2_PATH_GRAPH) return fused_layers(e);
    if (!e->ge_layers) {
        int rc = capture(e, fused_layers, &e->g_layers, &e->ge_layers);
        if (rc) return rc;
    }
    hipError_t he = hipGraphLaunch(e->ge_layers, e->stream);
    return he == hipSuccess ? SGPU_OK : (int)he;
}

int sgpu_gpt2_set_path(sgpu_gpt2 *e, int path) {
    if (!e || path < SGPU_GPT2_PATH_REFERENCE || path > SGPU_GPT2_PATH_GRAPH) return SGPU_ERR_INVALID_ARG;
    /* the fused attention keeps at most 8192 cached positions */
    if (path != SGPU_GPT2_PATH_REFERENCE && e->cfg.CTX > 8192) return SGPU_ERR_INVALID_ARG;
    e->path = path;
    return SGPU_OK;
}

static int forward_fused(sgpu_gpt2 *e, int token, int pos, int want_logits, float *logits_host) {
    const float *W = e->w;
    int rc = sgpu_internal_g2_embed(W + e->L.wte, W + e->L.wpe, token, pos, e->x, e->cfg.C, e->d_step,
                                    (void *)e->stream);
    if (!rc) rc = run_layers(e);
    if (rc || !want_logits) return rc;
    if ((rc = fused_lm_head(e))) return rc;
    if (!logits_host) return SGPU_OK;
    hipError_t he = hipMemcpyAsync(logits_host, e->logits, (size_t)e->cfg.V * 4, hipMemcpyDeviceToHost, e->stream);
    if (he != hipSuccess) return (int)he;
    return sgpu_stream_synchronize((void *)e->stream);
}

/* gpu_forward (gpt2_engine.c:174-264), `fused` = its --fused variant.  With trace_host, the
 * residual after each layer is copied there (NL x C floats, gpu_forward's trace argument). */
static int forward_reference(sgpu_gpt2 *e, int token, int pos, int want_logits, float *logits_host, int fused,
                             float *trace_host, sgpu_stage_sink *sink) {
    const sgpu_gpt2_cfg *c = &e->cfg;
    const int C = c->C, FC = c->FC, T = pos + 1;
    const float eps = c->eps, scale = 0.125f;   /* 1/sqrt(64), gpt2_engine.c:75 */
    void *s = (void *)e->stream;
    const float *W = e->w;
    int rc;
#define TRY(x) do { if ((rc = (x))) return rc; } while (0)
#define STAGE(tag, dev, n) do { if (sink && l == 0) TRY(sgpu_internal_stage_out(s, sink, tag, dev, n)); } while (0)
    const int NH = c->NH;
    /* x = wte[token] + wpe[pos] (the reference adds on the host, gpt2_engine.c:176-179) */
    TRY(sgpu_add2(W + e->L.wte + (size_t)token * C, W + e->L.wpe + (size_t)pos * C, e->x, C, s));
    for (int l = 0; l < c->NL; l++) {
        const float *b = W + e->L.l_base + (size_t)l * e->L.lstride;
        TRY(sgpu_layernorm(e->x, b + e->L.ln1w, b + e->L.ln1b, e->ln1, C, eps, 1, s));
        STAGE("ln1", e->ln1, C);
        TRY(proj(b + e->L.qkvw, e->ln1, b + e->L.qkvb, e->qkv, C, 3 * C, fused, s));
        STAGE("qkv", e->qkv, 3 * C);
        TRY(sgpu_memcpy_dtod_async(e->kc[l] + (size_t)pos * C, e->qkv + C, (size_t)C * 4, s));
        TRY(sgpu_memcpy_dtod_async(e->vc[l] + (size_t)pos * C, e->qkv + 2 * C, (size_t)C * 4, s));
        TRY(sgpu_gpt2_attn_scores(e->qkv, e->kc[l], e->scores, T, scale, s));
        TRY(sgpu_gpt2_attn_softmax(e->scores, e->probs, T, s));
        TRY(sgpu_gpt2_attn_mix(e->probs, e->vc[l], e->att, T, s));
        STAGE("scores", e->scores, T * NH);
        STAGE("probs", e->probs, T * NH);
        STAGE("attnout", e->att, C);
        TRY(proj(b + e->L.aow, e->att, b + e->L.aob, e->y, C, C, fused, s));
        STAGE("ao", e->y, C);
        TRY(sgpu_add2(e->x, e->y, e->x, C, s));
        STAGE("res1", e->x, C);
        TRY(sgpu_layernorm(e->x, b + e->L.ln2w, b + e->L.ln2b, e->ln2, C, eps, 1, s));
        STAGE("ln2", e->ln2, C);
        TRY(proj(b + e->L.fcw, e->ln2, b + e->L.fcb, e->fc, C, FC, fused, s));
        STAGE("fc", e->fc, FC);
        TRY(sgpu_gelu(e->fc, e->fc, FC, s));
        STAGE("gelu", e->fc, FC);
        TRY(proj(b + e->L.projw, e->fc, b + e->L.projb, e->y, FC, C, fused, s));
        STAGE("proj", e->y, C);
        TRY(sgpu_add2(e->x, e->y, e->x, C, s));
        STAGE("res2", e->x, C);
        if (trace_host) {
            hipError_t he = hipMemcpyAsync(trace_host + (size_t)l * C, e->x, (size_t)C * 4, hipMemcpyDeviceToHost,
                                           e->stream);
            if (he != hipSuccess) return (int)he;
        }
    }
    if (trace_host) TRY(sgpu_stream_synchronize(s));
#undef STAGE
#undef TRY
    return want_logits ? logits_out(e, e->x, logits_host) : SGPU_OK;
}

int sgpu_gpt2_forward(sgpu_gpt2 *e, int token, int pos, int want_logits, float *logits_host, int fused) {
    if (!e) return SGPU_ERR_INVALID_ARG;
    if (token < 0 || token >= e->cfg.V || pos < 0 || pos >= e->cfg.CTX) return SGPU_ERR_INVALID_ARG;
    if (e->path != SGPU_GPT2_PATH_REFERENCE) return forward_fused(e, token, pos, want_logits, logits_host);
    return forward_reference(e, token, pos, want_logits, logits_host, fused, NULL, NULL);
}

int sgpu_gpt2_forward_trace(sgpu_gpt2 *e, int token, int pos, float *logits_host, float *trace_host, int fused) {
    if (!e || !trace_host) return SGPU_ERR_INVALID_ARG;
    if (token < 0 || token >= e->cfg.V || pos < 0 || pos >= e->cfg.CTX) return SGPU_ERR_INVALID_ARG;
    return forward_reference(e, token, pos, logits_host != NULL, logits_host, fused, trace_host, NULL);
}

int sgpu_gpt2_forward_stages(sgpu_gpt2 *e, int token, int pos, float *logits_host, int fused, sgpu_stage_fn fn,
                             void *ctx) {
    if (!e || !fn) return SGPU_ERR_INVALID_ARG;
    const sgpu_gpt2_cfg *c = &e->cfg;
    if (token < 0 || token >= c->V || pos < 0 || pos >= c->CTX) return SGPU_ERR_INVALID_ARG;
    int cap = 3 * c->C > c->FC ? 3 * c->C : c->FC;
    if ((pos + 1) * c->NH > cap) cap = (pos + 1) * c->NH;
    sgpu_stage_sink sink = {fn, ctx, malloc(sizeof(float) * (size_t)cap), cap};
    if (!sink.host) return SGPU_ERR_HOST_ALLOC;
    int rc = forward_reference(e, token, pos, logits_host != NULL, logits_host, fused, NULL, &sink);
    free(sink.host);
    return rc;
}

/* gpu_prefill's layer loop: all T prompt rows through each layer, cache positions 0..T-1
 * filled, the final rows left in xT.  Attention: the reference's per-row launches (k/v copies,
 * scores, softmax, mix for each row), or -- with the cache within 8192 positions -- two
 * strided copies of every row's k and v into the caches and one launch of the batched causal
 * attention (one block per head and row, same arithmetic as the fused decode attention). */
static int prefill_layers(sgpu_gpt2 *e, const int *ids, int T) {
    const sgpu_gpt2_cfg *c = &e->cfg;
    const int C = c->C, FC = c->FC;
    const float eps = c->eps, scale = 0.125f;
    void *s = (void *)e->stream;
    const float *W = e->w;
    int rc;
#define TRY(x) do { if ((rc = (x))) return rc; } while (0)
    for (int t = 0; t < T; t++)
        TRY(sgpu_add2(W + e->L.wte + (size_t)ids[t] * C, W + e->L.wpe + (size_t)t * C, e->xT + (size_t)t * C, C, s));
    for (int l = 0; l < c->NL; l++) {
        const float *b = W + e->L.l_base + (size_t)l * e->L.lstride;
        TRY(sgpu_layernorm(e->xT, b + e->L.ln1w, b + e->L.ln1b, e->ln1T, C, eps, T, s));
        TRY(sgpu_internal_gemv_multi(b + e->L.qkvw, e->ln1T, b + e->L.qkvb, e->qkvT, C, 3 * C, T,
            e->d_split_ws, e->d_split_cnt, s));
        if (T <= 8192) {
            const size_t row = (size_t)C * 4, qrow = 3 * row;
            hipError_t he = hipMemcpy2DAsync(e->kc[l], row, e->qkvT + C, qrow, row, (size_t)T, hipMemcpyDeviceToDevice,
                                             e->stream);
            if (he == hipSuccess)
                he = hipMemcpy2DAsync(e->vc[l], row, e->qkvT + 2 * C, qrow, row, (size_t)T, hipMemcpyDeviceToDevice,
                                      e->stream);
            if (he != hipSuccess) return (int)he;
            TRY(sgpu_internal_pf_attn(e->qkvT, e->kc[l], e->vc[l], e->attT, T, 0, c->NH, c->NH, c->HD, scale, s));
        } else {
            for (int t = 0; t < T; t++) {     /* causal attention, one query row at a time */
                const float *qrow = e->qkvT + (size_t)t * 3 * C;
                TRY(sgpu_memcpy_dtod_async(e->kc[l] + (size_t)t * C, qrow + C, (size_t)C * 4, s));
                TRY(sgpu_memcpy_dtod_async(e->vc[l] + (size_t)t * C, qrow + 2 * C, (size_t)C * 4, s));
                TRY(sgpu_gpt2_attn_scores(qrow, e->kc[l], e->scores, t + 1, scale, s));
                TRY(sgpu_gpt2_attn_softmax(e->scores, e->probs, t + 1, s));
                TRY(sgpu_gpt2_attn_mix(e->probs, e->vc[l], e->attT + (size_t)t * C, t + 1, s));
            }
        }
        TRY(sgpu_internal_gemv_multi(b + e->L.aow, e->attT, b + e->L.aob, e->yT, C, C, T,
            e->d_split_ws, e->d_split_cnt, s));
        TRY(sgpu_add2(e->xT, e->yT, e->xT, T * C, s));
        TRY(sgpu_layernorm(e->xT, b + e->L.ln2w, b + e->L.ln2b, e->ln2T, C, eps, T, s));
        TRY(sgpu_internal_gemv_multi(b + e->L.fcw, e->ln2T, b + e->L.fcb, e->fcT, C, FC, T,
            e->d_split_ws, e->d_split_cnt, s));
        TRY(sgpu_gelu(e->fcT, e->fcT, T * FC, s));
        TRY(sgpu_internal_gemv_multi(b + e->L.projw, e->fcT, b + e->L.projb, e->yT, FC, C, T,
            e->d_split_ws, e->d_split_cnt, s));
        TRY(sgpu_add2(e->xT, e->yT, e->xT, T * C, s));
    }
#undef TRY
    return SGPU_OK;
}

int sgpu_gpt2_prefill(sgpu_gpt2 *e, const int *ids, int T, float *logits_host) {
    if (!e || !ids) return SGPU_ERR_INVALID_ARG;
    const sgpu_gpt2_cfg *c = &e->cfg;
    if (T <= 0 || T > c->CTX) return SGPU_ERR_INVALID_ARG;
    for (int t = 0; t < T; t++)
        if (ids[t] < 0 || ids[t] >= c->V) return SGPU_ERR_INVALID_ARG;
    int rc = prefill_layers(e, ids, T);
    return rc ? rc : logits_out(e, e->xT + (size_t)(T - 1) * c->C, logits_host);
}

int sgpu_gpt2_generate(sgpu_gpt2 *e, const int *prompt, int T, int n_gen, int *out_tokens) {
    if (!e || !prompt || !out_tokens || T <= 0 || n_gen < 0) return SGPU_ERR_INVALID_ARG;
    const sgpu_gpt2_cfg *c = &e->cfg;
    if ((long long)T + n_gen > c->CTX) return SGPU_ERR_INVALID_ARG;
    for (int p = 0; p < T; p++)
        if (prompt[p] < 0 || prompt[p] >= c->V) return SGPU_ERR_INVALID_ARG;
    int rc = SGPU_OK;
    if (e->path == SGPU_GPT2_PATH_REFERENCE) {       /* host-driven loop, the reference's own */
        float *logits = malloc(sizeof(float) * (size_t)c->V);
        if (!logits) return SGPU_ERR_HOST_ALLOC;
        for (int p = 0; p < T && !(rc = sgpu_gpt2_forward(e, prompt[p], p, p == T - 1, logits, 0)); p++) {
        }
        for (int g = 0; !rc && g <= n_gen; g++) {
            int b = 0;
            for (int i = 1; i < c->V; i++)
                if (logits[i] > logits[b]) b = i;
            out_tokens[g] = b;
            if (g < n_gen) rc = sgpu_gpt2_forward(e, b, T + g, 1, logits, 0);
        }
        free(logits);
        return rc;
    }
    /* the prompt in one batched pass; the last row through the fused lm_head, and the step
     * record {prompt[T-1], T-1} so the on-device loop continues at position T */
    if ((rc = prefill_layers(e, prompt, T))) return rc;
    if ((rc = sgpu_memcpy_dtod_async(e->x, e->xT + (size_t)(T - 1) * c->C, (size_t)c->C * 4, (void *)e->stream)) ||
        (rc = fused_lm_head(e)))
        return rc;
    const int st[2] = {prompt[T - 1], T - 1};
    hipError_t hs = hipMemcpyAsync(e->d_step, st, sizeof st, hipMemcpyHostToDevice, e->stream);
    if (hs != hipSuccess) return (int)hs;
    if ((rc = argmax_next(e))) return rc;
    for (int g = 0; g < n_gen; g++) {
        if (e->path == SGPU_GPT2_PATH_GRAPH) {
            if (!e->ge_step && (rc = capture(e, device_step, &e->g_step, &e->ge_step))) return rc;
            hipError_t he = hipGraphLaunch(e->ge_step, e->stream);
            if (he != hipSuccess) return (int)he;
        } else if ((rc = device_step(e))) {
            return rc;
        }
    }
    hipError_t he = hipMemcpyAsync(out_tokens, e->d_tokens + T, ((size_t)n_gen + 1) * sizeof(int),
                                   hipMemcpyDeviceToHost, e->stream);
    if (he != hipSuccess) return (int)he;
    return sgpu_stream_synchronize((void *)e->stream);
}
