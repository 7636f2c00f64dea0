/* qwen.c -- Qwen2.5 decode engine over the C-ABI launchers (part of libswitchgpu.so).
 *
 * The device side of qwen_engine.c: weight upload and buffers (gpu_setup, :137-189) and
 * the per-position forward (gpu_forward, :205-269) with the reference's per-layer launch
 * sequence -- rmsnorm, gemv_h qkv (+bias), rope q, rope k, K/V cache writes, attention
 * scores / softmax / mix, gemv_h o, residual add, rmsnorm, gemv_h gate|up, swiglu, gemv_h
 * down, residual add -- then final rmsnorm and the tied lm_head gemv_h.
 * Layout of the flat weight file: qwen_engine.c:8-16,61-75 (writer conv_qwen.py:63-99).
 */
#define __HIP_PLATFORM_AMD__ 1
#include <hip/hip_runtime_api.h>

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "sgpu_internal.h"
#include "switch_gpu.h"

typedef struct {
    size_t off_emb, off_cos, off_sin, l_base, lstride, off_lnfw, bytes;      /* bytes */
    size_t li_inln, li_qkvw, li_qkvb, li_ow, li_postln, li_gateup, li_down;  /* halves */
    int kvd, qkvd;
} qlayout;

static void q_layout(const sgpu_qwen_cfg *c, qlayout *L) {
    L->kvd = c->NKV * c->HD;
    L->qkvd = c->C + 2 * L->kvd;
    L->off_emb = 0;
    L->off_cos = (size_t)c->V * c->C * 2;
    L->off_sin = L->off_cos + (size_t)c->CTX * (c->HD / 2) * 4;
    L->l_base = L->off_sin + (size_t)c->CTX * (c->HD / 2) * 4;
    L->lstride = ((size_t)c->C + (size_t)L->qkvd * c->C + L->qkvd + (size_t)c->C * c->C + c->C +
                  (size_t)2 * c->FC * c->C + (size_t)c->C * c->FC) * 2;
    L->off_lnfw = L->l_base + (size_t)c->NL * L->lstride;
    L->bytes = L->off_lnfw + (size_t)c->C * 2;
    L->li_inln = 0;
    L->li_qkvw = (size_t)c->C;
    L->li_qkvb = (size_t)c->C + (size_t)L->qkvd * c->C;
    L->li_ow = L->li_qkvb + L->qkvd;
    L->li_postln = L->li_ow + (size_t)c->C * c->C;
    L->li_gateup = L->li_postln + c->C;
    L->li_down = L->li_gateup + (size_t)2 * c->FC * c->C;
}

static int cfg_ok(const sgpu_qwen_cfg *c) {
    return c && c->V > 0 && c->C > 0 && c->NL > 0 && c->NH > 0 && c->NKV > 0 && c->HD > 0 &&
           c->HD % 2 == 0 && c->NH % c->NKV == 0 && c->FC > 0 && c->CTX > 0 &&
           (long long)c->CTX * c->NH < 0x7fffffffLL;
}

void sgpu_qwen_default_cfg(sgpu_qwen_cfg *c) {
    /* qwen_engine.c:43-55, conv_qwen.py:23-27 */
    c->V = 151936; c->C = 896; c->NL = 24; c->NH = 14; c->NKV = 2; c->HD = 64; c->FC = 4864;
    c->CTX = 8192; c->eps = 1e-6f; c->theta = 1e6f;
}

size_t sgpu_qwen_file_bytes(const sgpu_qwen_cfg *cfg) {
    if (!cfg_ok(cfg)) return 0;
    qlayout L;
    q_layout(cfg, &L);
    return L.bytes;
}

/* N(0, std) fp16 for n halves at dst, continuing the LCG stream. */
static int fill_h(uint16_t *dst, size_t n, uint64_t *state, float std, float *tmp, size_t tmp_n) {
    for (size_t done = 0; done < n;) {
        size_t c = n - done < tmp_n ? n - done : tmp_n;
        sgpu_gen_normal(tmp, c, state, 0.0f, std);
        sgpu_f32_to_f16(tmp, dst + done, c);
        done += c;
    }
    return 0;
}

int sgpu_qwen_fill_random(void *blob, const sgpu_qwen_cfg *c, uint64_t seed, float std) {
    if (!blob || !cfg_ok(c)) return SGPU_ERR_INVALID_ARG;
    qlayout L;
    q_layout(c, &L);
    const size_t tmp_n = (size_t)1 << 22;   /* even: chunks continue the pair stream exactly */
    float *tmp = malloc(tmp_n * sizeof(float));
    if (!tmp) return SGPU_ERR_HOST_ALLOC;
    unsigned char *b = (unsigned char *)blob;
    uint64_t s = seed;
    fill_h((uint16_t *)(b + L.off_emb), (size_t)c->V * c->C, &s, std, tmp, tmp_n);
    /* RoPE tables, conv_qwen.py:75-80: freq_d = theta^(-2d/HD), angle = pos*freq_d (float64). */
    float *cosT = (float *)(b + L.off_cos), *sinT = (float *)(b + L.off_sin);
    const int h2 = c->HD / 2;
    for (int p = 0; p < c->CTX; p++)
        for (int d = 0; d < h2; d++) {
            double ang = (double)p * pow((double)c->theta, -2.0 * (double)d / (double)c->HD);
            cosT[(size_t)p * h2 + d] = (float)cos(ang);
            sinT[(size_t)p * h2 + d] = (float)sin(ang);
        }
    for (int l = 0; l < c->NL; l++)
        fill_h((uint16_t *)(b + L.l_base + (size_t)l * L.lstride), L.lstride / 2, &s, std, tmp, tmp_n);
    fill_h((uint16_t *)(b + L.off_lnfw), (size_t)c->C, &s, std, tmp, tmp_n);
    free(tmp);
    return SGPU_OK;
}

struct sgpu_qwen {
    sgpu_qwen_cfg cfg;
    qlayout L;
    int path;                                  /* SGPU_QWEN_PATH_* */
    hipStream_t stream;
    int *d_step;                               /* {token, pos} read by the fused kernels */
    int *d_tokens;                             /* CTX + 1 greedy ids, indexed by position */
    float *d_q;                                /* rotated q of the fused path */
    float *d_amax_v;                           /* argmax partials */
    int *d_amax_i;
    float *d_attn_ws;                          /* attention chunk partials */
    unsigned *d_attn_cnt;                      /* per-head chunk counters (kept at zero) */
    float *d_split_ws;                         /* prefill GEMM k-split partials */
    unsigned *d_split_cnt;                     /* ... and per-tile counters (kept at zero) */
    int *d_pf_ids;                             /* batched prefill: prompt ids and row buffers */
    float *d_pf_x, *d_pf_xn, *d_pf_qkv, *d_pf_att, *d_pf_y, *d_pf_g;
    hipGraph_t g_layers, g_step;
    hipGraphExec_t ge_layers, ge_step;
    uint16_t *d_emb, *d_lnfw;
    float *d_cos, *d_sin;
    uint16_t **d_ln1w, **d_qkvw, **d_ow, **d_ln2w, **d_gateupw, **d_downw;
    float **d_qkvb, **d_kc, **d_vc;
    float *d_x, *d_ln1, *d_qkv, *d_att, *d_y, *d_ln2, *d_gate, *d_down, *d_scores, *d_probs, *d_logits, *d_x2;
};

static int dalloc(void **p, size_t bytes, const void *src) {
    int rc = sgpu_malloc(p, bytes);
    if (rc) return rc;
    if (src) return sgpu_memcpy_htod(*p, src, bytes);
    return sgpu_memset_d8(*p, 0, bytes);
}

void sgpu_qwen_destroy(sgpu_qwen *e) {
    if (!e) return;
    /* the stream's work finishes, then the graphs that reference the buffers go, then the
     * buffers, then the stream */
    if (e->stream) hipStreamSynchronize(e->stream);
    if (e->ge_layers) hipGraphExecDestroy(e->ge_layers);
    if (e->g_layers) hipGraphDestroy(e->g_layers);
    if (e->ge_step) hipGraphExecDestroy(e->ge_step);
    if (e->g_step) hipGraphDestroy(e->g_step);
    const int NL = e->cfg.NL;
    void **single[] = {(void **)&e->d_emb, (void **)&e->d_lnfw, (void **)&e->d_cos, (void **)&e->d_sin,
                       (void **)&e->d_x, (void **)&e->d_ln1, (void **)&e->d_qkv, (void **)&e->d_att,
                       (void **)&e->d_y, (void **)&e->d_ln2, (void **)&e->d_gate, (void **)&e->d_down,
                       (void **)&e->d_scores, (void **)&e->d_probs, (void **)&e->d_logits, (void **)&e->d_x2};
    for (size_t i = 0; i < sizeof single / sizeof single[0]; i++) sgpu_free(*single[i]);
    void ***arrs[] = {(void ***)&e->d_ln1w, (void ***)&e->d_qkvw, (void ***)&e->d_ow, (void ***)&e->d_ln2w,
                      (void ***)&e->d_gateupw, (void ***)&e->d_downw, (void ***)&e->d_qkvb,
                      (void ***)&e->d_kc, (void ***)&e->d_vc};
    for (size_t a = 0; a < sizeof arrs / sizeof arrs[0]; a++) {
        void **arr = *arrs[a];
        if (!arr) continue;
        for (int l = 0; l < NL; l++) sgpu_free(arr[l]);
        free(arr);
    }
    sgpu_free(e->d_step);
    sgpu_free(e->d_tokens);
    sgpu_free(e->d_q);
    sgpu_free(e->d_amax_v);
    sgpu_free(e->d_amax_i);
    sgpu_free(e->d_attn_ws);
    sgpu_free(e->d_attn_cnt);
    sgpu_free(e->d_split_ws);
    sgpu_free(e->d_split_cnt);
    sgpu_free(e->d_pf_ids);
    float *pf[] = {e->d_pf_x, e->d_pf_xn, e->d_pf_qkv, e->d_pf_att, e->d_pf_y, e->d_pf_g};
    for (size_t i = 0; i < sizeof pf / sizeof pf[0]; i++) sgpu_free(pf[i]);
    if (e->stream) hipStreamDestroy(e->stream);
    free(e);
}

int sgpu_qwen_create(sgpu_qwen **out, const sgpu_qwen_cfg *c, const void *blob) {
    if (!out || !blob || !cfg_ok(c)) return SGPU_ERR_INVALID_ARG;
    *out = NULL;
    int rc;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return SGPU_ERR_NO_DEVICE;
    if ((rc = sgpu_init(dev))) return rc;
    sgpu_qwen *e = calloc(1, sizeof *e);
    if (!e) return SGPU_ERR_HOST_ALLOC;
    e->cfg = *c;
    q_layout(c, &e->L);
    const qlayout *L = &e->L;
    const int NL = c->NL, C = c->C, FC = c->FC, QKVD = L->qkvd, KVD = L->kvd;
    const unsigned char *b = (const unsigned char *)blob;
#define TRY(x) do { if ((rc = (x))) goto fail; } while (0)
    if (hipStreamCreate(&e->stream) != hipSuccess) { rc = SGPU_ERR_NO_DEVICE; goto fail; }
    e->d_ln1w = calloc(NL, sizeof(void *)); e->d_qkvw = calloc(NL, sizeof(void *));
    e->d_ow = calloc(NL, sizeof(void *)); e->d_ln2w = calloc(NL, sizeof(void *));
    e->d_gateupw = calloc(NL, sizeof(void *)); e->d_downw = calloc(NL, sizeof(void *));
    e->d_qkvb = calloc(NL, sizeof(void *)); e->d_kc = calloc(NL, sizeof(void *));
    e->d_vc = calloc(NL, sizeof(void *));
    if (!e->d_ln1w || !e->d_qkvw || !e->d_ow || !e->d_ln2w || !e->d_gateupw || !e->d_downw || !e->d_qkvb ||
        !e->d_kc || !e->d_vc) { rc = SGPU_ERR_HOST_ALLOC; goto fail; }
    TRY(dalloc((void **)&e->d_emb, (size_t)c->V * C * 2, b + L->off_emb));
    TRY(dalloc((void **)&e->d_cos, (size_t)c->CTX * (c->HD / 2) * 4, b + L->off_cos));
    TRY(dalloc((void **)&e->d_sin, (size_t)c->CTX * (c->HD / 2) * 4, b + L->off_sin));
    TRY(dalloc((void **)&e->d_lnfw, (size_t)C * 2, b + L->off_lnfw));
    {
        float *tmp = malloc(sizeof(float) * QKVD);
        if (!tmp) { rc = SGPU_ERR_HOST_ALLOC; goto fail; }
        for (int l = 0; l < NL && !rc; l++) {
            const uint16_t *lb = (const uint16_t *)(b + L->l_base + (size_t)l * L->lstride);
            if ((rc = dalloc((void **)&e->d_ln1w[l], (size_t)C * 2, lb + L->li_inln))) break;
            if ((rc = dalloc((void **)&e->d_qkvw[l], (size_t)QKVD * C * 2, lb + L->li_qkvw))) break;
            /* q/k/v bias decoded to fp32 on the host, as qwen_engine.c:170-175 */
            for (int i = 0; i < QKVD; i++) tmp[i] = sgpu_h2f_host(lb[L->li_qkvb + i]);
            if ((rc = dalloc((void **)&e->d_qkvb[l], (size_t)QKVD * 4, tmp))) break;
            if ((rc = dalloc((void **)&e->d_ow[l], (size_t)C * C * 2, lb + L->li_ow))) break;
            if ((rc = dalloc((void **)&e->d_ln2w[l], (size_t)C * 2, lb + L->li_postln))) break;
            if ((rc = dalloc((void **)&e->d_gateupw[l], (size_t)2 * FC * C * 2, lb + L->li_gateup))) break;
            if ((rc = dalloc((void **)&e->d_downw[l], (size_t)C * FC * 2, lb + L->li_down))) break;
            if ((rc = dalloc((void **)&e->d_kc[l], (size_t)c->CTX * KVD * 4, NULL))) break;
            if ((rc = dalloc((void **)&e->d_vc[l], (size_t)c->CTX * KVD * 4, NULL))) break;
        }
        free(tmp);
        if (rc) goto fail;
    }
    TRY(dalloc((void **)&e->d_x, (size_t)C * 4, NULL));
    TRY(dalloc((void **)&e->d_ln1, (size_t)C * 4, NULL));
    TRY(dalloc((void **)&e->d_qkv, (size_t)QKVD * 4, NULL));
    TRY(dalloc((void **)&e->d_att, (size_t)C * 4, NULL));
    TRY(dalloc((void **)&e->d_y, (size_t)C * 4, NULL));
    TRY(dalloc((void **)&e->d_ln2, (size_t)C * 4, NULL));
    TRY(dalloc((void **)&e->d_gate, (size_t)2 * FC * 4, NULL));
    TRY(dalloc((void **)&e->d_down, (size_t)FC * 4, NULL));
    TRY(dalloc((void **)&e->d_scores, (size_t)c->CTX * c->NH * 4, NULL));
    TRY(dalloc((void **)&e->d_probs, (size_t)c->CTX * c->NH * 4, NULL));
    TRY(dalloc((void **)&e->d_logits, (size_t)c->V * 4, NULL));
    TRY(dalloc((void **)&e->d_x2, (size_t)C * 4, NULL));
    TRY(dalloc((void **)&e->d_step, 4 * sizeof(int), NULL));
    TRY(dalloc((void **)&e->d_tokens, ((size_t)c->CTX + 1) * sizeof(int), NULL));
    TRY(dalloc((void **)&e->d_q, (size_t)c->NH * c->HD * 4, NULL));
    TRY(dalloc((void **)&e->d_amax_v, SGPU_ARGMAX_PARTS * sizeof(float), NULL));
    TRY(dalloc((void **)&e->d_amax_i, SGPU_ARGMAX_PARTS * sizeof(int), NULL));
    TRY(dalloc((void **)&e->d_attn_ws, SGPU_ATTN_WS_FLOATS(c->NH, c->HD) * sizeof(float), NULL));
    TRY(dalloc((void **)&e->d_attn_cnt, (size_t)c->NH * sizeof(unsigned), NULL));
    TRY(dalloc((void **)&e->d_split_ws, (size_t)SGPU_NT_WS_FLOATS * sizeof(float), NULL));
    TRY(dalloc((void **)&e->d_split_cnt, (size_t)SGPU_NT_CNT * sizeof(unsigned), NULL));
#undef TRY
    *out = e;
    return SGPU_OK;
fail:
    sgpu_qwen_destroy(e);
    return rc;
}

const float *sgpu_qwen_device_logits(const sgpu_qwen *e) { return e ? e->d_logits : NULL; }

/* The reference per-layer launch sequence (gpu_forward, qwen_engine.c:205-269).  With
 * trace_host, the residual after each layer is copied there (NL x C floats, the layer
 * trace of cpu_forward, qwen_engine.c:355). */
static int forward_reference(sgpu_qwen *e, int token, int pos, int want_logits, float *logits_host,
                             float *trace_host, sgpu_stage_sink *sink) {
    const sgpu_qwen_cfg *c = &e->cfg;
    const int C = c->C, NH = c->NH, NKV = c->NKV, HD = c->HD, FC = c->FC;
    const int KVD = e->L.kvd, QKVD = e->L.qkvd, Tp = pos + 1;
    const float eps = c->eps, scale = (float)(1.0 / sqrt((double)HD));
    void *s = (void *)e->stream;
    int rc;
#define TRY(x) do { if ((rc = (x))) return rc; } while (0)
#define STAGE(tag, dev, n) do { if (sink && l == 0) TRY(sgpu_internal_stage_out(s, sink, tag, dev, n)); } while (0)
    TRY(sgpu_internal_embed_h(e->d_emb, token, e->d_x, C, s));
    for (int l = 0; l < c->NL; l++) {
        TRY(sgpu_rmsnorm(e->d_x, e->d_ln1w[l], e->d_ln1, C, eps, 1, s));
        STAGE("ln1", e->d_ln1, C);
        TRY(sgpu_gemv_h(e->d_qkvw[l], e->d_ln1, e->d_qkvb[l], e->d_qkv, C, QKVD, s));
        TRY(sgpu_rope(e->d_qkv, e->d_cos, e->d_sin, 1, NH, HD, pos, s));
        TRY(sgpu_rope(e->d_qkv + (size_t)NH * HD, e->d_cos, e->d_sin, 1, NKV, HD, pos, s));
        STAGE("qkv", e->d_qkv, QKVD);
        TRY(sgpu_memcpy_dtod_async(e->d_kc[l] + (size_t)pos * KVD, e->d_qkv + (size_t)NH * HD, (size_t)KVD * 4, s));
        TRY(sgpu_memcpy_dtod_async(e->d_vc[l] + (size_t)pos * KVD, e->d_qkv + (size_t)NH * HD + KVD,
                                   (size_t)KVD * 4, s));
        TRY(sgpu_attn_scores_gqa(e->d_qkv, e->d_kc[l], e->d_scores, Tp, scale, NH, KVD, HD, s));
        TRY(sgpu_attn_softmax(e->d_scores, e->d_probs, Tp, NH, s));
        TRY(sgpu_attn_mix_gqa(e->d_probs, e->d_vc[l], e->d_att, Tp, NH, KVD, HD, s));
        STAGE("scores", e->d_scores, Tp * NH);
        STAGE("probs", e->d_probs, Tp * NH);
        STAGE("attnout", e->d_att, C);
        TRY(sgpu_gemv_h(e->d_ow[l], e->d_att, NULL, e->d_y, C, C, s));
        TRY(sgpu_add2(e->d_x, e->d_y, e->d_x, C, s));
        STAGE("res1", e->d_x, C);
        TRY(sgpu_rmsnorm(e->d_x, e->d_ln2w[l], e->d_ln2, C, eps, 1, s));
        TRY(sgpu_gemv_h(e->d_gateupw[l], e->d_ln2, NULL, e->d_gate, C, 2 * FC, s));
        STAGE("gate", e->d_gate, FC);
        TRY(sgpu_swiglu(e->d_gate, e->d_gate + FC, e->d_down, FC, s));
        STAGE("swiglu", e->d_down, FC);
        TRY(sgpu_gemv_h(e->d_downw[l], e->d_down, NULL, e->d_y, FC, C, s));
        TRY(sgpu_add2(e->d_x, e->d_y, e->d_x, C, s));
        STAGE("res2", e->d_x, C);
        if (trace_host) {
            hipError_t he = hipMemcpyAsync(trace_host + (size_t)l * C, e->d_x, (size_t)C * 4, hipMemcpyDeviceToHost,
                                           e->stream);
            if (he != hipSuccess) return (int)he;
        }
    }
    if (trace_host) TRY(sgpu_stream_synchronize(s));
    if (!want_logits) return SGPU_OK;
    TRY(sgpu_rmsnorm(e->d_x, e->d_lnfw, e->d_x2, C, eps, 1, s));
    TRY(sgpu_gemv_h(e->d_emb, e->d_x2, NULL, e->d_logits, C, c->V, s));
    if (logits_host) {
        hipError_t he = hipMemcpyAsync(logits_host, e->d_logits, (size_t)c->V * 4, hipMemcpyDeviceToHost, e->stream);
        if (he != hipSuccess) return (int)he;
        TRY(sgpu_stream_synchronize(s));
    }
#undef STAGE
#undef TRY
    return SGPU_OK;
}

/* ---- fused path: five kernels per layer (sgpu_decode.hip) ---- */
static int fused_ok(const sgpu_qwen_cfg *c) {
    return c->CTX <= 8192 && (c->HD == 32 || c->HD == 64 || c->HD == 128) && c->C % 8 == 0 && c->FC % 8 == 0;
}

static int fused_layers(sgpu_qwen *e) {
    const sgpu_qwen_cfg *c = &e->cfg;
    const int C = c->C, NH = c->NH, NKV = c->NKV, HD = c->HD, FC = c->FC, QKVD = e->L.qkvd;
    const float eps = c->eps, scale = (float)(1.0 / sqrt((double)HD));
    void *s = (void *)e->stream;
    int rc;
#define TRY(x) do { if ((rc = (x))) return rc; } while (0)
    for (int l = 0; l < c->NL; l++) {
        TRY(sgpu_internal_dec_qkv(e->d_qkvw[l], C, QKVD, e->d_x, e->d_ln1w[l], eps, e->d_qkvb[l], e->d_q, e->d_kc[l],
                                  e->d_vc[l], e->d_cos, e->d_sin, e->d_step, NH, NKV, HD, s));
        TRY(sgpu_internal_dec_attn(e->d_q, e->d_kc[l], e->d_vc[l], e->d_att, e->d_step, NH, NKV, HD, scale,
                                   e->d_attn_ws, e->d_attn_cnt, s));
        TRY(sgpu_internal_dec_res(e->d_ow[l], C, C, e->d_att, NULL, e->d_x, s));
        TRY(sgpu_internal_dec_gateup(e->d_gateupw[l], C, FC, e->d_x, e->d_ln2w[l], eps, e->d_down, s));
        TRY(sgpu_internal_dec_res(e->d_downw[l], FC, C, e->d_down, NULL, e->d_x, s));
    }
#undef TRY
    return SGPU_OK;
}

static int lm_head(sgpu_qwen *e) {
    return sgpu_internal_dec_lmhead(e->d_emb, e->cfg.C, e->cfg.V, e->d_x, e->d_lnfw, e->cfg.eps, e->d_logits,
                                    (void *)e->stream);
}

/* Greedy argmax of the logits into step[0] and the token list, then the next position's
 * input: x = embedding of that token, step[1] + 1. */
static int argmax_next(sgpu_qwen *e) {
    return sgpu_internal_dec_argmax_next(e->d_logits, e->cfg.V, e->d_amax_v, e->d_amax_i, e->d_step, e->d_tokens,
                                         e->d_emb, NULL, NULL, e->d_x, e->cfg.C, e->cfg.CTX, (void *)e->stream);
}

/* One greedy step entirely on the device, x and step already set for its position. */
static int device_step(sgpu_qwen *e) {
    int rc = fused_layers(e);
    if (!rc) rc = lm_head(e);
    if (!rc) rc = argmax_next(e);
    return rc;
}

/* Capture fn(e) on the engine stream into a graph and instantiate it. */
static int capture(sgpu_qwen *e, int (*fn)(sgpu_qwen *), hipGraph_t *g, hipGraphExec_t *ge) {
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

static int run_layers(sgpu_qwen *e) {
    if (e->path != SGPU_QWEN_PATH_GRAPH) return fused_layers(e);
    if (!e->ge_layers) {
        int rc = capture(e, fused_layers, &e->g_layers, &e->ge_layers);
        if (rc) return rc;
    }
    hipError_t he = hipGraphLaunch(e->ge_layers, e->stream);
    return he == hipSuccess ? SGPU_OK : (int)he;
}

static int logits_to_host(sgpu_qwen *e, float *logits_host) {
    if (!logits_host) return SGPU_OK;
    hipError_t he = hipMemcpyAsync(logits_host, e->d_logits, (size_t)e->cfg.V * 4, hipMemcpyDeviceToHost, e->stream);
    if (he != hipSuccess) return (int)he;
    return sgpu_stream_synchronize((void *)e->stream);
}

int sgpu_qwen_set_path(sgpu_qwen *e, int path) {
    if (!e || path < SGPU_QWEN_PATH_REFERENCE || path > SGPU_QWEN_PATH_GRAPH) return SGPU_ERR_INVALID_ARG;
    if (path != SGPU_QWEN_PATH_REFERENCE && !fused_ok(&e->cfg)) return SGPU_ERR_INVALID_ARG;
    e->path = path;
    return SGPU_OK;
}

int sgpu_qwen_forward(sgpu_qwen *e, int token, int pos, int want_logits, float *logits_host) {
    if (!e) return SGPU_ERR_INVALID_ARG;
    const sgpu_qwen_cfg *c = &e->cfg;
    if (token < 0 || token >= c->V || pos < 0 || pos >= c->CTX) return SGPU_ERR_INVALID_ARG;
    if (e->path == SGPU_QWEN_PATH_REFERENCE) return forward_reference(e, token, pos, want_logits, logits_host, NULL, NULL);
    int rc = sgpu_internal_dec_embed(e->d_emb, token, pos, e->d_x, c->C, e->d_step, (void *)e->stream);
    if (!rc) rc = run_layers(e);
    if (rc || !want_logits) return rc;
    if ((rc = lm_head(e))) return rc;
    return logits_to_host(e, logits_host);
}

int sgpu_qwen_forward_trace(sgpu_qwen *e, int token, int pos, float *logits_host, float *trace_host) {
    if (!e || !trace_host) return SGPU_ERR_INVALID_ARG;
    const sgpu_qwen_cfg *c = &e->cfg;
    if (token < 0 || token >= c->V || pos < 0 || pos >= c->CTX) return SGPU_ERR_INVALID_ARG;
    return forward_reference(e, token, pos, logits_host != NULL, logits_host, trace_host, NULL);
}

int sgpu_qwen_forward_stages(sgpu_qwen *e, int token, int pos, float *logits_host, sgpu_stage_fn fn, void *ctx) {
    if (!e || !fn) return SGPU_ERR_INVALID_ARG;
    const sgpu_qwen_cfg *c = &e->cfg;
    if (token < 0 || token >= c->V || pos < 0 || pos >= c->CTX) return SGPU_ERR_INVALID_ARG;
    int cap = e->L.qkvd > c->FC ? e->L.qkvd : c->FC;
    if (c->C > cap) cap = c->C;
    if ((pos + 1) * c->NH > cap) cap = (pos + 1) * c->NH;
    sgpu_stage_sink sink = {fn, ctx, malloc(sizeof(float) * (size_t)cap), cap};
    if (!sink.host) return SGPU_ERR_HOST_ALLOC;
    int rc = forward_reference(e, token, pos, logits_host != NULL, logits_host, NULL, &sink);
    free(sink.host);
    return rc;
}

/* ---- per-phase timing: each decode phase's 24 layer launches recorded in one graph ---- */
static int phase_layer(sgpu_qwen *e, int phase, int l) {
    const sgpu_qwen_cfg *c = &e->cfg;
    const int C = c->C, FC = c->FC;
    void *s = (void *)e->stream;
    switch (phase) {
    case 0:
        return sgpu_internal_dec_qkv(e->d_qkvw[l], C, e->L.qkvd, e->d_x, e->d_ln1w[l], c->eps, e->d_qkvb[l], e->d_q,
                                     e->d_kc[l], e->d_vc[l], e->d_cos, e->d_sin, e->d_step, c->NH, c->NKV, c->HD, s);
    case 1:
        return sgpu_internal_dec_attn(e->d_q, e->d_kc[l], e->d_vc[l], e->d_att, e->d_step, c->NH, c->NKV, c->HD,
                                      (float)(1.0 / sqrt((double)c->HD)), e->d_attn_ws, e->d_attn_cnt, s);
    case 2: return sgpu_internal_dec_res(e->d_ow[l], C, C, e->d_att, NULL, e->d_x, s);
    case 3: return sgpu_internal_dec_gateup(e->d_gateupw[l], C, FC, e->d_x, e->d_ln2w[l], c->eps, e->d_down, s);
    case 4: return sgpu_internal_dec_res(e->d_downw[l], FC, C, e->d_down, NULL, e->d_x, s);
    case 5: return lm_head(e);
    default:   /* the argmax and the next token's embedding, without the token list */
        return sgpu_internal_dec_argmax_next(e->d_logits, c->V, e->d_amax_v, e->d_amax_i, e->d_step, NULL, e->d_emb,
                                             NULL, NULL, e->d_x, C, c->CTX, s);
    }
}

int sgpu_qwen_phase_times(sgpu_qwen *e, int pos, int reps, float *us) {
    if (!e || !us || reps < 1 || !fused_ok(&e->cfg) || pos < 0 || pos >= e->cfg.CTX) return SGPU_ERR_INVALID_ARG;
    const int NL = e->cfg.NL;
    hipEvent_t e0 = NULL, e1 = NULL;
    int rc = (int)hipEventCreate(&e0);
    if (!rc) rc = (int)hipEventCreate(&e1);
    /* phases in order; the argmax (which advances the device position) last */
    for (int phase = 0; phase < SGPU_QWEN_NPHASES && !rc; phase++) {
        rc = sgpu_internal_dec_embed(e->d_emb, 0, pos, e->d_x, e->cfg.C, e->d_step, (void *)e->stream);
        if (rc) break;
        hipGraph_t g = NULL;
        hipGraphExec_t ge = NULL;
        hipError_t he = hipStreamBeginCapture(e->stream, hipStreamCaptureModeRelaxed);
        if (he != hipSuccess) { rc = (int)he; break; }
        for (int l = 0; l < NL && !rc; l++) rc = phase_layer(e, phase, l);
        he = hipStreamEndCapture(e->stream, &g);
        if (!rc && he != hipSuccess) rc = (int)he;
        if (!rc) rc = (int)hipGraphInstantiate(&ge, g, NULL, NULL, 0);
        float best = 1e30f;
        for (int r = 0; r <= reps && !rc; r++) {           /* r = 0: warm-up */
            if (phase == SGPU_QWEN_NPHASES - 1)
                rc = sgpu_internal_dec_embed(e->d_emb, 0, pos, e->d_x, e->cfg.C, e->d_step, (void *)e->stream);
            if (!rc) rc = (int)hipEventRecord(e0, e->stream);
            if (!rc) rc = (int)hipGraphLaunch(ge, e->stream);
            if (!rc) rc = (int)hipEventRecord(e1, e->stream);
            if (!rc) rc = (int)hipEventSynchronize(e1);
            float ms = 0;
            if (!rc) rc = (int)hipEventElapsedTime(&ms, e0, e1);
            if (!rc && r > 0 && ms < best) best = ms;
        }
        if (ge) hipGraphExecDestroy(ge);
        if (g) hipGraphDestroy(g);
        if (!rc) us[phase] = best * 1e3f / (float)NL;
    }
    /* leave the engine at `pos` with token 0's embedding, as sgpu_qwen_forward would start */
    if (!rc) rc = sgpu_internal_dec_embed(e->d_emb, 0, pos, e->d_x, e->cfg.C, e->d_step, (void *)e->stream);
    if (!rc) rc = sgpu_stream_synchronize((void *)e->stream);
    if (e0) hipEventDestroy(e0);
    if (e1) hipEventDestroy(e1);
    return rc;
}

/* ---- batched prompt prefill: the prompt's rows go through each layer together, so each
 * layer's weights stream once per chunk of up to PF_ROWS rows instead of once per position ---- */
#define PF_ROWS 512

/* Allocated on the first prefill and kept; a failed call leaves the buffers it did get in
 * place (freed with the engine) and the next call allocates only the missing ones. */
static int pf_alloc(sgpu_qwen *e) {
    const sgpu_qwen_cfg *c = &e->cfg;
    const size_t R = PF_ROWS, C = (size_t)c->C, FC = (size_t)c->FC, Q = (size_t)e->L.qkvd;
    const size_t ybig = 2 * FC > C ? 2 * FC : C;
    struct { void **p; size_t bytes; } need[] = {
        {(void **)&e->d_pf_ids, (size_t)c->CTX * sizeof(int)}, {(void **)&e->d_pf_x, R * C * 4},
        {(void **)&e->d_pf_xn, R * C * 4}, {(void **)&e->d_pf_qkv, R * Q * 4}, {(void **)&e->d_pf_att, R * C * 4},
        {(void **)&e->d_pf_y, R * ybig * 4}, {(void **)&e->d_pf_g, R * FC * 4}};
    for (size_t i = 0; i < sizeof need / sizeof need[0]; i++) {
        if (*need[i].p) continue;
        int rc = dalloc(need[i].p, need[i].bytes, NULL);
        if (rc) {                      /* allocated but not cleared: give it back */
            sgpu_free(*need[i].p);
            *need[i].p = NULL;
            return rc;
        }
    }
    return SGPU_OK;
}

/* Positions 0..T-1 of the prompt into the KV caches, the last row's logits into d_logits and
 * the step record {ids[T-1], T-1} (so the on-device greedy loop continues from position T). */
static int prefill_rows(sgpu_qwen *e, const int *ids, int T) {
    const sgpu_qwen_cfg *c = &e->cfg;
    const int C = c->C, NH = c->NH, NKV = c->NKV, HD = c->HD, FC = c->FC, QKVD = e->L.qkvd;
    const float eps = c->eps, scale = (float)(1.0 / sqrt((double)HD));
    void *s = (void *)e->stream;
    int rc;
    if ((rc = pf_alloc(e))) return rc;
    hipError_t he = hipMemcpyAsync(e->d_pf_ids, ids, (size_t)T * sizeof(int), hipMemcpyHostToDevice, e->stream);
    if (he != hipSuccess) return (int)he;
#define TRY(x) do { if ((rc = (x))) return rc; } while (0)
    int Tc = 0;
    for (int c0 = 0; c0 < T; c0 += PF_ROWS) {
        Tc = T - c0 < PF_ROWS ? T - c0 : PF_ROWS;
        TRY(sgpu_internal_pf_embed(e->d_emb, e->d_pf_ids + c0, Tc, e->d_pf_x, C, s));
        for (int l = 0; l < c->NL; l++) {
            TRY(sgpu_rmsnorm(e->d_pf_x, e->d_ln1w[l], e->d_pf_xn, C, eps, Tc, s));
            TRY(sgpu_internal_pf_gemm(e->d_qkvw[l], e->d_pf_xn, e->d_qkvb[l], e->d_pf_qkv, C, QKVD, Tc,
                e->d_split_ws, e->d_split_cnt, 0, s));
            TRY(sgpu_internal_pf_qkv_post(e->d_pf_qkv, Tc, c0, e->d_cos, e->d_sin, e->d_kc[l], e->d_vc[l], NH, NKV,
                                          HD, s));
            TRY(sgpu_internal_pf_attn(e->d_pf_qkv, e->d_kc[l], e->d_vc[l], e->d_pf_att, Tc, c0, NH, NKV, HD, scale, s));
            /* x += o(att): the residual add in the GEMM's store (x + y, as add2 computes it) */
            TRY(sgpu_internal_pf_gemm(e->d_ow[l], e->d_pf_att, NULL, e->d_pf_x, C, C, Tc,
                e->d_split_ws, e->d_split_cnt, 1, s));
            TRY(sgpu_rmsnorm(e->d_pf_x, e->d_ln2w[l], e->d_pf_xn, C, eps, Tc, s));
            TRY(sgpu_internal_pf_gemm(e->d_gateupw[l], e->d_pf_xn, NULL, e->d_pf_y, C, 2 * FC, Tc,
                e->d_split_ws, e->d_split_cnt, 0, s));
            TRY(sgpu_internal_pf_swiglu(e->d_pf_y, e->d_pf_g, FC, Tc, s));
            TRY(sgpu_internal_pf_gemm(e->d_downw[l], e->d_pf_g, NULL, e->d_pf_x, FC, C, Tc,
                e->d_split_ws, e->d_split_cnt, 1, s));
        }
    }
    TRY(sgpu_internal_dec_lmhead(e->d_emb, C, c->V, e->d_pf_x + (size_t)(Tc - 1) * C, e->d_lnfw, eps, e->d_logits, s));
#undef TRY
    const int st[2] = {ids[T - 1], T - 1};
    he = hipMemcpyAsync(e->d_step, st, sizeof st, hipMemcpyHostToDevice, e->stream);
    if (he != hipSuccess) return (int)he;
    return sgpu_stream_synchronize(s);
}

int sgpu_qwen_prefill(sgpu_qwen *e, const int *ids, int T, float *logits_host) {
    if (!e || !ids || T <= 0 || T > e->cfg.CTX || !fused_ok(&e->cfg)) return SGPU_ERR_INVALID_ARG;
    for (int p = 0; p < T; p++)
        if (ids[p] < 0 || ids[p] >= e->cfg.V) return SGPU_ERR_INVALID_ARG;
    int rc = prefill_rows(e, ids, T);
    if (rc || !logits_host) return rc;
    return sgpu_memcpy_dtoh(logits_host, e->d_logits, (size_t)e->cfg.V * sizeof(float));
}

int sgpu_qwen_generate(sgpu_qwen *e, const int *prompt, int T, int n_gen, int *out_tokens) {
    if (!e || !prompt || !out_tokens || T <= 0 || n_gen < 0) return SGPU_ERR_INVALID_ARG;
    const sgpu_qwen_cfg *c = &e->cfg;
    if ((long long)T + n_gen > c->CTX) return SGPU_ERR_INVALID_ARG;
    for (int p = 0; p < T; p++)
        if (prompt[p] < 0 || prompt[p] >= c->V) return SGPU_ERR_INVALID_ARG;
    int rc;
    if (e->path == SGPU_QWEN_PATH_REFERENCE) {       /* host-driven loop, the reference's own */
        float *logits = malloc(sizeof(float) * (size_t)c->V);
        if (!logits) return SGPU_ERR_HOST_ALLOC;
        for (int p = 0; p < T && !(rc = forward_reference(e, prompt[p], p, p == T - 1, logits, NULL, NULL)); p++) {
        }
        for (int g = 0; !rc && g <= n_gen; g++) {
            int b = 0;
            for (int i = 1; i < c->V; i++)
                if (logits[i] > logits[b]) b = i;
            out_tokens[g] = b;
            if (g < n_gen) rc = forward_reference(e, b, T + g, 1, logits, NULL, NULL);
        }
        free(logits);
        return rc;
    }
    if ((rc = prefill_rows(e, prompt, T))) return rc;
    if ((rc = argmax_next(e))) return rc;
    for (int g = 0; g < n_gen; g++) {
        if (e->path == SGPU_QWEN_PATH_GRAPH) {
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
