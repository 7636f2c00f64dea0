/* golden.c -- CPU golden models (the oracle).  TEST INFRASTRUCTURE ONLY: see golden.h.
 *
 * Restates, in this repository's own C, the serial CPU reference computations that the
 * reference harnesses and engines check their GPU kernels against.  Build flags matter:
 * -O2 -ffp-contract=off (no fused multiply-add), so every product and every sum is one
 * IEEE fp32 rounding in the reference's order.  OpenMP only ever splits *rows*; the
 * k-order of each dot product is the serial one, so threaded results are bit-identical.
 */
#include "golden.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* qwen_engine.c:90-98 */
float og_h2f(uint16_t h) {
    uint32_t e = (h >> 10) & 0x1fu;
    if (e == 0) return 0.0f;
    union { uint32_t u; float f; } cvt;
    cvt.u = ((uint32_t)(h & 0x8000u) << 16) | ((e - 15u + 127u) << 23) |
            ((uint32_t)(h & 0x3ffu) << 13);
    return cvt.f;
}

/* gpu_workload.c:97-98: float ref = 0; for k: ref += A[i*n+k] * B[k*n+j]; generalised to
 * M x N x K with the same strides (A stride K, B stride N). */
static void sgemm_row(const float *A, const float *B, float *C, int N, int K, int i) {
    const float *a = A + (size_t)i * K;
    float *c = C + (size_t)i * N;
    for (int j = 0; j < N; j++) {
        float ref = 0.0f;
        for (int k = 0; k < K; k++) ref += a[k] * B[(size_t)k * N + j];
        c[j] = ref;
    }
}

void og_sgemm(const float *A, const float *B, float *C, int M, int N, int K) {
    for (int i = 0; i < M; i++) sgemm_row(A, B, C, N, K, i);
}

void og_sgemm_rows(const float *A, const float *B, float *C, int M, int N, int K,
                   int row0, int row1, int nthreads) {
    if (row0 < 0) row0 = 0;
    if (row1 > M) row1 = M;
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for num_threads(nthreads) schedule(dynamic, 1)
    for (int i = row0; i < row1; i++) sgemm_row(A, B, C, N, K, i);
}

/* gpu_workload.c:95-112 (same predicate, same early stop: one bad cell per row, 5 rows). */
int og_sgemm_verdict_bad(const float *got, const float *ref, int M, int N) {
    int bad = 0;
    for (int i = 0; i < M && bad < 5; i++)
        for (int j = 0; j < N; j++) {
            float r = ref[(size_t)i * N + j];
            float d = got[(size_t)i * N + j] - r;
            if (d < 0) d = -d;
            if (d > 0.05f * (r < 0 ? -r : r) + 1e-3f) { bad++; break; }
        }
    return bad;
}

/* gemv_test.c:85-90 (float acc = 0; acc += row[k]*x[k]) with the nullable bias epilogue
 * of cpu_gemv, gpt2_engine.c:342-349 (y = acc + (bias ? bias[o] : 0)). */
void og_gemv(const float *W, const float *x, const float *bias, float *y, int K, int N,
             int nthreads) {
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int o = 0; o < N; o++) {
        const float *row = W + (size_t)o * K;
        float acc = 0.0f;
        for (int k = 0; k < K; k++) acc += row[k] * x[k];
        y[o] = acc + (bias ? bias[o] : 0.0f);
    }
}

/* cpu_gemv_h, qwen_engine.c:276-284 (bias is fp16, decoded with h2f). */
void og_gemv_h(const uint16_t *W, const float *x, const uint16_t *bias, float *y,
               int K, int N, int nthreads) {
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int o = 0; o < N; o++) {
        const uint16_t *row = W + (size_t)o * K;
        float acc = 0.0f;
        for (int k = 0; k < K; k++) acc += og_h2f(row[k]) * x[k];
        y[o] = acc + (bias ? og_h2f(bias[o]) : 0.0f);
    }
}

/* The same dot product with the fp32 bias the GPU kernel receives
 * (qwen_kernels.cu:66 adds bias[n] as float; qwen_engine.c:170-175 decodes it on the host). */
void og_gemv_h_fbias(const uint16_t *W, const float *x, const float *bias, float *y,
                     int K, int N, int nthreads) {
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int o = 0; o < N; o++) {
        const uint16_t *row = W + (size_t)o * K;
        float acc = 0.0f;
        for (int k = 0; k < K; k++) acc += og_h2f(row[k]) * x[k];
        y[o] = acc + (bias ? bias[o] : 0.0f);
    }
}

/* gemv_h's dot product (qwen_kernels.cu:34-70; serial golden qwen_engine.c:276-284) with x
 * given as fp16 bits: every x code decoded once with the reference h2f (qwen_engine.c:90-98),
 * then the same k-ascending sum as og_gemv_h_fbias. */
void og_gemv_hh(const uint16_t *W, const uint16_t *x, const float *bias, float *y,
                int K, int N, int nthreads) {
    float *xf = (float *)malloc((K > 0 ? (size_t)K : 1) * sizeof(float));
    if (!xf) return;
    for (int k = 0; k < K; k++) xf[k] = og_h2f(x[k]);
    og_gemv_h_fbias(W, xf, bias, y, K, N, nthreads);
    free(xf);
}

/* gpt2_kernels.cu:110-155 computes Y[t*N+n] = W[n,:].X[t,:] + bias?[n]; the golden is the
 * serial dot product per (t, n), as cpu_gemv (gpt2_engine.c:342-349) applied row by row. */
void og_gemv_multi(const float *W, const float *X, const float *bias, float *Y,
                   int K, int N, int T, int nthreads) {
    for (int t = 0; t < T; t++)
        og_gemv(W, X + (size_t)t * K, bias, Y + (size_t)t * N, K, N, nthreads);
}

/* cpu_rms, qwen_engine.c:285-290. */
void og_rms(const float *x, const uint16_t *w, float *y, int n, float eps) {
    float ss = 0.0f;
    for (int i = 0; i < n; i++) ss += x[i] * x[i];
    float inv = 1.0f / sqrtf(ss / n + eps);
    for (int i = 0; i < n; i++) y[i] = x[i] * inv * og_h2f(w[i]);
}

/* ---- Qwen layout (qwen_engine.c:61-75, writer conv_qwen.py:63-99) ---- */
typedef struct {
    size_t off_emb, off_cos, off_sin, l_base, lstride, off_lnfw, bytes;   /* bytes */
    size_t li_inln, li_qkvw, li_qkvb, li_ow, li_postln, li_gateup, li_down; /* halves */
    int kvd, qkvd;
} qlayout;

static void q_layout(const og_qwen_cfg *c, qlayout *L) {
    L->kvd = c->NKV * c->HD;
    L->qkvd = c->C + 2 * L->kvd;
    L->off_emb = 0;
    L->off_cos = L->off_emb + (size_t)c->V * c->C * 2;
    L->off_sin = L->off_cos + (size_t)c->CTX * (c->HD / 2) * 4;
    L->l_base = L->off_sin + (size_t)c->CTX * (c->HD / 2) * 4;
    L->lstride = ((size_t)c->C + (size_t)L->qkvd * c->C + L->qkvd + (size_t)c->C * c->C + c->C +
                  (size_t)2 * c->FC * c->C + (size_t)c->C * c->FC) * 2;
    L->off_lnfw = L->l_base + (size_t)c->NL * L->lstride;
    L->bytes = L->off_lnfw + (size_t)c->C * 2;
    L->li_inln = 0;
    L->li_qkvw = c->C;
    L->li_qkvb = (size_t)c->C + (size_t)L->qkvd * c->C;
    L->li_ow = L->li_qkvb + L->qkvd;
    L->li_postln = L->li_ow + (size_t)c->C * c->C;
    L->li_gateup = L->li_postln + c->C;
    L->li_down = L->li_gateup + (size_t)2 * c->FC * c->C;
}

size_t og_qwen_file_bytes(const og_qwen_cfg *cfg) {
    qlayout L;
    q_layout(cfg, &L);
    return L.bytes;
}

/* conv_qwen.py:75-80: freq_d = theta^(-2d/HD), angle = pos*freq_d in float64, stored fp32. */
void og_rope_tables(int ctx, int hd, double theta, float *cos_out, float *sin_out) {
    int h2 = hd / 2;
    for (int p = 0; p < ctx; p++)
        for (int d = 0; d < h2; d++) {
            double freq = pow(theta, -2.0 * (double)d / (double)hd);
            double ang = (double)p * freq;
            cos_out[(size_t)p * h2 + d] = (float)cos(ang);
            sin_out[(size_t)p * h2 + d] = (float)sin(ang);
        }
}

int og_argmax(const float *v, int n) {   /* qwen_engine.c:360-364: first max wins */
    int b = 0;
    float m = v[0];
    for (int i = 1; i < n; i++)
        if (v[i] > m) { m = v[i]; b = i; }
    return b;
}

/* cpu_forward, qwen_engine.c:292-358, for one position. */
int og_qwen_forward(const og_qwen_cfg *c, const void *blob, float *kc, float *vc,
                    int token, int pos, int want_logits, float *logits, float *trace,
                    int nthreads) {
    if (!c || !blob || !kc || !vc || token < 0 || token >= c->V || pos < 0 || pos >= c->CTX ||
        c->NH % c->NKV || c->HD % 2)
        return -1;
    qlayout L;
    q_layout(c, &L);
    const int C = c->C, NH = c->NH, NKV = c->NKV, HD = c->HD, FC = c->FC, CTX = c->CTX;
    const int KVD = L.kvd, QKVD = L.qkvd, H2 = HD / 2;
    const float SCALE = (float)(1.0 / sqrt((double)HD));   /* 0.125 at HD=64 (qwen_engine.c:55) */
    const unsigned char *base = (const unsigned char *)blob;
    const uint16_t *emb = (const uint16_t *)(base + L.off_emb);
    const float *cosT = (const float *)(base + L.off_cos);
    const float *sinT = (const float *)(base + L.off_sin);

    float *r_x = malloc(sizeof(float) * C), *r_ln = malloc(sizeof(float) * C);
    float *r_qkv = malloc(sizeof(float) * QKVD), *r_att = malloc(sizeof(float) * C);
    float *r_y = malloc(sizeof(float) * C), *r_ln2 = malloc(sizeof(float) * C);
    float *r_gate = malloc(sizeof(float) * 2 * FC), *r_down = malloc(sizeof(float) * FC);
    float *sc = malloc(sizeof(float) * (pos + 1));
    if (!r_x || !r_ln || !r_qkv || !r_att || !r_y || !r_ln2 || !r_gate || !r_down || !sc) {
        free(r_x); free(r_ln); free(r_qkv); free(r_att); free(r_y); free(r_ln2);
        free(r_gate); free(r_down); free(sc);
        return -1;
    }

    for (int i = 0; i < C; i++) r_x[i] = og_h2f(emb[(size_t)token * C + i]);
    for (int l = 0; l < c->NL; l++) {
        const uint16_t *b = (const uint16_t *)(base + L.l_base + (size_t)l * L.lstride);
        og_rms(r_x, b + L.li_inln, r_ln, C, c->eps);
        og_gemv_h(b + L.li_qkvw, r_ln, b + L.li_qkvb, r_qkv, C, QKVD, nthreads);
        for (int h = 0; h < NH; h++)            /* RoPE q (qwen_engine.c:303-309) */
            for (int i = 0; i < H2; i++) {
                float a = r_qkv[h * HD + i], b2 = r_qkv[h * HD + H2 + i];
                float cs = cosT[(size_t)pos * H2 + i], sn = sinT[(size_t)pos * H2 + i];
                r_qkv[h * HD + i] = a * cs - b2 * sn;
                r_qkv[h * HD + H2 + i] = a * sn + b2 * cs;
            }
        for (int g = 0; g < NKV; g++)           /* RoPE k (qwen_engine.c:311-317) */
            for (int i = 0; i < H2; i++) {
                float a = r_qkv[C + g * HD + i], b2 = r_qkv[C + g * HD + H2 + i];
                float cs = cosT[(size_t)pos * H2 + i], sn = sinT[(size_t)pos * H2 + i];
                r_qkv[C + g * HD + i] = a * cs - b2 * sn;
                r_qkv[C + g * HD + H2 + i] = a * sn + b2 * cs;
            }
        for (int i = 0; i < KVD; i++) {         /* cache write (qwen_engine.c:319-322) */
            kc[((size_t)l * CTX + pos) * KVD + i] = r_qkv[C + i];
            vc[((size_t)l * CTX + pos) * KVD + i] = r_qkv[C + KVD + i];
        }
        for (int h = 0; h < NH; h++) {          /* GQA attention (qwen_engine.c:324-342) */
            int g = h / (NH / NKV);
            float maxv = -1e30f;
            for (int t = 0; t <= pos; t++) {
                float acc = 0.0f;
                for (int d = 0; d < HD; d++)
                    acc += r_qkv[h * HD + d] * kc[((size_t)l * CTX + t) * KVD + g * HD + d];
                sc[t] = acc * SCALE;
                if (sc[t] > maxv) maxv = sc[t];
            }
            float sum = 0.0f;
            for (int t = 0; t <= pos; t++) { sc[t] = expf(sc[t] - maxv); sum += sc[t]; }
            for (int d = 0; d < HD; d++) {
                float acc = 0.0f;
                for (int t = 0; t <= pos; t++)
                    acc += (sc[t] / sum) * vc[((size_t)l * CTX + t) * KVD + g * HD + d];
                r_att[h * HD + d] = acc;
            }
        }
        og_gemv_h(b + L.li_ow, r_att, NULL, r_y, C, C, nthreads);
        for (int i = 0; i < C; i++) r_x[i] += r_y[i];
        og_rms(r_x, b + L.li_postln, r_ln2, C, c->eps);
        og_gemv_h(b + L.li_gateup, r_ln2, NULL, r_gate, C, 2 * FC, nthreads);
        for (int i = 0; i < FC; i++)            /* SwiGLU (qwen_engine.c:349-350) */
            r_down[i] = (r_gate[i] / (1.0f + expf(-r_gate[i]))) * r_gate[FC + i];
        og_gemv_h(b + L.li_down, r_down, NULL, r_y, FC, C, nthreads);
        for (int i = 0; i < C; i++) r_x[i] += r_y[i];
        if (trace) memcpy(trace + (size_t)l * C, r_x, sizeof(float) * C);
    }
    if (want_logits && logits) {                /* final norm + tied lm_head (:356-357) */
        og_rms(r_x, (const uint16_t *)(base + L.off_lnfw), r_ln, C, c->eps);
        og_gemv_h(emb, r_ln, NULL, logits, C, c->V, nthreads);
    }
    free(r_x); free(r_ln); free(r_qkv); free(r_att); free(r_y); free(r_ln2);
    free(r_gate); free(r_down); free(sc);
    return 0;
}

/* ---- GPT-2 ---- */
typedef struct {
    size_t wte, wpe, l_base, lstride, lnfw, lnfb, total;
    size_t ln1w, ln1b, qkvw, qkvb, aow, aob, ln2w, ln2b, fcw, fcb, projw, projb;
} g2layout;

/* gpt2_engine.c:50-70 */
static void g2_layout(const og_gpt2_cfg *c, g2layout *L) {
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

size_t og_gpt2_file_floats(const og_gpt2_cfg *cfg) {
    g2layout L;
    g2_layout(cfg, &L);
    return L.total;
}

/* cpu_ln, gpt2_engine.c:333-341 */
void og_layernorm(const float *x, const float *w, const float *b, float *y, int n, float eps) {
    float mean = 0.0f, var = 0.0f;
    for (int i = 0; i < n; i++) mean += x[i];
    mean /= n;
    for (int i = 0; i < n; i++) {
        float d = x[i] - mean;
        var += d * d;
    }
    var /= n;
    float inv = 1.0f / sqrtf(var + eps);
    for (int i = 0; i < n; i++) y[i] = (x[i] - mean) * inv * w[i] + b[i];
}

/* cpu_forward, gpt2_engine.c:363-421 (attention scale 0.125 = 1/sqrt(HD), gelu tanh form) */
int og_gpt2_forward(const og_gpt2_cfg *c, const float *w, float *kc, float *vc, int token, int pos,
                    int want_logits, float *logits, float *trace, int nthreads) {
    if (!c || !w || !kc || !vc || token < 0 || token >= c->V || pos < 0 || pos >= c->CTX || c->NH * c->HD != c->C)
        return -1;
    g2layout L;
    g2_layout(c, &L);
    const int C = c->C, NH = c->NH, HD = c->HD, FC = c->FC, CTX = c->CTX;
    const float scale = (float)(1.0 / sqrt((double)HD));
    float *r_x = malloc(sizeof(float) * C), *r_ln = malloc(sizeof(float) * C);
    float *r_qkv = malloc(sizeof(float) * 3 * C), *r_att = malloc(sizeof(float) * C);
    float *r_y = malloc(sizeof(float) * C), *r_fc = malloc(sizeof(float) * FC);
    float *sc = malloc(sizeof(float) * (pos + 1));
    if (!r_x || !r_ln || !r_qkv || !r_att || !r_y || !r_fc || !sc) {
        free(r_x); free(r_ln); free(r_qkv); free(r_att); free(r_y); free(r_fc); free(sc);
        return -1;
    }
    for (int i = 0; i < C; i++) r_x[i] = w[L.wte + (size_t)token * C + i] + w[L.wpe + (size_t)pos * C + i];
    for (int l = 0; l < c->NL; l++) {
        const float *b = w + L.l_base + (size_t)l * L.lstride;
        og_layernorm(r_x, b + L.ln1w, b + L.ln1b, r_ln, C, c->eps);
        og_gemv(b + L.qkvw, r_ln, b + L.qkvb, r_qkv, C, 3 * C, nthreads);
        for (int i = 0; i < C; i++) {
            kc[((size_t)l * CTX + pos) * C + i] = r_qkv[C + i];
            vc[((size_t)l * CTX + pos) * C + i] = r_qkv[2 * C + i];
        }
        for (int h = 0; h < NH; h++) {
            float maxv = -1e30f, sum = 0.0f;
            for (int t = 0; t <= pos; t++) {
                const float *kh = kc + ((size_t)l * CTX + t) * C + h * HD;
                const float *qh = r_qkv + h * HD;
                float acc = 0.0f;
                for (int d = 0; d < HD; d++) acc += qh[d] * kh[d];
                sc[t] = acc * scale;
                if (sc[t] > maxv) maxv = sc[t];
            }
            for (int t = 0; t <= pos; t++) { sc[t] = expf(sc[t] - maxv); sum += sc[t]; }
            for (int d = 0; d < HD; d++) {
                float acc = 0.0f;
                for (int t = 0; t <= pos; t++) acc += sc[t] * vc[((size_t)l * CTX + t) * C + h * HD + d];
                r_att[h * HD + d] = acc / sum;
            }
        }
        og_gemv(b + L.aow, r_att, b + L.aob, r_y, C, C, nthreads);
        for (int i = 0; i < C; i++) r_x[i] += r_y[i];
        og_layernorm(r_x, b + L.ln2w, b + L.ln2b, r_ln, C, c->eps);
        og_gemv(b + L.fcw, r_ln, b + L.fcb, r_fc, C, FC, nthreads);
        for (int i = 0; i < FC; i++) {
            float v = r_fc[i];
            float t = 0.7978845608f * (v + 0.044715f * v * v * v);
            r_fc[i] = 0.5f * v * (1.0f + tanhf(t));
        }
        og_gemv(b + L.projw, r_fc, b + L.projb, r_y, FC, C, nthreads);
        for (int i = 0; i < C; i++) r_x[i] += r_y[i];
        if (trace) memcpy(trace + (size_t)l * C, r_x, sizeof(float) * C);
    }
    if (want_logits && logits) {
        og_layernorm(r_x, w + L.lnfw, w + L.lnfb, r_ln, C, c->eps);
        og_gemv(w + L.wte, r_ln, NULL, logits, C, c->V, nthreads);   /* tied lm_head, no bias */
    }
    free(r_x); free(r_ln); free(r_qkv); free(r_att); free(r_y); free(r_fc); free(sc);
    return 0;
}
