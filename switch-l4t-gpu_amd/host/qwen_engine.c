/* qwen_engine.c -- Qwen2.5-0.5B-architecture fp16-weight decode on one MI355X (gfx950).
 *
 * Command-line front end of the reference engine (gpu-llm/engine/qwen_engine.c:446-558) over
 * libswitchgpu.so: load the flat weight file (or build a random-init one in memory), prime
 * the KV cache with the prompt one position at a time, then greedy-decode, printing tok/s.
 * The per-position device work is sgpu_qwen_forward on the chosen launch path.
 *
 * Usage: qwen_engine (--weights FILE | --random SEED) [--ids FILE | --prompt-random N]
 *                    [--gen N] [--greedy] [--serve] [--json] [--write-weights FILE]
 *                    [--path reference|fused|graph] [--batch-prefill]
 *   --weights        flat file in the qwen_engine.c:8-16 layout (conv_qwen.py writer)
 *   --random SEED    random-init model: every fp16 tensor N(0, 0.02), RoPE theta 1e6 tables
 *   --ids FILE       u32 count + u32 ids (qwen_engine.c:477-486)
 *   --prompt-random  N ids drawn from the seeded LCG (default: the 8 deterministic ids of
 *                    qwen_engine.c:488)
 *   --serve          u32 request protocol on stdin/stdout (qwen_engine.c:406-444), greedy
 *   --write-weights F  write the model (loaded or random-init) as a flat file in the same
 *                    layout and exit without touching the device (the writer role of
 *                    conv_qwen.py:63-99)
 *   --batch-prefill  prime the cache with all prompt positions in one batched pass
 *                    (sgpu_qwen_prefill) instead of one position at a time
 *   --path P         reference: the gpu_forward launch sequence (qwen_engine.c:205-269);
 *                    fused: five kernels per layer; graph (default): those replayed as a HIP
 *                    graph.  Same tokens on every path.
 *   --selftest S     before priming, run prompt positions 0..S-1 on the GPU and on this
 *                    program's own serial CPU forward (a restatement of the reference's
 *                    cpu_forward, qwen_engine.c:292-358) and compare: the residual after each
 *                    layer at position 0, then the logits at position S-1 (max |gpu-cpu|, top-5
 *                    ids, argmax MATCH/MISMATCH, SELFTEST: PASS/FAIL; qwen_engine.c:494-521).
 *                    The cache keeps those positions; priming continues from S.
 *   --debug          with --selftest: the layer-0 stage vectors at position 0 (first four
 *                    values and sum), first the GPU's (g.* lines, the reference launch sequence
 *                    waited for after each stage, qwen_engine.c:196-202,216-260) then the CPU
 *                    forward's (c.* lines, qwen_engine.c:297-346), and both layer traces written
 *                    to trace_g.bin / trace_c.bin (NL x C floats each).
 * Decoding is greedy (argmax, first max wins, qwen_engine.c:360-364) and stops at EOT or
 * <|im_end|> as the reference does (:539); --greedy is accepted for command-line
 * compatibility.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "switch_gpu.h"

#define CHK(x) do { int r_ = (int)(x); if (r_) { fprintf(stderr, "error %d (%s) at %s:%d\n", r_, \
    sgpu_error_string(r_), __FILE__, __LINE__); exit(1); } } while (0)

static const int EOT = 151643, IM_END = 151645;   /* qwen_engine.c:57-58 */

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec + ts.tv_nsec / 1e9;
}

static int argmax(const float *v, int n) {
    int b = 0;
    float m = v[0];
    for (int i = 1; i < n; i++)
        if (v[i] > m) { m = v[i]; b = i; }
    return b;
}

/* ---- the self-test's CPU side: the reference's serial cpu_forward restated over the flat
 * file in host memory (qwen_engine.c:276-358), independent of the library's kernels.  Rows of
 * a GEMV are spread over threads; each row's sum runs serially in k order, as the reference's
 * does, so the thread count changes no bit. ---- */
typedef struct {
    const sgpu_qwen_cfg *c;
    const uint16_t *h;                      /* the flat file as fp16 codes */
    const float *cosT, *sinT;               /* RoPE tables, CTX x HD/2 each */
    size_t l_base, lstride, off_lnfw;       /* in halves */
    size_t li_qkvw, li_qkvb, li_ow, li_postln, li_gateup, li_down;
    int kvd, qkvd;
    float *kc, *vc, *x, *ln, *qkv, *att, *y, *gate, *down, *sc, *logits;
    int debug;
} cpu_model;

/* h2f of qwen_engine.c:90-98: exponent 0 reads as +0, exponent 31 as a finite number. */
static float h2f(uint16_t h) {
    const uint32_t e = (h >> 10) & 0x1fu;
    if (e == 0) return 0.0f;
    union { uint32_t u; float f; } v;
    v.u = ((uint32_t)(h & 0x8000u) << 16) | ((e - 15u + 127u) << 23) | ((uint32_t)(h & 0x3ffu) << 13);
    return v.f;
}

static void cpu_gemv_h(const uint16_t *W, const float *x, const uint16_t *bias, float *y, int K, int N) {
#pragma omp parallel for schedule(static)
    for (int o = 0; o < N; o++) {
        const uint16_t *row = W + (size_t)o * K;
        float acc = 0.0f;
        for (int k = 0; k < K; k++) acc += h2f(row[k]) * x[k];
        y[o] = acc + (bias ? h2f(bias[o]) : 0.0f);
    }
}

static void cpu_rms(const float *x, const uint16_t *w, float *y, int n, float eps) {
    float ss = 0.0f;
    for (int i = 0; i < n; i++) ss += x[i] * x[i];
    const float inv = 1.0f / sqrtf(ss / n + eps);
    for (int i = 0; i < n; i++) y[i] = x[i] * inv * h2f(w[i]);
}

static void prvec(const char *tag, const float *v, int n) {
    float s = 0.0f;
    for (int i = 0; i < n; i++) s += v[i];
    printf("    c.%-8s first4=%.3f %.3f %.3f %.3f sum=%.3f\n", tag, v[0], v[1], v[2], v[3], s);
}

/* A GPU stage vector (sgpu_qwen_forward_stages) in the same format, tagged g. */
static void gprvec(void *ctx, const char *tag, const float *v, int n) {
    (void)ctx;
    float s = 0.0f;
    for (int i = 0; i < n; i++) s += v[i];
    printf("    g.%-8s first4=%.3f %.3f %.3f %.3f sum=%.3f\n", tag, v[0], v[1], v[2], v[3], s);
}

static int cpu_init(cpu_model *m, const sgpu_qwen_cfg *c, const void *blob, int debug) {
    memset(m, 0, sizeof *m);
    m->c = c;
    m->debug = debug;
    m->h = (const uint16_t *)blob;
    m->kvd = c->NKV * c->HD;
    m->qkvd = c->C + 2 * m->kvd;
    /* qwen_engine.c:61-75: embedding, cos and sin tables (fp32), the layers, the final norm */
    const size_t tab = (size_t)c->CTX * (c->HD / 2);
    m->cosT = (const float *)((const unsigned char *)blob + (size_t)c->V * c->C * 2);
    m->sinT = m->cosT + tab;
    m->l_base = ((size_t)c->V * c->C * 2 + 2 * tab * 4) / 2;
    m->li_qkvw = (size_t)c->C;
    m->li_qkvb = m->li_qkvw + (size_t)m->qkvd * c->C;
    m->li_ow = m->li_qkvb + m->qkvd;
    m->li_postln = m->li_ow + (size_t)c->C * c->C;
    m->li_gateup = m->li_postln + c->C;
    m->li_down = m->li_gateup + (size_t)2 * c->FC * c->C;
    m->lstride = m->li_down + (size_t)c->C * c->FC;
    m->off_lnfw = m->l_base + (size_t)c->NL * m->lstride;
    const size_t kv = (size_t)c->NL * c->CTX * m->kvd;
    m->kc = calloc(kv, 4);
    m->vc = calloc(kv, 4);
    m->x = malloc((size_t)c->C * 4);
    m->ln = malloc((size_t)c->C * 4);
    m->qkv = malloc((size_t)m->qkvd * 4);
    m->att = malloc((size_t)c->C * 4);
    m->y = malloc((size_t)c->C * 4);
    m->gate = malloc((size_t)2 * c->FC * 4);
    m->down = malloc((size_t)c->FC * 4);
    m->sc = malloc((size_t)c->CTX * 4);
    m->logits = malloc((size_t)c->V * 4);
    return m->kc && m->vc && m->x && m->ln && m->qkv && m->att && m->y && m->gate && m->down && m->sc && m->logits;
}

static void cpu_free(cpu_model *m) {
    float *p[] = {m->kc, m->vc, m->x, m->ln, m->qkv, m->att, m->y, m->gate, m->down, m->sc, m->logits};
    for (size_t i = 0; i < sizeof p / sizeof p[0]; i++) free(p[i]);
}

static void rope(float *v, int heads, int HD, const float *cs, const float *sn) {
    for (int h = 0; h < heads; h++)
        for (int i = 0; i < HD / 2; i++) {
            const float a = v[h * HD + i], b = v[h * HD + HD / 2 + i];
            v[h * HD + i] = a * cs[i] - b * sn[i];
            v[h * HD + HD / 2 + i] = a * sn[i] + b * cs[i];
        }
}

/* cpu_forward (qwen_engine.c:292-358): token at pos, the residual after each layer to trace
 * (NL x C, may be NULL), the logits to m->logits when want_logits. */
static void cpu_forward(cpu_model *m, int token, int pos, int want_logits, float *trace) {
    const sgpu_qwen_cfg *c = m->c;
    const int C = c->C, HD = c->HD, NH = c->NH, KVD = m->kvd, FC = c->FC;
    const float scale = (float)(1.0 / sqrt((double)HD));
    const int dbg = m->debug && pos == 0;
    for (int i = 0; i < C; i++) m->x[i] = h2f(m->h[(size_t)token * C + i]);
    for (int l = 0; l < c->NL; l++) {
        const uint16_t *b = m->h + m->l_base + (size_t)l * m->lstride;
        if (dbg && l == 0) prvec("embed", m->x, C);
        cpu_rms(m->x, b, m->ln, C, c->eps);
        if (dbg && l == 0) prvec("ln1", m->ln, C);
        cpu_gemv_h(b + m->li_qkvw, m->ln, b + m->li_qkvb, m->qkv, C, m->qkvd);
        if (dbg && l == 0) prvec("qkv", m->qkv, m->qkvd);
        const float *cs = m->cosT + (size_t)pos * (HD / 2), *sn = m->sinT + (size_t)pos * (HD / 2);
        rope(m->qkv, NH, HD, cs, sn);
        rope(m->qkv + C, c->NKV, HD, cs, sn);
        float *kl = m->kc + (size_t)l * c->CTX * KVD, *vl = m->vc + (size_t)l * c->CTX * KVD;
        memcpy(kl + (size_t)pos * KVD, m->qkv + C, (size_t)KVD * 4);
        memcpy(vl + (size_t)pos * KVD, m->qkv + C + KVD, (size_t)KVD * 4);
        for (int h = 0; h < NH; h++) {                   /* GQA attention */
            const int g = h / (NH / c->NKV);
            float mx = -1e30f;
            for (int t = 0; t <= pos; t++) {
                float acc = 0.0f;
                for (int d = 0; d < HD; d++) acc += m->qkv[h * HD + d] * kl[(size_t)t * KVD + g * HD + d];
                m->sc[t] = acc * scale;
                if (m->sc[t] > mx) mx = m->sc[t];
            }
            float sum = 0.0f;
            for (int t = 0; t <= pos; t++) {
                m->sc[t] = expf(m->sc[t] - mx);
                sum += m->sc[t];
            }
            for (int d = 0; d < HD; d++) {
                float acc = 0.0f;
                for (int t = 0; t <= pos; t++) acc += (m->sc[t] / sum) * vl[(size_t)t * KVD + g * HD + d];
                m->att[h * HD + d] = acc;
            }
        }
        cpu_gemv_h(b + m->li_ow, m->att, NULL, m->y, C, C);
        if (dbg && l == 0) prvec("ao", m->y, C);
        for (int i = 0; i < C; i++) m->x[i] += m->y[i];
        if (dbg && l == 0) prvec("res1", m->x, C);
        cpu_rms(m->x, b + m->li_postln, m->ln, C, c->eps);
        cpu_gemv_h(b + m->li_gateup, m->ln, NULL, m->gate, C, 2 * FC);
        for (int i = 0; i < FC; i++) m->down[i] = (m->gate[i] / (1.0f + expf(-m->gate[i]))) * m->gate[FC + i];
        cpu_gemv_h(b + m->li_down, m->down, NULL, m->y, FC, C);
        for (int i = 0; i < C; i++) m->x[i] += m->y[i];
        if (trace) memcpy(trace + (size_t)l * C, m->x, (size_t)C * 4);
    }
    if (!want_logits) return;
    cpu_rms(m->x, m->h + m->off_lnfw, m->ln, C, c->eps);
    cpu_gemv_h(m->h, m->ln, NULL, m->logits, C, c->V);   /* tied lm_head */
}

static void print_top5(const char *who, const float *v, int n) {
    float *t = malloc((size_t)n * 4);
    memcpy(t, v, (size_t)n * 4);
    printf("  %s top-5 ids:", who);
    for (int k = 0; k < 5; k++) {
        const int b = argmax(t, n);
        printf(" %d", b);
        t[b] = -1e30f;
    }
    printf("\n");
    free(t);
}

/* The self-test of qwen_engine.c:494-521 (plus the per-layer trace at position 0 that
 * gpt2_engine.c:478-494 prints): positions 0..S-1 on the GPU (position 0 on the reference
 * launch sequence with its layer trace, the rest on the engine's path) and on cpu_forward.
 * Returns 1 on PASS (same argmax at position S-1). */
static int selftest(sgpu_qwen *eng, const sgpu_qwen_cfg *cfg, const void *blob, const int *ids, int S, int debug,
                    float *logits) {
    const int NL = cfg->NL, C = cfg->C, V = cfg->V;
    printf("selftest: comparing GPU vs serial-CPU logits at position %d...\n", S - 1);
    cpu_model m;
    if (!cpu_init(&m, cfg, blob, debug)) { fprintf(stderr, "selftest: out of host memory\n"); exit(2); }
    float *tr_g = malloc((size_t)NL * C * 4), *tr_c = malloc((size_t)NL * C * 4);
    if (debug) CHK(sgpu_qwen_forward_stages(eng, ids[0], 0, NULL, gprvec, NULL));
    double t0 = now_s();
    CHK(sgpu_qwen_forward_trace(eng, ids[0], 0, logits, tr_g));
    for (int p = 1; p < S; p++) CHK(sgpu_qwen_forward(eng, ids[p], p, p == S - 1, logits));
    const double t_gpu = now_s() - t0;
    t0 = now_s();
    cpu_forward(&m, ids[0], 0, S == 1, tr_c);
    for (int p = 1; p < S; p++) cpu_forward(&m, ids[p], p, p == S - 1, NULL);
    const double t_cpu = now_s() - t0;
    for (int l = 0; l < NL; l++) {
        float d = 0.0f, g = 0.0f;
        for (int i = 0; i < C; i++) {
            const float e = fabsf(tr_g[(size_t)l * C + i] - tr_c[(size_t)l * C + i]);
            if (e > d) d = e;
            if (fabsf(tr_g[(size_t)l * C + i]) > g) g = fabsf(tr_g[(size_t)l * C + i]);
        }
        printf("  trace p0 L%02d: max|d|=%.6f (|gpu|~%.3f)\n", l, d, g);
    }
    if (debug) {
        FILE *f = fopen("trace_g.bin", "wb");
        if (f) { fwrite(tr_g, 4, (size_t)NL * C, f); fclose(f); }
        f = fopen("trace_c.bin", "wb");
        if (f) { fwrite(tr_c, 4, (size_t)NL * C, f); fclose(f); }
    }
    printf("  gpu forward x%d: %.3fs\n", S, t_gpu);
    printf("  cpu reference x%d: %.3fs\n", S, t_cpu);
    double maxerr = 0.0;
    for (int i = 0; i < V; i++) {
        const double e = fabs((double)logits[i] - (double)m.logits[i]);
        if (e > maxerr) maxerr = e;
    }
    const int ag = argmax(logits, V), ac = argmax(m.logits, V);
    print_top5("gpu", logits, V);
    print_top5("cpu", m.logits, V);
    printf("  max |gpu-cpu| logit err: %.4f  argmax gpu=%d cpu=%d %s\n", maxerr, ag, ac,
           ag == ac ? "MATCH" : "MISMATCH");
    printf(ag == ac ? "  SELFTEST: PASS\n" : "  SELFTEST: FAIL\n");
    cpu_free(&m);
    free(tr_g);
    free(tr_c);
    return ag == ac;
}

/* --serve: one weight load, then requests until stdin ends, in the wire format of
 * qwen_engine.c:406-444.  In: u32 n, n u32 token ids, u32 generation budget.  Out: u32 count,
 * then that many u32 ids: the kept prompt followed by the greedy continuation.  A prompt
 * longer than CTX - 16 ids keeps its last CTX - 16; the continuation is one token plus up to
 * `budget` more (at most CTX - n - 2), and ends early after an end-of-text or end-of-turn
 * token, which is included.  An empty prompt gets an empty reply. */
typedef struct {
    uint32_t *seq;        /* the request's ids, then the continuation (room for 2 CTX) */
    uint32_t n;           /* ids kept from the request */
    uint32_t budget;
} serve_request;

static int read_words(uint32_t *dst, size_t n) { return fread(dst, 4, n, stdin) == n; }

/* 0 at the end of input or on a malformed request (more than 2 CTX ids). */
static int serve_read(serve_request *r, uint32_t most, uint32_t keep) {
    uint32_t n;
    if (!read_words(&n, 1) || n > most) return 0;
    if (n && !read_words(r->seq, n)) return 0;
    if (n > keep) {
        memmove(r->seq, r->seq + (n - keep), (size_t)keep * 4);
        n = keep;
    }
    r->n = n;
    return read_words(&r->budget, 1);
}

static void serve_write(const uint32_t *ids, uint32_t n) {
    fwrite(&n, 4, 1, stdout);
    if (n) fwrite(ids, 4, n, stdout);
    fflush(stdout);
}

static void serve_loop(sgpu_qwen *eng, const sgpu_qwen_cfg *cfg, float *logits, int batch) {
    const uint32_t ctx = (uint32_t)cfg->CTX;
    serve_request r = {malloc(sizeof(uint32_t) * (size_t)ctx * 2), 0, 0};
    while (serve_read(&r, 2 * ctx, ctx - 16)) {
        if (r.n == 0) {
            serve_write(r.seq, 0);
            continue;
        }
        const uint32_t budget = r.budget < ctx - r.n - 2 ? r.budget : ctx - r.n - 2;
        /* ids are below 2^31, so the u32 words read as the engine's ints */
        if (batch) {
            CHK(sgpu_qwen_prefill(eng, (const int *)r.seq, (int)r.n, logits));
        } else {
            for (uint32_t p = 0; p < r.n; p++) CHK(sgpu_qwen_forward(eng, (int)r.seq[p], (int)p, p + 1 == r.n, logits));
        }
        uint32_t len = r.n, extra = 0;
        int tok = argmax(logits, cfg->V);
        r.seq[len++] = (uint32_t)tok;
        while (extra < budget && len < ctx && tok != EOT && tok != IM_END) {
            CHK(sgpu_qwen_forward(eng, tok, (int)len - 1, 1, logits));
            tok = argmax(logits, cfg->V);
            r.seq[len++] = (uint32_t)tok;
            extra++;
        }
        serve_write(r.seq, len);
        fprintf(stderr, "serve: %u prompt ids -> %u generated\n", r.n, extra + 1);
    }
    free(r.seq);
}

int main(int argc, char **argv) {
    setvbuf(stdout, NULL, _IONBF, 0);
    const char *weights = NULL, *ids_file = NULL, *write_weights = NULL;
    long long seed = -1;
    int n_gen = 24, prompt_random = 0, serve = 0, json = 0, batch = 0, path = SGPU_QWEN_PATH_GRAPH;
    int n_selftest = 0, debug = 0;
    for (int i = 1; i < argc; i++) {
        if (!strcmp(argv[i], "--weights") && i + 1 < argc) weights = argv[++i];
        else if (!strcmp(argv[i], "--random") && i + 1 < argc) seed = atoll(argv[++i]);
        else if (!strcmp(argv[i], "--ids") && i + 1 < argc) ids_file = argv[++i];
        else if (!strcmp(argv[i], "--prompt-random") && i + 1 < argc) prompt_random = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--gen") && i + 1 < argc) n_gen = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--write-weights") && i + 1 < argc) write_weights = argv[++i];
        else if (!strcmp(argv[i], "--greedy")) { /* always greedy */ }
        else if (!strcmp(argv[i], "--serve")) serve = 1;
        else if (!strcmp(argv[i], "--json")) json = 1;
        else if (!strcmp(argv[i], "--batch-prefill")) batch = 1;
        else if (!strcmp(argv[i], "--selftest") && i + 1 < argc) n_selftest = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--debug")) debug = 1;
        else if (!strcmp(argv[i], "--path") && i + 1 < argc) {
            const char *v = argv[++i];
            if (!strcmp(v, "reference")) path = SGPU_QWEN_PATH_REFERENCE;
            else if (!strcmp(v, "fused")) path = SGPU_QWEN_PATH_FUSED;
            else if (!strcmp(v, "graph")) path = SGPU_QWEN_PATH_GRAPH;
            else { fprintf(stderr, "unknown path %s\n", v); return 2; }
        }
        else { fprintf(stderr, "unknown arg %s\n", argv[i]); return 2; }
    }
    if (!weights && seed < 0) { fprintf(stderr, "--weights or --random required\n"); return 2; }
    FILE *log = serve ? stderr : stdout;
    sgpu_qwen_cfg cfg;
    sgpu_qwen_default_cfg(&cfg);
    if (n_gen > cfg.CTX) n_gen = cfg.CTX;
    const size_t bytes = sgpu_qwen_file_bytes(&cfg);
    void *blob = malloc(bytes);
    if (!blob) { fprintf(stderr, "cannot allocate %zu bytes\n", bytes); return 2; }
    if (weights) {                                   /* load_weights, qwen_engine.c:105-122 */
        FILE *f = fopen(weights, "rb");
        if (!f) { fprintf(stderr, "cannot open %s\n", weights); return 2; }
        fseek(f, 0, SEEK_END);
        long sz = ftell(f);
        if (sz != (long)bytes) { fprintf(stderr, "weight file is %ld bytes, expected %zu\n", sz, bytes); return 2; }
        fseek(f, 0, SEEK_SET);
        if (fread(blob, 1, bytes, f) != bytes) { fprintf(stderr, "short read\n"); return 2; }
        fclose(f);
    } else {
        CHK(sgpu_qwen_fill_random(blob, &cfg, (uint64_t)seed, 0.02f));
    }
    if (write_weights) {
        FILE *f = fopen(write_weights, "wb");
        if (!f || fwrite(blob, 1, bytes, f) != bytes) { fprintf(stderr, "cannot write %s\n", write_weights); return 2; }
        if (fclose(f)) { fprintf(stderr, "cannot write %s\n", write_weights); return 2; }
        fprintf(stderr, "wrote %zu bytes to %s\n", bytes, write_weights);
        free(blob);
        return 0;
    }
    fprintf(log, "weights: %.1f MiB (%d-layer Qwen2.5-0.5B architecture, fp16)\n", bytes / 1048576.0, cfg.NL);
    CHK(sgpu_init(0));
    sgpu_qwen *eng = NULL;
    CHK(sgpu_qwen_create(&eng, &cfg, blob));
    CHK(sgpu_qwen_set_path(eng, path));
    float *logits = malloc(sizeof(float) * (size_t)cfg.V);
    if (serve) {
        free(blob);
        serve_loop(eng, &cfg, logits, batch);
        sgpu_qwen_destroy(eng);
        return 0;
    }

    int *ids = malloc(sizeof(int) * (size_t)cfg.CTX * 2);
    int total = 0;
    if (ids_file) {
        FILE *f = fopen(ids_file, "rb");
        if (!f) { fprintf(stderr, "cannot open ids\n"); return 2; }
        uint32_t cnt;
        if (fread(&cnt, 4, 1, f) != 1) return 2;
        if (cnt > (uint32_t)cfg.CTX) cnt = (uint32_t)cfg.CTX;
        for (uint32_t i = 0; i < cnt; i++) {
            uint32_t v;
            if (fread(&v, 4, 1, f) != 1 || v >= (uint32_t)cfg.V) return 2;
            ids[i] = (int)v;
        }
        fclose(f);
        total = (int)cnt;
    } else if (prompt_random > 0) {
        uint64_t s = 1234;
        for (int i = 0; i < prompt_random && i < cfg.CTX; i++) ids[total++] = (int)(sgpu_frand(&s) * cfg.V) % cfg.V;
    } else {
        for (int i = 0; i < 8; i++) ids[i] = (i * 7919 + 42) % cfg.V;
        total = 8;
    }
    if (total <= 0) { fprintf(stderr, "empty prompt\n"); return 2; }
    fprintf(log, "prompt: %d token(s)\n", total);

    /* optional self-test; the positions it ran stay in the cache */
    if (n_selftest > total) n_selftest = total;
    if (n_selftest > 0) selftest(eng, &cfg, blob, ids, n_selftest, debug, logits);
    free(blob);

    double tp = now_s();
    if (batch)
        CHK(sgpu_qwen_prefill(eng, ids, total, logits));
    else
        for (int p = n_selftest; p < total; p++) CHK(sgpu_qwen_forward(eng, ids[p], p, p == total - 1, logits));
    double prime_s = now_s() - tp;
    if (n_selftest > 0 && !batch)
        fprintf(log, "primed %d prompt token(s) in %.1f ms (positions 0..%d by the self-test)\n", total,
                prime_s * 1e3, n_selftest - 1);
    else
        fprintf(log, "primed %d prompt token(s) in %.1f ms\n", total, prime_s * 1e3);

    int next = argmax(logits, cfg.V);
    const int prompt_len = total;
    ids[total++] = next;
    double t_start = now_s();
    int n_new = 0;
    for (int g = 0; g < n_gen && total < cfg.CTX; g++) {
        if (next == EOT || next == IM_END) break;
        CHK(sgpu_qwen_forward(eng, next, total - 1, 1, logits));
        next = argmax(logits, cfg.V);
        ids[total++] = next;
        n_new++;
    }
    double gen_s = now_s() - t_start;
    double tps = n_new / (gen_s > 0 ? gen_s : 1e-9);
    if (json) {
        printf("{\"prompt\":%d,\"generated\":%d,\"prime_ms\":%.3f,\"decode_s\":%.6f,\"tok_s\":%.2f,\"ids\":[",
               prompt_len, n_new, prime_s * 1e3, gen_s, tps);
        for (int i = 0; i < total; i++) printf("%s%d", i ? "," : "", ids[i]);
        printf("],\"done\":true}\n");
    } else {
        printf("generated %d token(s) in %.3fs -> %.1f tok/s (fp16 weights, %d-layer Qwen2.5-0.5B architecture)\n",
               n_new, gen_s, tps, cfg.NL);
        printf("ENGINE_DONE\n");
    }
    sgpu_qwen_destroy(eng);
    free(ids);
    free(logits);
    return 0;
}
