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
 * Decoding is greedy (argmax, first max wins, qwen_engine.c:360-364) and stops at EOT or
 * <|im_end|> as the reference does (:539); --greedy is accepted for command-line
 * compatibility.
 */
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

static void serve_loop(sgpu_qwen *eng, const sgpu_qwen_cfg *cfg, float *logits, int batch) {
    const int CTX = cfg->CTX;
    int *buf = malloc(sizeof(int) * (size_t)CTX);
    uint32_t *tmp = malloc(sizeof(uint32_t) * (size_t)CTX * 2);
    for (;;) {
        uint32_t T = 0;
        if (fread(&T, 4, 1, stdin) != 1) break;
        if (T > (uint32_t)CTX * 2) break;
        if (T > 0 && fread(tmp, 4, T, stdin) != T) break;
        uint32_t keep = T > (uint32_t)(CTX - 16) ? (uint32_t)(CTX - 16) : T;   /* keep the tail */
        for (uint32_t i = 0; i < keep; i++) buf[i] = (int)tmp[T - keep + i];
        T = keep;
        uint32_t maxg = 0;
        if (fread(&maxg, 4, 1, stdin) != 1) break;
        if (T == 0) { uint32_t z = 0; fwrite(&z, 4, 1, stdout); fflush(stdout); continue; }
        if (maxg > (uint32_t)CTX - T - 2) maxg = (uint32_t)CTX - T - 2;
        if (batch)
            CHK(sgpu_qwen_prefill(eng, buf, (int)T, logits));
        else
            for (uint32_t p = 0; p < T; p++) CHK(sgpu_qwen_forward(eng, buf[p], (int)p, p == T - 1, logits));
        int total = (int)T;
        int nxt = argmax(logits, cfg->V);
        buf[total++] = nxt;
        int emitted = 0;
        for (uint32_t g = 0; g < maxg && total < CTX; g++) {
            if (nxt == EOT || nxt == IM_END) break;
            CHK(sgpu_qwen_forward(eng, nxt, total - 1, 1, logits));
            nxt = argmax(logits, cfg->V);
            buf[total++] = nxt;
            emitted++;
        }
        uint32_t outn = (uint32_t)total;
        fwrite(&outn, 4, 1, stdout);
        for (int i = 0; i < total; i++) { uint32_t v = (uint32_t)buf[i]; fwrite(&v, 4, 1, stdout); }
        fflush(stdout);
        fprintf(stderr, "serve: T=%u emitted=%d\n", T, emitted);
    }
    free(buf);
    free(tmp);
}

int main(int argc, char **argv) {
    setvbuf(stdout, NULL, _IONBF, 0);
    const char *weights = NULL, *ids_file = NULL, *write_weights = NULL;
    long long seed = -1;
    int n_gen = 24, prompt_random = 0, serve = 0, json = 0, batch = 0, path = SGPU_QWEN_PATH_GRAPH;
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
    free(blob);
    float *logits = malloc(sizeof(float) * (size_t)cfg.V);
    if (serve) {
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

    double tp = now_s();
    if (batch)
        CHK(sgpu_qwen_prefill(eng, ids, total, logits));
    else
        for (int p = 0; p < total; p++) CHK(sgpu_qwen_forward(eng, ids[p], p, p == total - 1, logits));
    double prime_s = now_s() - tp;
    fprintf(log, "primed %d prompt token(s) in %.1f ms\n", total, prime_s * 1e3);

    int next = argmax(logits, cfg.V);
    const int prompt_len = total;
    ids[total++] = next;
    double t_start = now_s();
    int emitted = 0;
    for (int g = 0; g < n_gen && total < cfg.CTX; g++) {
        if (next == EOT || next == IM_END) break;
        CHK(sgpu_qwen_forward(eng, next, total - 1, 1, logits));
        next = argmax(logits, cfg.V);
        ids[total++] = next;
        emitted++;
    }
    double gen_s = now_s() - t_start;
    double tps = emitted / (gen_s > 0 ? gen_s : 1e-9);
    if (json) {
        printf("{\"prompt\":%d,\"generated\":%d,\"prime_ms\":%.3f,\"decode_s\":%.6f,\"tok_s\":%.2f,\"ids\":[",
               prompt_len, emitted, prime_s * 1e3, gen_s, tps);
        for (int i = 0; i < total; i++) printf("%s%d", i ? "," : "", ids[i]);
        printf("],\"done\":true}\n");
    } else {
        printf("generated %d token(s) in %.3fs -> %.1f tok/s (fp16 weights, %d-layer Qwen2.5-0.5B architecture)\n",
               emitted, gen_s, tps, cfg.NL);
        printf("ENGINE_DONE\n");
    }
    sgpu_qwen_destroy(eng);
    free(ids);
    free(logits);
    return 0;
}
