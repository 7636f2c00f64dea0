/* gpu_workload.c -- SGEMM suite + read bandwidth on one MI355X (gfx950), verify-then-time.
 *
 * The reference harness (gpu_workload.c:50-255) on the HIP module API: the switch_gpu code
 * object is loaded with hipModuleLoadData (from a file given on the command line, or the
 * copy embedded in libswitchgpu.so), kernels are resolved by name (sgemm_tiled and
 * membw_read4 required, sgemm_naive / sgemm_tiled4 / sgemm_opt optional) and launched with
 * hipModuleLaunchKernel.  Inputs, the n = 256 CPU golden check, the 10-launch timing and the
 * --json object follow the reference; additions are marked "extra" and never change the
 * meaning of the reference keys.
 *
 * Usage: gpu_workload [--json] [--ref-geometry] [--extra 2048,4096] [--ragged]
 *                     [--membw-mb MB] [--membw-iters N] [code_object]
 *        gpu_workload --diagnostics-selftest
 *   --ref-geometry  launch with the reference's own grid/block numbers ((n/32)^2 or (n/64)^2
 *                   blocks of 16x16) instead of the kernels' intended geometry
 *   --extra         more square sizes, timed and checked on a sample of rows
 *   --ragged        add M=1023, N=1025, K=997 to the extra shapes
 *   --membw-mb      bandwidth buffer size (default 1024 MB: larger than the 256 MB MALL)
 *   --diagnostics-selftest  print the golden check's mismatch report on planted errors, on the
 *                   host only, and exit
 */
#define __HIP_PLATFORM_AMD__ 1
#include <hip/hip_runtime_api.h>

#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "switch_gpu.h"

static int json_mode;
#define OUT(...) do { if (!json_mode) printf(__VA_ARGS__); } while (0)
#define CHK(x) do { int r_ = (int)(x); if (r_) { fprintf(stderr, "HIP error %d (%s) at %s:%d\n", r_, \
    sgpu_error_string(r_), __FILE__, __LINE__); exit(1); } } while (0)

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec + ts.tv_nsec / 1e9;
}

static char *read_file(const char *path, size_t *len) {
    FILE *f = fopen(path, "rb");
    if (!f) { perror(path); exit(1); }
    fseek(f, 0, SEEK_END);
    *len = (size_t)ftell(f);
    fseek(f, 0, SEEK_SET);
    char *buf = malloc(*len + 1);
    if (!buf || fread(buf, 1, *len, f) != *len) exit(1);
    buf[*len] = 0;
    fclose(f);
    return buf;
}

/* The serial fp32 k-ascending dot product of the reference golden (gpu_workload.c:97-98),
 * over k < kend. */
static float golden_dot(const float *A, const float *B, int N, int K, int i, int j, int kend) {
    float ref = 0;
    for (int k = 0; k < kend && k < K; k++) ref += A[(size_t)i * K + k] * B[(size_t)k * N + j];
    return ref;
}

/* The reference verdict predicate (gpu_workload.c:101): |got - ref| > 5%|ref| + 1e-3. */
static int cell_bad(float got, float ref) {
    float d = got - ref;
    if (d < 0) d = -d;
    return d > 0.05f * (ref < 0 ? -ref : ref) + 1e-3f;
}

/* The reference check (gpu_workload.c:95-112): at most one bad cell counted per row, stop after
 * 5 bad rows.  The first mismatch also prints the golden's partial sums over k < 32, 64 and 96
 * (which k-slice of a tiled kernel went wrong), the next two the short form; tag NULL prints
 * the reference's own line, a kernel name prefixes it.  rows == NULL checks every row. */
static int verify(const float *A, const float *B, const float *C, int M, int N, int K, const int *rows, int nrows,
                  const char *tag) {
    int bad = 0;
    const int count = rows ? nrows : M;
    for (int r = 0; r < count && bad < 5; r++) {
        const int i = rows ? rows[r] : r;
        for (int j = 0; j < N; j++) {
            const float got = C[(size_t)i * N + j], ref = golden_dot(A, B, N, K, i, j, K);
            if (!cell_bad(got, ref)) continue;
            if (bad == 0)
                OUT("  %s%smismatch [%d][%d]: got %.4f want %.4f (k<32:%.4f k<64:%.4f k<96:%.4f)\n", tag ? tag : "",
                    tag ? " " : "", i, j, got, ref, golden_dot(A, B, N, K, i, j, 32), golden_dot(A, B, N, K, i, j, 64),
                    golden_dot(A, B, N, K, i, j, 96));
            else if (bad < 3)
                OUT("  %s%smismatch [%d][%d]: got %.4f want %.4f\n", tag ? tag : "", tag ? " " : "", i, j, got, ref);
            bad++;
            break;
        }
    }
    return bad;
}

/* The naive bisect's count (gpu_workload.c:116-131): every bad cell of the whole matrix. */
static int count_bad(const float *A, const float *B, const float *C, int M, int N, int K) {
    int nbad = 0;
    for (int i = 0; i < M; i++)
        for (int j = 0; j < N; j++) nbad += cell_bad(C[(size_t)i * N + j], golden_dot(A, B, N, K, i, j, K));
    return nbad;
}

/* --diagnostics-selftest: the check's output on planted mismatches, on the host only (no
 * device call): C is the golden product of the n = 256 inputs with cells [3][7], [3][9],
 * [10][0], [11][5], [12][1] and [200][255] offset by +1, checked as the sgemm kernel and as
 * the naive bisect. */
static int diagnostics_selftest(void) {
    const int n = 256;
    float *A = malloc((size_t)n * n * 4), *B = malloc((size_t)n * n * 4), *C = malloc((size_t)n * n * 4);
    if (!A || !B || !C) return 1;
    sgpu_gen_sgemm_inputs(A, B, (size_t)n * n, 42);
    for (int i = 0; i < n; i++)
        for (int j = 0; j < n; j++) C[(size_t)i * n + j] = golden_dot(A, B, n, n, i, j, n);
    const int planted[6][2] = {{3, 7}, {3, 9}, {10, 0}, {11, 5}, {12, 1}, {200, 255}};
    for (int p = 0; p < 6; p++) C[(size_t)planted[p][0] * n + planted[p][1]] += 1.0f;
    const int bad = verify(A, B, C, n, n, n, NULL, 0, NULL);
    OUT("sgemm %d: %s\n", n, bad ? "WRONG" : "CORRECT");
    const int nbad = count_bad(A, B, C, n, n, n);
    OUT("sgemm_naive %d: %s (%d bad cells)\n", n, nbad ? "WRONG" : "CORRECT", nbad);
    free(A); free(B); free(C);
    return 0;
}

/* A JSON string body: '"' and '\\' escaped, as the reference escapes the path (gpu_workload.c:224-227). */
static void put_json_str(const char *p) {
    for (; *p; p++) {
        if (*p == '"' || *p == '\\') putchar('\\');
        putchar(*p);
    }
}

typedef struct { const char *name; hipFunction_t f; int ref_tile; } kern;

static void launch(const kern *k, void *A, void *B, void *C, int M, int N, int K, int ref_geom) {
    unsigned g[3], b[3];
    if (ref_geom && k->ref_tile) {          /* gpu_workload.c:90,142,168: (n/T, n/T) x (16,16) */
        g[0] = (unsigned)(N / k->ref_tile); g[1] = (unsigned)(M / k->ref_tile); g[2] = 1;
        b[0] = b[1] = 16; b[2] = 1;
    } else {
        CHK(sgpu_kernel_geometry(k->name, M, N, K, g, b));
    }
    void *args[] = {&A, &B, &C, &M, &N, &K};
    CHK(hipModuleLaunchKernel(k->f, g[0], g[1], g[2], b[0], b[1], b[2], 0, NULL, args, NULL));
}

static void parse_list(const char *s, int *out, int *n, int max) {
    *n = 0;
    while (*s && *n < max) {
        out[(*n)++] = atoi(s);
        const char *c = strchr(s, ',');
        if (!c) break;
        s = c + 1;
    }
}

int main(int argc, char **argv) {
    const char *co_path = NULL;
    int ref_geom = 0, ragged = 0, n_extra = 0, extra[8];
    long membw_mb = 1024;
    int membw_iters = 10;
    for (int i = 1; i < argc; i++) {
        if (!strcmp(argv[i], "--json")) json_mode = 1;
        else if (!strcmp(argv[i], "--ref-geometry")) ref_geom = 1;
        else if (!strcmp(argv[i], "--ragged")) ragged = 1;
        else if (!strcmp(argv[i], "--extra") && i + 1 < argc) parse_list(argv[++i], extra, &n_extra, 8);
        else if (!strcmp(argv[i], "--membw-mb") && i + 1 < argc) membw_mb = atol(argv[++i]);
        else if (!strcmp(argv[i], "--membw-iters") && i + 1 < argc) membw_iters = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--diagnostics-selftest")) return diagnostics_selftest();
        else co_path = argv[i];
    }
    if (membw_mb < 1 || membw_iters < 1) { fprintf(stderr, "bad --membw-mb / --membw-iters\n"); return 2; }
    const int sizes[] = {256, 512, 1024};
    const char *v_sgemm = NULL, *v_naive = NULL, *v_tiled4 = NULL, *v_opt = NULL;
    double ms[3][3] = {{0}}, gf[3][3] = {{0}};

    CHK(sgpu_init(0));
    sgpu_device_props props;
    CHK(sgpu_get_device_props(0, &props));
    char arch[64];
    snprintf(arch, sizeof arch, "%s", props.arch);
    arch[strcspn(arch, ":")] = 0;
    /* added line: the device, which selects a consumer's sanity bounds for a text report */
    OUT("device: %s, %d CUs (%s)\n", props.name, props.compute_units, arch);
    size_t colen = 0;
    const void *image = NULL;
    char *file_image = NULL;
    if (co_path) image = file_image = read_file(co_path, &colen);
    else image = sgpu_code_object("switch_gpu", &colen);
    hipModule_t mod;
    CHK(hipModuleLoadData(&mod, image));
    kern ks[4] = {{"sgemm_tiled", NULL, 32}, {"sgemm_tiled4", NULL, 64}, {"sgemm_opt", NULL, 64},
                  {"sgemm_naive", NULL, 16}};
    hipFunction_t membw;
    CHK(hipModuleGetFunction(&ks[0].f, mod, "sgemm_tiled"));
    CHK(hipModuleGetFunction(&membw, mod, "membw_read4"));
    for (int i = 1; i < 4; i++)                            /* optional (gpu_workload.c:71-74) */
        if (hipModuleGetFunction(&ks[i].f, mod, ks[i].name) != hipSuccess) ks[i].f = NULL;

    /* ---- SGEMM, reference sizes ---- */
    for (int si = 0; si < 3; si++) {
        int n = sizes[si];
        size_t bytes = (size_t)n * n * 4;
        float *A = malloc(bytes), *B = malloc(bytes), *C = malloc(bytes);
        sgpu_gen_sgemm_inputs(A, B, (size_t)n * n, 42);   /* srand(42), interleaved (:81-82) */
        void *dA, *dB, *dC;
        CHK(sgpu_malloc(&dA, bytes)); CHK(sgpu_malloc(&dB, bytes)); CHK(sgpu_malloc(&dC, bytes));
        CHK(sgpu_memcpy_htod(dA, A, bytes)); CHK(sgpu_memcpy_htod(dB, B, bytes));
        for (int v = 0; v < 3; v++) {
            const kern *k = &ks[v];
            if (!k->f) continue;
            launch(k, dA, dB, dC, n, n, n, ref_geom);      /* verify launch doubles as warm-up */
            CHK(sgpu_synchronize());
            if (n == 256) {
                CHK(sgpu_memcpy_dtoh(C, dC, bytes));
                const char *verdict = verify(A, B, C, n, n, n, NULL, 0, v == 0 ? NULL : k->name) ? "WRONG" : "CORRECT";
                OUT("%s %d: %s\n", v == 0 ? "sgemm" : k->name, n, verdict);
                if (v == 0) v_sgemm = verdict; else if (v == 1) v_tiled4 = verdict; else v_opt = verdict;
                if (v == 0 && ks[3].f) {                    /* bisect control (:116-131) */
                    CHK(sgpu_memset_d8(dC, 0, bytes));
                    launch(&ks[3], dA, dB, dC, n, n, n, ref_geom);
                    CHK(sgpu_synchronize());
                    CHK(sgpu_memcpy_dtoh(C, dC, bytes));
                    const int nbad = count_bad(A, B, C, n, n, n);
                    v_naive = nbad ? "WRONG" : "CORRECT";
                    OUT("sgemm_naive %d: %s (%d bad cells)\n", n, v_naive, nbad);
                }
            }
            double t0 = now_s();
            for (int r = 0; r < 10; r++) launch(k, dA, dB, dC, n, n, n, ref_geom);
            CHK(sgpu_synchronize());
            double dt = now_s() - t0;
            ms[v][si] = dt * 100.0;
            gf[v][si] = 10.0 * 2.0 * n * n * n / dt / 1e9;
            OUT("%s %dx%dx%d: %.3f ms/iter, %.1f GFLOPS\n", v == 0 ? "sgemm" : v == 1 ? "sgemm4" : "sgemm_opt", n,
                n, n, ms[v][si], gf[v][si]);
        }
        sgpu_free(dA); sgpu_free(dB); sgpu_free(dC);
        free(A); free(B); free(C);
    }

    /* ---- extra shapes: timed with hipEvents, checked on 16 sampled rows ---- */
    int shapes[10][3], nshapes = 0;
    for (int i = 0; i < n_extra; i++) { shapes[nshapes][0] = shapes[nshapes][1] = shapes[nshapes][2] = extra[i]; nshapes++; }
    if (ragged) { shapes[nshapes][0] = 1023; shapes[nshapes][1] = 1025; shapes[nshapes][2] = 997; nshapes++; }
    char extra_json[8192];
    size_t ej = 0;
    extra_json[0] = 0;
    int extra_bad = 0;
    for (int s = 0; s < nshapes; s++) {
        int M = shapes[s][0], N = shapes[s][1], K = shapes[s][2];
        if (M <= 0 || N <= 0 || K <= 0) continue;
        size_t na = (size_t)M * K, nb = (size_t)K * N, nc = (size_t)M * N;
        size_t nmax = na > nb ? na : nb;
        float *A = malloc(nmax * 4), *B = malloc(nmax * 4), *C = malloc(nc * 4);
        sgpu_gen_sgemm_inputs(A, B, nmax, 42);
        void *dA, *dB, *dC;
        CHK(sgpu_malloc(&dA, na * 4)); CHK(sgpu_malloc(&dB, nb * 4)); CHK(sgpu_malloc(&dC, nc * 4));
        CHK(sgpu_memcpy_htod(dA, A, na * 4)); CHK(sgpu_memcpy_htod(dB, B, nb * 4));
        int rows[16];
        for (int r = 0; r < 16; r++) rows[r] = (int)((long long)r * (M - 1) / 15);
        void *e0, *e1;
        CHK(sgpu_event_create(&e0)); CHK(sgpu_event_create(&e1));
        for (int v = 0; v < 3; v++) {
            const kern *k = &ks[v];
            if (!k->f) continue;
            launch(k, dA, dB, dC, M, N, K, 0);
            CHK(sgpu_synchronize());
            CHK(sgpu_memcpy_dtoh(C, dC, nc * 4));
            int bad = verify(A, B, C, M, N, K, rows, 16, k->name);
            extra_bad += bad;
            const int reps = 10;
            CHK(sgpu_event_record(e0, NULL));
            for (int r = 0; r < reps; r++) launch(k, dA, dB, dC, M, N, K, 0);
            CHK(sgpu_event_record(e1, NULL));
            float tms = 0;
            CHK(sgpu_event_elapsed_ms(&tms, e0, e1));
            double per = tms / reps, gfl = 2.0 * M * N * K / (per * 1e-3) / 1e9;
            OUT("%s %dx%dx%d: %s, %.3f ms/iter, %.1f GFLOPS\n", k->name, M, N, K, bad ? "WRONG" : "CORRECT", per, gfl);
            ej += (size_t)snprintf(extra_json + ej, sizeof extra_json - ej,
                                   "%s{\"kernel\":\"%s\",\"m\":%d,\"n\":%d,\"k\":%d,\"verdict\":\"%s\",\"ms\":%.4f,\"gflops\":%.1f}",
                                   ej ? "," : "", k->name, M, N, K, bad ? "WRONG" : "CORRECT", per, gfl);
        }
        sgpu_event_destroy(e0); sgpu_event_destroy(e1);
        sgpu_free(dA); sgpu_free(dB); sgpu_free(dC);
        free(A); free(B); free(C);
    }

    /* ---- read bandwidth (gpu_workload.c:197-220), buffer sized past the MALL ---- */
    double membw_gbs = 0;
    {
        long long n4ll = membw_mb * 1024LL * 1024LL / 16;
        if (n4ll > 0x7fffffffLL) n4ll = 0x7fffffffLL;
        int n4 = (int)n4ll;
        size_t bytes = (size_t)n4 * 16;
        float *buf = malloc(bytes);
        for (size_t i = 0; i < (size_t)n4 * 4; i++) buf[i] = (float)(i % 4096) * 0.001f;
        void *dbuf, *dout;
        unsigned g[3], b[3];
        CHK(sgpu_kernel_geometry("membw_read4", 0, 0, 0, g, b));
        CHK(sgpu_malloc(&dbuf, bytes));
        CHK(sgpu_malloc(&dout, (size_t)g[0] * b[0] * 4));
        CHK(sgpu_memcpy_htod(dbuf, buf, bytes));
        void *margs[] = {&dbuf, &dout, &n4, &membw_iters};
        CHK(hipModuleLaunchKernel(membw, g[0], 1, 1, b[0], 1, 1, 0, NULL, margs, NULL));
        CHK(sgpu_synchronize());
        double t0 = now_s();
        CHK(hipModuleLaunchKernel(membw, g[0], 1, 1, b[0], 1, 1, 0, NULL, margs, NULL));
        CHK(sgpu_synchronize());
        double dt = now_s() - t0;
        membw_gbs = (double)bytes * membw_iters / dt / 1e9;
        OUT("membw read (%ldMB x%d): %.4f s, %.1f GB/s\n", membw_mb, membw_iters, dt, membw_gbs);
        sgpu_free(dbuf); sgpu_free(dout); free(buf);
    }

    if (json_mode) {                                       /* schema of gpu_workload.c:222-251 */
        const char *path = co_path ? co_path : "(embedded switch_gpu)";
        printf("{\"ptx\":\"");
        put_json_str(path);
        printf("\",\"kernels\":{\"sgemm\":\"%s\"", v_sgemm ? v_sgemm : "NOT_RUN");
        if (v_naive) printf(",\"sgemm_naive\":\"%s\"", v_naive);
        if (v_tiled4) printf(",\"sgemm_tiled4\":\"%s\"", v_tiled4);
        if (v_opt) printf(",\"sgemm_opt\":\"%s\"", v_opt);
        printf("}");
        const char *keys[3] = {"sgemm", "sgemm4", "sgemm_opt"};
        for (int v = 0; v < 3; v++) {
            if (!ks[v].f) continue;
            printf(",\"%s\":[", keys[v]);
            for (int i = 0; i < 3; i++)
                /* reference keys in the reference's %.1f; "us" (added) keeps the precision */
                printf("%s{\"n\":%d,\"ms\":%.1f,\"gflops\":%.1f,\"us\":%.1f}", i ? "," : "", sizes[i], ms[v][i],
                       gf[v][i], ms[v][i] * 1e3);
            printf("]");
        }
        if (ej) printf(",\"sgemm_extra\":[%s]", extra_json);
        /* added keys: the buffer size, and the device, which selects a consumer's sanity bounds */
        printf(",\"membw_gbps\":%.1f,\"membw_mb\":%ld,\"arch\":\"", membw_gbs, membw_mb);
        put_json_str(arch);
        printf("\",\"device\":\"");
        put_json_str(props.name);
        printf("\",\"done\":true}\n");
    } else {
        printf("WORKLOAD_DONE\n");
    }
    free(file_image);
    return extra_bad ? 1 : 0;
}
