/* sgemm_floor.c -- the matrix-core floor of short SGEMM launches on one MI355X (gfx950), next
 * to the library's SGEMM at the same shapes.  Prints readable lines on stderr and one JSON object
 * on stdout.
 *
 * Usage: sgemm_floor [--quick]
 *
 * Legs, each a graph of 50 dependent launches replayed after at least 0.2 s of warm-up, the
 * best of the timed replays, us per launch:
 *   mfma  -- sgpu_probe_mfma (embedded "sgpu_probe" code object) on 256 blocks of 256 threads,
 *            one wave per SIMD, iters x 16 fp32 32x32x2 MFMAs per wave with operands in
 *            registers, then a 4 MB store: iters 0 (launch and store only) to 512.  At iters 32
 *            each SIMD issues the MFMA count of a 1024^3 SGEMM spread over the 256 CUs.
 *   sgemm -- sgpu_sgemm_opt at 1024^3 (sgemm_kwave), 768x1024x1024 and 1023x1025x997
 *            (sgemm_kwave_edge) on integer inputs, each result checked exactly before timing.
 */
#define __HIP_PLATFORM_AMD__ 1
#include <hip/hip_runtime_api.h>

#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "switch_gpu.h"

#define CHK(x) do { int r_ = (int)(x); if (r_) { fprintf(stderr, "error %d at %s:%d\n", r_, __FILE__, __LINE__); exit(1); } } while (0)

#define BLOCKS 256
#define LAUNCHES 50

static hipStream_t stream;
static hipEvent_t ev0, ev1;

static double now_s(void) {
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return t.tv_sec + t.tv_nsec * 1e-9;
}

/* Best us per launch of a graph of LAUNCHES launches, after >= warm_s of replays. */
static double time_graph(hipGraphExec_t ge, double warm_s, int reps) {
    for (double t0 = now_s(); now_s() - t0 < warm_s;) {
        CHK(hipGraphLaunch(ge, stream));
        CHK(hipStreamSynchronize(stream));
    }
    float best = 1e30f;
    for (int r = 0; r < reps; r++) {
        CHK(hipEventRecord(ev0, stream));
        CHK(hipGraphLaunch(ge, stream));
        CHK(hipEventRecord(ev1, stream));
        CHK(hipEventSynchronize(ev1));
        float ms = 0;
        CHK(hipEventElapsedTime(&ms, ev0, ev1));
        if (ms < best) best = ms;
    }
    return best * 1e3 / LAUNCHES;
}

static double mfma_leg(hipFunction_t f, float *out, long long nout, int iters, double warm_s, int reps) {
    float a0 = 1.0f, b0 = 1.0f;
    void *kp[] = {&out, &nout, &iters, &a0, &b0};
    hipGraph_t g;
    hipGraphExec_t ge;
    CHK(hipStreamBeginCapture(stream, hipStreamCaptureModeRelaxed));
    for (int l = 0; l < LAUNCHES; l++) CHK(hipModuleLaunchKernel(f, BLOCKS, 1, 1, 256, 1, 1, 0, stream, kp, NULL));
    CHK(hipStreamEndCapture(stream, &g));
    CHK(hipGraphInstantiate(&ge, g, NULL, NULL, 0));
    const double us = time_graph(ge, warm_s, reps);
    CHK(hipGraphExecDestroy(ge));
    CHK(hipGraphDestroy(g));
    return us;
}

/* sgpu_sgemm_opt on integer inputs in [-2, 2]: the result is checked exactly (every partial
 * sum is an integer below 2^24), then timed; -1 when the check fails. */
static double sgemm_leg(int M, int N, int K, double warm_s, int reps) {
    float *hA = malloc(sizeof(float) * M * K), *hB = malloc(sizeof(float) * K * N), *hC = malloc(sizeof(float) * M * N);
    uint32_t s = 12345u + M + N + K;
    for (long long i = 0; i < (long long)M * K; i++) s = s * 1664525u + 1013904223u, hA[i] = (float)((int)(s >> 24) % 5 - 2);
    for (long long i = 0; i < (long long)K * N; i++) s = s * 1664525u + 1013904223u, hB[i] = (float)((int)(s >> 24) % 5 - 2);
    float *dA, *dB, *dC;
    CHK(hipMalloc((void **)&dA, sizeof(float) * M * K));
    CHK(hipMalloc((void **)&dB, sizeof(float) * K * N));
    CHK(hipMalloc((void **)&dC, sizeof(float) * M * N));
    CHK(hipMemcpy(dA, hA, sizeof(float) * M * K, hipMemcpyHostToDevice));
    CHK(hipMemcpy(dB, hB, sizeof(float) * K * N, hipMemcpyHostToDevice));
    CHK(sgpu_sgemm_opt(dA, dB, dC, M, N, K, stream));
    CHK(hipStreamSynchronize(stream));
    CHK(hipMemcpy(hC, dC, sizeof(float) * M * N, hipMemcpyDeviceToHost));
    int bad = 0;
    for (int i = 0; i < M && !bad; i += 37)                  /* a sample of rows, every column */
        for (int j = 0; j < N; j++) {
            double acc = 0.0;
            for (int k = 0; k < K; k++) acc += (double)hA[(size_t)i * K + k] * hB[(size_t)k * N + j];
            if (hC[(size_t)i * N + j] != (float)acc) { bad = 1; break; }
        }
    double us = -1.0;
    if (!bad) {
        hipGraph_t g;
        hipGraphExec_t ge;
        CHK(hipStreamBeginCapture(stream, hipStreamCaptureModeRelaxed));
        for (int l = 0; l < LAUNCHES; l++) CHK(sgpu_sgemm_opt(dA, dB, dC, M, N, K, stream));
        CHK(hipStreamEndCapture(stream, &g));
        CHK(hipGraphInstantiate(&ge, g, NULL, NULL, 0));
        us = time_graph(ge, warm_s, reps);
        CHK(hipGraphExecDestroy(ge));
        CHK(hipGraphDestroy(g));
    }
    CHK(hipFree(dA));
    CHK(hipFree(dB));
    CHK(hipFree(dC));
    free(hA);
    free(hB);
    free(hC);
    return us;
}

int main(int argc, char **argv) {
    const int quick = argc > 1 && !strcmp(argv[1], "--quick");
    const int reps = quick ? 5 : 20;
    const double warm_s = quick ? 0.1 : 0.2;
    CHK(sgpu_init(0));
    size_t colen = 0;
    const void *co = sgpu_code_object("sgpu_probe", &colen);
    if (!co) { fprintf(stderr, "no sgpu_probe code object\n"); return 1; }
    hipModule_t mod;
    hipFunction_t f;
    CHK(hipModuleLoadData(&mod, co));
    CHK(hipModuleGetFunction(&f, mod, "sgpu_probe_mfma"));
    CHK(hipStreamCreate(&stream));
    CHK(hipEventCreate(&ev0));
    CHK(hipEventCreate(&ev1));
    const long long nout = (long long)BLOCKS * 256 * 16;       /* 4 MB, the size of a 1024^2 C */
    float *out;
    CHK(hipMalloc((void **)&out, sizeof(float) * nout));
    sgpu_device_props props;
    CHK(sgpu_get_device_props(0, &props));
    fprintf(stderr, "device: %s, %d CUs\n", props.name, props.compute_units);
    printf("{\"device\":\"%s\",\"cus\":%d,\"blocks\":%d,\"launches_per_graph\":%d", props.name, props.compute_units,
           BLOCKS, LAUNCHES);

    const int iters[] = {0, 4, 8, 16, 32, 64, 128, 512};
    printf(",\"mfma\":[");
    for (int i = 0; i < 8; i++) {
        const double us = mfma_leg(f, out, nout, iters[i], warm_s, reps);
        const double per_simd = iters[i] * 16.0, ideal = per_simd * 64 / 2400.0;
        fprintf(stderr, "mfma probe, %4d MFMAs per wave: %8.3f us per launch (issue time at 2.4 GHz %.3f us)\n",
                (int)per_simd, us, ideal);
        printf("%s{\"mfma_per_wave\":%d,\"us\":%.3f,\"issue_us_2p4ghz\":%.3f}", i ? "," : "", (int)per_simd, us, ideal);
    }
    printf("]");

    const int shapes[3][3] = {{1024, 1024, 1024}, {768, 1024, 1024}, {1023, 1025, 997}};
    int failed = 0;
    printf(",\"sgemm\":[");
    for (int i = 0; i < 3; i++) {
        const int M = shapes[i][0], N = shapes[i][1], K = shapes[i][2];
        const double us = sgemm_leg(M, N, K, warm_s, reps);
        failed |= us < 0;
        const double tf = us > 0 ? 2.0 * M * N * K / us / 1e6 : 0.0;
        fprintf(stderr, "sgpu_sgemm_opt %dx%dx%d: %.3f us per launch, %.1f TFLOP/s\n", M, N, K, us, tf);
        printf("%s{\"M\":%d,\"N\":%d,\"K\":%d,\"us\":%.3f,\"tflops\":%.2f}", i ? "," : "", M, N, K, us, tf);
    }
    printf("],\"checks\":\"%s\"}\n", failed ? "FAILED" : "ok");
    CHK(hipFree(out));
    CHK(hipModuleUnload(mod));
    return failed;
}
