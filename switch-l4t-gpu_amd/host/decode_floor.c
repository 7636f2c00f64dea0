/* decode_floor.c -- the launch and streaming costs that bound a decode step built from
 * dependent kernels, measured on one MI355X (gfx950).  Prints readable lines on stderr and one
 * JSON object on stdout.
 *
 * Usage: decode_floor [--quick]
 *
 * Legs (kernels from the embedded "sgpu_probe" code object):
 *   launch  -- chains of dependent launches recorded in a HIP graph, per-link time: an empty
 *              kernel, and one whose blocks each read a value another block wrote in the previous
 *              launch, at 1, 256 and 1024 blocks.
 *   stream  -- the streaming floor of each Qwen2.5-0.5B decode phase's weights (qkv, o, gate|up,
 *              down, lm_head, fp16): 24 dependent launches over distinct buffers (past the MALL)
 *              in one graph, each reading one value of the previous launch and then streaming
 *              its buffer with 16-byte nontemporal loads and no arithmetic; best of grids 128..2048.
 *   aql     -- the same chain links dispatched through a hand-written AQL queue: with the
 *              barrier bit (agent-scope fences, none, system-scope), and "launch-ahead": the
 *              barrier bit clear, so each link's blocks are dispatched while earlier links still
 *              run, issue their weight loads, then wait on device counters written by the earlier
 *              links (bounded waits; a give-up is reported, never a hang).
 * Every chain checks its result (each link adds 1 along the chain).
 */
#define __HIP_PLATFORM_AMD__ 1
#include <hip/hip_runtime_api.h>
#include <hsa/hsa.h>
#include <hsa/hsa_ext_amd.h>

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "switch_gpu.h"

#define CHK(x) do { int r_ = (int)(x); if (r_) { fprintf(stderr, "error %d at %s:%d\n", r_, __FILE__, __LINE__); exit(1); } } while (0)
#define HSA(x) do { hsa_status_t s_ = (x); if (s_ != HSA_STATUS_SUCCESS) { fprintf(stderr, "HSA error %#x at %s:%d\n", \
    (unsigned)s_, __FILE__, __LINE__); exit(1); } } while (0)

static double now_s(void) {
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return t.tv_sec + t.tv_nsec * 1e-9;
}

/* sgpu_probe_link's explicit arguments at their kernarg offsets (72 bytes, no hidden ones). */
typedef struct {
    const void *W; int P; int pad0;
    const float *xin; int nin; int pad1;
    float *xout;
    unsigned *counter; unsigned target; int pad2;
    unsigned *fail; int spin_limit; int mode;
} link_args;

#define MAXB 1024                 /* largest chain grid */
#define XLEN 4096                 /* floats per x buffer: every chain and stream grid (<= 2048) */
#define SPIN_LIMIT 20000          /* polls before a waiting block gives up (~tens of ms) */

static hipModule_t mod;
static hipFunction_t f_link, f_stream;
static hipStream_t stream;
static hipEvent_t ev0, ev1;
static float *xa, *xb;
static unsigned *counter, *failp;
static char *pool;                /* zeroed weight pool */
static size_t pool_bytes;

static void fill_link(link_args *a, int i, int B, int P, int mode, size_t wlink, size_t nring) {
    memset(a, 0, sizeof *a);
    a->W = wlink ? pool + (size_t)(i % nring) * wlink : NULL;
    a->P = P;
    a->xin = (i & 1) ? xb : xa;
    a->nin = B;
    a->xout = (i & 1) ? xa : xb;
    a->counter = counter;
    a->target = (unsigned)i * (unsigned)B;
    a->fail = failp;
    a->spin_limit = SPIN_LIMIT;
    a->mode = mode;
}

static void reset_chain(void) {
    CHK(hipMemset(xa, 0, XLEN * 4));
    CHK(hipMemset(xb, 0, XLEN * 4));
    CHK(hipMemset(counter, 0, 64));
    CHK(hipMemset(failp, 0, 4));
    CHK(hipDeviceSynchronize());
}

/* 0 when the chain of N links of B blocks ran through: no give-up, and every output = N. */
static int check_chain(int N, int B, int mode) {
    unsigned fl = 0;
    CHK(hipMemcpy(&fl, failp, 4, hipMemcpyDeviceToHost));
    if (mode & 4) return fl ? 1 : 0;
    float out[MAXB];
    CHK(hipMemcpy(out, (N & 1) ? xb : xa, (size_t)B * 4, hipMemcpyDeviceToHost));
    int bad = 0;
    for (int b = 0; b < B; b++) bad += out[b] != (float)N;
    if (fl || bad) fprintf(stderr, "  chain check failed: fail=%u, %d of %d outputs wrong\n", fl, bad, B);
    return fl || bad;
}

static double time_graph(hipGraphExec_t ge, int reps) {
    float best = 1e30f;
    CHK(hipGraphLaunch(ge, stream));                       /* warm-up replay */
    CHK(hipStreamSynchronize(stream));
    for (int r = 0; r < reps; r++) {
        CHK(hipEventRecord(ev0, stream));
        CHK(hipGraphLaunch(ge, stream));
        CHK(hipEventRecord(ev1, stream));
        CHK(hipEventSynchronize(ev1));
        float ms = 0;
        CHK(hipEventElapsedTime(&ms, ev0, ev1));
        if (ms < best) best = ms;
    }
    return best * 1e3;                                     /* us */
}

/* A chain of N links recorded in a graph; us per link, or -1 when its check fails. */
static double graph_chain(int N, int B, int P, int mode, int reps) {
    const size_t wlink = (size_t)B * P * 256 * 16;
    const size_t nring = wlink ? (pool_bytes / wlink < (size_t)N ? pool_bytes / wlink : (size_t)N) : 1;
    link_args *a = malloc(sizeof(link_args) * N);
    hipGraph_t g;
    hipGraphExec_t ge;
    CHK(hipStreamBeginCapture(stream, hipStreamCaptureModeRelaxed));
    for (int i = 0; i < N; i++) {
        fill_link(&a[i], i, B, P, mode, wlink, nring);
        void *kp[] = {&a[i].W, &a[i].P, &a[i].xin, &a[i].nin, &a[i].xout, &a[i].counter, &a[i].target,
                      &a[i].fail, &a[i].spin_limit, &a[i].mode};
        CHK(hipModuleLaunchKernel(f_link, B, 1, 1, 256, 1, 1, 0, stream, kp, NULL));
    }
    CHK(hipStreamEndCapture(stream, &g));
    CHK(hipGraphInstantiate(&ge, g, NULL, NULL, 0));
    double best = 1e30;
    int bad = 0;
    for (int r = 0; r <= reps; r++) {                      /* r = 0: warm-up; every replay checked */
        reset_chain();
        CHK(hipEventRecord(ev0, stream));
        CHK(hipGraphLaunch(ge, stream));
        CHK(hipEventRecord(ev1, stream));
        CHK(hipEventSynchronize(ev1));
        float ms = 0;
        CHK(hipEventElapsedTime(&ms, ev0, ev1));
        bad |= check_chain(N, B, mode);
        if (r > 0 && ms * 1e3 < best) best = ms * 1e3;
    }
    CHK(hipGraphExecDestroy(ge));
    CHK(hipGraphDestroy(g));
    free(a);
    return bad ? -1.0 : best / N;
}

/* ---- streaming floors ---- */
typedef struct { const char *name; size_t bytes; int copies; } phase_kind;

static double stream_floor(const phase_kind *k, int grid, int reps) {
    if (grid > 2048 || grid > XLEN) return 1e30;
    const int L = 24;
    const long long nvec = (long long)(k->bytes / 16);
    struct { const void *W; long long nvec; const float *prev; int nprev; int pad; float *out; unsigned *flag; } a[24];
    hipGraph_t g;
    hipGraphExec_t ge;
    CHK(hipStreamBeginCapture(stream, hipStreamCaptureModeRelaxed));
    for (int i = 0; i < L; i++) {
        a[i].W = pool + (size_t)(i % k->copies) * k->bytes;
        a[i].nvec = nvec;
        a[i].prev = (i & 1) ? xb : xa;
        a[i].nprev = grid;                                 /* grid <= 2048 <= XLEN */
        a[i].out = (i & 1) ? xa : xb;
        a[i].flag = failp;
        void *kp[] = {&a[i].W, &a[i].nvec, &a[i].prev, &a[i].nprev, &a[i].out, &a[i].flag};
        CHK(hipModuleLaunchKernel(f_stream, grid, 1, 1, 256, 1, 1, 0, stream, kp, NULL));
    }
    CHK(hipStreamEndCapture(stream, &g));
    CHK(hipGraphInstantiate(&ge, g, NULL, NULL, 0));
    const double us = time_graph(ge, reps) / L;
    CHK(hipGraphExecDestroy(ge));
    CHK(hipGraphDestroy(g));
    return us;
}

/* ---- the AQL queue ---- */
static hsa_agent_t gpu_agent;
static hsa_region_t kernarg_region;
static hsa_status_t find_gpu(hsa_agent_t a, void *d) {
    hsa_device_type_t t;
    hsa_agent_get_info(a, HSA_AGENT_INFO_DEVICE, &t);
    if (t == HSA_DEVICE_TYPE_GPU) { *(hsa_agent_t *)d = a; return HSA_STATUS_INFO_BREAK; }
    return HSA_STATUS_SUCCESS;
}
static hsa_status_t find_kernarg(hsa_region_t r, void *d) {
    hsa_region_segment_t seg;
    hsa_region_get_info(r, HSA_REGION_INFO_SEGMENT, &seg);
    if (seg != HSA_REGION_SEGMENT_GLOBAL) return HSA_STATUS_SUCCESS;
    uint32_t flags;
    hsa_region_get_info(r, HSA_REGION_INFO_GLOBAL_FLAGS, &flags);
    if (flags & HSA_REGION_GLOBAL_FLAG_KERNARG) { *(hsa_region_t *)d = r; return HSA_STATUS_INFO_BREAK; }
    return HSA_STATUS_SUCCESS;
}

typedef struct {
    hsa_queue_t *q;
    hsa_signal_t done;
    hsa_executable_t ex;
    hsa_code_object_reader_t rd;
    uint64_t kobj;
    uint32_t grp, priv;
    char *ka_host;                /* kernarg slots in the kernarg region (staging) */
    char *ka_dev;                 /* the same slots copied to device memory, as HIP places them */
    int nslots;
} aql_ctx;
#define KSLOT 128

static int aql_open(aql_ctx *c, int nslots) {
    memset(c, 0, sizeof *c);
    HSA(hsa_init());
    if (hsa_iterate_agents(find_gpu, &gpu_agent) != HSA_STATUS_INFO_BREAK) return 1;
    if (hsa_agent_iterate_regions(gpu_agent, find_kernarg, &kernarg_region) != HSA_STATUS_INFO_BREAK) return 1;
    size_t len = 0;
    const void *co = sgpu_code_object("sgpu_probe", &len);
    if (!co) return 1;
    HSA(hsa_code_object_reader_create_from_memory(co, len, &c->rd));
    HSA(hsa_executable_create_alt(HSA_PROFILE_FULL, HSA_DEFAULT_FLOAT_ROUNDING_MODE_DEFAULT, NULL, &c->ex));
    HSA(hsa_executable_load_agent_code_object(c->ex, gpu_agent, c->rd, NULL, NULL));
    HSA(hsa_executable_freeze(c->ex, NULL));
    hsa_executable_symbol_t sym;
    HSA(hsa_executable_get_symbol_by_name(c->ex, "sgpu_probe_link.kd", &gpu_agent, &sym));
    uint32_t ka_size = 0;
    HSA(hsa_executable_symbol_get_info(sym, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_OBJECT, &c->kobj));
    HSA(hsa_executable_symbol_get_info(sym, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_KERNARG_SEGMENT_SIZE, &ka_size));
    HSA(hsa_executable_symbol_get_info(sym, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_GROUP_SEGMENT_SIZE, &c->grp));
    HSA(hsa_executable_symbol_get_info(sym, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_PRIVATE_SEGMENT_SIZE, &c->priv));
    if (ka_size != sizeof(link_args)) {
        fprintf(stderr, "sgpu_probe_link kernarg segment is %u bytes, expected %zu\n", ka_size, sizeof(link_args));
        return 1;
    }
    HSA(hsa_queue_create(gpu_agent, 4096, HSA_QUEUE_TYPE_SINGLE, NULL, NULL, UINT32_MAX, UINT32_MAX, &c->q));
    HSA(hsa_signal_create(1, 0, NULL, &c->done));
    c->nslots = nslots;
    HSA(hsa_memory_allocate(kernarg_region, (size_t)KSLOT * nslots, (void **)&c->ka_host));
    CHK(hipMalloc((void **)&c->ka_dev, (size_t)KSLOT * nslots));
    return 0;
}

static void aql_close(aql_ctx *c) {
    hsa_signal_destroy(c->done);
    hsa_queue_destroy(c->q);
    hsa_memory_free(c->ka_host);
    hipFree(c->ka_dev);
    hsa_executable_destroy(c->ex);
    hsa_code_object_reader_destroy(c->rd);
    hsa_shut_down();
}

/* One chain of N links through the queue; us per link, -1 on a failed check, -2 if the chain
 * did not finish within 60 s.  barrier: the AQL barrier bit on every packet; scope: fence scope
 * of every packet's acquire and release (the first packet acquires and the last releases at
 * system scope in any case). */
static double aql_chain(aql_ctx *c, int N, int B, int P, int mode, int barrier, int scope, int reps) {
    if (N > c->nslots || N > (int)c->q->size) return -1.0;
    const size_t wlink = (size_t)B * P * 256 * 16;
    const size_t nring = wlink ? (pool_bytes / wlink < (size_t)N ? pool_bytes / wlink : (size_t)N) : 1;
    for (int i = 0; i < N; i++) {
        link_args a;
        fill_link(&a, i, B, P, mode, wlink, nring);
        memset(c->ka_host + (size_t)i * KSLOT, 0, KSLOT);
        memcpy(c->ka_host + (size_t)i * KSLOT, &a, sizeof a);
    }
    CHK(hipMemcpy(c->ka_dev, c->ka_host, (size_t)KSLOT * N, hipMemcpyHostToDevice));
    double best = 1e30;
    int bad = 0;
    for (int r = 0; r <= reps; r++) {                     /* r = 0: warm-up, also checked */
        reset_chain();
        hsa_signal_store_relaxed(c->done, 1);
        const uint64_t base = hsa_queue_load_write_index_relaxed(c->q);
        while (base + N - hsa_queue_load_read_index_scacquire(c->q) > c->q->size) {}
        hsa_kernel_dispatch_packet_t *pk = (hsa_kernel_dispatch_packet_t *)c->q->base_address;
        const double t0 = now_s();
        for (int i = 0; i < N; i++) {
            hsa_kernel_dispatch_packet_t *p = &pk[(base + i) & (c->q->size - 1)];
            memset((char *)p + 4, 0, sizeof *p - 4);
            p->workgroup_size_x = 256;
            p->workgroup_size_y = p->workgroup_size_z = 1;
            p->grid_size_x = 256u * (unsigned)B;
            p->grid_size_y = p->grid_size_z = 1;
            p->private_segment_size = c->priv;
            p->group_segment_size = c->grp;
            p->kernel_object = c->kobj;
            p->kernarg_address = c->ka_dev + (size_t)i * KSLOT;
            if (i == N - 1) p->completion_signal = c->done;
            const int acq = i == 0 ? HSA_FENCE_SCOPE_SYSTEM : scope;
            const int rel = i == N - 1 ? HSA_FENCE_SCOPE_SYSTEM : scope;
            const uint16_t header = (uint16_t)((HSA_PACKET_TYPE_KERNEL_DISPATCH << HSA_PACKET_HEADER_TYPE) |
                                               ((barrier ? 1 : 0) << HSA_PACKET_HEADER_BARRIER) |
                                               (acq << HSA_PACKET_HEADER_SCACQUIRE_FENCE_SCOPE) |
                                               (rel << HSA_PACKET_HEADER_SCRELEASE_FENCE_SCOPE));
            const uint32_t setup = 1u << HSA_KERNEL_DISPATCH_PACKET_SETUP_DIMENSIONS;
            __atomic_store_n((uint32_t *)p, header | (setup << 16), __ATOMIC_RELEASE);
        }
        hsa_queue_store_write_index_relaxed(c->q, base + N);
        hsa_signal_store_screlease(c->q->doorbell_signal, (hsa_signal_value_t)(base + N - 1));
        while (hsa_signal_wait_scacquire(c->done, HSA_SIGNAL_CONDITION_LT, 1, 1000000, HSA_WAIT_STATE_ACTIVE) >= 1)
            if (now_s() - t0 > 60.0) return -2.0;
        const double us = (now_s() - t0) * 1e6;
        bad |= check_chain(N, B, mode);
        if (r > 0 && us < best) best = us;
    }
    return bad ? -1.0 : best / N;
}

int main(int argc, char **argv) {
    int quick = argc > 1 && !strcmp(argv[1], "--quick");
    const int reps = quick ? 3 : 7, N = 240;
    CHK(sgpu_init(0));
    size_t colen = 0;
    const void *co = sgpu_code_object("sgpu_probe", &colen);
    if (!co) { fprintf(stderr, "no sgpu_probe code object\n"); return 1; }
    CHK(hipModuleLoadData(&mod, co));
    CHK(hipModuleGetFunction(&f_link, mod, "sgpu_probe_link"));
    CHK(hipModuleGetFunction(&f_stream, mod, "sgpu_probe_stream"));
    CHK(hipStreamCreate(&stream));
    CHK(hipEventCreate(&ev0));
    CHK(hipEventCreate(&ev1));
    CHK(hipMalloc((void **)&xa, XLEN * 4));
    CHK(hipMalloc((void **)&xb, XLEN * 4));
    CHK(hipMalloc((void **)&counter, 64));
    CHK(hipMalloc((void **)&failp, 4));
    /* weights: 4 copies of the lm_head (1.09 GB), past the 256 MB MALL; every leg carves it */
    const phase_kind kinds[] = {{"qkv", 1152ull * 896 * 2, 24}, {"o", 896ull * 896 * 2, 24},
                                {"gate_up", 9728ull * 896 * 2, 24}, {"down", 896ull * 4864 * 2, 24},
                                {"lm_head", 151936ull * 896 * 2, 4}};
    pool_bytes = kinds[4].bytes * 4;
    for (int k = 0; k < 4; k++)
        if (kinds[k].bytes * kinds[k].copies > pool_bytes) { fprintf(stderr, "pool too small\n"); return 1; }
    CHK(hipMalloc((void **)&pool, pool_bytes));
    CHK(hipMemset(pool, 0, pool_bytes));
    CHK(hipDeviceSynchronize());
    sgpu_device_props props;
    CHK(sgpu_get_device_props(0, &props));
    fprintf(stderr, "device: %s, %d CUs\n", props.name, props.compute_units);

    /* settle the clocks: a second of chains */
    for (double t0 = now_s(); now_s() - t0 < (quick ? 0.3 : 1.0);) graph_chain(N, 256, 4, 0, 1);

    printf("{\"device\":\"%s\",\"cus\":%d", props.name, props.compute_units);
    /* ---- dependent launches ---- */
    const int grids[3] = {1, 256, 1024};
    printf(",\"dependent_launch_us\":{");
    for (int m = 0; m < 2; m++)
        for (int gi = 0; gi < 3; gi++) {
            const double us = graph_chain(200, grids[gi], 0, m == 0 ? 4 : 0, reps);
            fprintf(stderr, "graph launch, %s, %4d blocks: %.3f us per link\n", m == 0 ? "empty kernel" : "cross-block read",
                    grids[gi], us);
            printf("%s\"%s_%d\":%.3f", m + gi ? "," : "", m == 0 ? "empty" : "read", grids[gi], us);
        }
    printf("}");
    /* ---- streaming floors ---- */
    const int sgrids[5] = {128, 256, 512, 1024, 2048};
    printf(",\"stream_floor\":{");
    for (int k = 0; k < 5; k++) {
        double best = 1e30;
        int bg = 0;
        for (int gi = 0; gi < 5; gi++) {
            const double us = stream_floor(&kinds[k], sgrids[gi], reps);
            if (us < best) best = us, bg = sgrids[gi];
        }
        fprintf(stderr, "stream floor %-8s %7.2f MB: %7.3f us (grid %d, %.0f GB/s)\n", kinds[k].name, kinds[k].bytes / 1e6,
                best, bg, kinds[k].bytes / best / 1e3);
        printf("%s\"%s\":{\"bytes\":%zu,\"us\":%.3f,\"grid\":%d,\"gbps\":%.1f}", k ? "," : "", kinds[k].name, kinds[k].bytes,
               best, bg, kinds[k].bytes / best / 1e3);
    }
    printf("}");
    /* ---- graph vs AQL, 240-link chains of 256 blocks ---- */
    const int Ps[3] = {0, 4, 8};
    printf(",\"chain_256_blocks\":{\"links\":%d,\"mb_per_link\":[0,%.2f,%.2f]", N, 256.0 * 4 * 4096 / 1e6,
           256.0 * 8 * 4096 / 1e6);
    printf(",\"graph\":[");
    for (int i = 0; i < 3; i++) {
        const double us = graph_chain(N, 256, Ps[i], 0, reps);
        fprintf(stderr, "graph chain, P %d: %.3f us per link\n", Ps[i], us);
        printf("%s%.3f", i ? "," : "", us);
    }
    printf("]");
    aql_ctx c;
    if (aql_open(&c, N)) {
        fprintf(stderr, "AQL legs skipped: no HSA queue\n");
        printf("}}\n");
        return 1;
    }
    int failed = 0;
    printf(",\"aql_barrier_agent\":[");
    for (int i = 0; i < 3; i++) {
        const double us = aql_chain(&c, N, 256, Ps[i], 0, 1, HSA_FENCE_SCOPE_AGENT, reps);
        failed |= us < 0;
        fprintf(stderr, "aql barrier, agent fences, P %d: %.3f us per link\n", Ps[i], us);
        printf("%s%.3f", i ? "," : "", us);
    }
    printf("]");
    const struct { const char *key; int scope; } fences[3] = {
        {"aql_barrier_agent_empty", HSA_FENCE_SCOPE_AGENT}, {"aql_barrier_nofence_empty", HSA_FENCE_SCOPE_NONE},
        {"aql_barrier_system_empty", HSA_FENCE_SCOPE_SYSTEM}};
    for (int f = 0; f < 3; f++) {
        const double us = aql_chain(&c, N, 256, 0, 4, 1, fences[f].scope, reps);
        failed |= us < 0;
        fprintf(stderr, "%s: %.3f us per link\n", fences[f].key, us);
        printf(",\"%s\":%.3f", fences[f].key, us);
    }
    printf(",\"aql_launch_ahead\":[");
    for (int i = 0; i < 3; i++) {
        const double us = aql_chain(&c, N, 256, Ps[i], 3, 0, HSA_FENCE_SCOPE_NONE, reps);
        failed |= us < 0;
        fprintf(stderr, "aql launch-ahead (no barrier, device counters), P %d: %.3f us per link\n", Ps[i], us);
        printf("%s%.3f", i ? "," : "", us);
    }
    printf("]}");
    const double us512 = aql_chain(&c, N, 512, 4, 3, 0, HSA_FENCE_SCOPE_NONE, reps);
    failed |= us512 < 0;
    fprintf(stderr, "aql launch-ahead, 512 blocks, P 4: %.3f us per link\n", us512);
    printf(",\"aql_launch_ahead_512_blocks_p4\":%.3f,\"checks\":\"%s\"}\n", us512, failed ? "FAILED" : "ok");
    aql_close(&c);
    return failed;
}
