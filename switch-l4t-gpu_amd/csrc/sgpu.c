/* sgpu.c -- libswitchgpu.so: the C-ABI host side of the gfx950 matmul hot path.
 *
 * Plain C over the HIP module API: the gfx950 code objects are embedded in this library
 * (code_objects.S) and loaded with hipModuleLoadData, kernels are resolved by name with
 * hipModuleGetFunction and launched with hipModuleLaunchKernel -- the HIP counterparts of
 * the reference's cuModuleLoadData / cuModuleGetFunction / cuLaunchKernel flow
 * (gpu_workload.c:68-74,90; qwen_engine.c:147-155,216-266).  The launchers own the launch
 * geometry (wave64 blocks), so callers pass only the reference kernels' own arguments.
 */
#define __HIP_PLATFORM_AMD__ 1
#include <hip/hip_runtime_api.h>

#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "sgpu_internal.h"
#include "switch_gpu.h"

#define SK_STREAMS 32        /* streams per device with their own split-K workspace */

/* ---- embedded code objects (code_objects.S) ---- */
extern const unsigned char sgpu_co_switch_gpu[], sgpu_co_switch_gpu_end[];
extern const unsigned char sgpu_co_gemv[], sgpu_co_gemv_end[];
extern const unsigned char sgpu_co_gpt2_kernels[], sgpu_co_gpt2_kernels_end[];
extern const unsigned char sgpu_co_qwen_kernels[], sgpu_co_qwen_kernels_end[];
extern const unsigned char sgpu_co_sgpu_tuned[], sgpu_co_sgpu_tuned_end[];
extern const unsigned char sgpu_co_sgpu_decode[], sgpu_co_sgpu_decode_end[];
extern const unsigned char sgpu_co_sgpu_probe[], sgpu_co_sgpu_probe_end[];

enum { MOD_SWITCH, MOD_GEMV, MOD_GPT2, MOD_QWEN, MOD_TUNED, MOD_DECODE, MOD_PROBE, NMOD };
static const struct {
    const char *name;
    const unsigned char *start, *end;
} g_cos[NMOD] = {
    {"switch_gpu", sgpu_co_switch_gpu, sgpu_co_switch_gpu_end},
    {"gemv", sgpu_co_gemv, sgpu_co_gemv_end},
    {"gpt2_kernels", sgpu_co_gpt2_kernels, sgpu_co_gpt2_kernels_end},
    {"qwen_kernels", sgpu_co_qwen_kernels, sgpu_co_qwen_kernels_end},
    {"sgpu_tuned", sgpu_co_sgpu_tuned, sgpu_co_sgpu_tuned_end},
    {"sgpu_decode", sgpu_co_sgpu_decode, sgpu_co_sgpu_decode_end},
    {"sgpu_probe", sgpu_co_sgpu_probe, sgpu_co_sgpu_probe_end},
};

/* Every kernel the launchers use: (module, symbol). */
enum {
    K_SGEMM_TILED, K_SGEMM_TILED4, K_SGEMM_OPT, K_SGEMM_OPT256, K_SGEMM_SPLITK, K_SGEMM_SMALL16, K_SGEMM_SMALL32,
    K_SGEMM_KWAVE, K_SGEMM_KWAVE_EDGE, K_SGEMM_KWAVE_WIDE, K_SGEMM_KWAVE_EDGE_WIDE, K_SGEMM_KWAVE128, K_SGEMM_NAIVE,
    K_MEMBW,
    K_GEMV, K_GEMV4, K_GEMV_WARP, K_GEMV_WARP_B, K_GEMV_MULTI, K_GEMV_MULTI_SPLITK, K_GEMV_MULTI_X8_64,
    K_GEMV_MULTI_X8_256,
    K_GEMV_H, K_GEMV_HH, K_RMSNORM, K_ROPE, K_SWIGLU, K_ASCORES, K_ASOFTMAX, K_AMIX, K_ADD2,
    K_EMBED_H,
    K_LAYERNORM, K_GELU, K_ADD_BIAS, K_G2_SCORES, K_G2_SOFTMAX, K_G2_MIX,
    NKERN
};
static const struct {
    int mod;
    const char *sym;
} g_kern[NKERN] = {
    {MOD_SWITCH, "sgemm_tiled"}, {MOD_SWITCH, "sgemm_tiled4"}, {MOD_SWITCH, "sgemm_opt"},
    {MOD_SWITCH, "sgemm_opt256"}, {MOD_SWITCH, "sgemm_splitk"}, {MOD_SWITCH, "sgemm_small16"},
    {MOD_SWITCH, "sgemm_small32"}, {MOD_SWITCH, "sgemm_kwave"}, {MOD_SWITCH, "sgemm_kwave_edge"},
    {MOD_SWITCH, "sgemm_kwave_wide"}, {MOD_SWITCH, "sgemm_kwave_edge_wide"}, {MOD_SWITCH, "sgemm_kwave128"},
    {MOD_SWITCH, "sgemm_naive"},
    {MOD_SWITCH, "membw_read4"},
    {MOD_GEMV, "gemv"}, {MOD_GEMV, "gemv4"}, {MOD_GEMV, "gemv_warp"},
    {MOD_GPT2, "gemv_warp_b"}, {MOD_GPT2, "gemv_multi"}, {MOD_GPT2, "gemv_multi_splitk"},
    {MOD_GPT2, "gemv_multi_x8_l64"}, {MOD_GPT2, "gemv_multi_x8_l256"},
    {MOD_QWEN, "gemv_h"}, {MOD_QWEN, "gemv_hh"}, {MOD_QWEN, "rmsnorm"}, {MOD_QWEN, "rope"}, {MOD_QWEN, "swiglu"},
    {MOD_QWEN, "attn_scores_gqa"}, {MOD_QWEN, "attn_softmax"}, {MOD_QWEN, "attn_mix_gqa"},
    {MOD_QWEN, "add2"},
    {MOD_TUNED, "sgpu_embed_h"},
    {MOD_GPT2, "layernorm"}, {MOD_GPT2, "gelu"}, {MOD_GPT2, "add_bias"}, {MOD_GPT2, "attn_scores"},
    {MOD_GPT2, "attn_softmax"}, {MOD_GPT2, "attn_mix"},
};

/* Tuned GEMV table: team sizes x segments-per-lane instantiated in sgpu_tuned.hip. */
static const int g_lpr[3] = {16, 64, 256};
static const int g_segs[10] = {1, 2, 3, 4, 6, 7, 8, 10, 12, 16};
#define NLPR 3
#define NSEG 10

/* Fused decode GEMV families (sgpu_decode.hip): (lanes per team, segments per lane). */
static const int g_dec_cfg[][2] = {{16, 1}, {16, 2}, {16, 4}, {16, 7}, {16, 8}, {64, 1}, {64, 2}, {64, 4},
                                   {64, 8}, {256, 1}, {256, 2}, {256, 3}, {256, 4}, {256, 8}, {64, 10}};
#define NDEC_PAIR 9      /* the first 9 entries: teams of up to one wave (two-row families) */
#define NDEC_ALL 15
enum { DEC_QKV, DEC_GATEUP, DEC_RES, DEC_LMHEAD, DEC_G2QKV, DEC_G2RES, DEC_G2FC, DEC_G2LMHEAD, NDECFAM };
static const char *g_dec_fam[NDECFAM] = {"qkv", "gateup", "res", "lmhead", "g2qkv", "g2res", "g2fc", "g2lmhead"};
/* Two-row (pair) families use the first NDEC_PAIR configurations; weights per 16-byte
 * segment: 8 fp16 (Qwen families) or 4 fp32 (GPT-2 families). */
static int dec_is_pair(int f) { return f == DEC_QKV || f == DEC_GATEUP; }
static int dec_vec(int f) { return f >= DEC_G2QKV ? 4 : 8; }

typedef struct {
    int ready;
    int cus;
    hipModule_t mod[NMOD];
    hipFunction_t fn[NKERN];
    hipFunction_t gemv_f32[NLPR][NSEG], gemv_h[NLPR][NSEG], gemv_hh[NLPR][NSEG];
    hipFunction_t dec[NDECFAM][NDEC_ALL];
    hipFunction_t dec_attn[3], dec_embed, dec_argmax_part, dec_argmax_embed;
    hipFunction_t dec_g2embed, dec_argmax_g2embed;
    hipFunction_t pf_embed, pf_gemm, pf_qkv_post, pf_attn[3], pf_swiglu;
    /* Split-K workspaces, one per stream that has launched split work (slot 0: the null
     * stream, made with the device state): partial tiles (SK_WS_FLOATS) and arrival counters
     * (SK_MAX_TILES, zero between launches).  Launches on one stream run in order, so a
     * stream's split launches never overlap; concurrent streams have separate workspaces. */
    struct {
        void *stream;
        float *ws;
        unsigned *cnt;
        int graphs;           /* recorded graphs (sgpu_graph_end) that reference this workspace */
        int orphan;           /* its stream was destroyed while graphs still referenced it */
    } sk[SK_STREAMS];
    int nsk;
} devstate;

static devstate g_dev[SGPU_MAX_DEVICES];

/* Split-K member (sgemm_splitk): 64x64 tiles, slices of 32; workspace for S x tiles partial
 * tiles of 4096 floats (32 MB: 4 splits of 512 tiles, the most the dispatch rule picks) and
 * one counter per tile. */
#define SK_TILE 64
#define SK_BK 32
#define SK_WS_FLOATS (8u << 20)
#define SK_MAX_TILES 16384u
static pthread_mutex_t g_lock = PTHREAD_MUTEX_INITIALIZER;

const char *sgpu_error_string(int status) {
    switch (status) {
    case SGPU_OK: return "success";
    case SGPU_ERR_INVALID_ARG: return "invalid argument (size, shape or pointer)";
    case SGPU_ERR_NOT_INITIALIZED: return "sgpu_init has not succeeded on the current device";
    case SGPU_ERR_NO_KERNEL: return "kernel not found in the code object";
    case SGPU_ERR_NO_DEVICE: return "no usable HIP device";
    case SGPU_ERR_HOST_ALLOC: return "host allocation failed";
    case SGPU_ERR_SCRATCH_LIMIT:
        return "the problem needs more than the allocation-free entry point's fixed scratch (32 MiB of partial "
               "tiles: splits x 64x64 tiles x 4096 floats, at most 16384 tiles)";
    case SGPU_ERR_NO_WORKSPACE:
        return "no split-K workspace for this stream (make the stream's first split-K call outside graph "
               "capture; at most 32 streams per device have one)";
    default: break;
    }
    if (status > 0) return hipGetErrorString((hipError_t)status);
    return "unknown sgpu error";
}

#define HIPCHK(x)                                \
    do {                                         \
        hipError_t e_ = (x);                     \
        if (e_ != hipSuccess) return (int)e_;    \
    } while (0)

/* Unload what a failed load_device left behind, so a later call starts from nothing. */
static void unload_device(devstate *d) {
    for (int m = 0; m < NMOD; m++)
        if (d->mod[m]) hipModuleUnload(d->mod[m]);
    if (d->nsk > 0) {
        hipFree(d->sk[0].ws);
        hipFree(d->sk[0].cnt);
    }
    memset(d, 0, sizeof *d);
}

static int load_device(int dev) {
    devstate *d = &g_dev[dev];
    if (__atomic_load_n(&d->ready, __ATOMIC_ACQUIRE)) return SGPU_OK;
    int rc = SGPU_OK;
    pthread_mutex_lock(&g_lock);
    if (__atomic_load_n(&d->ready, __ATOMIC_RELAXED)) goto out;
    hipDeviceProp_t p;
    hipError_t e = hipGetDeviceProperties(&p, dev);
    if (e != hipSuccess) { rc = (int)e; goto out; }
    d->cus = p.multiProcessorCount > 0 ? p.multiProcessorCount : 1;
    for (int m = 0; m < NMOD; m++) {
        e = hipModuleLoadData(&d->mod[m], g_cos[m].start);
        if (e != hipSuccess) { d->mod[m] = NULL; rc = (int)e; goto fail; }
    }
    for (int k = 0; k < NKERN; k++) {
        e = hipModuleGetFunction(&d->fn[k], d->mod[g_kern[k].mod], g_kern[k].sym);
        if (e != hipSuccess) { rc = SGPU_ERR_NO_KERNEL; goto fail; }
    }
    for (int i = 0; i < NLPR; i++)
        for (int j = 0; j < NSEG; j++) {
            char name[64];
            snprintf(name, sizeof name, "sgpu_gemv_f32_l%d_s%d", g_lpr[i], g_segs[j]);
            e = hipModuleGetFunction(&d->gemv_f32[i][j], d->mod[MOD_TUNED], name);
            if (e != hipSuccess) { rc = SGPU_ERR_NO_KERNEL; goto fail; }
            snprintf(name, sizeof name, "sgpu_gemv_h_l%d_s%d", g_lpr[i], g_segs[j]);
            e = hipModuleGetFunction(&d->gemv_h[i][j], d->mod[MOD_TUNED], name);
            if (e != hipSuccess) { rc = SGPU_ERR_NO_KERNEL; goto fail; }
            snprintf(name, sizeof name, "sgpu_gemv_hh_l%d_s%d", g_lpr[i], g_segs[j]);
            e = hipModuleGetFunction(&d->gemv_hh[i][j], d->mod[MOD_TUNED], name);
            if (e != hipSuccess) { rc = SGPU_ERR_NO_KERNEL; goto fail; }
        }
    for (int f = 0; f < NDECFAM; f++) {
        int n = dec_is_pair(f) ? NDEC_PAIR : NDEC_ALL;
        for (int j = 0; j < n; j++) {
            char name[64];
            snprintf(name, sizeof name, "sgpu_dec_%s_l%d_s%d", g_dec_fam[f], g_dec_cfg[j][0], g_dec_cfg[j][1]);
            e = hipModuleGetFunction(&d->dec[f][j], d->mod[MOD_DECODE], name);
            if (e != hipSuccess) { rc = SGPU_ERR_NO_KERNEL; goto fail; }
        }
    }
    {
        const char *attn[3] = {"sgpu_dec_attn32", "sgpu_dec_attn64", "sgpu_dec_attn128"};
        const char *pattn[3] = {"sgpu_pf_attn32", "sgpu_pf_attn64", "sgpu_pf_attn128"};
        for (int j = 0; j < 3; j++)
            if (hipModuleGetFunction(&d->dec_attn[j], d->mod[MOD_DECODE], attn[j]) != hipSuccess ||
                hipModuleGetFunction(&d->pf_attn[j], d->mod[MOD_DECODE], pattn[j]) != hipSuccess) {
                rc = SGPU_ERR_NO_KERNEL;
                goto fail;
            }
        if (hipModuleGetFunction(&d->dec_embed, d->mod[MOD_DECODE], "sgpu_dec_embed") != hipSuccess ||
            hipModuleGetFunction(&d->dec_argmax_part, d->mod[MOD_DECODE], "sgpu_dec_argmax_part") != hipSuccess ||
            hipModuleGetFunction(&d->dec_argmax_embed, d->mod[MOD_DECODE], "sgpu_dec_argmax_embed") != hipSuccess ||
            hipModuleGetFunction(&d->dec_argmax_g2embed, d->mod[MOD_DECODE], "sgpu_dec_argmax_g2embed") != hipSuccess ||
            hipModuleGetFunction(&d->dec_g2embed, d->mod[MOD_DECODE], "sgpu_dec_g2embed") != hipSuccess ||
            hipModuleGetFunction(&d->pf_embed, d->mod[MOD_DECODE], "sgpu_pf_embed") != hipSuccess ||
            hipModuleGetFunction(&d->pf_gemm, d->mod[MOD_DECODE], "sgpu_pf_gemm") != hipSuccess ||
            hipModuleGetFunction(&d->pf_qkv_post, d->mod[MOD_DECODE], "sgpu_pf_qkv_post") != hipSuccess ||
            hipModuleGetFunction(&d->pf_swiglu, d->mod[MOD_DECODE], "sgpu_pf_swiglu") != hipSuccess) {
            rc = SGPU_ERR_NO_KERNEL;
            goto fail;
        }
    }
    /* the null stream's split-K workspace, counters zeroed once (every launch leaves them at zero) */
    d->nsk = 1;
    d->sk[0].stream = NULL;
    e = hipMalloc((void **)&d->sk[0].ws, SK_WS_FLOATS * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void **)&d->sk[0].cnt, SK_MAX_TILES * sizeof(unsigned));
    if (e == hipSuccess) e = hipMemset(d->sk[0].cnt, 0, SK_MAX_TILES * sizeof(unsigned));
    if (e != hipSuccess) { rc = (int)e; goto fail; }
    /* the allocation-free entry point's fixed scratch: this device's copy resolved once */
    if ((rc = sgpu_internal_scratch_setup(dev)) != SGPU_OK) goto fail;
    __atomic_store_n(&d->ready, 1, __ATOMIC_RELEASE);
    goto out;
fail:
    unload_device(d);
out:
    pthread_mutex_unlock(&g_lock);
    return rc;
}

/* The split-K workspace of `stream` on device state d: the stream's own, made on its first
 * split launch outside graph capture and kept until sgpu_stream_destroy (streams made
 * elsewhere: until the process ends).  SGPU_ERR_NO_WORKSPACE
 * when the stream has none and cannot get one now (it is being recorded, or SK_STREAMS
 * streams already hold one). */
static int sk_workspace(devstate *d, void *stream, float **ws, unsigned **cnt) {
    int rc = SGPU_ERR_NO_WORKSPACE;
    /* hipStreamPerThread is one handle value naming a different stream in every host thread:
     * a workspace keyed by it would be shared by streams that run concurrently */
    if (stream == (void *)hipStreamPerThread) return rc;
    pthread_mutex_lock(&g_lock);
    for (int i = 0; i < d->nsk; i++)
        if (!d->sk[i].orphan && d->sk[i].stream == stream) {
            *ws = d->sk[i].ws;
            *cnt = d->sk[i].cnt;
            rc = SGPU_OK;
            goto out;
        }
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (d->nsk >= SK_STREAMS || hipStreamIsCapturing((hipStream_t)stream, &cs) != hipSuccess ||
        cs != hipStreamCaptureStatusNone)
        goto out;
    float *w = NULL;
    unsigned *c = NULL;
    if (hipMalloc((void **)&w, SK_WS_FLOATS * sizeof(float)) != hipSuccess ||
        hipMalloc((void **)&c, SK_MAX_TILES * sizeof(unsigned)) != hipSuccess ||
        hipMemset(c, 0, SK_MAX_TILES * sizeof(unsigned)) != hipSuccess) {
        hipFree(w);
        hipFree(c);
        goto out;
    }
    d->sk[d->nsk].stream = stream;
    d->sk[d->nsk].ws = *ws = w;
    d->sk[d->nsk].cnt = *cnt = c;
    d->sk[d->nsk].graphs = d->sk[d->nsk].orphan = 0;
    d->nsk++;
    rc = SGPU_OK;
out:
    pthread_mutex_unlock(&g_lock);
    return rc;
}

int sgpu_init(int device) {
    hipError_t e = hipInit(0);
    if (e != hipSuccess) return (int)e;
    int n = 0;
    e = hipGetDeviceCount(&n);
    if (e != hipSuccess) return (int)e;
    if (n <= 0) return SGPU_ERR_NO_DEVICE;
    if (device < 0 || device >= n || device >= SGPU_MAX_DEVICES) return SGPU_ERR_INVALID_ARG;
    HIPCHK(hipSetDevice(device));
    return load_device(device);
}

/* State of the current device, loading it on first use. */
static devstate *cur(int *rc) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) { *rc = (int)e; return NULL; }
    if (dev < 0 || dev >= SGPU_MAX_DEVICES) { *rc = SGPU_ERR_NO_DEVICE; return NULL; }
    if (!__atomic_load_n(&g_dev[dev].ready, __ATOMIC_ACQUIRE)) {
        *rc = load_device(dev);
        if (*rc) return NULL;
    }
    *rc = SGPU_OK;
    return &g_dev[dev];
}

int sgpu_device_count(int *count) {
    if (!count) return SGPU_ERR_INVALID_ARG;
    *count = 0;
    hipError_t e = hipGetDeviceCount(count);
    return e == hipSuccess ? SGPU_OK : (int)e;
}

int sgpu_get_device_props(int device, sgpu_device_props *props) {
    if (!props) return SGPU_ERR_INVALID_ARG;
    hipDeviceProp_t p;
    HIPCHK(hipGetDeviceProperties(&p, device));
    memset(props, 0, sizeof *props);
    snprintf(props->name, sizeof props->name, "%s", p.name);
    snprintf(props->arch, sizeof props->arch, "%.63s", p.gcnArchName);
    if (!props->name[0] && (hipDeviceGetName(props->name, (int)sizeof props->name, device) != hipSuccess ||
                            !props->name[0])) {
        /* no marketing name from the driver (an empty name table on some hosts): name the
         * device by its architecture and size instead of leaving the field empty */
        char arch[64];
        snprintf(arch, sizeof arch, "%s", props->arch);
        arch[strcspn(arch, ":")] = 0;
        snprintf(props->name, sizeof props->name, "AMD %s GPU, %d CUs", arch[0] ? arch : "(unknown arch)",
                 p.multiProcessorCount);
    }
    props->compute_units = p.multiProcessorCount;
    props->clock_khz = p.clockRate;
    props->memory_clock_khz = p.memoryClockRate;
    props->memory_bus_width = p.memoryBusWidth;
    props->total_mem = p.totalGlobalMem;
    props->lds_per_block = p.sharedMemPerBlock;
    props->l2_bytes = p.l2CacheSize;
    props->warp_size = p.warpSize;
    return SGPU_OK;
}

int sgpu_malloc(void **dptr, size_t bytes) {
    if (!dptr) return SGPU_ERR_INVALID_ARG;
    *dptr = NULL;
    if (bytes == 0) return SGPU_OK;
    HIPCHK(hipMalloc(dptr, bytes));
    return SGPU_OK;
}
int sgpu_free(void *dptr) {
    if (!dptr) return SGPU_OK;
    HIPCHK(hipFree(dptr));
    return SGPU_OK;
}
int sgpu_memcpy_htod(void *dst, const void *src, size_t bytes) {
    if (!bytes) return SGPU_OK;
    if (!dst || !src) return SGPU_ERR_INVALID_ARG;
    HIPCHK(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return SGPU_OK;
}
int sgpu_memcpy_dtoh(void *dst, const void *src, size_t bytes) {
    if (!bytes) return SGPU_OK;
    if (!dst || !src) return SGPU_ERR_INVALID_ARG;
    HIPCHK(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return SGPU_OK;
}
int sgpu_memcpy_dtod(void *dst, const void *src, size_t bytes) {
    if (!bytes) return SGPU_OK;
    if (!dst || !src) return SGPU_ERR_INVALID_ARG;
    HIPCHK(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice));
    return SGPU_OK;
}
int sgpu_memcpy_dtod_async(void *dst, const void *src, size_t bytes, void *stream) {
    if (!bytes) return SGPU_OK;
    if (!dst || !src) return SGPU_ERR_INVALID_ARG;
    HIPCHK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream));
    return SGPU_OK;
}
int sgpu_memset_d8(void *dst, int value, size_t bytes) {
    if (!bytes) return SGPU_OK;
    if (!dst) return SGPU_ERR_INVALID_ARG;
    HIPCHK(hipMemset(dst, value, bytes));
    return SGPU_OK;
}
int sgpu_synchronize(void) {
    HIPCHK(hipDeviceSynchronize());
    return SGPU_OK;
}
int sgpu_stream_synchronize(void *stream) {
    HIPCHK(hipStreamSynchronize((hipStream_t)stream));
    return SGPU_OK;
}

int sgpu_stream_create(void **stream) {
    if (!stream) return SGPU_ERR_INVALID_ARG;
    *stream = NULL;
    hipStream_t st;
    HIPCHK(hipStreamCreate(&st));               /* default priority */
    *stream = (void *)st;
    return SGPU_OK;
}
/* Recorded graphs that reference a split-K workspace (the one of the stream they were recorded
 * on), so that the workspace outlives its stream until the last such graph is destroyed. */
typedef struct {
    void *graph;
    int dev;
    float *ws;
} graph_ref;
static graph_ref *g_graph_refs;
static int g_ngraph_refs, g_cap_graph_refs;

/* Drop slot i of device dev's workspace table (g_lock held). */
static void sk_drop(devstate *d, int i) {
    hipFree(d->sk[i].ws);
    hipFree(d->sk[i].cnt);
    d->sk[i] = d->sk[--d->nsk];
}

/* Release the split-K workspaces of `stream` (its work finished): freed now, or, while recorded
 * graphs still reference them, kept (no longer found by the stream) until the last of those
 * graphs is destroyed. */
static void sk_release(void *stream) {
    pthread_mutex_lock(&g_lock);
    for (int dev = 0; dev < SGPU_MAX_DEVICES; dev++) {
        devstate *d = &g_dev[dev];
        if (!__atomic_load_n(&d->ready, __ATOMIC_RELAXED)) continue;
        for (int i = 1; i < d->nsk; i++)
            if (!d->sk[i].orphan && d->sk[i].stream == stream) {
                if (d->sk[i].graphs > 0) d->sk[i].orphan = 1;
                else sk_drop(d, i);
                break;
            }
    }
    pthread_mutex_unlock(&g_lock);
}

/* graph was recorded on stream: if the stream has a workspace, count the graph against it. */
static int sk_graph_recorded(void *graph, void *stream) {
    int rc = SGPU_OK;
    pthread_mutex_lock(&g_lock);
    for (int dev = 0; dev < SGPU_MAX_DEVICES && !rc; dev++) {
        devstate *d = &g_dev[dev];
        if (!__atomic_load_n(&d->ready, __ATOMIC_RELAXED)) continue;
        for (int i = 1; i < d->nsk; i++)
            if (!d->sk[i].orphan && d->sk[i].stream == stream) {
                if (g_ngraph_refs == g_cap_graph_refs) {
                    const int cap = g_cap_graph_refs ? 2 * g_cap_graph_refs : 16;
                    graph_ref *p = realloc(g_graph_refs, (size_t)cap * sizeof *p);
                    if (!p) { rc = SGPU_ERR_HOST_ALLOC; break; }
                    g_graph_refs = p;
                    g_cap_graph_refs = cap;
                }
                g_graph_refs[g_ngraph_refs++] = (graph_ref){graph, dev, d->sk[i].ws};
                d->sk[i].graphs++;
                break;
            }
    }
    pthread_mutex_unlock(&g_lock);
    return rc;
}

/* graph is being destroyed: uncount it, and free an orphaned workspace it held last (after the
 * device's work, which may include its replays, has finished). */
static void sk_graph_destroyed(void *graph) {
    pthread_mutex_lock(&g_lock);
    for (int r = 0; r < g_ngraph_refs; r++) {
        if (g_graph_refs[r].graph != graph) continue;
        devstate *d = &g_dev[g_graph_refs[r].dev];
        for (int i = 1; i < d->nsk; i++)
            if (d->sk[i].ws == g_graph_refs[r].ws) {
                if (--d->sk[i].graphs == 0 && d->sk[i].orphan) {
                    int cur = 0;
                    if (hipGetDevice(&cur) == hipSuccess && hipSetDevice(g_graph_refs[r].dev) == hipSuccess) {
                        hipDeviceSynchronize();
                        sk_drop(d, i);
                        hipSetDevice(cur);
                    }
                }
                break;
            }
        g_graph_refs[r] = g_graph_refs[--g_ngraph_refs];
        break;
    }
    pthread_mutex_unlock(&g_lock);
}

int sgpu_stream_destroy(void *stream) {
    if (!stream) return SGPU_OK;
    HIPCHK(hipStreamSynchronize((hipStream_t)stream));
    sk_release(stream);
    HIPCHK(hipStreamDestroy((hipStream_t)stream));
    return SGPU_OK;
}

/* Recorded launch sequences: stream capture in thread-local mode, instantiated at the end. */
int sgpu_graph_begin(void *stream) {
    if (!stream) return SGPU_ERR_INVALID_ARG;     /* the null stream cannot be captured */
    HIPCHK(hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal));
    return SGPU_OK;
}
int sgpu_graph_end(void *stream, void **graph) {
    if (!stream || !graph) return SGPU_ERR_INVALID_ARG;
    *graph = NULL;
    hipGraph_t g = NULL;
    HIPCHK(hipStreamEndCapture((hipStream_t)stream, &g));
    hipGraphExec_t ge = NULL;
    hipError_t e = hipGraphInstantiate(&ge, g, NULL, NULL, 0);
    hipGraphDestroy(g);
    if (e != hipSuccess) return (int)e;
    int rc = sk_graph_recorded((void *)ge, stream);
    if (rc) {
        hipGraphExecDestroy(ge);
        return rc;
    }
    *graph = (void *)ge;
    return SGPU_OK;
}
int sgpu_graph_launch(void *graph, void *stream) {
    if (!graph) return SGPU_ERR_INVALID_ARG;
    HIPCHK(hipGraphLaunch((hipGraphExec_t)graph, (hipStream_t)stream));
    return SGPU_OK;
}
int sgpu_graph_destroy(void *graph) {
    if (!graph) return SGPU_OK;
    hipError_t e = hipGraphExecDestroy((hipGraphExec_t)graph);
    sk_graph_destroyed(graph);
    return e == hipSuccess ? SGPU_OK : (int)e;
}

int sgpu_event_create(void **event) {
    if (!event) return SGPU_ERR_INVALID_ARG;
    hipEvent_t e;
    HIPCHK(hipEventCreate(&e));
    *event = (void *)e;
    return SGPU_OK;
}
int sgpu_event_destroy(void *event) {
    if (!event) return SGPU_OK;
    HIPCHK(hipEventDestroy((hipEvent_t)event));
    return SGPU_OK;
}
int sgpu_event_record(void *event, void *stream) {
    if (!event) return SGPU_ERR_INVALID_ARG;
    HIPCHK(hipEventRecord((hipEvent_t)event, (hipStream_t)stream));
    return SGPU_OK;
}
int sgpu_event_elapsed_ms(float *ms, void *start, void *stop) {
    if (!ms || !start || !stop) return SGPU_ERR_INVALID_ARG;
    HIPCHK(hipEventSynchronize((hipEvent_t)stop));
    HIPCHK(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
    return SGPU_OK;
}

const void *sgpu_code_object(const char *name, size_t *size) {
    if (size) *size = 0;
    if (!name) return NULL;
    for (int m = 0; m < NMOD; m++)
        if (!strcmp(name, g_cos[m].name)) {
            if (size) *size = (size_t)(g_cos[m].end - g_cos[m].start);
            return g_cos[m].start;
        }
    return NULL;
}

/* ---- geometry ---- */
static unsigned cdiv(long long a, long long b) { return (unsigned)((a + b - 1) / b); }
static unsigned umin(unsigned a, unsigned b) { return a < b ? a : b; }
/* sgemm_kwave_edge's blocks: the column past N/64 whole tiles (N % 64 == 1) rides on them. */
static long long kwave_edge_tiles(int M, int N) {
    return (long long)cdiv(M, 64) * (N % 64 == 1 ? (long long)(N / 64) : (long long)cdiv(N, 64));
}

/* Tile shape (rows x columns of C) of each tiled member; 0 for other kernels. */
static int sgemm_tile(const char *k, int *tn) {
    if (!strcmp(k, "sgemm_tiled")) return *tn = 64, 64;
    if (!strcmp(k, "sgemm_tiled4")) return *tn = 128, 128;
    if (!strcmp(k, "sgemm_opt")) return *tn = 256, 128;
    if (!strcmp(k, "sgemm_opt256")) return *tn = 256, 256;
    if (!strcmp(k, "sgemm_kwave") || !strcmp(k, "sgemm_kwave_wide")) return *tn = 64, 64;
    if (!strcmp(k, "sgemm_kwave128")) return *tn = 128, 128;
    return *tn = 0, 0;
}

static int geometry(const devstate *d, const char *kernel, int M, int N, int K, unsigned g[3], unsigned b[3]) {
    (void)K;
    const unsigned cus = d ? (unsigned)d->cus : 256u;
    g[0] = g[1] = g[2] = 1;
    b[0] = b[1] = b[2] = 1;
    if (!strcmp(kernel, "sgemm_kwave_edge") || !strcmp(kernel, "sgemm_kwave_edge_wide")) {
        long long nt = kwave_edge_tiles(M, N);
        g[0] = (unsigned)(nt > 0 ? nt : 1);
        b[0] = 256;
        return SGPU_OK;
    }
    int tile_n, tile = sgemm_tile(kernel, &tile_n);
    if (tile) {
        long long nt = (long long)cdiv(M, tile) * cdiv(N, tile_n);
        g[0] = (unsigned)(nt > 0 ? nt : 1);
        b[0] = 256;
        return SGPU_OK;
    }
    if (!strcmp(kernel, "sgemm_naive")) {
        g[0] = umin(cdiv(N > 0 ? N : 1, 16), 65535u);
        g[1] = umin(cdiv(M > 0 ? M : 1, 16), 65535u);
        b[0] = b[1] = 16;
        return SGPU_OK;
    }
    if (!strcmp(kernel, "membw_read4")) {
        g[0] = cus * 8;
        b[0] = 256;
        return SGPU_OK;
    }
    if (!strcmp(kernel, "gemv") || !strcmp(kernel, "gemv4") || !strcmp(kernel, "gemv_warp") ||
        !strcmp(kernel, "gemv_warp_b") || !strcmp(kernel, "gemv_h") || !strcmp(kernel, "gemv_hh")) {
        g[0] = umin(cdiv(N > 0 ? N : 1, 4), cus * 16);   /* a wave per row, 4 waves per block */
        b[0] = 256;
        return SGPU_OK;
    }
    if (!strcmp(kernel, "gemv_multi")) {   /* M carries T */
        /* One block per 32-token x 32-row tile on the matrix-core path; a wave per row (4 per
         * block, at most 16 blocks per CU) on the vector path.  The kernel takes the matrix
         * cores for T >= 4 (and T > 8 when K > 1024) on aligned rows (gemm_nt_ok). */
        if (M >= 4 && !(M <= 8 && K > 1024)) {
            long long nt = (long long)cdiv(M, 32) * cdiv(N > 0 ? N : 1, 32);
            g[0] = (unsigned)(nt < 0x7fffffffLL ? nt : 0x7fffffffLL);
        } else {
            g[0] = umin(cdiv(N > 0 ? N : 1, 4), cus * 16);
            g[1] = umin(cdiv(M > 0 ? M : 1, 16), 65535u);
        }
        b[0] = 256;
        return SGPU_OK;
    }
    return SGPU_ERR_NO_KERNEL;
}

int sgpu_kernel_geometry(const char *kernel, int M, int N, int K, unsigned grid[3], unsigned block[3]) {
    if (!kernel || !grid || !block || M < 0 || N < 0 || K < 0) return SGPU_ERR_INVALID_ARG;
    int dev = 0;
    const devstate *d = NULL;
    if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < SGPU_MAX_DEVICES &&
        __atomic_load_n(&g_dev[dev].ready, __ATOMIC_ACQUIRE))
        d = &g_dev[dev];
    return geometry(d, kernel, M, N, K, grid, block);
}

static int launch(hipFunction_t f, const unsigned g[3], const unsigned b[3], void *stream, void **args) {
    hipError_t e = hipModuleLaunchKernel(f, g[0], g[1], g[2], b[0], b[1], b[2], 0, (hipStream_t)stream, args, NULL);
    return (int)e;
}

/* ---- SGEMM ---- */
static int sgemm_common(int kid, const char *name, const float *A, const float *B, float *C, int M, int N,
                        int K, void *stream) {
    if (M < 0 || N < 0 || K < 0) return SGPU_ERR_INVALID_ARG;
    if (M == 0 || N == 0) return SGPU_OK;
    if (!C || (K > 0 && (!A || !B))) return SGPU_ERR_INVALID_ARG;
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    unsigned g[3], b[3];
    if ((rc = geometry(d, name, M, N, K, g, b))) return rc;
    void *args[] = {&A, &B, &C, &M, &N, &K};
    return launch(d->fn[kid], g, b, stream, args);
}
int sgpu_sgemm_tiled(const float *A, const float *B, float *C, int M, int N, int K, void *stream) {
    return sgemm_common(K_SGEMM_TILED, "sgemm_tiled", A, B, C, M, N, K, stream);
}
int sgpu_sgemm_tiled4(const float *A, const float *B, float *C, int M, int N, int K, void *stream) {
    return sgemm_common(K_SGEMM_TILED4, "sgemm_tiled4", A, B, C, M, N, K, stream);
}
int sgpu_sgemm_opt256(const float *A, const float *B, float *C, int M, int N, int K, void *stream) {
    return sgemm_common(K_SGEMM_OPT256, "sgemm_opt256", A, B, C, M, N, K, stream);
}
/* sgemm_kwave's problems: M, N multiples of 64, K a multiple of 32 (the operands' 16-byte
 * alignment is the launcher's check). */
static int kwave_shape(int M, int N, int K) { return M > 0 && N > 0 && K > 0 && M % 64 == 0 && N % 64 == 0 && K % 32 == 0; }
/* The K-over-waves members load their operands through 32-bit buffer offsets while a 64-row A
 * panel (64*K floats) and a 16-row B slice (16*N floats) stay under 2^31 bytes; larger operands
 * go to the LDS-staged forms with 64-bit addresses (the *_wide kernels). */
static int kwave_direct(int N, int K) { return (long long)K * 256 < (1LL << 31) && (long long)N * 64 < (1LL << 31); }
static int kwave_launch(int edge, const float *A, const float *B, float *C, int M, int N, int K, void *stream) {
    if (kwave_direct(N, K))
        return edge ? sgemm_common(K_SGEMM_KWAVE_EDGE, "sgemm_kwave_edge", A, B, C, M, N, K, stream)
                    : sgemm_common(K_SGEMM_KWAVE, "sgemm_kwave", A, B, C, M, N, K, stream);
    return edge ? sgemm_common(K_SGEMM_KWAVE_EDGE_WIDE, "sgemm_kwave_edge_wide", A, B, C, M, N, K, stream)
                : sgemm_common(K_SGEMM_KWAVE_WIDE, "sgemm_kwave_wide", A, B, C, M, N, K, stream);
}
int sgpu_sgemm_kwave(const float *A, const float *B, float *C, int M, int N, int K, void *stream) {
    if (M < 0 || N < 0 || K < 0) return SGPU_ERR_INVALID_ARG;
    if (M == 0 || N == 0) return SGPU_OK;
    if (!kwave_shape(M, N, K) || !A || !B || !C || (((uintptr_t)A | (uintptr_t)B) & 15)) return SGPU_ERR_INVALID_ARG;
    return kwave_launch(0, A, B, C, M, N, K, stream);
}
/* sgemm_kwave128's problems: M, N multiples of 128, K a multiple of 32, a 128-row A panel and a
 * 16-row B slice each under 2^31 bytes (32-bit buffer offsets; there is no wide form), and
 * 16-byte aligned A and B (the launcher's check). */
static int kwave128_shape(int M, int N, int K) {
    return M > 0 && N > 0 && K > 0 && M % 128 == 0 && N % 128 == 0 && K % 32 == 0 &&
           (long long)K * 512 < (1LL << 31) && (long long)N * 64 < (1LL << 31);
}
int sgpu_sgemm_kwave128(const float *A, const float *B, float *C, int M, int N, int K, void *stream) {
    if (M < 0 || N < 0 || K < 0) return SGPU_ERR_INVALID_ARG;
    if (M == 0 || N == 0) return SGPU_OK;
    if (!kwave128_shape(M, N, K) || !A || !B || !C || (((uintptr_t)A | (uintptr_t)B) & 15)) return SGPU_ERR_INVALID_ARG;
    return sgemm_common(K_SGEMM_KWAVE128, "sgemm_kwave128", A, B, C, M, N, K, stream);
}
/* sgemm_kwave_edge's problems: M, N at least 64 (a partial last row or column of tiles is the
 * 64 rows or columns ending at the last one), K at least 1, float-aligned operands. */
static int kwave_edge_shape(int M, int N, int K) { return M >= 64 && N >= 64 && K >= 1; }

int sgpu_sgemm_kwave_edge(const float *A, const float *B, float *C, int M, int N, int K, void *stream) {
    if (M < 0 || N < 0 || K < 0) return SGPU_ERR_INVALID_ARG;
    if (M == 0 || N == 0) return SGPU_OK;
    if (!kwave_edge_shape(M, N, K) || !A || !B || !C || (((uintptr_t)A | (uintptr_t)B | (uintptr_t)C) & 3))
        return SGPU_ERR_INVALID_ARG;
    return kwave_launch(1, A, B, C, M, N, K, stream);
}
/* The optimised entry picks the member with the least work on its busiest CU: tiles are one
 * block each, dealt over the CUs, so a launch lasts about ceil(tiles / CUs) tile times, and a
 * tile time is the tile's area over the member's sustained rate.  Rates are each member's
 * measured steady-state TFLOP/s at 4096^3 on MI355X (srand inputs): edge tiles and K tails
 * run at about the same rate as whole tiles. */
static const struct {
    int kid;
    const char *name;
    int bm, bn;
    double tflops;
} g_sgemm_members[] = {
    {K_SGEMM_OPT256, "sgemm_opt256", 256, 256, 145.8},
    {K_SGEMM_OPT, "sgemm_opt", 128, 256, 142.6},
    {K_SGEMM_TILED4, "sgemm_tiled4", 128, 128, 139.6},
    {K_SGEMM_TILED, "sgemm_tiled", 64, 64, 129.8},
};

static int sgemm_pick(int M, int N, int cus) {
    int best = 0;
    double best_t = 0.0;
    for (int m = 0; m < (int)(sizeof g_sgemm_members / sizeof g_sgemm_members[0]); m++) {
        const long long tiles = (long long)cdiv(M, g_sgemm_members[m].bm) * cdiv(N, g_sgemm_members[m].bn);
        const double t = (double)((tiles + cus - 1) / cus) * g_sgemm_members[m].bm * g_sgemm_members[m].bn /
                         g_sgemm_members[m].tflops;
        if (m == 0 || t < best_t) {
            best = m;
            best_t = t;
        }
    }
    return best;
}

/* sgemm_splitk: S k-splits of every 64x64 tile.  The count is reduced so that every split
 * holds at least one 32-deep slice (per = cdiv(nk, S) slices each, cdiv(nk, per) splits). */
static int sk_splits(int K, int S) {
    const int nk = cdiv(K, SK_BK);
    if (S > nk) S = nk;
    const int per = cdiv(nk, S);
    return cdiv(nk, per);
}
static int splitk_fits(int M, int N, int S) {
    const long long tiles = (long long)cdiv(M, SK_TILE) * cdiv(N, SK_TILE);
    return tiles <= SK_MAX_TILES && (unsigned long long)S * tiles * SK_TILE * SK_TILE <= SK_WS_FLOATS;
}
static int splitk_launch(devstate *d, const float *A, const float *B, float *C, int M, int N, int K, int S,
                         float *ws, unsigned *cnt, void *stream) {
    const long long tiles = (long long)cdiv(M, SK_TILE) * cdiv(N, SK_TILE);
    if (!splitk_fits(M, N, S)) return SGPU_ERR_INVALID_ARG;
    unsigned g[3] = {(unsigned)(tiles * S), 1, 1}, b[3] = {256, 1, 1};
    void *args[] = {&A, &B, &C, &M, &N, &K, &S, &ws, &cnt};
    return launch(d->fn[K_SGEMM_SPLITK], g, b, stream, args);
}
int sgpu_sgemm_splitk(const float *A, const float *B, float *C, int M, int N, int K, int S, void *stream) {
    if (M < 0 || N < 0 || K < 0 || S < 1) return SGPU_ERR_INVALID_ARG;
    if (M == 0 || N == 0) return SGPU_OK;
    S = K > 0 ? sk_splits(K, S) : 1;
    if (!splitk_fits(M, N, S)) return SGPU_ERR_INVALID_ARG;
    if (!C || (K > 0 && (!A || !B))) return SGPU_ERR_INVALID_ARG;
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    float *ws;
    unsigned *cnt;
    if ((rc = sk_workspace(d, stream, &ws, &cnt))) return rc;
    return splitk_launch(d, A, B, C, M, N, K, S, ws, cnt, stream);
}
/* sgpu_sgemm_splitk with the partials and counters in the library's fixed device scratch: no
 * allocation on any path (the device must be set up by sgpu_init first; the launch itself
 * allocates nothing), problems beyond the scratch rejected.  Calls that overlap on one device
 * share the scratch and race. */
int sgpu_sgemm_splitk_noalloc(const float *A, const float *B, float *C, int M, int N, int K, int S, void *stream) {
    if (M < 0 || N < 0 || K < 0 || S < 1) return SGPU_ERR_INVALID_ARG;
    if (M == 0 || N == 0) return SGPU_OK;
    S = K > 0 ? sk_splits(K, S) : 1;
    const long long tiles = (long long)cdiv(M, SK_TILE) * cdiv(N, SK_TILE);
    if (tiles > (long long)SGPU_SCRATCH_TILES ||
        (unsigned long long)S * tiles * SK_TILE * SK_TILE > (unsigned long long)SGPU_SCRATCH_FLOATS)
        return SGPU_ERR_SCRATCH_LIMIT;
    if (!C || (K > 0 && (!A || !B))) return SGPU_ERR_INVALID_ARG;
    int dev = 0;
    HIPCHK(hipGetDevice(&dev));
    if (dev < 0 || dev >= SGPU_MAX_DEVICES || !__atomic_load_n(&g_dev[dev].ready, __ATOMIC_ACQUIRE))
        return SGPU_ERR_NOT_INITIALIZED;                  /* set-up (which allocates) is sgpu_init's */
    float *ws;
    unsigned *cnt;
    int rc = sgpu_internal_scratch(dev, &ws, &cnt);
    if (rc) return rc;
    return splitk_launch(&g_dev[dev], A, B, C, M, N, K, S, ws, cnt, stream);
}

/* When sgpu_sgemm_opt splits K, and how many ways: the count (1 = unsplit, up to 8; 16 for
 * a problem of at most half the CUs' tiles whose splits still hold 512 of K each) with the
 * least modelled time, over problems of at most two rounds of 64x64 tiles.  Each CU runs
 * ceil(tiles * S / CUs) units of `per` = ceil(nk / S) 32-deep k-slices; the model charges,
 * in hundredths of a first-round slice:
 *   100 per slice of the first round,
 *    89 per slice of each further round (co-resident blocks overlap their latencies),
 *    36 per first-round slice on the masked pipeline (with a K tail: the unsplit tile's
 *       slices, or the last split's),
 *   220 per round of split hand-offs (partials written, the last split's sum).
 * Fitted to graph-replayed timings of sgemm_tiled and sgemm_splitk S = 2..8 at 26 shapes of
 * 100 to 512 tiles (640^2 to 2048x1024, K 997 to 4096): the pick's time is within 0.7% of
 * the fastest measured on average and 4.1% at worst (e.g. 1088x1024x1024 S = 4 29.5 us vs
 * 36.7 unsplit, 1200x1200x1024 S = 2 35.2 vs 42.6, 768x768x1000 S = 5 18.8 vs 27.6,
 * 2048x1024x1000 unsplit 41.2 vs 47.5 at S = 4).  Every split keeps at least two slices.
 * Returns 1 for no split. */
static int splitk_pick(int M, int N, int K, int cus) {
    const long long tiles = (long long)cdiv(M, SK_TILE) * cdiv(N, SK_TILE);
    const int nk = cdiv(K, SK_BK);
    if (cus < 1 || tiles > 2LL * cus) return 1;
    const int cap = tiles * 2 <= cus && K / 16 >= 512 ? 16 : 8;
    const int tail = K % SK_BK != 0;
    int best_s = 1;
    long long best = 0;
    for (int s = 1; s <= cap && s <= nk / 2; s++) {
        const int S = sk_splits(K, s), per = cdiv(nk, S);
        if (S != s || (S > 1 && !splitk_fits(M, N, S))) continue;   /* same split as a smaller s */
        const long long rounds = (tiles * S + cus - 1) / cus;
        const long long c = 100LL * per + 89LL * per * (rounds - 1) + (tail ? 36LL * per : 0) +
                            (S > 1 ? 220LL * rounds : 0);
        if (s == 1 || c < best) {
            best = c;
            best_s = S;
        }
    }
    return best_s;
}

/* sgemm_small16 / sgemm_small32: one 16x16 / 32x32 tile of C per block, operands read through
 * buffer resources with 32-bit offsets, which must not wrap: a wave's last batch of k-groups
 * reads up to 4 * 4 groups (4 * 4 * 16 = 256 rows of B, 256 floats of an A row) past K, and
 * rows past M up to the tile edge (32 rows of A); those reads land past the buffers' ends
 * and return zero only while every offset stays below 2^31. */
static int small_fits(int M, int N, int K) {
    return (long long)(M + 32) * K * 4 + (K + 272) * 4LL < (1LL << 31) &&
           (long long)(K + 256) * N * 4 + 256 < (1LL << 31);
}
static int small_launch(devstate *d, int ts, const float *A, const float *B, float *C, int M, int N, int K,
                        void *stream) {
    const long long tiles = (long long)cdiv(M, ts) * cdiv(N, ts);
    unsigned g[3] = {(unsigned)(tiles < (long long)d->cus * 16 ? tiles : (long long)d->cus * 16), 1, 1};
    unsigned b[3] = {256, 1, 1};
    void *args[] = {&A, &B, &C, &M, &N, &K};
    return launch(d->fn[ts == 16 ? K_SGEMM_SMALL16 : K_SGEMM_SMALL32], g, b, stream, args);
}
int sgpu_sgemm_small(const float *A, const float *B, float *C, int M, int N, int K, int tile, void *stream) {
    if (M < 0 || N < 0 || K < 0 || (tile != 16 && tile != 32)) return SGPU_ERR_INVALID_ARG;
    if (M == 0 || N == 0) return SGPU_OK;
    if (!small_fits(M, N, K) || !C || (K > 0 && (!A || !B))) return SGPU_ERR_INVALID_ARG;
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    return small_launch(d, tile, A, B, C, M, N, K, stream);
}

/* The launch sgpu_sgemm_opt makes for an M x N x K problem on `cus` CUs: PLAN_SMALL16 /
 * PLAN_SMALL32, PLAN_SPLITK with *S splits (the unsplit member is launched instead when the
 * stream has no workspace), or an index into g_sgemm_members. */
enum { PLAN_SMALL16 = -1, PLAN_SMALL32 = -2, PLAN_SPLITK = -3, PLAN_KWAVE = -4, PLAN_KWAVE_EDGE = -5, PLAN_KWAVE128 = -6 };
static int opt_plan(int M, int N, int K, int cus, int *S) {
    *S = 1;
    /* Problems whose 16x16 (32x32) tiles fit the CUs in one round go to the small members
     * (measured in recorded graphs, srand inputs: 256^3 4.0 vs 7.7 us, 512^3 7.6 vs 9.7,
     * 256x256x2048 9.4 vs 13.7, 100x70x3000 11.3 vs 16.0, 1x4096x4096 23.6 vs 27.8); past
     * K 2048 a full round of 16x16 blocks' serial k-chains outlasts the split-K member
     * (256x256x4096 22.0 vs 18.2) unless the tiles are few or the problem is one row or
     * column of tiles, and past K 4096 (1024 for 32x32) it always does. */
    if (small_fits(M, N, K)) {
        const long long t16 = (long long)cdiv(M, 16) * cdiv(N, 16), t32 = (long long)cdiv(M, 32) * cdiv(N, 32);
        if (t16 <= cus && K <= 4096 && (K <= 2048 || t16 * 4 <= cus || M <= 16 || N <= 16)) return PLAN_SMALL16;
        if (t32 <= cus && K <= 1024) return PLAN_SMALL32;
    }
    /* One round of 64x64 tiles filling 3/4 to all of the CUs, K of 256 or more: the 64x64 tile
     * with K split over its four waves and the operands loaded straight into the matrix-core
     * registers, on whole tiles (sgemm_kwave: M, N multiples of 64, K of 32) or with clamped
     * edge tiles and a zero-padded first k-slice (sgemm_kwave_edge).  Recorded graphs, random
     * inputs in [-1, 1), us, against the 64x64 member: 1024^3 18.1 vs 20.5; 1024x1024x512
     * 10.9 vs 11.9; 1024x1024x256 7.4 vs 7.7; 1023x1025x997 20.2 vs 40.3 (S = 4 split: 31.1);
     * 1000^3 19.4 vs 27.3; 1000x1000x256 8.5 vs 9.1.  With fewer tiles the K splits across
     * blocks win (512x1024x1024 15.3 at S = 2 vs 17.7; 768x768x2048 31.0 at S = 8 vs 32.6). */
    if (M >= 64 && N >= 64 && K >= 256) {
        const int exact = kwave_shape(M, N, K);
        const long long tiles = exact ? (long long)(M / 64) * (N / 64) : kwave_edge_tiles(M, N);
        if (tiles <= cus && 4 * tiles >= 3LL * cus) return exact ? PLAN_KWAVE : PLAN_KWAVE_EDGE;
    }
    /* K from 128 to 255 on edge tiles that fill 3/4 to all of the CUs in one round while the
     * 64x64 member would need a second (N % 64 == 1 rides on the last column of whole tiles):
     * 1023x1025x128 7.0 vs 7.0, against 5.6 vs 6.0 for the 64x64 member at K 64. */
    if (kwave_edge_shape(M, N, K) && K >= 128) {
        const long long tiles = kwave_edge_tiles(M, N), tiles64 = (long long)cdiv(M, 64) * cdiv(N, 64);
        if (tiles <= cus && 4 * tiles >= 3LL * cus && tiles64 > cus) return PLAN_KWAVE_EDGE;
    }
    if (K > 0 && (*S = splitk_pick(M, N, K, cus)) > 1) return PLAN_SPLITK;
    *S = 1;
    /* Where the busiest-CU model picks the 64x64 member over several rounds, the K-over-waves
     * members run the same tiles faster (random inputs, us: 3072^3 422 vs 452; 2048x1024x1024
     * 33.8 vs 37.2; 4097^3 1107 vs 1222; 2047x2049x2047 140 vs 179).  The larger tiles keep
     * their shapes: they move half the bytes per flop or less, and with random operands the
     * 64x64 tiles' extra traffic costs clock (4096^3 945 us on sgemm_opt256 vs 989; 2048^3 127
     * on sgemm_tiled4 vs 130; 8192x1024x1024 131 vs 133). */
    const int pick = sgemm_pick(M, N, cus);
    /* The 128x128 K-over-waves member where its tiles fill whole rounds of the CUs (the last
     * round at least 94% full) and K is deep enough to carry its per-round cost (about 6.6 us:
     * the first slices' latency, the partial-tile sum through LDS, the C store): K >= 512
     * against the 128x128 and 128x256 members, K >= 4096 against sgemm_opt256, which needs
     * fewer rounds.  Recorded graphs, random inputs in [-1, 1), us, against the pick before it:
     * 2048^3 121.7 vs 127.7 (sgemm_tiled4); 2048x2048x512 36.5 vs 37.3; 6144^3 3156 vs 3326;
     * 2048x4096x2048 242.3 vs 252.7 (sgemm_opt); 2816^3 327 vs 345; 4096^3 935 vs 947
     * (sgemm_opt256); 8192^3 7465 vs 7526; 4096x4096x8192 1836 vs 1893.  Where it loses:
     * 4096x4096x2048 482 vs 478, 2048x8192x1024 255 vs 246 (both sgemm_opt256), 2048x2048x256
     * 22.3 vs 22.1, and every shape with a partly empty last round (5120^3 2036 vs 1980 at 89%
     * full, 3072^3 525 vs 437 at 75%). */
    if (kwave128_shape(M, N, K)) {
        const long long t128 = (long long)(M / 128) * (N / 128), r128 = (t128 + cus - 1) / cus;
        const int deep = g_sgemm_members[pick].kid == K_SGEMM_OPT256 ? K >= 4096 : K >= 512;
        if (50 * t128 >= 47 * r128 * cus && deep) return PLAN_KWAVE128;
    }
    if (g_sgemm_members[pick].kid == K_SGEMM_TILED && M >= 64 && N >= 64 && K >= 256)
        return kwave_shape(M, N, K) ? PLAN_KWAVE : PLAN_KWAVE_EDGE;
    return pick;
}
const char *sgpu_sgemm_opt_plan(int M, int N, int K, int cus, int *splits) {
    if (M < 1 || N < 1 || K < 0 || cus < 1) return NULL;
    int S;
    const int p = opt_plan(M, N, K, cus, &S);
    if (splits) *splits = S;
    if (p == PLAN_SMALL16) return "sgemm_small16";
    if (p == PLAN_SMALL32) return "sgemm_small32";
    if (p == PLAN_SPLITK) return "sgemm_splitk";
    if (p == PLAN_KWAVE) return "sgemm_kwave";
    if (p == PLAN_KWAVE_EDGE) return "sgemm_kwave_edge";
    if (p == PLAN_KWAVE128) return "sgemm_kwave128";
    return g_sgemm_members[p].name;
}

int sgpu_sgemm_opt(const float *A, const float *B, float *C, int M, int N, int K, void *stream) {
    if (M < 0 || N < 0 || K < 0) return SGPU_ERR_INVALID_ARG;
    if (M == 0 || N == 0) return SGPU_OK;
    if (!C || (K > 0 && (!A || !B))) return SGPU_ERR_INVALID_ARG;
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    int S;
    const int p = opt_plan(M, N, K, d->cus, &S);
    if (p == PLAN_SMALL16 || p == PLAN_SMALL32) return small_launch(d, p == PLAN_SMALL16 ? 16 : 32, A, B, C, M, N, K, stream);
    float *ws;
    unsigned *cnt;
    if (p == PLAN_SPLITK && sk_workspace(d, stream, &ws, &cnt) == SGPU_OK)    /* else: the unsplit member */
        return splitk_launch(d, A, B, C, M, N, K, S, ws, cnt, stream);
    if (p == PLAN_KWAVE128 && !(((uintptr_t)A | (uintptr_t)B) & 15))
        return sgemm_common(K_SGEMM_KWAVE128, "sgemm_kwave128", A, B, C, M, N, K, stream);
    if (p == PLAN_KWAVE && !(((uintptr_t)A | (uintptr_t)B) & 15)) return kwave_launch(0, A, B, C, M, N, K, stream);
    if ((p == PLAN_KWAVE || p == PLAN_KWAVE_EDGE) && !(((uintptr_t)A | (uintptr_t)B | (uintptr_t)C) & 3))
        return kwave_launch(1, A, B, C, M, N, K, stream);   /* rows of any float alignment */
    const int m = p >= 0 ? p : sgemm_pick(M, N, d->cus);
    return sgemm_common(g_sgemm_members[m].kid, g_sgemm_members[m].name, A, B, C, M, N, K, stream);
}
int sgpu_sgemm_naive(const float *A, const float *B, float *C, int M, int N, int K, void *stream) {
    return sgemm_common(K_SGEMM_NAIVE, "sgemm_naive", A, B, C, M, N, K, stream);
}

int sgpu_membw_read4(const void *buf, float *out, int n4, int iters, int *threads, void *stream) {
    if (n4 < 0 || iters < 0) return SGPU_ERR_INVALID_ARG;
    if (n4 > 0 && (!buf || !out || ((uintptr_t)buf & 15))) return SGPU_ERR_INVALID_ARG;
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    unsigned g[3], b[3];
    geometry(d, "membw_read4", 0, 0, 0, g, b);
    if (threads) *threads = (int)(g[0] * b[0]);
    if (n4 == 0) return SGPU_OK;
    void *args[] = {&buf, &out, &n4, &iters};
    return launch(d->fn[K_MEMBW], g, b, stream, args);
}

/* ---- GEMV ---- */
/* Pick the tuned instantiation for a K x N GEMV (VEC elements per 16 bytes), or -1/-1 for
 * the generic kernel.  Smallest team that still gives >= 8 waves per CU, else the largest
 * that fits in 16 segments per lane. */
static void pick_tuned(const devstate *d, int K, int N, int vec, int *li, int *si) {
    *li = *si = -1;
    if (K <= 0 || N <= 0 || K % vec) return;
    const long long nseg = K / vec;
    const long long want_waves = 8LL * d->cus;
    int best_l = -1;
    for (int i = 0; i < NLPR; i++) {
        long long s = (nseg + g_lpr[i] - 1) / g_lpr[i];
        if (s > g_segs[NSEG - 1]) continue;
        best_l = i;
        if ((long long)N * g_lpr[i] / 64 >= want_waves) break;
    }
    if (best_l < 0) return;
    long long s = (nseg + g_lpr[best_l] - 1) / g_lpr[best_l];
    for (int j = 0; j < NSEG; j++)
        if (g_segs[j] >= s) { *li = best_l; *si = j; return; }
}

/* Weight / x storage of a GEMV launch: fp32 W and x, fp16 W with fp32 x (gemv_h), or fp16 W
 * with fp16 x (gemv_hh). */
enum { GV_F32, GV_H, GV_HH };

/* Grid cap of the persistent tuned GEMVs (blocks per CU), reached only by lm_head-sized row
 * counts.  Measured on the lm_head shapes with rotating weight copies: fp16 [151936 x 896]
 * peaks at 18 blocks per CU (86.2% of HBM; 84.0% at 8), fp32 [50257 x 768] at 4 (81.5%;
 * 80.3% at 8) -- its lanes keep 1.7x more bytes in flight. */
static unsigned gemv_blocks_per_cu(int kind) { return kind != GV_F32 ? 18u : 4u; }

static int gemv_launch(int generic_kid, int kind, const void *W, const void *x, const float *bias, float *y,
                       int K, int N, void *stream) {
    if (K < 0 || N < 0) return SGPU_ERR_INVALID_ARG;
    if (N == 0) return SGPU_OK;
    if (!y || (K > 0 && (!W || !x))) return SGPU_ERR_INVALID_ARG;
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    void *args[] = {(void *)&W, (void *)&x, (void *)&bias, (void *)&y, &K, &N};
    const int vec = kind == GV_F32 ? 4 : 8;
    int li, si;
    pick_tuned(d, K, N, vec, &li, &si);
    const int aligned = ((((uintptr_t)W) | ((uintptr_t)x)) & 15) == 0;
    if (li >= 0 && aligned) {
        const int teams = 256 / g_lpr[li];
        unsigned g[3] = {umin(cdiv(N, teams), (unsigned)d->cus * gemv_blocks_per_cu(kind)), 1, 1}, b[3] = {256, 1, 1};
        hipFunction_t f = kind == GV_F32 ? d->gemv_f32[li][si] : kind == GV_H ? d->gemv_h[li][si] : d->gemv_hh[li][si];
        return launch(f, g, b, stream, args);
    }
    unsigned g[3], b[3];
    geometry(d, "gemv_h", 0, N, K, g, b);
    if (generic_kid == K_GEMV || generic_kid == K_GEMV4 || generic_kid == K_GEMV_WARP) {
        void *args5[] = {(void *)&W, (void *)&x, (void *)&y, &K, &N};   /* no bias slot */
        return launch(d->fn[generic_kid], g, b, stream, args5);
    }
    return launch(d->fn[generic_kid], g, b, stream, args);
}

int sgpu_gemv(const float *W, const float *x, float *y, int K, int N, void *stream) {
    return gemv_launch(K_GEMV, GV_F32, W, x, NULL, y, K, N, stream);
}
int sgpu_gemv4(const float *W, const float *x, float *y, int K, int N, void *stream) {
    return gemv_launch(K_GEMV4, GV_F32, W, x, NULL, y, K, N, stream);
}
int sgpu_gemv_warp(const float *W, const float *x, float *y, int K, int N, void *stream) {
    return gemv_launch(K_GEMV_WARP, GV_F32, W, x, NULL, y, K, N, stream);
}
int sgpu_gemv_warp_b(const float *W, const float *x, const float *bias, float *y, int K, int N, void *stream) {
    return gemv_launch(K_GEMV_WARP_B, GV_F32, W, x, bias, y, K, N, stream);
}
int sgpu_gemv_h(const uint16_t *W, const float *x, const float *bias, float *y, int K, int N, void *stream) {
    return gemv_launch(K_GEMV_H, GV_H, W, x, bias, y, K, N, stream);
}
int sgpu_gemv_hh(const uint16_t *W, const uint16_t *x, const float *bias, float *y, int K, int N, void *stream) {
    return gemv_launch(K_GEMV_HH, GV_HH, W, x, bias, y, K, N, stream);
}

/* K splits for the batched matrix-core GEMM (32-token x 32-row tiles): with fewer tiles than
 * CUs, about two units per CU, each split keeping at least four 32-deep chunks (one per
 * wave), at most 16 splits, within SGPU_NT_WS_FLOATS of partials.  1 = no split. */
static int nt_splits(int T, int N, int K, int cus) {
    const long long tiles = (long long)cdiv(T, 32) * cdiv(N, 32);
    const int nch = cdiv(K, 32);
    if (tiles >= cus || tiles > (long long)SGPU_NT_CNT) return 1;
    long long S = 2LL * cus / tiles;
    if (S > nch / 4) S = nch / 4;
    if (S > 16) S = 16;
    while (S > 1 && S * tiles * 1024 > (long long)SGPU_NT_WS_FLOATS) S--;
    return S < 1 ? 1 : (int)S;
}

/* The batched GEMV's kernel choice: up to 8 tokens on aligned rows of at most 4096 take the
 * register-resident team GEMV; otherwise the matrix-core tile, with K split over S blocks when
 * there are too few 32x32 tiles to fill the CUs (whole aligned quads and at least 4 tokens).
 * *S is the split the tile path would take given a workspace (1: none). */
static int gemv_multi_x8(const float *W, const float *X, int K, int T) {
    const int aligned = K > 0 && K % 4 == 0 && !(((uintptr_t)W | (uintptr_t)X) & 15);
    return aligned && T <= 8 && K <= 4096;
}
static int gemv_multi_splits(const devstate *d, const float *W, const float *X, int K, int N, int T) {
    const int aligned = K > 0 && K % 4 == 0 && !(((uintptr_t)W | (uintptr_t)X) & 15);
    if (gemv_multi_x8(W, X, K, T) || !aligned || T < 4) return 1;
    return nt_splits(T, N, K, d->cus);
}

int sgpu_internal_gemv_multi(const float *W, const float *X, const float *bias, float *Y, int K, int N, int T,
                             float *ws, unsigned *cnt, void *stream) {
    if (K < 0 || N < 0 || T < 0) return SGPU_ERR_INVALID_ARG;
    if (N == 0 || T == 0) return SGPU_OK;
    if (!Y || (K > 0 && (!W || !X))) return SGPU_ERR_INVALID_ARG;
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    /* Up to 8 tokens on aligned rows of at most 4096: the register-resident team GEMV with
     * eight input vectors (a wave per row up to K = 1024, a block per row beyond; one block
     * per 4 or 1 rows, capped at the 2 or 3 blocks per CU their registers allow). */
    if (gemv_multi_x8(W, X, K, T)) {
        const int wide = K > 1024;
        const unsigned teams = wide ? 1u : 4u, cap = (unsigned)d->cus * (wide ? 3u : 2u);
        unsigned g[3] = {umin(cdiv(N, (int)teams), cap), 1, 1}, b[3] = {256, 1, 1};
        void *args[] = {(void *)&W, (void *)&X, (void *)&bias, (void *)&Y, &K, &N, &T};
        return launch(d->fn[wide ? K_GEMV_MULTI_X8_256 : K_GEMV_MULTI_X8_64], g, b, stream, args);
    }
    /* Too few 32x32 tiles to fill the CUs: split each tile's K over blocks (matrix-core path
     * conditions: whole aligned quads and at least 4 tokens). */
    const int S = (ws && cnt) ? gemv_multi_splits(d, W, X, K, N, T) : 1;
    if (S > 1) {
        const long long tiles = (long long)cdiv(T, 32) * cdiv(N, 32);
        unsigned g[3] = {(unsigned)(tiles * S), 1, 1}, b[3] = {256, 1, 1};
        void *args[] = {(void *)&W, (void *)&X, (void *)&bias, (void *)&Y, &K, &N, &T, (void *)&S, &ws, &cnt};
        return launch(d->fn[K_GEMV_MULTI_SPLITK], g, b, stream, args);
    }
    unsigned g[3], b[3];
    geometry(d, "gemv_multi", T, N, K, g, b);
    void *args[] = {(void *)&W, (void *)&X, (void *)&bias, (void *)&Y, &K, &N, &T};
    return launch(d->fn[K_GEMV_MULTI], g, b, stream, args);
}

int sgpu_gemv_multi(const float *W, const float *X, const float *bias, float *Y, int K, int N, int T,
                    void *stream) {
    int rc;
    devstate *d = (N > 0 && T > 0 && K >= 0) ? cur(&rc) : NULL;
    float *ws = NULL;
    unsigned *cnt = NULL;
    /* a workspace only for a launch that splits (unsplit kernels without one) */
    if (d && (!Y || K == 0 || (W && X)) && gemv_multi_splits(d, W, X, K, N, T) > 1 &&
        sk_workspace(d, stream, &ws, &cnt) != SGPU_OK)
        ws = NULL, cnt = NULL;
    return sgpu_internal_gemv_multi(W, X, bias, Y, K, N, T, ws, cnt, stream);
}

int sgpu_internal_stage_out(void *stream, sgpu_stage_sink *k, const char *tag, const float *dev, int n) {
    if (n > k->cap) n = k->cap;
    hipError_t he = hipMemcpyAsync(k->host, dev, (size_t)n * 4, hipMemcpyDeviceToHost, (hipStream_t)stream);
    if (he == hipSuccess) he = hipStreamSynchronize((hipStream_t)stream);
    if (he != hipSuccess) return (int)he;
    k->fn(k->ctx, tag, k->host, n);
    return SGPU_OK;
}

/* ---- Qwen support kernels ---- */
static int elem_grid(int n) { return (int)umin(cdiv(n > 0 ? n : 1, 256), 65535u); }

int sgpu_rmsnorm(const float *x, const uint16_t *w, float *y, int n, float eps, int rows, void *stream) {
    if (n < 0 || rows < 0) return SGPU_ERR_INVALID_ARG;
    if (n == 0 || rows == 0) return SGPU_OK;
    if (!x || !w || !y || rows > 65535 * 1024) return SGPU_ERR_INVALID_ARG;
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    unsigned g[3] = {(unsigned)rows, 1, 1}, b[3] = {256, 1, 1};
    void *args[] = {(void *)&x, (void *)&w, (void *)&y, &n, &eps};
    return launch(d->fn[K_RMSNORM], g, b, stream, args);
}

int sgpu_rope(float *x, const float *cosT, const float *sinT, int T, int H, int HD, int pos0, void *stream) {
    if (T < 0 || H < 0 || HD < 0 || HD % 2 || pos0 < 0) return SGPU_ERR_INVALID_ARG;
    long long total = (long long)T * H * (HD / 2);
    if (total == 0) return SGPU_OK;
    if (!x || !cosT || !sinT || total > 0x7fffffffLL) return SGPU_ERR_INVALID_ARG;
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    unsigned g[3] = {(unsigned)elem_grid((int)total), 1, 1}, b[3] = {256, 1, 1};
    void *args[] = {(void *)&x, (void *)&cosT, (void *)&sinT, &T, &H, &HD, &pos0};
    return launch(d->fn[K_ROPE], g, b, stream, args);
}

int sgpu_swiglu(const float *gt, const float *u, float *y, int n, void *stream) {
    if (n < 0) return SGPU_ERR_INVALID_ARG;
    if (n == 0) return SGPU_OK;
    if (!gt || !u || !y) return SGPU_ERR_INVALID_ARG;
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    unsigned g[3] = {(unsigned)elem_grid(n), 1, 1}, b[3] = {256, 1, 1};
    void *args[] = {(void *)&gt, (void *)&u, (void *)&y, &n};
    return launch(d->fn[K_SWIGLU], g, b, stream, args);
}

static int gqa_ok(int NH, int KV, int HD) {
    return NH > 0 && HD > 0 && KV > 0 && KV % HD == 0 && NH % (KV / HD) == 0;
}

int sgpu_attn_scores_gqa(const float *q, const float *kc, float *scores, int T, float scale, int NH, int KV,
                         int HD, void *stream) {
    if (T < 0 || !gqa_ok(NH, KV, HD)) return SGPU_ERR_INVALID_ARG;
    if (T == 0) return SGPU_OK;
    if (!q || !kc || !scores || (long long)T * NH > 0x7fffffffLL) return SGPU_ERR_INVALID_ARG;
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    unsigned g[3] = {(unsigned)elem_grid(T * NH), 1, 1}, b[3] = {256, 1, 1};
    void *args[] = {(void *)&q, (void *)&kc, (void *)&scores, &T, &scale, &NH, &KV, &HD};
    return launch(d->fn[K_ASCORES], g, b, stream, args);
}

int sgpu_attn_softmax(const float *scores, float *probs, int T, int NH, void *stream) {
    if (T < 0 || NH < 0) return SGPU_ERR_INVALID_ARG;
    if (T == 0 || NH == 0) return SGPU_OK;
    if (!scores || !probs) return SGPU_ERR_INVALID_ARG;
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    unsigned g[3] = {umin(cdiv(NH, 4), 65535u), 1, 1}, b[3] = {256, 1, 1};   /* a wave per head */
    void *args[] = {(void *)&scores, (void *)&probs, &T, &NH};
    return launch(d->fn[K_ASOFTMAX], g, b, stream, args);
}

int sgpu_attn_mix_gqa(const float *probs, const float *vc, float *out, int T, int NH, int KV, int HD,
                      void *stream) {
    if (T < 0 || !gqa_ok(NH, KV, HD)) return SGPU_ERR_INVALID_ARG;
    if (!probs || !vc || !out) return SGPU_ERR_INVALID_ARG;
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    unsigned g[3] = {(unsigned)elem_grid(NH * HD), 1, 1}, b[3] = {256, 1, 1};
    void *args[] = {(void *)&probs, (void *)&vc, (void *)&out, &T, &NH, &KV, &HD};
    return launch(d->fn[K_AMIX], g, b, stream, args);
}

int sgpu_add2(const float *a, const float *bb, float *out, int n, void *stream) {
    if (n < 0) return SGPU_ERR_INVALID_ARG;
    if (n == 0) return SGPU_OK;
    if (!a || !bb || !out) return SGPU_ERR_INVALID_ARG;
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    unsigned g[3] = {(unsigned)elem_grid(n), 1, 1}, b[3] = {256, 1, 1};
    void *args[] = {(void *)&a, (void *)&bb, (void *)&out, &n};
    return launch(d->fn[K_ADD2], g, b, stream, args);
}

/* ---- GPT-2 support kernels (fixed 12 x 64 head layout) ---- */
int sgpu_layernorm(const float *x, const float *w, const float *bb, float *y, int n, float eps, int rows,
                   void *stream) {
    if (n < 0 || rows < 0) return SGPU_ERR_INVALID_ARG;
    if (n == 0 || rows == 0) return SGPU_OK;
    if (!x || !w || !bb || !y || rows > 0x7fffffff / 1) return SGPU_ERR_INVALID_ARG;
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    unsigned g[3] = {(unsigned)rows, 1, 1}, b[3] = {256, 1, 1};
    void *args[] = {(void *)&x, (void *)&w, (void *)&bb, (void *)&y, &n, &eps};
    return launch(d->fn[K_LAYERNORM], g, b, stream, args);
}

int sgpu_gelu(const float *x, float *y, int n, void *stream) {
    if (n < 0) return SGPU_ERR_INVALID_ARG;
    if (n == 0) return SGPU_OK;
    if (!x || !y) return SGPU_ERR_INVALID_ARG;
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    unsigned g[3] = {(unsigned)elem_grid(n), 1, 1}, b[3] = {256, 1, 1};
    void *args[] = {(void *)&x, (void *)&y, &n};
    return launch(d->fn[K_GELU], g, b, stream, args);
}

int sgpu_add_bias(float *y, const float *bias, int n, void *stream) {
    if (n < 0) return SGPU_ERR_INVALID_ARG;
    if (n == 0) return SGPU_OK;
    if (!y || !bias) return SGPU_ERR_INVALID_ARG;
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    unsigned g[3] = {(unsigned)elem_grid(n), 1, 1}, b[3] = {256, 1, 1};
    void *args[] = {(void *)&y, (void *)&bias, &n};
    return launch(d->fn[K_ADD_BIAS], g, b, stream, args);
}

int sgpu_gpt2_attn_scores(const float *q, const float *kcache, float *scores, int T, float scale, void *stream) {
    if (T < 0) return SGPU_ERR_INVALID_ARG;
    if (T == 0) return SGPU_OK;
    if (!q || !kcache || !scores || T > 0x7fffffff / 12) return SGPU_ERR_INVALID_ARG;
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    unsigned g[3] = {(unsigned)elem_grid(T * 12), 1, 1}, b[3] = {256, 1, 1};
    void *args[] = {(void *)&q, (void *)&kcache, (void *)&scores, &T, &scale};
    return launch(d->fn[K_G2_SCORES], g, b, stream, args);
}

int sgpu_gpt2_attn_softmax(const float *scores, float *probs, int T, void *stream) {
    if (T < 0) return SGPU_ERR_INVALID_ARG;
    if (T == 0) return SGPU_OK;
    if (!scores || !probs) return SGPU_ERR_INVALID_ARG;
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    unsigned g[3] = {3, 1, 1}, b[3] = {256, 1, 1};     /* 12 waves: one per head */
    void *args[] = {(void *)&scores, (void *)&probs, &T};
    return launch(d->fn[K_G2_SOFTMAX], g, b, stream, args);
}

int sgpu_gpt2_attn_mix(const float *probs, const float *vcache, float *out, int T, void *stream) {
    if (T < 0 || !probs || !vcache || !out) return SGPU_ERR_INVALID_ARG;
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    unsigned g[3] = {3, 1, 1}, b[3] = {256, 1, 1};     /* 768 outputs */
    void *args[] = {(void *)&probs, (void *)&vcache, (void *)&out, &T};
    return launch(d->fn[K_G2_MIX], g, b, stream, args);
}

/* ---- seeded generators ---- */
void sgpu_gen_sgemm_inputs(float *A, float *B, size_t count, unsigned seed) {
    srand(seed);
    for (size_t i = 0; i < count; i++) {
        A[i] = (rand() % 2000 - 1000) / 1000.0f;
        B[i] = (rand() % 2000 - 1000) / 1000.0f;
    }
}

#define LCG_A 6364136223846793005ULL
#define LCG_C 1442695040888963407ULL

float sgpu_frand(uint64_t *state) {
    *state = *state * LCG_A + LCG_C;
    return (float)((*state >> 40) & 0xFFFFFF) / (float)0x1000000;
}

/* Advance the LCG by n steps in O(log n) (affine map composition), so a long stream can be
 * produced in parallel chunks that equal the serial stream. */
static uint64_t lcg_skip(uint64_t s, uint64_t n) {
    uint64_t acc_a = 1, acc_c = 0, a = LCG_A, c = LCG_C;
    while (n) {
        if (n & 1) { acc_a *= a; acc_c = acc_c * a + c; }
        c = c * (a + 1);
        a = a * a;
        n >>= 1;
    }
    return s * acc_a + acc_c;
}

void sgpu_gen_uniform(float *out, size_t n, uint64_t *state, float offset) {
    const uint64_t s0 = *state;
#pragma omp parallel for schedule(static)
    for (long long c = 0; c < (long long)((n + 65535) / 65536); c++) {
        uint64_t s = lcg_skip(s0, (uint64_t)c * 65536);
        size_t end = (size_t)(c + 1) * 65536 < n ? (size_t)(c + 1) * 65536 : n;
        for (size_t i = (size_t)c * 65536; i < end; i++) out[i] = sgpu_frand(&s) + offset;
    }
    *state = lcg_skip(s0, n);
}

static void normal_pair(uint64_t *s, float mean, float std, float *z0, float *z1) {
    double u1 = sgpu_frand(s), u2 = sgpu_frand(s);
    if (u1 <= 0.0) u1 = 1.0 / 16777216.0;
    double r = sqrt(-2.0 * log(u1)), th = 6.283185307179586 * u2;
    *z0 = (float)(mean + std * (r * cos(th)));
    *z1 = (float)(mean + std * (r * sin(th)));
}

void sgpu_gen_normal(float *out, size_t n, uint64_t *state, float mean, float std) {
    const uint64_t s0 = *state;
    const size_t pairs = (n + 1) / 2;
#pragma omp parallel for schedule(static)
    for (long long c = 0; c < (long long)((pairs + 32767) / 32768); c++) {
        uint64_t s = lcg_skip(s0, (uint64_t)c * 65536);
        size_t p_end = (size_t)(c + 1) * 32768 < pairs ? (size_t)(c + 1) * 32768 : pairs;
        for (size_t p = (size_t)c * 32768; p < p_end; p++) {
            float z0, z1;
            normal_pair(&s, mean, std, &z0, &z1);
            out[2 * p] = z0;
            if (2 * p + 1 < n) out[2 * p + 1] = z1;
        }
    }
    *state = lcg_skip(s0, 2 * pairs);
}

static uint16_t f32_to_f16_rne(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t absu = u & 0x7fffffffu;
    if (absu >= 0x7f800000u) return (uint16_t)(sign | (absu > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (absu >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);        /* rounds to >= 65520 */
    if (absu < 0x38800000u) {                                          /* below 2^-14: subnormal */
        if (absu < 0x33000000u) return (uint16_t)sign;                   /* < 2^-25 rounds to 0 */
        uint32_t e = absu >> 23, m = (absu & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126 - e;                                      /* 14 + (127-e) - 1 ... */
        /* value = m * 2^(e-150); fp16 subnormal unit = 2^-24 -> q = m * 2^(e-126) */
        uint32_t q = m >> (shift), rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t h = ((absu - 0x38000000u) >> 13);                          /* rebias 127 -> 15 */
    uint32_t rem = absu & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) h++;
    return (uint16_t)(sign | h);
}

void sgpu_f32_to_f16(const float *in, uint16_t *out, size_t n) {
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; i++) out[i] = f32_to_f16_rne(in[i]);
}

float sgpu_h2f_host(uint16_t h) {
    uint32_t e = (h >> 10) & 0x1fu;
    if (e == 0) return 0.0f;
    uint32_t u = ((uint32_t)(h & 0x8000u) << 16) | ((e + 112u) << 23) | ((uint32_t)(h & 0x3ffu) << 13);
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* ---- library-internal launches ---- */
int sgpu_internal_embed_h(const uint16_t *emb, int token, float *x, int C, void *stream) {
    if (C <= 0 || token < 0 || !emb || !x) return SGPU_ERR_INVALID_ARG;
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    unsigned g[3] = {(unsigned)elem_grid(C), 1, 1}, b[3] = {256, 1, 1};
    void *args[] = {(void *)&emb, &token, (void *)&x, &C};
    return launch(d->fn[K_EMBED_H], g, b, stream, args);
}

/* ---- fused decode kernels (sgpu_decode.hip) ---- */
/* Pick a (team, segments) instance for K columns and nteams teams: the smallest team that
 * still gives >= 8 waves per CU, else the largest that fits; -1 if none fits. */
static int dec_pick(const devstate *d, int K, int nteams, int n_entries, int vec) {
    if (K <= 0 || K % vec || nteams <= 0) return -1;
    const long long nseg = K / vec, want = 8LL * d->cus;
    int best = -1, best_lpr = 0;
    const int lprs[3] = {16, 64, 256};
    for (int li = 0; li < 3; li++) {
        int pick = -1;
        for (int j = 0; j < n_entries; j++)
            if (g_dec_cfg[j][0] == lprs[li] && (long long)g_dec_cfg[j][1] * lprs[li] >= nseg &&
                (pick < 0 || g_dec_cfg[j][1] < g_dec_cfg[pick][1]))
                pick = j;
        if (pick < 0) continue;
        best = pick;
        best_lpr = lprs[li];
        if ((long long)nteams * best_lpr / 64 >= want) break;
    }
    return best;
}

/* One-wave teams (64 lanes) for the residual GEMVs whenever one fits K (up to 10 segments a
 * lane): their sums need no cross-wave LDS reduction or block barriers.  Qwen2.5-0.5B's o
 * (K 896) and down (K 4864) projections then run on 64x2 and 64x10 teams instead of 256x1 and
 * 256x3; decode 1911-1916 vs 1898-1901 tok/s, same-box A/B. */
static int dec_pick_res(int K, int vec) {
    const int nseg = K / vec;
    int best = -1;
    for (int e = 0; e < NDEC_ALL; e++)
        if (g_dec_cfg[e][0] == 64 && g_dec_cfg[e][1] * 64 >= nseg && (best < 0 || g_dec_cfg[e][1] < g_dec_cfg[best][1]))
            best = e;
    return best;
}

static int dec_launch_team(devstate *d, int fam, int K, int nteams, void **args, void *stream) {
    const int n_entries = dec_is_pair(fam) ? NDEC_PAIR : NDEC_ALL;
    int j = -1;
    if (fam == DEC_RES && K > 0 && K % dec_vec(fam) == 0) j = dec_pick_res(K, dec_vec(fam));
    if (j < 0) j = dec_pick(d, K, nteams, n_entries, dec_vec(fam));
    if (j < 0) return SGPU_ERR_INVALID_ARG;
    const unsigned teams = 256u / (unsigned)g_dec_cfg[j][0];
    /* at most 8 blocks per CU: for the decode lm_head too (the standalone GEMV's 18 per CU
     * measured 1.4% fewer tokens/s in the replayed decode step) */
    unsigned g[3] = {umin(cdiv(nteams, teams), (unsigned)d->cus * 8u), 1, 1}, b[3] = {256, 1, 1};
    return launch(d->dec[fam][j], g, b, stream, args);
}

int sgpu_internal_dec_qkv(const uint16_t *W, int K, int nrows, const float *x, const uint16_t *lnw, float eps,
                          const float *bias, float *q, float *kc, float *vc, const float *cosT, const float *sinT,
                          const int *step, int NH, int NKV, int HD, void *stream) {
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    if ((uintptr_t)lnw & 15) return SGPU_ERR_INVALID_ARG;     /* gains loaded 8 codes at a time */
    if (HD <= 0 || HD % 2 || nrows != (NH + 2 * NKV) * HD) return SGPU_ERR_INVALID_ARG;
    int nteams = nrows / 2;
    void *args[] = {(void *)&W, &K, &nteams, (void *)&x, (void *)&lnw, &eps, (void *)&bias, (void *)&q,
                    (void *)&kc, (void *)&vc, (void *)&cosT, (void *)&sinT, (void *)&step, &NH, &NKV, &HD};
    return dec_launch_team(d, DEC_QKV, K, nteams, args, stream);
}

int sgpu_internal_dec_gateup(const uint16_t *W, int K, int FC, const float *x, const uint16_t *lnw, float eps,
                             float *y, void *stream) {
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    if ((uintptr_t)lnw & 15) return SGPU_ERR_INVALID_ARG;     /* gains loaded 8 codes at a time */
    void *args[] = {(void *)&W, &K, &FC, (void *)&x, (void *)&lnw, &eps, (void *)&y};
    return dec_launch_team(d, DEC_GATEUP, K, FC, args, stream);
}

int sgpu_internal_dec_res(const uint16_t *W, int K, int N, const float *a, const float *bias, float *x,
                          void *stream) {
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    void *args[] = {(void *)&W, &K, &N, (void *)&a, (void *)&bias, (void *)&x};
    return dec_launch_team(d, DEC_RES, K, N, args, stream);
}

int sgpu_internal_dec_lmhead(const uint16_t *W, int K, int N, const float *x, const uint16_t *lnw, float eps,
                             float *y, void *stream) {
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    if ((uintptr_t)lnw & 15) return SGPU_ERR_INVALID_ARG;     /* gains loaded 8 codes at a time */
    void *args[] = {(void *)&W, &K, &N, (void *)&x, (void *)&lnw, &eps, (void *)&y};
    return dec_launch_team(d, DEC_LMHEAD, K, N, args, stream);
}

int sgpu_internal_dec_attn(const float *q, const float *kc, const float *vc, float *out, const int *step, int NH,
                           int NKV, int HD, float scale, float *ws, unsigned *cnt, void *stream) {
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    const int j = HD == 32 ? 0 : HD == 64 ? 1 : HD == 128 ? 2 : -1;
    if (j < 0 || NKV <= 0 || NH <= 0 || NH % NKV || !ws || !cnt) return SGPU_ERR_INVALID_ARG;
    /* 8 * G * ceil(NKV * splits / 8) blocks: block b is head (b / 8) % G of unit
     * ((b / 8) / G) * 8 + b % 8 (KV group unit % NKV, chunk unit / NKV); units past
     * NKV * splits fall at chunk >= splits and exit. */
    const unsigned G = (unsigned)(NH / NKV), units = (unsigned)NKV * SGPU_ATTN_SPLITS;
    unsigned g[3] = {8u * G * ((units + 7u) / 8u), 1, 1}, b[3] = {256, 1, 1};
    void *args[] = {(void *)&q, (void *)&kc, (void *)&vc, (void *)&out, (void *)&step, &NH, &NKV, &scale,
                    (void *)&ws, (void *)&cnt};
    return launch(d->dec_attn[j], g, b, stream, args);
}

int sgpu_internal_dec_embed(const uint16_t *emb, int token, int pos, float *x, int C, int *step, void *stream) {
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    unsigned g[3] = {(unsigned)elem_grid(C), 1, 1}, b[3] = {256, 1, 1};
    void *args[] = {(void *)&emb, &token, &pos, (void *)&x, &C, (void *)&step};
    return launch(d->dec_embed, g, b, stream, args);
}

int sgpu_internal_dec_argmax_next(const float *v, int n, float *part_v, int *part_i, int *step, int *out,
                                  const uint16_t *emb, const float *wte, const float *wpe, float *x, int C, int ctx,
                                  void *stream) {
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    if (n <= 0 || C <= 0 || !x || (!emb && (!wte || !wpe))) return SGPU_ERR_INVALID_ARG;
    int np = SGPU_ARGMAX_PARTS;
    unsigned g[3] = {(unsigned)np, 1, 1}, b[3] = {256, 1, 1};
    void *a1[] = {(void *)&v, &n, (void *)&part_v, (void *)&part_i};
    if ((rc = launch(d->dec_argmax_part, g, b, stream, a1))) return rc;
    unsigned g2[3] = {1, 1, 1};
    if (emb) {
        void *a2[] = {(void *)&part_v, (void *)&part_i, &np, (void *)&step, (void *)&out, (void *)&emb, (void *)&x, &C};
        return launch(d->dec_argmax_embed, g2, b, stream, a2);
    }
    void *a2[] = {(void *)&part_v, (void *)&part_i, &np,          (void *)&step, (void *)&out,
                  (void *)&wte,    (void *)&wpe,    (void *)&x, &C, &ctx};
    return launch(d->dec_argmax_g2embed, g2, b, stream, a2);
}

/* ---- batched prompt prefill (sgpu_decode.hip sgpu_pf_*) ---- */
int sgpu_internal_pf_embed(const uint16_t *emb, const int *ids, int T, float *x, int C, void *stream) {
    if (!emb || !ids || !x || T <= 0 || C <= 0) return SGPU_ERR_INVALID_ARG;
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    unsigned g[3] = {(unsigned)elem_grid((int)umin((unsigned)((long long)T * C), 0x7fffffffu)), 1, 1}, b[3] = {256, 1, 1};
    void *args[] = {(void *)&emb, (void *)&ids, &T, (void *)&x, &C};
    return launch(d->pf_embed, g, b, stream, args);
}

int sgpu_internal_pf_gemm(const uint16_t *W, const float *X, const float *bias, float *Y, int K, int N, int T,
                          float *ws, unsigned *cnt, int accum, void *stream) {
    if (!W || !X || !Y || K <= 0 || N <= 0 || T <= 0 || K % 4 || ((uintptr_t)W & 7) || ((uintptr_t)X & 15))
        return SGPU_ERR_INVALID_ARG;
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    const int S = (ws && cnt) ? nt_splits(T, N, K, d->cus) : 1;
    const long long units = (long long)cdiv(T, 32) * cdiv(N, 32) * S;
    unsigned g[3] = {(unsigned)(units < 0x7fffffffLL ? units : 0x7fffffffLL), 1, 1}, b[3] = {256, 1, 1};
    void *args[] = {(void *)&W, (void *)&X, (void *)&bias, (void *)&Y, &K, &N, &T, (void *)&S, &ws, &cnt, &accum};
    return launch(d->pf_gemm, g, b, stream, args);
}

int sgpu_internal_pf_qkv_post(float *qkv, int T, int pos0, const float *cosT, const float *sinT, float *kc,
                              float *vc, int NH, int NKV, int HD, void *stream) {
    if (!qkv || !cosT || !sinT || !kc || !vc || T <= 0 || pos0 < 0 || NH <= 0 || NKV <= 0 || HD <= 0 || HD % 2)
        return SGPU_ERR_INVALID_ARG;
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    const long long per = (long long)(NH + NKV) * (HD / 2) + (long long)NKV * HD;
    unsigned g[3] = {(unsigned)elem_grid((int)umin((unsigned)(T * per), 0x7fffffffu)), 1, 1}, b[3] = {256, 1, 1};
    void *args[] = {(void *)&qkv, &T, &pos0, (void *)&cosT, (void *)&sinT, (void *)&kc, (void *)&vc, &NH, &NKV, &HD};
    return launch(d->pf_qkv_post, g, b, stream, args);
}

int sgpu_internal_pf_attn(const float *qkv, const float *kc, const float *vc, float *out, int T, int pos0, int NH,
                          int NKV, int HD, float scale, void *stream) {
    const int j = HD == 32 ? 0 : HD == 64 ? 1 : HD == 128 ? 2 : -1;
    if (j < 0 || !qkv || !kc || !vc || !out || T <= 0 || T > 65535 || pos0 < 0 || pos0 + T > 8192 || NKV <= 0 ||
        NH <= 0 || NH % NKV)
        return SGPU_ERR_INVALID_ARG;
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    int QKVD = (NH + 2 * NKV) * HD;
    unsigned g[3] = {(unsigned)NH, (unsigned)T, 1}, b[3] = {256, 1, 1};
    void *args[] = {(void *)&qkv, (void *)&kc, (void *)&vc, (void *)&out, &pos0, &NH, &NKV, &scale, &QKVD};
    return launch(d->pf_attn[j], g, b, stream, args);
}

int sgpu_internal_pf_swiglu(const float *Y, float *G, int FC, int T, void *stream) {
    if (!Y || !G || FC <= 0 || T <= 0) return SGPU_ERR_INVALID_ARG;
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    unsigned g[3] = {(unsigned)elem_grid((int)umin((unsigned)((long long)T * FC), 0x7fffffffu)), 1, 1}, b[3] = {256, 1, 1};
    void *args[] = {(void *)&Y, (void *)&G, &FC, &T};
    return launch(d->pf_swiglu, g, b, stream, args);
}

/* ---- GPT-2 fused decode (sgpu_decode.hip, fp32 weights) ---- */
int sgpu_internal_g2_qkv(const float *W, int K, int N, const float *x, const float *lnw, const float *lnb, float eps,
                         const float *bias, float *q, float *kc, float *vc, const int *step, void *stream) {
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    if (N != 3 * K || ((uintptr_t)W & 15) || ((uintptr_t)x & 15)) return SGPU_ERR_INVALID_ARG;
    void *args[] = {(void *)&W, &K, &N, (void *)&x, (void *)&lnw, (void *)&lnb, &eps, (void *)&bias,
                    (void *)&q, (void *)&kc, (void *)&vc, (void *)&step};
    return dec_launch_team(d, DEC_G2QKV, K, N, args, stream);
}

int sgpu_internal_g2_res(const float *W, int K, int N, const float *a, const float *bias, float *x, void *stream) {
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    if (((uintptr_t)W & 15) || ((uintptr_t)a & 15)) return SGPU_ERR_INVALID_ARG;
    void *args[] = {(void *)&W, &K, &N, (void *)&a, (void *)&bias, (void *)&x};
    return dec_launch_team(d, DEC_G2RES, K, N, args, stream);
}

int sgpu_internal_g2_fc(const float *W, int K, int N, const float *x, const float *lnw, const float *lnb, float eps,
                        const float *bias, float *y, void *stream) {
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    if (((uintptr_t)W & 15) || ((uintptr_t)x & 15)) return SGPU_ERR_INVALID_ARG;
    void *args[] = {(void *)&W, &K, &N, (void *)&x, (void *)&lnw, (void *)&lnb, &eps, (void *)&bias, (void *)&y};
    return dec_launch_team(d, DEC_G2FC, K, N, args, stream);
}

int sgpu_internal_g2_lmhead(const float *W, int K, int N, const float *x, const float *lnw, const float *lnb,
                            float eps, float *y, void *stream) {
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    if (((uintptr_t)W & 15) || ((uintptr_t)x & 15)) return SGPU_ERR_INVALID_ARG;
    void *args[] = {(void *)&W, &K, &N, (void *)&x, (void *)&lnw, (void *)&lnb, &eps, (void *)&y};
    return dec_launch_team(d, DEC_G2LMHEAD, K, N, args, stream);
}

int sgpu_internal_g2_embed(const float *wte, const float *wpe, int token, int pos, float *x, int C, int *step,
                           void *stream) {
    int rc;
    devstate *d = cur(&rc);
    if (!d) return rc;
    unsigned g[3] = {(unsigned)elem_grid(C), 1, 1}, b[3] = {256, 1, 1};
    void *args[] = {(void *)&wte, (void *)&wpe, &token, &pos, (void *)&x, &C, (void *)&step};
    return launch(d->dec_g2embed, g, b, stream, args);
}

