/* switch_gpu.h -- C ABI of libswitchgpu.so, the MI355X (gfx950) matmul hot path.
 *
 * Drop-in for the reference's driver-API path: the SGEMM family of switch_gpu.cu, the
 * fp32 / fp16-weight batch-1 GEMV kernels of gpu-llm/kernels, and the host calls that
 * load and launch them (cuda_drv.h:14-32 and the per-file copies of those prototypes,
 * e.g. gpu_workload.c:19-31, qwen_engine.c:27-39).
 *
 * Conventions (kept from the reference, cuda_drv.h:9-40):
 *  - Every call returns an int status, 0 on success.  Positive values are hipError_t
 *    codes from the HIP runtime; negative values are this library's own (SGPU_ERR_*).
 *    sgpu_error_string() names both (cuGetErrorString role).
 *  - All buffer arguments are device pointers unless stated otherwise; sizes are element
 *    counts as in the reference kernels (ints, K before N in GEMV calls).  Sub-buffers
 *    are plain byte offsets from a device pointer.
 *  - The caller owns all memory; nothing here allocates except sgpu_malloc, the engine
 *    objects (sgpu_qwen_*, sgpu_gpt2_*) and the library's per-stream split-K workspaces (see
 *    sgpu_sgemm_splitk).  Outputs are fully overwritten (no accumulate-into-y/C).
 *  - `stream` is a hipStream_t passed as void*; NULL is the default stream, as the
 *    reference's cuLaunchKernel(..., NULL, ...) calls use.  Launchers are asynchronous.
 *  - bias pointers are nullable wherever the reference kernel reads `bias ? bias[n] : 0`.
 *
 * Launchers pick their own wave64 launch geometry; the code objects they use can also be
 * loaded by callers that resolve kernels by name (sgpu_code_object + hipModuleLoadData).
 */
#ifndef SWITCH_GPU_H
#define SWITCH_GPU_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---- */
#define SGPU_OK 0
#define SGPU_ERR_INVALID_ARG (-1)    /* a size, pointer or shape the call cannot accept */
#define SGPU_ERR_NOT_INITIALIZED (-2) /* sgpu_init has not succeeded on the current device */
#define SGPU_ERR_NO_KERNEL (-3)      /* a code object lacks a kernel the call needs */
#define SGPU_ERR_NO_DEVICE (-4)      /* no usable HIP device */
#define SGPU_ERR_HOST_ALLOC (-5)     /* host memory exhausted */
#define SGPU_ERR_NO_WORKSPACE (-6)   /* a split-K launch on a stream that has no workspace and cannot
                                        get one now (being recorded, or 32 streams already hold one) */
#define SGPU_ERR_SCRATCH_LIMIT (-7)  /* more than the allocation-free entry point's fixed scratch */

/* Replaces cuGetErrorString (cuda_drv.h:31).  Never NULL. */
const char *sgpu_error_string(int status);

/* ---- runtime: device, memory, synchronisation (cuda_drv.h:14-30) ---- */

/* Replaces cuInit + cuDeviceGet + cuCtxCreate_v2 + cuModuleLoadData + cuModuleGetFunction
 * (gpu_workload.c:65-74, qwen_engine.c:144-155): makes `device` current and loads every
 * embedded gfx950 code object on it, resolving all kernels.  Idempotent per device. */
int sgpu_init(int device);
/* cuDeviceGetCount (cuda_drv.h:16). */
int sgpu_device_count(int *count);

typedef struct {
    char name[256];           /* marketing name, e.g. "AMD Instinct MI355X" */
    char arch[64];            /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    int compute_units;        /* CU count (cuDeviceGetAttribute SM_COUNT role) */
    int clock_khz;            /* peak shader clock (CU_ATTR_CLOCK_KHZ role) */
    int memory_clock_khz;
    int memory_bus_width;     /* bits */
    size_t total_mem;         /* bytes (cuDeviceTotalMem_v2 role) */
    size_t lds_per_block;     /* bytes */
    int l2_bytes;
    int warp_size;            /* 64 on CDNA */
} sgpu_device_props;
/* cuDeviceGetName / cuDeviceTotalMem_v2 / cuDeviceGetAttribute (cuda_drv.h:17-19). */
int sgpu_get_device_props(int device, sgpu_device_props *props);

int sgpu_malloc(void **dptr, size_t bytes);                          /* cuMemAlloc_v2 */
int sgpu_free(void *dptr);                                           /* cuMemFree_v2 */
int sgpu_memcpy_htod(void *dst, const void *src, size_t bytes);      /* cuMemcpyHtoD_v2 */
int sgpu_memcpy_dtoh(void *dst, const void *src, size_t bytes);      /* cuMemcpyDtoH_v2 */
int sgpu_memcpy_dtod(void *dst, const void *src, size_t bytes);      /* cuMemcpyDtoD_v2 (qwen_engine.c:229-230) */
int sgpu_memcpy_dtod_async(void *dst, const void *src, size_t bytes, void *stream);
int sgpu_memset_d8(void *dst, int value, size_t bytes);              /* synchronous byte fill */
int sgpu_synchronize(void);                                          /* cuCtxSynchronize */
int sgpu_stream_synchronize(void *stream);

/* Streams and recorded launch sequences.  A caller that issues the same launches many times
 * (a serving loop, a benchmark of a short kernel) records them once on a stream made here and
 * replays them with one call: every sgpu_* launcher that takes a stream can be recorded, and
 * recorded launches do not run until the graph is launched.  Recording is thread-local: other
 * threads' HIP work is unaffected, while the recording thread must not call the synchronous
 * sgpu_* functions (copies, fills, synchronize) until sgpu_graph_end.  Streams are created at
 * the default priority.  No reference counterpart (the reference launches one kernel per
 * host call). */
int sgpu_stream_create(void **stream);
int sgpu_stream_destroy(void *stream);              /* waits for the stream's work first */
int sgpu_graph_begin(void *stream);                 /* stream must not be NULL */
int sgpu_graph_end(void *stream, void **graph);     /* instantiated; *graph NULL on error */
int sgpu_graph_launch(void *graph, void *stream);
int sgpu_graph_destroy(void *graph);

/* Timing with HIP events on a stream (the reference times with CLOCK_MONOTONIC around a
 * synchronised batch, gpu_workload.c:133-139; events time the stream itself). */
int sgpu_event_create(void **event);
int sgpu_event_destroy(void *event);
int sgpu_event_record(void *event, void *stream);
int sgpu_event_elapsed_ms(float *ms, void *start, void *stop);

/* ---- code objects (the PTX modules' role: switch_gpu.ptx, gemv.ptx, gpt2.ptx, qwen.ptx) ----
 * Returns the embedded gfx950 ELF code object named "switch_gpu", "gemv", "gpt2_kernels",
 * "qwen_kernels", "sgpu_tuned", "sgpu_decode" or "sgpu_probe" (and its size), ready for
 * hipModuleLoadData; NULL if the name is unknown.  The first four export the reference's
 * kernel names and arguments; "sgpu_probe" holds the measurement kernels of bin/decode_floor. */
const void *sgpu_code_object(const char *name, size_t *size);

/* Launch geometry the launchers use for a reference-named kernel at a given shape
 * (SGEMM: M, N, K; GEMV family: N rows, K columns, M unused).  Lets a host that keeps its
 * own hipModuleLaunchKernel calls (the gpu_workload flow) launch the code objects with the
 * kernels' intended wave64 geometry.  Returns SGPU_ERR_NO_KERNEL for an unknown name. */
int sgpu_kernel_geometry(const char *kernel, int M, int N, int K, unsigned grid[3], unsigned block[3]);

/* ---- SGEMM family: C = A*B, fp32 row-major, alpha 1, beta 0 ----
 * A: MxK (stride K), B: KxN (stride N), C: MxN (stride N).  Any M, N, K >= 0 (the
 * reference kernels require multiples of 32/64, switch_gpu.cu:58,98).
 * Replaces cuLaunchKernel(sgemm_*, ...) at gpu_workload.c:90,117,142,168; kernel
 * signatures switch_gpu.cu:5-8 (sgemm_tiled), :59-62 (sgemm_tiled4), :99-102 (sgemm_opt),
 * :140-143 (sgemm_naive).
 * sgpu_sgemm_tiled / _tiled4 / _naive launch their own code-object symbol (tiles 64x64,
 * 128x128; one output per thread).  sgpu_sgemm_opt is the tuned entry: it launches the
 * member (sgemm_opt256 256x256, sgemm_opt 128x256, sgemm_tiled4 128x128 or sgemm_tiled
 * 64x64 tiles) whose busiest CU has the least work: ceil(tiles / CUs) tiles times the
 * tile's area over the member's sustained rate.  Problems whose 16x16 tiles fit the CUs in
 * one round go to sgemm_small16 (K <= 2048, or K <= 4096 with a quarter of the CUs' tiles
 * or one row or column of tiles), else those whose 32x32 tiles do (K <= 1024) to
 * sgemm_small32; of the rest, problems of at most two rounds of 64x64 tiles go to
 * sgemm_splitk when a cost model of the busiest CU's k-slices, masked tail slices and split
 * hand-offs prefers a 2-8 way split (16 for a few tiles of tall K) to none -- except that
 * problems of whole 64x64 tiles filling 3/4 to all of the CUs in one round, with K a
 * multiple of 32 and at least 1024, go to sgemm_kwave (to sgemm_kwave_edge when A or B is
 * off 16-byte alignment), and other problems whose sgemm_kwave_edge tiles fill 3/4 to all
 * of the CUs in one round, with K >= 384 (K >= 128 when the 64x64 tiles would not fit the
 * CUs in one round), go to sgemm_kwave_edge.  Of the problems left for the size rule, those
 * with M, N multiples of 128 and K of 32 whose 128x128 tiles fill whole rounds of the CUs
 * (the last at least 94% full), with K >= 512 (K >= 4096 where the size rule picks
 * sgemm_opt256), go to sgemm_kwave128 (to the size rule's member when A or B is off
 * 16-byte alignment). */
int sgpu_sgemm_tiled(const float *A, const float *B, float *C, int M, int N, int K, void *stream);
int sgpu_sgemm_tiled4(const float *A, const float *B, float *C, int M, int N, int K, void *stream);
int sgpu_sgemm_opt(const float *A, const float *B, float *C, int M, int N, int K, void *stream);
/* The symbol sgpu_sgemm_opt launches for an M x N x K problem on a device of `cus` compute
 * units ("sgemm_small16", "sgemm_splitk", "sgemm_opt256", ...), with the split count in
 * *splits (1 unless "sgemm_splitk"); a pure function, no device needed.  NULL when nothing
 * is launched (M or N < 1) or an argument is invalid.  sgpu_sgemm_opt launches the unsplit
 * member instead of "sgemm_splitk" on a stream being recorded that has no workspace yet;
 * the plan assumes 16-byte aligned A and B: with A or B off 16 bytes, "sgemm_kwave" becomes
 * "sgemm_kwave_edge" and "sgemm_kwave128" the member the size rule picks, and with an operand
 * off 4 bytes "sgemm_kwave" or "sgemm_kwave_edge" becomes the 64x64-or-larger member the size
 * rule picks.
 * No counterpart in the reference (its sgemm_opt is one kernel). */
const char *sgpu_sgemm_opt_plan(int M, int N, int K, int cus, int *splits);
/* The sgemm_opt256 member alone (any shape; masked loads on edge tiles).  No
 * counterpart in the reference: an added member of the same family, with the same
 * (A, B, C, M, N, K) symbol arguments, for hosts that launch members by name. */
int sgpu_sgemm_opt256(const float *A, const float *B, float *C, int M, int N, int K, void *stream);
/* The sgemm_kwave member: 64x64 tiles of C, each computed by a block of four waves that
 * split K four ways, every wave accumulating the whole tile with its MFMA operands loaded
 * straight from memory into registers, the four partial tiles summed in wave order.  M and
 * N multiples of 64, K a multiple of 32, A and B 16-byte aligned (SGPU_ERR_INVALID_ARG
 * otherwise).  Operands whose 64-row A panel or 16-row B slice reach 2^31 bytes run on the
 * LDS-staged sgemm_kwave_wide instead (same results).  No counterpart in the reference: an
 * added member of the family with the (A, B, C, M, N, K) symbol arguments. */
int sgpu_sgemm_kwave(const float *A, const float *B, float *C, int M, int N, int K, void *stream);
/* The sgemm_kwave_edge member: sgemm_kwave's structure for any M >= 64, N >= 64, K >= 1 and
 * float-aligned A, B, C (SGPU_ERR_INVALID_ARG otherwise; M or N == 0 is a no-op).  A partial
 * last row or column of tiles is computed as the 64 rows or columns ending at the last one
 * and stored from its first new row or column on; with K % 16 != 0 the first 16-deep k-slice
 * is the partial one (k < K % 16), read with zeros past it.  Operands past the 2^31-byte
 * windows run on the LDS-staged sgemm_kwave_edge_wide (32-deep slices).
 * With N % 64 == 1 the last column is computed by the last column of whole tiles alongside
 * their MFMAs, so ceil(M/64) * (N/64) blocks; otherwise ceil(M/64) * ceil(N/64).  No
 * counterpart in the reference: an added member of the family with the (A, B, C, M, N, K)
 * symbol arguments. */
int sgpu_sgemm_kwave_edge(const float *A, const float *B, float *C, int M, int N, int K, void *stream);
/* The sgemm_kwave128 member: sgemm_kwave's structure on 128x128 tiles (each wave accumulates
 * the whole tile over a quarter of K, 16-deep k-slices handed out in pairs).  M and N multiples
 * of 128, K a multiple of 32, A and B 16-byte aligned, a 128-row A panel (128*K floats) and a
 * 16-row B slice (16*N floats) each under 2^31 bytes (SGPU_ERR_INVALID_ARG otherwise; there
 * is no wide form).  One block of 256 threads per tile, (M/128) * (N/128) blocks.  No
 * counterpart in the reference: an added member of the family with the (A, B, C, M, N, K)
 * symbol arguments. */
int sgpu_sgemm_kwave128(const float *A, const float *B, float *C, int M, int N, int K, void *stream);
/* The sgemm_splitk member: 64x64 tiles with K split S ways (S >= 1; reduced so that every
 * split holds at least one 32-deep slice), each (tile, split) a block.  Every split writes its
 * partial tile to a library-owned workspace of the launch's stream and the last split of a
 * tile sums all S partials in split order, so results do not depend on arrival order.
 * Rejects problems needing more than 16384 tiles or S x tiles x 4096 floats (32 MB) of
 * workspace (SGPU_ERR_INVALID_ARG).  No counterpart in the reference.
 * Split-K workspaces (also used by sgpu_sgemm_opt and sgpu_gemv_multi when they split K): one
 * per stream, so launches on different streams or from different host threads may overlap;
 * launches on one stream run in order.  The null stream's is made by sgpu_init; another
 * stream's on its first launch that splits (32 MB + 64 KB, at most 32 streams per device),
 * kept until sgpu_stream_destroy releases it (streams not made by sgpu_stream_create keep
 * theirs until the process ends).  hipStreamPerThread names a different stream in every host
 * thread and gets none: sgpu_sgemm_splitk returns SGPU_ERR_NO_WORKSPACE on it.  A stream
 * being recorded (sgpu_graph_begin) cannot get one: make its first split launch before
 * recording, else sgpu_sgemm_splitk returns SGPU_ERR_NO_WORKSPACE; on either kind of stream
 * sgpu_sgemm_opt / sgpu_gemv_multi launch their unsplit kernels instead.  A recorded graph
 * uses the workspace of the stream it was recorded on, which stays allocated while the graph
 * exists, also after that stream is destroyed; do not replay the graph concurrently with
 * itself or with other split launches on that stream. */
int sgpu_sgemm_splitk(const float *A, const float *B, float *C, int M, int N, int K, int S, void *stream);
/* sgpu_sgemm_splitk that allocates nothing, for callers that cannot allocate device memory
 * (code under graph capture, tight serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference.  Same kernel and arguments, same results bit for bit; the
 * partial tiles and tile counters live in a fixed scratch array compiled into the library,
 * one copy per device, held until the process ends: at most 32 MiB of partial tiles
 * (splits x 64x64 tiles x 4096 floats <= 8 Mi floats) and 16384 tiles, larger problems
 * rejected with SGPU_ERR_SCRATCH_LIMIT.  The device must be set up by sgpu_init first
 * (SGPU_ERR_NOT_INITIALIZED otherwise).  Every call on a device shares that device's scratch
 * (counters zeroed at set-up; each launch leaves them at zero): calls that overlap in time
 * on one device -- other streams, other host threads, a replayed graph -- race. */
int sgpu_sgemm_splitk_noalloc(const float *A, const float *B, float *C, int M, int N, int K, int S,
                              void *stream);
/* The small-problem members sgemm_small16 / sgemm_small32 (tile = 16 or 32): one tile x tile
 * block of C per workgroup, A and B read straight into the matrix cores (no LDS staging), the
 * workgroup's four waves splitting K and summing their partials in a fixed order.  Any shape
 * whose A (plus 32 rows) and B (plus 256 rows) stay under 2 GB (SGPU_ERR_INVALID_ARG
 * otherwise).  No counterpart in the reference. */
int sgpu_sgemm_small(const float *A, const float *B, float *C, int M, int N, int K, int tile, void *stream);
int sgpu_sgemm_naive(const float *A, const float *B, float *C, int M, int N, int K, void *stream);

/* Read-bandwidth probe, membw_read4 (switch_gpu.cu:41-54; launched gpu_workload.c:210-213):
 * every thread sums its grid-stride float4 sweep `iters` times into out[first index].
 * buf: n4 float4 (16-byte aligned); out: one float per launched thread with index < n4.
 * `threads` returns the launched thread count (may be NULL). */
int sgpu_membw_read4(const void *buf, float *out, int n4, int iters, int *threads, void *stream);

/* ---- batch-1 GEMV, fp32 weights: y[n] = sum_k W[n*K+k] x[k] (+ bias[n]) ----
 * W: NxK row-major.  Any K (the reference float4 kernels need K % 4 == 0).
 * gemv / gemv4 / gemv_warp: gemv.cu:3-6,18-21,51-54 and gpt2_kernels.cu:38-41, launched
 * gemv_test.c:109 and gpt2_engine.c:188,214,230,243,260.  gemv_warp_b: gpt2_kernels.cu:75-79,
 * launched gpt2_engine.c:185,211,227,240 (bias nullable here). */
int sgpu_gemv(const float *W, const float *x, float *y, int K, int N, void *stream);
int sgpu_gemv4(const float *W, const float *x, float *y, int K, int N, void *stream);
int sgpu_gemv_warp(const float *W, const float *x, float *y, int K, int N, void *stream);
int sgpu_gemv_warp_b(const float *W, const float *x, const float *bias, float *y, int K, int N,
                     void *stream);

/* Weight-stationary batched GEMV, gemv_multi (gpt2_kernels.cu:110-155, launched
 * gpt2_engine.c:280,295,304,311): Y[t*N+n] = W[n,:].X[t,:] + (bias ? bias[n] : 0), X: TxK. */
int sgpu_gemv_multi(const float *W, const float *X, const float *bias, float *Y, int K, int N, int T,
                    void *stream);

/* fp16-weight GEMV, gemv_h (qwen_kernels.cu:34-38, launched qwen_engine.c:219,242,249,256,265):
 * W holds fp16 bit patterns decoded with the reference h2f (qwen_kernels.cu:6-14), x and
 * bias are fp32, bias nullable.  Any K (the reference needs K % 4 == 0). */
int sgpu_gemv_h(const uint16_t *W, const float *x, const float *bias, float *y, int K, int N,
                void *stream);
/* fp16-x GEMV, gemv_hh: gemv_h (qwen_kernels.cu:34-70) with x stored as fp16 bit patterns
 * as well, decoded with the same h2f contract as W (qwen_kernels.cu:6-14), fp32 accumulate,
 * fp32 bias (nullable): y[n] = sum_k h2f(W[n*K+k]) * h2f(x[k]) + bias?[n] -- bit for bit
 * what sgpu_gemv_h gives for x = h2f(x16).  Any K; the tuned path needs W and x 16-byte
 * aligned (K % 8 == 0), other calls take the by-name gemv_hh symbol.  No counterpart in the
 * reference, whose gemv_h reads fp32 x only: the fp16-activation variant of the Qwen GEMV
 * shapes (qwen_engine.c:219,242,249,256,265). */
int sgpu_gemv_hh(const uint16_t *W, const uint16_t *x, const float *bias, float *y, int K, int N,
                 void *stream);

/* ---- Qwen2.5 decode support kernels (qwen_kernels.cu:72-189), launched per layer by
 * gpu_forward (qwen_engine.c:216-264). ---- */
/* rows independent rows of n; w fp16 bits (qwen_kernels.cu:74-93, grid = rows). */
int sgpu_rmsnorm(const float *x, const uint16_t *w, float *y, int n, float eps, int rows, void *stream);
/* qwen_kernels.cu:97-116, launched qwen_engine.c:222-226. */
int sgpu_rope(float *x, const float *cosT, const float *sinT, int T, int H, int HD, int pos0, void *stream);
/* qwen_kernels.cu:119-126, launched qwen_engine.c:253-254. */
int sgpu_swiglu(const float *g, const float *u, float *y, int n, void *stream);
/* qwen_kernels.cu:130-144, launched qwen_engine.c:231-232. */
int sgpu_attn_scores_gqa(const float *q, const float *kc, float *scores, int T, float scale, int NH, int KV,
                         int HD, void *stream);
/* qwen_kernels.cu:147-164, launched qwen_engine.c:233-234. */
int sgpu_attn_softmax(const float *scores, float *probs, int T, int NH, void *stream);
/* qwen_kernels.cu:167-180, launched qwen_engine.c:235-236. */
int sgpu_attn_mix_gqa(const float *probs, const float *vc, float *out, int T, int NH, int KV, int HD,
                      void *stream);
/* qwen_kernels.cu:183-189, launched qwen_engine.c:244,258. */
int sgpu_add2(const float *a, const float *b, float *out, int n, void *stream);

/* ---- GPT-2 124M decode support kernels (gpt2_kernels.cu:157-268), launched per layer by
 * gpt2_engine.c gpu_forward (:174-264) and gpu_prefill (:269-326).  The attention kernels keep
 * the reference's fixed layout: 12 heads of 64, K/V cache rows of 768 floats. ---- */
/* rows independent rows of n: (x - mean)/sqrt(var + eps) * w + b (gpt2_kernels.cu:160-196). */
int sgpu_layernorm(const float *x, const float *w, const float *b, float *y, int n, float eps, int rows,
                   void *stream);
/* tanh-form GELU, y may alias x (gpt2_kernels.cu:199-206, launched gpt2_engine.c:236). */
int sgpu_gelu(const float *x, float *y, int n, void *stream);
/* y += bias (gpt2_kernels.cu:209-212, launched gpt2_engine.c:190,216,232,245). */
int sgpu_add_bias(float *y, const float *bias, int n, void *stream);
/* attn_scores (gpt2_kernels.cu:221-234, launched gpt2_engine.c:199-200). */
int sgpu_gpt2_attn_scores(const float *q, const float *kcache, float *scores, int T, float scale, void *stream);
/* attn_softmax (gpt2_kernels.cu:238-253, launched gpt2_engine.c:201-202). */
int sgpu_gpt2_attn_softmax(const float *scores, float *probs, int T, void *stream);
/* attn_mix (gpt2_kernels.cu:258-268, launched gpt2_engine.c:203-204). */
int sgpu_gpt2_attn_mix(const float *probs, const float *vcache, float *out, int T, void *stream);

/* ---- GPT-2 124M fp32 decode engine (gpt2_engine.c:88-326) ---- */
typedef struct {
    int V, C, NL, NH, HD, FC, CTX;
    float eps;       /* LayerNorm eps (gpt2_engine.c:77: 1e-5) */
} sgpu_gpt2_cfg;
/* gpt2_engine.c:40-48: V 50257, C 768, 12 heads of 64, 12 layers, FC 3072, CTX 1024.  The
 * attention kernels fix C = 768, NH = 12, HD = 64; V, NL, CTX and FC may differ. */
void sgpu_gpt2_default_cfg(sgpu_gpt2_cfg *cfg);
/* Float count of the flat fp32 weight file (gpt2_engine.c:50-70 layout; conv_gpt2.py writer):
 * 124,439,808 at the default dims. */
size_t sgpu_gpt2_file_floats(const sgpu_gpt2_cfg *cfg);
/* Random-init weights in that layout (make_random_bin.py role): every float
 * (frand() - 0.5) * 2 * amp from the seeded LCG. */
int sgpu_gpt2_fill_random(float *blob, const sgpu_gpt2_cfg *cfg, uint64_t seed, float amp);

typedef struct sgpu_gpt2 sgpu_gpt2;
/* gpu_setup (gpt2_engine.c:108-166): uploads the host weights, allocates fp32 KV caches and
 * the batched-prefill buffers. */
int sgpu_gpt2_create(sgpu_gpt2 **engine, const sgpu_gpt2_cfg *cfg, const float *blob);
void sgpu_gpt2_destroy(sgpu_gpt2 *engine);
/* gpu_forward (gpt2_engine.c:174-264): fused != 0 takes the --fused path (gemv_warp_b),
 * otherwise gemv_warp + add_bias.  Logits (V floats) copied to logits_host if want_logits. */
int sgpu_gpt2_forward(sgpu_gpt2 *engine, int token, int pos, int want_logits, float *logits_host, int fused);
/* The reference launch sequence (fused = its --fused variant), whatever the engine's path,
 * copying the residual stream after each layer to trace_host (NL x C floats): the per-layer
 * trace of the reference's self-test (gpt2_engine.c:478-494).  Logits to logits_host when it
 * is not NULL.  Synchronous; the KV cache gains `pos` as with sgpu_gpt2_forward. */
int sgpu_gpt2_forward_trace(sgpu_gpt2 *engine, int token, int pos, float *logits_host, float *trace_host, int fused);
/* Receives one stage vector of a traced forward (sgpu_gpt2_forward_stages,
 * sgpu_qwen_forward_stages): the stage's name and a host copy of its n floats, valid during the
 * call. */
typedef void (*sgpu_stage_fn)(void *ctx, const char *stage, const float *v, int n);
/* The GPU stage tracer of the reference's --debug (gprvec, gpt2_engine.c:173-251,356-362):
 * sgpu_gpt2_forward on the REFERENCE launch sequence (fused: the bias epilogue GEMVs), whatever
 * the engine's path, which at layer 0 waits for each stage and hands its vector to fn: "ln1",
 * "qkv" (3C), "scores" and "probs" ((pos+1) x NH), "attnout", "ao", "res1", "ln2", "fc" (FC),
 * "gelu" (FC), "proj", "res2" (C unless noted).  Logits to logits_host when it is not NULL.
 * Synchronous; the KV cache gains `pos`. */
int sgpu_gpt2_forward_stages(sgpu_gpt2 *engine, int token, int pos, float *logits_host, int fused, sgpu_stage_fn fn,
                             void *ctx);
/* gpu_prefill (gpt2_engine.c:269-326): all T prompt positions through the layers with the
 * weight-stationary gemv_multi; fills cache positions 0..T-1; logits of the last row. */
int sgpu_gpt2_prefill(sgpu_gpt2 *engine, const int *ids, int T, float *logits_host);
/* Execution paths of sgpu_gpt2_forward / sgpu_gpt2_generate (same arithmetic, results within
 * fp32 reordering of each other):
 *  REFERENCE -- the gpu_forward launch sequence above (its `fused` flag chooses gemv_warp_b)
 *  FUSED     -- five kernels per layer: LayerNorm+qkv+bias+KV-cache write, attention,
 *               o+bias+residual, LayerNorm+fc+bias+GELU, proj+bias+residual (`fused` ignored)
 *  GRAPH     -- FUSED with the layer stack captured once as a HIP graph and replayed
 * FUSED and GRAPH need CTX <= 8192 (SGPU_ERR_INVALID_ARG otherwise).
 * No counterpart in the reference beyond the sequence it restates. */
#define SGPU_GPT2_PATH_REFERENCE 0
#define SGPU_GPT2_PATH_FUSED 1
#define SGPU_GPT2_PATH_GRAPH 2
int sgpu_gpt2_set_path(sgpu_gpt2 *engine, int path);
/* Greedy decode (the reference generation loop, gpt2_engine.c:551-562, without its EOT stop):
 * prime with prompt[0..T-1], then n_gen more positions; out_tokens receives n_gen + 1 ids, the
 * argmax (first max) after the prompt and after each generated position.  FUSED/GRAPH keep
 * the argmax and the next embedding on the device. */
int sgpu_gpt2_generate(sgpu_gpt2 *engine, const int *prompt, int T, int n_gen, int *out_tokens);

/* ---- Qwen2.5 decode engine (qwen_engine.c:105-269): weights resident on the device,
 * fp32 KV cache, the reference's per-layer launch sequence per position. ---- */
typedef struct {
    int V, C, NL, NH, NKV, HD, FC, CTX;
    float eps;       /* RMSNorm eps (qwen_engine.c:55: 1e-6) */
    float theta;     /* RoPE base used by the weight writer (conv_qwen.py:27: 1e6) */
} sgpu_qwen_cfg;
/* The Qwen2.5-0.5B dims of qwen_engine.c:43-55 (V 151936, C 896, 24 layers, 14/2 heads,
 * HD 64, FC 4864, CTX 8192). */
void sgpu_qwen_default_cfg(sgpu_qwen_cfg *cfg);
/* Byte size of the flat weight file (qwen_engine.c:61-67 layout). */
size_t sgpu_qwen_file_bytes(const sgpu_qwen_cfg *cfg);
/* Fill a host blob of sgpu_qwen_file_bytes() with a random-init model in that layout:
 * every fp16 tensor N(0, std) from the seeded LCG + Box-Muller (cast to fp16 RNE), RoPE
 * tables from conv_qwen.py:75-80 (float64 angles, stored fp32). */
int sgpu_qwen_fill_random(void *blob, const sgpu_qwen_cfg *cfg, uint64_t seed, float std);

typedef struct sgpu_qwen sgpu_qwen;
/* gpu_setup (qwen_engine.c:137-189): uploads the host blob, allocates KV caches and
 * activation buffers on the current device. */
int sgpu_qwen_create(sgpu_qwen **engine, const sgpu_qwen_cfg *cfg, const void *blob);
void sgpu_qwen_destroy(sgpu_qwen *engine);
/* gpu_forward (qwen_engine.c:205-269): token at `pos` (cache holds 0..pos-1 and gains pos).
 * If want_logits, the V logits are copied to host `logits_host` (may be NULL to leave them on
 * the device).  Synchronous when logits are requested, asynchronous otherwise. */
int sgpu_qwen_forward(sgpu_qwen *engine, int token, int pos, int want_logits, float *logits_host);
/* sgpu_qwen_forward on the REFERENCE launch sequence, whatever the engine's path, copying the
 * residual stream after each layer to trace_host (NL x C floats): the layer trace the
 * reference's self-test compares against its CPU forward (cpu_forward's trace argument,
 * qwen_engine.c:355; gpt2_engine.c:478-494).  Logits to logits_host when it is not NULL.
 * Synchronous.  The KV cache gains `pos` as with sgpu_qwen_forward. */
int sgpu_qwen_forward_trace(sgpu_qwen *engine, int token, int pos, float *logits_host, float *trace_host);
/* The GPU stage tracer of the reference's --debug (gprvec, qwen_engine.c:196-202,216-260):
 * sgpu_qwen_forward on the REFERENCE launch sequence, whatever the engine's path, which at
 * layer 0 waits for each stage and hands its vector to fn, as a host copy valid during the
 * call: "ln1" (C), "qkv" (after RoPE, QKVD), "scores" and "probs" ((pos+1) x NH), "attnout"
 * (C), "res1" (C), "gate" (the gate half, FC), "swiglu" (FC), "res2" (C).  Logits to
 * logits_host when it is not NULL.  Synchronous; the KV cache gains `pos`. */
int sgpu_qwen_forward_stages(sgpu_qwen *engine, int token, int pos, float *logits_host, sgpu_stage_fn fn, void *ctx);
/* Execution paths of sgpu_qwen_forward / sgpu_qwen_generate.  All compute the same
 * function (checked against the CPU golden); they differ in launch structure:
 *  REFERENCE -- the reference's per-layer sequence above, 14 launches + 2 copies per layer
 *  FUSED     -- five fused kernels per layer: RMSNorm+qkv+bias+RoPE+KV write, attention,
 *               o_proj+residual, RMSNorm+gate|up+SwiGLU, down+residual
 *  GRAPH     -- FUSED with the layer stack captured once as a HIP graph and replayed
 * FUSED and GRAPH need CTX <= 8192, HD in {32, 64, 128}, C and FC multiples of 8. */
#define SGPU_QWEN_PATH_REFERENCE 0
#define SGPU_QWEN_PATH_FUSED 1
#define SGPU_QWEN_PATH_GRAPH 2
int sgpu_qwen_set_path(sgpu_qwen *engine, int path);
/* In-graph cost of each decode phase on the FUSED kernels at position `pos` (0 <= pos < CTX):
 * for each phase, its launches for all NL layers recorded in one graph (the argmax and the
 * lm_head NL times over the same buffers), replayed reps times after a warm-up; us[i] gets the
 * best replay's time per launch, in the order qkv (RMSNorm + qkv + RoPE + KV write),
 * attention, o + residual, gate|up (RMSNorm + gate|up + SwiGLU), down + residual, lm_head
 * (final RMSNorm + lm_head), argmax + next embedding (SGPU_QWEN_NPHASES values).  The replays
 * overwrite the KV cache at `pos` and the activations; the engine is left at `pos` with token
 * 0's embedding.  No counterpart in the reference (a measurement of the decode structure). */
#define SGPU_QWEN_NPHASES 7
int sgpu_qwen_phase_times(sgpu_qwen *engine, int pos, int reps, float *us);
/* Greedy decode (the reference generation loop, qwen_engine.c:534-548, without its EOT
 * stop): prime with prompt[0..T-1], then n_gen more positions.  out_tokens receives n_gen + 1
 * ids -- the argmax after the prompt and after each generated position, first max winning.
 * On the FUSED/GRAPH paths the prompt goes through sgpu_qwen_prefill and the argmax runs on
 * the device, so the loop never waits for the host; on the REFERENCE path it is the host loop
 * over sgpu_qwen_forward. */
int sgpu_qwen_generate(sgpu_qwen *engine, const int *prompt, int T, int n_gen, int *out_tokens);
/* Batched prompt prefill: positions 0..T-1 of ids through every layer together (each layer's
 * weights stream once per 512 prompt rows: matrix-core GEMMs on the fp16 weights, causal
 * attention over the cache), filling KV-cache positions 0..T-1; the last row's V logits are
 * copied to logits_host if it is not NULL.  sgpu_qwen_forward(engine, token, T, ...) then
 * continues.  Needs the FUSED/GRAPH conditions (any path may be selected).  No counterpart
 * in the Qwen reference, which primes the cache one position at a time
 * (qwen_engine.c:526-531); the GPT-2 engine's gpu_prefill (gpt2_engine.c:269-326) is the
 * model. */
int sgpu_qwen_prefill(sgpu_qwen *engine, const int *ids, int T, float *logits_host);
/* Device pointer to the last logits (V floats). */
const float *sgpu_qwen_device_logits(const sgpu_qwen *engine);

/* ---- seeded input generators (host only; no device needed) ----
 * gpu_workload.c:81-82: srand(seed); A[i], B[i] interleaved = (rand()%2000 - 1000)/1000.0f. */
void sgpu_gen_sgemm_inputs(float *A, float *B, size_t count, unsigned seed);
/* gemv_test.c:46-50 LCG: s = s*6364136223846793005 + 1442695040888963407,
 * value ((s >> 40) & 0xFFFFFF) / 2^24 in [0, 1). */
float sgpu_frand(uint64_t *state);
/* n values frand() + offset (gemv_test.c:80-81 uses offset -0.5). */
void sgpu_gen_uniform(float *out, size_t n, uint64_t *state, float offset);
/* n values mean + std * N(0,1), Box-Muller on two frand() draws (cosine branch). */
void sgpu_gen_normal(float *out, size_t n, uint64_t *state, float mean, float std);
/* fp32 -> fp16 bits, round to nearest even (overflow to inf, subnormals kept). */
void sgpu_f32_to_f16(const float *in, uint16_t *out, size_t n);
/* fp16 bits -> fp32 with the reference h2f contract (qwen_engine.c:90-98). */
float sgpu_h2f_host(uint16_t h);

#ifdef __cplusplus
}
#endif
#endif /* SWITCH_GPU_H */
