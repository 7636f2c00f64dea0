// sgpu_decode.hip -- fused Qwen2.5 decode kernels for gfx950 (five launches per layer).
//
// The reference runs 14 launches and 2 device copies per layer (qwen_engine.c:216-259).
// Here the same arithmetic is grouped so every kernel streams one weight matrix and keeps
// the small steps around it in its prologue or epilogue:
//   sgpu_dec_qkv_*    RMSNorm(x) -> qkv GEMV + bias -> RoPE on q and k -> q to its buffer,
//                     k and v straight into the layer's KV cache at `pos`
//   sgpu_dec_attn     GQA attention: blocks per head and position chunk, scores, softmax, mix,
//                     chunk partials combined by the head's last block
//   sgpu_dec_res_*    GEMV + residual add in place: x[n] += W[n,:].a (o_proj, down_proj)
//   sgpu_dec_gateup_* RMSNorm(x) -> gate and up rows of the same output -> SwiGLU
//   sgpu_dec_lmhead_* final RMSNorm -> tied lm_head GEMV
//   sgpu_dec_embed    token embedding (h2f) and the step record {token, pos} for the layers
//   sgpu_dec_argmax_* first-max argmax of the logits into the step record (greedy decode),
//                     the second stage also writing the next token's embedding
//   sgpu_dec_g2*      the GPT-2 (fp32) counterparts: LayerNorm+qkv+bias+KV write, GEMV+bias+
//                     residual, LayerNorm+fc+bias+GELU, LayerNorm+lm_head, wte+wpe embedding
// The position lives in device memory (`step`), so a whole position can be captured once as
// a HIP graph and replayed.  Weight rows are fp16 bits with the reference h2f contract (see
// gemv_core.h); this code object is built with the fp16 denormal mode set to flush.
#include "gemv_core.h"

namespace {

// ---- epilogues ----
// y[row] = resid[row] + (acc + bias?[row]); y may alias resid (each row touched by one lane).
struct EpiResidual {
    const float* resid;
    const float* bias;
    float* y;
    struct Pre {
        float res, b;
    };
    __device__ __forceinline__ void load(int, const int* rows, Pre& p) const {
        p.res = resid[rows[0]];                   // only this team writes row rows[0]
        p.b = bias ? bias[rows[0]] : 0.0f;
    }
    __device__ __forceinline__ void operator()(int, const int* rows, const float* acc, const Pre& p) const {
        y[rows[0]] = p.res + (acc[0] + p.b);
    }
};

// y[t] = silu(gate) * up, gate = rows t, up = rows t + FC (qwen_engine.c:349-350 form).
struct EpiSwiGLU {
    float* y;
    struct Pre {};
    __device__ __forceinline__ void load(int, const int*, Pre&) const {}
    __device__ __forceinline__ void operator()(int t, const int*, const float* acc, const Pre&) const {
#pragma clang fp contract(off)
        const float g = acc[0];
        y[t] = (g / (1.0f + expf(-g))) * acc[1];
    }
};

// Team t owns rows (i, i + HD/2) of head block hb: add the q/k/v bias, rotate q and k by the
// RoPE angle of `pos` (qwen_engine.c:303-317 arithmetic), write q to its buffer and k, v to
// the KV cache row of `pos` (the reference's cache copies, qwen_engine.c:229-230).
struct EpiQkvRope {
    const float* bias;
    float* q;
    float* kc;
    float* vc;
    const float* cosT;
    const float* sinT;
    const int* step;
    int NH, NKV, HD;
    struct Pre {
        float b0, b1, c, s;
        int pos;
    };
    __device__ __forceinline__ void load(int t, const int* rows, Pre& p) const {
        const int h2 = HD / 2, i = t % h2;
        p.pos = step[1];
        p.b0 = bias[rows[0]];
        p.b1 = bias[rows[1]];
        p.c = cosT[(size_t)p.pos * h2 + i];
        p.s = sinT[(size_t)p.pos * h2 + i];
    }
    __device__ __forceinline__ void operator()(int t, const int* rows, const float* acc, const Pre& p) const {
#pragma clang fp contract(off)
        const int h2 = HD / 2, hb = t / h2, i = t % h2, pos = p.pos;
        const int KVD = NKV * HD;
        const float a = acc[0] + p.b0, b = acc[1] + p.b1;
        if (hb < NH + NKV) {
            const float c = p.c, s = p.s;
            const float ra = a * c - b * s, rb = a * s + b * c;
            float* dst = hb < NH ? q + (size_t)hb * HD : kc + (size_t)pos * KVD + (size_t)(hb - NH) * HD;
            dst[i] = ra;
            dst[i + h2] = rb;
        } else {
            float* dst = vc + (size_t)pos * KVD + (size_t)(hb - NH - NKV) * HD;
            dst[i] = a;
            dst[i + h2] = b;
        }
    }
};

// GPT-2 qkv epilogue: row r of the fused [3C x C] projection plus its bias goes to q (rows
// 0..C-1) or to the layer's K / V cache row of `pos` (rows C..2C-1 / 2C..3C-1): the
// reference's add_bias and its two cache copies (gpt2_engine.c:184-196).
struct EpiG2Qkv {
    const float* bias;
    float* q;
    float* kc;
    float* vc;
    const int* step;
    int C;
    struct Pre {
        float b;
        int pos;
    };
    __device__ __forceinline__ void load(int, const int* rows, Pre& p) const {
        p.b = bias[rows[0]];
        p.pos = step[1];
    }
    __device__ __forceinline__ void operator()(int, const int* rows, const float* acc, const Pre& p) const {
        const int r = rows[0], pos = p.pos;
        const float v = acc[0] + p.b;
        if (r < C) q[r] = v;
        else if (r < 2 * C) kc[(size_t)pos * C + (r - C)] = v;
        else vc[(size_t)pos * C + (r - 2 * C)] = v;
    }
};

// y[r] = gelu(acc + bias[r]), the tanh form of the reference gelu kernel
// (gpt2_kernels.cu:199-206) with the arithmetic of the gelu kernel in gpt2_kernels.hip.
struct EpiBiasGelu {
    const float* bias;
    float* y;
    struct Pre {
        float b;
    };
    __device__ __forceinline__ void load(int, const int* rows, Pre& p) const { p.b = bias[rows[0]]; }
    __device__ __forceinline__ void operator()(int, const int* rows, const float* acc, const Pre& p) const {
#pragma clang fp contract(off)
        const int r = rows[0];
        const float v = acc[0] + p.b;
        const float t = 0.7978845608f * (v + 0.044715f * v * v * v);
        y[r] = 0.5f * v * (1.0f + tanhf(t));
    }
};

constexpr int kMaxCtx = 8192;    // longest cache the fused attention takes
constexpr int kAttnSplits = 32;  // position chunks per head at most (blocks per head in the grid)
constexpr int kAttnChunk = 256;  // positions per chunk before a second chunk is used
constexpr int kAttnMaxLen = kMaxCtx / kAttnSplits;   // longest chunk (256): scores kept in LDS

// Block max / sum over 256 threads (4 waves), result in every thread.
__device__ __forceinline__ float block_max256(float v, float* red) {
    v = sgpu_wave_max(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}
__device__ __forceinline__ float block_sum256(float v, float* red) {
    v = sgpu_wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// One query head over cached positions p0..p1-1 (p1 - p0 <= the length of sc): scores in
// sc, block max m and sum of exp(s - m) returned in every thread, and the exp-weighted sum of
// V returned in the lanes tid < HD (dim tid).  Scores: LPT lanes per position (DPL dims each),
// 256/LPT positions per pass, KU passes' K loads issued before any of their dot products.
// Mix: HD/4 lanes per cached row (a float4 of V each), 1024/HD rows per pass, VU passes' V
// loads issued before any of their FMAs; each lane sums its rows in position order, then the
// 1024/HD row slices are summed in slice order through part (1024 floats).  The round trips
// to the cache are per round of KU or VU passes, not per position.
template <int HD>
__device__ __forceinline__ float attn_chunk(const float* __restrict__ qh, const float* __restrict__ kg,
                                            const float* __restrict__ vg, int KVD, int p0, int p1, float scale,
                                            float* sc, float* red, float* part, float& m_out, float& sum_out) {
    constexpr int LPT = HD >= 64 ? HD / 16 : 4;   // lanes per position
    constexpr int DPL = HD / LPT;                  // dims per lane (16 or 8)
    constexpr int PPP = 256 / LPT;                 // positions per pass
    constexpr int KU = 4;                          // score passes per round
    constexpr int VL = HD / 4, VR = 256 / VL;      // mix: lanes per row, rows per pass
    constexpr int VU = HD >= 128 ? 8 : 16;         // mix passes per round
    const int tid = threadIdx.x;
    const int d0 = (tid % LPT) * DPL;
    float qv[DPL];
#pragma unroll
    for (int e = 0; e < DPL; e += 4) {
        const sgpu_f32x4 a = *reinterpret_cast<const sgpu_f32x4*>(qh + d0 + e);
#pragma unroll
        for (int i = 0; i < 4; i++) qv[e + i] = a[i];
    }
    const sgpu_f32x4 z4 = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int tb = p0; tb < p1; tb += PPP * KU) {
        sgpu_f32x4 kv[KU][DPL / 4];
#pragma unroll
        for (int u = 0; u < KU; u++) {
            const int t = tb + u * PPP + tid / LPT;
            const float* kr = kg + (size_t)t * KVD + d0;
#pragma unroll
            for (int e = 0; e < DPL / 4; e++) kv[u][e] = t < p1 ? *reinterpret_cast<const sgpu_f32x4*>(kr + 4 * e) : z4;
        }
#pragma unroll
        for (int u = 0; u < KU; u++) {
            const int t = tb + u * PPP + tid / LPT;
            float s = 0.0f;
#pragma unroll
            for (int e = 0; e < DPL / 4; e++)
#pragma unroll
                for (int i = 0; i < 4; i++) s = __builtin_fmaf(qv[4 * e + i], kv[u][e][i], s);
            s = sgpu_group_sum<LPT>(s);
            if (tid % LPT == LPT - 1 && t < p1) sc[t - p0] = s * scale;
        }
    }
    __syncthreads();
    const int n = p1 - p0;
    float m = -1e30f;
    for (int t = tid; t < n; t += 256) m = fmaxf(m, sc[t]);
    m = block_max256(m, red);
    float sum = 0.0f;
    for (int t = tid; t < n; t += 256) {
        const float e = expf(sc[t] - m);
        sc[t] = e;
        sum += e;
    }
    sum = block_sum256(sum, red);          // its barriers also publish sc[]
    const int vs = tid / VL, vq = tid % VL;
    sgpu_f32x4 acc = z4;
    for (int t0 = 0; t0 < n; t0 += VR * VU) {
        sgpu_f32x4 vv[VU];
        float w[VU];
#pragma unroll
        for (int u = 0; u < VU; u++) {
            const int t = t0 + u * VR + vs;
            vv[u] = t < n ? *reinterpret_cast<const sgpu_f32x4*>(vg + (size_t)(p0 + t) * KVD + 4 * vq) : z4;
            w[u] = t < n ? sc[t] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < VU; u++)
#pragma unroll
            for (int e = 0; e < 4; e++) acc[e] = __builtin_fmaf(w[u], vv[u][e], acc[e]);
    }
    *reinterpret_cast<sgpu_f32x4*>(&part[vs * HD + 4 * vq]) = acc;
    __syncthreads();
    float tot = 0.0f;
    if (tid < HD) {
#pragma unroll
        for (int s2 = 0; s2 < VR; s2++) tot += part[s2 * HD + tid];
    }
    m_out = m;
    sum_out = sum;
    return tot;
}

// Attention over T = pos + 1 cached positions, one 256-thread block per query head h and
// position chunk c (the launcher's grid covers NKV x kAttnSplits units of G = NH/NKV heads).  T <= kAttnChunk: one chunk per head and
// block (h, 0) computes the head as a whole (the other blocks exit).  Longer caches are cut
// into S = ceil(T / kAttnChunk) <= kAttnSplits chunks; each block writes its chunk's partial
// (max score m, sum of exp(s - m), the exp-weighted sum of V) to ws, and the last of the S
// blocks of head h to finish (per-head counter in cnt, reset by that block) combines them in
// chunk order: out = sum_c o_c e^(m_c - M) / sum_c l_c e^(m_c - M), M = max_c m_c.
template <int HD>
__device__ __forceinline__ void dec_attn(const float* __restrict__ q, const float* __restrict__ kc,
                                         const float* __restrict__ vc, float* __restrict__ out,
                                         const int* __restrict__ step, int NH, int NKV, float scale,
                                         float* __restrict__ ws, unsigned* __restrict__ cnt) {
    static_assert(HD == 32 || HD == 64 || HD == 128, "head dim");
    constexpr int WSTRIDE = HD + 2;                // ws record: o[HD], m, l
    __shared__ float sc[kAttnMaxLen];
    __shared__ float red[4];
    __shared__ __attribute__((aligned(16))) float part[1024];
    __shared__ int last_s;
    // Block b -> XCD b % 8 (blocks are dealt round-robin to the 8 XCDs).  The G query heads
    // that share KV group g and chunk c get the same b % 8, so the chunk's K and V come from
    // HBM once into that XCD's L2; units (g, c) are numbered chunk-major so chunk 0 of every
    // group is dispatched first.
    const int G = NH / NKV, tid = threadIdx.x;
    const int xcd = blockIdx.x % 8, i8 = blockIdx.x / 8;
    const int u = (i8 / G) * 8 + xcd;              // unit (g, c) = (u % NKV, u / NKV)
    const int g = u % NKV, c = u / NKV, h = g * G + i8 % G;
    const int T = min(step[1] + 1, kMaxCtx), KVD = NKV * HD;
    const int S = T <= kAttnChunk ? 1 : min(kAttnSplits, (T + kAttnChunk - 1) / kAttnChunk);
    if (c >= S) return;                            // block-uniform (c < kAttnSplits, see launcher)
    const int len = (T + S - 1) / S, p0 = c * len, p1 = min(T, p0 + len);   // p0 < p1 (see launcher)
    float m, sum;
    const float tot = attn_chunk<HD>(q + (size_t)h * HD, kc + (size_t)g * HD, vc + (size_t)g * HD, KVD, p0, p1,
                                     scale, sc, red, part, m, sum);
    const int slice = tid / HD, d = tid % HD;
    if (S == 1) {
        if (slice == 0) out[(size_t)h * HD + d] = tot / sum;
        return;
    }
    // Partials go to the head's last block by the hand-off protocol of sgpu_device.h
    // (device-coherent stores waited for, a per-head counter, an acquire by the last arriver).
    float* rec = ws + ((size_t)h * kAttnSplits + c) * WSTRIDE;
    if (slice == 0) __hip_atomic_store(rec + d, tot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (tid == 0) {
        __hip_atomic_store(rec + HD, m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(rec + HD + 1, sum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(0);          // this wave's partial stores are acknowledged
    __syncthreads();
    if (tid == 0) {
        last_s = __hip_atomic_fetch_add(cnt + h, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(S - 1);
        if (last_s) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");   // before the others' partials
    }
    __syncthreads();
    if (!last_s) return;
    // All S partials of head h into LDS with one round of device-coherent loads, then
    // combined in chunk order.
    __shared__ float stage[kAttnSplits * WSTRIDE];
    {
        const float* hr = ws + (size_t)h * kAttnSplits * WSTRIDE;
        const int nf = S * WSTRIDE;
        float r[(kAttnSplits * (HD + 2) + 255) / 256];
#pragma unroll
        for (int k = 0; k < (kAttnSplits * (HD + 2) + 255) / 256; k++) {
            const int i = tid + 256 * k;
            r[k] = i < nf ? __hip_atomic_load(hr + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < (kAttnSplits * (HD + 2) + 255) / 256; k++) {
            const int i = tid + 256 * k;
            if (i < nf) stage[i] = r[k];
        }
        __syncthreads();
    }
    if (slice == 0) {
        float M = -1e30f;
        for (int c2 = 0; c2 < S; c2++) M = fmaxf(M, stage[c2 * WSTRIDE + HD]);
        float L = 0.0f, O = 0.0f;
        for (int c2 = 0; c2 < S; c2++) {
            const float w = expf(stage[c2 * WSTRIDE + HD] - M);
            L = __builtin_fmaf(stage[c2 * WSTRIDE + HD + 1], w, L);
            O = __builtin_fmaf(stage[c2 * WSTRIDE + d], w, O);
        }
        out[(size_t)h * HD + d] = O / L;
    }
    if (tid == 0) __hip_atomic_store(cnt + h, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// (value, index) of the first maximum: larger value wins, equal values keep the lower index.
__device__ __forceinline__ void amax_merge(float& bv, int& bi, float ov, int oi) {
    if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
}
__device__ __forceinline__ void amax_block256(float& bv, int& bi, float* sv, int* si) {
    for (int off = 32; off > 0; off >>= 1) amax_merge(bv, bi, __shfl_xor(bv, off), __shfl_xor(bi, off));
    if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = bv; si[threadIdx.x >> 6] = bi; }
    __syncthreads();
    bv = sv[0];
    bi = si[0];
    for (int i = 1; i < 4; i++) amax_merge(bv, bi, sv[i], si[i]);
}

// Causal attention for prompt rows: block (h, t) is query head h of prompt row t (position
// pos0 + t, q rotated in place in the row's qkv vector of length QKVD), over cached positions
// 0..pos0+t; output row t of out (NH*HD floats per row).
template <int HD>
__device__ __forceinline__ void pf_attn(const float* __restrict__ qkv, const float* __restrict__ kc,
                                        const float* __restrict__ vc, float* __restrict__ out, int pos0, int NH,
                                        int NKV, float scale, int QKVD) {
    __shared__ float sc[kMaxCtx];
    __shared__ float red[4];
    __shared__ __attribute__((aligned(16))) float part[1024];
    const int h = blockIdx.x, t = blockIdx.y, KVD = NKV * HD, g = h / (NH / NKV);
    const int n = min(pos0 + t + 1, kMaxCtx);
    float m, sum;
    const float tot = attn_chunk<HD>(qkv + (size_t)t * QKVD + (size_t)h * HD, kc + (size_t)g * HD,
                                     vc + (size_t)g * HD, KVD, 0, n, scale, sc, red, part, m, sum);
    if (threadIdx.x < HD) out[(size_t)t * NH * HD + (size_t)h * HD + threadIdx.x] = tot / sum;
}

}  // namespace

using sgpu::WF16;
using sgpu::WF32;

extern "C" {

// x[i] = h2f(emb[token*C + i]); step = {token, pos} for the kernels that follow.
__global__ void sgpu_dec_embed(const uint16_t* __restrict__ emb, int token, int pos, float* __restrict__ x, int C,
                               int* __restrict__ step) {
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        step[0] = token;
        step[1] = pos;
    }
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < C; i += gridDim.x * blockDim.x)
        x[i] = sgpu_h2f(emb[(size_t)token * C + i]);
}

// GPT-2: x = wte[token] + wpe[pos] (fp32; the reference adds on the host,
// gpt2_engine.c:176-179); step = {token, pos}.
__global__ void sgpu_dec_g2embed(const float* __restrict__ wte, const float* __restrict__ wpe, int token, int pos,
                                 float* __restrict__ x, int C, int* __restrict__ step) {
#pragma clang fp contract(off)
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        step[0] = token;
        step[1] = pos;
    }
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < C; i += gridDim.x * blockDim.x)
        x[i] = wte[(size_t)token * C + i] + wpe[(size_t)pos * C + i];
}

// First-max argmax over n logits (qwen_engine.c:360-364 tie rule), stage 1: each of the
// grid's blocks (256 threads) reduces a contiguous chunk to one (value, index) pair.
__global__ void __launch_bounds__(256) sgpu_dec_argmax_part(const float* __restrict__ v, int n,
                                                            float* __restrict__ pv, int* __restrict__ pi) {
    __shared__ float sv[4];
    __shared__ int si[4];
    const int chunk = (n + gridDim.x - 1) / gridDim.x;
    const int lo = blockIdx.x * chunk, hi = min(n, lo + chunk);
    float best = -INFINITY;
    int idx = 0x7fffffff;
    for (int i = lo + (int)threadIdx.x; i < hi; i += 256)
        if (v[i] > best) { best = v[i]; idx = i; }
    amax_block256(best, idx, sv, si);
    if (threadIdx.x == 0) { pv[blockIdx.x] = best; pi[blockIdx.x] = idx; }
}

// Stage 2, one block of 256 threads over np <= 256 partials, fused with the next step's
// embedding: the index goes to step[0] and, if out != NULL, to out[step[1] + 1]; then the
// position advances (step[1] + 1) and x becomes the new token's embedding -- h2f(emb[token])
// (Qwen) or wte[token] + wpe[position] (GPT-2, skipped once the position reaches ctx).
__device__ __forceinline__ int amax_final(const float* __restrict__ pv, const int* __restrict__ pi, int np) {
    __shared__ float sv[4];
    __shared__ int si[4];
    float best = -INFINITY;
    int idx = 0x7fffffff;
    if ((int)threadIdx.x < np) { best = pv[threadIdx.x]; idx = pi[threadIdx.x]; }
    amax_block256(best, idx, sv, si);
    return idx == 0x7fffffff ? 0 : idx;
}
__global__ void __launch_bounds__(256) sgpu_dec_argmax_embed(const float* __restrict__ pv, const int* __restrict__ pi,
                                                             int np, int* __restrict__ step, int* __restrict__ out,
                                                             const uint16_t* __restrict__ emb, float* __restrict__ x,
                                                             int C) {
    __shared__ int pos;
    const int idx = amax_final(pv, pi, np);
    if (threadIdx.x == 0) {
        pos = step[1];
        step[0] = idx;
        if (out) out[pos + 1] = idx;
        step[1] = pos + 1;
    }
    for (int i = threadIdx.x; i < C; i += blockDim.x) x[i] = sgpu_h2f(emb[(size_t)idx * C + i]);
}
__global__ void __launch_bounds__(256) sgpu_dec_argmax_g2embed(const float* __restrict__ pv, const int* __restrict__ pi,
                                                               int np, int* __restrict__ step, int* __restrict__ out,
                                                               const float* __restrict__ wte,
                                                               const float* __restrict__ wpe, float* __restrict__ x,
                                                               int C, int ctx) {
#pragma clang fp contract(off)
    __shared__ int pos;
    const int idx = amax_final(pv, pi, np);
    if (threadIdx.x == 0) {
        pos = step[1] + 1;
        step[0] = idx;
        if (out) out[pos] = idx;
        step[1] = pos;
    }
    __syncthreads();
    if (pos < ctx)
        for (int i = threadIdx.x; i < C; i += blockDim.x) x[i] = wte[(size_t)idx * C + i] + wpe[(size_t)pos * C + i];
}

// ---- batched prompt prefill (T rows at positions pos0..pos0+T-1) ----

// x[t] = h2f(emb[ids[t]]) for the T rows.
__global__ void sgpu_pf_embed(const uint16_t* __restrict__ emb, const int* __restrict__ ids, int T,
                              float* __restrict__ x, int C) {
    const long long total = (long long)T * C;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total; i += (long long)gridDim.x * blockDim.x) {
        const int t = (int)(i / C), k = (int)(i % C);
        x[i] = sgpu_h2f(emb[(size_t)ids[t] * C + k]);
    }
}

// Y[t][n] = sum_k X[t][k] * h2f(W[n][k]) + bias?[n] on the fp32 matrix cores (one block per
// 32-token x 32-row tile and k-split, grid-stride over units; blockDim 256, K % 4 == 0,
// 16-byte X rows).  S > 1 splits each tile's K over S blocks (ws: S * tiles * 1024 floats,
// cnt: one zeroed counter per tile, left at zero).  accum != 0: Y += result (the residual).
__global__ void __launch_bounds__(256) sgpu_pf_gemm(const uint16_t* __restrict__ W, const float* __restrict__ X,
                                                    const float* __restrict__ bias, float* __restrict__ Y, int K,
                                                    int N, int T, int S, float* __restrict__ ws,
                                                    unsigned* __restrict__ cnt, int accum) {
    if (blockDim.x != 256) return;
    sgpu::gemm_nt_mfma<1, WF16, true>(W, X, bias, Y, K, N, T, S, ws, cnt, accum);
}

// Per prompt row t (position pos0 + t) of the qkv matrix (rows of QKVD = (NH + 2*NKV)*HD):
// RoPE on the q heads in place, RoPE on the k heads into the key cache, v into the value
// cache (qwen_engine.c:227-230 order and rotation, the rope kernel's arithmetic).
__global__ void sgpu_pf_qkv_post(float* __restrict__ qkv, int T, int pos0, const float* __restrict__ cosT,
                                 const float* __restrict__ sinT, float* __restrict__ kc, float* __restrict__ vc,
                                 int NH, int NKV, int HD) {
#pragma clang fp contract(off)
    const int hd2 = HD / 2, KVD = NKV * HD, QKVD = (NH + 2 * NKV) * HD;
    const int per = (NH + NKV) * hd2 + KVD;          // work items per row: q pairs, k pairs, v
    const long long total = (long long)T * per;
    for (long long idx = blockIdx.x * (long long)blockDim.x + threadIdx.x; idx < total;
         idx += (long long)gridDim.x * blockDim.x) {
        const int t = (int)(idx / per), r = (int)(idx % per), pos = pos0 + t;
        float* row = qkv + (size_t)t * QKVD;
        if (r < (NH + NKV) * hd2) {
            const int hh = r / hd2, i = r % hd2;     // heads 0..NH-1 are q, NH.. are k
            const float a = row[hh * HD + i], b = row[hh * HD + hd2 + i];
            const float c = cosT[(size_t)pos * hd2 + i], sn = sinT[(size_t)pos * hd2 + i];
            const float o0 = a * c - b * sn, o1 = a * sn + b * c;
            if (hh < NH) {
                row[hh * HD + i] = o0;
                row[hh * HD + hd2 + i] = o1;
            } else {
                float* kr = kc + (size_t)pos * KVD + (hh - NH) * HD;
                kr[i] = o0;
                kr[hd2 + i] = o1;
            }
        } else {
            const int j = r - (NH + NKV) * hd2;
            vc[(size_t)pos * KVD + j] = row[(NH + NKV) * HD + j];
        }
    }
}

__global__ void __launch_bounds__(256) sgpu_pf_attn64(const float* __restrict__ qkv, const float* __restrict__ kc,
                                                      const float* __restrict__ vc, float* __restrict__ out, int pos0,
                                                      int NH, int NKV, float scale, int QKVD) {
    pf_attn<64>(qkv, kc, vc, out, pos0, NH, NKV, scale, QKVD);
}
__global__ void __launch_bounds__(256) sgpu_pf_attn32(const float* __restrict__ qkv, const float* __restrict__ kc,
                                                      const float* __restrict__ vc, float* __restrict__ out, int pos0,
                                                      int NH, int NKV, float scale, int QKVD) {
    pf_attn<32>(qkv, kc, vc, out, pos0, NH, NKV, scale, QKVD);
}
__global__ void __launch_bounds__(256) sgpu_pf_attn128(const float* __restrict__ qkv, const float* __restrict__ kc,
                                                       const float* __restrict__ vc, float* __restrict__ out, int pos0,
                                                       int NH, int NKV, float scale, int QKVD) {
    pf_attn<128>(qkv, kc, vc, out, pos0, NH, NKV, scale, QKVD);
}

// G[t][i] = silu(Y[t][i]) * Y[t][FC + i] for gate|up rows of 2*FC (the swiglu kernel's
// arithmetic, qwen_kernels.cu:119-126).
__global__ void sgpu_pf_swiglu(const float* __restrict__ Y, float* __restrict__ G, int FC, int T) {
#pragma clang fp contract(off)
    const long long total = (long long)T * FC;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total; i += (long long)gridDim.x * blockDim.x) {
        const int t = (int)(i / FC), k = (int)(i % FC);
        const float gv = Y[(size_t)t * 2 * FC + k];
        G[i] = (gv / (1.0f + expf(-gv))) * Y[(size_t)t * 2 * FC + FC + k];
    }
}

__global__ void __launch_bounds__(256) sgpu_dec_attn64(const float* __restrict__ q, const float* __restrict__ kc,
                                                       const float* __restrict__ vc, float* __restrict__ out,
                                                       const int* __restrict__ step, int NH, int NKV, float scale,
                                                       float* __restrict__ ws, unsigned* __restrict__ cnt) {
    dec_attn<64>(q, kc, vc, out, step, NH, NKV, scale, ws, cnt);
}
__global__ void __launch_bounds__(256) sgpu_dec_attn32(const float* __restrict__ q, const float* __restrict__ kc,
                                                       const float* __restrict__ vc, float* __restrict__ out,
                                                       const int* __restrict__ step, int NH, int NKV, float scale,
                                                       float* __restrict__ ws, unsigned* __restrict__ cnt) {
    dec_attn<32>(q, kc, vc, out, step, NH, NKV, scale, ws, cnt);
}
__global__ void __launch_bounds__(256) sgpu_dec_attn128(const float* __restrict__ q, const float* __restrict__ kc,
                                                        const float* __restrict__ vc, float* __restrict__ out,
                                                        const int* __restrict__ step, int NH, int NKV, float scale,
                                                       float* __restrict__ ws, unsigned* __restrict__ cnt) {
    dec_attn<128>(q, kc, vc, out, step, NH, NKV, scale, ws, cnt);
}

}  // extern "C"

// ---- GEMV families, one instantiation per (lanes per team, segments per lane) ----
#define SGPU_DEC_QKV(LPR, S)                                                                                   \
    extern "C" __global__ void __launch_bounds__(256) sgpu_dec_qkv_l##LPR##_s##S(                              \
        const uint16_t* __restrict__ W, int K, int nteams, const float* __restrict__ x,                        \
        const uint16_t* __restrict__ lnw, float eps, const float* __restrict__ bias, float* q, float* kc,      \
        float* vc, const float* __restrict__ cosT, const float* __restrict__ sinT, const int* __restrict__ step, \
        int NH, int NKV, int HD) {                                                                             \
        sgpu::gemv_team<WF16, LPR, S, 2>(W, K, nteams, sgpu::XRms{x, lnw, eps, 0.0f}, sgpu::MapHalfPairs{HD / 2}, \
                                         EpiQkvRope{bias, q, kc, vc, cosT, sinT, step, NH, NKV, HD});         \
    }
#define SGPU_DEC_GATEUP(LPR, S)                                                                                \
    extern "C" __global__ void __launch_bounds__(256) sgpu_dec_gateup_l##LPR##_s##S(                           \
        const uint16_t* __restrict__ W, int K, int FC, const float* __restrict__ x,                            \
        const uint16_t* __restrict__ lnw, float eps, float* __restrict__ y) {                                  \
        sgpu::gemv_team<WF16, LPR, S, 2>(W, K, FC, sgpu::XRms{x, lnw, eps, 0.0f}, sgpu::MapPair{FC},           \
                                         EpiSwiGLU{y});                                                        \
    }
#define SGPU_DEC_RES(LPR, S)                                                                                   \
    extern "C" __global__ void __launch_bounds__(256) sgpu_dec_res_l##LPR##_s##S(                              \
        const uint16_t* __restrict__ W, int K, int N, const float* __restrict__ a, const float* bias, float* x) { \
        sgpu::gemv_team<WF16, LPR, S, 1>(W, K, N, sgpu::XPlain{a}, sgpu::MapRows{}, EpiResidual{x, bias, x});  \
    }
#define SGPU_DEC_LMHEAD(LPR, S)                                                                                \
    extern "C" __global__ void __launch_bounds__(256) sgpu_dec_lmhead_l##LPR##_s##S(                           \
        const uint16_t* __restrict__ W, int K, int N, const float* __restrict__ x,                             \
        const uint16_t* __restrict__ lnw, float eps, float* __restrict__ y) {                                  \
        sgpu::gemv_team<WF16, LPR, S, 1>(W, K, N, sgpu::XRms{x, lnw, eps, 0.0f}, sgpu::MapRows{},              \
                                         sgpu::EpiStore{nullptr, y});                                          \
    }

// GPT-2 (fp32 weights): LayerNorm + qkv + bias + KV-cache write; GEMV + bias + residual
// (attention output and MLP projections); LayerNorm + fc + bias + GELU; LayerNorm + tied
// lm_head.
#define SGPU_DEC_G2QKV(LPR, S)                                                                                 \
    extern "C" __global__ void __launch_bounds__(256) sgpu_dec_g2qkv_l##LPR##_s##S(                            \
        const float* __restrict__ W, int K, int N, const float* __restrict__ x, const float* __restrict__ lnw, \
        const float* __restrict__ lnb, float eps, const float* __restrict__ bias, float* q, float* kc, float* vc, \
        const int* __restrict__ step) {                                                                        \
        sgpu::gemv_team<WF32, LPR, S, 1>(W, K, N, sgpu::XLn{x, lnw, lnb, eps, 0.0f, 0.0f}, sgpu::MapRows{},    \
                                         EpiG2Qkv{bias, q, kc, vc, step, K});                                 \
    }
#define SGPU_DEC_G2RES(LPR, S)                                                                                 \
    extern "C" __global__ void __launch_bounds__(256) sgpu_dec_g2res_l##LPR##_s##S(                            \
        const float* __restrict__ W, int K, int N, const float* __restrict__ a, const float* bias, float* x) {  \
        sgpu::gemv_team<WF32, LPR, S, 1>(W, K, N, sgpu::XPlain{a}, sgpu::MapRows{}, EpiResidual{x, bias, x});  \
    }
#define SGPU_DEC_G2FC(LPR, S)                                                                                  \
    extern "C" __global__ void __launch_bounds__(256) sgpu_dec_g2fc_l##LPR##_s##S(                             \
        const float* __restrict__ W, int K, int N, const float* __restrict__ x, const float* __restrict__ lnw, \
        const float* __restrict__ lnb, float eps, const float* __restrict__ bias, float* __restrict__ y) {     \
        sgpu::gemv_team<WF32, LPR, S, 1>(W, K, N, sgpu::XLn{x, lnw, lnb, eps, 0.0f, 0.0f}, sgpu::MapRows{},    \
                                         EpiBiasGelu{bias, y});                                                \
    }
#define SGPU_DEC_G2LMHEAD(LPR, S)                                                                              \
    extern "C" __global__ void __launch_bounds__(256) sgpu_dec_g2lmhead_l##LPR##_s##S(                         \
        const float* __restrict__ W, int K, int N, const float* __restrict__ x, const float* __restrict__ lnw, \
        const float* __restrict__ lnb, float eps, float* __restrict__ y) {                                     \
        sgpu::gemv_team<WF32, LPR, S, 1>(W, K, N, sgpu::XLn{x, lnw, lnb, eps, 0.0f, 0.0f}, sgpu::MapRows{},    \
                                         sgpu::EpiStore{nullptr, y});                                          \
    }

#define SGPU_DEC_PAIRS(F) F(16, 1) F(16, 2) F(16, 4) F(16, 7) F(16, 8) F(64, 1) F(64, 2) F(64, 4) F(64, 8)
#define SGPU_DEC_SINGLE(F) SGPU_DEC_PAIRS(F) F(256, 1) F(256, 2) F(256, 3) F(256, 4) F(256, 8) F(64, 10)

SGPU_DEC_PAIRS(SGPU_DEC_QKV)
SGPU_DEC_PAIRS(SGPU_DEC_GATEUP)
SGPU_DEC_SINGLE(SGPU_DEC_RES)
SGPU_DEC_SINGLE(SGPU_DEC_LMHEAD)
SGPU_DEC_SINGLE(SGPU_DEC_G2QKV)
SGPU_DEC_SINGLE(SGPU_DEC_G2RES)
SGPU_DEC_SINGLE(SGPU_DEC_G2FC)
SGPU_DEC_SINGLE(SGPU_DEC_G2LMHEAD)
