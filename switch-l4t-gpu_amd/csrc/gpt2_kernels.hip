// gpt2_kernels.hip -- the GPT-2 engine's code object (reference
// gpu-llm/kernels/gpt2_kernels.cu:38-268), gfx950.  fp32 throughout.
//
//   gemv_warp    (W, x, y, K, N)              y = W x                 (gpt2_kernels.cu:38-72)
//   gemv_warp_b  (W, x, bias, y, K, N)        y = W x + bias          (gpt2_kernels.cu:75-108)
//   gemv_multi   (W, X, bias, Y, K, N, T)     Y[t] = W X[t] + bias?   (gpt2_kernels.cu:110-155)
//   layernorm    (x, w, b, y, n, eps)         grid = rows             (gpt2_kernels.cu:160-196)
//   gelu         (x, y, n)                    tanh form               (gpt2_kernels.cu:199-206)
//   add_bias     (y, b, n)                    y += b                  (gpt2_kernels.cu:209-212)
//   add2         (a, b, out, n)               out = a + b             (gpt2_kernels.cu:213-217)
//   attn_scores  (q, kcache, scores, T, scale)                        (gpt2_kernels.cu:221-234)
//   attn_softmax (scores, probs, T)                                   (gpt2_kernels.cu:238-253)
//   attn_mix     (probs, vcache, out, T)                              (gpt2_kernels.cu:258-268)
// The attention kernels keep the reference's fixed GPT-2 124M head layout (12 heads of 64,
// rows of 768).  bias is nullable in the GEMVs.  The GEMVs take any grid (wave-granular
// grid-stride); the support kernels expect their launchers' geometry (256-thread blocks;
// attn_softmax one wave per head).  Elementwise arithmetic rounds like the serial CPU
// golden (contraction off); tanh/exp are the device libm functions, not the reference's
// local polynomials (gpt2_kernels.cu:12-34).
#include "gemv_core.h"

namespace {
constexpr int kHeads = 12, kHeadDim = 64, kWidth = kHeads * kHeadDim;   // gpt2_kernels.cu:5

// Sum over a block of up to 1024 threads (multiple of 64); result returned to every thread.
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = sgpu_group_sum<64>(v);
    const int tid = threadIdx.x, nw = blockDim.x >> 6;
    __syncthreads();                                   // red reused across calls
    if ((tid & 63) == 63) red[tid >> 6] = v;
    __syncthreads();
    float s = 0.0f;
    for (int i = 0; i < nw; i++) s += red[i];
    return s;
}
}  // namespace

extern "C" {

__global__ void __launch_bounds__(256) gemv_warp(const float* __restrict__ W, const float* __restrict__ x, float* __restrict__ y,
                          int K, int N) {
    sgpu::gemv_byname<sgpu::WF32, float>(W, x, nullptr, y, K, N);
}

__global__ void __launch_bounds__(256) gemv_warp_b(const float* __restrict__ W, const float* __restrict__ x,
                            const float* __restrict__ bias, float* __restrict__ y, int K, int N) {
    sgpu::gemv_byname<sgpu::WF32, float>(W, x, bias, y, K, N);
}

// Matrix-core path (32-token x 32-row tiles) for whole-quad aligned rows, 256-thread blocks
// and four or more tokens; otherwise the wave-per-row vector path (any K, alignment, block
// size, token count).
__global__ void __launch_bounds__(256) gemv_multi(const float* __restrict__ W, const float* __restrict__ X,
                                                  const float* __restrict__ bias, float* __restrict__ Y,
                                                  int K, int N, int T) {
    if (sgpu::gemm_nt_ok(W, X, K, T))
        sgpu::gemm_nt_mfma<1>(W, X, bias, Y, K, N, T);
    else
        sgpu::gemv_multi_f32<16>(W, X, bias, Y, K, N, T);
}

// gemv_multi with each 32x32 tile's K split S ways across blocks (grid = tiles * S): the
// matrix-core path for problems with too few tiles to fill the CUs.  Same operand
// conditions as gemv_multi's matrix-core path (checked by the launcher); ws holds
// S * tiles * 1024 floats, cnt one zeroed counter per tile (left at zero).
__global__ void __launch_bounds__(256) gemv_multi_splitk(const float* __restrict__ W, const float* __restrict__ X,
                                                         const float* __restrict__ bias, float* __restrict__ Y,
                                                         int K, int N, int T, int S, float* __restrict__ ws,
                                                         unsigned* __restrict__ cnt) {
    if (blockDim.x != 256) return;
    sgpu::gemm_nt_mfma<1, sgpu::WF32, true>(W, X, bias, Y, K, N, T, S, ws, cnt);
}

// gemv_multi for 1..8 tokens on aligned rows: the register-resident team GEMV with eight
// input vectors, a wave per row for K <= 1024 and a block per row for K <= 4096 (launcher's
// choice; any grid of 256-thread blocks).
__global__ void __launch_bounds__(256) gemv_multi_x8_l64(const float* __restrict__ W, const float* __restrict__ X,
                                                         const float* __restrict__ bias, float* __restrict__ Y,
                                                         int K, int N, int T) {
    if (blockDim.x != 256) return;
    sgpu::gemv_multi_xreg<64, 4, 8>(W, X, bias, Y, K, N, T);
}
__global__ void __launch_bounds__(256) gemv_multi_x8_l256(const float* __restrict__ W, const float* __restrict__ X,
                                                          const float* __restrict__ bias, float* __restrict__ Y,
                                                          int K, int N, int T) {
    if (blockDim.x != 256) return;
    sgpu::gemv_multi_xreg<256, 4, 8>(W, X, bias, Y, K, N, T);
}

// y = (x - mean) / sqrt(var + eps) * w + b per row (grid = rows), with the two-pass
// mean/variance of the CPU golden (gpt2_engine.c:331-339).
__global__ void __launch_bounds__(1024) layernorm(const float* __restrict__ x, const float* __restrict__ w,
                                                  const float* __restrict__ b, float* __restrict__ y, int n,
                                                  float eps) {
#pragma clang fp contract(off)
    __shared__ float red[16];
    const int tid = threadIdx.x, nt = blockDim.x;
    x += (size_t)blockIdx.x * n;
    y += (size_t)blockIdx.x * n;
    float s = 0.0f;
    for (int i = tid; i < n; i += nt) s += x[i];
    const float mean = block_sum(s, red) / (float)n;
    float q = 0.0f;
    for (int i = tid; i < n; i += nt) {
        const float d = x[i] - mean;
        q += d * d;
    }
    const float var = block_sum(q, red) / (float)n;
    const float inv = 1.0f / __builtin_sqrtf(var + eps);
    for (int i = tid; i < n; i += nt) y[i] = (x[i] - mean) * inv * w[i] + b[i];
}

__global__ void gelu(const float* __restrict__ x, float* __restrict__ y, int n) {
#pragma clang fp contract(off)
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        const float v = x[i];
        const float t = 0.7978845608f * (v + 0.044715f * v * v * v);
        y[i] = 0.5f * v * (1.0f + tanhf(t));
    }
}

__global__ void add_bias(float* __restrict__ y, const float* __restrict__ b, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) y[i] += b[i];
}

__global__ void add2(const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ out, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) out[i] = a[i] + b[i];
}

// scores[t*12 + h] = (q_h . k_{t,h}) * scale, serial d order.
__global__ void attn_scores(const float* __restrict__ q, const float* __restrict__ kcache,
                            float* __restrict__ scores, int T, float scale) {
#pragma clang fp contract(off)
    for (int idx = blockIdx.x * blockDim.x + threadIdx.x; idx < T * kHeads; idx += gridDim.x * blockDim.x) {
        const int t = idx / kHeads, h = idx % kHeads;
        const float* qh = q + h * kHeadDim;
        const float* kh = kcache + (size_t)t * kWidth + h * kHeadDim;
        float acc = 0.0f;
        for (int d = 0; d < kHeadDim; d++) acc += qh[d] * kh[d];
        scores[idx] = acc * scale;
    }
}

// Softmax over t per head, a wave per head: probs = exp(s - max) / sum.
__global__ void __launch_bounds__(256) attn_softmax(const float* __restrict__ scores, float* __restrict__ probs,
                                                    int T) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int nwaves = (gridDim.x * blockDim.x) >> 6;
    for (int h = wave; h < kHeads; h += nwaves) {
        float m = -1e30f;
        for (int t = lane; t < T; t += 64) m = fmaxf(m, scores[(size_t)t * kHeads + h]);
        m = sgpu_wave_max(m);
        float s = 0.0f;
        for (int t = lane; t < T; t += 64) {
            const float e = expf(scores[(size_t)t * kHeads + h] - m);
            probs[(size_t)t * kHeads + h] = e;
            s += e;
        }
        s = sgpu_wave_sum(s);
        for (int t = lane; t < T; t += 64) probs[(size_t)t * kHeads + h] = probs[(size_t)t * kHeads + h] / s;
    }
}

// out[d] = sum_t probs[t*12 + d/64] * vcache[t*768 + d], serial in t.
__global__ void attn_mix(const float* __restrict__ probs, const float* __restrict__ vcache,
                         float* __restrict__ out, int T) {
#pragma clang fp contract(off)
    for (int d = blockIdx.x * blockDim.x + threadIdx.x; d < kWidth; d += gridDim.x * blockDim.x) {
        const int h = d / kHeadDim;
        float acc = 0.0f;
        for (int t = 0; t < T; t++) acc += probs[(size_t)t * kHeads + h] * vcache[(size_t)t * kWidth + d];
        out[d] = acc;
    }
}

}  // extern "C"
