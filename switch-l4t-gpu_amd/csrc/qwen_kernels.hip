// qwen_kernels.hip -- the Qwen2.5 engine's code object (reference
// gpu-llm/kernels/qwen_kernels.cu:34-189), gfx950.
//
// Symbols and arguments as the reference; activations fp32, weights fp16 bits decoded with
// the reference's h2f contract (subnormals -> +0, exponent 31 finite):
//   gemv_h          (const u16*W, const float*x, const float*bias, float*y, int K, int N)
//   gemv_hh         (const u16*W, const u16*x, const float*bias, float*y, int K, int N)
//                   the fp16-x form of gemv_h (no reference counterpart): x holds fp16 bit
//                   patterns decoded with the same h2f contract as W, fp32 accumulate
//   rmsnorm         (const float*x, const u16*w, float*y, int n, float eps)   grid = rows
//   rope            (float*x, const float*cosT, const float*sinT, int T, int H, int HD, int pos0)
//   swiglu          (const float*g, const float*u, float*y, int n)
//   attn_scores_gqa (const float*q, const float*kc, float*scores, int T, float scale, int NH, int KV, int HD)
//   attn_softmax    (const float*scores, float*probs, int T, int NH)
//   attn_mix_gqa    (const float*probs, const float*vc, float*out, int T, int NH, int KV, int HD)
//   add2            (const float*a, const float*b, float*out, int n)
// gemv_h / gemv_hh take any grid of blocks of up to 256 threads (gemv_core.h gemv_byname).
// The support kernels expect the geometry their
// launchers in the host library use (blocks of 256 threads; one wave per head for
// attn_softmax).  Elementwise arithmetic is written with contraction off so it rounds like
// the serial CPU golden; exp is the correctly-rounded-to-1-ulp device expf (the reference's
// 4-term polynomial, qwen_kernels.cu:18-29, is ~0.08% off and is not reproduced).
#include "gemv_core.h"

extern "C" {

__global__ void __launch_bounds__(256) gemv_h(const uint16_t* __restrict__ W, const float* __restrict__ x,
                       const float* __restrict__ bias, float* __restrict__ y, int K, int N) {
    sgpu::gemv_byname<sgpu::WF16, float>(W, x, bias, y, K, N);
}

// y[n] = sum_k h2f(W[n*K+k]) * h2f(x[k]) + (bias ? bias[n] : 0): gemv_h's contract with x
// stored as fp16 bits (half the x bytes; activations kept in fp16).  Any grid.
__global__ void __launch_bounds__(256) gemv_hh(const uint16_t* __restrict__ W, const uint16_t* __restrict__ x,
                        const float* __restrict__ bias, float* __restrict__ y, int K, int N) {
    sgpu::gemv_byname<sgpu::WF16, uint16_t>(W, x, bias, y, K, N);
}

// One block per row (grid = rows), blockDim a multiple of 64 (256 from the launcher).
__global__ void __launch_bounds__(1024) rmsnorm(const float* __restrict__ x, const uint16_t* __restrict__ w,
                                                float* __restrict__ y, int n, float eps) {
#pragma clang fp contract(off)
    __shared__ float red[16];
    __shared__ float s_ss;
    const int tid = threadIdx.x, nt = blockDim.x;
    x += (size_t)blockIdx.x * n;
    y += (size_t)blockIdx.x * n;
    float local = 0.0f;
    for (int i = tid; i < n; i += nt) local += x[i] * x[i];
    local = sgpu_group_sum<64>(local);
    if ((tid & 63) == 63) red[tid >> 6] = local;
    __syncthreads();
    if (tid == 0) {
        float s = 0.0f;
        for (int i = 0; i < (nt >> 6); i++) s += red[i];
        s_ss = s / (float)n;
    }
    __syncthreads();
    const float inv = 1.0f / __builtin_sqrtf(s_ss + eps);
    for (int i = tid; i < n; i += nt) y[i] = x[i] * inv * sgpu_h2f(w[i]);
}

// Half-split rotation of every (i, i+HD/2) pair of every head of T rows at positions
// pos0..pos0+T-1 (qwen_kernels.cu:95-116).
__global__ void rope(float* __restrict__ x, const float* __restrict__ cosT, const float* __restrict__ sinT,
                     int T, int H, int HD, int pos0) {
#pragma clang fp contract(off)
    const int hd2 = HD / 2;
    const int total = T * H * hd2;
    for (int idx = blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += gridDim.x * blockDim.x) {
        const int t = idx / (H * hd2), r = idx % (H * hd2);
        const int h = r / hd2, i = r % hd2;
        float* row = x + (size_t)t * H * HD;
        const float a = row[h * HD + i], b = row[h * HD + hd2 + i];
        const float c = cosT[(size_t)(pos0 + t) * hd2 + i], s = sinT[(size_t)(pos0 + t) * hd2 + i];
        row[h * HD + i] = a * c - b * s;
        row[h * HD + hd2 + i] = a * s + b * c;
    }
}

__global__ void swiglu(const float* __restrict__ g, const float* __restrict__ u, float* __restrict__ y, int n) {
#pragma clang fp contract(off)
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        const float gv = g[i];
        y[i] = (gv / (1.0f + expf(-gv))) * u[i];
    }
}

// scores[t*NH + h] = (q_h . k_{t,g}) * scale, g = h / (NH/NKV), NKV = KV/HD.  Serial d order.
__global__ void attn_scores_gqa(const float* __restrict__ q, const float* __restrict__ kc,
                                float* __restrict__ scores, int T, float scale, int NH, int KV, int HD) {
#pragma clang fp contract(off)
    const int grp = NH / (KV / HD);
    for (int idx = blockIdx.x * blockDim.x + threadIdx.x; idx < T * NH; idx += gridDim.x * blockDim.x) {
        const int t = idx / NH, h = idx % NH, g = h / grp;
        const float* qp = q + (size_t)h * HD;
        const float* kp = kc + (size_t)t * KV + (size_t)g * HD;
        float acc = 0.0f;
        for (int d = 0; d < HD; d++) acc += qp[d] * kp[d];
        scores[idx] = acc * scale;
    }
}

// Softmax over t for each head: one wave per head (grid-stride over heads by wave).
// probs = exp(s - max) / sum, the division form of the CPU golden (qwen_engine.c:339).
__global__ void __launch_bounds__(256) attn_softmax(const float* __restrict__ scores, float* __restrict__ probs,
                                                    int T, int NH) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int nwaves = (gridDim.x * blockDim.x) >> 6;
    for (int h = wave; h < NH; h += nwaves) {
        float m = -1e30f;
        for (int t = lane; t < T; t += 64) m = fmaxf(m, scores[(size_t)t * NH + h]);
        m = sgpu_wave_max(m);
        float s = 0.0f;
        for (int t = lane; t < T; t += 64) {
            const float e = expf(scores[(size_t)t * NH + h] - m);
            probs[(size_t)t * NH + h] = e;
            s += e;
        }
        s = sgpu_wave_sum(s);
        for (int t = lane; t < T; t += 64) probs[(size_t)t * NH + h] = probs[(size_t)t * NH + h] / s;
    }
}

// out[h*HD + d] = sum_t probs[t*NH + h] * vc[t*KV + g*HD + d], serial in t.
__global__ void attn_mix_gqa(const float* __restrict__ probs, const float* __restrict__ vc,
                             float* __restrict__ out, int T, int NH, int KV, int HD) {
#pragma clang fp contract(off)
    const int grp = NH / (KV / HD);
    for (int idx = blockIdx.x * blockDim.x + threadIdx.x; idx < NH * HD; idx += gridDim.x * blockDim.x) {
        const int h = idx / HD, d = idx % HD, g = h / grp;
        float acc = 0.0f;
        for (int t = 0; t < T; t++) acc += probs[(size_t)t * NH + h] * vc[(size_t)t * KV + (size_t)g * HD + d];
        out[idx] = acc;
    }
}

__global__ void add2(const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ out, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) out[i] = a[i] + b[i];
}

}  // extern "C"
