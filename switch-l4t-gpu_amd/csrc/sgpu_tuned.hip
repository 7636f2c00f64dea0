// sgpu_tuned.hip -- tuned GEMV instantiations the host launchers pick from (gfx950).
//
//   sgpu_gemv_f32_l<LPR>_s<S>(const float*W,  const float*x, const float*bias, float*y, int K, int N)
//   sgpu_gemv_h_l<LPR>_s<S>  (const u16*W,    const float*x, const float*bias, float*y, int K, int N)
//   sgpu_gemv_hh_l<LPR>_s<S> (const u16*W,    const u16*x,   const float*bias, float*y, int K, int N)
//     (fp16 x, decoded with the reference h2f; fp32 accumulate)
//
// LPR = lanes per row (16, 64, or 256 = four waves split-K), S = 16-byte segments per lane.
// Launch: blocks of 256 threads; preconditions in gemv_core.h (gemv_xreg).
#include "gemv_core.h"

#define SGPU_GEMV_INST(LPR, S)                                                                     \
    extern "C" __global__ void __launch_bounds__(256) sgpu_gemv_f32_l##LPR##_s##S(                 \
        const float* __restrict__ W, const float* __restrict__ x, const float* __restrict__ bias,  \
        float* __restrict__ y, int K, int N) {                                                     \
        sgpu::gemv_xreg<sgpu::WF32, LPR, S>(W, x, bias, y, K, N);                                  \
    }                                                                                              \
    extern "C" __global__ void __launch_bounds__(256) sgpu_gemv_h_l##LPR##_s##S(                   \
        const uint16_t* __restrict__ W, const float* __restrict__ x, const float* __restrict__ bias, \
        float* __restrict__ y, int K, int N) {                                                     \
        sgpu::gemv_xreg<sgpu::WF16, LPR, S>(W, x, bias, y, K, N);                                  \
    }                                                                                              \
    extern "C" __global__ void __launch_bounds__(256) sgpu_gemv_hh_l##LPR##_s##S(                  \
        const uint16_t* __restrict__ W, const uint16_t* __restrict__ x, const float* __restrict__ bias, \
        float* __restrict__ y, int K, int N) {                                                     \
        sgpu::gemv_xreg_hh<LPR, S>(W, x, bias, y, K, N);                                           \
    }

#define SGPU_GEMV_INST_S(LPR) \
    SGPU_GEMV_INST(LPR, 1) SGPU_GEMV_INST(LPR, 2) SGPU_GEMV_INST(LPR, 3) SGPU_GEMV_INST(LPR, 4) \
    SGPU_GEMV_INST(LPR, 6) SGPU_GEMV_INST(LPR, 7) SGPU_GEMV_INST(LPR, 8) SGPU_GEMV_INST(LPR, 10) \
    SGPU_GEMV_INST(LPR, 12) SGPU_GEMV_INST(LPR, 16)

SGPU_GEMV_INST_S(16)
SGPU_GEMV_INST_S(64)
SGPU_GEMV_INST_S(256)

// Embedding row gather + h2f decode on the device: x[i] = h2f(emb[token*C + i]).  The
// reference decodes the row on the host and uploads it (qwen_engine.c:209-211); doing it
// here removes a host->device copy from every decode step.
extern "C" __global__ void sgpu_embed_h(const uint16_t* __restrict__ emb, int token, float* __restrict__ x, int C) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < C; i += gridDim.x * blockDim.x)
        x[i] = sgpu_h2f(emb[(size_t)token * C + i]);
}
