// gpt2_kernels.hip -- the GPT-2 engine's GEMV code object (reference
// gpu-llm/kernels/gpt2_kernels.cu:38-155), gfx950.
//
//   gemv_warp   (W, x, y, K, N)              y = W x                 (gpt2_kernels.cu:38-72)
//   gemv_warp_b (W, x, bias, y, K, N)        y = W x + bias          (gpt2_kernels.cu:75-108)
//   gemv_multi  (W, X, bias, Y, K, N, T)     Y[t] = W X[t] + bias?   (gpt2_kernels.cu:110-155)
// fp32 throughout.  bias is nullable in all three.  Any grid works (wave-granular
// grid-stride); gemv_multi walks token chunks of 16 over grid.y as the reference does.
#include "gemv_core.h"

extern "C" {

__global__ void gemv_warp(const float* __restrict__ W, const float* __restrict__ x, float* __restrict__ y,
                          int K, int N) {
    sgpu::gemv_generic<sgpu::WF32>(W, x, nullptr, y, K, N);
}

__global__ void gemv_warp_b(const float* __restrict__ W, const float* __restrict__ x,
                            const float* __restrict__ bias, float* __restrict__ y, int K, int N) {
    sgpu::gemv_generic<sgpu::WF32>(W, x, bias, y, K, N);
}

__global__ void __launch_bounds__(256) gemv_multi(const float* __restrict__ W, const float* __restrict__ X,
                                                  const float* __restrict__ bias, float* __restrict__ Y,
                                                  int K, int N, int T) {
    sgpu::gemv_multi_f32<16>(W, X, bias, Y, K, N, T);
}

}  // extern "C"
