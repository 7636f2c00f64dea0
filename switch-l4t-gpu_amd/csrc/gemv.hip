// gemv.hip -- the M0 GEMV code object (reference gpu-llm/kernels/gemv.cu:3-71), gfx950.
//
// Same symbols and argument order as the reference, (const float*W, const float*x, float*y,
// int K, int N) with K before N, y[n] = sum_k W[n*K+k]*x[k].  The reference's three shapes
// (thread-per-row, thread-per-row float4, warp-per-row) are one design here
// (sgpu::gemv_byname): on 256-thread blocks and 16-byte rows a team of 16, 64 or 256 lanes
// per row with the lane's x slice in registers, walking row blocks with a block-stride loop;
// otherwise a wave per row.  Any K is accepted (the reference's float4 variants need
// K % 4 == 0) and any grid of blocks of up to 256 threads works: the host may keep
// gemv_test's (N+255)/256 or (N+7)/8 blocks of 256 threads.
#include "gemv_core.h"

extern "C" {

__global__ void __launch_bounds__(256) gemv(const float* __restrict__ W, const float* __restrict__ x, float* __restrict__ y,
                     int K, int N) {
    sgpu::gemv_byname<sgpu::WF32, float>(W, x, nullptr, y, K, N);
}

__global__ void __launch_bounds__(256) gemv4(const float* __restrict__ W, const float* __restrict__ x, float* __restrict__ y,
                      int K, int N) {
    sgpu::gemv_byname<sgpu::WF32, float>(W, x, nullptr, y, K, N);
}

__global__ void __launch_bounds__(256) gemv_warp(const float* __restrict__ W, const float* __restrict__ x, float* __restrict__ y,
                          int K, int N) {
    sgpu::gemv_byname<sgpu::WF32, float>(W, x, nullptr, y, K, N);
}

}  // extern "C"
