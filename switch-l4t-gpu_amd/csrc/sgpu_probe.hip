// sgpu_probe.hip -- measurement kernels behind bin/decode_floor and bin/sgemm_floor: the costs
// that bound a decode step built from dependent kernels (a kernel boundary, a weight stream
// after it, a device-side hand-off between kernels in flight together), and the matrix-core
// floor of a short SGEMM launch.  Not on the hot path; nothing here computes a result of the
// library.
#include "sgpu_device.h"

extern "C" {

// The streaming floor of one decode phase: block b reads prev[(7b + 1) % nprev], written by
// another block of the previous launch, streams its share of W (nvec 16-byte vectors, grid-
// stride, four loads in flight per thread, nontemporal), and writes out[b] = that value + 1, so
// the next launch depends on this one.  The weights are OR-folded into a test that is never
// true for the zero weights the host provides, which keeps every load live.
__global__ void __launch_bounds__(256) sgpu_probe_stream(const sgpu_u32x4* __restrict__ W, long long nvec,
                                                        const float* __restrict__ prev, int nprev,
                                                        float* __restrict__ out, unsigned* __restrict__ flag) {
    const long long stride = (long long)gridDim.x * 256;
    const long long gid = (long long)blockIdx.x * 256 + threadIdx.x;
    unsigned fold = 0;
    long long i = gid;
    for (; i + 3 * stride < nvec; i += 4 * stride) {
        sgpu_u32x4 w[4];
#pragma unroll
        for (int u = 0; u < 4; u++) w[u] = sgpu_ldnt(W + i + u * stride);
#pragma unroll
        for (int u = 0; u < 4; u++) fold |= w[u][0] | w[u][1] | w[u][2] | w[u][3];
    }
    for (; i < nvec; i += stride) {
        const sgpu_u32x4 w = sgpu_ldnt(W + i);
        fold |= w[0] | w[1] | w[2] | w[3];
    }
    if (fold == 0xdeadbeefu) flag[0] = 1u;
    if (threadIdx.x == 0) out[blockIdx.x] = prev[(blockIdx.x * 7 + 1) % nprev] + 1.0f;
}

// One link of a dependent chain.  Block b first issues P (<= 8) 16-byte weight loads per thread
// from its slice of W, then
//   mode bit 0 (wait): lanes 0..7 wait until counter[i] >= target / 8 (bounded by spin_limit
//                      polls; a give-up sets fail bit 0 and the block goes on), then an
//                      agent-scope acquire;
// reads xin[(7b + 1) % nin] (an agent-scope load when waiting, a plain load after a kernel
// boundary), writes xout[b] = that + 1, and
//   mode bit 1 (signal): the store is written through (agent scope) and acknowledged, then the
//                        block adds 1 to counter[b % 8];
//   mode bit 2 (empty):  the block does nothing at all.
// Blocks count into eight counters (b % 8) so that arrivals spread over eight addresses; a chain
// of links with B blocks each (B a multiple of 8) gives link i the target i * B.
__global__ void __launch_bounds__(256) sgpu_probe_link(const sgpu_u32x4* __restrict__ W, int P, const float* xin,
                                                      int nin, float* xout, unsigned* counter, unsigned target,
                                                      unsigned* fail, int spin_limit, int mode) {
    if (mode & 4) return;
    const int tid = threadIdx.x, b = blockIdx.x;
    sgpu_u32x4 w[8];
#pragma unroll
    for (int i = 0; i < 8; i++)
        if (i < P) w[i] = sgpu_ldnt(W + ((size_t)b * P + i) * 256 + tid);
    if ((mode & 1) && tid < 8) {
        const unsigned t = target / 8;
        int spins = 0, ok = 1;
        while ((int)(__hip_atomic_load(counter + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - t) < 0) {
            if (++spins > spin_limit) {
                ok = 0;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (!ok) __hip_atomic_fetch_or(fail, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    if (mode & 1) __syncthreads();
    unsigned fold = 0;
#pragma unroll
    for (int i = 0; i < 8; i++)
        if (i < P) fold |= w[i][0] | w[i][1] | w[i][2] | w[i][3];
    if (fold == 0xdeadbeefu) __hip_atomic_fetch_or(fail, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (tid == 0) {
        const int src = (b * 7 + 1) % nin;
        const float v = ((mode & 1) ? __hip_atomic_load(xin + src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                    : xin[src]) + 1.0f;
        if (mode & 2) __hip_atomic_store(xout + b, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else xout[b] = v;
    }
    if (mode & 2) {
        __builtin_amdgcn_s_waitcnt(0);          // the write-through store is acknowledged
        __syncthreads();
        if (tid == 0) __hip_atomic_fetch_add(counter + (b & 7), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}


// The matrix-core floor of an SGEMM launch: each wave of a 256-thread block issues iters x 16
// v_mfma_f32_32x32x2f32 on four independent accumulators, operands in registers, then writes
// its 16 sums, out[r * nthreads + gid] for gid < nout / 16 (gid the thread's grid index,
// nthreads the grid's): every store instruction covers consecutive floats, as an SGEMM's C
// write does, and that is the only memory it touches.  One block per CU (one wave per SIMD,
// as sgemm_kwave) and iters 32 give each SIMD the MFMA count of a 1024^3 SGEMM, with none of
// its loads and a C-sized store.
typedef float sgpu_f32x16_p __attribute__((ext_vector_type(16)));
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1)))
sgpu_probe_mfma(float* __restrict__ out, long long nout, int iters, float a0, float b0) {
    sgpu_f32x16_p acc[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[i][r] = 0.0f;
    const float a = a0 + threadIdx.x * 1e-7f, b = b0 - threadIdx.x * 1e-7f;
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int k = 0; k < 4; k++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc[i] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc[i], 0, 0, 0);
    }
    const long long nthreads = (long long)sgpu_gdim(0) * 256, gid = (long long)blockIdx.x * 256 + threadIdx.x;
    if (gid < nout / 16) {
#pragma unroll
        for (int r = 0; r < 16; r++) out[r * nthreads + gid] = ((acc[0][r] + acc[1][r]) + acc[2][r]) + acc[3][r];
    }
}

}  // extern "C"
