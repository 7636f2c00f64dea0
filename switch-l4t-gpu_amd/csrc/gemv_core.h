// gemv_core.h -- batch-1 GEMV kernels for gfx950, fp32 and fp16-bit weights.
//
//   y[n] = sum_k W[n*K + k] * x[k] + (bias ? bias[n] : 0)      W: N x K row-major
//
// This is HBM streaming work (one flop per weight byte for fp16): the kernels are built to
// keep enough 128-bit weight loads in flight per CU, not to reach the matrix cores.
//
// Two shapes of kernel:
//  * gemv_generic: a wave per row, lanes striding the row in 16-byte segments, x read
//    through the vector L1.  Any K, any pointer alignment (scalar path when a row is not
//    16-byte aligned), any grid (wave-granular grid-stride).  Backs the reference-named
//    symbols so hosts that keep the reference's own launch geometry stay correct.
//  * gemv_xreg<LPR, S>: a team of LPR lanes per row (16, 64 or 256 = four waves split-K),
//    each lane owning up to S fixed 16-byte segments of every row.  The lane's slice of x
//    (S*VEC floats) is loaded once into VGPRs and reused for every row of a persistent
//    grid-stride loop; all S weight loads of a row are issued before the first FMA.
//    Lane partials are combined with DPP row shifts/broadcasts (no LDS, no barrier) and,
//    for 256-lane teams, one LDS exchange across the four waves.
// Weights are read with the nontemporal hint: each byte is used exactly once per call.
#pragma once
#include "sgpu_device.h"

namespace sgpu {

// Weight element traits: 16 bytes = 4 fp32 or 8 fp16.
struct WF32 {
    typedef float elem;
    typedef sgpu_f32x4 vec;
    static constexpr int VEC = 4;
    static constexpr bool NEEDS_RECHECK = false;
    __device__ static __forceinline__ float dot(const vec& w, const float* xv, float acc) {
        acc = __builtin_fmaf(w[0], xv[0], acc);
        acc = __builtin_fmaf(w[1], xv[1], acc);
        acc = __builtin_fmaf(w[2], xv[2], acc);
        acc = __builtin_fmaf(w[3], xv[3], acc);
        return acc;
    }
    __device__ static __forceinline__ float one(elem w) { return w; }
};
// fp16 weights.  The hot loop converts with the hardware (one v_fma_mix_f32 or
// v_cvt_f32_f16 + FMA per weight).  The code objects holding these kernels are built with
// the fp16 denormal mode set to flush, so an fp16 subnormal reads as +-0 -- which sums to
// exactly what the reference's +0 gives (a running sum that starts at +0 never becomes -0).
// The one code class the hardware converts differently is exponent 31 (inf/NaN in IEEE, the
// finite 2^16 (1 + m/1024) in the reference); any such weight makes the row's sum
// non-finite, and those rows are recomputed with the exact integer decode (recompute_row).
struct WF16 {
    typedef uint16_t elem;
    typedef sgpu_u32x4 vec;
    static constexpr int VEC = 8;
    static constexpr bool NEEDS_RECHECK = true;
    __device__ static __forceinline__ float cvt(uint32_t bits16) {
        return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
    }
    __device__ static __forceinline__ float dot(const vec& w, const float* xv, float acc) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            acc = __builtin_fmaf(cvt(w[i] & 0xffffu), xv[2 * i], acc);
            acc = __builtin_fmaf(cvt(w[i] >> 16), xv[2 * i + 1], acc);
        }
        return acc;
    }
    __device__ static __forceinline__ float one(elem w) { return sgpu_h2f(w); }
};

// Serial k-ascending dot product of one row with the exact reference decode; used for the
// rare rows whose fast sum is not finite.
template <class WT>
__device__ __noinline__ float recompute_row(const typename WT::elem* __restrict__ row, const float* __restrict__ x,
                                            int K) {
    float acc = 0.0f;
    for (int k = 0; k < K; k++) acc = __builtin_fmaf(WT::one(row[k]), x[k], acc);
    return acc;
}

// ---------------------------------------------------------------------------------------
// Generic: wave per row.
template <class WT>
__device__ __forceinline__ void gemv_generic(const typename WT::elem* __restrict__ W,
                                             const float* __restrict__ x,
                                             const float* __restrict__ bias,
                                             float* __restrict__ y, int K, int N) {
    typedef typename WT::vec vec;
    constexpr int VEC = WT::VEC;
    const int lane = sgpu_tid() & 63;
    const int wave = (sgpu_bid() * sgpu_nthreads() + sgpu_tid()) >> 6;
    const int nwaves = (sgpu_nblocks() * sgpu_nthreads()) >> 6;
    if (((sgpu_nthreads()) & 63) != 0) {
        // Partial waves cannot run the DPP reduction: fall back to one thread per row.
        const int t = sgpu_bid() * sgpu_nthreads() + sgpu_tid();
        const int nt = sgpu_nblocks() * sgpu_nthreads();
        for (int n = t; n < N; n += nt) {
            const typename WT::elem* row = W + (size_t)n * K;
            float acc = 0.0f;
            for (int k = 0; k < K; k++) acc = __builtin_fmaf(WT::one(row[k]), x[k], acc);
            y[n] = acc + (bias ? bias[n] : 0.0f);
        }
        return;
    }
    const bool vec_ok = (K % VEC == 0) && ((((uintptr_t)W) | ((uintptr_t)x)) & 15) == 0;
    const int nseg = K / VEC;
    for (int n = wave; n < N; n += nwaves) {          // wave-uniform loop: no barriers inside
        const typename WT::elem* row = W + (size_t)n * K;
        float acc = 0.0f;
        if (vec_ok) {
            const vec* rv = reinterpret_cast<const vec*>(row);
            const sgpu_f32x4* xv4 = reinterpret_cast<const sgpu_f32x4*>(x);
            int s = lane;
            for (; s + 64 < nseg; s += 128) {         // two segments in flight per lane
                const vec w0 = sgpu_ldnt(rv + s), w1 = sgpu_ldnt(rv + s + 64);
                float xa[VEC], xb[VEC];
#pragma unroll
                for (int q = 0; q < VEC / 4; q++) {
                    const sgpu_f32x4 a = xv4[s * (VEC / 4) + q], b = xv4[(s + 64) * (VEC / 4) + q];
#pragma unroll
                    for (int e = 0; e < 4; e++) { xa[4 * q + e] = a[e]; xb[4 * q + e] = b[e]; }
                }
                acc = WT::dot(w0, xa, acc);
                acc = WT::dot(w1, xb, acc);
            }
            for (; s < nseg; s += 64) {
                const vec w0 = sgpu_ldnt(rv + s);
                float xa[VEC];
#pragma unroll
                for (int q = 0; q < VEC / 4; q++) {
                    const sgpu_f32x4 a = xv4[s * (VEC / 4) + q];
#pragma unroll
                    for (int e = 0; e < 4; e++) xa[4 * q + e] = a[e];
                }
                acc = WT::dot(w0, xa, acc);
            }
        } else {
            for (int k = lane; k < K; k += 64) acc = __builtin_fmaf(WT::one(row[k]), x[k], acc);
        }
        acc = sgpu_group_sum<64>(acc);
        if (lane == 63) {
            if (WT::NEEDS_RECHECK && !__builtin_isfinite(acc)) acc = recompute_row<WT>(row, x, K);
            y[n] = acc + (bias ? bias[n] : 0.0f);
        }
    }
}

// ---------------------------------------------------------------------------------------
// Tuned: a team of LPR lanes per row (or per NR rows), the lane's x slice in VGPRs,
// persistent over rows.  Three hooks make the same loop serve the plain GEMV and the fused
// decode kernels:
//   Pro  -- how x is obtained: XPlain (x as given) or XRms (RMSNorm applied on the fly; the
//           block computes mean(x^2) once, every lane scales its own slice)
//   Map  -- which weight rows team t reduces: MapRows (row t), MapPair (t and t + off),
//           MapHalfPairs (rows i and i + H/2 of each H-row block, the RoPE pairs)
//   Epi  -- what the reducing lane does with the NR sums of team t
// Preconditions (checked by the launchers): blockDim == 256, K % VEC == 0, W and x 16-byte
// aligned, K/VEC <= S*LPR, NR == 1 when LPR > 64.

// Sum of v over the team of LPR lanes that holds this lane (teams are aligned groups of LPR
// consecutive threads), returned to every lane of the team.  Teams of up to one wave use DPP
// and a cross-lane read; wider teams combine wave sums through LDS (block-wide barriers).
template <int LPR>
__device__ __forceinline__ float team_sum_bcast(float v, float* red) {
    if constexpr (LPR <= 64) {
        v = sgpu_group_sum<LPR>(v);
        return __shfl(v, (threadIdx.x & 63) | (LPR - 1));
    } else {
        v = sgpu_group_sum<64>(v);
        __syncthreads();
        if ((threadIdx.x & 63) == 63) red[threadIdx.x >> 6] = v;
        __syncthreads();
        const int first = (threadIdx.x / LPR) * (LPR / 64);
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < LPR / 64; i++) t += red[first + i];
        __syncthreads();
        return t;
    }
}

struct XPlain {
    const float* x;
    __device__ __forceinline__ sgpu_f32x4 load4(int k) const { return *reinterpret_cast<const sgpu_f32x4*>(x + k); }
    __device__ __forceinline__ float at(int k) const { return x[k]; }
    template <int LPR, int S, int VEC>
    __device__ __forceinline__ void prepare(float (&)[S][VEC], const bool (&)[S], int, int, float*) {}
};

// x'[k] = x[k] * inv * h2f(w[k]), inv = 1 / sqrt(mean(x^2) + eps): cpu_rms (qwen_engine.c:285-290)
// with the same product order.  A team's lanes together hold all K values of x, so the sum of
// squares is a team reduction over the registers already loaded: no extra loads, and no
// barrier for teams of up to one wave.
struct XRms {
    const float* x;
    const uint16_t* w;
    float eps;
    float inv;
    __device__ __forceinline__ sgpu_f32x4 load4(int k) const { return *reinterpret_cast<const sgpu_f32x4*>(x + k); }
    __device__ __forceinline__ float at(int k) const {
#pragma clang fp contract(off)
        return x[k] * inv * sgpu_h2f(w[k]);
    }
    template <int LPR, int S, int VEC>
    __device__ __forceinline__ void prepare(float (&xr)[S][VEC], const bool (&has)[S], int sub, int K, float* red) {
#pragma clang fp contract(off)
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < S; j++)
#pragma unroll
            for (int e = 0; e < VEC; e++) ss += xr[j][e] * xr[j][e];   // zero where !has
        ss = team_sum_bcast<LPR>(ss, red);
        inv = 1.0f / __builtin_sqrtf(ss / (float)K + eps);
#pragma unroll
        for (int j = 0; j < S; j++) {
            if (!has[j]) continue;
            const int k0 = (sub + LPR * j) * VEC;
#pragma unroll
            for (int e = 0; e < VEC; e++) xr[j][e] = xr[j][e] * inv * sgpu_h2f(w[k0 + e]);
        }
    }
};

struct MapRows {
    __device__ __forceinline__ int row(int t, int) const { return t; }
};
struct MapPair {
    int off;
    __device__ __forceinline__ int row(int t, int j) const { return t + j * off; }
};
struct MapHalfPairs {
    int half;   // H/2: team t covers rows (t/half)*2*half + t%half and that + half
    __device__ __forceinline__ int row(int t, int j) const { return (t / half) * 2 * half + t % half + j * half; }
};

// y[row] = acc + bias?[row]
struct EpiStore {
    const float* bias;
    float* y;
    __device__ __forceinline__ void operator()(int, const int* rows, const float* acc) const {
        y[rows[0]] = acc[0] + (bias ? bias[rows[0]] : 0.0f);
    }
};

// Serial k-ascending re-evaluation of one row with the exact reference decode and the same x.
template <class WT, class Pro>
__device__ __noinline__ float recompute_row_x(const typename WT::elem* __restrict__ row, Pro pro, int K) {
    float acc = 0.0f;
    for (int k = 0; k < K; k++) acc = __builtin_fmaf(WT::one(row[k]), pro.at(k), acc);
    return acc;
}

template <class WT, int LPR, int S, int NR, class Pro, class Map, class Epi>
__device__ __forceinline__ void gemv_team(const typename WT::elem* __restrict__ W, int K, int nteams, Pro pro,
                                          Map map, Epi epi) {
    static_assert(LPR == 16 || LPR == 32 || LPR == 64 || LPR == 128 || LPR == 256, "team size");
    static_assert(NR == 1 || LPR <= 64, "multi-row teams must fit in one wave");
    typedef typename WT::vec vec;
    constexpr int VEC = WT::VEC;
    constexpr int NT = 256;
    constexpr int TEAMS = NT / LPR;                   // teams per block iteration
    constexpr int WAVES_PER_TEAM = LPR > 64 ? LPR / 64 : 1;
    __shared__ float red[NT / 64];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int team = tid / LPR, sub = tid % LPR;
    const int nseg = K / VEC;
    bool has[S];
#pragma unroll
    for (int j = 0; j < S; j++) has[j] = sub + LPR * j < nseg;

    // Weight loads of a row block; issued one block ahead of their use, so the first block's
    // fetch overlaps the x prologue and each later fetch overlaps the previous reduction.
    vec w[NR][S];
    int rows[NR];
    bool valid = false;
    auto fetch = [&](int rb) {
        const int t = rb * TEAMS + team;
        valid = t < nteams;
#pragma unroll
        for (int r = 0; r < NR; r++) rows[r] = valid ? map.row(t, r) : 0;
        if (valid) {
#pragma unroll
            for (int r = 0; r < NR; r++) {
                const vec* rv = reinterpret_cast<const vec*>(W + (size_t)rows[r] * K) + sub;
#pragma unroll
                for (int j = 0; j < S; j++)
                    if (has[j]) w[r][j] = sgpu_ldnt(rv + LPR * j);
            }
        }
    };
    int rb = blockIdx.x;
    if (rb * TEAMS < nteams) fetch(rb);

    // This lane's x slice: segments sub, sub+LPR, ..., kept for every row.
    float xr[S][VEC];
#pragma unroll
    for (int j = 0; j < S; j++) {
        const int seg = sub + LPR * j;
#pragma unroll
        for (int q = 0; q < VEC / 4; q++) {
            const sgpu_f32x4 a = has[j] ? pro.load4(seg * VEC + 4 * q) : sgpu_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int e = 0; e < 4; e++) xr[j][4 * q + e] = a[e];
        }
    }
    pro.template prepare<LPR, S, VEC>(xr, has, sub, K, red);

    for (; rb * TEAMS < nteams; rb += gridDim.x) {    // block-uniform loop
        const int t = rb * TEAMS + team;
        const bool cur_valid = valid;
        int cur_rows[NR];
        float acc[NR];
#pragma unroll
        for (int r = 0; r < NR; r++) {
            cur_rows[r] = rows[r];
            acc[r] = 0.0f;
        }
        if (cur_valid) {
#pragma unroll
            for (int r = 0; r < NR; r++)
#pragma unroll
                for (int j = 0; j < S; j++)
                    if (has[j]) acc[r] = WT::dot(w[r][j], xr[j], acc[r]);
        }
        if ((rb + (int)gridDim.x) * TEAMS < nteams) fetch(rb + gridDim.x);
        if constexpr (LPR <= 64) {
#pragma unroll
            for (int r = 0; r < NR; r++) acc[r] = sgpu_group_sum<LPR>(acc[r]);
            if (sub == LPR - 1 && cur_valid) {
#pragma unroll
                for (int r = 0; r < NR; r++)
                    if (WT::NEEDS_RECHECK && !__builtin_isfinite(acc[r]))
                        acc[r] = recompute_row_x<WT>(W + (size_t)cur_rows[r] * K, pro, K);
                epi(t, cur_rows, acc);
            }
        } else {
            acc[0] = sgpu_group_sum<64>(acc[0]);
            if (lane == 63) red[wave] = acc[0];
            __syncthreads();
            if (sub == 0 && cur_valid) {
                float s = 0.0f;
#pragma unroll
                for (int i = 0; i < WAVES_PER_TEAM; i++) s += red[team * WAVES_PER_TEAM + i];
                if (WT::NEEDS_RECHECK && !__builtin_isfinite(s)) s = recompute_row_x<WT>(W + (size_t)cur_rows[0] * K, pro, K);
                acc[0] = s;
                epi(t, cur_rows, acc);
            }
            __syncthreads();
        }
    }
}

// The plain tuned GEMV: y[n] = W[n,:].x + bias?[n].
template <class WT, int LPR, int S>
__device__ __forceinline__ void gemv_xreg(const typename WT::elem* __restrict__ W, const float* __restrict__ x,
                                          const float* __restrict__ bias, float* __restrict__ y, int K, int N) {
    gemv_team<WT, LPR, S, 1>(W, K, N, XPlain{x}, MapRows{}, EpiStore{bias, y});
}

// ---------------------------------------------------------------------------------------
// Weight-stationary batched GEMV (gemv_multi role): Y[t*N+n] = W[n,:].X[t,:] + bias?[n].
// A wave owns one row and a chunk of up to TW tokens: the row is streamed once per chunk
// while TW register accumulators collect the chunk's dot products.
template <int TW>
__device__ __forceinline__ void gemv_multi_f32(const float* __restrict__ W, const float* __restrict__ X,
                                               const float* __restrict__ bias, float* __restrict__ Y,
                                               int K, int N, int T) {
    if ((sgpu_nthreads() & 63) != 0) {
        // Partial waves: one thread per (row, token), serial dot product.
        const int t0 = sgpu_bid() * sgpu_nthreads() + sgpu_tid();
        const int nt = sgpu_nblocks() * sgpu_nthreads();
        for (long long i = t0; i < (long long)N * T; i += nt) {
            const int n = (int)(i % N), t = (int)(i / N);
            float acc = 0.0f;
            for (int k = 0; k < K; k++) acc = __builtin_fmaf(W[(size_t)n * K + k], X[(size_t)t * K + k], acc);
            Y[(size_t)t * N + n] = acc + (bias ? bias[n] : 0.0f);
        }
        return;
    }
    const int lane = sgpu_tid() & 63;
    const int wave = (blockIdx.x * sgpu_nthreads() + sgpu_tid()) >> 6;
    const int nwaves = (gridDim.x * sgpu_nthreads()) >> 6;
    const bool vec_ok = (K % 4 == 0) && ((((uintptr_t)W) | ((uintptr_t)X)) & 15) == 0;
    const int nseg = K / 4;
    for (int c = blockIdx.y; c * TW < T; c += gridDim.y) {
        const int t0 = c * TW;
        const int tn = min(TW, T - t0);
        for (int n = wave; n < N; n += nwaves) {
            float acc[TW];
#pragma unroll
            for (int j = 0; j < TW; j++) acc[j] = 0.0f;
            if (vec_ok) {
                const sgpu_f32x4* wr = reinterpret_cast<const sgpu_f32x4*>(W + (size_t)n * K);
                for (int s = lane; s < nseg; s += 64) {
                    const sgpu_f32x4 w = sgpu_ldnt(wr + s);
#pragma unroll
                    for (int j = 0; j < TW; j++)
                        if (j < tn) {
                            const sgpu_f32x4 v = *reinterpret_cast<const sgpu_f32x4*>(X + (size_t)(t0 + j) * K + 4 * s);
                            acc[j] = __builtin_fmaf(w[0], v[0], acc[j]);
                            acc[j] = __builtin_fmaf(w[1], v[1], acc[j]);
                            acc[j] = __builtin_fmaf(w[2], v[2], acc[j]);
                            acc[j] = __builtin_fmaf(w[3], v[3], acc[j]);
                        }
                }
            } else {
                for (int k = lane; k < K; k += 64) {
                    const float w = W[(size_t)n * K + k];
#pragma unroll
                    for (int j = 0; j < TW; j++)
                        if (j < tn) acc[j] = __builtin_fmaf(w, X[(size_t)(t0 + j) * K + k], acc[j]);
                }
            }
            const float b = bias ? bias[n] : 0.0f;
#pragma unroll
            for (int j = 0; j < TW; j++) {
                const float s = sgpu_group_sum<64>(acc[j]);
                if (j < tn && lane == 63) Y[(size_t)(t0 + j) * N + n] = s + b;
            }
        }
    }
}

}  // namespace sgpu
