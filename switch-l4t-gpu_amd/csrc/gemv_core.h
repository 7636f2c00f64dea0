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
//    16-byte aligned), any grid (wave-granular grid-stride).  The reference-named symbols
//    (gemv_byname) fall back to it when the team kernel below cannot run.
//  * gemv_xreg<LPR, S>: a team of LPR lanes per row (16, 64 or 256 = four waves split-K),
//    each lane owning up to S fixed 16-byte segments of every row.  The lane's slice of x
//    (S*VEC floats) is loaded once into VGPRs and reused for every row of a persistent
//    grid-stride loop; all S weight loads of a row are issued before the first FMA.
//    Lane partials are combined with DPP row shifts/broadcasts (no LDS, no barrier) and,
//    for 256-lane teams, one LDS exchange across the four waves.
// Weights are read with the nontemporal hint: each byte is used exactly once per call.
#pragma once
#include <type_traits>

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

// x element k as fp32: fp32 x as is, fp16-bit x (the fp16-x GEMV) with the exact reference
// h2f decode -- the same operand values gemv_h sees for x = h2f(x16).
__device__ __forceinline__ float x_at(const float* x, int k) { return x[k]; }
__device__ __forceinline__ float x_at(const uint16_t* x, int k) { return sgpu_h2f(x[k]); }
// The VEC values of x behind weight segment s (16 bytes of weights): fp32 x is read as
// VEC/4 float4; fp16 x (VEC = 8 fp16 weights per segment) as one 16-byte load of 8 codes.
template <int VEC>
__device__ __forceinline__ void x_seg(const float* x, int s, float (&xa)[VEC]) {
    const sgpu_f32x4* xv4 = reinterpret_cast<const sgpu_f32x4*>(x);
#pragma unroll
    for (int q = 0; q < VEC / 4; q++) {
        const sgpu_f32x4 a = xv4[s * (VEC / 4) + q];
#pragma unroll
        for (int e = 0; e < 4; e++) xa[4 * q + e] = a[e];
    }
}
template <int VEC>
__device__ __forceinline__ void x_seg(const uint16_t* x, int s, float (&xa)[VEC]) {
    static_assert(VEC == 8, "fp16 x pairs with fp16 weights: 8 codes per 16-byte segment");
    const sgpu_u32x4 h = reinterpret_cast<const sgpu_u32x4*>(x)[s];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        xa[2 * i] = sgpu_h2f_lo(h[i]);
        xa[2 * i + 1] = sgpu_h2f_hi(h[i]);
    }
}

// Serial k-ascending dot product of one row with the exact reference decode; used for the
// rare rows whose fast sum is not finite.
template <class WT, class XT>
__device__ __noinline__ float recompute_row(const typename WT::elem* __restrict__ row, const XT* __restrict__ x,
                                            int K) {
    float acc = 0.0f;
    for (int k = 0; k < K; k++) acc = __builtin_fmaf(WT::one(row[k]), x_at(x, k), acc);
    return acc;
}

// ---------------------------------------------------------------------------------------
// Generic: wave per row.  XT = float, or uint16_t for fp16-bit x (fp16 weights only).
template <class WT, class XT = float>
__device__ __forceinline__ void gemv_generic(const typename WT::elem* __restrict__ W,
                                             const XT* __restrict__ x,
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
            for (int k = 0; k < K; k++) acc = __builtin_fmaf(WT::one(row[k]), x_at(x, k), acc);
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
            int s = lane;
            for (; s + 192 < nseg; s += 256) {        // four segments in flight per lane
                vec w[4];
#pragma unroll
                for (int u = 0; u < 4; u++) w[u] = sgpu_ldnt(rv + s + 64 * u);
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    float xa[VEC];
                    x_seg<VEC>(x, s + 64 * u, xa);
                    acc = WT::dot(w[u], xa, acc);
                }
            }
            for (; s + 64 < nseg; s += 128) {         // two
                const vec w0 = sgpu_ldnt(rv + s), w1 = sgpu_ldnt(rv + s + 64);
                float xa[VEC], xb[VEC];
                x_seg<VEC>(x, s, xa);
                x_seg<VEC>(x, s + 64, xb);
                acc = WT::dot(w0, xa, acc);
                acc = WT::dot(w1, xb, acc);
            }
            for (; s < nseg; s += 64) {
                const vec w0 = sgpu_ldnt(rv + s);
                float xa[VEC];
                x_seg<VEC>(x, s, xa);
                acc = WT::dot(w0, xa, acc);
            }
        } else {
            for (int k = lane; k < K; k += 64) acc = __builtin_fmaf(WT::one(row[k]), x_at(x, k), acc);
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

// preload(g, has, sub): operands the prologue needs besides x that do not depend on it (the
// RMSNorm gains), loaded before the weights so that they arrive with them.
struct XPlain {
    const float* x;
    __device__ __forceinline__ sgpu_f32x4 load4(int k) const { return *reinterpret_cast<const sgpu_f32x4*>(x + k); }
    __device__ __forceinline__ float at(int k) const { return x[k]; }
    template <int LPR, int S, int VEC>
    __device__ __forceinline__ void preload(sgpu_u32x4 (&)[S], const bool (&)[S], int) const {}
    template <int LPR, int S, int VEC>
    __device__ __forceinline__ void prepare(float (&)[S][VEC], const sgpu_u32x4 (&)[S], const bool (&)[S], int, int,
                                            float*) {}
};

// x given as fp16 bit patterns (the fp16-x GEMV): each lane converts its slice once into its
// registers with the hardware conversion, as the weights are converted (the code objects run
// with fp16 denormals flushed: subnormal codes read as +-0, which sums exactly as the
// reference's +0 does, since a running sum that starts at +0 never becomes -0).  Exponent-31
// codes convert to inf/NaN instead of the reference's finite 2^16 (1 + m/1024), which makes
// every row sum non-finite, and those rows are recomputed with the exact decode (at()).  So
// every sum equals gemv_h's for x = h2f(x16).  load4(k) returns the four raw codes at k as two
// dwords (slots 0, 1) and prepare() converts them after the whole slice is loaded: converting
// inside each load made the compiler wait for every load in turn.  load4 needs k % 4 == 0 and
// x 8-byte aligned.
struct XHalf {
    const uint16_t* x;
    __device__ __forceinline__ sgpu_f32x4 load4(int k) const {
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 h = *reinterpret_cast<const u32x2*>(x + k);
        return sgpu_f32x4{__uint_as_float(h[0]), __uint_as_float(h[1]), 0.0f, 0.0f};
    }
    __device__ __forceinline__ float at(int k) const { return sgpu_h2f(x[k]); }
    template <int LPR, int S, int VEC>
    __device__ __forceinline__ void preload(sgpu_u32x4 (&)[S], const bool (&)[S], int) const {}
    template <int LPR, int S, int VEC>
    __device__ __forceinline__ void prepare(float (&xr)[S][VEC], const sgpu_u32x4 (&)[S], const bool (&)[S], int, int,
                                            float*) {
#pragma unroll
        for (int j = 0; j < S; j++)
#pragma unroll
            for (int q = 0; q < VEC / 4; q++) {
                const uint32_t u0 = __float_as_uint(xr[j][4 * q]), u1 = __float_as_uint(xr[j][4 * q + 1]);
                xr[j][4 * q] = WF16::cvt(u0 & 0xffffu);         // zero codes (no segment) stay +0
                xr[j][4 * q + 1] = WF16::cvt(u0 >> 16);
                xr[j][4 * q + 2] = WF16::cvt(u1 & 0xffffu);
                xr[j][4 * q + 3] = WF16::cvt(u1 >> 16);
            }
    }
};

// x'[k] = x[k] * inv * h2f(w[k]), inv = 1 / sqrt(mean(x^2) + eps): cpu_rms (qwen_engine.c:285-290)
// with the same product order.  A team's lanes together hold all K values of x, so the sum of
// squares is a team reduction over the registers already loaded (no barrier for teams of up
// to one wave).  The lane's gain segments are loaded by preload(), ahead of the weights, so
// they arrive with them instead of costing a round trip after the reduction.
struct XRms {
    const float* x;
    const uint16_t* w;                   // 16-byte aligned (segments of 8 codes are loaded whole)
    float eps;
    float inv;
    __device__ __forceinline__ sgpu_f32x4 load4(int k) const { return *reinterpret_cast<const sgpu_f32x4*>(x + k); }
    __device__ __forceinline__ float at(int k) const {
#pragma clang fp contract(off)
        return x[k] * inv * sgpu_h2f(w[k]);
    }
    template <int LPR, int S, int VEC>
    __device__ __forceinline__ void preload(sgpu_u32x4 (&g)[S], const bool (&has)[S], int sub) const {
        if constexpr (VEC == 8) {
#pragma unroll
            for (int j = 0; j < S; j++)          // a lane without the segment reads segment 0, unused
                g[j] = *reinterpret_cast<const sgpu_u32x4*>(w + (has[j] ? (sub + LPR * j) * VEC : 0));
        }
    }
    template <int LPR, int S, int VEC>
    __device__ __forceinline__ void prepare(float (&xr)[S][VEC], const sgpu_u32x4 (&gp)[S], const bool (&has)[S], int sub,
                                            int K, float* red) {
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
            if constexpr (VEC == 8) {
                // the segment's 8 gain codes, preloaded, by the hardware conversion as the
                // weights are: a code of exponent 31 converts to inf/NaN instead of the
                // reference's finite value, every row sum then comes out non-finite and is
                // recomputed with the exact decode (at()); subnormal codes flush to 0 as there
                const sgpu_u32x4 g = gp[j];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    xr[j][2 * e] = xr[j][2 * e] * inv * WF16::cvt(g[e] & 0xffffu);
                    xr[j][2 * e + 1] = xr[j][2 * e + 1] * inv * WF16::cvt(g[e] >> 16);
                }
            } else {
#pragma unroll
                for (int e = 0; e < VEC; e++) xr[j][e] = xr[j][e] * inv * sgpu_h2f(w[k0 + e]);
            }
        }
    }
};

// x'[k] = (x[k] - mean) * inv * w[k] + b[k], the two-pass mean/variance LayerNorm of the
// GPT-2 CPU golden (gpt2_engine.c:333-341) with the same operation order.  As with XRms the
// team's lanes hold all K values, so both passes are team reductions over registers.
struct XLn {
    const float* x;
    const float* w;
    const float* b;
    float eps;
    float mean;
    float inv;
    __device__ __forceinline__ sgpu_f32x4 load4(int k) const { return *reinterpret_cast<const sgpu_f32x4*>(x + k); }
    __device__ __forceinline__ float at(int k) const {
#pragma clang fp contract(off)
        return (x[k] - mean) * inv * w[k] + b[k];
    }
    template <int LPR, int S, int VEC>
    __device__ __forceinline__ void preload(sgpu_u32x4 (&)[S], const bool (&)[S], int) const {}
    template <int LPR, int S, int VEC>
    __device__ __forceinline__ void prepare(float (&xr)[S][VEC], const sgpu_u32x4 (&)[S], const bool (&has)[S], int sub,
                                            int K, float* red) {
#pragma clang fp contract(off)
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < S; j++)
#pragma unroll
            for (int e = 0; e < VEC; e++) s += xr[j][e];             // zero where !has
        mean = team_sum_bcast<LPR>(s, red) / (float)K;
        float q = 0.0f;
#pragma unroll
        for (int j = 0; j < S; j++) {
            if (!has[j]) continue;
#pragma unroll
            for (int e = 0; e < VEC; e++) {
                const float d = xr[j][e] - mean;
                q += d * d;
            }
        }
        const float var = team_sum_bcast<LPR>(q, red) / (float)K;
        inv = 1.0f / __builtin_sqrtf(var + eps);
#pragma unroll
        for (int j = 0; j < S; j++) {
            if (!has[j]) continue;
            const int k0 = (sub + LPR * j) * VEC;
#pragma unroll
            for (int e = 0; e < VEC; e++) xr[j][e] = (xr[j][e] - mean) * inv * w[k0 + e] + b[k0 + e];
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

// Epilogues.  Per-row operands an epilogue needs besides the dot products (bias, residual,
// tables) are read by load(t, rows, pre) when the row block's weights are fetched -- one block
// ahead of use -- so they arrive with the weights instead of after the reduction;
// operator()(t, rows, acc, pre) then writes the outputs.

// y[row] = acc + bias?[row]
struct EpiStore {
    const float* bias;
    float* y;
    struct Pre {
        float b;
    };
    __device__ __forceinline__ void load(int, const int* rows, Pre& p) const { p.b = bias ? bias[rows[0]] : 0.0f; }
    __device__ __forceinline__ void operator()(int, const int* rows, const float* acc, const Pre& p) const {
        y[rows[0]] = acc[0] + p.b;
    }
};

// Serial k-ascending re-evaluation of one row with the exact reference decode and the same x.
template <class WT, class Pro>
__device__ __noinline__ float recompute_row_x(const typename WT::elem* __restrict__ row, Pro pro, int K) {
    float acc = 0.0f;
    for (int k = 0; k < K; k++) acc = __builtin_fmaf(WT::one(row[k]), pro.at(k), acc);
    return acc;
}

// nblk: the blocks that take part (blocks 0..nblk-1 walk the row blocks with stride nblk; any
// others return at once); 0 means the whole grid.
template <class WT, int LPR, int S, int NR, class Pro, class Map, class Epi>
__device__ __forceinline__ void gemv_team(const typename WT::elem* __restrict__ W, int K, int nteams, Pro pro,
                                          Map map, Epi epi, int nblk = 0) {
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
    typename Epi::Pre pre{};
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
            epi.load(t, rows, pre);
        }
    };
    // With nblk == 0 every block takes part, and the grid size is first needed as the stride to
    // a block's second row block: the first fetch does not wait for it (a kernel whose own
    // arguments fill the preloaded SGPRs reads it with a scalar load).
    if (nblk > 0 && (int)blockIdx.x >= nblk) return;  // block-uniform
    const int nb = nblk > 0 ? nblk : sgpu_gdim(0);
    int rb = blockIdx.x;
    sgpu_u32x4 gpre[S];
    pro.template preload<LPR, S, VEC>(gpre, has, sub);
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
    pro.template prepare<LPR, S, VEC>(xr, gpre, has, sub, K, red);

    for (; rb * TEAMS < nteams; rb += nb) {           // block-uniform loop
        const int t = rb * TEAMS + team;
        const bool cur_valid = valid;
        const typename Epi::Pre cur_pre = pre;
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
        if ((rb + nb) * TEAMS < nteams) fetch(rb + nb);
        if constexpr (LPR <= 64) {
#pragma unroll
            for (int r = 0; r < NR; r++) acc[r] = sgpu_group_sum<LPR>(acc[r]);
            if (sub == LPR - 1 && cur_valid) {
#pragma unroll
                for (int r = 0; r < NR; r++)
                    if (WT::NEEDS_RECHECK && !__builtin_isfinite(acc[r]))
                        acc[r] = recompute_row_x<WT>(W + (size_t)cur_rows[r] * K, pro, K);
                epi(t, cur_rows, acc, cur_pre);
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
                epi(t, cur_rows, acc, cur_pre);
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
// The tuned fp16-x GEMV: fp16 weights and fp16 x, fp32 accumulate, fp32 bias.
template <int LPR, int S>
__device__ __forceinline__ void gemv_xreg_hh(const uint16_t* __restrict__ W, const uint16_t* __restrict__ x,
                                             const float* __restrict__ bias, float* __restrict__ y, int K, int N) {
    gemv_team<WF16, LPR, S, 1>(W, K, N, XHalf{x}, MapRows{}, EpiStore{bias, y});
}

// The x source of the team GEMV for fp32 or fp16-bit x.
__device__ __forceinline__ XPlain x_source(const float* x) { return XPlain{x}; }
__device__ __forceinline__ XHalf x_source(const uint16_t* x) { return XHalf{x}; }

// The team GEMV of the reference-named symbols: a team of LPR lanes per row (16, 32 or 64; a
// block iteration covers 256/LPR rows), each lane owning up to S fixed 16-byte segments of
// every row (as gemv_team<WT, LPR, S>), but with x staged once per block in LDS as fp32 (fp16-bit
// x converted there as XHalf converts it) and read back for each row, so a lane's registers hold
// only its weight segments.  Blocks 0..nb-1 walk the row blocks with stride nb, the next one's
// weights fetched one block ahead of use.  Preconditions (gemv_byname): blockDim 256,
// K % VEC == 0, K <= LPR*S*VEC, W and x 16-byte aligned, xs holds K floats.
template <class WT, int LPR, int S, int NR, class XT>
__device__ __forceinline__ void gemv_team_xlds(const typename WT::elem* __restrict__ W, const XT* __restrict__ x,
                                               const float* __restrict__ bias, float* __restrict__ y, int K, int N,
                                               int nb, float* __restrict__ xs) {
    static_assert(LPR == 16 || LPR == 32 || LPR == 64, "teams within one wave");
    typedef typename WT::vec vec;
    constexpr int VEC = WT::VEC, TEAMS = 256 / LPR, RPB = TEAMS * NR;   // rows per block iteration
    const int tid = threadIdx.x, team = tid / LPR, sub = tid % LPR;
    const int nseg = K / VEC;
    bool has[S];
#pragma unroll
    for (int j = 0; j < S; j++) has[j] = sub + LPR * j < nseg;
    if ((int)blockIdx.x >= nb) return;                // block-uniform
    vec w[NR][S];
    int row[NR];
    bool valid[NR];
    float b[NR];
    auto fetch = [&](int rb) {
#pragma unroll
        for (int r = 0; r < NR; r++) {
            const int t = (rb * TEAMS + team) * NR + r;
            valid[r] = t < N;
            row[r] = valid[r] ? t : 0;
            b[r] = 0.0f;
            if (valid[r]) {
                const vec* rv = reinterpret_cast<const vec*>(W + (size_t)row[r] * K) + sub;
#pragma unroll
                for (int j = 0; j < S; j++)
                    if (has[j]) w[r][j] = sgpu_ldnt(rv + LPR * j);
                b[r] = bias ? bias[row[r]] : 0.0f;
            }
        }
    };
    int rb = blockIdx.x;
    if (rb * RPB < N) fetch(rb);
    const auto src = x_source(x);
    for (int k = 4 * tid; k < K; k += 4 * 256) {
        sgpu_f32x4 v = src.load4(k);
        if constexpr (std::is_same<XT, uint16_t>::value) {
            const uint32_t u0 = __float_as_uint(v[0]), u1 = __float_as_uint(v[1]);
            v = sgpu_f32x4{WF16::cvt(u0 & 0xffffu), WF16::cvt(u0 >> 16), WF16::cvt(u1 & 0xffffu), WF16::cvt(u1 >> 16)};
        }
        *reinterpret_cast<sgpu_f32x4*>(xs + k) = v;
    }
    __syncthreads();
    for (; rb * RPB < N; rb += nb) {                  // block-uniform loop
        bool cur_valid[NR];
        int cur_row[NR];
        float cur_b[NR], acc[NR];
#pragma unroll
        for (int r = 0; r < NR; r++) {
            cur_valid[r] = valid[r];
            cur_row[r] = row[r];
            cur_b[r] = b[r];
            acc[r] = 0.0f;
        }
        // x in rounds of U segments (16 floats): all of a round's LDS reads are issued before its
        // FMAs (the scheduler is kept from merging rounds, which would hold every segment's x in
        // registers at once), and one read of a segment's x serves the NR rows
        constexpr int U = 16 / VEC;
#pragma unroll
        for (int j0 = 0; j0 < S; j0 += U) {
            float xa[U][VEC];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int j = j0 + u;
                const sgpu_f32x4* xp = reinterpret_cast<const sgpu_f32x4*>(xs + (sub + LPR * j) * VEC);
#pragma unroll
                for (int q = 0; q < VEC / 4; q++) {
                    const sgpu_f32x4 a = (j < S && has[j]) ? xp[q] : sgpu_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int e = 0; e < 4; e++) xa[u][4 * q + e] = a[e];
                }
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int j = j0 + u;
                if (j >= S || !has[j]) continue;
#pragma unroll
                for (int r = 0; r < NR; r++)
                    if (cur_valid[r]) acc[r] = WT::dot(w[r][j], xa[u], acc[r]);
            }
            __asm__ volatile("" ::: "memory");       // rounds stay in order: U segments of x live at a time
        }
        // the next row block's weights load into the registers this one's just left: the dot
        // products are pinned before the fetch (each sum is an operand of an empty asm), so the
        // two sets of weights are never live together
#pragma unroll
        for (int r = 0; r < NR; r++) __asm__ volatile("" : "+v"(acc[r]));
        __asm__ volatile("" ::: "memory");
        if ((rb + nb) * RPB < N) fetch(rb + nb);
#pragma unroll
        for (int r = 0; r < NR; r++) acc[r] = sgpu_group_sum<LPR>(acc[r]);
        if (sub == LPR - 1) {
#pragma unroll
            for (int r = 0; r < NR; r++) {
                if (!cur_valid[r]) continue;
                float a = acc[r];
                if (WT::NEEDS_RECHECK && !__builtin_isfinite(a)) a = recompute_row_x<WT>(W + (size_t)cur_row[r] * K, src, K);
                y[cur_row[r]] = a + cur_b[r];
            }
        }
    }
}

// Body of the reference-named GEMV symbols (gemv, gemv4, gemv_warp, gemv_warp_b, gemv_h,
// gemv_hh), which hosts launch by name with their own geometry -- (N+7)/8 or (N+255)/256
// blocks of 256 in the reference callers.  When the launch has 1-D blocks of 256 threads and
// 16-byte aligned rows, with at least one block per 8 rows, it runs a team GEMV on a capped
// number of blocks (a persistent grid: those blocks walk the row blocks with the next one's
// weights in flight; surplus blocks exit):
//  * fp16 weights (gemv_h, gemv_hh): x staged in LDS (gemv_team_xlds), 16 lanes x 7 segments
//    (K <= 896), then 64 lanes x 10 segments with two rows per team (K <= 5120); at most
//    4608 blocks (18 per CU).  With x in LDS a lane's registers hold only its weights, so the
//    symbols take 4 waves per SIMD where x in registers (the wide member's 80 floats of it)
//    allowed 3;
//  * fp32 weights: x in registers (gemv_team), 16 x 12 (K <= 768), 64 x 16 (K <= 4096), 256 x 8
//    beyond, up to 2048 segments; at most 2048 blocks (8 per CU).  For fp32 the LDS form gains
//    on the GPT-2 lm_head but loses more on its 3072-wide rows.
// Other launches (unaligned rows, other block shapes, longer rows) take the wave-per-row
// kernel.  The choice is block-uniform.
template <class WT, class XT>
__device__ __forceinline__ void gemv_byname(const typename WT::elem* __restrict__ W, const XT* __restrict__ x,
                                            const float* __restrict__ bias, float* __restrict__ y, int K, int N) {
    constexpr int VEC = WT::VEC;
    // a grid of one thread per row or fewer ((N+255)/256 blocks, gemv_test.c:108) keeps a wave
    // per row: with so few waves the team kernel's one row block in flight per block is slower
    const bool team = sgpu_bdim_x() == 256 && sgpu_block256() && sgpu_gdim(1) == 1 &&
                      sgpu_gdim(2) == 1 && K > 0 && K % VEC == 0 && ((((uintptr_t)W) | ((uintptr_t)x)) & 15) == 0 &&
                      (long long)sgpu_gdim(0) * 8 >= N;
    const int nseg = K / VEC;
    if constexpr (VEC == 8) {
        const int nb = min(sgpu_gdim(0), 4608);
        __shared__ __attribute__((aligned(16))) float xs[64 * 10 * VEC];
        if (team && nseg <= 16 * 7)
            gemv_team_xlds<WT, 16, 7, 1, XT>(W, x, bias, y, K, N, nb, xs);
        else if (team && nseg <= 64 * 10)
            gemv_team_xlds<WT, 64, 10, 2, XT>(W, x, bias, y, K, N, nb, xs);
        else
            gemv_generic<WT, XT>(W, x, bias, y, K, N);
    } else {
        const int nb = min(sgpu_gdim(0), 2048);
        if (team && nseg <= 16 * 12)
            gemv_team<WT, 16, 12, 1>(W, K, N, x_source(x), MapRows{}, EpiStore{bias, y}, nb);
        else if (team && nseg <= 64 * 16)
            gemv_team<WT, 64, 16, 1>(W, K, N, x_source(x), MapRows{}, EpiStore{bias, y}, nb);
        else if (team && nseg <= 256 * 8)
            gemv_team<WT, 256, 8, 1>(W, K, N, x_source(x), MapRows{}, EpiStore{bias, y}, nb);
        else
            gemv_generic<WT, XT>(W, x, bias, y, K, N);
    }
}

// ---------------------------------------------------------------------------------------
// Few-token batched GEMV (gemv_multi role for T <= TT on aligned fp32 rows):
// Y[t*N+n] = W[n,:].X[t,:] + bias?[n].  The decode GEMV's team scheme with TT input vectors:
// a team of LPR lanes owns one row at a time, each lane holds S fixed 16-byte segments of
// every token's X row in registers for the whole persistent row loop, streams its segments of
// the row once (issued one row ahead of use) and accumulates all TT tokens from them; the
// team then reduces the TT sums (DPP within a wave, wave sums through LDS for 256-lane
// teams, fixed order).  Preconditions (launcher): blockDim 256, K % 4 == 0, W and X 16-byte
// aligned, K/4 <= S*LPR, 1 <= T <= TT.
template <int LPR, int S, int TT>
__device__ __forceinline__ void gemv_multi_xreg(const float* __restrict__ W, const float* __restrict__ X,
                                                const float* __restrict__ bias, float* __restrict__ Y, int K, int N,
                                                int T) {
    static_assert(LPR == 64 || LPR == 256, "team of one wave or of the block");
    constexpr int TEAMS = 256 / LPR, WPT = LPR / 64;
    __shared__ float red[TT][4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int team = tid / LPR, sub = tid % LPR;
    const int nseg = K / 4;
    bool has[S];
#pragma unroll
    for (int j = 0; j < S; j++) has[j] = sub + LPR * j < nseg;
    sgpu_f32x4 w[S];
    auto fetch = [&](int n) __attribute__((always_inline)) {
        const sgpu_f32x4* rv = reinterpret_cast<const sgpu_f32x4*>(W + (size_t)n * K) + sub;
#pragma unroll
        for (int j = 0; j < S; j++)
            if (has[j]) w[j] = sgpu_ldnt(rv + LPR * j);
    };
    int n = blockIdx.x * TEAMS + team;
    if (n < N) fetch(n);
    float xr[TT][S][4];
#pragma unroll
    for (int t = 0; t < TT; t++)
#pragma unroll
        for (int j = 0; j < S; j++) {
            const sgpu_f32x4 a = (t < T && has[j])
                ? *reinterpret_cast<const sgpu_f32x4*>(X + (size_t)t * K + 4 * (sub + LPR * j))
                : sgpu_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int e = 0; e < 4; e++) xr[t][j][e] = a[e];
        }
    const int stride = gridDim.x * TEAMS;
    for (int nb = blockIdx.x * TEAMS; nb < N; nb += stride) {   // block-uniform loop
        const bool cur = n < N;
        const int cur_n = n;
        float acc[TT];
#pragma unroll
        for (int t = 0; t < TT; t++) acc[t] = 0.0f;
        if (cur) {
#pragma unroll
            for (int j = 0; j < S; j++)
                if (has[j])
#pragma unroll
                    for (int t = 0; t < TT; t++) acc[t] = WF32::dot(w[j], xr[t][j], acc[t]);
        }
        n += stride;
        if (n < N) fetch(n);
        if constexpr (LPR == 64) {
#pragma unroll
            for (int t = 0; t < TT; t++) acc[t] = sgpu_group_sum<64>(acc[t]);
            if (lane == 63 && cur) {
                const float bv = bias ? bias[cur_n] : 0.0f;
#pragma unroll
                for (int t = 0; t < TT; t++)
                    if (t < T) Y[(size_t)t * N + cur_n] = acc[t] + bv;
            }
        } else {
#pragma unroll
            for (int t = 0; t < TT; t++) {
                acc[t] = sgpu_group_sum<64>(acc[t]);
                if (lane == 63) red[t][wave] = acc[t];
            }
            __syncthreads();
            if (tid < TT && tid < T && cur) {
                float v = red[tid][0];
#pragma unroll
                for (int i = 1; i < WPT; i++) v += red[tid][i];
                Y[(size_t)tid * N + cur_n] = v + (bias ? bias[cur_n] : 0.0f);
            }
            __syncthreads();
        }
    }
}

// ---------------------------------------------------------------------------------------
// Batched GEMV on the fp32 matrix cores (gemv_multi role when K % 4 == 0 and the rows are
// 16-byte aligned): Y[t*N+n] = sum_k W[n*K+k] * X[t*K+k] + bias?[n], with
// v_mfma_f32_32x32x2_f32 (fp32 inputs, fp32 accumulate).
//
// A 256-thread block owns a 32-token x 32*FN-row output tile; its four waves split K into
// contiguous ranges of 32-deep chunks and their partial tiles are summed through LDS in wave
// order (deterministic).  Per chunk a wave loads its 32 token rows and 32*FN weight rows with
// coalesced dwordx4 loads (8 lanes cover one 128-byte row segment), writes them to its own
// LDS region (row pitch 36 floats) and reads them back in the MFMA operand layout: lane
// (i, h) (i = lane % 32, h = lane / 32) takes floats k0 + 16h + 4v .. +3 of row i as one
// ds_read_b128 per v, and MFMA step s = 4v + e uses element e, so lane half h covers
// k = k0 + 16h + s on both operands.  The region is private to the wave: a wave-level
// barrier with wavefront-scope fences (wave_sync) orders the writes before the cross-lane
// reads and the reads before the next chunk's writes; no block barrier.  The next chunk's
// global loads are issued before the current
// chunk's MFMAs.  Rows past T or N read a clamped (valid) row and are never stored; a K tail
// chunk loads zeros past K.  Tiles are walked grid-stride over a linear block id (any grid of
// 256-thread blocks); with one block per tile, block ids are regrouped so each XCD runs a
// contiguous run of tiles (token tiles fastest: the blocks on one XCD share W panels in its
// L2).
// WT = WF32: fp32 weight rows, 16-byte loads.  WT = WF16: fp16 weight rows (8-byte loads of
// four codes), converted to fp32 while staged with the exact reference decode (sgpu_h2f), so
// the MFMAs see the same operands as the CPU golden.
// SPLIT: blocks are (tile, k-split) units, split-major; split s takes chunks
// [s*nch/S, (s+1)*nch/S) and its four waves divide those.  Each unit's block-summed partial
// tile goes to ws and the unit counts in on cnt[tile] (the hand-off protocol of sgpu_device.h);
// the last split of a tile sums the S partials in split order (deterministic), adds the bias,
// writes Y and resets the counter.  ws holds
// S * ntiles * 1024 * FN floats, cnt one zeroed counter per tile.  accum != 0 adds the
// result to Y instead of overwriting it (Y[t][n] = Y[t][n] + (sum + bias), the residual
// add of the decoders, in the order the separate add kernel computes it).
// Lanes of one wave exchanging data through LDS: every LDS access of this wave before the
// call happens before every access after it (wavefront-scope release, wave barrier, acquire;
// no instructions beyond the ordering itself).
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int FN, class WT = WF32, bool SPLIT = false>
__device__ __forceinline__ void gemm_nt_mfma(const typename WT::elem* __restrict__ W, const float* __restrict__ X,
                                             const float* __restrict__ bias, float* __restrict__ Y,
                                             int K, int N, int T, int S = 1, float* __restrict__ ws = nullptr,
                                             unsigned* __restrict__ cnt = nullptr, int accum = 0) {
    typedef float f32x16 __attribute__((ext_vector_type(16)));
    constexpr int NW = 4;                                   // waves per block (K split)
    constexpr int R = 32 * (1 + FN);                        // staged rows per wave: tokens, then W
    constexpr int NI = R / 8;                               // coalesced loads per lane per chunk
    constexpr int P = 36;                                   // LDS row pitch (floats)
    __shared__ __attribute__((aligned(16))) float stage[NW][R][P];
    static_assert(16 * FN * 64 <= R * P, "partial tile fits the wave's staging region");
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int i = lane & 31, h = lane >> 5;
    const int lr = lane >> 3, lq = lane & 7;                // coalesced: row in 8-row group, quad
    const int ntt = (T + 31) / 32, ntn = (N + 32 * FN - 1) / (32 * FN), ntiles = ntt * ntn;
    const int nch = (K + 31) / 32;
    const int nsplit = SPLIT ? S : 1;
    const int nb = gridDim.x * gridDim.y;
    const int bid = blockIdx.x + blockIdx.y * gridDim.x;
    const bool remap = nsplit == 1 && (nb == ntiles) && (ntiles % 8 == 0);
    float (*st)[P] = stage[wave];
    __shared__ int last_s;

    for (int unit = bid; unit < ntiles * nsplit; unit += nb) {
        const int tile = SPLIT ? unit % ntiles : unit, sp = SPLIT ? unit / ntiles : 0;
        const int uc0 = sp * nch / nsplit, uc1 = (sp + 1) * nch / nsplit;
        const int c0 = uc0 + wave * (uc1 - uc0) / NW, c1 = uc0 + (wave + 1) * (uc1 - uc0) / NW;
        const int tl = remap ? (tile % 8) * (ntiles / 8) + tile / 8 : tile;
        const int t0 = (tl % ntt) * 32, n0 = (tl / ntt) * 32 * FN;
        // Row q*8 + lr of the staged block: token rows first (q < 4), then weight rows.
        const float* xsrc[4];
        const typename WT::elem* wsrc[NI - 4];
#pragma unroll
        for (int q = 0; q < 4; q++) xsrc[q] = X + (size_t)min(t0 + 8 * q + lr, T - 1) * K + 4 * lq;
#pragma unroll
        for (int q = 4; q < NI; q++) wsrc[q - 4] = W + (size_t)min(n0 + 8 * q + lr - 32, N - 1) * K + 4 * lq;

        f32x16 acc[FN];
#pragma unroll
        for (int f = 0; f < FN; f++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[f][r] = 0.0f;
        // Staged chunk in registers: fp32 rows as loaded; fp16 rows as their raw codes, decoded
        // only when written to LDS, so the loads stay in flight under the previous chunk's MFMAs.
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        constexpr bool H = sizeof(typename WT::elem) == 2;
        sgpu_f32x4 g[H ? 4 : NI];
        u32x2 gh[H ? NI - 4 : 1];
        auto load = [&](int c) __attribute__((always_inline)) {
            const int k0 = 32 * c;
            const bool ok = k0 + 4 * lq < K;                // K % 4 == 0: whole quads
            const sgpu_f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int q = 0; q < 4; q++) g[q] = ok ? *reinterpret_cast<const sgpu_f32x4*>(xsrc[q] + k0) : z;
#pragma unroll
            for (int q = 4; q < NI; q++) {
                if constexpr (!H)
                    g[q] = ok ? *reinterpret_cast<const sgpu_f32x4*>(wsrc[q - 4] + k0) : z;
                else
                    gh[q - 4] = ok ? *reinterpret_cast<const u32x2*>(wsrc[q - 4] + k0) : u32x2{0u, 0u};
            }
        };
        auto chunk = [&](bool more, int cn) __attribute__((always_inline)) {
#pragma unroll
            for (int q = 0; q < NI; q++) {
                sgpu_f32x4 v;
                if constexpr (!H) {
                    v = g[q];
                } else if (q < 4) {
                    v = g[q];
                } else {
                    const u32x2 h = gh[q - 4];
                    v = sgpu_f32x4{sgpu_h2f_lo(h[0]), sgpu_h2f_hi(h[0]), sgpu_h2f_lo(h[1]), sgpu_h2f_hi(h[1])};
                }
                *reinterpret_cast<sgpu_f32x4*>(&st[8 * q + lr][4 * lq]) = v;
            }
            if (more) load(cn);                             // next chunk in flight during the MFMAs
            wave_sync();                                    // other lanes' stage writes are visible
            sgpu_f32x4 xa[4], wa[FN][4];
#pragma unroll
            for (int v = 0; v < 4; v++) {
                xa[v] = *reinterpret_cast<const sgpu_f32x4*>(&st[i][16 * h + 4 * v]);
#pragma unroll
                for (int f = 0; f < FN; f++)
                    wa[f][v] = *reinterpret_cast<const sgpu_f32x4*>(&st[32 + 32 * f + i][16 * h + 4 * v]);
            }
            wave_sync();                                    // reads done before the next chunk's writes
#pragma unroll
            for (int s = 0; s < 16; s++)
#pragma unroll
                for (int f = 0; f < FN; f++)
                    acc[f] = __builtin_amdgcn_mfma_f32_32x32x2f32(xa[s >> 2][s & 3], wa[f][s >> 2][s & 3], acc[f], 0, 0, 0);
        };
        if (c0 < c1) load(c0);
        for (int c = c0; c < c1; c++) chunk(c + 1 < c1, c + 1);

        // Partial tiles go to each wave's own staging region (done with it for this tile).
        auto red = [&](int w, int a) __attribute__((always_inline)) -> float& {
            return (&stage[w][0][0])[a * 64 + lane];
        };
#pragma unroll
        for (int f = 0; f < FN; f++)
#pragma unroll
            for (int r = 0; r < 16; r++) red(wave, 16 * f + r) = acc[f][r];
        __syncthreads();
        // Wave w finishes accumulator rows r = w*16/NW .. (w+1)*16/NW - 1 of every block,
        // summing the NW partials in wave order.  D layout: lane l, acc r -> token
        // 8*(r/4) + 4*(l/32) + r%4, row l%32.
        constexpr int RPW = 16 / NW;
        float v[FN][RPW];
#pragma unroll
        for (int f = 0; f < FN; f++)
#pragma unroll
            for (int rr = 0; rr < RPW; rr++) {
                const int r = RPW * wave + rr;
                v[f][rr] = red(0, 16 * f + r);
#pragma unroll
                for (int w = 1; w < NW; w++) v[f][rr] += red(w, 16 * f + r);
            }
        if (SPLIT && nsplit > 1) {
            // This thread's values: (f, rr) at ws + unit record + (f*RPW + rr)*256 + tid.
            constexpr int REC = 1024 * FN;
            float* rec = ws + (size_t)(sp * ntiles + tile) * REC + tid;
#pragma unroll
            for (int f = 0; f < FN; f++)
#pragma unroll
                for (int rr = 0; rr < RPW; rr++)
                    __hip_atomic_store(rec + (f * RPW + rr) * 256, v[f][rr], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __builtin_amdgcn_s_waitcnt(0);          // this wave's partial stores are acknowledged
            __syncthreads();
            if (tid == 0) {
                last_s = __hip_atomic_fetch_add(cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                         (unsigned)(nsplit - 1);
                if (last_s) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");   // before the others' partials
            }
            __syncthreads();
            if (!last_s) continue;                  // block-uniform; staging is free again
            // Partials come back U splits at a time, every load of a round issued before the
            // first add (one round trip per round instead of one per split), summed in split order.
            constexpr int U = 16;
            float sum[FN][RPW];
            for (int s0 = 0; s0 < nsplit; s0 += U) {
                float o[U][FN][RPW];
#pragma unroll
                for (int u = 0; u < U; u++) {
                    const int s2 = s0 + u;
                    const float* src = ws + (size_t)(s2 * ntiles + tile) * REC + tid;
#pragma unroll
                    for (int f = 0; f < FN; f++)
#pragma unroll
                        for (int rr = 0; rr < RPW; rr++)
                            o[u][f][rr] = s2 >= nsplit || s2 == sp
                                              ? v[f][rr]
                                              : __hip_atomic_load(src + (f * RPW + rr) * 256, __ATOMIC_RELAXED,
                                                                  __HIP_MEMORY_SCOPE_AGENT);
                }
#pragma unroll
                for (int u = 0; u < U; u++)
                    if (s0 + u < nsplit)
#pragma unroll
                        for (int f = 0; f < FN; f++)
#pragma unroll
                            for (int rr = 0; rr < RPW; rr++)
                                sum[f][rr] = s0 + u == 0 ? o[u][f][rr] : sum[f][rr] + o[u][f][rr];
            }
#pragma unroll
            for (int f = 0; f < FN; f++)
#pragma unroll
                for (int rr = 0; rr < RPW; rr++) v[f][rr] = sum[f][rr];
            if (tid == 0) __hip_atomic_store(cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
#pragma unroll
        for (int f = 0; f < FN; f++) {
            const int n = n0 + 32 * f + i;
            const float bv = (bias && n < N) ? bias[n] : 0.0f;
#pragma unroll
            for (int rr = 0; rr < RPW; rr++) {
                const int r = RPW * wave + rr;
                const int t = t0 + 8 * (r >> 2) + 4 * h + (r & 3);
                if (t < T && n < N) {
                    float* y = Y + (size_t)t * N + n;
                    *y = accum ? *y + (v[f][rr] + bv) : v[f][rr] + bv;
                }
            }
        }
        __syncthreads();                          // staging is reused by the next tile
    }
}

// Choice of the matrix-core path: whole 16-byte quads on 16-byte aligned rows, blocks of
// exactly 256 threads in x, and enough tokens to beat the vector path (below 4 tokens, or
// up to 8 tokens on rows longer than 1024, the wave-per-row kernel is as fast or faster:
// with so few 32x32 tiles the weight stream runs on too few CUs).  The host launcher
// applies the same rule (sgpu.c) to size the grid.
__device__ __forceinline__ bool gemm_nt_ok(const float* W, const float* X, int K, int T) {
    return K > 0 && (K % 4 == 0) && ((((uintptr_t)W) | ((uintptr_t)X)) & 15) == 0 && sgpu_bdim_x() == 256 &&
           sgpu_block256() && T >= 4 && !(T <= 8 && K > 1024);
}

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
