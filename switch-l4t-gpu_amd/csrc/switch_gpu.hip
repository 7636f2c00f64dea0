// switch_gpu.hip -- SGEMM family + read-bandwidth probe for gfx950 (the switch_gpu code object).
//
// Exported symbols keep the reference names and argument lists (switch_gpu.cu:5-8,41-43,59-62,
// 99-102,140-143) so a host that resolves them by name keeps working:
//   sgemm_tiled, sgemm_tiled4, sgemm_opt : (const float*A, const float*B, float*C, int M, int N, int K)
//   sgemm_naive                          : same arguments, one output per thread
//   membw_read4                          : (const float4*buf, float*out, int n4, int iters)
//
// C = A*B, fp32, row-major (A: MxK stride K, B: KxN stride N, C: MxN stride N), overwrite
// (alpha 1, beta 0).  Unlike the reference kernels, every shape is accepted: edge tiles and
// unaligned K/N take a bounds-checked load/store path, interior tiles take dwordx4 loads.
//
// The tiled kernels run on the fp32 matrix cores: v_mfma_f32_32x32x2_f32 (true fp32 inputs,
// fp32 accumulate; no reduced-precision xf32).  A block of 64*WGM*WGN threads owns a BMxBN
// tile of C; each wave owns a (BM/WGM)x(BN/WGN) sub-tile held in AGPRs as 32x32 MFMA blocks.
// A and B k-slices of depth BK are staged through LDS, double-buffered (one barrier per
// slice): A transposed to k-major with a 2-float row pad (conflict-free transposing stores),
// B row-major.  Tiles are walked with a grid-stride loop over a linear tile index, so any
// grid of 64*WGM*WGN-thread blocks is correct (surplus blocks exit); with one block per tile
// the index is remapped so each XCD (blocks are dealt round-robin to the 8 XCDs) works on a
// compact group of tiles that shares A and B panels in its own L2.
#include "sgpu_device.h"

typedef float sgpu_f32x16 __attribute__((ext_vector_type(16)));

namespace {

constexpr int kXcds = 8;       // MI355X: 8 XCDs, blocks dispatched round-robin across them
constexpr int kGroupM = 8;     // tile rows per swizzle group

template <int BM, int BN, int BK, int WGM, int WGN>
struct MfmaTile {
    static constexpr int NT = 64 * WGM * WGN;
    static constexpr int WTM = BM / WGM, WTN = BN / WGN;   // wave tile
    static constexpr int FM = WTM / 32, FN = WTN / 32;      // 32x32 MFMA blocks per wave
    static constexpr int LDA = BM + 2;                      // As[BK][LDA], k-major
    static constexpr int LDB = BN;                          // Bs[BK][LDB]
    static constexpr int KQ = BK / 4, NQ = BN / 4;          // float4 per A row / per B row
    static constexpr int A_PER_T = (BM * KQ) / NT;          // float4 loads per thread
    static constexpr int B_PER_T = (BK * NQ) / NT;
    static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be whole 32x32 blocks");
    static_assert(BK % 4 == 0 && (BM * KQ) % NT == 0 && (BK * NQ) % NT == 0, "load split");
    static_assert(BM % 8 == 0, "LDA pad trick needs BM % 8 == 0");
};

// Map a linear tile id to (tile_m, tile_n).  With exactly one block per tile and a tile
// count divisible by the XCD count, first regroup so XCD x gets a contiguous run of ids,
// then walk tiles in kGroupM-row groups (column-major inside a group).
__device__ __forceinline__ void sgemm_tile_coords(int t, int ntm, int ntn, bool remap, int& tm, int& tn) {
    const int ntiles = ntm * ntn;
    if (remap) t = (t % kXcds) * (ntiles / kXcds) + t / kXcds;
    const int per_group = kGroupM * ntn;
    const int first_m = (t / per_group) * kGroupM;
    const int gsz = min(ntm - first_m, kGroupM);
    const int r = t % per_group;
    tm = first_m + r % gsz;
    tn = r / gsz;
}

template <int BM, int BN, int BK, int WGM, int WGN>
__device__ __forceinline__ void sgemm_mfma(const float* __restrict__ A, const float* __restrict__ B,
                                           float* __restrict__ C, int M, int N, int K) {
    using T = MfmaTile<BM, BN, BK, WGM, WGN>;
    __shared__ __attribute__((aligned(16))) float As[2][BK][T::LDA];
    __shared__ __attribute__((aligned(16))) float Bs[2][BK][T::LDB];   // rows written as float4

    // The tile split assumes exactly NT threads per block; any other block size is rejected
    // by every thread alike (no barrier is reached, C is left untouched).
    if (sgpu_nthreads() != T::NT) return;
    const int tid = sgpu_tid();
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WGN, wn = wave % WGN;
    const int l32 = lane & 31, khalf = lane >> 5;

    const int ntm = (M + BM - 1) / BM, ntn = (N + BN - 1) / BN, ntiles = ntm * ntn;
    const int nb = sgpu_nblocks();
    const bool remap = (nb == ntiles) && (ntiles % kXcds == 0);
    const bool aligned = ((K & 3) == 0) && ((N & 3) == 0) &&
                         ((((uintptr_t)A) | ((uintptr_t)B)) & 15) == 0;
    const int nk = (K + BK - 1) / BK;

    for (int t = sgpu_bid(); t < ntiles; t += nb) {
        int tm, tn;
        sgemm_tile_coords(t, ntm, ntn, remap, tm, tn);
        const int m0 = tm * BM, n0 = tn * BN;
        const bool interior = (m0 + BM <= M) && (n0 + BN <= N);

        float4 ra[T::A_PER_T], rb[T::B_PER_T];
        // Global -> registers for k-slice kt (fast dwordx4 path or bounds-checked scalars).
        auto load_slice = [&](int kt) {
            const int k0 = kt * BK;
            const bool fast = interior && aligned && (k0 + BK <= K);
#pragma unroll
            for (int r = 0; r < T::A_PER_T; r++) {
                const int idx = tid + r * T::NT, row = idx / T::KQ, kq = idx % T::KQ;
                const int gm = m0 + row, gk = k0 + 4 * kq;
                if (fast) {
                    ra[r] = *reinterpret_cast<const float4*>(A + (size_t)gm * K + gk);
                } else {
                    float v[4];
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        v[j] = (gm < M && gk + j < K) ? A[(size_t)gm * K + gk + j] : 0.0f;
                    ra[r] = make_float4(v[0], v[1], v[2], v[3]);
                }
            }
#pragma unroll
            for (int r = 0; r < T::B_PER_T; r++) {
                const int idx = tid + r * T::NT, kr = idx / T::NQ, nq = idx % T::NQ;
                const int gk = k0 + kr, gn = n0 + 4 * nq;
                if (fast) {
                    rb[r] = *reinterpret_cast<const float4*>(B + (size_t)gk * N + gn);
                } else {
                    float v[4];
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        v[j] = (gk < K && gn + j < N) ? B[(size_t)gk * N + gn + j] : 0.0f;
                    rb[r] = make_float4(v[0], v[1], v[2], v[3]);
                }
            }
        };
        // Registers -> LDS buffer s (A transposed to k-major).
        auto store_slice = [&](int s) {
#pragma unroll
            for (int r = 0; r < T::A_PER_T; r++) {
                const int idx = tid + r * T::NT, row = idx / T::KQ, kq = idx % T::KQ;
                As[s][4 * kq + 0][row] = ra[r].x;
                As[s][4 * kq + 1][row] = ra[r].y;
                As[s][4 * kq + 2][row] = ra[r].z;
                As[s][4 * kq + 3][row] = ra[r].w;
            }
#pragma unroll
            for (int r = 0; r < T::B_PER_T; r++) {
                const int idx = tid + r * T::NT, kr = idx / T::NQ, nq = idx % T::NQ;
                *reinterpret_cast<float4*>(&Bs[s][kr][4 * nq]) = rb[r];
            }
        };

        sgpu_f32x16 acc[T::FM][T::FN];
#pragma unroll
        for (int i = 0; i < T::FM; i++)
#pragma unroll
            for (int j = 0; j < T::FN; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

        if (nk > 0) {
            load_slice(0);
            store_slice(0);
        }
        __syncthreads();
        for (int kt = 0; kt < nk; kt++) {
            const int s = kt & 1;
            if (kt + 1 < nk) load_slice(kt + 1);      // in flight while the MFMAs run
#pragma unroll
            for (int ks = 0; ks < BK / 2; ks++) {
                const int kk = 2 * ks + khalf;        // MFMA src layout: lane = i + 32*k
                float a[T::FM], b[T::FN];
#pragma unroll
                for (int i = 0; i < T::FM; i++) a[i] = As[s][kk][wm * T::WTM + i * 32 + l32];
#pragma unroll
                for (int j = 0; j < T::FN; j++) b[j] = Bs[s][kk][wn * T::WTN + j * 32 + l32];
#pragma unroll
                for (int i = 0; i < T::FM; i++)
#pragma unroll
                    for (int j = 0; j < T::FN; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
            }
            if (kt + 1 < nk) store_slice(s ^ 1);
            __syncthreads();
        }

        // D layout of a 32x32 block: lane l, acc r -> row 8*(r/4) + 4*(l/32) + r%4, col l%32.
#pragma unroll
        for (int i = 0; i < T::FM; i++)
#pragma unroll
            for (int j = 0; j < T::FN; j++) {
                const int gn = n0 + wn * T::WTN + j * 32 + l32;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int gm = m0 + wm * T::WTM + i * 32 + 8 * (r >> 2) + 4 * khalf + (r & 3);
                    if (interior || (gm < M && gn < N)) C[(size_t)gm * N + gn] = acc[i][j][r];
                }
            }
    }
}

}  // namespace

extern "C" {

// 64x64 tile, 4 waves of 32x32: the small-tile member (more blocks at small sizes).
__global__ void __launch_bounds__(256) sgemm_tiled(const float* __restrict__ A, const float* __restrict__ B,
                                                   float* __restrict__ C, int M, int N, int K) {
    sgemm_mfma<64, 64, 16, 2, 2>(A, B, C, M, N, K);
}

// 128x128 tile, 4 waves of 64x64 (2x2 MFMA blocks per wave).
__global__ void __launch_bounds__(256) sgemm_tiled4(const float* __restrict__ A, const float* __restrict__ B,
                                                    float* __restrict__ C, int M, int N, int K) {
    sgemm_mfma<128, 128, 16, 2, 2>(A, B, C, M, N, K);
}

// Large-matrix member: 128x128 tile, BK 32.
__global__ void __launch_bounds__(256) sgemm_opt(const float* __restrict__ A, const float* __restrict__ B,
                                                 float* __restrict__ C, int M, int N, int K) {
    sgemm_mfma<128, 128, 32, 2, 2>(A, B, C, M, N, K);
}

// One output per thread, direct global reads, bounds-checked (switch_gpu.cu:139-152 role:
// the bisect/control kernel).  Grid-stride in both dimensions, any 2-D geometry.
__global__ void sgemm_naive(const float* __restrict__ A, const float* __restrict__ B,
                            float* __restrict__ C, int M, int N, int K) {
    for (int row = blockIdx.y * blockDim.y + threadIdx.y; row < M; row += gridDim.y * blockDim.y)
        for (int col = blockIdx.x * blockDim.x + threadIdx.x; col < N; col += gridDim.x * blockDim.x) {
            float acc = 0.0f;
            for (int k = 0; k < K; ++k) acc = __builtin_fmaf(A[(size_t)row * K + k], B[(size_t)k * N + col], acc);
            C[(size_t)row * N + col] = acc;
        }
}

// Read-bandwidth probe with the reference's output contract (switch_gpu.cu:41-54): each
// thread sums its grid-stride float4 sweep `iters` times (in sweep order) and, if its first
// index is in range, writes the sum to out[first index].  Loads are issued four at a time
// per lane so enough bytes are in flight to cover HBM latency.
__global__ void __launch_bounds__(256) membw_read4(const float4* __restrict__ buf4, float* __restrict__ out,
                                                   int n4, int iters) {
    const sgpu_f32x4* buf = reinterpret_cast<const sgpu_f32x4*>(buf4);
    const int i0 = threadIdx.x + blockIdx.x * blockDim.x;
    const int stride = gridDim.x * blockDim.x;
    float acc = 0.0f;
    for (int it = 0; it < iters; ++it) {
        int i = i0;
        for (; i + 3 * stride < n4; i += 4 * stride) {
            const sgpu_f32x4 v0 = sgpu_ldnt(buf + i);
            const sgpu_f32x4 v1 = sgpu_ldnt(buf + i + stride);
            const sgpu_f32x4 v2 = sgpu_ldnt(buf + i + 2 * stride);
            const sgpu_f32x4 v3 = sgpu_ldnt(buf + i + 3 * stride);
            acc += ((v0.x + v0.y) + v0.z) + v0.w;
            acc += ((v1.x + v1.y) + v1.z) + v1.w;
            acc += ((v2.x + v2.y) + v2.z) + v2.w;
            acc += ((v3.x + v3.y) + v3.z) + v3.w;
        }
        for (; i < n4; i += stride) {
            const sgpu_f32x4 v = sgpu_ldnt(buf + i);
            acc += ((v.x + v.y) + v.z) + v.w;
        }
    }
    if (i0 < n4) out[i0] = acc;
}

}  // extern "C"
