// switch_gpu.hip -- SGEMM family + read-bandwidth probe for gfx950 (the switch_gpu code object).
//
// Exported symbols keep the reference names and argument lists (switch_gpu.cu:5-8,41-43,59-62,
// 99-102,140-143) so a host that resolves them by name keeps working:
//   sgemm_tiled, sgemm_tiled4, sgemm_opt : (const float*A, const float*B, float*C, int M, int N, int K)
//   sgemm_naive                          : same arguments, one output per thread
//   membw_read4                          : (const float4*buf, float*out, int n4, int iters)
// plus sgemm_opt256, a larger-tile member with the same arguments, sgemm_splitk
//   (A, B, C, M, N, K, int S, float* ws, unsigned* cnt), the 64x64 tile with K split S ways,
// sgemm_small16 / sgemm_small32 (same arguments as the reference members), one 16x16 /
// 32x32 tile per block with the operands read straight into MFMA registers, no LDS staging,
// sgemm_kwave (same arguments), the 64x64 tile with K split over the block's waves and its
// operands loaded straight into MFMA registers, its edge form sgemm_kwave_edge (any M, N >= 64,
// any K), and their LDS-staged forms for operands past 2^31-byte windows, sgemm_kwave_wide and
// sgemm_kwave_edge_wide.
//
// C = A*B, fp32, row-major (A: MxK stride K, B: KxN stride N, C: MxN stride N), overwrite
// (alpha 1, beta 0).  Unlike the reference kernels, every shape is accepted: interior tiles
// of problems with 16-byte rows take dwordx4 loads, edge tiles, K tails and unaligned rows
// take masked loads, both through the same software pipeline.
//
// The tiled kernels run on the fp32 matrix cores: v_mfma_f32_32x32x2_f32 (true fp32 inputs,
// fp32 accumulate; no reduced-precision xf32).  A block of 64*WGM*WGN threads owns a BMxBN
// tile of C; each wave owns a (BM/WGM)x(BN/WGN) sub-tile held as 32x32 MFMA blocks.
// A and B k-slices of depth BK are staged through LDS, double-buffered (one barrier per
// slice, before the slice's last MFMA group on whole tiles, so the next slice's first
// operand reads overlap that group): A m-major with a 4-float row pad, B row-major with an
// 8-float pad.  The 64x64 and 128x128 members keep two slices' global loads in flight (their
// slices are short next to the load latency).  Tiles are walked with a grid-stride
// loop over a linear tile index, so any grid of 64*WGM*WGN-thread blocks is correct (surplus
// blocks exit); with one block per tile the index is remapped so each XCD (blocks are dealt
// round-robin to the 8 XCDs) works on a compact group of tiles that shares A and B panels in
// its own L2.  sgemm_splitk walks (tile, k-split) units the same way and sums a tile's splits
// in the last split to finish.  The small members (for problems whose few tiles cannot keep
// a slice pipeline busy) are described where they are defined.
#include <type_traits>

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
    static constexpr int KQ = BK / 4, NQ = BN / 4;          // float4 per A row / per B row
    static constexpr int A_PER_T = (BM * KQ) / NT;          // float4 loads per thread
    static constexpr int B_PER_T = (BK * NQ) / NT;
    static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be whole 32x32 blocks");
    static_assert(BK % 4 == 0 && (BM * KQ) % NT == 0 && (BK * NQ) % NT == 0, "load split");
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

// Per-thread constants of one tile's staging and operand reads.
template <int BM, int BN, int BK, int WGM, int WGN>
struct SgemmThread {
    using T = MfmaTile<BM, BN, BK, WGM, WGN>;
    int tid, wm, wn, l32, khalf;
    __device__ __forceinline__ SgemmThread() {
        tid = sgpu_tid();
        const int lane = tid & 63, wave = tid >> 6;
        wm = wave / WGN;
        wn = wave % WGN;
        l32 = lane & 31;
        khalf = lane >> 5;
    }
};

// D layout of a 32x32 block: lane l, acc r -> row 8*(r/4) + 4*(l/32) + r%4, col l%32.
template <int BM, int BN, int BK, int WGM, int WGN>
__device__ __forceinline__ void sgemm_store_c(float* __restrict__ C, int M, int N, int m0, int n0, bool interior,
                                              const SgemmThread<BM, BN, BK, WGM, WGN>& th,
                                              sgpu_f32x16 (&acc)[BM / WGM / 32][BN / WGN / 32]) {
    using T = MfmaTile<BM, BN, BK, WGM, WGN>;
#pragma unroll
    for (int i = 0; i < T::FM; i++)
#pragma unroll
        for (int j = 0; j < T::FN; j++) {
            const int gn = n0 + th.wn * T::WTN + j * 32 + th.l32;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int gm = m0 + th.wm * T::WTM + i * 32 + 8 * (r >> 2) + 4 * th.khalf + (r & 3);
                if (interior || (gm < M && gn < N)) C[(size_t)gm * N + gn] = acc[i][j][r];
            }
        }
}

// LDS layout of the pipeline: A m-major (row pitch BK+4 floats), B k-major
// (row pitch BN+8).  Both are written straight from the dwordx4 global loads.  Inside a
// slice the MFMA k-steps run in groups of four with the k order permuted per lane half:
// at step t of group g, lane half h supplies k = 8g + 4h + t, so a lane's four A operands of
// a group are four consecutive floats of one LDS row (one ds_read_b128; rows BK+4 apart put
// 16 lanes on 64 distinct banks) and its B operands are four single floats of rows
// 8g+4h+t (the two lane halves 4 rows = 32 banks apart).
template <int BM, int BN, int BK, int WGM, int WGN>
struct SgemmLdsM {
    static constexpr int LDAM = BK + 4, LDBM = BN + 8;
    float As[2][BM][LDAM];
    float Bs[2][BK][LDBM];
};

// MODE 0: interior tile, K whole slices, 16-byte rows: dwordx4 loads, as above.
// MODE 1 and 2: any tile, any K >= 1, rows of any 4-byte alignment, cdiv(K, BK) slices.
//   MODE 1 (A tile rows and B slices within 2^31 bytes): consecutive lanes load consecutive
//   floats (element j of a thread is A row tid/BK + j*NT/BK, k tid%BK; B row tid/BN + j*NT/BN,
//   column tid%BN) with buffer loads; rows past M or K fall outside the buffer's range and
//   read as zero, and k >= K or columns >= N are sent outside it (offset 2^31), so no mask
//   is applied to data.  Floats are written to LDS one each.
//   MODE 2 (larger operands): dwordx4-shaped map, each float loaded from a clamped
//   (in-bounds) 64-bit address and zeroed outside A or B when the slice is written to LDS.
template <int BM, int BN, int BK, int WGM, int WGN, int STORE_G, int MODE = 0, bool EARLY = false, int PF = 1>
__device__ __forceinline__ void sgemm_tile_fast_m(const float* __restrict__ A, const float* __restrict__ B,
                                                  int M, int N, int K, int lda, int m0, int n0,
                                                  SgemmLdsM<BM, BN, BK, WGM, WGN>& L,
                                                  const SgemmThread<BM, BN, BK, WGM, WGN>& th,
                                                  sgpu_f32x16 (&acc)[BM / WGM / 32][BN / WGN / 32]) {
    using T = MfmaTile<BM, BN, BK, WGM, WGN>;
    constexpr bool MASKED = MODE != 0;
    constexpr int NG = BK / 8;                    // 4-step groups per slice
    static_assert(BK % 8 == 0, "k slice of whole 8-deep groups");
    static_assert(STORE_G >= 0 && STORE_G < NG, "store point inside the slice");
    static_assert(!EARLY || (STORE_G < NG - 1 && NG % 2 == 0), "early barrier: store before the last group");
    static_assert(PF == 1 || (PF == 2 && MODE == 0), "two slices in flight on the dwordx4 path only");
    static_assert(T::NT % T::KQ == 0 && T::NT % T::NQ == 0, "whole rows per load round");
    static_assert(MODE != 1 || (T::NT % BK == 0 && T::NT % BN == 0), "lane map: whole rows per round");
    constexpr int AE = 4 * T::A_PER_T, BE = 4 * T::B_PER_T;   // staged floats per thread
    constexpr int AR = MODE == 1 ? T::NT / BK : 1, BR = MODE == 1 ? T::NT / BN : 1;
    constexpr unsigned kOut = 0x80000000u;       // an offset past every MODE-1 buffer range
    const int tid = th.tid, nk = MASKED ? (K + BK - 1) / BK : K / BK;
    const float* pa = A + (size_t)(m0 + tid / T::KQ) * lda + 4 * (tid % T::KQ);
    const float* pb = B + (size_t)(tid / T::NQ) * N + n0 + 4 * (tid % T::NQ);
    const size_t astep = (size_t)(T::NT / T::KQ) * lda, bstep_r = (size_t)(T::NT / T::NQ) * N;
    const size_t bstep = (size_t)BK * N;
    // MODE 1 map and buffers: A from row m0 (range: the tile's valid rows), B from row kt*BK
    const int ar = tid / BK, ak = tid % BK, bkr = tid / BN, bc = tid % BN;
    const unsigned a_off0 = (unsigned)(ar * lda + ak) * 4u, a_step = (unsigned)(AR * lda) * 4u;
    const unsigned b_off0 = (unsigned)(bkr * N + n0 + bc) * 4u, b_step = (unsigned)(BR * N) * 4u;
    const bool b_col_ok = n0 + bc < N;
    const __amdgpu_buffer_rsrc_t rs_a = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(A + (size_t)m0 * lda), (short)0, MODE == 1 ? min(M - m0, BM) * lda * 4 : 0, 0x00020000);
    // MODE 2 map
    const int ar0 = m0 + tid / T::KQ, ak0 = 4 * (tid % T::KQ);
    const int bk0 = tid / T::NQ, bn0 = n0 + 4 * (tid % T::NQ);
    // Staging registers: PF sets (PF = 2: slice kt+1 waits in one set while slice kt+2 loads
    // into the other).  Set indices are compile-time (set_c) everywhere.
    sgpu_f32x4 ras[PF][T::A_PER_T], rbs[PF][T::B_PER_T];
    sgpu_f32x4 (&ra)[T::A_PER_T] = ras[0];
    sgpu_f32x4 (&rb)[T::B_PER_T] = rbs[0];
    float sa[AE], sb[BE];
    auto load_slice = [&](int kt, auto set_c) __attribute__((always_inline)) {
        constexpr int SET = decltype(set_c)::value;
        if constexpr (MODE == 0) {
#pragma unroll
            for (int r = 0; r < T::A_PER_T; r++)
                ras[SET][r] = *reinterpret_cast<const sgpu_f32x4*>(pa + r * astep + (size_t)kt * BK);
#pragma unroll
            for (int r = 0; r < T::B_PER_T; r++)
                rbs[SET][r] = *reinterpret_cast<const sgpu_f32x4*>(pb + r * bstep_r + (size_t)kt * bstep);
        } else if constexpr (MODE == 1) {
            const unsigned ao = kt * BK + ak < K ? a_off0 + (unsigned)(kt * BK) * 4u : kOut;
#pragma unroll
            for (int j = 0; j < AE; j++)
                sa[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs_a, (int)(ao + j * a_step), 0, 0));
            const __amdgpu_buffer_rsrc_t rs_b = __builtin_amdgcn_make_buffer_rsrc(
                (void*)(B + (size_t)kt * BK * N), (short)0, min(K - kt * BK, BK) * N * 4, 0x00020000);
            const unsigned bo = b_col_ok ? b_off0 : kOut;
#pragma unroll
            for (int j = 0; j < BE; j++)
                sb[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs_b, (int)(bo + j * b_step), 0, 0));
        } else {
#pragma unroll
            for (int r = 0; r < T::A_PER_T; r++) {
                const float* rp = A + (size_t)min(ar0 + r * (T::NT / T::KQ), M - 1) * lda;
#pragma unroll
                for (int e = 0; e < 4; e++) ra[r][e] = rp[min(kt * BK + ak0 + e, K - 1)];
            }
#pragma unroll
            for (int r = 0; r < T::B_PER_T; r++) {
                const float* rp = B + (size_t)min(kt * BK + bk0 + r * (T::NT / T::NQ), K - 1) * N;
#pragma unroll
                for (int e = 0; e < 4; e++) rb[r][e] = rp[min(bn0 + e, N - 1)];
            }
        }
    };
    // MODE 2: zero the staged elements of slice kt that lie outside A or B
    auto mask_slice = [&](int kt) __attribute__((always_inline)) {
        if constexpr (MODE == 2) {
#pragma unroll
            for (int r = 0; r < T::A_PER_T; r++) {
                const bool row_ok = ar0 + r * (T::NT / T::KQ) < M;
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (!(row_ok && kt * BK + ak0 + e < K)) ra[r][e] = 0.0f;
            }
#pragma unroll
            for (int r = 0; r < T::B_PER_T; r++) {
                const bool k_ok = kt * BK + bk0 + r * (T::NT / T::NQ) < K;
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (!(k_ok && bn0 + e < N)) rb[r][e] = 0.0f;
            }
        }
    };
    auto store_slice = [&](int s, auto set_c) __attribute__((always_inline)) {
        constexpr int SET = decltype(set_c)::value;
        if constexpr (MODE != 1) {
#pragma unroll
            for (int r = 0; r < T::A_PER_T; r++) {
                const int idx = tid + r * T::NT;
                *reinterpret_cast<sgpu_f32x4*>(&L.As[s][idx / T::KQ][4 * (idx % T::KQ)]) = ras[SET][r];
            }
#pragma unroll
            for (int r = 0; r < T::B_PER_T; r++) {
                const int idx = tid + r * T::NT;
                *reinterpret_cast<sgpu_f32x4*>(&L.Bs[s][idx / T::NQ][4 * (idx % T::NQ)]) = rbs[SET][r];
            }
        } else {
#pragma unroll
            for (int j = 0; j < AE; j++) L.As[s][ar + j * AR][ak] = sa[j];
#pragma unroll
            for (int j = 0; j < BE; j++) L.Bs[s][bkr + j * BR][bc] = sb[j];
        }
    };
    auto read_group = [&](int s, int g, sgpu_f32x4* a, sgpu_f32x4* b) __attribute__((always_inline)) {
        const int kc = 8 * g + 4 * th.khalf;
#pragma unroll
        for (int i = 0; i < T::FM; i++)
            a[i] = *reinterpret_cast<const sgpu_f32x4*>(&L.As[s][th.wm * T::WTM + i * 32 + th.l32][kc]);
#pragma unroll
        for (int t = 0; t < 4; t++)                // step-major, so step 0 can start first
#pragma unroll
            for (int j = 0; j < T::FN; j++) b[j][t] = L.Bs[s][kc + t][th.wn * T::WTN + j * 32 + th.l32];
    };
    // The slice's memory instructions (next slice's global loads in group 0, next group's LDS
    // reads, the slice store in group STORE_G) are dealt out one per MFMA instead of issued in
    // bursts, so the MFMA stream never waits behind a full memory queue.
    // EARLY: the slice's barrier sits before its last group instead of after it, and that
    // group's MFMAs run under the LDS reads of the next slice's first group (the next slice
    // was stored at group STORE_G < NG-1; every read of this slice's buffer except the last
    // group's was issued, and waited for, before the barrier), so no LDS latency is exposed
    // between slices.
    // A slice with `more` loads slice kt_ld into staging set LS (in group 0) and writes set SS,
    // holding slice kt_st, to the idle buffer s^1 (at group STORE_G).
    sgpu_f32x4 a[2][T::FM], b[2][T::FN];
    using Z = std::integral_constant<int, 0>;
    auto slice = [&](int s, int kt_ld, int kt_st, auto more_c, auto ls_c, auto ss_c) __attribute__((always_inline)) {
        constexpr bool more = decltype(more_c)::value;
        constexpr int NMF = 4 * T::FM * T::FN;
        constexpr int NLD = (MASKED ? 4 : 1) * (T::A_PER_T + T::B_PER_T);   // global loads
        constexpr int LPM = (NLD + NMF - 1) / NMF;                            // ... per MFMA slot
        constexpr int NST = (MODE == 1 ? 4 : 1) * (T::A_PER_T + T::B_PER_T);  // LDS writes
        constexpr int WPM = (NST + NMF / 2 - 1) / (NMF / 2);                  // ... per slot (half group)
        if constexpr (!EARLY) read_group(s, 0, a[0], b[0]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int g = 0; g < NG; g++) {
            const int c = g & 1;
            constexpr bool rd_next = EARLY && more;    // last group reads the next slice's group 0
            if (rd_next && g == NG - 1) {
                __syncthreads();
                __builtin_amdgcn_sched_barrier(0);
            }
            if (more && g == 0) load_slice(kt_ld, ls_c);
            if (g + 1 < NG) read_group(s, g + 1, a[c ^ 1], b[c ^ 1]);
            else if (rd_next) read_group(s ^ 1, 0, a[c ^ 1], b[c ^ 1]);
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int i = 0; i < T::FM; i++)
#pragma unroll
                    for (int j = 0; j < T::FN; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[c][i][t], b[c][j][t], acc[i][j], 0, 0, 0);
            if (more && g == STORE_G) {
                if constexpr (MASKED) mask_slice(kt_st);
                store_slice(s ^ 1, ss_c);
            }
#pragma unroll
            for (int q = 0; q < NMF; q++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                      // 1 MFMA
                if (more && g == 0 && q * LPM < NLD)
                    __builtin_amdgcn_sched_group_barrier(0x020, LPM, 0);                // global loads
                if ((g + 1 < NG || rd_next) && q < T::FM + 4 * T::FN)
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                  // 1 LDS read
                if (more && g == STORE_G && q >= NMF / 2 && (q - NMF / 2) * WPM < NST)
                    __builtin_amdgcn_sched_group_barrier(0x200, WPM, 0);                // LDS writes
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    load_slice(0, Z{});
    if constexpr (MASKED) mask_slice(0);
    store_slice(0, Z{});
    if constexpr (PF == 2) {
        // Slice 1 into set 1 before the loop; slice kt (buffer kt & 1) loads slice kt+2 into
        // set kt & 1 and writes slice kt+1 from the other set, so each slice's loads have a
        // whole slice to land.  Loads past the last slice re-read slice nk-1 (never stored).
        using O = std::integral_constant<int, 1>;
        load_slice(min(1, nk - 1), O{});
        __syncthreads();
        if constexpr (EARLY) read_group(0, 0, a[0], b[0]);
        for (int kt = 0;; kt += 2) {
            if (kt + 1 >= nk) {
                slice(0, 0, 0, std::false_type{}, Z{}, Z{});
                break;
            }
            slice(0, min(kt + 2, nk - 1), kt + 1, std::true_type{}, Z{}, O{});
            if constexpr (!EARLY) __syncthreads();
            if (kt + 2 >= nk) {
                slice(1, 0, 0, std::false_type{}, O{}, O{});
                break;
            }
            slice(1, min(kt + 3, nk - 1), kt + 2, std::true_type{}, O{}, Z{});
            if constexpr (!EARLY) __syncthreads();
        }
    } else {
        __syncthreads();
        if constexpr (EARLY) read_group(0, 0, a[0], b[0]);
        for (int kt = 0; kt + 1 < nk; kt++) {
            slice(kt & 1, kt + 1, kt + 1, std::true_type{}, Z{}, Z{});
            if constexpr (!EARLY) __syncthreads();
        }
        slice((nk - 1) & 1, 0, 0, std::false_type{}, Z{}, Z{});
    }
    __syncthreads();
}

// Whole tiles of a problem with 16-byte rows and K whole slices run the dwordx4 pipeline
// with the slice store after 4-step group STORE_AT; LAYOUT 2: memory instructions spread one
// per MFMA; 3: as 2, with each slice's barrier moved before its last group; 4: as 3, with
// two slices' loads in flight.  All other tiles run the masked pipeline (spread, barrier at
// the end of the slice).
template <int BM, int BN, int BK, int WGM, int WGN, int STORE_AT, int LAYOUT, bool SPLIT = false>
__device__ __forceinline__ void sgemm_mfma(const float* __restrict__ A, const float* __restrict__ B,
                                           float* __restrict__ C, int M, int N, int K, int S = 1,
                                           float* __restrict__ ws = nullptr, unsigned* __restrict__ cnt = nullptr) {
    using T = MfmaTile<BM, BN, BK, WGM, WGN>;
    static_assert(STORE_AT >= 0 && LAYOUT >= 2 && LAYOUT <= 4, "store point and layout");
    __shared__ __attribute__((aligned(16))) SgemmLdsM<BM, BN, BK, WGM, WGN> LM;

    // The tile split assumes exactly NT = 256 threads per block (the kernels' launch bound);
    // any other block size is rejected by every thread alike (no barrier is reached, C is
    // left untouched).
    static_assert(T::NT == 256, "four waves per block");
    if (!sgpu_block256()) return;
    const SgemmThread<BM, BN, BK, WGM, WGN> th;

    const int ntm = (M + BM - 1) / BM, ntn = (N + BN - 1) / BN, ntiles = ntm * ntn;
    const int nb = sgpu_nblocks();
    const bool remap = !SPLIT && (nb == ntiles) && (ntiles % kXcds == 0);
    const bool aligned = ((K & 3) == 0) && ((N & 3) == 0) &&
                         ((((uintptr_t)A) | ((uintptr_t)B)) & 15) == 0;
    // Work units: (tile, k-split) pairs, split-major.  Split s covers slices [s*per, (s+1)*per)
    // of the cdiv(K, BK) slices; every split of a tile holds at least one slice (the launcher
    // chooses S so), and the last one may end in a partial slice.
    const int nsplit = SPLIT ? S : 1;
    const int per = SPLIT ? ((K + BK - 1) / BK + nsplit - 1) / nsplit : 0;
    const int nunits = ntiles * nsplit;
    auto unit = [&](int u, int& m0, int& n0, int& k0, int& kext) __attribute__((always_inline)) {
        int tm, tn;
        sgemm_tile_coords(SPLIT ? u % ntiles : u, ntm, ntn, remap, tm, tn);
        m0 = tm * BM;
        n0 = tn * BN;
        k0 = SPLIT ? (u / ntiles) * per * BK : 0;
        kext = SPLIT ? min(K - k0, per * BK) : K;
    };
    // A unit's result: with one split, straight to C; with several, the split hands its
    // partial tile to the tile's last split (the cross-block hand-off set out in
    // sgpu_device.h: device-coherent stores waited for, a counter, an acquire by the last
    // arriver), which sums all S in split order -- the same order whichever block is last --
    // and writes C.
    __shared__ int last_s;
    auto finish = [&](int u, int m0, int n0, bool interior, sgpu_f32x16 (&acc)[T::FM][T::FN]) __attribute__((always_inline)) {
        if constexpr (SPLIT) {
            if (nsplit > 1) {
                const int t = u % ntiles, sp = u / ntiles;
                constexpr int TILE = BM * BN;
                float* rec = ws + (size_t)(sp * ntiles + t) * TILE + th.tid;
#pragma unroll
                for (int i = 0; i < T::FM; i++)
#pragma unroll
                    for (int j = 0; j < T::FN; j++)
#pragma unroll
                        for (int r = 0; r < 16; r++)
                            __hip_atomic_store(rec + ((i * T::FN + j) * 16 + r) * T::NT, acc[i][j][r], __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
                __builtin_amdgcn_s_waitcnt(0);          // this wave's partial stores are acknowledged
                __syncthreads();
                if (th.tid == 0) {
                    last_s = __hip_atomic_fetch_add(cnt + t, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                             (unsigned)(nsplit - 1);
                    if (last_s) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");   // before the others' partials
                }
                __syncthreads();
                if (!last_s) return;
                // U splits per round, every load of a round issued before the first add (one
                // round trip per round, not per split); sums in split order.
                constexpr int U = 4;
                sgpu_f32x16 sum[T::FM][T::FN];
                for (int s0 = 0; s0 < nsplit; s0 += U) {
                    sgpu_f32x16 o[U][T::FM][T::FN];
#pragma unroll
                    for (int u = 0; u < U; u++) {
                        const int s2 = s0 + u;
                        const float* src = ws + (size_t)(s2 * ntiles + t) * TILE + th.tid;
#pragma unroll
                        for (int i = 0; i < T::FM; i++)
#pragma unroll
                            for (int j = 0; j < T::FN; j++)
#pragma unroll
                                for (int r = 0; r < 16; r++)
                                    o[u][i][j][r] = s2 >= nsplit || s2 == sp
                                                        ? acc[i][j][r]
                                                        : __hip_atomic_load(src + ((i * T::FN + j) * 16 + r) * T::NT,
                                                                            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
#pragma unroll
                    for (int u = 0; u < U; u++)
                        if (s0 + u < nsplit)
#pragma unroll
                            for (int i = 0; i < T::FM; i++)
#pragma unroll
                                for (int j = 0; j < T::FN; j++)
#pragma unroll
                                    for (int r = 0; r < 16; r++)
                                        sum[i][j][r] = s0 + u == 0 ? o[u][i][j][r] : sum[i][j][r] + o[u][i][j][r];
                }
                sgemm_store_c(C, M, N, m0, n0, interior, th, sum);
                if (th.tid == 0) __hip_atomic_store(cnt + t, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                return;
            }
        }
        sgemm_store_c(C, M, N, m0, n0, interior, th, acc);
    };

    // Per unit: interior tiles of a problem with 16-byte rows and a k range of whole slices
    // (at least two) take the dwordx4 pipeline; every other unit (edges, K tails, unaligned
    // rows) takes the same pipeline with masked loads (K = 0 writes zeros).  Each kind gets
    // its own loop, so neither carries the other's registers.
    {
        const bool kfast_k = aligned && K % BK == 0 && K >= 2 * BK;
        auto kfast = [&](int kext) __attribute__((always_inline)) {
            return SPLIT ? aligned && kext % BK == 0 && kext >= 2 * BK : kfast_k;
        };
        constexpr int SG = STORE_AT < BK / 8 ? STORE_AT : 0;      // a group index for the masked path
        // Buffer-load windows (BM rows of A, BK rows of B) within 2^31 bytes: MODE 1, else 2.
        // Each mode has its own loop (one accumulator set per loop, no merge of the two).
        const bool win = (long long)BM * K * 4 < 0x7fffffffLL && (long long)BK * N * 4 < 0x7fffffffLL;
        auto masked_tiles = [&](auto mode_c) __attribute__((always_inline)) {
            constexpr int MODE = decltype(mode_c)::value;
            for (int u = sgpu_bid(); u < nunits; u += nb) {
                int m0, n0, k0, kext;
                unit(u, m0, n0, k0, kext);
                const bool interior = (m0 + BM <= M) && (n0 + BN <= N);
                if (kfast(kext) && interior) continue;
                sgpu_f32x16 acc[T::FM][T::FN];
#pragma unroll
                for (int i = 0; i < T::FM; i++)
#pragma unroll
                    for (int j = 0; j < T::FN; j++)
#pragma unroll
                        for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;
                if (kext > 0)
                    sgemm_tile_fast_m<BM, BN, BK, WGM, WGN, SG, MODE, false>(
                        A + k0, B + (size_t)k0 * N, M, N, kext, K, m0, n0, LM, th, acc);
                finish(u, m0, n0, interior, acc);
            }
        };
        // Masked units first, then interior ones: with this order the interior loop's code
        // measured 7% faster on sgemm_tiled4 at 4096^3 (1% on sgemm_opt).
        if (win)
            masked_tiles(std::integral_constant<int, 1>{});
        else
            masked_tiles(std::integral_constant<int, 2>{});
        if (SPLIT ? aligned : kfast_k) {
            for (int u = sgpu_bid(); u < nunits; u += nb) {
                int m0, n0, k0, kext;
                unit(u, m0, n0, k0, kext);
                if (m0 + BM > M || n0 + BN > N || !kfast(kext)) continue;
                sgpu_f32x16 acc[T::FM][T::FN];
#pragma unroll
                for (int i = 0; i < T::FM; i++)
#pragma unroll
                    for (int j = 0; j < T::FN; j++)
#pragma unroll
                        for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;
                sgemm_tile_fast_m<BM, BN, BK, WGM, WGN, STORE_AT, 0, LAYOUT >= 3, LAYOUT == 4 ? 2 : 1>(
                    A + k0, B + (size_t)k0 * N, M, N, kext, K, m0, n0, LM, th, acc);
                finish(u, m0, n0, true, acc);
            }
        }
    }
}

// Small problems: one TSxTS tile of C per block of 256 threads (grid-stride over tiles), the
// operands read straight from global memory into MFMA registers (at these sizes A and B stay
// in L2, and there is no slice pipeline to fill), no LDS staging.  The four waves take
// interleaved k-groups (group g to wave g % 4) and sum their partial tiles through LDS in
// wave order.  Any M, N >= 1, K >= 0 with A and B under 2^31 bytes each; VEC (K % 4 == 0,
// A 16-byte aligned) reads A with 16-byte loads.
//   TS 32: v_mfma_f32_32x32x2f32, k-groups 8 deep: in group kb, lane half h = lane / 32
//          holds A[m][kb + 4h + t] and B[kb + 4h + t][n] for MFMA step t = 0..3.
//   TS 16: v_mfma_f32_16x16x4f32, k-groups 16 deep: lane quarter q = lane / 16 holds
//          A[m][kb + 4q + t] and B[kb + 4q + t][n] for step t.
// Reads go through buffer resources sized to A and B, the whole offset in the range-checked
// vector offset: B past row K-1 and A past its last element read as zero (no memory past
// either is touched); A elements past K (the next row's) are zeroed explicitly; columns past N
// read the next row's elements and are not stored, nor are rows past M.
template <int TS, int U, bool VEC>
__device__ __forceinline__ void sgemm_small_tiles(const float* __restrict__ A, const float* __restrict__ B,
                                                  float* __restrict__ C, int M, int N, int K,
                                                  float (&red)[4][TS * TS / 64][64]) {
    static_assert(TS == 16 || TS == 32, "tile size");
    constexpr int R = TS * TS / 64;               // accumulator registers per lane
    constexpr int KG = 4 * (64 / TS);             // k per group
    typedef float accv __attribute__((ext_vector_type(R)));
    const int tid = sgpu_tid(), lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = lane % TS, hq = lane / TS;
    const int ntn = (N + TS - 1) / TS, ntiles = ((M + TS - 1) / TS) * ntn;
    const int ng = (K + KG - 1) / KG;                        // k-groups
    const int nper = ng > wave ? (ng - wave + 3) / 4 : 0;    // this wave's groups
    const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc((void*)A, (short)0, M * K * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc((void*)B, (short)0, K * N * 4, 0x00020000);
    for (int tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {   // block-uniform loop
        const int m0 = (tile / ntn) * TS, n0 = (tile % ntn) * TS;
        // byte offsets of this lane's k = 4*hq in its A row and its B column
        const int aoff = ((m0 + li) * K + 4 * hq) * 4, boff = (4 * hq * N + n0 + li) * 4;
        sgpu_f32x4 a[2][U], b[2][U];
        // The whole byte offset of every load, k part included, is its vector offset: the
        // hardware range check covers the vector offset but not the scalar offset field, so
        // only this way do B rows past K-1 and A elements past A's end read as zero without
        // touching memory past either operand.  Batches load k-groups strictly in order, so
        // the offsets are five running registers advanced in place by one group stride.
        unsigned va = (unsigned)(aoff + wave * KG * 4), vb[4];
#pragma unroll
        for (int t = 0; t < 4; t++) vb[t] = (unsigned)(boff + (wave * KG + t) * N * 4);
        const unsigned astride = 4u * KG * 4u, bstride = 4u * KG * (unsigned)N * 4u;   // 4 waves' groups
        auto load = [&](int i0, auto set_c) __attribute__((always_inline)) {
            constexpr int SET = decltype(set_c)::value;
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int kb = (wave + 4 * (i0 + u)) * KG;          // wave-uniform
                if constexpr (VEC) {
                    a[SET][u] = __builtin_bit_cast(sgpu_f32x4, __builtin_amdgcn_raw_buffer_load_b128(rsa, (int)va, 0, 0));
                } else {
#pragma unroll
                    for (int t = 0; t < 4; t++)
                        a[SET][u][t] = __builtin_bit_cast(
                            float, __builtin_amdgcn_raw_buffer_load_b32(rsa, (int)(va + t * 4u), 0, 0));
                }
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    if (kb + 4 * hq + t >= K) a[SET][u][t] = 0.0f;
                    b[SET][u][t] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsb, (int)vb[t], 0, 0));
                    vb[t] += bstride;
                }
                va += astride;
            }
        };
        accv acc0 = {}, acc1 = {};                 // two chains: even and odd steps
        auto mfma = [&](auto set_c) __attribute__((always_inline)) {
            constexpr int SET = decltype(set_c)::value;
#pragma unroll
            for (int u = 0; u < U; u++)
#pragma unroll
                for (int t = 0; t < 4; t += 2) {
                    if constexpr (TS == 32) {
                        acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a[SET][u][t], b[SET][u][t], acc0, 0, 0, 0);
                        acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a[SET][u][t + 1], b[SET][u][t + 1], acc1, 0, 0, 0);
                    } else {
                        acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a[SET][u][t], b[SET][u][t], acc0, 0, 0, 0);
                        acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(a[SET][u][t + 1], b[SET][u][t + 1], acc1, 0, 0, 0);
                    }
                }
        };
        using S0 = std::integral_constant<int, 0>;
        using S1 = std::integral_constant<int, 1>;
        // batches of U groups, the next batch's loads issued before this batch's MFMAs
        if (nper > 0) load(0, S0{});
        for (int i = 0; i < nper; i += 2 * U) {
            if (i + U < nper) load(i + U, S1{});
            mfma(S0{});
            if (i + U >= nper) break;
            if (i + 2 * U < nper) load(i + 2 * U, S0{});
            mfma(S1{});
        }
#pragma unroll
        for (int r = 0; r < R; r++) red[wave][r][lane] = acc0[r] + acc1[r];
        __syncthreads();
        // D layout: TS 32, lane l, register r -> row 8*(r/4) + 4*(l/32) + r%4, column l%32;
        // TS 16 -> row 4*(l/16) + r, column l%16
#pragma unroll
        for (int e = tid; e < R * 64; e += 256) {
            const int r = e / 64, l = e % 64;
            const int row = TS == 32 ? 8 * (r / 4) + 4 * (l / 32) + r % 4 : 4 * (l / 16) + r;
            const int gm = m0 + row, gn = n0 + l % TS;
            const float v = ((red[0][r][l] + red[1][r][l]) + red[2][r][l]) + red[3][r][l];
            if (gm < M && gn < N) C[(size_t)gm * N + gn] = v;
        }
        __syncthreads();
    }
}
template <int TS, int U>
__device__ __forceinline__ void sgemm_small(const float* __restrict__ A, const float* __restrict__ B,
                                            float* __restrict__ C, int M, int N, int K) {
    __shared__ __attribute__((aligned(16))) float red[4][TS * TS / 64][64];
    if (!sgpu_block256()) return;
    if (K % 4 == 0 && ((uintptr_t)A & 15) == 0) sgemm_small_tiles<TS, U, true>(A, B, C, M, N, K, red);
    else sgemm_small_tiles<TS, U, false>(A, B, C, M, N, K, red);
}

// Lanes of one wave exchanging data through LDS: every LDS access of this wave before the
// call happens before every access after it.
__device__ __forceinline__ void kw_wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// sgemm_kwave: a 64x64 tile of C per block of four waves, each wave computing the WHOLE tile
// (2x2 blocks of 32x32 MFMA accumulators) over its own quarter of the 32-deep k-slices, in
// its own double-buffered LDS staging.  No barrier is shared by the waves inside the k loop:
// a wave's slice pipeline waits only for its own loads and LDS traffic, so one wave per SIMD
// runs its MFMAs without the block-wide slice barrier the 64x64 member pays every 16 MFMAs
// (here 64 MFMAs separate a wave's slice boundaries).  The four partial tiles are summed in
// wave order through LDS at the end (deterministic).  Problems: M, N multiples of 64, K a
// multiple of 32, A and B 16-byte aligned (any other shape is left to the other members:
// the kernel returns without writing C).
//   Staging per wave and slice: A rows 8q + lane/8, float4 lane%8 (m-major, pitch 36); B
//   k-rows 4q + lane/16, float4 lane%16 (pitch 72); the MFMA operands are read in 8-deep
//   groups exactly as the LDS-staged members read theirs (lane half h, step t -> k = 8g+4h+t).
//   Inside a slice: group g's 16 MFMAs run while group g+1's operands are read; the next
//   slice (already in registers) is stored to the other buffer during group 1 and the loads
//   of the slice after it are issued during group 2; group 3 starts with a wave sync and reads
//   the next slice's first group.  Memory instructions are dealt out one per MFMA.
// EDGE (sgemm_kwave_edge): any M, N >= 64, any K >= 1, rows of any float alignment.  A partial
//   last row of tiles is computed as the 64 rows ending at row M-1 and stored from row m0 on;
//   a partial last column of tiles likewise.  With K % 32 != 0 the partial k-slice is slice 0
//   (k < K % 32; the later slices shifted to end at K): it reads zeros past K % 32 (A's
//   elements element-wise past the last whole quad, B's rows past it not at all), and only the
//   prologue of the wave holding slice 0 loads it, so every slice of the pipelined loop is
//   whole, as in the exact member.
// TH (with EDGE, N % 64 == 1, the last column of whole tiles): the tile also computes column
//   N-1 of its rows.  Lane l stages that column's element of the slice's k-row l%32 in Bt; each
//   group's A operands already in registers (rows l32 and 32+l32, k = 8g+4h+t) meet it in 8
//   VALU FMAs, and the four waves' partials are summed at the end.  One column costs a few
//   VALU FMAs per MFMA group instead of a 64-column tile of MFMAs.
constexpr int KW_BK = 32, KW_PA = KW_BK + 4, KW_PB = 64 + 8;
struct KwaveLds {
    float As[2][64][KW_PA];
    float Bs[2][KW_BK][KW_PB];
};
struct KwaveLdsEdge : KwaveLds {
    float Bt[2][KW_BK];           // column N-1 of the slice's k-rows (TH tiles)
};
template <bool EDGE, bool TH, class Lds>
__device__ __forceinline__ void sgemm_kwave_tile(const float* __restrict__ A, const float* __restrict__ B,
                                                 float* __restrict__ C, int M, int N, int K, int m0, int n0,
                                                 Lds& L, sgpu_f32x4* __restrict__ red) {
    static_assert(EDGE || !TH, "the extra column is an edge case");
    const int lane = sgpu_tid() & 63;
    const int wave = EDGE ? __builtin_amdgcn_readfirstlane(sgpu_tid() >> 6) : sgpu_tid() >> 6;
    const int l32 = lane & 31, h = lane >> 5;
    const int nk = EDGE ? (K + KW_BK - 1) / KW_BK : K / KW_BK;
    // EDGE, K % 32 != 0: slice 0 is the partial one, k in [0, K % 32), and slice s >= 1 covers
    // k from 32 s - kshift; only the prologue of the wave holding slice 0 loads a partial slice
    const int kpart = EDGE ? K % KW_BK : 0;
    const int kshift = kpart ? KW_BK - kpart : 0;
    const int s0 = wave * nk / 4, s1 = (wave + 1) * nk / 4;      // this wave's slices
    const int mt = EDGE ? min(m0, M - 64) : m0;                  // the tile's first computed row
    const int nt = EDGE ? min(n0, N - 64) : n0;                  // and column
    const float* pa = A + (size_t)(mt + (lane >> 3)) * K + 4 * (lane & 7);
    const float* pb = B + (size_t)(lane >> 4) * N + nt + 4 * (lane & 15);
    const size_t astep = (size_t)8 * K, bstep = (size_t)4 * N;
    sgpu_f32x4 ra[8], rb[8];
    float tb = 0.0f;                                             // TH: B[k of slice row l%32][N-1]
    const float* pt = B + (size_t)l32 * N + (N - 1);
    // a whole slice s (s >= 1 when K % 32 != 0: slice 0 is then the partial one)
    auto load_whole = [&](int s) __attribute__((always_inline)) {
        const size_t k0 = (size_t)s * KW_BK - kshift;
        const float* a = pa + k0;
        const float* b = pb + k0 * N;
#pragma unroll
        for (int q = 0; q < 8; q++) ra[q] = sgpu_ld4<!EDGE>(a + q * astep);
#pragma unroll
        for (int q = 0; q < 8; q++) rb[q] = sgpu_ld4<!EDGE>(b + q * bstep);
        if constexpr (TH) tb = pt[k0 * N];
    };
    // the partial slice 0: k >= K % 32 reads as zero, nothing past A or B is touched
    auto load_part = [&]() __attribute__((always_inline)) {
        const int kq = 4 * (lane & 7);
#pragma unroll
        for (int q = 0; q < 8; q++) {
            const float* a = pa + q * astep;
            if (kq + 3 < kpart) {
                ra[q] = sgpu_ld4<!EDGE>(a);
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++) ra[q][e] = kq + e < kpart ? a[e] : 0.0f;
            }
        }
#pragma unroll
        for (int q = 0; q < 8; q++)
            rb[q] = (lane >> 4) + 4 * q < kpart ? sgpu_ld4<!EDGE>(pb + (size_t)(4 * q) * N)
                                                : sgpu_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (TH) tb = l32 < kpart ? pt[0] : 0.0f;
    };
    auto load = [&](int s) __attribute__((always_inline)) {
        if (EDGE && kpart && s == 0) load_part();
        else load_whole(s);
    };
    auto store = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < 8; q++)
            *reinterpret_cast<sgpu_f32x4*>(&L.As[buf][8 * q + (lane >> 3)][4 * (lane & 7)]) = ra[q];
#pragma unroll
        for (int q = 0; q < 8; q++)
            *reinterpret_cast<sgpu_f32x4*>(&L.Bs[buf][4 * q + (lane >> 4)][4 * (lane & 15)]) = rb[q];
        if constexpr (TH) L.Bt[buf][l32] = tb;                   // lanes l and l+32 store the same value
    };
    sgpu_f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;
    sgpu_f32x4 a[2][2], b[2][2];                                  // [operand set][block]
    float tacc[2] = {0.0f, 0.0f};                                 // TH: rows l32, 32+l32 of column N-1
    sgpu_f32x4 tk[2];                                             // TH: [operand set] column N-1, k = kc..kc+3
    auto read_group = [&](int buf, int g, auto set_c) __attribute__((always_inline)) {
        constexpr int RS = decltype(set_c)::value;
        const int kc = 8 * g + 4 * h;
#pragma unroll
        for (int i = 0; i < 2; i++) a[RS][i] = *reinterpret_cast<const sgpu_f32x4*>(&L.As[buf][i * 32 + l32][kc]);
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int j = 0; j < 2; j++) b[RS][j][t] = L.Bs[buf][kc + t][j * 32 + l32];
        if constexpr (TH) tk[RS] = *reinterpret_cast<const sgpu_f32x4*>(&L.Bt[buf][kc]);
    };
    using Z = std::integral_constant<int, 0>;
    using O = std::integral_constant<int, 1>;
    // ST: this slice stores the next one (and reads its first group); LD: it loads slice s+2
    // (always a whole slice: s+2 >= 2).
    auto slice = [&](int s, auto st_c, auto ld_c) __attribute__((always_inline)) {
        constexpr bool ST = decltype(st_c)::value, LD = decltype(ld_c)::value;
        const int buf = (s - s0) & 1;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            if (g == 3 && ST) kw_wave_sync();                     // the next slice's stores are visible
            __builtin_amdgcn_sched_barrier(0);
            if (g + 1 < 4) {
                if (g & 1) read_group(buf, g + 1, Z{});
                else read_group(buf, g + 1, O{});
            } else if (ST) {
                read_group(buf ^ 1, 0, Z{});
            }
            if (g == 1 && ST) store(buf ^ 1);
            if (g == 2 && LD) load_whole(s + 2);
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        if (g & 1)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[1][i][t], b[1][j][t], acc[i][j], 0, 0, 0);
                        else
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[0][i][t], b[0][j][t], acc[i][j], 0, 0, 0);
                    }
            if constexpr (TH) {
#pragma unroll
                for (int t = 0; t < 4; t++)
#pragma unroll
                    for (int i = 0; i < 2; i++)
                        tacc[i] = (g & 1) ? __builtin_fmaf(a[1][i][t], tk[1][t], tacc[i])
                                          : __builtin_fmaf(a[0][i][t], tk[0][t], tacc[i]);
            }
            // TH adds one operand read per group, one LDS store and one global load per slice
#pragma unroll
            for (int q = 0; q < 16; q++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                            // 1 MFMA
                if ((g + 1 < 4 || ST) && q < (TH ? 7 : 6)) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // operand read
                if (g == 1 && ST) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);                // LDS store
                if (g == 1 && ST && TH && q == 15) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
                if (g == 2 && LD) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                // global load
                if (g == 2 && LD && TH && q == 15) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    if (s0 < s1) {
        load(s0);
        store(0);
        if (s0 + 1 < s1) load(s0 + 1);
        kw_wave_sync();
        read_group(0, 0, Z{});
        int s = s0;
        for (; s + 2 < s1; s++) slice(s, std::true_type{}, std::true_type{});
        if (s + 1 < s1) {
            slice(s, std::true_type{}, std::false_type{});
            s++;
        }
        slice(s, std::false_type{}, std::false_type{});
    }
    // Partial tiles: lane l's accumulator registers 4rq..4rq+3 of block (i, j) at
    // red[((w*4 + 2i+j)*4 + rq)*64 + l]; wave w then finishes block (w/2, w%2), summing the
    // four waves' partials in wave order.  D layout: lane l, register r -> row
    // 8*(r/4) + 4*(l/32) + r%4, column l%32 of the block.
    __syncthreads();                                              // every wave is done with its staging
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int rq = 0; rq < 4; rq++)
                red[((wave * 4 + i * 2 + j) * 4 + rq) * 64 + lane] =
                    sgpu_f32x4{acc[i][j][4 * rq], acc[i][j][4 * rq + 1], acc[i][j][4 * rq + 2], acc[i][j][4 * rq + 3]};
    // TH: the column's partials after the tile partials, tred[(w*2 + h)*64 + row]; wave 0 sums
    // them in (wave, h) order
    float* tred = reinterpret_cast<float*>(red + 4 * 4 * 4 * 64);
    if constexpr (TH) {
#pragma unroll
        for (int i = 0; i < 2; i++) tred[(wave * 2 + h) * 64 + i * 32 + l32] = tacc[i];
    }
    __syncthreads();
    if constexpr (TH) {
        if (wave == 0) {
            float v = 0.0f;
#pragma unroll
            for (int w = 0; w < 8; w++) v += tred[w * 64 + lane];
            if (mt + lane >= m0) C[(size_t)(mt + lane) * N + (N - 1)] = v;
        }
    }
    const int bi = wave >> 1, bj = wave & 1, blk = wave;
    sgpu_f32x4 p[4][4];
#pragma unroll
    for (int w = 0; w < 4; w++)
#pragma unroll
        for (int rq = 0; rq < 4; rq++) p[w][rq] = red[((w * 4 + blk) * 4 + rq) * 64 + lane];
#pragma unroll
    for (int rq = 0; rq < 4; rq++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float v = ((p[0][rq][e] + p[1][rq][e]) + p[2][rq][e]) + p[3][rq][e];
            if constexpr (EDGE) p[0][rq][e] = v;
            else C[(size_t)(m0 + bi * 32 + 8 * rq + 4 * h + e) * N + n0 + bj * 32 + l32] = v;
        }
    // EDGE: a clamped edge tile stores only its new rows and columns, every other tile all of
    // them (the per-element test costs ~0.7 us a launch when every tile takes it)
    if constexpr (EDGE) {
        if (mt == m0 && nt == n0) {
#pragma unroll
            for (int rq = 0; rq < 4; rq++)
#pragma unroll
                for (int e = 0; e < 4; e++)
                    C[(size_t)(m0 + bi * 32 + 8 * rq + 4 * h + e) * N + n0 + bj * 32 + l32] = p[0][rq][e];
        } else {
#pragma unroll
            for (int rq = 0; rq < 4; rq++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int gm = mt + bi * 32 + 8 * rq + 4 * h + e, gn = nt + bj * 32 + l32;
                    if (gm >= m0 && gn >= n0) C[(size_t)gm * N + gn] = p[0][rq][e];
                }
        }
    }
    __syncthreads();                                              // the staging is reused by the next tile
}

// The same K-over-waves tile with each wave's MFMA operands loaded straight from memory into
// registers in the 32x32x2 operand layout: no LDS staging, no wave syncs in the k loop
// (sgemm_kwave, sgemm_kwave_edge).  A 64-row A panel and a 16-row B slice must each span less
// than 2^31 bytes (kd_fits: every buffer offset is a non-negative int); sgemm_kwave_tile above,
// with 64-bit addresses, takes larger operands (the *_wide kernels).
//   Slices are KD_SD = 16 deep.  In a slice starting at k0, lane (l32, h) holds A rows
//   mt+l32 and mt+32+l32 at k0+8h .. k0+8h+7 (two 16-byte loads per row) and, for MFMA step
//   t = 0..7, row k0+8h+t of B at columns nt+2*l32 and nt+2*l32+1 (one 8-byte load): column
//   block j of the tile is columns nt+2c+j (c = 0..31), so one load feeds both column blocks and
//   a lane stores C two adjacent columns at a time.  MFMA step t sums k = k0+8h+t over the two
//   lane halves for all four 32x32 blocks.
//   Two register sets alternate between slices, and each register is reloaded with the slice
//   after next right after the MFMAs that read it have issued, so a slice's loads are in flight
//   for about two slices of MFMAs (the same structure with a whole set loaded one slice ahead
//   stalls on the load latency).  Loads go through buffer resources rebased to each slice, with
//   every offset in range, so nothing is masked in the loop.
// EDGE: as sgemm_kwave_tile's EDGE (clamped edge tiles stored from their first new row and
//   column, any K, rows of any float alignment), with the partial slice (k < K % 16) loaded
//   element by element by the wave holding slice 0: A elements and B rows past K % 16 read as
//   zero (clamped in-range addresses, then replaced), so a non-finite value never meets a
//   padded zero.
// TH (EDGE, N % 64 == 1, the last column of whole tiles): lane (l32, h) also loads column N-1
//   of its eight B rows per slice and meets its A operands in 16 VALU FMAs per slice, issued
//   together before the slice's MFMAs; the eight (wave, lane half) partials of each row are
//   summed at the end.
constexpr int KD_SD = 16;
__host__ __device__ constexpr bool kd_fits(long long N, long long K) {
    return K * 64 * 4 < 2147483648LL && N * KD_SD * 4 < 2147483648LL;
}
typedef float kd_f32x2 __attribute__((ext_vector_type(2)));
typedef float kd_f32x2_a4 __attribute__((ext_vector_type(2), aligned(4)));
template <bool EDGE, bool TH>
__device__ __forceinline__ void sgemm_kdirect_tile(const float* __restrict__ A, const float* __restrict__ B,
                                                   float* __restrict__ C, int M, int N, int K, int m0, int n0,
                                                   sgpu_f32x4* __restrict__ red) {
    static_assert(EDGE || !TH, "the extra column is an edge case");
    constexpr int NST = KD_SD / 2;                                // MFMA steps per slice
    const int lane = sgpu_tid() & 63, wave = __builtin_amdgcn_readfirstlane(sgpu_tid() >> 6);
    const int l32 = lane & 31, h = lane >> 5;
    const int nk = EDGE ? (K + KD_SD - 1) / KD_SD : K / KD_SD;
    const int kpart = EDGE ? K % KD_SD : 0;                       // slice 0 is partial when != 0
    const int kshift = kpart ? KD_SD - kpart : 0;
    const int s0 = wave * nk / 4, s1 = (wave + 1) * nk / 4;      // this wave's slices
    const int mt = EDGE ? min(m0, M - 64) : m0;
    const int nt = EDGE ? min(n0, N - 64) : n0;
    // byte offsets inside a slice's resources
    const unsigned va0 = ((unsigned)l32 * K + NST * h) * 4u, va1 = ((unsigned)(32 + l32) * K + NST * h) * 4u;
    const unsigned vb = ((unsigned)NST * h * N + 2 * l32) * 4u;
    const unsigned vt = ((unsigned)NST * h * N + (N - 1 - nt)) * 4u;
    sgpu_f32x4 a[2][2][2];                                        // [set][row block][quad]
    kd_f32x2 b[2][NST];                                           // [set][step]: columns 2c, 2c+1
    float tb[2][NST];                                             // TH: [set][step] column N-1
    struct Rs {
        __amdgpu_buffer_rsrc_t a, b;
    };
    // slice s >= 1 starts at k0 = 16 s - kshift; slice 0 (whole or partial) at k0 = 0.  With
    // live false both ranges are empty: every load through them returns zero and touches nothing.
    auto rsrc = [&](int s, bool live = true) __attribute__((always_inline)) -> Rs {
        const long long k0 = s ? (long long)s * KD_SD - kshift : 0;
        return {__builtin_amdgcn_make_buffer_rsrc((void*)(A + (size_t)mt * K + k0), (short)0,
                                                  live ? (int)((64LL * K - k0) * 4) : 0, 0x00020000),
                __builtin_amdgcn_make_buffer_rsrc((void*)(B + (size_t)k0 * N + nt), (short)0,
                                                  live ? (int)((long long)KD_SD * N * 4) : 0, 0x00020000)};
    };
    auto lda = [&](const Rs& r, unsigned off) __attribute__((always_inline)) {
        return __builtin_bit_cast(sgpu_f32x4, __builtin_amdgcn_raw_buffer_load_b128(r.a, (int)off, 0, 0));
    };
    auto ldb = [&](const Rs& r, int st) __attribute__((always_inline)) {
        return __builtin_bit_cast(kd_f32x2, __builtin_amdgcn_raw_buffer_load_b64(r.b, (int)vb, st * N * 4, 0));
    };
    auto ldt = [&](const Rs& r, int st) __attribute__((always_inline)) {
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r.b, (int)vt, st * N * 4, 0));
    };
    // a whole slice s into set D (s >= 1 when K % 16 != 0; live false: zeros, nothing read)
    auto load_whole = [&](int s, auto d_c, bool live = true) __attribute__((always_inline)) {
        constexpr int D = decltype(d_c)::value;
        const Rs r = rsrc(s, live);
#pragma unroll
        for (int v = 0; v < 2; v++) {
            a[D][0][v] = lda(r, va0 + 16 * v);
            a[D][1][v] = lda(r, va1 + 16 * v);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                b[D][4 * v + e] = ldb(r, 4 * v + e);
                if constexpr (TH) tb[D][4 * v + e] = ldt(r, 4 * v + e);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    // EDGE, K % 16 != 0: the partial slice 0 in registers of its own (pa, pb, pt).  An element at
    // k >= K % 16 is given the offset 2^31, past the resource's range (under 2^31 bytes), so the
    // hardware returns zero without touching memory: no loaded value is selected on, and the
    // loads need not complete before the pipeline's loads are issued.
    sgpu_f32x4 pa[2][2];
    kd_f32x2 pb[NST];
    float pt[NST];
    auto load_part = [&](bool live) __attribute__((always_inline)) {
        const Rs r = rsrc(0, live);
        constexpr unsigned OUT = 0x80000000u;
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int v = 0; v < 2; v++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int k = NST * h + 4 * v + e;
                    const unsigned off = k < kpart ? ((unsigned)(32 * i + l32) * K + k) * 4u : OUT;
                    pa[i][v][e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r.a, (int)off, 0, 0));
                }
#pragma unroll
        for (int st = 0; st < NST; st++) {
            const int row = NST * h + st;
            const unsigned ro = (unsigned)row * N * 4u;
            pb[st] = __builtin_bit_cast(
                kd_f32x2, __builtin_amdgcn_raw_buffer_load_b64(r.b, (int)(row < kpart ? ro + 8u * l32 : OUT), 0, 0));
            if constexpr (TH)
                pt[st] = __builtin_bit_cast(
                    float, __builtin_amdgcn_raw_buffer_load_b32(
                               r.b, (int)(row < kpart ? ro + (unsigned)(N - 1 - nt) * 4u : OUT), 0, 0));
        }
    };
    sgpu_f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;
    // TH: rows l32 and 32+l32 of column N-1, in two chains (even and odd MFMA steps) summed at
    // the end
    float tacc[2][2] = {{0.0f, 0.0f}, {0.0f, 0.0f}};
    // TH: a slice's 16 column FMAs, issued together ahead of its MFMAs (0.2-0.3 µs a launch
    // faster than one pair after each MFMA step)
    auto column = [&](const sgpu_f32x4 (&xa)[2][2], const float (&xt)[NST]) __attribute__((always_inline)) {
#pragma unroll
        for (int st = 0; st < NST; st++)
#pragma unroll
            for (int i = 0; i < 2; i++) tacc[st & 1][i] = __builtin_fmaf(xa[i][st >> 2][st & 3], xt[st], tacc[st & 1][i]);
    };
    // MFMA step st on operands xa (two row blocks' quads) and xb (column pair)
    auto step = [&](const sgpu_f32x4 (&xa)[2][2], const kd_f32x2& xb, int st) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(xa[i][st >> 2][st & 3], xb[j], acc[i][j], 0, 0, 0);
    };
    // the MFMAs of the slice in set D, each register of the set reloaded with slice sn as soon
    // as the MFMAs reading it have issued (RELOAD false: the last slice, nothing to load)
    auto slice = [&](auto d_c, int sn, auto reload_c) __attribute__((always_inline)) {
        constexpr int D = decltype(d_c)::value;
        constexpr bool RELOAD = decltype(reload_c)::value;
        Rs r;
        if constexpr (RELOAD) r = rsrc(sn);
        if constexpr (TH) column(a[D], tb[D]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int st = 0; st < NST; st++) {
            step(a[D], b[D][st], st);
            if constexpr (RELOAD) {
                if ((st & 3) == 3) {
                    a[D][0][st >> 2] = lda(r, va0 + 16 * (st >> 2));
                    a[D][1][st >> 2] = lda(r, va1 + 16 * (st >> 2));
                }
                b[D][st] = ldb(r, st);
                if constexpr (TH) tb[D][st] = ldt(r, st);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    using Z = std::integral_constant<int, 0>;
    using O = std::integral_constant<int, 1>;
    // Before the loop: the partial slice (EDGE, only in the wave holding slice 0), then every
    // wave's first two whole slices, unconditionally (a wave with one re-reads it, a wave with
    // none reads nothing: empty ranges return zeros).  Every path into the loop then has the same
    // loads newest in flight in the same order, which keeps the compiler's wait counts in the
    // loop exact (a load issued after them on one path only makes them all conservative).  The
    // wave holding a partial slice computes it before its whole slices sw...
    const bool part = EDGE && kpart && s0 == 0 && s0 < s1;
    const int sw = part ? 1 : s0;                                 // first whole slice
    if (part) load_part(true);
    __builtin_amdgcn_sched_barrier(0);
    load_whole(sw, Z{}, sw < s1);
    load_whole(min(sw + 1, max(s1 - 1, sw)), O{}, sw < s1);
    if (part) {
#pragma unroll
        for (int st = 0; st < NST; st++) step(pa, pb[st], st);
        if constexpr (TH) column(pa, pt);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (sw < s1) {
        // pairs of slices; the reloads of the last pair re-read slice s1-1 (in range, unused)
        int s = sw;
        for (; s + 2 <= s1; s += 2) {
            slice(Z{}, min(s + 2, s1 - 1), std::true_type{});
            slice(O{}, min(s + 3, s1 - 1), std::true_type{});
        }
        if (s < s1) slice(Z{}, 0, std::false_type{});
    }
    // Partial tiles: lane l's accumulator registers 4rq..4rq+3 of block (i, j) at
    // red[((w*4 + 2i+j)*4 + rq)*64 + l] (red is used by nothing else: no barrier before it).
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int rq = 0; rq < 4; rq++)
                red[((wave * 4 + i * 2 + j) * 4 + rq) * 64 + lane] =
                    sgpu_f32x4{acc[i][j][4 * rq], acc[i][j][4 * rq + 1], acc[i][j][4 * rq + 2], acc[i][j][4 * rq + 3]};
    float* tred = reinterpret_cast<float*>(red + 4 * 4 * 4 * 64);
    if constexpr (TH) {
#pragma unroll
        for (int i = 0; i < 2; i++) tred[(wave * 2 + h) * 64 + i * 32 + l32] = tacc[0][i] + tacc[1][i];
    }
    __syncthreads();
    if constexpr (TH) {
        if (wave == 0) {
            float v = 0.0f;
#pragma unroll
            for (int w = 0; w < 8; w++) v += tred[w * 64 + lane];
            if (mt + lane >= m0) __builtin_nontemporal_store(v, C + (size_t)(mt + lane) * N + (N - 1));
        }
    }
    // Wave w finishes row block w/2, accumulator quads 2(w%2) and 2(w%2)+1 of both column
    // blocks, summing the four waves' partials in wave order.  D layout: lane l, register r ->
    // row 8*(r/4) + 4*(l/32) + r%4 of the block; column block j, lane l -> column nt + 2*(l%32) + j.
    const int bi = wave >> 1;
    const bool whole = !EDGE || (mt == m0 && nt == n0);
#pragma unroll
    for (int q = 0; q < 2; q++) {
        const int rq = 2 * (wave & 1) + q;
        sgpu_f32x4 v[2];
#pragma unroll
        for (int j = 0; j < 2; j++) {
            sgpu_f32x4 p[4];
#pragma unroll
            for (int w = 0; w < 4; w++) p[w] = red[((w * 4 + bi * 2 + j) * 4 + rq) * 64 + lane];
            v[j] = ((p[0] + p[1]) + p[2]) + p[3];
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int gm = mt + bi * 32 + 8 * rq + 4 * h + e, gn = nt + 2 * l32;
            float* dst = C + (size_t)gm * N + gn;
            if (whole) {
                __builtin_nontemporal_store(kd_f32x2_a4{v[0][e], v[1][e]}, reinterpret_cast<kd_f32x2_a4*>(dst));
            } else if (gm >= m0) {
                if (gn >= n0) __builtin_nontemporal_store(v[0][e], dst);
                if (gn + 1 >= n0) __builtin_nontemporal_store(v[1][e], dst + 1);
            }
        }
    }
    __syncthreads();                                              // red is reused by the next tile
}

// The K-over-waves structure on a 128x128 tile (sgemm_kwave128): half the operand bytes per
// flop of the 64x64 tile, 4x4 MFMA blocks per wave (256 accumulator registers), so one block
// per CU.  Slices are 16 deep, handed to the waves in pairs (K % 32 == 0): every wave has an
// even count and the loop has no odd tail, whose separate copy made the compiler spill.
//   Lane (l32, h) holds A rows mt+32i+l32 (i = 0..3) at k0+8h .. k0+8h+7 (two 16-byte loads
//   per row; the row block through the scalar offset) and, for MFMA step t, B's row k0+8h+t at
//   columns nt+4*l32 .. nt+4*l32+3 (one 16-byte load): column block j of the tile is the
//   columns nt+4c+j, and a lane stores C four adjacent columns at a time.
//   Two register sets, each register reloaded with the slice after next right after the MFMAs
//   that read it, as in sgemm_kdirect_tile.
//   The four partial tiles are summed through LDS in two rounds of two row blocks (128 KB a
//   round), in wave order.
// A 128-row A panel (128*K floats) and a 16-row B slice must each be under 2^31 bytes.
constexpr int K128_SD = 16;
__host__ __device__ constexpr bool k128_fits(long long N, long long K) {
    return K * 128 * 4 < 2147483648LL && N * K128_SD * 4 < 2147483648LL;
}
__device__ __forceinline__ void sgemm_k128_tile(const float* __restrict__ A, const float* __restrict__ B,
                                                float* __restrict__ C, int N, int K, int mt, int nt,
                                                sgpu_f32x4* __restrict__ red) {
    constexpr int SD = K128_SD, NST = SD / 2;
    const int lane = sgpu_tid() & 63, wave = __builtin_amdgcn_readfirstlane(sgpu_tid() >> 6);
    const int l32 = lane & 31, h = lane >> 5;
    const int np = K / (2 * SD);                                   // slice pairs
    const int s0 = 2 * (wave * np / 4), s1 = 2 * ((wave + 1) * np / 4);
    const unsigned va = ((unsigned)l32 * K + NST * h) * 4u;
    const unsigned rowstep = 32u * (unsigned)K * 4u;               // one row block of A
    const unsigned vb = ((unsigned)NST * h * N + 4 * l32) * 4u;
    sgpu_f32x4 a[2][4][2];                                        // [set][row block][quad]
    sgpu_f32x4 b[2][NST];                                         // [set][step]: columns 4c..4c+3
    struct Rs {
        __amdgpu_buffer_rsrc_t a, b;
    };
    // slice s at k0 = 16 s; live false: empty ranges, every load returns zero
    auto rsrc = [&](int s, bool live = true) __attribute__((always_inline)) -> Rs {
        const long long k0 = (long long)s * SD;
        return {__builtin_amdgcn_make_buffer_rsrc((void*)(A + (size_t)mt * K + k0), (short)0,
                                                  live ? (int)((128LL * K - k0) * 4) : 0, 0x00020000),
                __builtin_amdgcn_make_buffer_rsrc((void*)(B + (size_t)k0 * N + nt), (short)0,
                                                  live ? (int)((long long)SD * N * 4) : 0, 0x00020000)};
    };
    auto lda = [&](const Rs& r, int i, int v) __attribute__((always_inline)) {
        return __builtin_bit_cast(sgpu_f32x4,
                                  __builtin_amdgcn_raw_buffer_load_b128(r.a, (int)(va + 16 * v), (int)(i * rowstep), 0));
    };
    auto ldb = [&](const Rs& r, int st) __attribute__((always_inline)) {
        return __builtin_bit_cast(sgpu_f32x4, __builtin_amdgcn_raw_buffer_load_b128(r.b, (int)vb, st * N * 4, 0));
    };
    auto load_whole = [&](int s, auto d_c, bool live = true) __attribute__((always_inline)) {
        constexpr int D = decltype(d_c)::value;
        const Rs r = rsrc(s, live);
#pragma unroll
        for (int v = 0; v < 2; v++) {
#pragma unroll
            for (int i = 0; i < 4; i++) a[D][i][v] = lda(r, i, v);
#pragma unroll
            for (int e = 0; e < 4; e++) b[D][4 * v + e] = ldb(r, 4 * v + e);
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    sgpu_f32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;
    auto step = [&](const sgpu_f32x4 (&xa)[4][2], const sgpu_f32x4& xb, int st) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(xa[i][st >> 2][st & 3], xb[j], acc[i][j], 0, 0, 0);
    };
    auto slice = [&](auto d_c, int sn) __attribute__((always_inline)) {
        constexpr int D = decltype(d_c)::value;
        const Rs r = rsrc(sn);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int st = 0; st < NST; st++) {
            step(a[D], b[D][st], st);
            if ((st & 3) == 3) {
#pragma unroll
                for (int i = 0; i < 4; i++) a[D][i][st >> 2] = lda(r, i, st >> 2);
            }
            b[D][st] = ldb(r, st);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    using Z = std::integral_constant<int, 0>;
    using O = std::integral_constant<int, 1>;
    // both sets before the loop, unconditionally (a wave with no slices reads nothing), so every
    // path into the loop has the same loads in flight and its wait counts stay exact; the last
    // pair's reloads re-read slice s1-1 (in range, unused)
    load_whole(s0, Z{}, s0 < s1);
    load_whole(min(s0 + 1, max(s1 - 1, s0)), O{}, s0 < s1);
    __builtin_amdgcn_sched_barrier(0);
    for (int s = s0; s < s1; s += 2) {
        slice(Z{}, min(s + 2, s1 - 1));
        slice(O{}, min(s + 3, s1 - 1));
    }
    // Round r sums row blocks 2r and 2r+1: lane l's accumulator quad rq of block (2r+ii, j) goes
    // to red[(w*32 + ii*16 + j*4 + rq)*64 + l]; wave w finishes row block 2r + (w >> 1), quads
    // 2(w & 1) and 2(w & 1)+1 of all four column blocks.  D layout: lane l, register r -> row
    // 8*(r/4) + 4*(l/32) + r%4 of the block; column block j, lane l -> column nt + 4*(l%32) + j.
#pragma unroll
    for (int r = 0; r < 2; r++) {
#pragma unroll
        for (int ii = 0; ii < 2; ii++)
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int rq = 0; rq < 4; rq++)
                    red[(wave * 32 + ii * 16 + j * 4 + rq) * 64 + lane] =
                        sgpu_f32x4{acc[2 * r + ii][j][4 * rq], acc[2 * r + ii][j][4 * rq + 1],
                                   acc[2 * r + ii][j][4 * rq + 2], acc[2 * r + ii][j][4 * rq + 3]};
        __syncthreads();
        const int ii = wave >> 1;
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const int rq = 2 * (wave & 1) + q;
            sgpu_f32x4 v[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                sgpu_f32x4 p[4];
#pragma unroll
                for (int w = 0; w < 4; w++) p[w] = red[(w * 32 + ii * 16 + j * 4 + rq) * 64 + lane];
                v[j] = ((p[0] + p[1]) + p[2]) + p[3];
            }
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int gm = mt + 32 * (2 * r + ii) + 8 * rq + 4 * h + e;
                __builtin_nontemporal_store(sgpu_f32x4{v[0][e], v[1][e], v[2][e], v[3][e]},
                                            reinterpret_cast<sgpu_f32x4*>(C + (size_t)gm * N + nt + 4 * l32));
            }
        }
        __syncthreads();                                          // red is rewritten next
    }
}

}  // namespace

extern "C" {

// The tiled members differ only in tile shape and staging; each runs interior tiles of
// 16-byte-row problems with K a multiple of BK on the dwordx4 pipeline and every other tile
// on the masked pipeline (edges, K tails, unaligned rows).
// All of them stage A m-major, deal their memory instructions out over the MFMA stream and
// put the slice barrier before the last MFMA group.
//   sgemm_tiled  : 64x64 tile, BK 32, 4 waves of 32x32 (1 MFMA block each), two slices'
//                  loads in flight, unconstrained register budget (172) -- small shapes
//   sgemm_tiled4 : 128x128 tile, BK 32, 4 waves of 64x64 (2x2 blocks), two slices' loads
//                  in flight, one wave per SIMD (288 registers, 70 KB of LDS)
//   sgemm_opt    : 128x256 tile, BK 16, 4 waves of 64x128 (2x4 blocks) -- large shapes
//   sgemm_opt256 : 256x256 tile, BK 32, 4 waves of 128x128 (4x4 blocks), one wave per SIMD
//                  (138 KB of LDS, 256 accumulator registers): half the LDS operand traffic
//                  per flop of the 64x128 wave tile and 16384 MFMA cycles between barriers --
//                  shapes whose 256x256 tiles fill the CUs in whole rounds
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1)))
sgemm_tiled(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M, int N, int K) {
    sgemm_mfma<64, 64, 32, 2, 2, 1, 4>(A, B, C, M, N, K);
}

__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1)))
sgemm_tiled4(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M, int N, int K) {
    sgemm_mfma<128, 128, 32, 2, 2, 1, 4>(A, B, C, M, N, K);
}

__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
sgemm_opt(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M, int N, int K) {
    sgemm_mfma<128, 256, 16, 2, 2, 0, 3>(A, B, C, M, N, K);
}

__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1)))
sgemm_opt256(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M, int N, int K) {
    sgemm_mfma<256, 256, 32, 2, 2, 1, 3>(A, B, C, M, N, K);
}

// sgemm_splitk: the 64x64 tile with K split S ways: blocks are (tile, split) units, so a
// problem with fewer tiles than CUs still spreads over the chip.  ws holds S*ntiles*4096
// floats of partial tiles, cnt one zero-initialised counter per tile (left at zero again).
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
sgemm_splitk(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M, int N, int K,
             int S, float* __restrict__ ws, unsigned* __restrict__ cnt) {
    sgemm_mfma<64, 64, 32, 2, 2, 1, 4, true>(A, B, C, M, N, K, S, ws, cnt);
}

// sgemm_small16 / sgemm_small32: problems too small to fill the chip with 64x64 tiles (one
// 16x16 or 32x32 tile of C per block, operands straight from memory into the matrix cores,
// the block's four waves splitting K).
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3)))
sgemm_small16(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M, int N, int K) {
    sgemm_small<16, 4>(A, B, C, M, N, K);
}
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
sgemm_small32(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M, int N, int K) {
    sgemm_small<32, 4>(A, B, C, M, N, K);
}

// sgemm_kwave: the 64x64 tile with K split over the block's four waves, operands loaded straight
// into the matrix-core registers, for problems with M, N multiples of 64, K a multiple of 32,
// 16-byte aligned A and B, a 64-row A panel (64*K floats) and a 16-row B slice (16*N floats)
// each under 2^31 bytes (any other problem, or a block size other than 256, returns without
// writing C; sgemm_kwave_wide takes the larger operands).  Grid-stride over tiles, one block per
// tile remapped XCD-compact as the other members; 64 KB of LDS for the partial-tile sum.
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1)))
sgemm_kwave(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M, int N, int K) {
    __shared__ __attribute__((aligned(16))) sgpu_f32x4 red[4 * 4 * 4 * 64];
    if (!sgpu_block256() || M <= 0 || N <= 0 || K <= 0 || M % 64 || N % 64 || K % KW_BK ||
        ((((uintptr_t)A) | ((uintptr_t)B)) & 15) || !kd_fits(N, K))
        return;
    const int ntm = M / 64, ntn = N / 64, ntiles = ntm * ntn;
    const int nb = sgpu_nblocks();
    const bool remap = nb == ntiles && ntiles % kXcds == 0;
    for (int t = sgpu_bid(); t < ntiles; t += nb) {
        int tm, tn;
        sgemm_tile_coords(t, ntm, ntn, remap, tm, tn);
        sgemm_kdirect_tile<false, false>(A, B, C, M, N, K, tm * 64, tn * 64, red);
    }
}

// sgemm_kwave_edge: sgemm_kwave for any M >= 64, N >= 64 and K >= 1, rows of any float
// alignment, under the same 2^31-byte bounds (sgemm_kwave_edge_wide beyond them).  A partial
// last row or column of tiles is computed as the 64 rows (columns) ending at the last one and
// stored from its first new row (column) on; with K % 16 != 0 the first k-slice is the partial
// one (k < K % 16, zeros past it).  N % 64 == 1 (one column past the last whole tile) is
// computed by the last column of whole tiles alongside their MFMAs (TH) rather than by a column
// of 64-wide tiles; every other N rounds the tile columns up.  Tiles: ceil(M/64) times N/64
// (N % 64 == 1) or ceil(N/64); grid-stride as sgemm_kwave; 66 KB of LDS.
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1)))
sgemm_kwave_edge(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M, int N, int K) {
    __shared__ __attribute__((aligned(16))) sgpu_f32x4 red[4 * 4 * 4 * 64 + 8 * 64 / 4];
    if (!sgpu_block256() || M < 64 || N < 64 || K < 1 || !kd_fits(N, K)) return;
    const bool th = N % 64 == 1;
    const int ntm = (M + 63) / 64, ntn = th ? N / 64 : (N + 63) / 64, ntiles = ntm * ntn;
    const int nb = sgpu_nblocks();
    const bool remap = nb == ntiles && ntiles % kXcds == 0;
    for (int t = sgpu_bid(); t < ntiles; t += nb) {
        int tm, tn;
        sgemm_tile_coords(t, ntm, ntn, remap, tm, tn);
        if (th && tn == ntn - 1) sgemm_kdirect_tile<true, true>(A, B, C, M, N, K, tm * 64, tn * 64, red);
        else sgemm_kdirect_tile<true, false>(A, B, C, M, N, K, tm * 64, tn * 64, red);
    }
}

// sgemm_kwave128: 128x128 tiles, K split over the block's four waves, operands straight into
// the matrix-core registers (sgemm_k128_tile), for M and N multiples of 128, K a multiple of 32,
// 16-byte aligned A and B, a 128-row A panel and a 16-row B slice each under 2^31 bytes (any
// other problem, or a block size other than 256, returns without writing C).  Grid-stride over
// tiles, one block per tile remapped XCD-compact as the other members; 128 KB of LDS for the
// partial-tile sum.
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1)))
sgemm_kwave128(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M, int N, int K) {
    __shared__ __attribute__((aligned(16))) sgpu_f32x4 red[4 * 32 * 64];
    if (!sgpu_block256() || M <= 0 || N <= 0 || K <= 0 || M % 128 || N % 128 || K % (2 * K128_SD) ||
        ((((uintptr_t)A) | ((uintptr_t)B)) & 15) || !k128_fits(N, K))
        return;
    const int ntm = M / 128, ntn = N / 128, ntiles = ntm * ntn;
    const int nb = sgpu_nblocks();
    const bool remap = nb == ntiles && ntiles % kXcds == 0;
    for (int t = sgpu_bid(); t < ntiles; t += nb) {
        int tm, tn;
        sgemm_tile_coords(t, ntm, ntn, remap, tm, tn);
        sgemm_k128_tile(A, B, C, N, K, tm * 128, tn * 128, red);
    }
}

// sgemm_kwave_wide / sgemm_kwave_edge_wide: the same members for operands past those bounds,
// staged through LDS with 64-bit addresses (sgemm_kwave_tile: 32-deep slices, K % 32 for the
// exact member); 144 / 145 KB of LDS, one block per CU.  Any other problem as above.
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1)))
sgemm_kwave_wide(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M, int N, int K) {
    __shared__ __attribute__((aligned(16))) KwaveLds L[4];
    static_assert(sizeof(L) >= 4 * 4 * 4 * 64 * sizeof(sgpu_f32x4), "the partial tiles fit the staging");
    if (!sgpu_block256() || M <= 0 || N <= 0 || K <= 0 || M % 64 || N % 64 || K % KW_BK ||
        ((((uintptr_t)A) | ((uintptr_t)B)) & 15))
        return;
    const int ntm = M / 64, ntn = N / 64, ntiles = ntm * ntn;
    const int nb = sgpu_nblocks();
    const bool remap = nb == ntiles && ntiles % kXcds == 0;
    for (int t = sgpu_bid(); t < ntiles; t += nb) {
        int tm, tn;
        sgemm_tile_coords(t, ntm, ntn, remap, tm, tn);
        sgemm_kwave_tile<false, false>(A, B, C, M, N, K, tm * 64, tn * 64, L[sgpu_tid() >> 6],
                                       reinterpret_cast<sgpu_f32x4*>(&L[0]));
    }
}
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1)))
sgemm_kwave_edge_wide(const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M, int N,
                      int K) {
    __shared__ __attribute__((aligned(16))) KwaveLdsEdge L[4];
    static_assert(sizeof(L) >= 4 * 4 * 4 * 64 * sizeof(sgpu_f32x4) + 8 * 64 * sizeof(float),
                  "the partial tiles and the extra column's partials fit the staging");
    if (!sgpu_block256() || M < 64 || N < 64 || K < 1) return;
    const bool th = N % 64 == 1;
    const int ntm = (M + 63) / 64, ntn = th ? N / 64 : (N + 63) / 64, ntiles = ntm * ntn;
    const int nb = sgpu_nblocks();
    const bool remap = nb == ntiles && ntiles % kXcds == 0;
    for (int t = sgpu_bid(); t < ntiles; t += nb) {
        int tm, tn;
        sgemm_tile_coords(t, ntm, ntn, remap, tm, tn);
        sgpu_f32x4* red = reinterpret_cast<sgpu_f32x4*>(&L[0]);
        if (th && tn == ntn - 1)
            sgemm_kwave_tile<true, true>(A, B, C, M, N, K, tm * 64, tn * 64, L[sgpu_tid() >> 6], red);
        else
            sgemm_kwave_tile<true, false>(A, B, C, M, N, K, tm * 64, tn * 64, L[sgpu_tid() >> 6], red);
    }
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
    auto sum4 = [](const sgpu_f32x4& v) { return ((v.x + v.y) + v.z) + v.w; };
    constexpr int G = 8;                          // loads per lane per group
    for (int it = 0; it < iters; ++it) {
        int i = i0;
        // Groups of G loads, software-pipelined: the next group is issued before the current
        // one is added, so every lane keeps G loads in flight across the loop edge (the sums
        // keep the element order of the plain loop).
        if (i + (G - 1) * stride < n4) {
            sgpu_f32x4 v[G];
#pragma unroll
            for (int u = 0; u < G; u++) v[u] = sgpu_ldnt(buf + i + u * stride);
            for (; i + (2 * G - 1) * stride < n4; i += G * stride) {
                sgpu_f32x4 w[G];
#pragma unroll
                for (int u = 0; u < G; u++) w[u] = sgpu_ldnt(buf + i + (G + u) * stride);
#pragma unroll
                for (int u = 0; u < G; u++) {
                    acc += sum4(v[u]);
                    v[u] = w[u];
                }
            }
#pragma unroll
            for (int u = 0; u < G; u++) acc += sum4(v[u]);
            i += G * stride;
        }
        for (; i < n4; i += stride) {
            const sgpu_f32x4 v = sgpu_ldnt(buf + i);
            acc += ((v.x + v.y) + v.z) + v.w;
        }
    }
    if (i0 < n4) out[i0] = acc;
}

}  // extern "C"
