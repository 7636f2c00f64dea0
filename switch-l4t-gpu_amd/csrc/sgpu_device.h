// sgpu_device.h -- device helpers shared by the gfx950 code objects.
//
// Everything here is written for CDNA4 (gfx950): 64-lane wavefronts, DPP row
// operations (a "row" is 16 lanes), AGPR-backed MFMA accumulators.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define SGPU_WAVE 64

typedef float sgpu_f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t sgpu_u32x4 __attribute__((ext_vector_type(4)));
// The same four floats at any float alignment (4 bytes): a load through this type tells the
// compiler no more than the address guarantees; gfx950 still loads it with one dwordx4.
typedef float sgpu_f32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

// Four consecutive floats from p: 16-byte aligned (ALIGNED) or any float alignment.
template <bool ALIGNED>
__device__ __forceinline__ sgpu_f32x4 sgpu_ld4(const float* p) {
    if constexpr (ALIGNED) return *reinterpret_cast<const sgpu_f32x4*>(p);
    else return *reinterpret_cast<const sgpu_f32x4_a4*>(p);
}

// 128-bit streaming loads (global_load_dwordx4 with the nontemporal hint): data read once.
__device__ __forceinline__ sgpu_f32x4 sgpu_ldnt(const sgpu_f32x4* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ sgpu_u32x4 sgpu_ldnt(const sgpu_u32x4* p) { return __builtin_nontemporal_load(p); }

// fp16 bits -> fp32 with the reference contract (qwen_kernels.cu:6-14): exponent 0 gives
// +0.0 (subnormals and -0 flushed, sign dropped), exponent 31 gives the finite value
// +-2^16 * (1 + m/1024), every other code converts exactly.  Pure integer arithmetic, so
// it does not depend on the wave's denormal mode.  0x38000000 = 112 << 23 re-biases the
// exponent from 15 to 127.
__device__ __forceinline__ float sgpu_h2f_lo(uint32_t w) {
    uint32_t t = (((w & 0x7fffu) << 13) + 0x38000000u) | ((w & 0x8000u) << 16);
    return __uint_as_float((w & 0x7c00u) ? t : 0u);
}
__device__ __forceinline__ float sgpu_h2f_hi(uint32_t w) {
    uint32_t t = ((((w >> 16) & 0x7fffu) << 13) + 0x38000000u) | (w & 0x80000000u);
    return __uint_as_float((w & 0x7c000000u) ? t : 0u);
}
__device__ __forceinline__ float sgpu_h2f(uint16_t h) { return sgpu_h2f_lo((uint32_t)h); }

// DPP controls (GFX9 encoding).
#define SGPU_DPP_ROW_SHR(n) (0x110 + (n))
#define SGPU_DPP_ROW_BCAST15 0x142
#define SGPU_DPP_ROW_BCAST31 0x143

template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float sgpu_dpp(float v) {
    // Lanes whose source is outside the row (or masked off) read 0.
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, true));
}

// Sum over groups of LANES consecutive lanes (4, 8, 16, 32 or 64).  The total of each group ends
// up in the group's LAST lane (lane % LANES == LANES-1); other lanes hold partial sums.
// Must run with the whole wave active.
template <int LANES>
__device__ __forceinline__ float sgpu_group_sum(float v) {
    static_assert(LANES == 4 || LANES == 8 || LANES == 16 || LANES == 32 || LANES == 64, "group of 4..64 lanes");
    // row_shr prefix sums: after the shifts 1, 2, .., LANES/2 (within 16-lane rows) lane
    // LANES*g + LANES-1 holds exactly the sum of its group's LANES lanes.
    v += sgpu_dpp<SGPU_DPP_ROW_SHR(1)>(v);
    v += sgpu_dpp<SGPU_DPP_ROW_SHR(2)>(v);
    if (LANES >= 8) v += sgpu_dpp<SGPU_DPP_ROW_SHR(4)>(v);
    if (LANES >= 16) v += sgpu_dpp<SGPU_DPP_ROW_SHR(8)>(v);
    if (LANES >= 32) v += sgpu_dpp<SGPU_DPP_ROW_BCAST15, 0xa>(v);
    if (LANES >= 64) v += sgpu_dpp<SGPU_DPP_ROW_BCAST31, 0xc>(v);
    return v;
}

// Whole-wave reductions returning the result in every lane (via lane 63 / readlane).
__device__ __forceinline__ float sgpu_wave_sum(float v) {
    v = sgpu_group_sum<64>(v);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
__device__ __forceinline__ float sgpu_wave_max(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), SGPU_DPP_ROW_SHR(1), 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), SGPU_DPP_ROW_SHR(2), 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), SGPU_DPP_ROW_SHR(4), 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), SGPU_DPP_ROW_SHR(8), 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), SGPU_DPP_ROW_BCAST15, 0xa, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), SGPU_DPP_ROW_BCAST31, 0xc, 0xf, false)));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Cross-block hand-off of partial results (split-K SGEMM, the split batched GEMM, the decode
// attention's position chunks): the units of one output tile each write a partial record and
// count in on the tile's counter; the last to arrive combines all records in a fixed order.
//   writer: partials are written with agent-scope atomic stores (global_store ... sc1: written
//           through to the device's coherence point past the per-XCD L2s), every wave waits for
//           their acknowledgment (s_waitcnt vmcnt(0)), a block barrier, then thread 0 adds 1 to
//           the counter (agent-scope atomic, relaxed);
//   reader: the thread that sees the final count takes an agent-scope acquire fence (buffer_inv
//           sc1) before a block barrier, then the block reads the records with agent-scope atomic
//           loads (sc1) and resets the counter.
// The writer side replaces an agent-scope release (buffer_wbl2 sc1 per unit) by the
// acknowledgment of stores that bypass the L2 write-back: the release measured +55% on split
// SGEMM (1023x1025x997 at 4 splits 31.7 -> 48.9 us, 1024x768x1024 21.8 -> 33.1) while the
// acquire costs ~0.5 us per launch.

// Launch geometry from the hidden kernel arguments (code object v5): the grid's block counts
// x, y, z (32-bit, bytes 0, 4, 8) and the 16-bit group sizes x, y, z (bytes 12, 14, 16).
// HIP's blockDim also allows for a partial last block and picks, per block, between the group
// size and the remainder field.  That pick can compile to 16-bit vector loads that run one
// after another, through the vector cache a streaming kernel keeps full, before the block's
// first useful load.  HIP launches whole blocks only, so the group sizes are the block sizes.
// Read as below, the block counts and the x, y group sizes come from the argument SGPRs
// preloaded at wave launch (for kernels whose own arguments take at most 40 bytes), and the z
// group size from one scalar load.  Each block count passes through an empty asm so that
// neighbouring fields are not merged into one wider load, which the preload would not serve.
__device__ __forceinline__ uint32_t sgpu_hidden_u32(int dword) {
    typedef const uint32_t __attribute__((address_space(4))) * cu32;
    return ((cu32)__builtin_amdgcn_implicitarg_ptr())[dword];
}
__device__ __forceinline__ int sgpu_gdim(int d) {
    uint32_t v = sgpu_hidden_u32(d);
    __asm__("" : "+s"(v));
    return (int)v;
}
__device__ __forceinline__ int sgpu_bdim_x() { return __builtin_amdgcn_workgroup_size_x(); }
__device__ __forceinline__ int sgpu_bdim_y() { return __builtin_amdgcn_workgroup_size_y(); }
__device__ __forceinline__ int sgpu_bdim_z() { return (int)(sgpu_hidden_u32(4) & 0xffffu); }

// Linear thread index / block size for any block shape.
__device__ __forceinline__ int sgpu_tid() {
    return threadIdx.x + sgpu_bdim_x() * (threadIdx.y + sgpu_bdim_y() * threadIdx.z);
}
__device__ __forceinline__ int sgpu_nthreads() { return sgpu_bdim_x() * sgpu_bdim_y() * sgpu_bdim_z(); }
// A block of exactly 256 threads, for kernels declared __launch_bounds__(256) only: HIP refuses
// a launch whose block holds more threads than the kernel's bound, so x*y == 256 leaves z == 1
// and the check needs no load of the z size.
__device__ __forceinline__ bool sgpu_block256() { return sgpu_bdim_x() * sgpu_bdim_y() == 256; }
__device__ __forceinline__ int sgpu_bid() {
    return blockIdx.x + sgpu_gdim(0) * (blockIdx.y + sgpu_gdim(1) * blockIdx.z);
}
__device__ __forceinline__ int sgpu_nblocks() { return sgpu_gdim(0) * sgpu_gdim(1) * sgpu_gdim(2); }
