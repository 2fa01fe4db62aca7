// Wavefront helpers shared by the per-atom record kernels (message.hip,
// equivariant.hip): lane exchanges, slot folds and the XCD-aware atom of a
// wave.
#pragma once

#include "model.hpp"

namespace rune {

// Lane permutations for reductions: DPP quad_perm (xor 1, xor 2) and row
// rotations (4, 8 lanes within a 16-lane row) are VALU operations;
// ds_swizzle in bit mode exchanges lanes l and l ^ m within 32 lanes.
template <int kCtrl>
__device__ inline float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xF, 0xF,
                                                      false));
}
template <int kXor>
__device__ inline float swz(float v) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1F | (kXor << 10)));
}
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppRor4 = 0x124, kDppRor8 = 0x128;

// Sum over the w lanes of a lane group (w a power of two <= 64, groups
// aligned); every lane of the group receives the sum.
__device__ inline float group_sum(float v, int w) {
    if (w >= 2) v += dpp<kDppXor1>(v);
    if (w >= 4) v += dpp<kDppXor2>(v);
    if (w == 8) v += swz<4>(v);
    if (w >= 16) {
        v += dpp<kDppRor4>(v);
        v += dpp<kDppRor8>(v);
    }
    if (w >= 32) v += swz<16>(v);
    if (w >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}

// Orders LDS traffic of one wave (lanes exchange data through LDS).
__device__ inline void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int N>
__device__ inline void zero(float (&v)[N]) {
#pragma unroll
    for (int k = 0; k < N; ++k) v[k] = 0.0f;
}

template <int N>
__device__ inline void copy(float (&d)[N], const float (&s)[N]) {
#pragma unroll
    for (int k = 0; k < N; ++k) d[k] = s[k];
}

// Adds the partial sums of the S slots of W = 64 / S lanes (fixed tree
// order); every slot ends with the total.
template <int S, int N>
__device__ inline void fold_slots(float (&v)[N]) {
#pragma unroll
    for (int off = 32; off >= 64 / S; off >>= 1) {
#pragma unroll
        for (int k = 0; k < N; ++k) v[k] += __shfl_xor(v[k], off, 64);
    }
}

// Record metadata is read 64 records at a time, lane-parallel, and handed to
// the slots by shuffles, so the row loads of the next records depend on no
// other load.
__device__ inline int bcast(int v, int src) { return __shfl(v, src, 64); }
__device__ inline float bcast(float v, int src) { return __shfl(v, src, 64); }

// ---- work assignment of the per-atom kernels ----
// One atom per wave, kWavesPerBlock waves per block.  Blocks are dealt to the
// 8 XCDs round-robin; xcd_rank renumbers them so that each XCD walks one
// contiguous range of the processing order.  The order is the neighbour
// builder's Morton-ordered cell bins, so the rows an XCD gathers stay in its L2.
__device__ inline int xcd_rank(int b, int nb) {
    const int x = b & 7, k = b >> 3, q = nb >> 3, r = nb & 7;
    return x * q + min(x, r) + k;
}

template <int kWavesPerBlock = 4>
__device__ inline int wave_atom(const Records &r) {
    const int t = __builtin_amdgcn_readfirstlane(xcd_rank(blockIdx.x, gridDim.x) *
                                                     kWavesPerBlock +
                                                 int(threadIdx.x >> 6));
    if (t >= r.n_atoms) return -1;
    return r.order ? __builtin_amdgcn_readfirstlane(r.order[t]) : t;
}

}  // namespace rune
