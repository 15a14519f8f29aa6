// frnn_device.hpp -- device-side helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "frnn_internal.hpp"

namespace frnn {

constexpr int kWave = 64;

typedef float floatx16 __attribute__((ext_vector_type(16)));

// Cell coordinate of one gridded axis: floor(x * inv_cell) clamped to
// [0, res-1] (insert_points.cu:72 with min_val = 0; the clamp replaces the
// reference's drop of out-of-domain points, insert_points.cu:74-87).  The
// query side of the reference truncates and clamps (find_nbrs.cu:154-155,
// 278-279); after the clamp both agree.  NaN bins to 0 (fmaxf drops NaN).
__device__ __forceinline__ int bin_coord(float x, float inv_cell, int res) {
    float t = x * inv_cell;
    float f = floorf(t);
    f = fmaxf(f, 0.0f);
    f = fminf(f, (float)(res - 1));
    return (int)f;
}

// Sub-bin of a refinement axis: floor((x - lo) * inv) clamped to [0, nb-1].
// Monotone in x, so an interval of x maps onto an interval of sub-bins.
__device__ __forceinline__ int sub_bin(float x, float lo, float inv, int nb) {
    float t = (x - lo) * inv;
    float f = floorf(t);
    f = fmaxf(f, 0.0f);
    f = fminf(f, (float)(nb - 1));
    return (int)f;
}

// Projections of a point onto frame directions k0 .. k0+M-1: for each, the
// sequential fma chain over the terms of fl(x[coord[t]] - mean[t]) weighted by
// dir[k][t], with coord(c) returning coordinate c of the point.  Binning and
// the search both use it; each value is within Frame::margin of the exact
// projection.
template <int M, class Coord>
__device__ __forceinline__ void frame_project(const Frame* __restrict__ f, int k0, Coord coord, float (&s)[M]) {
#pragma unroll
    for (int m = 0; m < M; ++m) s[m] = 0.0f;
    const int T = f->terms;
    for (int t = 0; t < T; ++t) {
        const float y = coord(f->coord[t]) - f->mean[t];
#pragma unroll
        for (int m = 0; m < M; ++m) s[m] = fmaf(f->dir[k0 + m][t], y, s[m]);
    }
}

// Total order on (d2, idx): non-negative fp32 bit patterns order like the
// values, so one 64-bit compare ranks (d2, idx) lexicographically.
__device__ __forceinline__ unsigned long long make_key(float d2, int idx) {
    return ((unsigned long long)__float_as_uint(d2) << 32) | (unsigned int)idx;
}
__device__ __forceinline__ float key_d2(unsigned long long key) {
    return __uint_as_float((unsigned int)(key >> 32));
}

// Value of lane (lane ^ j) for j = 1, 2, 4, 8, 16, 32: DPP moves for 1, 2
// (quad permutes) and 8 (rotation by 8 within 16-lane rows), the LDS
// crossbar for the rest (swizzle xor 4 and xor 16 within 32-lane halves,
// a backward permute for 32), which keeps those exchanges off the VALU.
// j must fold to a constant (loops over it are fully unrolled).
__device__ __forceinline__ unsigned xor_lane_u32(unsigned v, int j) {
    switch (j) {
        case 1: return (unsigned)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, true);   // quad_perm [1,0,3,2]
        case 2: return (unsigned)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, true);   // quad_perm [2,3,0,1]
        case 4: return (unsigned)__builtin_amdgcn_ds_swizzle((int)v, 0x101F);              // bitmask mode, xor 4
        case 8: return (unsigned)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xF, 0xF, true);  // row_ror:8
        case 16: return (unsigned)__builtin_amdgcn_ds_swizzle((int)v, 0x401F);             // bitmask mode, xor 16
        default: {
            const int lane = (int)(threadIdx.x & (kWave - 1));
            return (unsigned)__builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, (int)v);
        }
    }
}

__device__ __forceinline__ unsigned long long xor_lane_u64(unsigned long long v, int j) {
    const unsigned lo = xor_lane_u32((unsigned)v, j);
    const unsigned hi = xor_lane_u32((unsigned)(v >> 32), j);
    return ((unsigned long long)hi << 32) | lo;
}

__device__ __forceinline__ unsigned long long shfl_u64(unsigned long long v, int src) {
    const unsigned int lo = (unsigned int)__shfl((int)(unsigned int)v, src);
    const unsigned int hi = (unsigned int)__shfl((int)(unsigned int)(v >> 32), src);
    return ((unsigned long long)hi << 32) | lo;
}

// Compare-exchange step of a bitonic network on 64*E keys held across one
// wave (x[e] is element e*64 + lane): partner distance j, ascending where
// bit k of the element index is clear (k = 0: ascending everywhere).
template <int E>
__device__ __forceinline__ void bitonic_step(unsigned long long (&x)[E], int k, int j) {
    const int lane = threadIdx.x & (kWave - 1);
    if (j >= kWave) {
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int ep = e ^ (j / kWave);
            if (ep > e) {
                const bool up = ((e * kWave) & k) == 0;
                const unsigned long long p = x[e], q = x[ep];
                const bool sw = (p > q) == up;
                x[e] = sw ? q : p;
                x[ep] = sw ? p : q;
            }
        }
    } else {
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const unsigned long long y = xor_lane_u64(x[e], j);
            const bool up = (((e * kWave) | lane) & k) == 0;
            const bool keep_min = ((lane & j) == 0) == up;
            const bool lt = x[e] < y;
            x[e] = (lt == keep_min) ? x[e] : y;
        }
    }
}

template <int E>
constexpr int log2_keys() { return 6 + (E == 1 ? 0 : E == 2 ? 1 : E == 4 ? 2 : 3); }

// Ascending bitonic sort of the 64*E keys x[] (no LDS, no barriers).
template <int E>
__device__ __forceinline__ void wave_sort_u64(unsigned long long (&x)[E]) {
    static_assert(E == 1 || E == 2 || E == 4 || E == 8, "power-of-two register count");
    // affine loops over log2 distances so that both unroll fully and x[] stays in registers
#pragma unroll
    for (int lk = 1; lk <= log2_keys<E>(); ++lk) {
#pragma unroll
        for (int lj = lk - 1; lj >= 0; --lj) bitonic_step<E>(x, 1 << lk, 1 << lj);
    }
}

// Ascending sort of a bitonic sequence of 64*E keys (the half-cleaner stages).
template <int E>
__device__ __forceinline__ void wave_bitonic_merge_u64(unsigned long long (&x)[E]) {
#pragma unroll
    for (int lj = log2_keys<E>() - 1; lj >= 0; --lj) bitonic_step<E>(x, 0, 1 << lj);
}

__device__ __forceinline__ int wave_min_i32(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ int wave_max_i32(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ float wave_min_f32(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fminf(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ long long wave_sum_i64(long long v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

}  // namespace frnn
