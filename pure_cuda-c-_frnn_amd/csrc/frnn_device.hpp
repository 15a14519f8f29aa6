// frnn_device.hpp -- device-side helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "frnn_internal.hpp"

namespace frnn {

// A compile-time int as a value (selects a template instance from a lambda).
template <int V>
struct IntC { static constexpr int value = V; };

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

// Cell of a frame axis: floor((x - lo) * inv) clamped to [0, nb-1].
// Monotone in x, so an interval of x maps onto an interval of cells.
__device__ __forceinline__ int sub_bin(float x, float lo, float inv, int nb) {
    float t = (x - lo) * inv;
    float f = floorf(t);
    f = fmaxf(f, 0.0f);
    f = fminf(f, (float)(nb - 1));
    return (int)f;
}

// Projections of a point onto frame directions 0 .. M-1: for each, the
// sequential fma chain over the terms of fl(x[coord[t]] - mean[t]) weighted by
// dir[k][t], with coord(c) returning coordinate c of the point.  Binning and
// the search both use it; each value is within Frame::margin of the exact
// projection.
template <int M, class Coord>
__device__ __forceinline__ void frame_project(const Frame* __restrict__ f, Coord coord, float (&s)[M]) {
#pragma unroll
    for (int m = 0; m < M; ++m) s[m] = 0.0f;
    const int T = f->terms;
    for (int t = 0; t < T; ++t) {
        const float y = coord(f->coord[t]) - f->mean[t];
#pragma unroll
        for (int m = 0; m < M; ++m) s[m] = fmaf(f->dir[m][t], y, s[m]);
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

// Lane exchanges at xor distance j = 1, 2, 4, 8, 16, 32, all on the VALU
// (no LDS round trip, which would put its latency on every step of a
// dependent sort or reduction).  xor_pair_u32 yields {v(lane), v(lane ^ j)}
// as (a, b) in a lane-dependent order, which is all a symmetric
// compare-exchange, min, max or sum needs:
//   j = 1, 2  DPP quad permutes [1,0,3,2] / [2,3,0,1]
//   j = 4     DPP row rotations by 4 and 12 (lanes with bit 2 set take the
//             one reading lane - 4)
//   j = 8     DPP row_ror:8
//   j = 16    v_permlane16_swap (rows 0/1 and 2/3 of a and b hold each other)
//   j = 32    v_permlane32_swap (the two 32-lane halves)
// j must fold to a constant (loops over it are fully unrolled).
// Lane masks as compile-time constants: bit i of kLaneBitClear[l] is set iff
// bit l of lane i is clear.  Selections by these masks stay scalar constants
// the compiler can rematerialise; masks computed from the lane id are not
// constant to it and would each hold a scalar register pair for the whole
// kernel.
constexpr unsigned long long kLaneBitClear[6] = {
    0x5555555555555555ull, 0x3333333333333333ull, 0x0F0F0F0F0F0F0F0Full,
    0x00FF00FF00FF00FFull, 0x0000FFFF0000FFFFull, 0x00000000FFFFFFFFull};
__device__ __forceinline__ bool lane_mask(unsigned long long m) { return __builtin_amdgcn_inverse_ballot_w64(m); }
// lane < 32 (the lower half of the wave) and lane == 0, in the same form
__device__ __forceinline__ bool lower_half() { return lane_mask(0x00000000FFFFFFFFull); }
__device__ __forceinline__ bool first_lane() { return lane_mask(1ull); }

__device__ __forceinline__ void xor_pair_u32(unsigned v, int j, unsigned& a, unsigned& b) {
    switch (j) {
        case 1: a = v; b = (unsigned)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, true); return;
        case 2: a = v; b = (unsigned)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, true); return;
        case 4: {
            const unsigned dn = (unsigned)__builtin_amdgcn_mov_dpp((int)v, 0x124, 0xF, 0xF, true);  // lane - 4
            const unsigned up = (unsigned)__builtin_amdgcn_mov_dpp((int)v, 0x12C, 0xF, 0xF, true);  // lane + 4
            a = v;
            b = lane_mask(kLaneBitClear[2]) ? up : dn;
            return;
        }
        case 8: a = v; b = (unsigned)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xF, 0xF, true); return;
        case 16: {
            const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
            a = r[0];
            b = r[1];
            return;
        }
        default: {
            const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
            a = r[0];
            b = r[1];
            return;
        }
    }
}

__device__ __forceinline__ void xor_pair_u64(unsigned long long v, int j, unsigned long long& a,
                                             unsigned long long& b) {
    unsigned alo, blo, ahi, bhi;
    xor_pair_u32((unsigned)v, j, alo, blo);
    xor_pair_u32((unsigned)(v >> 32), j, ahi, bhi);
    a = ((unsigned long long)ahi << 32) | alo;
    b = ((unsigned long long)bhi << 32) | blo;
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
            unsigned long long p, q;
            xor_pair_u64(x[e], j, p, q);
            // lanes ascending: bit k of the element index clear (k < 64: a
            // lane bit; otherwise the register's, the same for all lanes)
            const unsigned long long up = k == 0 ? ~0ull
                                          : k < kWave ? kLaneBitClear[__builtin_ctz(k)]
                                                      : (((e * kWave) & k) == 0 ? ~0ull : 0ull);
            // a lane keeps the minimum iff (its bit j is clear) == ascending
            const unsigned long long keep_min = ~(kLaneBitClear[__builtin_ctz(j)] ^ up);
            x[e] = ((p < q) == lane_mask(keep_min)) ? p : q;
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

// Wave-wide reductions over the VALU lane exchanges above (the six steps are
// spelled out: a loop over the distance was left rolled by the compiler in
// places, with a run-time dispatch on every step).
template <class Op>
__device__ __forceinline__ unsigned wave_reduce_u32(unsigned v, Op op) {
    unsigned p, q;
    xor_pair_u32(v, 32, p, q); v = op(p, q);
    xor_pair_u32(v, 16, p, q); v = op(p, q);
    xor_pair_u32(v, 8, p, q); v = op(p, q);
    xor_pair_u32(v, 4, p, q); v = op(p, q);
    xor_pair_u32(v, 2, p, q); v = op(p, q);
    xor_pair_u32(v, 1, p, q); v = op(p, q);
    // every lane holds the result: as a scalar, it keeps the control flow
    // that depends on it uniform
    return (unsigned)__builtin_amdgcn_readfirstlane((int)v);
}
__device__ __forceinline__ int wave_min_i32(int v) {
    return (int)wave_reduce_u32((unsigned)v, [](unsigned p, unsigned q) { return (unsigned)min((int)p, (int)q); });
}
__device__ __forceinline__ int wave_max_i32(int v) {
    return (int)wave_reduce_u32((unsigned)v, [](unsigned p, unsigned q) { return (unsigned)max((int)p, (int)q); });
}
__device__ __forceinline__ float wave_min_f32(float v) {
    return __uint_as_float(wave_reduce_u32(__float_as_uint(v), [](unsigned p, unsigned q) {
        return __float_as_uint(fminf(__uint_as_float(p), __uint_as_float(q)));
    }));
}
__device__ __forceinline__ float wave_max_f32(float v) {
    return __uint_as_float(wave_reduce_u32(__float_as_uint(v), [](unsigned p, unsigned q) {
        return __float_as_uint(fmaxf(__uint_as_float(p), __uint_as_float(q)));
    }));
}
__device__ __forceinline__ long long wave_sum_i64(long long v) {
    unsigned long long x = (unsigned long long)v, p, q;
    xor_pair_u64(x, 32, p, q); x = p + q;
    xor_pair_u64(x, 16, p, q); x = p + q;
    xor_pair_u64(x, 8, p, q); x = p + q;
    xor_pair_u64(x, 4, p, q); x = p + q;
    xor_pair_u64(x, 2, p, q); x = p + q;
    xor_pair_u64(x, 1, p, q); x = p + q;
    const unsigned lo = (unsigned)__builtin_amdgcn_readfirstlane((int)(unsigned)x);
    const unsigned hi = (unsigned)__builtin_amdgcn_readfirstlane((int)(unsigned)(x >> 32));
    return (long long)(((unsigned long long)hi << 32) | lo);
}

}  // namespace frnn
