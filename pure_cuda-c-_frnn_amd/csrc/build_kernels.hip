// build_kernels.hip -- uniform-grid build and output kernels for gfx950.
//
// Grid build = zero-fill + bin/count + exclusive scan + reorder, replacing
// CountPointsNDKernel / thrust::exclusive_scan / CountingSort{ND,AoS3}Kernel
// (insert_points.cu:45-88,142-164,205-226; frnn_engine.cu:89-96,159-174).
// Differences by design:
//   * bin/count records each point's arrival slot in its cell (rank), so the
//     reorder is a pure gather-free scatter pos = start[cell] + rank and the
//     scanned offsets stay cell STARTS (the reference's second atomic pass turns
//     them into cell ends, insert_points.cu:156-158);
//   * the reorder writes one padded AoS row per point (stride roundup(D,4)),
//     i.e. 16-byte-aligned vector stores of whole rows instead of D scattered
//     4-byte stores into SoA planes, and also records the inverse permutation;
//   * the scan is two passes over 4096-element tiles (16-byte coalesced
//     accesses) with no inter-block spin waits: a reduce writes each tile's
//     sum, then each tile adds the earlier tiles' sums (from L2) to its own
//     block scan.
#include <mutex>

#include "frnn_device.hpp"
#include "frnn_internal.hpp"

namespace frnn {

constexpr int kScanThreads = 256;
constexpr int kScanRows = 4;                              // int4 rows per thread
constexpr int kScanTile = kScanThreads * 4 * kScanRows;   // 4096

// 16-byte stores where the array is 16-byte aligned (head and tail as ints).
__global__ void fill_i32_kernel(int* __restrict__ p, long long n, int v) {
    const long long stride = (long long)gridDim.x * blockDim.x;
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long head = (long long)((16 - ((uintptr_t)p & 15)) & 15) / 4;
    if (((uintptr_t)p & 3) != 0 || head >= n) {
        for (; i < n; i += stride) p[i] = v;
        return;
    }
    if (i < head) p[i] = v;
    int4* q = reinterpret_cast<int4*>(p + head);
    const long long nv = (n - head) / 4;
    const int4 w = make_int4(v, v, v, v);
    for (long long k = i; k < nv; k += stride) q[k] = w;
    const long long t = head + 4 * nv + i;
    if (t < n) p[t] = v;
}

// One thread per point; coordinates of the first g axes are read SoA, so a
// wave reads 64 consecutive floats per axis.
__global__ __launch_bounds__(256) void bin_count_kernel(const float* __restrict__ pts, int N, int g,
                                                        int res, float inv_cell,
                                                        int* __restrict__ cell_of,
                                                        int* __restrict__ rank,
                                                        int* __restrict__ cnt) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N) return;
    long long h = 0, s = 1;
    for (int d = 0; d < g; ++d) {
        h += (long long)bin_coord(pts[(size_t)d * N + i], inv_cell, res) * s;
        s *= res;
    }
    cell_of[i] = (int)h;
    rank[i] = atomicAdd(&cnt[h], 1);
}

// Exclusive scan in three passes over tiles of 4096 ints (256 threads x 4
// rows of one int4; a row is 1024 consecutive ints, so every load and store
// instruction of a wave covers 1 KB contiguously).  VEC: in and out are
// 16-byte aligned (int4 accesses; the last partial int4 per element).
template <bool VEC>
__device__ __forceinline__ int4 scan_load4(const int* __restrict__ in, long long e, int n) {
    if (VEC && e + 3 < n) return *reinterpret_cast<const int4*>(in + e);
    return make_int4(e < n ? in[e] : 0, e + 1 < n ? in[e + 1] : 0, e + 2 < n ? in[e + 2] : 0,
                     e + 3 < n ? in[e + 3] : 0);
}

template <bool VEC>
__device__ __forceinline__ void scan_store4(int* __restrict__ out, long long e, int n, int4 v) {
    if (VEC && e + 3 < n) {
        *reinterpret_cast<int4*>(out + e) = v;
        return;
    }
    if (e < n) out[e] = v.x;
    if (e + 1 < n) out[e + 1] = v.y;
    if (e + 2 < n) out[e + 2] = v.z;
    if (e + 3 < n) out[e + 3] = v.w;
}

// Exclusive scan of one int per thread over the 256-thread block: wave
// inclusive scans (lane exchanges), then the four wave totals through LDS.
__device__ __forceinline__ int block_exclusive_scan_256(int v, int* s_w, int* total) {
    const int lane = threadIdx.x & (kWave - 1);
    const int w = threadIdx.x / kWave;
    int incl = v;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const int x = __shfl_up(incl, o);
        if (lane >= o) incl += x;
    }
    if (lane == kWave - 1) s_w[w] = incl;
    __syncthreads();
    int off = 0, tot = 0;
#pragma unroll
    for (int k = 0; k < kScanThreads / kWave; ++k) {
        const int t = s_w[k];
        off += k < w ? t : 0;
        tot += t;
    }
    __syncthreads();   // s_w is reused by the next call
    *total = tot;
    return off + incl - v;
}

// bound (may be null): a device count; the scan then covers min(n, *bound +
// 1) entries (the frame's cells + 1 of a count array sized for its capacity).
__device__ __forceinline__ int scan_extent(int n, const int* bound) {
    return bound ? min(n, __builtin_amdgcn_readfirstlane(bound[0]) + 1) : n;
}

template <bool VEC>
__global__ __launch_bounds__(kScanThreads) void scan_reduce_kernel(const int* __restrict__ in, int n,
                                                                   int* __restrict__ partials,
                                                                   const int* __restrict__ bound) {
    __shared__ int s_w[kScanThreads / kWave];
    n = scan_extent(n, bound);
    const long long base = (long long)blockIdx.x * kScanTile + 4 * threadIdx.x;
    int sum = 0;
#pragma unroll
    for (int j = 0; j < kScanRows; ++j) {
        const int4 v = scan_load4<VEC>(in, base + j * 4 * kScanThreads, n);
        sum += (v.x + v.y) + (v.z + v.w);
    }
    int total;
    block_exclusive_scan_256(sum, s_w, &total);
    if (threadIdx.x == 0) partials[blockIdx.x] = total;
}

// CLEAR: the input entries are zeroed once read (the count array starts the
// next binning clean, with no separate fill).
template <bool VEC, bool CLEAR>
__global__ __launch_bounds__(kScanThreads) void scan_final_kernel(int* __restrict__ in, int n,
                                                                  const int* __restrict__ partials,
                                                                  int* __restrict__ out,
                                                                  const int* __restrict__ bound) {
    __shared__ int s_w[kScanThreads / kWave];
    n = scan_extent(n, bound);
    const long long base = (long long)blockIdx.x * kScanTile + 4 * threadIdx.x;
    int4 v[kScanRows];
#pragma unroll
    for (int j = 0; j < kScanRows; ++j) v[j] = scan_load4<VEC>(in, base + j * 4 * kScanThreads, n);
    if constexpr (CLEAR) {
#pragma unroll
        for (int j = 0; j < kScanRows; ++j) scan_store4<VEC>(in, base + j * 4 * kScanThreads, n, make_int4(0, 0, 0, 0));
    }
    // the tile's carry: the sum of the earlier tiles' partial sums (at most
    // kScanTile of them, read from L2 while this tile's loads are in flight)
    int pre = 0;
    for (int k = threadIdx.x; k < (int)blockIdx.x; k += kScanThreads) pre += partials[k];
    int carry;
    block_exclusive_scan_256(pre, s_w, &carry);
#pragma unroll
    for (int j = 0; j < kScanRows; ++j) {
        int total;
        const int x = carry + block_exclusive_scan_256((v[j].x + v[j].y) + (v[j].z + v[j].w), s_w, &total);
        int4 o;
        o.x = x;
        o.y = o.x + v[j].x;
        o.z = o.y + v[j].y;
        o.w = o.z + v[j].z;
        scan_store4<VEC>(out, base + j * 4 * kScanThreads, n, o);
        carry += total;
    }
}

// Row `pos` of the AoS array gets point i (zero padded to ds); with frows,
// row `pos` of frows also gets the centred row fl(x - mean) (zero padded).
__device__ __forceinline__ void write_row(const float* __restrict__ pts, int N, int D, int ds, int i, int pos,
                                          float* __restrict__ aos, const DimStat* __restrict__ st,
                                          float* __restrict__ frows) {
    float4* row = reinterpret_cast<float4*>(aos + (size_t)pos * ds);
    float4* frow = frows ? reinterpret_cast<float4*>(frows + (size_t)pos * ds) : nullptr;
    for (int d = 0; d < ds; d += 4) {
        float4 v;
        v.x = (d + 0 < D) ? pts[(size_t)(d + 0) * N + i] : 0.0f;
        v.y = (d + 1 < D) ? pts[(size_t)(d + 1) * N + i] : 0.0f;
        v.z = (d + 2 < D) ? pts[(size_t)(d + 2) * N + i] : 0.0f;
        v.w = (d + 3 < D) ? pts[(size_t)(d + 3) * N + i] : 0.0f;
        row[d >> 2] = v;
        if (frow) {
            float4 f;
            f.x = (d + 0 < D) ? v.x - st[d + 0].mean : 0.0f;
            f.y = (d + 1 < D) ? v.y - st[d + 1].mean : 0.0f;
            f.z = (d + 2 < D) ? v.z - st[d + 2].mean : 0.0f;
            f.w = (d + 3 < D) ? v.w - st[d + 3].mean : 0.0f;
            frow[d >> 2] = f;
        }
    }
}

// One thread per point: SoA reads are coalesced per axis; the AoS row store
// is ds/4 16-byte vector stores to one contiguous row.
__global__ __launch_bounds__(256) void reorder_kernel(const float* __restrict__ pts, int N, int D, int ds,
                                                      const int* __restrict__ cell_of,
                                                      const int* __restrict__ rank,
                                                      const int* __restrict__ start,
                                                      int* __restrict__ sorted_idx,
                                                      int* __restrict__ inv,
                                                      float* __restrict__ aos,
                                                      const DimStat* __restrict__ st,
                                                      float* __restrict__ frows) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N) return;
    const int pos = start[cell_of[i]] + rank[i];
    sorted_idx[pos] = i;
    inv[i] = pos;
    write_row(pts, N, D, ds, i, pos, aos, st, frows);
}

// Per-coordinate statistics.  Block (b, d) reduces coordinate d over its
// slice of the points: fp64 sums of x - x0 and (x - x0)^2 (x0 = the
// coordinate's first value, a shift that keeps the variance well conditioned),
// minimum and maximum.  stats_setup_kernel adds the slices in a fixed order.
__global__ __launch_bounds__(256) void dim_stats_kernel(const float* __restrict__ pts, int N,
                                                        double* __restrict__ part) {
    __shared__ double s_sum[256], s_sq[256];
    __shared__ float s_mn[256], s_mx[256];
    const int t = threadIdx.x;
    const int d = blockIdx.y;
    const float* col = pts + (size_t)d * N;
    const double pivot = col[0];
    double sum = 0.0, sq = 0.0;
    float mn = __builtin_huge_valf(), mx = -__builtin_huge_valf();
    auto take = [&](float v) __attribute__((always_inline)) {
        const double dv = (double)v - pivot;
        sum += dv;
        sq += dv * dv;
        mn = fminf(mn, v);
        mx = fmaxf(mx, v);
    };
    // 16-byte loads, four per thread in flight (a column is 16-byte aligned
    // when d * N is a multiple of 4); the block's slices interleave at 1 KB
    const bool vec = ((reinterpret_cast<uintptr_t>(col) & 15) == 0);
    const long long n4 = vec ? N / 4 : 0;
    const float4* col4 = reinterpret_cast<const float4*>(col);
    const long long step = 256LL * gridDim.x;
    long long j = (long long)blockIdx.x * 256 + t;
    for (; j + 3 * step < n4; j += 4 * step) {
        float4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = col4[j + u * step];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            take(v[u].x); take(v[u].y); take(v[u].z); take(v[u].w);
        }
    }
    for (; j < n4; j += step) {
        const float4 v = col4[j];
        take(v.x); take(v.y); take(v.z); take(v.w);
    }
    for (long long i = 4 * n4 + (long long)blockIdx.x * 256 + t; i < N; i += step) take(col[i]);
    s_sum[t] = sum; s_sq[t] = sq; s_mn[t] = mn; s_mx[t] = mx;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (t < o) {
            s_sum[t] += s_sum[t + o];
            s_sq[t] += s_sq[t + o];
            s_mn[t] = fminf(s_mn[t], s_mn[t + o]);
            s_mx[t] = fmaxf(s_mx[t], s_mx[t + o]);
        }
        __syncthreads();
    }
    if (t == 0) {
        double* p = part + ((size_t)d * gridDim.x + blockIdx.x) * 4;
        p[0] = s_sum[0]; p[1] = s_sq[0]; p[2] = s_mn[0]; p[3] = s_mx[0];
    }
}

// Adds the slices of each coordinate (fixed order) into one DimStat.  A
// non-finite mean (NaN or infinite data) centres at 0 instead.
__global__ __launch_bounds__(128) void stats_setup_kernel(const float* __restrict__ pts,
                                                          const double* __restrict__ part, int nblk, int N, int D,
                                                          DimStat* __restrict__ st) {
    for (int d = threadIdx.x; d < D; d += blockDim.x) {
        const double pivot = pts[(size_t)d * N];
        double sum = 0.0, sq = 0.0;
        float mn = __builtin_huge_valf(), mx = -__builtin_huge_valf();
        const double* p = part + (size_t)d * nblk * 4;
#pragma unroll 8
        for (int b = 0; b < nblk; ++b) {
            sum += p[b * 4 + 0];
            sq += p[b * 4 + 1];
            mn = fminf(mn, (float)p[b * 4 + 2]);
            mx = fmaxf(mx, (float)p[b * 4 + 3]);
        }
        const double shifted = sum / N;
        double var = sq / N - shifted * shifted;
        if (!(var >= 0.0)) var = -1.0;        // NaN data: never preferred as an axis
        float m = (float)(pivot + shifted);
        if (!(m > -3.0e38f && m < 3.0e38f)) m = 0.0f;
        st[d] = DimStat{m, (float)var, mn, mx};
    }
}

// Picks the projection terms of a frame: the kMaxTerms largest-variance
// coordinates (lower index on ties), their centres, the direction count and
// the projection rounding margin.  One thread.
//
// Margin: with y_t = fl(x_t - m_t) = (x_t - m_t)(1 + d_t), |d_t| <= u, the
// sequential fma chain over T terms satisfies
//   |s - sum w_t (x_t - m_t)| <= (gamma_T (1 + u) + u) sum |w_t| |x_t - m_t|
//                             <= (T + 2) u |x - m|     (|w| <= 1, Cauchy-Schwarz)
// and |x - m|^2 <= sum_t max(hi_t - m_t, m_t - lo_t)^2 over the input.  A
// non-finite bound (infinite input) is stored as +inf; frame_dirs_kernel then
// falls back to the raw first coordinates.
__global__ __launch_bounds__(128) void frame_terms_kernel(const DimStat* __restrict__ st, int g, int D,
                                                          Frame* __restrict__ f) {
    __shared__ float s_var[FRNN_MAX_DIM];
    __shared__ int s_coord[kMaxTerms];
    const int tid = threadIdx.x;
    const int T = D < kMaxTerms ? D : kMaxTerms;
    if (tid < D) s_var[tid] = st[tid].var;
    for (int i = tid; i < kMaxTerms; i += blockDim.x) {
        f->coord[i] = 0;
        f->mean[i] = 0.0f;
    }
    for (int i = tid; i < FRNN_FRAME_DIRS * kMaxTerms; i += blockDim.x) (&f->dir[0][0])[i] = 0.0f;
    __syncthreads();
    // rank of coordinate tid in (variance descending, index ascending); the
    // variances are never NaN (the statistics store -1 for NaN data)
    if (tid < D) {
        const float v = s_var[tid];
        int rank = 0;
        for (int e = 0; e < D; ++e) {
            const float w = s_var[e];
            rank += (w > v || (w == v && e < tid)) ? 1 : 0;
        }
        if (rank < T) s_coord[rank] = tid;
    }
    __syncthreads();
    if (tid < T) {
        f->coord[tid] = s_coord[tid];
        f->mean[tid] = st[s_coord[tid]].mean;
    }
    if (tid != 0) return;
    double R2 = 0.0;
    for (int t = 0; t < T; ++t) {
        const DimStat sd = st[s_coord[t]];
        const double e = fmax((double)sd.hi - (double)sd.mean, (double)sd.mean - (double)sd.lo);
        R2 += e * e;
    }
    f->g = g;
    f->terms = T;
    const double E = (T + 2) * 5.9604644775390625e-08 * sqrt(R2) * (1.0 + 9.765625e-04);
    f->margin = E < 1.0e30 ? (float)(E * (1.0 + 9.5367431640625e-07)) : __builtin_huge_valf();
    f->projected = 1;
}

// Pair p of the upper triangle (row-major over a <= b) of a T x T matrix.
__device__ __forceinline__ void pair_of(int p, int T, int& a, int& b) {
    a = 0;
    while (p >= T - a) {
        p -= T - a;
        ++a;
    }
    b = a + p;
}

// Partial covariance sums of the projection terms over a sample of the input:
// block b takes the 256 consecutive points starting at b * tile_stride (every
// point when N <= kCovBlocks * 256), stages y = fl(x - mean) in LDS
// (non-finite values as 0; row stride kMaxTerms + 1 so a wave's reads of one
// point's terms hit distinct banks) and sums y_a * y_b in fp64 for every pair
// a <= b.  Threads split the pairs and, with fewer than 256 pairs, the points.
// The directions only steer the pruning, so a sample of >= 128K points serves.
__global__ __launch_bounds__(256) void cov_kernel(const float* __restrict__ pts, int N, long long tile_stride,
                                                  const Frame* __restrict__ f, double* __restrict__ part) {
    constexpr int kStride = kMaxTerms + 1;
    __shared__ float s_y[256 * kStride];
    __shared__ double s_acc[256];
    const int tid = threadIdx.x;
    const int T = f->terms;
    const int P = T * (T + 1) / 2;
    const int slices = P >= 256 ? 1 : 256 / P;
    int pa[3] = {0, 0, 0}, pb[3] = {0, 0, 0};
    int np = 0, slice = 0;
    if (slices == 1) {
        for (int p = tid; p < P; p += 256) {
            pair_of(p, T, pa[np], pb[np]);
            ++np;
        }
    } else if (tid < P * slices) {
        pair_of(tid % P, T, pa[0], pb[0]);
        slice = tid / P;
        np = 1;
    }
    const long long i0 = (long long)blockIdx.x * tile_stride;
    const int cnt = (int)max(0LL, min(256LL, (long long)N - i0));
    {
        // all of this thread's term loads in flight before the first is used
        float x[kMaxTerms];
#pragma unroll
        for (int t = 0; t < kMaxTerms; ++t)
            x[t] = (t < T && tid < cnt) ? pts[(size_t)f->coord[t] * N + i0 + tid] : 0.0f;
#pragma unroll
        for (int t = 0; t < kMaxTerms; ++t) {
            if (t < T) {
                float y = tid < cnt ? x[t] - f->mean[t] : 0.0f;
                if (!(fabsf(y) <= 3.4e38f)) y = 0.0f;
                s_y[tid * kStride + t] = y;
            }
        }
    }
    __syncthreads();
    // eight interleaved partial sums per pair (point j goes to sum (j / slices)
    // mod 8), added in a fixed order: eight LDS read pairs in flight per step
    double acc[3] = {0.0, 0.0, 0.0};
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        if (k < np) {
            const float* ya = s_y + pa[k];
            const float* yb = s_y + pb[k];
            double sum[8] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
            int j = slice;
            for (; j + 7 * slices < cnt; j += 8 * slices) {
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int r = (j + u * slices) * kStride;
                    sum[u] = fma((double)ya[r], (double)yb[r], sum[u]);
                }
            }
#pragma unroll
            for (int u = 0; u < 7; ++u) {
                const int jj = j + u * slices;
                if (jj < cnt) sum[u] = fma((double)ya[jj * kStride], (double)yb[jj * kStride], sum[u]);
            }
            acc[k] = ((sum[0] + sum[1]) + (sum[2] + sum[3])) + ((sum[4] + sum[5]) + (sum[6] + sum[7]));
        }
    }
    double* out = part + (size_t)blockIdx.x * kMaxPairs;
    if (slices == 1) {
        for (int k = 0; k < np; ++k) out[tid + 256 * k] = acc[k];
    } else {
        s_acc[tid] = acc[0];
        __syncthreads();
        if (tid < P) {
            double sum = 0.0;
            for (int sl = 0; sl < slices; ++sl) sum += s_acc[sl * P + tid];
            out[tid] = sum;
        }
    }
}

// Sum of the covariance partials of pair blockIdx.x over the sampled tiles, in
// a fixed order (strided per thread, then a tree), so the frame is
// reproducible run to run.
__global__ __launch_bounds__(256) void cov_reduce_kernel(const double* __restrict__ part, int nblk,
                                                         const Frame* __restrict__ f,
                                                         double* __restrict__ covsum) {
    __shared__ double s_sum[256];
    const int p = blockIdx.x;
    const int T = f->terms;
    if (p >= T * (T + 1) / 2) return;
    const int tid = threadIdx.x;
    double sum = 0.0;
    for (int b = tid; b < nblk; b += 256) sum += part[(size_t)b * kMaxPairs + p];
    s_sum[tid] = sum;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (tid < w) s_sum[tid] += s_sum[tid + w];
        __syncthreads();
    }
    if (tid == 0) covsum[p] = s_sum[0];
}

// Wave sum of a double that is 0 on lanes 32..63 (a frame has at most 32
// terms, one per lane): five lane-exchange steps over lanes 0..31, then lane
// 0's total to every lane (the same value the full six-step butterfly gives).
__device__ __forceinline__ double wave_sum_f64(double v) {
    static_assert(kMaxTerms <= 32, "terms live in lanes 0..31");
#pragma unroll
    for (int lj = 0; lj < 5; ++lj) {
        unsigned long long a, b;
        xor_pair_u64((unsigned long long)__double_as_longlong(v), 1 << lj, a, b);
        v = __longlong_as_double((long long)a) + __longlong_as_double((long long)b);
    }
    const unsigned long long u = (unsigned long long)__double_as_longlong(v);
    const unsigned lo = (unsigned)__builtin_amdgcn_readfirstlane((int)(unsigned)u);
    const unsigned hi = (unsigned)__builtin_amdgcn_readfirstlane((int)(unsigned)(u >> 32));
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

constexpr int kMaxDirs = FRNN_FRAME_DIRS;

// Raw-coordinate geometry: the first g coordinates on the plan's own cells
// (origin 0, edge cell_raw, binning reciprocal inv_cell_raw, res_raw cells per
// axis), axis 0 split fine0 ways (a power of two, so h0 and inv_h0 are exact
// scalings and a fine cell / fine0 is the plan's cell).  No projection, so no
// rounding margin or slack.  One thread.
__device__ void set_raw_geometry(Frame* __restrict__ f, int g, float cell_raw, float inv_cell_raw, int res_raw,
                                 int fine0) {
    f->projected = 0;
    f->fine0 = fine0;
    f->margin = 0.0f;
    f->slack = 0.0f;
    f->h = cell_raw;
    f->inv_h = inv_cell_raw;
    f->h0 = cell_raw / (float)fine0;
    f->inv_h0 = inv_cell_raw * (float)fine0;
    int stride = 1;
    for (int d = 0; d < kFrameGrid; ++d) {
        f->res[d] = d < g ? (d == 0 ? res_raw * fine0 : res_raw) : 1;
        f->lo[d] = 0.0f;
        f->stride[d] = stride;
        stride *= f->res[d];
    }
    f->cells = stride;
}

// Raw frame of a grid plan without a projection (one wave): no terms or
// directions, the plan's own cells with a fine axis 0.
__global__ __launch_bounds__(64) void raw_frame_kernel(int g, float cell_raw, float inv_cell_raw, int res_raw,
                                                       int fine0, Frame* __restrict__ f) {
    for (int i = threadIdx.x; i < kMaxTerms; i += blockDim.x) {
        f->coord[i] = 0;
        f->mean[i] = 0.0f;
    }
    for (int i = threadIdx.x; i < kFrameGrid * kMaxTerms; i += blockDim.x) (&f->dir[0][0])[i] = 0.0f;
    if (threadIdx.x != 0) return;
    f->g = g;
    f->terms = 0;
    for (int d = 0; d < kFrameGrid; ++d) f->sigma[d] = 0.0f;
    set_raw_geometry(f, g, cell_raw, inv_cell_raw, res_raw, fine0);
}

// Principal directions and geometry of a frame (fp64, one wave; lane t holds
// component t of every direction).  The g leading eigenvectors of the sampled
// covariance C come from orthogonal iteration on (C / cmax)^8 (three
// squarings in LDS, then 2 steps: 16 steps' worth on C; modified
// Gram-Schmidt); each direction's variance is its Rayleigh quotient on C.
// They become the grid axes; weights are scaled by 1 - 2^-18, so the fp32
// directions stay orthonormal up to a shrink (|U d| <= |d| for any d) and
// every direction has norm < 1.
//
// Grid geometry: res_d = max(1, floor(8 sigma_d / h)) cells of edge
//   h >= r (1 + 2^-12) + 2 margin + 2 slack,  slack = 2^-18 (4 sigma_max + h0),
// per axis, h enlarged until prod res <= cells_cap, and an axis of two or
// more cells centred on the mean (origin -res h / 2, |origin| <= 4 sigma).
// Rounding the count down and centring keep the end layers of thin axes from
// holding a distribution tail next to a dense layer: chunks of such a sparse
// layer span many rows, each query then streaming dense neighbouring rows
// alone (one such layer of 1% of the points made a search 3.5x slower).
// Points beyond the cells clamp into the edge cells, which every pruning test
// treats as unbounded outward.  Two points within the radius (fp32
// distance < r2, so |p - q| <= r (1 + 2^-15)) have computed projections closer
// than r (1 + 2^-15) + 2 margin; with the rounding of the binning (bounded by
// slack) their cell coordinates differ by at most one, so every neighbour lies
// in the query's 3^g shell of cells of edge h (axis 0: fine0 cells of edge
// h / fine0 each).  An infinite margin falls back to the raw first g
// coordinates with the plan's cell size.
__global__ __launch_bounds__(64) void frame_dirs_kernel(const double* __restrict__ covsum, double nsamp,
                                                        float radius, float cell_raw, float inv_cell_raw,
                                                        int res_raw, int cells_cap, int fine0,
                                                        Frame* __restrict__ f) {
    __shared__ double s_C[kMaxTerms][kMaxTerms + 1];   // covariance
    __shared__ double s_A[kMaxTerms][kMaxTerms + 1];   // (C / cmax)^2
    __shared__ double s_P[kMaxTerms][kMaxTerms + 1];   // C / cmax, then (C / cmax)^4
    __shared__ double s_v[kMaxDirs][kMaxTerms];          // directions
    __shared__ double s_w[kMaxDirs][kMaxTerms];          // their product with a matrix
    const int t = threadIdx.x;
    const int T = f->terms;
    const int g = f->g;
    const int m = g;
    const int P = T * (T + 1) / 2;
    for (int i = t; i < kMaxTerms * (kMaxTerms + 1); i += kWave) {
        (&s_C[0][0])[i] = 0.0;
        (&s_A[0][0])[i] = 0.0;
        (&s_P[0][0])[i] = 0.0;
    }
    const bool on = t < T;
    auto lds_fence = [&]() {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    };
    lds_fence();
    for (int p = t; p < P; p += kWave) {
        int a, c;
        pair_of(p, T, a, c);
        const double v = covsum[p] / nsamp;
        s_C[a][c] = v;
        s_C[c][a] = v;
    }
    lds_fence();
    // The iteration runs on (C / cmax)^4 (cmax the largest diagonal entry, so
    // the powers stay in range): one step there is four steps on C.  Row t of
    // a product is formed by lane t.
    double cmax = 0.0;
    for (int k = 0; k < T; ++k) cmax = fmax(cmax, s_C[k][k]);
    const double cs = (cmax > 0.0 && cmax < 1.0e300) ? 1.0 / cmax : 1.0;
    if (on)
#pragma unroll 1
        for (int k = 0; k < kMaxTerms; ++k) s_P[t][k] = s_C[t][k] * cs;
    lds_fence();
    // Every lane takes NC entries of one row: 4 lanes x 4 columns per row for
    // T <= 16, 2 lanes x 16 columns for T <= 32 (entries outside T x T stay
    // 0).  Each entry sums over l in order, as a one-lane-per-row product would.
    auto square_cols = [&](auto nc_const, double (*src)[kMaxTerms + 1], double (*dst)[kMaxTerms + 1]) {
        constexpr int NC = decltype(nc_const)::value;
        constexpr int R = NC == 4 ? 16 : 32;   // rows covered by the wave
        const int row = t % R;
        const int c0 = (t / R) * NC;
        double acc[NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[c] = 0.0;
        for (int l = 0; l < T; ++l) {
            const double a = src[row][l];
#pragma unroll
            for (int c = 0; c < NC; ++c) acc[c] = fma(a, src[l][c0 + c], acc[c]);
        }
        lds_fence();
#pragma unroll
        for (int c = 0; c < NC; ++c) dst[row][c0 + c] = (row < T && c0 + c < T) ? acc[c] : 0.0;
        lds_fence();
    };
    auto square = [&](double (*src)[kMaxTerms + 1], double (*dst)[kMaxTerms + 1]) {
        if (T <= 16) square_cols(IntC<4>{}, src, dst);
        else square_cols(IntC<16>{}, src, dst);
    };
    square(s_P, s_A);
    square(s_A, s_P);
    square(s_P, s_A);   // s_A = (C / cmax)^8
    // The directions live in LDS (s_v[j][k]: component k of direction j;
    // s_w: a product M v), lane t < kMaxTerms owning component t, and every
    // loop below stays rolled: this one-wave kernel runs each instruction a
    // few times at most, so its time goes to fetching code, which a compact
    // body keeps short.
    const int tc = t < kMaxTerms ? t : 0;   // lanes >= kMaxTerms read lane 0's slot, store nothing
    for (int j = 0; j < kMaxDirs; ++j)
        if (t < kMaxTerms) s_v[j][t] = (on && j < m) ? ((t == j) ? 1.0 : 0.0625 * (double)((t * (2 * j + 3)) % 7 - 3)) : 0.0;
    lds_fence();
    // w_j = M v_j (M = C or its scaled eighth power): lane (r, j0) forms row r
    // of directions j0 and j0 + 2, summing over k in order
    auto matvec = [&](double (*M)[kMaxTerms + 1]) {
        const int r = t & 31;
        for (int j = t >> 5; j < m; j += 2) {
            double w = 0.0;
            for (int k = 0; k < T; ++k) w = fma(M[r][k], s_v[j][k], w);
            s_w[j][r] = r < T ? w : 0.0;
        }
        lds_fence();
    };
    // modified Gram-Schmidt of s_w into s_v; a collapsed vector is replaced by
    // the first coordinate direction with a substantial residual (one exists:
    // j < m <= T).  Lanes >= kMaxTerms carry 0, as the wave sums require.
    auto orthonormalise = [&]() {
        for (int j = 0; j < m; ++j) {
            double x = t < kMaxTerms ? s_w[j][tc] : 0.0;
            const double n_in = sqrt(wave_sum_f64(x * x));
            for (int k = 0; k < j; ++k) {
                const double vk = t < kMaxTerms ? s_v[k][tc] : 0.0;
                x -= wave_sum_f64(x * vk) * vk;
            }
            double nrm = sqrt(wave_sum_f64(x * x));
            if (!(nrm > 1.0e-300 && nrm > 1.0e-12 * n_in && nrm < 1.0e300)) {
                for (int c = 0; c < T; ++c) {
                    double cand = (t == c) ? 1.0 : 0.0;
                    for (int k = 0; k < j; ++k) {
                        const double vk = t < kMaxTerms ? s_v[k][tc] : 0.0;
                        cand -= wave_sum_f64(cand * vk) * vk;
                    }
                    const double nc = sqrt(wave_sum_f64(cand * cand));
                    if (nc > 0.1) {
                        x = cand;
                        nrm = nc;
                        break;
                    }
                }
            }
            if (t < kMaxTerms) s_v[j][t] = x / nrm;
            lds_fence();
        }
    };
    // (the start vectors are independent; the first product needs no
    // orthonormal start)
    for (int it = 0; it < 2; ++it) {
        matvec(s_A);
        orthonormalise();
    }
    // Orthogonal iteration leaves direction j converged towards eigenvector j
    // (descending eigenvalues); its variance is the Rayleigh quotient v_j' C v_j.
    // A rotation inside the subspace would not change the captured variance.
    matvec(s_C);
    constexpr double kShrink = 1.0 - 3.814697265625e-06;   // 1 - 2^-18
    for (int j = 0; j < m; ++j) {
        const double x = t < kMaxTerms ? s_v[j][tc] : 0.0;
        const double lam = wave_sum_f64(x * (t < kMaxTerms ? s_w[j][tc] : 0.0));
        if (on) f->dir[j][t] = (float)(x * kShrink);
        if (t == 0) f->sigma[j] = (float)sqrt(fmax(lam, 0.0));
    }
    if (t != 0) return;
    // ---- geometry (one thread) ----
    const bool exact = f->margin < 1.0e30f;
    f->fine0 = fine0;
    if (!exact) {
        // infinite input: grid on the raw first g coordinates (axis 0 still
        // in fine0 cells per plan cell)
        set_raw_geometry(f, g, cell_raw, inv_cell_raw, res_raw, fine0);
        return;
    }
    double sig[kFrameGrid];
    double smax = 0.0;
    for (int d = 0; d < kFrameGrid; ++d) {
        sig[d] = d < g ? (double)f->sigma[d] : 0.0;
        smax = fmax(smax, sig[d]);
    }
    const double h0 = (double)radius * (1.0 + 2.44140625e-04) + 2.0 * (double)f->margin;
    // slack as stored (fp32, rounded up by the 2^-10 factor), so h covers it
    const double slack = (double)(float)(3.814697265625e-06 * (4.0 * smax + h0) * (1.0 + 9.765625e-04));
    // start where no axis needs more than 2^20 cells, then grow h by 1/16
    // until the grid fits (at most ~700 steps from there; a bounded loop with
    // a single-cell fallback keeps the thread finite whatever the input)
    double h = fmax(h0 + 2.0 * slack, 8.0 * smax / 1048576.0);
    int res[kFrameGrid];
    long long cells = 0;
    // the cells of edge h fit cells_cap / fine0; axis 0 is then split fine0 ways
    const long long coarse_cap = cells_cap / fine0;
    for (int pass = 0; pass < 4096 && !(cells >= 1 && cells <= coarse_cap); ++pass) {
        if (pass > 0) h *= 1.0625;
        cells = 1;
        for (int d = 0; d < kFrameGrid; ++d) {
            double rd = d < g ? floor(8.0 * sig[d] / h) : 1.0;
            rd = fmin(fmax(rd, 1.0), 1048576.0);
            res[d] = (int)rd;
            cells *= res[d];
        }
    }
    if (!(cells >= 1 && cells <= coarse_cap))
        for (int d = 0; d < kFrameGrid; ++d) res[d] = 1;
    if (g >= 1) res[0] *= fine0;
    // store h rounded up and inv_h rounded down, so the binning never
    // narrows a cell below h
    // (both positive: one ulp up / down is the bit pattern +- 1)
    float hf = (float)h;
    if ((double)hf < h) hf = __uint_as_float(__float_as_uint(hf) + 1u);
    float ih = (float)(1.0 / (double)hf);
    if ((double)ih > 1.0 / (double)hf) ih = __uint_as_float(__float_as_uint(ih) - 1u);
    f->h = hf;
    f->inv_h = ih;
    // axis 0: fine0 (a power of two) cells per h, exact scalings of h, inv_h
    f->h0 = hf / (float)fine0;
    f->inv_h0 = ih * (float)fine0;
    f->slack = (float)slack;
    int stride = 1;
    for (int d = 0; d < kFrameGrid; ++d) {
        f->res[d] = res[d];
        // a split axis is centred on the mean (res h <= 8 sigma, so |lo| <= 4 sigma);
        // an axis of one cell bins everything to it whatever its origin
        const int coarse = d == 0 && g >= 1 ? res[0] / fine0 : res[d];
        f->lo[d] = d < g ? (float)(coarse >= 2 ? -0.5 * (double)coarse * (double)hf : -4.0 * sig[d]) : 0.0f;
        f->stride[d] = stride;
        stride *= res[d];
    }
    f->cells = stride;
}

// Binning on a frame's grid directions: projections (or, without a
// projection, the raw first g coordinates), clamped cell coordinates, cell id
// and the arrival slot in the cell.
__global__ __launch_bounds__(256) void bin_frame_kernel(const float* __restrict__ pts, int N,
                                                        const Frame* __restrict__ f, int cells,
                                                        int* __restrict__ cell_of, int* __restrict__ rank,
                                                        int* __restrict__ cnt) {
    // the projection terms, staged once per block: each point's coordinate
    // loads then issue together instead of one term's load waiting on the
    // term's coordinate index
    __shared__ int s_coord[kMaxTerms];
    __shared__ float s_mean[kMaxTerms];
    __shared__ float s_dir[kFrameGrid][kMaxTerms];
    const int tid = threadIdx.x;
    if (tid < kMaxTerms) {
        s_coord[tid] = f->coord[tid];
        s_mean[tid] = f->mean[tid];
#pragma unroll
        for (int m = 0; m < kFrameGrid; ++m) s_dir[m][tid] = f->dir[m][tid];
    }
    __syncthreads();
    const int i = blockIdx.x * blockDim.x + tid;
    if (i >= N) return;
    const int g = f->g;
    float s[kFrameGrid];
    if (f->projected) {
        // frame_project's sums: the fma chain over the terms in order
        const int T = f->terms;
        float x[kMaxTerms];
#pragma unroll
        for (int t = 0; t < kMaxTerms; ++t) x[t] = t < T ? pts[(size_t)s_coord[t] * N + i] : 0.0f;
#pragma unroll
        for (int m = 0; m < kFrameGrid; ++m) s[m] = 0.0f;
#pragma unroll
        for (int t = 0; t < kMaxTerms; ++t) {
            if (t < T) {
                const float y = x[t] - s_mean[t];
#pragma unroll
                for (int m = 0; m < kFrameGrid; ++m) s[m] = fmaf(s_dir[m][t], y, s[m]);
            }
        }
    } else {
#pragma unroll
        for (int d = 0; d < kFrameGrid; ++d) s[d] = d < g ? pts[(size_t)d * N + i] : 0.0f;
    }
    int c = 0;
#pragma unroll
    for (int d = 0; d < kFrameGrid; ++d)
        if (d < g) c += sub_bin(s[d], f->lo[d], d == 0 ? f->inv_h0 : f->inv_h, f->res[d]) * f->stride[d];
    c = c < cells ? c : cells - 1;   // the frame fits `cells`; a mismatched count array stays in bounds
    cell_of[i] = c;
    rank[i] = atomicAdd(&cnt[c], 1);
}

__global__ __launch_bounds__(256) void transpose_kernel(const float* __restrict__ pts, int N, int D, int ds,
                                                        float* __restrict__ aos,
                                                        const DimStat* __restrict__ st,
                                                        float* __restrict__ frows) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N) return;
    write_row(pts, N, D, ds, i, i, aos, st, frows);
}

// Output transpose through LDS, qt original queries per workgroup (64, or 32
// for K > 64): the workgroup's sorted positions inv[i] go to LDS first; each
// query's K keys (row inv[i] of the sorted order, contiguous) are then read as
// 16-byte pairs, kUnpermBatch per thread in flight before any is stored, and
// split into index and distance columns of two padded LDS tiles [k][query];
// then the workgroup writes whole output rows k, qt consecutive queries per
// store.  Lists and outputs are touched once: nontemporal loads and stores.
// The tiles take 2 * K * (qt + 1) * 4 bytes of dynamic LDS plus qt ints of
// positions; pairs is set when K and cap are even and lists is 16-byte
// aligned.
constexpr int kUnpermBatch = 8;

__global__ __launch_bounds__(256) void unpermute_kernel(const unsigned long long* __restrict__ lists,
                                                        int cap, const int* __restrict__ inv, int N,
                                                        int K, int qt, int pairs, int* __restrict__ idxs,
                                                        float* __restrict__ dists) {
    typedef unsigned long long u64x2 __attribute__((ext_vector_type(2)));
    const int kPitch = qt + 1;
    extern __shared__ int s_dyn[];
    int* const s_idx = s_dyn;
    float* const s_d2 = reinterpret_cast<float*>(s_dyn + K * kPitch);
    int* const s_sp = s_dyn + 2 * K * kPitch;
    const int i0 = blockIdx.x * qt;
    const int nq = min(qt, N - i0);
    const int tid = threadIdx.x;
    const int nt = blockDim.x;
    for (int q = tid; q < nq; q += nt) s_sp[q] = inv ? inv[i0 + q] : i0 + q;
    __syncthreads();
    auto put = [&](int q, int k, unsigned long long key) __attribute__((always_inline)) {
        s_idx[k * kPitch + q] = (int)(unsigned int)key;
        s_d2[k * kPitch + q] = key_d2(key);
    };
    if (pairs) {
        const int half = K >> 1;   // key pairs per query
        const int total = nq * half;
        for (int j0 = 0; j0 < total; j0 += kUnpermBatch * nt) {
            u64x2 kv[kUnpermBatch];
#pragma unroll
            for (int u = 0; u < kUnpermBatch; ++u) {
                const int j = j0 + u * nt + tid;
                if (j < total) {
                    const int q = j / half;
                    const int k = 2 * (j - q * half);
                    kv[u] = __builtin_nontemporal_load(
                        reinterpret_cast<const u64x2*>(lists + (size_t)s_sp[q] * cap + k));
                }
            }
#pragma unroll
            for (int u = 0; u < kUnpermBatch; ++u) {
                const int j = j0 + u * nt + tid;
                if (j < total) {
                    const int q = j / half;
                    const int k = 2 * (j - q * half);
                    put(q, k, kv[u].x);
                    put(q, k + 1, kv[u].y);
                }
            }
        }
    } else {
        const int total = nq * K;
        for (int j0 = 0; j0 < total; j0 += kUnpermBatch * nt) {
            unsigned long long kv[kUnpermBatch];
#pragma unroll
            for (int u = 0; u < kUnpermBatch; ++u) {
                const int j = j0 + u * nt + tid;
                if (j < total) {
                    const int q = j / K;
                    kv[u] = __builtin_nontemporal_load(lists + (size_t)s_sp[q] * cap + (j - q * K));
                }
            }
#pragma unroll
            for (int u = 0; u < kUnpermBatch; ++u) {
                const int j = j0 + u * nt + tid;
                if (j < total) {
                    const int q = j / K;
                    put(q, j - q * K, kv[u]);
                }
            }
        }
    }
    __syncthreads();
    for (int j = tid; j < K * qt; j += nt) {
        const int k = j / qt;
        const int q = j - k * qt;
        if (q < nq) {
            __builtin_nontemporal_store(s_idx[k * kPitch + q], &idxs[(size_t)k * N + i0 + q]);
            __builtin_nontemporal_store(s_d2[k * kPitch + q], &dists[(size_t)k * N + i0 + q]);
        }
    }
}

static int blocks_for(long long n, int threads) { return (int)((n + threads - 1) / threads); }

static thread_local hipError_t g_launch_error = hipSuccess;

int launch_result() {
    const hipError_t e = hipGetLastError();
    if (e == hipSuccess) return 0;
    g_launch_error = e;
    return 3;
}

hipError_t last_launch_error() { return g_launch_error; }

int launch_fill_i32(int* p, long long n, int v, hipStream_t s) {
    if (n <= 0) return 0;
    long long nb = (n / 4 + 255) / 256;   // one int4 per thread
    nb = nb < 1 ? 1 : (nb > 65536 ? 65536 : nb);
    hipLaunchKernelGGL(fill_i32_kernel, dim3((unsigned)nb), dim3(256), 0, s, p, n, v);
    return launch_result();
}

int launch_bin_count(const float* pts, int N, int g, int res, float inv_cell, const void* frame_ws,
                     int cells, int* cell_of, int* rank, int* cnt, hipStream_t s) {
    if (N <= 0) return 0;
    if (frame_ws) {
        if (cells < 1) return 1;
        const Frame* f = reinterpret_cast<const Frame*>(static_cast<const char*>(frame_ws));
        hipLaunchKernelGGL(bin_frame_kernel, dim3(blocks_for(N, 256)), dim3(256), 0, s, pts, N, f, cells,
                           cell_of, rank, cnt);
    } else {
        hipLaunchKernelGGL(bin_count_kernel, dim3(blocks_for(N, 256)), dim3(256), 0, s, pts, N, g, res,
                           inv_cell, cell_of, rank, cnt);
    }
    return launch_result();
}

int scan_partials_count(int n) { return (n + kScanTile - 1) / kScanTile + 1; }

// ---- allocation-free scan ----------------------------------------------------
// The scan's only scratch is one partial sum per tile of kScanTile ints, at most
// kScanTile of them (n <= kScanTile^2).  launch_exclusive_scan_noalloc keeps
// them in this file-scope device array (16 KB per device, held until the
// process ends) instead of a caller's workspace.  In host code `scratch` names
// a host-side stand-in, not a device address: the device address of each
// device's copy comes from hipGetSymbolAddress, looked up once per device
// (with that device current, on its first call) and used for every kernel
// argument.  Every call on one device shares the array: calls that overlap on
// a device race.  Nothing in it needs clearing: the reduce pass writes every
// partial the final pass reads.
static __device__ __align__(256) int scratch[kScanTile];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
int* g_scratch_dev[kMaxDevices] = {};
hipError_t g_scratch_err = hipSuccess;
}  // namespace

int scan_noalloc_max() { return kScanTile * kScanTile; }

int launch_exclusive_scan_noalloc(const int* in, int n, int* out, hipStream_t s) {
    if (n <= 0) return 0;
    if (n > scan_noalloc_max()) return 2;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        g_scratch_err = e != hipSuccess ? e : hipErrorInvalidDevice;
        return 4;
    }
    int* p = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        if (!g_scratch_dev[dev]) {
            void* a = nullptr;
            e = hipGetSymbolAddress(&a, HIP_SYMBOL(scratch));
            if (e != hipSuccess || !a) {
                g_scratch_err = e != hipSuccess ? e : hipErrorInvalidSymbol;
                return 4;
            }
            g_scratch_dev[dev] = static_cast<int*>(a);
        }
        p = g_scratch_dev[dev];
    }
    return launch_exclusive_scan(in, n, out, p, s);
}

hipError_t scan_noalloc_error() { return g_scratch_err; }

namespace {
template <bool CLEAR>
int scan_launch(const int* in, int n, int* out, int* partials, const int* bound, hipStream_t s) {
    if (n <= 0) return 0;
    const int nb = (n + kScanTile - 1) / kScanTile;
    if (nb > kScanTile) return 2;
    const bool vec = (((uintptr_t)in | (uintptr_t)out) & 15) == 0;
    int* const io = const_cast<int*>(in);   // written only with CLEAR
    if (vec)
        hipLaunchKernelGGL(scan_reduce_kernel<true>, dim3(nb), dim3(kScanThreads), 0, s, in, n, partials, bound);
    else
        hipLaunchKernelGGL(scan_reduce_kernel<false>, dim3(nb), dim3(kScanThreads), 0, s, in, n, partials, bound);
    if (vec)
        hipLaunchKernelGGL((scan_final_kernel<true, CLEAR>), dim3(nb), dim3(kScanThreads), 0, s, io, n, partials,
                           out, bound);
    else
        hipLaunchKernelGGL((scan_final_kernel<false, CLEAR>), dim3(nb), dim3(kScanThreads), 0, s, io, n,
                           partials, out, bound);
    return launch_result();
}
}  // namespace

int launch_exclusive_scan(const int* in, int n, int* out, int* partials, hipStream_t s) {
    return scan_launch<false>(in, n, out, partials, nullptr, s);
}

int launch_count_scan(int* cnt, int n, const int* bound, int* out, int* partials, hipStream_t s) {
    return scan_launch<true>(cnt, n, out, partials, bound, s);
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

FrameLayout frame_layout() {
    FrameLayout L{};
    size_t off = 0;
    L.frame = off;    off = align256(off + sizeof(Frame));
    L.cov = off;      off = align256(off + (size_t)kCovBlocks * kMaxPairs * sizeof(double));
    L.covsum = off;   off = align256(off + (size_t)kMaxPairs * sizeof(double));
    L.total = off;
    return L;
}

StatsLayout stats_layout(int D) {
    StatsLayout L{};
    L.dims = 0;
    L.part = align256((size_t)FRNN_MAX_DIM * sizeof(DimStat));
    L.total = align256(L.part + (size_t)kStatBlocks * (D > 0 ? D : 1) * 4 * sizeof(double));
    return L;
}

int launch_point_stats(const float* pts, int N, int D, void* stats_ws, hipStream_t s) {
    if (N <= 0) return 0;
    const StatsLayout L = stats_layout(D);
    char* base = static_cast<char*>(stats_ws);
    double* part = reinterpret_cast<double*>(base + L.part);
    hipLaunchKernelGGL(dim_stats_kernel, dim3(kStatBlocks, D), dim3(256), 0, s, pts, N, part);
    hipLaunchKernelGGL(stats_setup_kernel, dim3(1), dim3(128), 0, s, pts, part, kStatBlocks, N, D,
                       reinterpret_cast<DimStat*>(base + L.dims));
    return launch_result();
}

int launch_frame(const float* pts, int N, int D, const frnn_plan_t& plan, long long cells,
                 const void* stats_ws, void* ws, hipStream_t s) {
    if (N <= 0 || !has_frame(plan, D)) return 0;
    const FrameLayout L = frame_layout();
    char* base = static_cast<char*>(ws);
    Frame* f = reinterpret_cast<Frame*>(base + L.frame);
    if (!has_projected_frame(plan, D)) {
        hipLaunchKernelGGL(raw_frame_kernel, dim3(1), dim3(kWave), 0, s, plan.grid_dim, plan.cell_size,
                           plan.inv_cell, plan.res, kFine0, f);
        return launch_result();
    }
    const DimStat* st = reinterpret_cast<const DimStat*>(static_cast<const char*>(stats_ws) + stats_layout(D).dims);
    double* cov = reinterpret_cast<double*>(base + L.cov);
    hipLaunchKernelGGL(frame_terms_kernel, dim3(1), dim3(128), 0, s, st, plan.grid_dim, D, f);
    // covariance sample: kCovBlocks tiles of 256 consecutive points, evenly spaced
    const long long tile_stride = N <= (long long)kCovBlocks * 256 ? 256 : (long long)N / kCovBlocks;
    long long nsamp = 0;
    for (int b = 0; b < kCovBlocks; ++b) {
        const long long i0 = (long long)b * tile_stride;
        nsamp += i0 < N ? (N - i0 < 256 ? N - i0 : 256) : 0;
    }
    double* covsum = reinterpret_cast<double*>(base + L.covsum);
    hipLaunchKernelGGL(cov_kernel, dim3(kCovBlocks), dim3(256), 0, s, pts, N, tile_stride, f, cov);
    hipLaunchKernelGGL(cov_reduce_kernel, dim3(kMaxPairs), dim3(256), 0, s, cov, kCovBlocks, f, covsum);
    hipLaunchKernelGGL(frame_dirs_kernel, dim3(1), dim3(kWave), 0, s, covsum, (double)nsamp,
                       plan.cell_size, plan.cell_size, plan.inv_cell, plan.res, (int)cells, kFine0, f);
    return launch_result();
}

static const DimStat* stats_of(const void* stats_ws, int D) {
    return stats_ws ? reinterpret_cast<const DimStat*>(static_cast<const char*>(stats_ws) + stats_layout(D).dims)
                    : nullptr;
}

int launch_reorder(const float* pts, int N, int D, const int* cell_of, const int* rank, const int* start,
                   int* sorted_idx, int* inv, float* aos, const void* stats_ws, float* frows, hipStream_t s) {
    if (N <= 0) return 0;
    if (frows && !stats_ws) return 1;
    hipLaunchKernelGGL(reorder_kernel, dim3(blocks_for(N, 256)), dim3(256), 0, s, pts, N, D,
                       aos_stride(D), cell_of, rank, start, sorted_idx, inv, aos, stats_of(stats_ws, D), frows);
    return launch_result();
}

int launch_transpose(const float* pts, int N, int D, float* aos, const void* stats_ws, float* frows,
                     hipStream_t s) {
    if (N <= 0) return 0;
    if (frows && !stats_ws) return 1;
    hipLaunchKernelGGL(transpose_kernel, dim3(blocks_for(N, 256)), dim3(256), 0, s, pts, N, D,
                       aos_stride(D), aos, stats_of(stats_ws, D), frows);
    return launch_result();
}

int launch_unpermute(const unsigned long long* lists, int cap, const int* inv, int N, int K, int* idxs,
                     float* dists, hipStream_t s) {
    if (N <= 0) return 0;
    if (K < 1 || K > FRNN_MAX_K || cap < K) return 1;   // the LDS tile holds K <= FRNN_MAX_K keys
    const int pairs = (K % 2 == 0 && cap % 2 == 0 && (reinterpret_cast<uintptr_t>(lists) & 15) == 0) ? 1 : 0;
    const int qt = K > 64 ? 32 : 64;
    const size_t lds = ((size_t)2 * K * (qt + 1) + qt) * sizeof(int);   // <= 33 KiB
    hipLaunchKernelGGL(unpermute_kernel, dim3(blocks_for(N, qt)), dim3(256), lds, s, lists, cap, inv, N,
                       K, qt, pairs, idxs, dists);
    return launch_result();
}

}  // namespace frnn
