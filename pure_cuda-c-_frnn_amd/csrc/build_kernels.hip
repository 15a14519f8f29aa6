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
//   * the scan is a three-phase reduce/scan/propagate over 4096-element tiles
//     with no inter-block spin waits.
#include "frnn_device.hpp"
#include "frnn_internal.hpp"

namespace frnn {

constexpr int kScanThreads = 256;
constexpr int kScanItems = 16;
constexpr int kScanTile = kScanThreads * kScanItems;   // 4096

__global__ void fill_i32_kernel(int* __restrict__ p, long long n, int v) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (; i < n; i += stride) p[i] = v;
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

__device__ __forceinline__ int block_exclusive_scan_256(int v, int* s_tmp, int* total) {
    // Hillis-Steele over 256 per-thread values in LDS.
    const int t = threadIdx.x;
    s_tmp[t] = v;
    __syncthreads();
    for (int o = 1; o < kScanThreads; o <<= 1) {
        int x = (t >= o) ? s_tmp[t - o] : 0;
        __syncthreads();
        s_tmp[t] += x;
        __syncthreads();
    }
    const int incl = s_tmp[t];
    *total = s_tmp[kScanThreads - 1];
    __syncthreads();
    return incl - v;
}

// flag_min > 0: the scanned value is (in[i] >= flag_min), e.g. "cell is big".
__device__ __forceinline__ int scan_value(const int* __restrict__ in, long long idx, int n, int flag_min) {
    if (idx >= n) return 0;
    const int v = in[idx];
    return flag_min > 0 ? (v >= flag_min ? 1 : 0) : v;
}

__global__ __launch_bounds__(kScanThreads) void scan_reduce_kernel(const int* __restrict__ in, int n,
                                                                   int* __restrict__ partials, int flag_min) {
    __shared__ int s_tmp[kScanThreads];
    const long long base = (long long)blockIdx.x * kScanTile + (long long)threadIdx.x * kScanItems;
    int sum = 0;
#pragma unroll
    for (int j = 0; j < kScanItems; ++j) sum += scan_value(in, base + j, n, flag_min);
    int total;
    block_exclusive_scan_256(sum, s_tmp, &total);
    if (threadIdx.x == 0) partials[blockIdx.x] = total;
}

// Single block: exclusive scan of up to kScanTile partial sums, in place.
__global__ __launch_bounds__(kScanThreads) void scan_partials_kernel(int* __restrict__ partials, int nb) {
    __shared__ int s_tmp[kScanThreads];
    const int base = threadIdx.x * kScanItems;
    int v[kScanItems];
    int sum = 0;
#pragma unroll
    for (int j = 0; j < kScanItems; ++j) {
        v[j] = (base + j < nb) ? partials[base + j] : 0;
        sum += v[j];
    }
    int total;
    int run = block_exclusive_scan_256(sum, s_tmp, &total);
#pragma unroll
    for (int j = 0; j < kScanItems; ++j) {
        if (base + j < nb) partials[base + j] = run;
        run += v[j];
    }
}

__global__ __launch_bounds__(kScanThreads) void scan_final_kernel(const int* __restrict__ in, int n,
                                                                  const int* __restrict__ partials,
                                                                  int* __restrict__ out, int flag_min) {
    __shared__ int s_tmp[kScanThreads];
    const long long base = (long long)blockIdx.x * kScanTile + (long long)threadIdx.x * kScanItems;
    int v[kScanItems];
    int sum = 0;
#pragma unroll
    for (int j = 0; j < kScanItems; ++j) {
        v[j] = scan_value(in, base + j, n, flag_min);
        sum += v[j];
    }
    int total;
    int run = block_exclusive_scan_256(sum, s_tmp, &total) + partials[blockIdx.x];
#pragma unroll
    for (int j = 0; j < kScanItems; ++j) {
        long long idx = base + j;
        if (idx < n) out[idx] = run;
        run += v[j];
    }
}

// Row `pos` of the AoS array gets point i (zero padded to ds); when filter
// rows are requested, row `pos` of frows gets fl(x - mean) and fnorm[pos] its
// squared norm (sequential fma).
__device__ __forceinline__ void write_rows(const float* __restrict__ pts, int N, int D, int ds, int i, int pos,
                                           float* __restrict__ aos, const DimStat* __restrict__ st,
                                           float* __restrict__ frows, float* __restrict__ fnorm) {
    float4* row = reinterpret_cast<float4*>(aos + (size_t)pos * ds);
    float4* frow = frows ? reinterpret_cast<float4*>(frows + (size_t)pos * ds) : nullptr;
    float nrm = 0.0f;
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
            nrm = fmaf(f.x, f.x, nrm);
            nrm = fmaf(f.y, f.y, nrm);
            nrm = fmaf(f.z, f.z, nrm);
            nrm = fmaf(f.w, f.w, nrm);
        }
    }
    if (frow) fnorm[pos] = nrm;
}

// One thread per point: SoA reads are coalesced per axis; the AoS row store
// is ds/4 16-byte vector stores to one contiguous row.  Points of big cells go
// to their sub-bin's range of the cell (within-cell refinement order, sub-bin
// key from sub_count_kernel).
__global__ __launch_bounds__(256) void reorder_kernel(const float* __restrict__ pts, int N, int D, int ds,
                                                      const int* __restrict__ cell_of,
                                                      const int* __restrict__ rank,
                                                      const int* __restrict__ start,
                                                      const int* __restrict__ cnt,
                                                      const int* __restrict__ subkey,
                                                      const int* __restrict__ bidx,
                                                      const int* __restrict__ substart,
                                                      int* __restrict__ sorted_idx,
                                                      int* __restrict__ inv,
                                                      float* __restrict__ aos,
                                                      const DimStat* __restrict__ st,
                                                      float* __restrict__ frows,
                                                      float* __restrict__ fnorm) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N) return;
    const int c = cell_of[i];
    int pos = start[c] + rank[i];
    if (subkey && cnt[c] >= kBigCell) {
        const size_t base = (size_t)bidx[c] * kSubBins;
        pos += substart[base + subkey[i]] - substart[base];
    }
    sorted_idx[pos] = i;
    inv[i] = pos;
    write_rows(pts, N, D, ds, i, pos, aos, st, frows, fnorm);
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
    for (long long i = (long long)blockIdx.x * 256 + t; i < N; i += 256LL * gridDim.x) {
        const float v = col[i];
        const double dv = (double)v - pivot;
        sum += dv;
        sq += dv * dv;
        mn = fminf(mn, v);
        mx = fmaxf(mx, v);
    }
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

// Picks the projection terms among coordinates g..D-1 (the kMaxTerms largest
// variances, lower index on ties), their centres, the sub-bin split and the
// projection rounding margin.  One thread.
//
// Margin: with y_t = fl(x_t - m_t) = (x_t - m_t)(1 + d_t), |d_t| <= u, the
// sequential fma chain over T terms satisfies
//   |s - sum w_t (x_t - m_t)| <= (gamma_T (1 + u) + u) sum |w_t| |x_t - m_t|
//                             <= (T + 2) u |x - m|     (|w| <= 1, Cauchy-Schwarz)
// and |x - m|^2 <= sum_t max(hi_t - m_t, m_t - lo_t)^2 over the input.  A
// non-finite bound (infinite input) is stored as +inf: one sub-bin then.
__global__ void refine_terms_kernel(const DimStat* __restrict__ st, int g, int D, RefineInfo* __restrict__ info) {
    if (threadIdx.x != 0) return;
    const int nd = D - g;
    const int T = nd < kMaxTerms ? nd : kMaxTerms;
    unsigned long long taken0 = 0ull, taken1 = 0ull;
    double R2 = 0.0;
    for (int t = 0; t < kMaxTerms; ++t) {
        info->coord[t] = 0;
        info->mean[t] = 0.0f;
        info->w0[t] = 0.0f;
        info->w1[t] = 0.0f;
    }
    for (int t = 0; t < T; ++t) {
        int best = -1;
        for (int d = g; d < D; ++d) {
            const unsigned long long bit = 1ull << (d & 63);
            if ((d < 64 ? taken0 : taken1) & bit) continue;
            if (best < 0 || st[d].var > st[best].var) best = d;
        }
        if (best < 64) taken0 |= 1ull << best;
        else taken1 |= 1ull << (best - 64);
        const DimStat s = st[best];
        info->coord[t] = best;
        info->mean[t] = s.mean;
        const double e = fmax((double)s.hi - (double)s.mean, (double)s.mean - (double)s.lo);
        R2 += e * e;
    }
    const int L = T >= 2 ? 2 : 1;
    info->L = L;
    info->nb1 = L == 2 ? 32 : kSubBins;
    info->nb2 = L == 2 ? 32 : 1;
    info->terms = T;
    info->lo0 = info->lo1 = info->inv0 = info->inv1 = 0.0f;
    const double E = (T + 2) * 5.9604644775390625e-08 * sqrt(R2) * (1.0 + 9.765625e-04);
    info->margin = E < 1.0e30 ? (float)(E * (1.0 + 9.5367431640625e-07)) : __builtin_huge_valf();
    for (int k = 0; k < 7; ++k) info->pad[k] = 0;
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
                                                  const RefineInfo* __restrict__ ri, double* __restrict__ part) {
    constexpr int kStride = kMaxTerms + 1;
    __shared__ float s_y[256 * kStride];
    __shared__ double s_acc[256];
    const int tid = threadIdx.x;
    const int T = ri->terms;
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
    for (int t = 0; t < T; ++t) {
        float y = 0.0f;
        if (tid < cnt) {
            y = pts[(size_t)ri->coord[t] * N + i0 + tid] - ri->mean[t];
            if (!(fabsf(y) <= 3.4e38f)) y = 0.0f;
        }
        s_y[tid * kStride + t] = y;
    }
    __syncthreads();
    double acc[3] = {0.0, 0.0, 0.0};
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        if (k < np) {
            double sum = 0.0;
            for (int j = slice; j < cnt; j += slices)
                sum = fma((double)s_y[j * kStride + pa[k]], (double)s_y[j * kStride + pb[k]], sum);
            acc[k] = sum;
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

// Wave sum of a double through the lane exchanges (no LDS).
__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
    for (int lj = 0; lj < 6; ++lj) {
        const unsigned long long u = xor_lane_u64((unsigned long long)__double_as_longlong(v), 1 << lj);
        v += __longlong_as_double((long long)u);
    }
    return v;
}
__device__ __forceinline__ double wave_max_f64(double v) {
#pragma unroll
    for (int lj = 0; lj < 6; ++lj) {
        const unsigned long long u = xor_lane_u64((unsigned long long)__double_as_longlong(v), 1 << lj);
        v = fmax(v, __longlong_as_double((long long)u));
    }
    return v;
}

// Reduces the covariance partials (fixed order), finds the top two principal
// directions of the terms by subspace iteration with a final Rayleigh-Ritz
// rotation (fp64, one wave, lane t = term t; the iterate is broadcast through
// LDS), and stores the weights scaled by 1 - 2^-20 (so the fp32 weight
// vectors have norm < 1) with the sub-bin geometry: each direction's bins span
// +-2.5 standard deviations of its projections; points beyond clamp into the
// end bins.  Only quality depends on these choices: the search's windows are
// exact for any weights of norm <= 1.
__global__ __launch_bounds__(256) void refine_dirs_kernel(const double* __restrict__ part, int nblk,
                                                          double nsamp, RefineInfo* __restrict__ ri) {
    __shared__ double s_C[kMaxTerms][kMaxTerms + 1];
    __shared__ double s_v[2][kMaxTerms];
    const int tid = threadIdx.x;
    const int T = ri->terms;
    const int P = T * (T + 1) / 2;
    for (int p = tid; p < P; p += 256) {
        double sum = 0.0;
#pragma unroll 8
        for (int b = 0; b < nblk; ++b) sum += part[(size_t)b * kMaxPairs + p];
        int a, c;
        pair_of(p, T, a, c);
        sum /= nsamp;
        s_C[a][c] = sum;
        s_C[c][a] = sum;
    }
    __syncthreads();
    if (tid >= kWave) return;
    const int t = tid;
    const bool on = t < T;
    // both products C v0, C v1 from one LDS broadcast of the iterate
    auto matvec2 = [&](double& v0, double& v1) {
        if (on) {
            s_v[0][t] = v0;
            s_v[1][t] = v1;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        double w0 = 0.0, w1 = 0.0;
        for (int j = 0; j < T; ++j) {
            const double c = s_C[on ? t : 0][j];
            w0 = fma(c, s_v[0][j], w0);
            w1 = fma(c, s_v[1][j], w1);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        v0 = on ? w0 : 0.0;
        v1 = on ? w1 : 0.0;
    };
    // orthonormal (x0, x1) spanning what (x0, x1) span; degenerate inputs fall
    // back to coordinate directions
    auto orthonormalise = [&](double& x0, double& x1) {
        double n0 = sqrt(wave_sum_f64(x0 * x0));
        if (!(n0 > 1.0e-300 && n0 < 1.0e300)) {
            x0 = (t == 0) ? 1.0 : 0.0;
            n0 = 1.0;
        }
        x0 /= n0;
        x1 -= wave_sum_f64(x1 * x0) * x0;
        const double n1 = sqrt(wave_sum_f64(x1 * x1));
        if (!(n1 > 1.0e-300 && n1 > 1.0e-14 * n0 && n1 < 1.0e300)) {
            // e_k with k != argmax |x0| is never parallel to x0
            const double m = fabs(x0);
            const double mx = wave_max_f64(on ? m : -1.0);
            const int kmax = __ffsll((long long)__ballot(on && m == mx)) - 1;
            const int k = kmax == 0 ? 1 : 0;
            x1 = (t == k) ? 1.0 : 0.0;
            x1 -= wave_sum_f64(x1 * x0) * x0;
            x1 /= sqrt(wave_sum_f64(x1 * x1));
        } else {
            x1 /= n1;
        }
    };
    double u0, u1, l0, l1;
    if (T == 1) {
        u0 = (t == 0) ? 1.0 : 0.0;
        u1 = 0.0;
        l0 = s_C[0][0];
        l1 = 0.0;
    } else {
        double v0 = on ? (t == 0 ? 1.0 : 0.0625 * (double)((t * 7) % 5 - 2)) : 0.0;
        double v1 = on ? (t == 1 ? 1.0 : 0.0625 * (double)((t * 3) % 7 - 3)) : 0.0;
        orthonormalise(v0, v1);
        for (int it = 0; it < 24; ++it) {
            matvec2(v0, v1);
            orthonormalise(v0, v1);
        }
        double c0 = v0, c1 = v1;
        matvec2(c0, c1);
        const double a = wave_sum_f64(v0 * c0), b = wave_sum_f64(v0 * c1), c = wave_sum_f64(v1 * c1);
        const double th = 0.5 * atan2(2.0 * b, a - c);
        const double cs = cos(th), sn = sin(th);
        u0 = cs * v0 + sn * v1;
        u1 = cs * v1 - sn * v0;
        l0 = a * cs * cs + 2.0 * b * sn * cs + c * sn * sn;
        l1 = a * sn * sn - 2.0 * b * sn * cs + c * cs * cs;
    }
    constexpr double kShrink = 1.0 - 9.5367431640625e-07;   // 1 - 2^-20
    if (on) {
        ri->w0[t] = (float)(u0 * kShrink);
        ri->w1[t] = ri->L > 1 ? (float)(u1 * kShrink) : 0.0f;
    }
    if (t == 0) {
        const bool exact = ri->margin < 1.0e30f;
        float lo[2] = {0.0f, 0.0f}, inv[2] = {0.0f, 0.0f};
        const double lam[2] = {l0, l1};
        const int nb[2] = {ri->nb1, ri->nb2};
        for (int k = 0; k < ri->L; ++k) {
            const double sg = sqrt(fmax(lam[k], 0.0));
            const double iv = (double)nb[k] / (5.0 * sg);
            if (exact && sg > 0.0 && iv < 1.0e30) {
                lo[k] = (float)(-2.5 * sg);
                inv[k] = (float)iv;
            }
        }
        ri->lo0 = lo[0];
        ri->lo1 = lo[1];
        ri->inv0 = inv[0];
        ri->inv1 = inv[1];
    }
}

// Sub-bin key and counting inside big cells; the arrival slot in the sub-bin
// replaces the cell rank, and the key is kept for the reorder.
__global__ __launch_bounds__(256) void sub_count_kernel(const float* __restrict__ pts, int N,
                                                        const int* __restrict__ cell_of,
                                                        const int* __restrict__ cnt,
                                                        const int* __restrict__ bidx,
                                                        const RefineInfo* __restrict__ ref,
                                                        int* __restrict__ subcnt, int* __restrict__ rank,
                                                        int* __restrict__ subkey) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N) return;
    const int c = cell_of[i];
    if (cnt[c] < kBigCell) return;
    float s0, s1;
    refine_project(ref, [&](int d) { return pts[(size_t)d * N + i]; }, s0, s1);
    const int q1 = sub_bin(s0, ref->lo0, ref->inv0, ref->nb1);
    const int q2 = ref->L > 1 ? sub_bin(s1, ref->lo1, ref->inv1, ref->nb2) : 0;
    const int key = q1 * ref->nb2 + q2;
    subkey[i] = key;
    rank[i] = atomicAdd(&subcnt[(size_t)bidx[c] * kSubBins + key], 1);
}

__global__ __launch_bounds__(256) void transpose_kernel(const float* __restrict__ pts, int N, int D, int ds,
                                                        float* __restrict__ aos,
                                                        const DimStat* __restrict__ st,
                                                        float* __restrict__ frows,
                                                        float* __restrict__ fnorm) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N) return;
    write_rows(pts, N, D, ds, i, i, aos, st, frows, fnorm);
}

// Output transpose through LDS, 32 original queries per workgroup: the K keys
// of each query's list (row inv[i] of the sorted order) are read with
// consecutive threads on consecutive keys, then each k writes the 32 queries'
// index and distance as one contiguous 128-byte segment of the SoA outputs.
constexpr int kUnpermQ = 32;
__global__ __launch_bounds__(256) void unpermute_kernel(const unsigned long long* __restrict__ lists,
                                                        int cap, const int* __restrict__ inv, int N,
                                                        int K, int* __restrict__ idxs,
                                                        float* __restrict__ dists) {
    __shared__ unsigned long long s_t[kUnpermQ * (FRNN_MAX_K + 1)];
    const int i0 = blockIdx.x * kUnpermQ;
    const int nq = min(kUnpermQ, N - i0);
    const int stride = K + 1;
    for (int j = threadIdx.x; j < nq * K; j += blockDim.x) {
        const int q = j / K;
        const int k = j - q * K;
        const int sp = inv ? inv[i0 + q] : i0 + q;
        s_t[q * stride + k] = lists[(size_t)sp * cap + k];
    }
    __syncthreads();
    for (int j = threadIdx.x; j < K * kUnpermQ; j += blockDim.x) {
        const int k = j / kUnpermQ;
        const int q = j - k * kUnpermQ;
        if (q < nq) {
            const unsigned long long key = s_t[q * stride + k];
            idxs[(size_t)k * N + i0 + q] = (int)(unsigned int)key;
            dists[(size_t)k * N + i0 + q] = key_d2(key);
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
    long long nb = (n + 255) / 256;
    if (nb > 65536) nb = 65536;
    hipLaunchKernelGGL(fill_i32_kernel, dim3((unsigned)nb), dim3(256), 0, s, p, n, v);
    return launch_result();
}

int launch_bin_count(const float* pts, int N, int g, int res, float inv_cell, int* cell_of, int* rank,
                     int* cnt, hipStream_t s) {
    if (N <= 0) return 0;
    hipLaunchKernelGGL(bin_count_kernel, dim3(blocks_for(N, 256)), dim3(256), 0, s, pts, N, g, res,
                       inv_cell, cell_of, rank, cnt);
    return launch_result();
}

int scan_partials_count(int n) { return (n + kScanTile - 1) / kScanTile + 1; }

int launch_exclusive_scan(const int* in, int n, int* out, int* partials, hipStream_t s, int flag_min) {
    if (n <= 0) return 0;
    const int nb = (n + kScanTile - 1) / kScanTile;
    if (nb > kScanTile) return 2;
    hipLaunchKernelGGL(scan_reduce_kernel, dim3(nb), dim3(kScanThreads), 0, s, in, n, partials, flag_min);
    hipLaunchKernelGGL(scan_partials_kernel, dim3(1), dim3(kScanThreads), 0, s, partials, nb);
    hipLaunchKernelGGL(scan_final_kernel, dim3(nb), dim3(kScanThreads), 0, s, in, n, partials, out, flag_min);
    return launch_result();
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

RefineLayout refine_layout(int N, int D, long long cells) {
    RefineLayout L{};
    L.max_big = N / kBigCell;
    L.nsub = L.max_big * kSubBins + 1;
    size_t off = 0;
    L.info = off;     off = align256(off + sizeof(RefineInfo));
    L.bidx = off;     off = align256(off + (size_t)(cells + 1) * sizeof(int));
    L.subcnt = off;   off = align256(off + (size_t)L.nsub * sizeof(int));
    L.substart = off; off = align256(off + (size_t)L.nsub * sizeof(int));
    const int np = scan_partials_count(L.nsub > cells + 1 ? L.nsub : (int)(cells + 1));
    L.scanpart = off; off = align256(off + (size_t)np * sizeof(int));
    L.cov = off;      off = align256(off + (size_t)kCovBlocks * kMaxPairs * sizeof(double));
    L.subkey = off;   off = align256(off + (size_t)N * sizeof(int));
    L.total = off;
    (void)D;
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

int launch_refine(const float* pts, int N, int D, int g, long long cells, const int* cell_of, const int* cnt,
                  int* rank, const void* stats_ws, void* ws, hipStream_t s) {
    if (N <= 0 || D <= g) return 0;
    const RefineLayout L = refine_layout(N, D, cells);
    char* base = static_cast<char*>(ws);
    RefineInfo* info = reinterpret_cast<RefineInfo*>(base + L.info);
    int* bidx = reinterpret_cast<int*>(base + L.bidx);
    int* subcnt = reinterpret_cast<int*>(base + L.subcnt);
    int* substart = reinterpret_cast<int*>(base + L.substart);
    int* scanpart = reinterpret_cast<int*>(base + L.scanpart);
    const DimStat* st = reinterpret_cast<const DimStat*>(static_cast<const char*>(stats_ws) + stats_layout(D).dims);
    double* cov = reinterpret_cast<double*>(base + L.cov);
    int* subkey = reinterpret_cast<int*>(base + L.subkey);
    hipLaunchKernelGGL(refine_terms_kernel, dim3(1), dim3(64), 0, s, st, g, D, info);
    // covariance sample: kCovBlocks tiles of 256 consecutive points, evenly spaced
    const long long tile_stride = N <= (long long)kCovBlocks * 256 ? 256 : (long long)N / kCovBlocks;
    long long nsamp = 0;
    for (int b = 0; b < kCovBlocks; ++b) {
        const long long i0 = (long long)b * tile_stride;
        nsamp += i0 < N ? (N - i0 < 256 ? N - i0 : 256) : 0;
    }
    hipLaunchKernelGGL(cov_kernel, dim3(kCovBlocks), dim3(256), 0, s, pts, N, tile_stride, info, cov);
    hipLaunchKernelGGL(refine_dirs_kernel, dim3(1), dim3(256), 0, s, cov, kCovBlocks, (double)nsamp, info);
    int rc = launch_exclusive_scan(cnt, (int)cells + 1, bidx, scanpart, s, kBigCell);
    if (rc) return rc;
    rc = launch_fill_i32(subcnt, L.nsub, 0, s);
    if (rc) return rc;
    hipLaunchKernelGGL(sub_count_kernel, dim3(blocks_for(N, 256)), dim3(256), 0, s, pts, N, cell_of, cnt,
                       bidx, info, subcnt, rank, subkey);
    rc = launch_exclusive_scan(subcnt, L.nsub, substart, scanpart, s);
    if (rc) return rc;
    return launch_result();
}

int launch_reorder(const float* pts, int N, int D, const int* cell_of, const int* rank, const int* start,
                   const int* cnt, const void* refine_ws, long long cells, int* sorted_idx, int* inv,
                   float* aos, const void* stats_ws, float* frows, float* fnorm, hipStream_t s) {
    if (N <= 0) return 0;
    const int* subkey = nullptr;
    const int* bidx = nullptr;
    const int* substart = nullptr;
    if (refine_ws) {
        const RefineLayout L = refine_layout(N, D, cells);
        const char* base = static_cast<const char*>(refine_ws);
        subkey = reinterpret_cast<const int*>(base + L.subkey);
        bidx = reinterpret_cast<const int*>(base + L.bidx);
        substart = reinterpret_cast<const int*>(base + L.substart);
    }
    const DimStat* st = stats_ws ? reinterpret_cast<const DimStat*>(static_cast<const char*>(stats_ws) +
                                                                    stats_layout(D).dims)
                                 : nullptr;
    if (!st) frows = nullptr;
    hipLaunchKernelGGL(reorder_kernel, dim3(blocks_for(N, 256)), dim3(256), 0, s, pts, N, D,
                       aos_stride(D), cell_of, rank, start, cnt, subkey, bidx, substart, sorted_idx, inv, aos,
                       st, frows, fnorm);
    return launch_result();
}

int launch_transpose(const float* pts, int N, int D, float* aos, const void* stats_ws, float* frows,
                     float* fnorm, hipStream_t s) {
    if (N <= 0) return 0;
    const DimStat* st = stats_ws ? reinterpret_cast<const DimStat*>(static_cast<const char*>(stats_ws) +
                                                                    stats_layout(D).dims)
                                 : nullptr;
    if (!st) frows = nullptr;
    hipLaunchKernelGGL(transpose_kernel, dim3(blocks_for(N, 256)), dim3(256), 0, s, pts, N, D,
                       aos_stride(D), aos, st, frows, fnorm);
    return launch_result();
}

int launch_unpermute(const unsigned long long* lists, int cap, const int* inv, int N, int K, int* idxs,
                     float* dists, hipStream_t s) {
    if (N <= 0) return 0;
    if (K < 1 || K > FRNN_MAX_K || cap < K) return 1;   // the LDS tile holds K <= FRNN_MAX_K keys
    hipLaunchKernelGGL(unpermute_kernel, dim3(blocks_for(N, kUnpermQ)), dim3(256), 0, s, lists, cap, inv, N,
                       K, idxs, dists);
    return launch_result();
}

}  // namespace frnn
