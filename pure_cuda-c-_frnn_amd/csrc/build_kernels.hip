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

__global__ __launch_bounds__(kScanThreads) void scan_reduce_kernel(const int* __restrict__ in, int n,
                                                                   int* __restrict__ partials) {
    __shared__ int s_tmp[kScanThreads];
    const long long base = (long long)blockIdx.x * kScanTile + (long long)threadIdx.x * kScanItems;
    int sum = 0;
#pragma unroll
    for (int j = 0; j < kScanItems; ++j) {
        long long idx = base + j;
        sum += (idx < n) ? in[idx] : 0;
    }
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
                                                                  int* __restrict__ out) {
    __shared__ int s_tmp[kScanThreads];
    const long long base = (long long)blockIdx.x * kScanTile + (long long)threadIdx.x * kScanItems;
    int v[kScanItems];
    int sum = 0;
#pragma unroll
    for (int j = 0; j < kScanItems; ++j) {
        long long idx = base + j;
        v[j] = (idx < n) ? in[idx] : 0;
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

// One thread per point: SoA reads are coalesced per axis; the AoS row store
// is ds/4 16-byte vector stores to one contiguous row.
__global__ __launch_bounds__(256) void reorder_kernel(const float* __restrict__ pts, int N, int D, int ds,
                                                      const int* __restrict__ cell_of,
                                                      const int* __restrict__ rank,
                                                      const int* __restrict__ start,
                                                      int* __restrict__ sorted_idx,
                                                      int* __restrict__ inv,
                                                      float* __restrict__ aos) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N) return;
    const int pos = start[cell_of[i]] + rank[i];
    sorted_idx[pos] = i;
    inv[i] = pos;
    float4* row = reinterpret_cast<float4*>(aos + (size_t)pos * ds);
    for (int d = 0; d < ds; d += 4) {
        float4 v;
        v.x = (d + 0 < D) ? pts[(size_t)(d + 0) * N + i] : 0.0f;
        v.y = (d + 1 < D) ? pts[(size_t)(d + 1) * N + i] : 0.0f;
        v.z = (d + 2 < D) ? pts[(size_t)(d + 2) * N + i] : 0.0f;
        v.w = (d + 3 < D) ? pts[(size_t)(d + 3) * N + i] : 0.0f;
        row[d >> 2] = v;
    }
}

__global__ __launch_bounds__(256) void transpose_kernel(const float* __restrict__ pts, int N, int D, int ds,
                                                        float* __restrict__ aos) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N) return;
    float4* row = reinterpret_cast<float4*>(aos + (size_t)i * ds);
    for (int d = 0; d < ds; d += 4) {
        float4 v;
        v.x = (d + 0 < D) ? pts[(size_t)(d + 0) * N + i] : 0.0f;
        v.y = (d + 1 < D) ? pts[(size_t)(d + 1) * N + i] : 0.0f;
        v.z = (d + 2 < D) ? pts[(size_t)(d + 2) * N + i] : 0.0f;
        v.w = (d + 3 < D) ? pts[(size_t)(d + 3) * N + i] : 0.0f;
        row[d >> 2] = v;
    }
}

// One thread per original query: reads its K sorted keys (contiguous, 16-byte
// loads) and writes the SoA outputs, coalesced across the wave for each k.
__global__ __launch_bounds__(256) void unpermute_kernel(const unsigned long long* __restrict__ lists,
                                                        int cap, const int* __restrict__ inv, int N,
                                                        int K, int* __restrict__ idxs,
                                                        float* __restrict__ dists) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N) return;
    const int sp = inv ? inv[i] : i;
    const unsigned long long* L = lists + (size_t)sp * cap;
    for (int k = 0; k < K; ++k) {
        const unsigned long long key = L[k];
        idxs[(size_t)k * N + i] = (int)(unsigned int)key;
        dists[(size_t)k * N + i] = key_d2(key);
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

int launch_exclusive_scan(const int* in, int n, int* out, int* partials, hipStream_t s) {
    if (n <= 0) return 0;
    const int nb = (n + kScanTile - 1) / kScanTile;
    if (nb > kScanTile) return 2;
    hipLaunchKernelGGL(scan_reduce_kernel, dim3(nb), dim3(kScanThreads), 0, s, in, n, partials);
    hipLaunchKernelGGL(scan_partials_kernel, dim3(1), dim3(kScanThreads), 0, s, partials, nb);
    hipLaunchKernelGGL(scan_final_kernel, dim3(nb), dim3(kScanThreads), 0, s, in, n, partials, out);
    return launch_result();
}

int launch_reorder(const float* pts, int N, int D, const int* cell_of, const int* rank, const int* start,
                   int* sorted_idx, int* inv, float* aos, hipStream_t s) {
    if (N <= 0) return 0;
    hipLaunchKernelGGL(reorder_kernel, dim3(blocks_for(N, 256)), dim3(256), 0, s, pts, N, D,
                       aos_stride(D), cell_of, rank, start, sorted_idx, inv, aos);
    return launch_result();
}

int launch_transpose(const float* pts, int N, int D, float* aos, hipStream_t s) {
    if (N <= 0) return 0;
    hipLaunchKernelGGL(transpose_kernel, dim3(blocks_for(N, 256)), dim3(256), 0, s, pts, N, D,
                       aos_stride(D), aos);
    return launch_result();
}

int launch_unpermute(const unsigned long long* lists, int cap, const int* inv, int N, int K, int* idxs,
                     float* dists, hipStream_t s) {
    if (N <= 0) return 0;
    hipLaunchKernelGGL(unpermute_kernel, dim3(blocks_for(N, 256)), dim3(256), 0, s, lists, cap, inv, N,
                       K, idxs, dists);
    return launch_result();
}

}  // namespace frnn
