// frnn_internal.hpp -- host-side declarations shared by the engine and the kernel files.
#pragma once

#include <hip/hip_runtime.h>

#include "frnn_mi355x.h"

namespace frnn {

// Padded AoS row length (floats).  It is also the dimension the MFMA search is
// instantiated for; padding coordinates are zero in every row, which leaves
// both the MFMA dot products and the exact fp32 distances unchanged.
__host__ __device__ inline int aos_stride(int D) {
    return D <= 4 ? 4 : D <= 8 ? 8 : D <= 12 ? 12 : D <= 16 ? 16 : D <= 32 ? 32 : D <= 64 ? 64 : 128;
}

// Per-query candidate list entries: K kept after a compaction plus room for a
// full 64-entry recheck batch and K more arrivals between compactions.
inline int list_capacity(int K) { return 2 * K + 64; }

int scan_partials_count(int n);

// Launchers return 0, 1 (bad argument), 2 (size limit) or 3 (HIP launch error;
// the error code is kept for last_launch_error()).
int launch_result();
hipError_t last_launch_error();

int launch_fill_i32(int* p, long long n, int v, hipStream_t s);
int launch_bin_count(const float* pts, int N, int g, int res, float inv_cell, int* cell_of, int* rank,
                     int* cnt, hipStream_t s);
int launch_exclusive_scan(const int* in, int n, int* out, int* partials, hipStream_t s);
int launch_reorder(const float* pts, int N, int D, const int* cell_of, const int* rank, const int* start,
                   int* sorted_idx, int* inv, float* aos, hipStream_t s);
int launch_transpose(const float* pts, int N, int D, float* aos, hipStream_t s);
int launch_unpermute(const unsigned long long* lists, int cap, const int* inv, int N, int K, int* idxs,
                     float* dists, hipStream_t s);
int launch_search(const float* aos, const int* sorted_idx, const int* start, int N, int D, int K,
                  const frnn_plan_t& plan, unsigned long long* lists, int cap,
                  unsigned long long* counters, hipStream_t s);

}  // namespace frnn
