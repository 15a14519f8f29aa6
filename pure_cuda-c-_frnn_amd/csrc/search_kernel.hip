// search_kernel.hip -- all-points fixed-radius K-nearest search for gfx950.
//
// One kernel serves every path of the reference dispatch:
//   full-D grid        FindNbrsNDKernel / FindNbrsAoS3Kernel (find_nbrs.cu:116-214, 400-491)
//   first-coord grid   FindNbrsGridDimKernel               (find_nbrs.cu:243-353)
//   brute force        TiledBruteforce{ND,16}Kernel        (no_grid_frnn.cu:121-257)
//
// Work decomposition (one 64-lane wave per workgroup):
//   * a wave owns 32 consecutive queries of the cell-sorted order (grid paths)
//     or of the original order (brute force);
//   * for grid paths the wave walks, for each run of its queries' rows, the
//     3^(g-1) neighbouring rows; in each neighbouring row the cells x-1..x+1 of
//     one query are a contiguous span of the sorted points, so the union over
//     the wave is one contiguous candidate range per neighbouring row.  Each
//     query only accepts candidates inside its own 3^g shell ([lo, hi) per row),
//     with conservative AABB trimming of the outer x cells;
//   * candidates stream through in tiles of 32.  The distance tile
//     32 candidates x 32 queries is one chain of v_mfma_f32_32x32x2f32 on the
//     augmented vectors  a = [-2p', (1-c)|p'|^2, 1],  b = [q', 1, (1-c)|q'|^2]
//     (p', q' centred on the first query of the wave), so the accumulator is a
//     filter value F <= the exact distance plus a proven rounding bound;
//   * pairs with F below the query's threshold (plus a relative margin) are
//     queued in LDS and re-evaluated 64 at a time with the reference's exact fp32
//     distance order; accepted (d2, idx) keys go to a per-query candidate list;
//   * when a list nears capacity the wave sorts it cooperatively (bitonic in
//     LDS), keeps the K smallest and tightens the query's threshold to the K-th
//     key; at the end every list is sorted and its first K keys (plus padding)
//     are the result for that sorted position.
//
// Exactness: a pair is returned iff its exact fp32 distance in the reference
// order is < r2 and it is among the K smallest (d2, idx) keys.  The MFMA value
// only decides which pairs are re-evaluated; its margin (norm_scale, thr_rel,
// thr_abs, set on the host) covers the rounding of the centring, the norms, the
// fp32 MFMA accumulation (with a factor 2 on the unit roundoff) and the exact
// order, so no pair that could qualify is dropped.  NaN or overflowed filter
// values are always re-evaluated.
#include "frnn_device.hpp"
#include "frnn_internal.hpp"

namespace frnn {

constexpr int kQB = 32;                      // queries per wave
constexpr int kBatch = 64;                   // exact re-evaluations per batch
constexpr int kQueueCap = kBatch + kQB * 32; // leftover batch + one full tile of hits
constexpr int kSortCap = 512;                // >= next_pow2(list_capacity(128))

struct SearchArgs {
    const float* pts;            // AoS rows, stride DS (sorted order for grids)
    const int* sorted_idx;       // sorted position -> original index (grid paths)
    const int* start;            // cells+1 exclusive cell offsets (grid paths)
    unsigned long long* lists;   // [N][cap] candidate keys
    unsigned long long* counters;
    int N, K, cap, G, res;
    float r2, cell, inv_cell;
    float norm_scale;            // 1 - c_norm
    float thr_rel, thr_abs;      // filter threshold margin
    int nchunks, chunks_per_xcd;
};

__device__ __forceinline__ float filter_threshold(float thr, const SearchArgs& a) {
    return fmaf(thr, a.thr_rel, thr) + a.thr_abs;
}

// Lower bound of |q - x| over points x binned into cell c of one axis.  The
// 2^-21 relative shrink covers the rounding of the binning product, of c*cell
// and of the subtraction; edge cells are unbounded outward because binning
// clamps.
__device__ __forceinline__ float axis_gap(float q, int c, int res, float cell) {
    const float eps = 4.76837158203125e-07f;
    float g = 0.0f;
    if (c > 0) {
        const float lo = (float)c * cell;
        float t = lo - q;
        t -= eps * (fabsf(lo) + fabsf(q));
        g = fmaxf(g, t);
    }
    if (c < res - 1) {
        const float hi = (float)(c + 1) * cell;
        float t = q - hi;
        t -= eps * (fabsf(hi) + fabsf(q));
        g = fmaxf(g, t);
    }
    return g;
}

// Exact fp32 squared distance in the reference's order: sequential
// fmaf(diff, diff, d2) over d = 0..D-1 (find_nbrs.cu:194-199, 335-340), or the
// D=3 grid order fmaf(dx,dx,fmaf(dy,dy,dz*dz)) as the reversed sequence
// (find_nbrs.cu:474-477).  Zero padding dims leave the value unchanged.
template <int DS, bool REV>
__device__ __forceinline__ float exact_d2(const float* q, const float* __restrict__ p) {
    float acc = 0.0f;
    if constexpr (REV) {
        float pv[DS];
#pragma unroll
        for (int d = 0; d < DS; d += 4) {
            const float4 v = *reinterpret_cast<const float4*>(p + d);
            pv[d] = v.x; pv[d + 1] = v.y; pv[d + 2] = v.z; pv[d + 3] = v.w;
        }
#pragma unroll
        for (int d = DS - 1; d >= 0; --d) {
            const float diff = q[d] - pv[d];
            acc = fmaf(diff, diff, acc);
        }
    } else {
#pragma unroll
        for (int d = 0; d < DS; d += 4) {
            const float4 v = *reinterpret_cast<const float4*>(p + d);
            float diff = q[d] - v.x;
            acc = fmaf(diff, diff, acc);
            diff = q[d + 1] - v.y;
            acc = fmaf(diff, diff, acc);
            diff = q[d + 2] - v.z;
            acc = fmaf(diff, diff, acc);
            diff = q[d + 3] - v.w;
            acc = fmaf(diff, diff, acc);
        }
    }
    return acc;
}

template <int DS, bool REV, bool BF>
__global__ __launch_bounds__(64) void search_kernel(SearchArgs a) {
    constexpr int HD = DS / 2;
    __shared__ __align__(16) float s_q[kQB * DS];
    __shared__ float s_o[DS];
    __shared__ int s_cnt[kQB];
    __shared__ unsigned long long s_thr[kQB];
    __shared__ int s_qn[kQueueCap];
    __shared__ int s_qpos[kQueueCap];
    __shared__ unsigned long long s_sort[kSortCap];
    __shared__ int s_qsize;

    const int lane = threadIdx.x;
    const int n = lane & 31;
    const int h = lane >> 5;
    // The dispatcher places workgroup b on XCD b % 8; give each XCD a
    // contiguous range of chunks so neighbouring queries share its L2.
    const int b = blockIdx.x;
    const int chunk = (b & 7) * a.chunks_per_xcd + (b >> 3);
    if (chunk >= a.nchunks) return;
    const int q0 = chunk * kQB;
    const int nq = min(kQB, a.N - q0);
    const bool qvalid = n < nq;
    unsigned long long* const lists = a.lists + (size_t)q0 * a.cap;

    {
        const float* src = a.pts + (size_t)(q0 + (qvalid ? n : 0)) * DS + h * HD;
        float* dst = s_q + n * DS + h * HD;
#pragma unroll
        for (int j = 0; j < HD; j += 2) {
            float2 v = *reinterpret_cast<const float2*>(src + j);
            if (!qvalid) v = make_float2(0.0f, 0.0f);
            dst[j] = v.x;
            dst[j + 1] = v.y;
        }
    }
    if (lane < kQB) {
        s_cnt[lane] = 0;
        s_thr[lane] = make_key(a.r2, 0);
    }
    if (lane == 0) s_qsize = 0;
    __syncthreads();
    for (int d = lane; d < DS; d += kWave) s_o[d] = BF ? 0.0f : s_q[d];
    __syncthreads();

    // B operand: this lane's half of query n, centred, plus the norm column.
    float bop[HD + 1];
    float qn2p = 0.0f;
#pragma unroll
    for (int j = 0; j < HD; ++j) {
        const float v = s_q[n * DS + h * HD + j] - s_o[h * HD + j];
        bop[j] = v;
        qn2p = fmaf(v, v, qn2p);
    }
    const float qn2 = qn2p + __shfl_xor(qn2p, 32);
    bop[HD] = (h == 0) ? 1.0f : qn2 * a.norm_scale;
    if (!qvalid) {
#pragma unroll
        for (int j = 0; j <= HD; ++j) bop[j] = 0.0f;
    }
    float thr_f = qvalid ? filter_threshold(a.r2, a) : -__builtin_huge_valf();

    long long c_shell = 0, c_hit = 0, c_acc = 0, c_ovf = 0;

    auto select_topk = [&](int qn, bool final_pass) {
        const int c = s_cnt[qn];
        int P = kWave;
        while (P < c) P <<= 1;
        unsigned long long* L = lists + (size_t)qn * a.cap;
        for (int i = lane; i < P; i += kWave) s_sort[i] = (i < c) ? L[i] : ~0ull;
        __syncthreads();
        for (int k = 2; k <= P; k <<= 1) {
            for (int j = k >> 1; j > 0; j >>= 1) {
                for (int i = lane; i < P; i += kWave) {
                    const int ixj = i ^ j;
                    if (ixj > i) {
                        const unsigned long long x = s_sort[i];
                        const unsigned long long y = s_sort[ixj];
                        const bool up = (i & k) == 0;
                        if ((x > y) == up) {
                            s_sort[i] = y;
                            s_sort[ixj] = x;
                        }
                    }
                }
                __syncthreads();
            }
        }
        if (final_pass) {
            const unsigned long long pad = make_key(a.r2, -1);
            for (int k = lane; k < a.K; k += kWave) L[k] = (k < c) ? s_sort[k] : pad;
        } else {
            const int keep = min(c, a.K);
            for (int k = lane; k < keep; k += kWave) L[k] = s_sort[k];
            if (lane == 0) {
                s_cnt[qn] = keep;
                if (c >= a.K) s_thr[qn] = s_sort[a.K - 1];
            }
        }
        __syncthreads();
    };

    auto process_batch = [&](int base, int count) {
        // make room for a full batch in every list
        const bool need = (lane < kQB) && (s_cnt[lane] > a.cap - kBatch);
        unsigned long long m = __ballot(need);
        if (m) {
            while (m) {
                const int qn = __ffsll((long long)m) - 1;
                m &= m - 1;
                select_topk(qn, false);
            }
            if (qvalid) thr_f = filter_threshold(key_d2(s_thr[n]), a);
        }
        if (lane < count) {
            const int qn = s_qn[base + lane];
            const int pos = s_qpos[base + lane];
            const float e = exact_d2<DS, REV>(s_q + qn * DS, a.pts + (size_t)pos * DS);
            const int idx = BF ? pos : a.sorted_idx[pos];
            const unsigned long long key = make_key(e, idx);
            if (key < s_thr[qn]) {
                const int slot = atomicAdd(&s_cnt[qn], 1);
                // compaction above leaves >= kBatch free slots; the guard only
                // keeps a logic error from writing past the list
                if (slot < a.cap) lists[(size_t)qn * a.cap + slot] = key;
                else ++c_ovf;
                ++c_acc;
            }
        }
        __syncthreads();
        if (lane == 0) s_qsize = base;
        __syncthreads();
    };

    auto process_run = [&](int A, int B, int lo, int hi) {
        for (int t0 = A; t0 < B; t0 += 32) {
            const int m = t0 + n;
            const bool mvalid = m < B;
            const float* src = a.pts + (size_t)(mvalid ? m : A) * DS + h * HD;
            float aop[HD + 1];
            float pn2p = 0.0f;
#pragma unroll
            for (int j = 0; j < HD; j += 2) {
                const float2 v = *reinterpret_cast<const float2*>(src + j);
                const float d0 = v.x - s_o[h * HD + j];
                const float d1 = v.y - s_o[h * HD + j + 1];
                aop[j] = -2.0f * d0;
                aop[j + 1] = -2.0f * d1;
                pn2p = fmaf(d0, d0, pn2p);
                pn2p = fmaf(d1, d1, pn2p);
            }
            const float pn2 = pn2p + __shfl_xor(pn2p, 32);
            aop[HD] = (h == 0) ? (mvalid ? pn2 * a.norm_scale : 3.0e38f) : 1.0f;

            floatx16 acc;
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
#pragma unroll
            for (int j = 0; j <= HD; ++j)
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(aop[j], bop[j], acc, 0, 0, 0);

            bool any = false;
#pragma unroll
            for (int r = 0; r < 16; ++r) any |= !(acc[r] >= thr_f);
            if (__ballot(any)) {
                if (any) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        if (!(acc[r] >= thr_f)) {
                            // 32x32 accumulator layout: lane (n, h), register r holds
                            // row 8*(r/4) + 4*h + r%4 (the candidate) of column n.
                            const int pos = t0 + 8 * (r >> 2) + 4 * h + (r & 3);
                            if (pos >= lo && pos < hi) {
                                const int s = atomicAdd(&s_qsize, 1);
                                if (s < kQueueCap) {
                                    s_qn[s] = n;
                                    s_qpos[s] = pos;
                                } else {
                                    ++c_ovf;
                                }
                                ++c_hit;
                            }
                        }
                    }
                }
                __syncthreads();
                int qs = min(s_qsize, kQueueCap);
                while (qs >= kBatch) {
                    process_batch(qs - kBatch, kBatch);
                    qs -= kBatch;
                }
            }
        }
    };

    if constexpr (BF) {
        if (qvalid && h == 0) c_shell += a.N;
        process_run(0, a.N, 0, qvalid ? a.N : 0);
    } else {
        const float* qrow = s_q + n * DS;
        int x_n = bin_coord(qrow[0], a.inv_cell, a.res);
        int row_n = 0;
        {
            int mul = 1;
            for (int d = 1; d < a.G; ++d) {
                row_n += bin_coord(qrow[d], a.inv_cell, a.res) * mul;
                mul *= a.res;
            }
        }
        if (!qvalid) row_n = 0x7fffffff;
        int nrows = 1;
        for (int d = 1; d < a.G; ++d) nrows *= 3;
        const float keep = 0.9999847412109375f;   // 1 - 2^-16

        int seg = 0;
        while (seg < nq) {
            const int R = __shfl(row_n, seg);
            const bool in_seg = (row_n == R);
            const int xlo = wave_min_i32(in_seg ? x_n : 0x7fffffff);
            const int xhi = wave_max_i32(in_seg ? x_n : -1);
            const int seg_end = __popcll(__ballot(row_n <= R) & 0xffffffffull);

            for (int t = 0; t < nrows; ++t) {
                int tt = t, Rt = R, Rn = 0, mul = 1;
                bool ok = true;
                float lbr = 0.0f;
                for (int d = 1; d < a.G; ++d) {
                    const int rc = Rt % a.res;
                    Rt /= a.res;
                    const int cc = rc + (tt % 3) - 1;
                    tt /= 3;
                    ok = ok && cc >= 0 && cc < a.res;
                    Rn += cc * mul;
                    mul *= a.res;
                    const float gd = axis_gap(qrow[d], cc, a.res, a.cell);
                    lbr = fmaf(gd, gd, lbr);
                }
                if (!ok) continue;
                const int base = Rn * a.res;
                const int A = a.start[base + max(xlo - 1, 0)];
                const int B = a.start[base + min(xhi + 1, a.res - 1) + 1];
                if (A >= B) continue;

                int lo = 0, hi = 0;
                if (in_seg) {
                    const int xl = max(x_n - 1, 0);
                    const int xh = min(x_n + 1, a.res - 1);
                    lo = a.start[base + xl];
                    hi = a.start[base + xh + 1];
                    if (h == 0) c_shell += hi - lo;
                    const float thrE = key_d2(s_thr[n]);
                    if (lbr * keep > thrE) {
                        lo = hi;
                    } else {
                        if (xl < x_n) {
                            const float gx = axis_gap(qrow[0], xl, a.res, a.cell);
                            if (fmaf(gx, gx, lbr) * keep > thrE) lo = a.start[base + x_n];
                        }
                        if (xh > x_n) {
                            const float gx = axis_gap(qrow[0], xh, a.res, a.cell);
                            if (fmaf(gx, gx, lbr) * keep > thrE) hi = a.start[base + x_n + 1];
                        }
                    }
                }
                const int wlo = wave_min_i32(lo < hi ? lo : 0x7fffffff);
                const int whi = wave_max_i32(lo < hi ? hi : -1);
                if (wlo >= whi) continue;
                process_run(wlo, whi, lo, hi);
            }
            seg = seg_end;
        }
    }

    __syncthreads();
    {
        const int qs = s_qsize;
        if (qs > 0) process_batch(0, qs);
    }
    for (int qn = 0; qn < nq; ++qn) select_topk(qn, true);

    if (a.counters) {
        const long long s0 = wave_sum_i64(c_shell);
        const long long s1 = wave_sum_i64(c_hit);
        const long long s2 = wave_sum_i64(c_acc);
        const long long s3 = wave_sum_i64(c_ovf);
        if (lane == 0) {
            atomicAdd(&a.counters[0], (unsigned long long)s0);
            atomicAdd(&a.counters[1], (unsigned long long)s1);
            atomicAdd(&a.counters[2], (unsigned long long)s2);
            if (s3) atomicAdd(&a.counters[3], (unsigned long long)s3);
        }
    }
}

template <int DS, bool REV, bool BF>
static void launch_one(const SearchArgs& a, hipStream_t s) {
    hipLaunchKernelGGL((search_kernel<DS, REV, BF>), dim3(8 * a.chunks_per_xcd), dim3(kWave), 0, s, a);
}

template <int DS>
static void launch_ds(const SearchArgs& a, bool bf, hipStream_t s) {
    if (bf) launch_one<DS, false, true>(a, s);
    else launch_one<DS, false, false>(a, s);
}

int launch_search(const float* aos, const int* sorted_idx, const int* start, int N, int D, int K,
                  const frnn_plan_t& plan, unsigned long long* lists, int cap,
                  unsigned long long* counters, hipStream_t s) {
    if (N <= 0) return 0;
    const bool bf = plan.path == FRNN_PATH_BRUTEFORCE;
    if (!bf && (plan.grid_dim < 1 || plan.grid_dim > 9)) return 1;
    if (cap < list_capacity(K) || K > FRNN_MAX_K) return 1;
    SearchArgs a{};
    a.pts = aos;
    a.sorted_idx = sorted_idx;
    a.start = start;
    a.lists = lists;
    a.counters = counters;
    a.N = N;
    a.K = K;
    a.cap = cap;
    a.G = bf ? 0 : plan.grid_dim;
    a.res = bf ? 1 : plan.res;
    a.r2 = plan.r2;
    a.inv_cell = plan.inv_cell;
    const int DS = aos_stride(D);
    a.cell = bf ? 1.0f : plan.cell_size;
    const double u = 5.9604644775390625e-08;   // 2^-24
    a.norm_scale = (float)(1.0 - (6.0 * DS + 32.0) * u);
    a.thr_rel = (float)(2.0 * (DS + 8.0) * u);
    a.thr_abs = 1.0e-35f;
    a.nchunks = (N + kQB - 1) / kQB;
    a.chunks_per_xcd = (a.nchunks + 7) / 8;
    if (plan.rev_order && !bf && DS == 4) {
        launch_one<4, true, false>(a, s);
    } else {
        switch (DS) {
            case 4: launch_ds<4>(a, bf, s); break;
            case 8: launch_ds<8>(a, bf, s); break;
            case 12: launch_ds<12>(a, bf, s); break;
            case 16: launch_ds<16>(a, bf, s); break;
            case 32: launch_ds<32>(a, bf, s); break;
            case 64: launch_ds<64>(a, bf, s); break;
            case 128: launch_ds<128>(a, bf, s); break;
            default: return 1;
        }
    }
    return launch_result();
}

}  // namespace frnn
