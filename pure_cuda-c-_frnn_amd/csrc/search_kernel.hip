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
//   * for grid paths the wave walks, for each run of its queries sharing a
//     row (the cells of equal coordinates on axes 1..g-1), the 3^(g-1)
//     neighbouring rows, skipping rows whose box is farther than every
//     query's threshold; in each row it streams, on a frame's fine axis 0,
//     the one stretch of cells that the run's threshold can still reach
//     (grids without a frame, above 4 axes: the cells x-1..x+1 around the
//     run's queries);
//   * candidates stream through in tiles of 32.  The distance tile
//     32 candidates x 32 queries is one chain of v_mfma_f32_32x32x2f32 on the
//     augmented vectors  a = [p', |p'|^2, 1],  b = [-2q', 1-c, (1-c)|q'|^2]
//     (p', q' the rows centred on the input mean as they are loaded, with
//     their squared norms), so the accumulator is a filter value F <= the
//     exact distance plus a proven rounding bound;
//   * pairs with F below the query's threshold (plus a relative margin) are
//     re-evaluated with the reference's exact fp32 distance order: right after
//     the tile from its raw rows staged in LDS (rows up to 32 floats), or
//     queued and re-evaluated 64 at a time from memory (wider rows); accepted
//     (d2, idx) keys go to a per-query candidate list.  Every pair within the
//     radius lies in the query's shell, so candidates streamed for other
//     queries of the wave need no membership test: they fail the exact test;
//   * every query keeps a histogram of its list's keys by distance; as soon as
//     K keys lie below a bucket edge its threshold drops to that edge.  A list
//     that nears capacity first drops its keys above the threshold; if it is
//     still long, the wave sorts it cooperatively (bitonic in registers, up to
//     4 keys per lane), keeps the K smallest and tightens the threshold to the
//     K-th key; at the end every list is sorted and its first K keys (plus
//     padding) are the result for that sorted position.
//
// Exactness: a pair is returned iff its exact fp32 distance in the reference
// order is < r2 and it is among the K smallest (d2, idx) keys.  The MFMA value
// only decides which pairs are re-evaluated; its margin (norm_scale, thr_rel,
// thr_abs, set on the host) covers the rounding of the centring, the norms, the
// fp32 MFMA accumulation (with a factor 2 on the unit roundoff) and the exact
// order, so no pair that could qualify is dropped.  NaN or overflowed filter
// values are always re-evaluated.
#include <cstring>

#include "frnn_device.hpp"
#include "frnn_internal.hpp"

namespace frnn {

constexpr int kQB = 32;                      // queries per wave
constexpr int kBatch = 64;                   // exact re-evaluations per batch
constexpr int kQueueCap = kBatch + 16 * kWave;  // leftover batch + one tile's hits
static_assert(FRNN_MAX_K + 128 <= 4 * kWave, "a candidate list fits the largest register sort");

// Workgroups are one wave, so lanes only need their LDS accesses ordered: an
// LDS-only fence around the barrier leaves outstanding global loads (the
// prefetched tile) in flight, where __syncthreads() would wait for them.
__device__ __forceinline__ void lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}
// Frames walk each segment's rows in two passes: the first at the inner
// threshold inner_frac2(K) r^2 (or the segment's threshold if smaller), the
// second at the segment's threshold as the first pass's candidates have
// tightened it, streaming only what the first pass has not.
constexpr int kPasses = 2;
constexpr float kK16Frac2 = 2.0f;   // K <= 16: one pass
constexpr int kRing = 128;                   // pending candidate runs (<= 31 + 64 in use)
constexpr int kMaxG = 9;

// Threshold histograms.  Each query counts the keys of its list by bucket of
// their squared distance below r2.  Non-negative fp32 bit patterns order like
// the values, so with top = bits(r2) and d2 < r2
//   bucket(d2) = B - 1 - min((top - 1 - bits(d2)) >> S, B - 1):
// bucket b >= 1 holds the bit patterns [top - (B-b) 2^S, top - (B-1-b) 2^S),
// bucket 0 everything below its upper edge top - (B-1) 2^S.  Once the buckets
// up to b hold at least K keys of the list, the K-th smallest key lies below
// bucket b's upper edge, so no key at or above it can be among the K results:
// the query's threshold drops to that edge without sorting the list.  Buckets
// are 2^S fp32 ulps of d2 wide: S = 21 (a quarter octave, the buckets reach 4
// octaves below r2) for K <= 32, S = 20 (an eighth, 2 octaves) for larger K,
// whose K-th distance lies nearer the radius; hist_shift picks S.  Counts are
// bytes, four to a word (a list never holds more than 255 keys).
constexpr int kHB = 16;                      // buckets per query
constexpr int kHW = kHB / 4;                 // histogram words per query
constexpr int kMaxRoom = 255;                // list entries in use (byte counts)

__device__ __forceinline__ int hist_bucket(float d2, unsigned top, int hs) {
    const unsigned u = (top - 1u - __float_as_uint(d2)) >> hs;
    return kHB - 1 - (int)min(u, (unsigned)(kHB - 1));
}
// key just above bucket b: a key is below it iff its d2 lies in a bucket <= b
__device__ __forceinline__ unsigned long long hist_edge_key(int b, unsigned top, int hs) {
    return (unsigned long long)(top - ((unsigned)(kHB - 1 - b) << hs)) << 32;
}

// Traversal order of a segment's 3^m neighbouring rows (m = g - 1 axes): by
// the number of axes on which the row is offset (the segment's own row, then
// faces, edges, corners), so the nearest candidates stream first and a list's
// first compaction already sets a threshold near its K-th distance.  Entries
// are natural row indices, digit d (0, 1, 2) = offset -1, 0, +1 on axis d + 1.
struct RowOrder { unsigned char v[27]; };
constexpr RowOrder make_row_order(int m) {
    RowOrder r{};
    int n = 1;
    for (int i = 0; i < m; ++i) n *= 3;
    int k = 0;
    for (int w = 0; w <= m; ++w)
        for (int t = 0; t < n; ++t) {
            int tt = t, nz = 0;
            for (int d = 0; d < m; ++d) {
                nz += (tt % 3) != 1;
                tt /= 3;
            }
            if (nz == w) r.v[k++] = (unsigned char)t;
        }
    return r;
}
__constant__ RowOrder kRowOrder[4] = {make_row_order(0), make_row_order(1), make_row_order(2),
                                      make_row_order(3)};
// natural index of the o-th row in traversal order; more than 3 row axes map
// each base-3 digit 0, 1, 2 to offset 0, -1, +1 (own row first)
__device__ __forceinline__ int natural_row(int o, int m) {
    if (m <= 3) return kRowOrder[m].v[o];
    int t = 0, p = 1;
    for (int d = 0; d < m; ++d) {
        const int dg = o % 3;
        o /= 3;
        t += (dg == 0 ? 1 : dg == 1 ? 0 : 2) * p;
        p *= 3;
    }
    return t;
}

struct SearchArgs {
    const float* pts;            // AoS rows, stride DS (sorted order for grids)
    const float* frows;          // the same rows centred, fl(x - mean) (wide rows only)
    const DimStat* st;           // per-coordinate statistics: the filter centre is the mean
    const int* sorted_idx;       // sorted position -> original index (grid paths)
    const int* cell_of;          // original index -> cell id (grid paths)
    const int* start;            // cells+1 exclusive cell offsets (grid paths)
    const Frame* frame;          // grid frame, or nullptr (grids above 4 axes)
    // the queries in search order (the points themselves for an all-points
    // search): AoS rows, centred rows (wide rows only), search position ->
    // original query index and original query index -> cell id (grid paths)
    const float* qpts;
    const float* qfrows;
    const int* qsorted_idx;
    const int* qcell_of;
    unsigned long long* lists;   // [M][cap] candidate keys
    unsigned long long* counters;
    unsigned* status;            // set to 1 if a capacity guard fired (may be null)
    int N, M, D, K, cap, G, res; // N points, M queries; res: raw-grid cells per axis
    int gstride[kMaxG];          // raw-grid cell-id stride per axis
    int room;                    // usable list entries: min(cap, kMaxRoom)
    int hist_on;                 // threshold histograms in use (r2 is not tiny)
    int exact_limit;             // a filtered list above this gets the exact compaction
    unsigned r2bits;             // bits(r2)
    int hist_shift;              // histogram bucket width: 2^hist_shift ulps of d2
    float inner2;                // the first pass's threshold on frames (>= r2: one pass)
    float r2, cell, radius;      // cell: raw-grid cell edge
    float norm_scale;            // 1 - c_norm
    float thr_rel, thr_abs;      // filter threshold margin
    int nchunks;
    // brute force on wide rows: the points split into `slices` ranges of
    // slice_tiles 32-point tiles, one workgroup per (query block, range); range
    // s writes its own lists at rows s * M + query (merged afterwards)
    int slices, slice_tiles;
};

__device__ __forceinline__ float filter_threshold(float thr, const SearchArgs& a) {
    return fmaf(thr, a.thr_rel, thr) + a.thr_abs;
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

// Rows of 4 floats keep six waves per SIMD resident (register budget 80),
// rows of 8 and 12 five (96), rows of 16 four (128): the search is bound by
// the latency of its gathers, list round trips and sorts, so the extra wave
// outweighs a few spilled registers (measured: DS = 4 about 1% faster at six
// than at five, DS = 12 fastest at five, DS = 8 the same at four or five; at
// DS = 16 the compiler cannot fit five).
// Larger rows keep two (256 VGPRs + AGPRs), so a second wave's MFMA chain can
// overlap one wave's hit handling.
template <int DS>
struct WavesPerEU { static constexpr int value = DS <= 4 ? 6 : DS <= 12 ? 5 : DS <= 16 ? 4 : 2; };

// CNT: the profiling build of the kernel, which also keeps the work counters
// (a separate instantiation, so the counting code costs the plain kernel no
// registers).  NW: waves per workgroup.  One wave for every grid path (each
// wave streams its own candidates); brute force on wide rows runs NW waves
// that share each candidate tile through LDS (below).
template <int DS, bool REV, bool BF, bool CNT, int NW = 1>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(WavesPerEU<DS>::value)))
void search_kernel(SearchArgs a) {
    constexpr bool MW = NW > 1;
    static_assert(!MW || (BF && DS >= 64), "shared candidate tiles: brute force on wide rows");
    constexpr int HD = DS / 2;
    // The chunk's query rows: staged in LDS for DS <= 32; wider rows are read
    // from the AoS array (the same 32 rows, cache resident), which keeps LDS
    // small enough for two workgroups per SIMD.  LDS rows are RS floats apart:
    // DS padded by 4 when DS is a multiple of 8, so the 16-byte reads of
    // different rows spread over all eight 4-bank groups.
    constexpr bool kQueryLds = DS <= 32;
    constexpr int RS = (DS % 8 == 0) ? DS + 4 : DS;
    __shared__ __align__(16) float s_q[kQueryLds ? kQB * RS : 4];
    // Per-wave state (one slice per wave of the workgroup): list lengths,
    // sorted prefix lengths, thresholds, histograms, counters and the queue.
    __shared__ int s_cnt_w[NW * kQB];
    __shared__ int s_srt_w[NW * kQB];       // sorted prefix length of each list
    __shared__ unsigned long long s_thr_w[NW * kQB];
    // threshold histograms: byte b of query n's words is its bucket b count;
    // s_hb[n], the lowest bucket whose keys and those below number at least K
    // once that happens (B - 1 before); s_hcle[n], the number of keys in
    // buckets <= s_hb[n].  Every accepted key is below the threshold, which
    // never exceeds bucket s_hb[n]'s upper edge, so it lands in such a bucket.
    __shared__ unsigned s_hist_w[NW * kQB * kHW];
    __shared__ int s_hcle_w[NW * kQB];
    __shared__ unsigned char s_hb_w[NW * kQB];
    __shared__ unsigned long long s_ctr_w[NW * 5];
    // Rows of up to 32 floats re-evaluate a tile's hits right after its MFMA
    // chain, from the tile's raw rows staged in LDS; wider rows queue hits as
    // (query, sorted position) and re-evaluate them 64 at a time from memory.
    constexpr bool kTileExact = DS <= 32;
    __shared__ unsigned char s_qn_w[kTileExact ? 1 : NW * kQueueCap];
    __shared__ __align__(8) int s_qpos_w[kTileExact ? 1 : NW * kQueueCap];
    // candidate run ring: [start, start + (vend - vbeg)) of the sorted points
    // at virtual stream positions [vbeg, vend).  Runs are contiguous in the
    // stream, so a run's vbeg is the vend of the run before it (slot
    // kRing - 1 starts at 0 for the first run; at most 96 slots are in use,
    // so the slot before a pending run is never overwritten).
    __shared__ int r_start[kRing], r_vend[kRing];
    // current tile, per candidate row: the sorted position (queue path) or
    // the original index and the raw row (tile-exact path), and the hit
    // entries (row << 5 | query).  Staged rows are TS floats apart: RS as s_q, except
    // at DS = 16 (four waves per SIMD), where unpadded rows keep the
    // workgroup within a quarter of the LDS per SIMD.
    constexpr int TS = DS == 16 ? DS : RS;
    __shared__ int t_pos_w[kTileExact ? 1 : NW * 32];
    __shared__ int t_idx[kTileExact ? 32 : 1];
    __shared__ __align__(16) float t_rows[kTileExact ? 32 * TS : 4];
    // (a tile holds at most 32 x 32 hits)
    __shared__ __align__(8) unsigned short s_hit[kTileExact ? 32 * 32 : 2];
    // The final selection compacts a list into up to 128 keys of LDS: the hit
    // entries (tile-exact path) or the wave's queue slice, both idle by then.
    static_assert(sizeof(unsigned short) * 32 * 32 >= 128 * 8 && sizeof(int) * kQueueCap >= 128 * 8,
                  "final selection staging");
    // grid geometry per axis (cells, cell-id stride, origin), the segment's
    // bounding box and row coordinates, and each query's grid coordinates
    __shared__ int s_res[kMaxG], s_stride[kMaxG];
    __shared__ float s_org[kMaxG];
    __shared__ float s_blo[kMaxG], s_bhi[kMaxG];
    __shared__ int s_rc[kMaxG];
    // rows of 16 or more floats only occur on first-coordinate grids (g <= 4;
    // a full-D grid needs res^D <= 1M cells with res > 3, so D <= 9)
    constexpr int kGA = DS >= 16 ? kFrameGrid : kMaxG;
    __shared__ float s_qg[BF ? 1 : kQB * kGA];
    // brute force with shared tiles: two buffers of 32 centred candidate rows,
    // BRS floats apart (DS + 4: the 16-byte reads of 8 consecutive rows cover
    // all bank groups)
    constexpr int BRS = DS + 4;
    __shared__ __align__(16) float bf_tile[MW ? 2 * 32 * BRS : 4];

    const int lane = MW ? (int)(threadIdx.x & (kWave - 1)) : (int)threadIdx.x;
    const int wave = MW ? (int)(threadIdx.x / kWave) : 0;
    int* const s_cnt = s_cnt_w + wave * kQB;
    int* const s_srt = s_srt_w + wave * kQB;
    unsigned long long* const s_thr = s_thr_w + wave * kQB;
    unsigned* const s_hist = s_hist_w + wave * kQB * kHW;
    int* const s_hcle = s_hcle_w + wave * kQB;
    unsigned char* const s_hb = s_hb_w + wave * kQB;
    unsigned long long* const s_ctr = s_ctr_w + wave * 5;
    unsigned char* const s_qn = s_qn_w + (kTileExact ? 0 : wave * kQueueCap);
    int* const s_qpos = s_qpos_w + (kTileExact ? 0 : wave * kQueueCap);
    int* const t_pos = t_pos_w + (kTileExact ? 0 : wave * 32);
    unsigned long long* const s_fin =
        kTileExact ? reinterpret_cast<unsigned long long*>(s_hit) : reinterpret_cast<unsigned long long*>(s_qpos);
    // Synchronisation of a wave's own LDS traffic.  A one-wave workgroup uses
    // the barrier with LDS-only fences; in a multi-wave workgroup the per-wave
    // code (hits, lists, selection) must not use the workgroup barrier (its
    // waves reach different numbers of those): one wave's LDS accesses take
    // effect in program order, so a compiler fence suffices there.
    auto lsync = [&]() __attribute__((always_inline)) {
        if constexpr (MW) __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront", "local");
        else lds_sync();
    };
    const int n = lane & 31;
    const int h = lane >> 5;
    // Workgroup b runs on XCD b % 8, so consecutive chunks of the cell order
    // spread over all XCDs.  Work per chunk follows the point density, and a
    // contiguous range per XCD left the XCDs holding dense regions finishing
    // up to 2x later than the rest; interleaving keeps them balanced.  A
    // multi-wave workgroup keeps waves without queries (the last workgroup's)
    // running: every wave passes the tile barriers.
    const int chunk = blockIdx.x * NW + wave;
    if (!MW && chunk >= a.nchunks) return;
    const int q0 = chunk * kQB;
    // (waves of a multi-wave workgroup past the last chunk have no queries)
    const int nq = MW ? max(min(kQB, a.M - q0), 0) : min(kQB, a.M - q0);
    const bool qvalid = n < nq;
    unsigned long long* const lists =
        a.lists + ((size_t)(MW ? blockIdx.y : 0) * a.M + (size_t)(MW ? min(q0, a.M) : q0)) * a.cap;

    if constexpr (kQueryLds) {
        const float* src = a.qpts + (size_t)(q0 + (qvalid ? n : 0)) * DS + h * HD;
        float* dst = s_q + n * RS + h * HD;
#pragma unroll
        for (int j = 0; j < HD; j += 2) {
            float2 v = *reinterpret_cast<const float2*>(src + j);
            if (!qvalid) v = make_float2(0.0f, 0.0f);
            dst[j] = v.x;
            dst[j + 1] = v.y;
        }
    }
    // row of query qn (a valid query of the chunk; queue path, wide rows)
    auto query_row = [&](int qn) -> const float* { return a.qpts + (size_t)(q0 + qn) * DS; };
    if (CNT && lane < 5) s_ctr[lane] = 0;
    if (lower_half()) {
        s_cnt[lane] = 0;
        s_srt[lane] = 0;
        s_thr[lane] = make_key(a.r2, 0);
        s_hcle[lane] = 0;
        s_hb[lane] = (unsigned char)(kHB - 1);
    }
#pragma unroll
    for (int i = lane; i < kQB * kHW; i += kWave) s_hist[i] = 0u;
    if (first_lane() && wave == 0) r_vend[kRing - 1] = 0;
    lsync();
    // Filter operands are the rows centred on the input mean, fl(x - mean).
    // Rows of up to 32 floats are centred in registers as they are loaded
    // (this lane's half of the means stays in registers); wider rows stream
    // the centred copy the reorder wrote, which keeps their loads ahead of the
    // MFMA chain.
    constexpr bool kCentredRows = DS >= 64;
    float mh[kCentredRows ? 1 : HD];
    if constexpr (!kCentredRows) {
#pragma unroll
        for (int j = 0; j < HD; ++j) {
            const int d = h * HD + j;
            mh[j] = d < a.D ? a.st[d].mean : 0.0f;
        }
    }
    const float* const op_rows = kCentredRows ? a.frows : a.pts;
    auto centre = [&](float x, int j) __attribute__((always_inline)) -> float {
        if constexpr (kCentredRows) return x;
        else return x - mh[j];
    };
    // B operand: this lane's half of query n's centred row, scaled by -2, plus
    // the norm column (the squared norm of the centred row, summed from both
    // halves).  Rows of a chunk are the queries q0..q0+31 of the search order.
    float bop[HD + 1];
    float qn2 = 0.0f;
    {
        // (invalid lanes read a valid row: the chunk's first, or row 0 in a
        // wave without queries)
        const int qrow = MW ? (qvalid ? q0 + n : 0) : q0 + (qvalid ? n : 0);
        const float* qr = (kCentredRows ? a.qfrows : a.qpts) + (size_t)qrow * DS + h * HD;
        float pn = 0.0f;
#pragma unroll
        for (int j = 0; j < HD; j += 2) {
            const float2 v = *reinterpret_cast<const float2*>(qr + j);
            const float c0 = centre(v.x, j), c1 = centre(v.y, j + 1);
            bop[j] = -2.0f * c0;
            bop[j + 1] = -2.0f * c1;
            pn = fmaf(c0, c0, pn);
            pn = fmaf(c1, c1, pn);
        }
        unsigned pa, pb;
        xor_pair_u32(__float_as_uint(pn), 32, pa, pb);
        qn2 = __uint_as_float(pa) + __uint_as_float(pb);
        bop[HD] = lower_half() ? a.norm_scale : qn2 * a.norm_scale;
    }
    if (!qvalid) {
#pragma unroll
        for (int j = 0; j <= HD; ++j) bop[j] = 0.0f;
    }
    float thr_f = qvalid ? filter_threshold(a.r2, a) : -__builtin_huge_valf();
    // Queries whose centred norm could overflow the filter always take the
    // per-value (NaN-aware) hit test.
    const bool robust_q = __ballot(qvalid && !(qn2 < 1.0e37f)) != 0;

    // Profiling counters (CNT): wave totals kept in LDS by lane 0 from ballot
    // counts.  Slots: shell candidates, filter hits, accepted keys, streamed
    // (query, candidate) pairs, list/queue capacity overflows.
    constexpr bool counting = CNT;
    auto bump = [&](int i, unsigned long long v) __attribute__((always_inline)) {
        if (counting && first_lane()) s_ctr[i] += v;
    };
    // A capacity guard fired (a logic error): the caller's status word says so
    // (wave-uniform call).
    auto report_overflow = [&](bool ovf) __attribute__((always_inline)) {
        if (counting) bump(4, __popcll(__ballot(ovf)));
        if (a.status && __ballot(ovf) != 0 && first_lane()) a.status[0] = 1u;
    };
    int q_size = 0;                     // queue entries (wave-uniform)

    // An exactly re-evaluated key below query qn's threshold joins its list.
    auto accept = [&](int qn, unsigned long long key, bool& ovf) __attribute__((always_inline)) {
        const int slot = atomicAdd(&s_cnt[qn], 1);
        // compaction before each round leaves >= kBatch free slots; the guard
        // only keeps a logic error (or a caller's too-small list) from writing
        // past the list
        if (slot < a.room) lists[(size_t)qn * a.cap + slot] = key;
        else ovf = true;
    };
    // End of a round (wave-uniform call; acc: this lane accepted `key` for
    // query qn).  The accepted keys join their queries' histograms; then every
    // query whose buckets up to a lower one now hold >= K keys moves s_hb down
    // and its threshold to that bucket's upper edge.  Only query n's own lanes
    // use its threshold before the next barrier (the hit tests of the next
    // tile), so they take it into thr_f directly; other lanes read s_thr after
    // the barrier that starts the next staging or round.  (The histogram
    // update waits for the round's end, when the rows of the exact evaluation
    // are no longer live.)
    auto end_round = [&](bool acc, int qn, unsigned long long key) __attribute__((always_inline)) {
        const bool any = __ballot(acc) != 0;
        if (a.hist_on && any && acc) {
            const int b = hist_bucket(key_d2(key), a.r2bits, a.hist_shift);
            atomicAdd(&s_hist[qn * kHW + (b >> 2)], 1u << (8 * (b & 3)));
            atomicAdd(&s_hcle[qn], 1);
        }
        lsync();
        if (a.hist_on && any && qvalid) {
            int cle = s_hcle[n];
            if (cle >= a.K) {
                const unsigned char* hb = reinterpret_cast<const unsigned char*>(s_hist) + n * kHB;
                const int b0 = s_hb[n];
                int b = b0;
                int cb = hb[b];
                while (b > 0 && cle - cb >= a.K) {
                    cle -= cb;
                    --b;
                    cb = hb[b];
                }
                if (b != b0) {
                    const unsigned long long ek = hist_edge_key(b, a.r2bits, a.hist_shift);
                    const unsigned long long t = s_thr[n];
                    const unsigned long long nt = ek < t ? ek : t;
                    thr_f = filter_threshold(key_d2(nt), a);
                    if (lower_half()) {
                        s_hb[n] = (unsigned char)b;
                        s_hcle[n] = cle;
                        s_thr[n] = nt;
                    }
                }
            }
        }
        // one wave: its LDS accesses execute in program order; the fence keeps
        // the compiler from moving later reads of s_thr above these writes
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront", "local");
    };

    // Selection on query qn's candidate list.  A list keeps its first s_srt[qn]
    // keys sorted (the K kept at the last compaction); later arrivals follow
    // unsorted.  The new keys are sorted in registers (wave_sort_u64 over the
    // smallest power-of-two multiple of 64 holding them, ~0 filling the rest)
    // and their first P = 64*EK (>= K) are merged with the sorted prefix A:
    // C[i] = min(A[i], B[P-1-i]) holds the P smallest of both and is bitonic,
    // so the half-cleaner stages sort it.  Compaction keeps the K smallest and
    // tightens the query's threshold to the K-th key; the final pass writes the
    // K smallest (padded with (r2, -1)).
    auto select_merge = [&](auto ek_const, auto en_const, int qn, int c, int m,
                            bool final_pass) __attribute__((always_inline)) {
        constexpr int EK = decltype(ek_const)::value;
        constexpr int EN = decltype(en_const)::value;
        unsigned long long* L = lists + (size_t)qn * a.cap;
        // the list entries were stored by other lanes of this wave
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
        // new keys and the sorted prefix in one round trip (the prefix loads
        // stay in flight during the sort)
        unsigned long long b[EN], av[EK];
#pragma unroll
        for (int e = 0; e < EN; ++e) {
            const int i = m + e * kWave + lane;
            b[e] = (i < c) ? L[i] : ~0ull;
        }
#pragma unroll
        for (int e = 0; e < EK; ++e) {
            const int i = e * kWave + lane;
            av[e] = (i < m) ? L[i] : ~0ull;
        }
        wave_sort_u64<EN>(b);
        unsigned long long x[EK];
#pragma unroll
        for (int e = 0; e < EK; ++e) x[e] = (e < EN) ? b[e] : ~0ull;
        if (m > 0) {
            // element i of C pairs A[i] with B[P-1-i]: register EK-1-e, lane 63-lane
            unsigned long long cm[EK];
#pragma unroll
            for (int e = 0; e < EK; ++e) {
                const unsigned long long rb = shfl_u64(x[EK - 1 - e], kWave - 1 - lane);
                cm[e] = av[e] < rb ? av[e] : rb;
            }
#pragma unroll
            for (int e = 0; e < EK; ++e) x[e] = cm[e];
            wave_bitonic_merge_u64<EK>(x);
        }
        if (final_pass) {
            const unsigned long long pad = make_key(a.r2, -1);
#pragma unroll
            for (int e = 0; e < EK; ++e) {
                const int i = e * kWave + lane;
                if (i < a.K) L[i] = (i < c) ? x[e] : pad;
            }
        } else {
            const int keep = min(c, a.K);
#pragma unroll
            for (int e = 0; e < EK; ++e) {
                const int i = e * kWave + lane;
                if (i < keep) L[i] = x[e];
            }
            unsigned long long kth = 0;
            if (c >= a.K) {
                const int ek = (a.K - 1) / kWave;
                kth = x[0];
#pragma unroll
                for (int e = 1; e < EK; ++e)
                    if (e == ek) kth = x[e];
                kth = shfl_u64(kth, (a.K - 1) & (kWave - 1));
                if (first_lane()) s_thr[qn] = kth;
            }
            if (first_lane()) {
                s_cnt[qn] = keep;
                s_srt[qn] = keep;
            }
            if (a.hist_on) {
                // the list now holds the `keep` smallest keys: rebuild its
                // histogram from them (every kept key is <= the K-th, so in a
                // bucket <= the K-th key's)
                if (lane < kHW) s_hist[qn * kHW + lane] = 0u;
                lsync();
#pragma unroll
                for (int e = 0; e < EK; ++e) {
                    const int i = e * kWave + lane;
                    if (i < keep) {
                        const int b = hist_bucket(key_d2(x[e]), a.r2bits, a.hist_shift);
                        atomicAdd(&s_hist[qn * kHW + (b >> 2)], 1u << (8 * (b & 3)));
                    }
                }
                if (first_lane()) {
                    s_hcle[qn] = keep;
                    s_hb[qn] = (unsigned char)(c >= a.K ? hist_bucket(key_d2(kth), a.r2bits, a.hist_shift) : kHB - 1);
                }
            }
        }
        lsync();
    };
    // Filter compaction of query qn's list: drop the keys above its threshold
    // (they can no longer be among the K results), keeping the order, so the
    // sorted prefix stays sorted.  Every key counted in the histogram's
    // buckets <= s_hb[qn] is <= the threshold and stays.  Returns the new length.
    auto filter_list = [&](int qn) __attribute__((always_inline)) -> int {
        unsigned long long* L = lists + (size_t)qn * a.cap;
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
        const int c = min(s_cnt[qn], a.room);
        const int m = s_srt[qn];
        const unsigned long long thr = s_thr[qn];
        // chunk by chunk: the kept keys of chunks <= e move to positions below
        // (e + 1) * 64, so no store reaches a chunk not yet loaded
        int base = 0, nm = 0;
        for (int e = 0; e * kWave < c; ++e) {
            const int i = e * kWave + lane;
            const unsigned long long v = (i < c) ? L[i] : ~0ull;
            const bool kp = i < c && v <= thr;
            const unsigned long long mk = __ballot(kp);
            const int pos = base + (int)__builtin_amdgcn_mbcnt_hi((unsigned)(mk >> 32),
                                                                 __builtin_amdgcn_mbcnt_lo((unsigned)mk, 0u));
            if (kp) L[pos] = v;
            nm += __popcll(__ballot(kp && i < m));
            base += __popcll(mk);
        }
        if (first_lane()) {
            s_cnt[qn] = base;
            s_srt[qn] = nm;
        }
        lsync();
        return base;
    };
    // Final selection of query qn's list for K <= 64 (one sort register).  The
    // keys at or below the query's threshold, a superset of its K smallest,
    // are compacted into LDS in list order.  Up to 64 of them take one
    // register sort.  Up to 128 fill a second register x1 that is brought into
    // descending order, so that min(x0[i], x1[i]) is bitonic and holds the 64
    // smallest of both, which the half-cleaners sort: a second register of at
    // most 16 keys sits in lanes 48..63, where the first four levels of the
    // network (blocks of 16, lanes with bit 4 set descending) already sort it
    // descending behind the ~0 fill; a fuller one is sorted and reversed.
    // Returns false, having changed nothing, when more than 128 keys lie at
    // or below the threshold (the general path then runs).
    auto final_small = [&](int qn) __attribute__((always_inline)) -> bool {
        unsigned long long* L = lists + (size_t)qn * a.cap;
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
        const int c = min(s_cnt[qn], a.room);
        const unsigned long long thr = s_thr[qn];
        // the whole list in one round trip (c <= 255 < 4 * 64)
        unsigned long long v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int i = e * kWave + lane;
            v[e] = (i < c) ? L[i] : ~0ull;
        }
        int cnt = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int i = e * kWave + lane;
            const bool kp = i < c && v[e] <= thr;
            const unsigned long long mk = __ballot(kp);
            const int pos = cnt + (int)__builtin_amdgcn_mbcnt_hi((unsigned)(mk >> 32),
                                                                 __builtin_amdgcn_mbcnt_lo((unsigned)mk, 0u));
            if (kp && pos < 2 * kWave) s_fin[pos] = v[e];
            cnt += __popcll(mk);
        }
        if (cnt > 2 * kWave) return false;
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront", "local");
        unsigned long long x0[1];
        x0[0] = lane < cnt ? s_fin[lane] : ~0ull;
        if (cnt > kWave) {
            const int w = cnt - kWave;
            unsigned long long x1[1];
            if (w <= 16) {
                x1[0] = lane >= kWave - 16 && lane - (kWave - 16) < w ? s_fin[lane + 16] : ~0ull;
                wave_sort_u64<1>(x0);
#pragma unroll
                for (int lk = 1; lk <= 4; ++lk) {
#pragma unroll
                    for (int lj = lk - 1; lj >= 0; --lj) bitonic_step<1>(x1, 1 << lk, 1 << lj);
                }
            } else {
                x1[0] = lane < w ? s_fin[kWave + lane] : ~0ull;
                wave_sort_u64<1>(x0);
                wave_sort_u64<1>(x1);
                x1[0] = shfl_u64(x1[0], kWave - 1 - lane);
            }
            x0[0] = x0[0] < x1[0] ? x0[0] : x1[0];
            wave_bitonic_merge_u64<1>(x0);
        } else {
            wave_sort_u64<1>(x0);
        }
        if (lane < a.K) L[lane] = lane < cnt ? x0[0] : make_key(a.r2, -1);
        lsync();
        return true;
    };
    // Final selection of 64 / W lists of at most W keys each (W = 16 or 32,
    // K <= W), one per W-lane block of the wave: query qs[g]'s keys in block
    // g (qs[g] < 0: none), ~0 filling the rest.  The network's first levels
    // sort blocks of W / 2 in alternating directions; the last merges each
    // block ascending (the direction of element bit 6, clear for every lane),
    // so one sort of log2(W) levels (10 or 15 stages) serves them all.
    auto final_group = [&](auto lw_const, const int (&qs)[4]) __attribute__((always_inline)) {
        constexpr int LW = decltype(lw_const)::value;   // log2(W)
        constexpr int W = 1 << LW;
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
        const int g = lane >> LW;
        const int qq = g == 0 ? qs[0] : g == 1 ? qs[1] : g == 2 ? qs[2] : qs[3];
        const int cq = qq >= 0 ? min(s_cnt[qq], a.room) : 0;
        const int i = lane & (W - 1);
        unsigned long long* L = lists + (size_t)(qq >= 0 ? qq : 0) * a.cap;
        unsigned long long x[1];
        x[0] = i < cq ? L[i] : ~0ull;
#pragma unroll
        for (int lk = 1; lk < LW; ++lk) {
#pragma unroll
            for (int lj = lk - 1; lj >= 0; --lj) bitonic_step<1>(x, 1 << lk, 1 << lj);
        }
#pragma unroll
        for (int lj = LW - 1; lj >= 0; --lj) bitonic_step<1>(x, kWave, 1 << lj);
        if (qq >= 0 && i < a.K) L[i] = i < cq ? x[0] : make_key(a.r2, -1);
        lsync();
    };
    auto select_topk = [&](int qn, bool final_pass) __attribute__((always_inline)) {
        // (lists whose new keys fit one register take the general path: the
        // same single sort without the staging)
        if (final_pass && a.K <= kWave && min(s_cnt[qn], a.room) - s_srt[qn] > kWave && final_small(qn)) return;
        // a final list with stale keys beyond two sort registers is filtered
        // first (a smaller sort)
        if (final_pass && a.hist_on && min(s_cnt[qn], a.room) - s_srt[qn] > 2 * kWave) filter_list(qn);
        const int c = min(s_cnt[qn], a.room);
        const int m = s_srt[qn];
        const int nn = c - m;
        if (a.K <= kWave) {
            if (nn <= kWave) select_merge(IntC<1>{}, IntC<1>{}, qn, c, m, final_pass);
            else if (nn <= 2 * kWave) select_merge(IntC<1>{}, IntC<2>{}, qn, c, m, final_pass);
            else select_merge(IntC<1>{}, IntC<4>{}, qn, c, m, final_pass);
        } else {
            if (nn <= kWave) select_merge(IntC<2>{}, IntC<1>{}, qn, c, m, final_pass);
            else if (nn <= 2 * kWave) select_merge(IntC<2>{}, IntC<2>{}, qn, c, m, final_pass);
            else select_merge(IntC<2>{}, IntC<4>{}, qn, c, m, final_pass);
        }
    };
    // Room for a round in query qn's list: first the filter compaction; if
    // the list is still long (keys crowded into one bucket, or histograms
    // off), the exact one, which keeps the K smallest.
    auto compact = [&](int qn) __attribute__((always_inline)) {
        if (a.hist_on && filter_list(qn) <= a.exact_limit) return;
        select_topk(qn, false);
    };
    // Before a round: compact every list that could overflow during it, then
    // reload the filter thresholds.
    auto make_room = [&]() __attribute__((always_inline)) {
        const bool need = lower_half() && s_cnt[lane] > a.room - kBatch;
        unsigned long long m = __ballot(need);
        if (m) {
            while (m) {
                const int qn = __ffsll((long long)m) - 1;
                m &= m - 1;
                compact(qn);
            }
            if (qvalid) thr_f = filter_threshold(key_d2(s_thr[n]), a);
        }
    };

    // Exact re-evaluation of queue entries [base, base + count) (queue path).
    // First every list that could overflow during the batch is compacted; with
    // final_pass every list of the chunk gets its final selection instead.
    auto process_batch = [&](int base, int count, bool final_pass) __attribute__((always_inline)) {
        // (one call site of the selection for both uses keeps a single
        // inlined copy of the sorts)
        const bool need = lower_half() && (final_pass ? lane < nq : s_cnt[lane] > a.room - kBatch);
        unsigned long long m = __ballot(need);
        if (m) {
            if (final_pass && a.K <= 32) {
                // lists of at most 16 keys (K <= 16): four per sort; of at
                // most 32: two per sort
                const int cn = min(s_cnt[n], a.room);
                auto take = [&](unsigned long long& sm) __attribute__((always_inline)) -> int {
                    if (!sm) return -1;
                    const int q = __ffsll((long long)sm) - 1;
                    sm &= sm - 1;
                    return q;
                };
                if (a.K <= 16) {
                    unsigned long long s16 = __ballot(need && cn <= 16);
                    m &= ~s16;
                    while (s16) {
                        int qs[4];
#pragma unroll
                        for (int g = 0; g < 4; ++g) qs[g] = take(s16);
                        final_group(IntC<4>{}, qs);
                    }
                }
                unsigned long long s32 = __ballot(need && cn <= 32) & m;
                m &= ~s32;
                while (s32) {
                    int qs[4];
                    qs[0] = take(s32);
                    qs[1] = take(s32);
                    qs[2] = qs[3] = -1;
                    final_group(IntC<5>{}, qs);
                }
            }
            while (m) {
                const int qn = __ffsll((long long)m) - 1;
                m &= m - 1;
                if (final_pass || !(a.hist_on && filter_list(qn) <= a.exact_limit)) select_topk(qn, final_pass);
            }
            if (qvalid) thr_f = filter_threshold(key_d2(s_thr[n]), a);
        }
        bool accepted = false, ovf = false;
        int qn = 0;
        unsigned long long key = 0;
        if (!kTileExact && lane < count) {
            qn = s_qn[base + lane];
            const int pos = s_qpos[base + lane];
            const float e = exact_d2<DS, REV>(query_row(qn), a.pts + (size_t)pos * DS);
            const int idx = BF ? pos : a.sorted_idx[pos];
            key = make_key(e, idx);
            accepted = key < s_thr[qn];
            if (accepted) accept(qn, key, ovf);
        }
        if constexpr (counting) bump(2, __popcll(__ballot(accepted)));
        report_overflow(ovf);
        end_round(accepted, qn, key);
        q_size = base;
    };

    // ---- candidate stream -------------------------------------------------
    int ring_head = 0, ring_tail = 0;   // absolute run indices (wave-uniform)
    int v_total = 0, v_done = 0;        // virtual candidate positions (wave-uniform)
    int jr = 0;                         // this lane's current run
    int x_n = 0;                        // cell x of this lane's query
    // stream positions of the candidates streamed for this lane's query's
    // row segment (the segment still streaming ends at INT_MAX)
    int q_vbeg = 0, q_vend = 0;

    // Gather one tile of the stream into operand registers: the run lookup for
    // stream position v0 + n, the centred row half and the norm column.
    struct Tile {
        float op[HD];
        int pos, count;
        int v0;                         // stream position of row 0
        int idx;                        // original index (tile-exact path)
    };
    auto gather = [&](int v0, int count, Tile& t) __attribute__((always_inline)) {
        const int v = v0 + n;
        const bool mvalid = n < count;
        t.count = count;
        t.v0 = v0;
        t.pos = 0;
        t.idx = -1;
        if (mvalid) {
            if (jr < ring_tail) jr = ring_tail;
            while (r_vend[jr & (kRing - 1)] <= v) ++jr;
            const int j = jr & (kRing - 1);
            t.pos = r_start[j] + (v - r_vend[(jr - 1) & (kRing - 1)]);
            if constexpr (kTileExact) {
                // both halves of the wave load it (the same address: one
                // coalesced access, and no per-half exec mask in the tile loop)
                t.idx = BF ? t.pos : a.sorted_idx[t.pos];
            }
        }
        const float* pr = op_rows + (size_t)t.pos * DS + h * HD;
#pragma unroll
        for (int j = 0; j < HD; j += 2) {
            const float2 vv = *reinterpret_cast<const float2*>(pr + j);
            t.op[j] = vv.x;
            t.op[j + 1] = vv.y;
        }
    };

    // MFMA filter of one gathered tile: the 32 x 32 accumulator of filter values.
    // The norm column |p'|^2 is summed here from the row halves of lanes n and
    // n + 32 (the filter's rounding bound holds for any summation order of the
    // norm), which saves a random 4-byte load per candidate row; rows past the
    // tile read as far away.  cand_norm returns the norm (the same on both
    // halves of the wave).
    auto mfma_tile = [&](const Tile& t, float& cand_norm) __attribute__((always_inline)) {
        floatx16 acc;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
        float pn = 0.0f;
#pragma unroll
        for (int j = 0; j < HD; ++j) {
            const float c = centre(t.op[j], j);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(c, bop[j], acc, 0, 0, 0);
            pn = fmaf(c, c, pn);
        }
        unsigned pa, pb;
        xor_pair_u32(__float_as_uint(pn), 32, pa, pb);
        const float nrm = __uint_as_float(pa) + __uint_as_float(pb);
        cand_norm = nrm;
        const float last = lower_half() ? (n < t.count ? nrm : 3.0e38f) : 1.0f;
        return __builtin_amdgcn_mfma_f32_32x32x2f32(last, bop[HD], acc, 0, 0, 0);
    };

    // A hit is a pair (candidate row, query) whose filter value is below the
    // query's threshold (NaN counts as a hit) and whose candidate was streamed
    // for the query's own row segment: stream positions [q_vbeg, q_vend) of
    // this lane's query (empty for invalid queries), clipped to the tile's
    // rows.  That keeps each candidate to one evaluation per query (the
    // neighbourhoods of a wave's segments overlap).  Inside its segment's
    // stream a candidate needs no finer shell test: every pair within the
    // radius lies in the query's 3^g shell (the grid's cell edge covers the
    // radius plus all rounding), so other candidates fail the exact test, and
    // the filter passes them only within its margin of the radius.
    //
    // The 32 x 32 accumulator layout: lane (n, h), register r holds row
    // 8*(r/4) + 4*h + r%4 (the candidate) of column n.  For a tile at stream
    // position v0, rows_of returns this lane's accepted range of rowlo =
    // 8*(r/4) + r%4 as (first, width); hit_in tests register r.
    auto rows_of = [&](int v0, int count, int& first, int& width) __attribute__((always_inline)) {
        const int lo = max(q_vbeg - v0, 0);
        const int hi = min(q_vend - v0, count);
        first = lo - 4 * h;
        width = max(hi - lo, 0);
    };
    auto hit_in = [&](const floatx16& acc, int r, int first, int width) __attribute__((always_inline)) {
        const int rowlo = 8 * (r >> 2) + (r & 3);
        return !(acc[r] >= thr_f) && (unsigned)(rowlo - first) < (unsigned)width;
    };
    // whether any lane's filter values might hold a hit (a cheap first test:
    // the smallest of the 16 values, or always when NaN may occur)
    auto any_hit = [&](const floatx16& acc, bool robust) __attribute__((always_inline)) {
        if (robust) return true;
        float mn = acc[0];
#pragma unroll
        for (int r = 1; r < 16; ++r) mn = fminf(mn, acc[r]);
        return __ballot(qvalid && mn < thr_f) != 0;
    };

    // Tile-exact path: the tile's original indices and raw rows go to LDS,
    // the hits (row << 5 | query) are written register by register at ballot
    // prefix offsets, and they are re-evaluated in rounds of 64 lanes, each
    // round preceded by the compaction of any list that could overflow in it.
    auto hits_tile_exact = [&](const Tile& t, const floatx16& acc, float cand_norm) __attribute__((always_inline)) {
        // the first test only skips work; rows of 4 floats go without it
        // (nearly every one of their tiles holds a hit: C1 -2%, C2 -2%)
        const bool robust = robust_q || (__ballot(n < t.count && !(cand_norm < 1.0e37f)) != 0);
        if (DS > 4 && !any_hit(acc, robust)) return;
        lsync();
        // both halves store the same values
        t_idx[n] = t.idx;
        {
            float* dst = t_rows + n * TS + h * HD;
#pragma unroll
            for (int j = 0; j < HD; ++j) dst[j] = t.op[j];
        }
        const int lane_code = (h << 7) | n;   // (4h << 5) | n
        int first, width;
        rows_of(t.v0, t.count, first, width);
        // fast path: every lane takes all of its rows or none (the tile lies
        // inside or outside each query's segment range and is full)
        const bool whole = (first == -4 * h && width == 32) || width == 0;
        const bool fast = __ballot(!whole) == 0;
        const bool take = width != 0;
        int total = 0;
        // m is the mask of register r's hits (each condition a single
        // compare, combined in scalar registers).  Most registers of a tile
        // with hits have none (about 60% at the headline workload): those
        // skip on a scalar test; otherwise the hit lanes write their entries
        // at the ballot prefix offsets past `total` (the running count is the
        // mbcnt accumulator).
        auto push = [&](int r, unsigned long long m) __attribute__((always_inline)) {
            if (m == 0) return;
            if (__builtin_amdgcn_inverse_ballot_w64(m)) {
                const int pos = (int)__builtin_amdgcn_mbcnt_hi((unsigned)(m >> 32),
                                                               __builtin_amdgcn_mbcnt_lo((unsigned)m, (unsigned)total));
                s_hit[pos] = (unsigned short)(((8 * (r >> 2) + (r & 3)) << 5) + lane_code);
            }
            total += __popcll(m);
        };
        if (fast) {
            const unsigned long long tk = __builtin_amdgcn_ballot_w64(take);
#pragma unroll
            for (int r = 0; r < 16; ++r) push(r, __builtin_amdgcn_ballot_w64(!(acc[r] >= thr_f)) & tk);
        } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int rowlo = 8 * (r >> 2) + (r & 3);
                push(r, __builtin_amdgcn_ballot_w64(!(acc[r] >= thr_f)) &
                            __builtin_amdgcn_ballot_w64((unsigned)(rowlo - first) < (unsigned)width));
            }
        }
        bump(1, total);
        if (total == 0) return;
        lsync();
        for (int base = 0; base < total; base += kWave) {
            make_room();
            bool accepted = false, ovf = false;
            int qn = 0;
            unsigned long long key = 0;
            if (base + lane < total) {
                const int e = s_hit[base + lane];
                qn = e & 31;
                const int row = e >> 5;
                const float d2 = exact_d2<DS, REV>(s_q + qn * RS, t_rows + row * TS);
                key = make_key(d2, t_idx[row]);
                accepted = key < s_thr[qn];
                if (accepted) accept(qn, key, ovf);
            }
            if constexpr (counting) bump(2, __popcll(__ballot(accepted)));
            report_overflow(ovf);
            end_round(accepted, qn, key);
        }
    };

    // Queue path: the tile's hits are queued as (query, sorted position) and
    // re-evaluated 64 at a time from memory.  All hits of the tile are queued
    // first (at most 1024, so the queue never exceeds 63 + 1024 entries); the
    // exact batches run after, when the accumulator registers are no longer
    // live.
    auto hits_queue = [&](const Tile& t, const floatx16& acc, float cand_norm) __attribute__((always_inline)) {
        const bool robust = robust_q || (__ballot(n < t.count && !(cand_norm < 1.0e37f)) != 0);
        // hits are sparse here: first find the groups of four registers that
        // might hold one
        bool gh[4];
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
            if (!robust) {
                const float m = fminf(fminf(acc[4 * g4], acc[4 * g4 + 1]), fminf(acc[4 * g4 + 2], acc[4 * g4 + 3]));
                gh[g4] = qvalid && m < thr_f;
            } else {
                gh[g4] = qvalid;
            }
        }
        if (__ballot(gh[0] || gh[1] || gh[2] || gh[3]) == 0) return;
        lsync();
        if (lower_half()) t_pos[n] = t.pos;
        lsync();
        int first, width;
        rows_of(t.v0, t.count, first, width);
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
            if (__ballot(gh[g4]) == 0) continue;
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const int r = 4 * g4 + rr;
                const bool hr = gh[g4] && hit_in(acc, r, first, width);
                const unsigned long long m = __ballot(hr);
                if (m) {
                    if (hr) {
                        const int row = 8 * g4 + 4 * h + rr;
                        const int s = q_size + (int)__builtin_amdgcn_mbcnt_hi(
                                                  (unsigned)(m >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)m, 0u));
                        if (s < kQueueCap) {
                            s_qn[s] = (unsigned char)n;
                            s_qpos[s] = t_pos[row];
                        }
                    }
                    bump(1, __popcll(m));
                    // entries past the queue's capacity (a logic error) are counted
                    const int over = q_size + __popcll(m) - kQueueCap;
                    if (over > 0) bump(4, min(over, __popcll(m)));
                    q_size += __popcll(m);
                }
            }
        }
        if (q_size > kQueueCap && a.status && first_lane()) a.status[0] = 1u;
        lsync();
        int qs = min(q_size, kQueueCap);
        while (qs >= kBatch) {
            process_batch(qs - kBatch, kBatch, false);
            qs -= kBatch;
        }
    };

    // Stream the available candidates: each tile's MFMA chain is issued first,
    // then the next tile's rows are gathered, so those loads are in flight
    // while the MFMAs run and the current tile's hits are handled.  Every row
    // width takes this order.  (Gathering the next tile only after the
    // consumed runs retire gave rows missing some neighbours at 64- and
    // 128-float rows, although the same index arithmetic checks out on the
    // CPU and adding a check of every gathered position made the misses
    // vanish; that order is not used.)
    auto consume = [&](bool final_pass) __attribute__((always_inline)) {
        int avail = v_total - v_done;
        if (!(avail >= 32 || (final_pass && avail > 0))) return;
        Tile cur;
        gather(v_done, min(32, avail), cur);
        while (true) {
            const int vn = v_done + cur.count;
            const int an = v_total - vn;
            const bool has_next = an >= 32 || (final_pass && an > 0);
            float cand_norm;
            const floatx16 acc = mfma_tile(cur, cand_norm);
            Tile nxt;
            if (has_next) gather(vn, min(32, an), nxt);
            if constexpr (kTileExact) hits_tile_exact(cur, acc, cand_norm);
            else hits_queue(cur, acc, cand_norm);
            bump(3, (unsigned long long)cur.count * kQB);
            v_done = vn;
            while (ring_tail < ring_head &&
                   __builtin_amdgcn_readfirstlane(r_vend[ring_tail & (kRing - 1)]) <= v_done)
                ++ring_tail;
            if (!has_next) break;
            cur = nxt;
        }
    };

    // Append at most one run per lane (in lane order) to the ring.
    auto append_runs = [&](int start, int len) __attribute__((always_inline)) {
        const bool has = len > 0;
        const unsigned long long mask = __ballot(has);
        if (mask == 0) return;
        int incl = has ? len : 0;
#pragma unroll
        for (int o = 1; o < kWave; o <<= 1) {
            const int y = __shfl_up(incl, o);
            if (lane_mask(~((1ull << o) - 1ull))) incl += y;
        }
        // (the stream length is wave-uniform: kept in a scalar register, so
        // the tile loop's control flow stays scalar)
        const int total = __builtin_amdgcn_readfirstlane(__shfl(incl, kWave - 1));
        const int k = __popcll(mask & ((1ull << lane) - 1ull));
        if (has) {
            const int slot = (ring_head + k) & (kRing - 1);
            r_start[slot] = start;
            r_vend[slot] = v_total + incl;
        }
        ring_head += __popcll(mask);
        v_total += total;
        lsync();
    };

    if constexpr (MW) {
        // Brute force, NW waves per workgroup: every wave streams all N points
        // in tiles of 32 centred rows, which the workgroup stages once per tile
        // in LDS (tile t in buffer t & 1).  Each thread loads its share of tile
        // t + 1 into registers before tile t's MFMA chain and stores it after
        // the tile's hits; one workgroup barrier per tile separates the two
        // buffers' uses.  The per-wave hit handling never uses the workgroup
        // barrier, so every wave passes the same barriers (t1 - t0 of them).
        if (qvalid) q_vend = 0x7fffffff;
        constexpr int kRowF4 = DS / 4;                    // float4 per row
        constexpr int kPer = 32 * kRowF4 / (kWave * NW);  // float4 per thread and tile
        static_assert(32 * kRowF4 % (kWave * NW) == 0, "tile loads split evenly");
        const int tid = threadIdx.x;
        // this workgroup's range of the points: tiles [t0, t1)
        const int t0 = (int)blockIdx.y * a.slice_tiles;
        const int t1 = min((a.N + 31) / 32, t0 + a.slice_tiles);
        bump(0, (unsigned long long)nq * (unsigned long long)max(min(a.N, 32 * t1) - 32 * t0, 0));
        float4 pf[kPer];
        auto tile_load = [&](int t) __attribute__((always_inline)) {
#pragma unroll
            for (int k = 0; k < kPer; ++k) {
                const int f = tid + k * kWave * NW;
                const int p = 32 * t + f / kRowF4;
                pf[k] = p < a.N ? *reinterpret_cast<const float4*>(a.frows + (size_t)p * DS + 4 * (f % kRowF4))
                                : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
        };
        auto tile_store = [&](int t) __attribute__((always_inline)) {
            float* buf = bf_tile + (t & 1) * 32 * BRS;
#pragma unroll
            for (int k = 0; k < kPer; ++k) {
                const int f = tid + k * kWave * NW;
                *reinterpret_cast<float4*>(buf + (f / kRowF4) * BRS + 4 * (f % kRowF4)) = pf[k];
            }
        };
        if (t0 < t1) {
            tile_load(t0);
            tile_store(t0);
        }
        __syncthreads();
        for (int t = t0; t < t1; ++t) {
            const bool more = t + 1 < t1;
            if (more) tile_load(t + 1);
            Tile cur;
            cur.v0 = 32 * t;
            cur.count = min(32, a.N - 32 * t);
            cur.pos = cur.v0 + n;
            cur.idx = -1;
            {
                const float* src = bf_tile + (t & 1) * 32 * BRS + n * BRS + h * HD;
#pragma unroll
                for (int j = 0; j < HD; j += 4) {
                    const float4 v = *reinterpret_cast<const float4*>(src + j);
                    cur.op[j] = v.x;
                    cur.op[j + 1] = v.y;
                    cur.op[j + 2] = v.z;
                    cur.op[j + 3] = v.w;
                }
            }
            float cand_norm;
            const floatx16 acc = mfma_tile(cur, cand_norm);
            hits_queue(cur, acc, cand_norm);
            bump(3, nq > 0 ? (unsigned long long)cur.count * kQB : 0ull);
            if (more) tile_store(t + 1);
            __syncthreads();
        }
    } else if constexpr (BF) {
        bump(0, (unsigned long long)nq * a.N);
        if (qvalid) q_vend = 0x7fffffff;
        append_runs(0, first_lane() ? a.N : 0);
        consume(true);
    } else {
        // Grid geometry: a projected frame's axes (first-coordinate plans with
        // D > g), or the raw coordinates on the plan's cells (raw frames and
        // grids without a frame).  Cell ci of axis d spans
        // [org_d + ci h_d, org_d + (ci + 1) h_d]; the binned values of its
        // points lie within slack of that span (edge cells are unbounded
        // outward, as binning clamps) and within margin of the exact
        // projections, so the per-axis gaps below shrink by slack + 2 margin
        // (0 on raw grids).  Frame directions have norm < 1 and are
        // orthonormal up to a shrink, so the gaps lower-bound the distance.
        const Frame* fr = a.frame;
        const bool proj = fr != nullptr && fr->projected != 0;
        const int G = a.G;
        // (wave-uniform values, kept in scalar registers)
        auto su = [](int v) __attribute__((always_inline)) { return __builtin_amdgcn_readfirstlane(v); };
        auto sf = [](float v) __attribute__((always_inline)) {
            return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
        };
        const int res0 = su(fr ? fr->res[0] : a.res);
        const float gh = sf(fr ? fr->h : a.cell);
        const float gh0 = sf(fr ? fr->h0 : a.cell);
        const float ginv0 = sf(fr ? fr->inv_h0 : 0.0f);
        const int fine0 = su(fr ? fr->fine0 : 1);
        const float gsm = sf(fr ? fr->slack + 2.0f * fr->margin : 0.0f);
        if (lane < G) {
            s_res[lane] = fr ? fr->res[lane] : a.res;
            s_stride[lane] = fr ? fr->stride[lane] : a.gstride[lane];
            s_org[lane] = fr ? fr->lo[lane] : 0.0f;
        }
        // this lane's query: grid coordinates (projections or raw values)
        const float* qrow = query_row(qvalid ? n : 0);
        if (proj) {
            float sp[kFrameGrid];
            frame_project(fr, [&](int d) { return qrow[d]; }, sp);
            if (lower_half()) {
#pragma unroll
                for (int d = 0; d < kFrameGrid; ++d)
                    if (d < G) s_qg[n * kGA + d] = sp[d];
            }
        } else if (lower_half()) {
            for (int d = 0; d < G; ++d) s_qg[n * kGA + d] = qrow[d];
        }
        // the query's cell, as binned: x along axis 0, the row as the id of
        // the row's x = 0 cell (rows are non-decreasing in the sorted order)
        int row_n = 0x7fffffff;
        if (qvalid) {
            const int c = a.qcell_of[a.qsorted_idx[q0 + n]];
            x_n = c % res0;
            row_n = c - x_n;
        }
        lsync();
        int nrows = 1;
        for (int d = 1; d < G; ++d) nrows *= 3;
        const float keep = 0.9999847412109375f;   // 1 - 2^-16
        const float eps = 4.76837158203125e-07f;  // 2^-21
        // lower bound of the distance along axis d from the segment's box to
        // cell ci
        auto axis_gap = [&](int d, int ci) __attribute__((always_inline)) -> float {
            float gap = 0.0f;
            const float org = s_org[d];
            const float hd = d == 0 ? gh0 : gh;
            if (ci > 0) {
                const float lo = fmaf((float)ci, hd, org);
                const float bh = s_bhi[d];
                gap = fmaxf(gap, (lo - bh) - eps * (fabsf(lo) + fabsf(bh)));
            }
            if (ci < s_res[d] - 1) {
                const float hi = fmaf((float)(ci + 1), hd, org);
                const float bl = s_blo[d];
                gap = fmaxf(gap, (bl - hi) - eps * (fabsf(hi) + fabsf(bl)));
            }
            return fmaxf(gap - gsm, 0.0f);
        };

        // One loop walks the segments (runs of queries sharing a row) and, per
        // segment, batches of 64 items (one per lane); every iteration appends
        // at most one run per lane and streams what is available, so the tile
        // loop below is inlined once.  Items: on a frame, the 3^(g-1)
        // neighbouring rows, each contributing the stretch of its fine axis-0
        // cells within reach of the segment (one contiguous run); on a grid
        // without a frame, the cells x-1..x+1 around the segment's queries in
        // those rows.
        int seg = 0;
        int ib = 0, NI = 0;
        int xa = 0, nx = 1;
        float thr_seg = 0.0f;
        float thr_out = 0.0f;               // this batch's pass: stretches up to this threshold
        float thr_done = -1.0f;             // ... beyond those of earlier passes (-1: none)
        bool two = false;                   // the segment's rows are walked in kPasses passes
        bool seg_mine = false;              // this lane's query is in the current segment
        bool last = false;
        while (!last) {
            if (ib >= NI && seg < nq) {
                const int R = __builtin_amdgcn_readlane(row_n, seg);
                const bool in_seg = (row_n == R);
                seg_mine = in_seg;
                // the previous segment's stream ends here, this one's starts
                if (q_vend == 0x7fffffff) q_vend = v_total;
                if (in_seg) {
                    q_vbeg = v_total;
                    q_vend = 0x7fffffff;
                }
                const int xlo = wave_min_i32(in_seg ? x_n : 0x7fffffff);
                const int xhi = wave_max_i32(in_seg ? x_n : -1);
                // next segment: the queries past those with row <= R (rows are
                // non-decreasing in the cell-sorted order); at least one step,
                // so every wave terminates even on unsorted input
                seg = max(seg + 1, (int)__popcll(__ballot(row_n <= R) & 0xffffffffull));
                // segment bounding box on the grid axes
                for (int d = 0; d < G; ++d) {
                    const float qd = s_qg[n * kGA + d];
                    const float lo = wave_min_f32(in_seg ? qd : __builtin_huge_valf());
                    const float hi = wave_max_f32(in_seg ? qd : -__builtin_huge_valf());
                    if (first_lane()) {
                        s_blo[d] = lo;
                        s_bhi[d] = hi;
                        s_rc[d] = d > 0 ? (R / s_stride[d]) % s_res[d] : 0;
                    }
                }
                lsync();

                if constexpr (counting) {
                    // the reference's shell candidates of this segment's queries:
                    // the cells x-1..x+1 of edge h (fine0 axis-0 cells each) in
                    // the 3^(g-1) rows
                    long long sh = 0;
                    if (in_seg && lower_half()) {
                        const int xc = x_n / fine0;
                        const int f0 = max(xc - 1, 0) * fine0;
                        const int f1 = min((xc + 2) * fine0, res0) - 1;
                        for (int t = 0; t < nrows; ++t) {
                            int tt = t, Rb = 0;
                            bool ok = true;
                            for (int d = 1; d < G; ++d) {
                                const int cc = s_rc[d] + (tt % 3) - 1;
                                tt /= 3;
                                ok = ok && cc >= 0 && cc < s_res[d];
                                Rb += cc * s_stride[d];
                            }
                            if (!ok) continue;
                            sh += a.start[Rb + f1 + 1] - a.start[Rb + f0];
                        }
                    }
                    bump(0, (unsigned long long)wave_sum_i64(sh));
                }

                xa = max(xlo - 1, 0);
                nx = fr ? 1 : min(xhi + 1, res0 - 1) - xa + 1;
                two = fr && a.inner2 < a.r2;
                NI = two ? kWave * (kPasses - 1) + 2 * nrows : nx * nrows;
                thr_done = -1.0f;
                ib = 0;
            }
            if (ib < NI) {
                // the segment's largest threshold, as tightened by the
                // compactions so far (nothing beyond it can still be accepted)
                thr_seg = wave_max_f32(seg_mine ? key_d2(s_thr[n]) : -__builtin_huge_valf());
                // passes: batch p (items p kWave + ...) is pass p; pass 0
                // takes one item per row, later passes two: the parts of the
                // row's stretch left (side 0) and right (side 1) of what the
                // earlier passes streamed
                const int pass = ib / kWave;
                if (two) thr_out = pass < kPasses - 1 ? fminf(thr_seg, a.inner2) : thr_seg;
                const int item = ib + lane;
                int rowi = item / nx, side = 0;
                bool valid = item < NI;
                if (two) {
                    const int j = item - pass * kWave;
                    rowi = pass == 0 ? j : j >> 1;
                    side = pass == 0 ? 0 : j & 1;
                    valid = rowi < nrows;
                }
                int rs = 0, rl = 0;
                if (valid) {
                    const int x = xa + item % nx;
                    int tt = natural_row(rowi, G - 1), Rb = 0;
                    bool ok = true;
                    float lb = 0.0f;     // squared gaps on axes 1..g-1
                    for (int d = 1; d < G; ++d) {
                        const int cc = s_rc[d] + (tt % 3) - 1;
                        tt /= 3;
                        const bool in = cc >= 0 && cc < s_res[d];
                        ok = ok && in;
                        Rb += cc * s_stride[d];
                        if (in) {
                            const float gp = axis_gap(d, cc);
                            lb = fmaf(gp, gp, lb);
                        }
                    }
                    if (ok && fr) {
                        // the row's stretch: a candidate p within the threshold
                        // of a segment query q has (s0(p) - s0(q))^2 <= |p - q|^2
                        // - (its gaps on the other axes)^2, and |p - q|^2 < thr
                        // (1 + 2^-13) for an fp32 distance below thr, so its
                        // axis-0 projection lies within w of the segment's box
                        // (w adds sqrt's rounding and slack + 2 margin); binning
                        // is monotone in the projection, so the stretch is the
                        // cell range of the window's ends (rounded outward).
                        // Pass p streams the row's stretch at thr_out minus
                        // the stretch at thr_done (the largest threshold of
                        // the passes before it): stretches are monotone in the
                        // threshold, so the passes together cover the stretch
                        // at the segment's final-pass threshold, each
                        // candidate once.
                        auto stretch = [&](float thr, int& f0, int& f1) -> bool {
                            if (lb * keep > thr) return false;
                            const float w2 = fmaxf(thr * 1.0001220703125f - lb * keep, 0.0f);
                            const float w = sqrtf(w2) * 1.00000095367431640625f + gsm;
                            const float bl = s_blo[0], bh = s_bhi[0];
                            const float wl = (bl - w) - eps * (fabsf(bl) + w);
                            const float wh = (bh + w) + eps * (fabsf(bh) + w);
                            f0 = wl == wl ? sub_bin(wl, s_org[0], ginv0, res0) : 0;
                            f1 = wh == wh ? sub_bin(wh, s_org[0], ginv0, res0) : res0 - 1;
                            return true;
                        };
                        int f0 = 1, f1 = 0;
                        if (!two || pass == 0) {
                            if (!stretch(two ? thr_out : thr_seg, f0, f1)) f1 = f0 - 1;
                        } else {
                            int i0 = 0, i1 = 0;
                            const bool inner = thr_done >= 0.0f && stretch(thr_done, i0, i1);
                            if (!stretch(thr_out, f0, f1)) {
                                f1 = f0 - 1;
                            } else if (inner) {
                                if (side == 0) f1 = min(f1, i0 - 1);
                                else f0 = max(f0, i1 + 1);
                            } else if (side == 1) {
                                f1 = f0 - 1;
                            }
                        }
                        if (f0 <= f1) {
                            rs = a.start[Rb + f0];
                            rl = max(a.start[Rb + f1 + 1] - rs, 0);
                        }
                    } else if (ok) {
                        const float gp = axis_gap(0, x);
                        lb = fmaf(gp, gp, lb);
                        const int c = x + Rb;
                        const int cs = a.start[c];
                        const int ce = a.start[c + 1];
                        if (ce > cs && !(lb * keep > thr_seg)) {
                            rs = cs;
                            rl = ce - cs;
                        }
                    }
                }
                append_runs(rs, rl);
                if (two) thr_done = fmaxf(thr_done, thr_out);
                ib += kWave;
            }
            last = ib >= NI && seg >= nq;
            consume(last);
        }
    }

    lsync();
    {
        // the last partial batch, then the final selection of every list
        // (one call site for both keeps a single inlined copy of the sorts)
        const int qs = min(q_size, kQueueCap);
#pragma nounroll
        for (int pass = 0; pass < 2; ++pass) process_batch(0, pass == 0 ? qs : 0, pass == 1);
    }

    if constexpr (counting) {
        lsync();
        if (lane < 5 && (lane != 4 || s_ctr[4] != 0)) atomicAdd(&a.counters[lane], s_ctr[lane]);
    }
}

// The first pass's threshold as a fraction of r^2, by K: the inner ball
// should hold about K points, so that pass sets thresholds near the K-th
// distance.  Measured on the BASELINE configs (ms per call, one pass /
// fraction 0.06 / 0.16): metric (K=64) 3.89 / 3.74 / 3.71, C4 (K=64)
// 6.91 / 6.33 / 6.26, C3 (K=32) 1.80 / 1.34 / 1.43, C2 (K=32) 1.61 / 1.46 /
// 1.50, C1 (K=16) 0.30 / 0.31 / 0.31.
static float inner_frac2(int K) {
    if (K <= 16) return kK16Frac2;
    return K <= 32 ? 0.06f : 0.16f;
}

static unsigned f32_bits(float f) {
    unsigned u;
    std::memcpy(&u, &f, sizeof(u));
    return u;
}

// Waves per workgroup of brute force on wide rows (the waves share each
// candidate tile through LDS); every other path runs one-wave workgroups.
constexpr int kBFWaves = 4;

// Merge after brute force split over point ranges: row q of range 0 gets the
// K smallest keys of rows q of ranges 0..S-1.  Each of those holds its range's
// K smallest keys, ascending, padded with (r2, -1) (larger than every key
// within the radius), so their union holds the K smallest overall.  One wave
// per query, one pairwise bitonic merge per range: C[i] = min(X[i], Y[P-1-i])
// (P = 64 EK) is bitonic and holds the P smallest of both, and the
// half-cleaners sort it.
template <int EK>
__global__ __launch_bounds__(256) void merge_ranges_kernel(unsigned long long* __restrict__ lists, int cap, int M,
                                                           int K, int S) {
    const int lane = threadIdx.x & (kWave - 1);
    const int q = (int)blockIdx.x * 4 + (int)(threadIdx.x / kWave);
    if (q >= M) return;
    unsigned long long* L0 = lists + (size_t)q * cap;
    unsigned long long x[EK];
#pragma unroll
    for (int e = 0; e < EK; ++e) {
        const int i = e * kWave + lane;
        x[e] = i < K ? L0[i] : ~0ull;
    }
    for (int r = 1; r < S; ++r) {
        const unsigned long long* Lr = lists + ((size_t)r * M + q) * cap;
        unsigned long long y[EK];
#pragma unroll
        for (int e = 0; e < EK; ++e) {
            const int i = e * kWave + lane;
            y[e] = i < K ? Lr[i] : ~0ull;
        }
#pragma unroll
        for (int e = 0; e < EK; ++e) {
            const unsigned long long rb = shfl_u64(y[EK - 1 - e], kWave - 1 - lane);
            x[e] = x[e] < rb ? x[e] : rb;
        }
        wave_bitonic_merge_u64<EK>(x);
    }
#pragma unroll
    for (int e = 0; e < EK; ++e) {
        const int i = e * kWave + lane;
        if (i < K) L0[i] = x[e];
    }
}

template <int DS, bool REV, bool BF>
static void launch_one(const SearchArgs& a, hipStream_t s) {
    constexpr int NW = (BF && DS >= 64) ? kBFWaves : 1;
    const dim3 grid((a.nchunks + NW - 1) / NW, NW > 1 ? a.slices : 1), block(kWave * NW);
    if (a.counters)
        hipLaunchKernelGGL((search_kernel<DS, REV, BF, true, NW>), grid, block, 0, s, a);
    else
        hipLaunchKernelGGL((search_kernel<DS, REV, BF, false, NW>), grid, block, 0, s, a);
}

template <int DS>
static void launch_ds(const SearchArgs& a, bool bf, hipStream_t s) {
    if (bf) launch_one<DS, false, true>(a, s);
    else launch_one<DS, false, false>(a, s);
}

// Point ranges for brute force on wide rows.  Every (query block, range)
// workgroup streams the same number of tiles, so the kernel runs in whole
// rounds of the device's resident workgroups; with too few blocks for the last
// round, most of the device idles through it.  Splitting the points into S
// ranges gives S times as many shorter workgroups: S is the smallest count
// (at most 8) whose rounds are at least 97% full, else the fullest.  Each
// range keeps its own K keys per query (more accepted keys, one more merge
// step per range), which the fuller rounds outweigh: C5 (1 563 workgroups, 512
// resident) 104.0 ms at S = 3 (92% full), 101.7 at S = 5 (95%), 101.2 at S = 7.
static int resident_bf_blocks(int DS) {
    static int cached[2] = {0, 0};
    const int k = DS >= 128 ? 1 : 0;
    if (cached[k] > 0) return cached[k];
    int dev = 0, cus = 0, per = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    hipError_t e = DS >= 128
        ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, search_kernel<128, false, true, false, kBFWaves>,
                                                       kWave * kBFWaves, 0)
        : hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, search_kernel<64, false, true, false, kBFWaves>,
                                                       kWave * kBFWaves, 0);
    if (e != hipSuccess || per < 1) {
        (void)hipGetLastError();
        return 0;
    }
    cached[k] = cus * per;
    return cached[k];
}

int search_ranges(const frnn_plan_t& plan, int D, int N, int M) {
    if (plan.path != FRNN_PATH_BRUTEFORCE || aos_stride(D) < 64 || N <= 0 || M <= 0) return 1;
    const long long slots = resident_bf_blocks(aos_stride(D));
    if (slots <= 0) return 1;
    const long long blocks = ((long long)(M + kQB - 1) / kQB + kBFWaves - 1) / kBFWaves;
    const int tiles = (N + 31) / 32;
    int best = 1;
    double best_fill = 0.0;
    for (int S = 1; S <= 8 && S <= tiles; ++S) {
        const long long units = blocks * S;
        const long long rounds = (units + slots - 1) / slots;
        const double fill = (double)units / (double)(rounds * slots);
        if (fill >= 0.97) return S;
        if (fill > best_fill + 1e-9) {
            best_fill = fill;
            best = S;
        }
    }
    return best;
}

int launch_search(const float* aos, const float* frows, const void* stats_ws, const int* sorted_idx,
                  const int* cell_of, const int* start, const void* frame_ws, int N, int D, int K,
                  const frnn_plan_t& plan, unsigned long long* lists, int cap, unsigned long long* counters,
                  unsigned* status, hipStream_t s, const QuerySet* queries, int ranges) {
    if (N <= 0) return 0;
    const bool bf = plan.path == FRNN_PATH_BRUTEFORCE;
    const QuerySet self{aos, frows, sorted_idx, cell_of, N};
    const QuerySet& Q = queries ? *queries : self;
    if (Q.M <= 0) return 0;
    if (!Q.aos || (!bf && (!Q.sorted_idx || !Q.cell_of)) || (uses_filter_rows(D) && !Q.frows)) return 1;
    if (!bf && (plan.grid_dim < 1 || plan.grid_dim > kMaxG || !sorted_idx || !cell_of || !start)) return 1;
    if (!bf && frame_ws && plan.grid_dim > kFrameGrid) return 1;
    if (!bf && aos_stride(D) >= 16 && plan.grid_dim > kFrameGrid) return 1;   // kernels size s_qg for g <= 4
    // a list must hold the K results; below list_capacity(K) a round can
    // overflow it, which the capacity guard reports through `status`
    if (K < 1 || cap < K || K > FRNN_MAX_K || !stats_ws || D < 1 || D > FRNN_MAX_DIM) return 1;
    if (uses_filter_rows(D) && !frows) return 1;
    SearchArgs a{};
    a.pts = aos;
    a.frows = frows;
    a.st = reinterpret_cast<const DimStat*>(static_cast<const char*>(stats_ws) + stats_layout(D).dims);
    a.D = D;
    a.sorted_idx = sorted_idx;
    a.cell_of = cell_of;
    a.start = start;
    a.qpts = Q.aos;
    a.qfrows = Q.frows;
    a.qsorted_idx = Q.sorted_idx;
    a.qcell_of = Q.cell_of;
    a.lists = lists;
    a.counters = counters;
    a.status = status;
    a.N = N;
    a.M = Q.M;
    a.K = K;
    a.cap = cap;
    a.room = min(cap, kMaxRoom);
    // the histogram's lowest bucket edge stays positive unless r2 < 2^-123
    a.r2bits = f32_bits(plan.r2);
    // (at K <= 16 the lists rarely fill, and the histogram upkeep after every
    // exact round costs more than its tighter thresholds save: C1 0.30 ->
    // 0.28 ms, the reference's K=16 sweep cells 3-4% faster without it)
    a.hist_shift = K <= 32 ? 21 : 20;
    a.hist_on = (K > 16 && a.r2bits >= ((unsigned)kHB << a.hist_shift)) ? 1 : 0;
    a.exact_limit = (K + a.room - kBatch) / 2;
    a.G = bf ? 0 : plan.grid_dim;
    a.res = bf ? 1 : plan.res;
    {
        long long st = 1;
        for (int d = 0; d < kMaxG; ++d) {
            a.gstride[d] = (int)st;
            if (d < a.G) st *= a.res;
            if (st > FRNN_MAX_CELLS) st = FRNN_MAX_CELLS;
        }
    }
    a.r2 = plan.r2;
    a.inner2 = inner_frac2(K) * plan.r2;
    const int DS = aos_stride(D);
    a.cell = bf ? 1.0f : plan.cell_size;
    a.radius = plan.cell_size;
    if (frame_ws && !bf) {
        a.frame = reinterpret_cast<const Frame*>(static_cast<const char*>(frame_ws) + frame_layout().frame);
    }
    const double u = 5.9604644775390625e-08;   // 2^-24
    a.norm_scale = (float)(1.0 - (6.0 * DS + 32.0) * u);
    a.thr_rel = (float)(2.0 * (DS + 8.0) * u);
    a.thr_abs = 1.0e-35f;
    a.nchunks = (Q.M + kQB - 1) / kQB;
    // point ranges (brute force on wide rows only)
    a.slices = (bf && DS >= 64) ? max(1, min(ranges, 8)) : 1;
    a.slice_tiles = ((N + 31) / 32 + a.slices - 1) / a.slices;
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
    if (a.slices > 1) {
        const int rc = launch_result();
        if (rc != 0) return rc;
        const dim3 mgrid((Q.M + 3) / 4), mblock(256);
        if (K <= kWave) hipLaunchKernelGGL(merge_ranges_kernel<1>, mgrid, mblock, 0, s, lists, cap, Q.M, K, a.slices);
        else hipLaunchKernelGGL(merge_ranges_kernel<2>, mgrid, mblock, 0, s, lists, cap, Q.M, K, a.slices);
    }
    return launch_result();
}

}  // namespace frnn
