// range_scan.hip -- RaBitQ range-posting scan over posting segments and the
// per-query segment merge on gfx950.
//
// Reference: range_posting_rabitq_scan_kernel (src/search/rabitq/
// backend_rabitq.cu:5846-6015), posting_segments::merge_one_query /
// merge_shortlists (src/search/common/posting_segment_merge.cuh:12-61) and
// the host segment plan posting_segments::make_plan (src/execution/
// posting_segment_plan.h:20-51, implemented in range_posting.cpp).
//
// Segment s scans the sample ids posting[offsets[s] .. + sizes[s]) (clipped
// to resident_rows) for route route_ids[s].  A row is skipped when its
// sample is >= base_rows or the route has no active range.  Filter-first: an
// enabled predicate decides; otherwise, with more than one active range,
// every active range must match (the posting slice already satisfies one);
// a single active range passes by construction.  Score-first (requested and
// the predicate enabled): the predicate is consulted only for rows that can
// enter the shortlist.  Pass counts: filter-first counts every row that
// passes the filter; score-first counts the rows that could enter the heap
// at their scan position and matched.
//
// One 256-thread workgroup per segment.  A chunk of rows is scored in
// parallel into LDS at its scan positions; rows whose (distance, id) is not
// below the running k-th pair are dropped at once (they could not enter the
// heap).  The survivors are merged into the running top-k: with none the
// chunk costs nothing more, with at most k_pow2 they are sorted on their
// own and bitonic-merged with the running list, otherwise the whole LDS
// region is sorted.  The running list is the k least admissible pairs of
// the rows scanned so far -- the multiset the reference heap holds -- so the
// ascending output equals the reference heap sorted.
//
// Score-first pass counts: a row enters the reference heap iff fewer than k
// admitted rows before it are <= it in (distance, id) order.  Rows of
// earlier chunks are counted by binary search in the running list (only its
// first k matter), rows earlier in the same chunk by a scan of the
// survivors before it (a dropped row is larger than every survivor).
//
// Merge: output row p takes the segments [query_indptr[p], [p+1]); each
// segment's sorted list is bitonic-merged into the running top-k (skipped
// when its best pair cannot enter) and the pass counts are summed, as
// merge_one_query's heap inserts do.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cfloat>
#include <cstdint>

#include "device_common.hpp"
#include "gofann_internal.hpp"
#include "scan_common.hpp"

namespace gofann {

constexpr int kRangeMaxShortlist = 4096;  // max_range_posting_postfilter_shortlist

struct RangeScanArgs {
    gofann_predicate_view pred;
    gofann_routes routes;  // route_query + the query range table
    const uint32_t* posting;
    uint64_t resident_rows;
    const uint32_t* seg_route;
    const uint64_t* seg_offset;
    const uint64_t* seg_size;
    uint32_t segments;
    uint32_t base_rows;
    int k;
    int k_pow2;
    int slots;        // LDS pairs, a power of two >= k_pow2 + chunk and >= 2 k_pow2
    int chunk;        // rows scored per pass: 1024 or 2048 (4 or 8 per thread)
    uint32_t planes_bytes;
    int score_first;
    uint32_t* out_ids;
    float* out_dists;
    uint32_t* pass_counts;
    // Label-posting modes (group-per-row kernel only); the rows are
    // filtered by the route predicate alone and counted when it is enabled.
    // kLabelSlices: segment s is slice s % slices of route s / slices over
    // cand_ids[cand_offsets[route] .. + cand_sizes[route]).  kLabelSegments:
    // segment s scans posting[seg_offset[s] .. + seg_size[s]) (clipped to
    // resident_rows) for route seg_route[s].
    int label_mode;
    const uint32_t* cand_offsets;
    const uint32_t* cand_sizes;
    uint32_t slices;
    // Posting-order copies of the rows (group kernel; may be null): codes
    // [rows][padded_dim/8] and aux [rows] = {f_add, f_rescale, anchor, 0}.
    // Row r of the posting is read from them, not gathered.
    const uint4* pcodes;
    const uint4* paux;
    // Posting-order predicate columns (label modes; may be null): the
    // row's label slab and its base range row [rows][range_columns(pred)].
    const uint4* pslab;
    const float* pranges;
};

constexpr int kRangeMode = 0;
constexpr int kLabelSlices = 1;
constexpr int kLabelSegments = 2;

// pred_matches for a posting row whose label slab and range row were read
// in posting order: the same clause walk, each label test the serial scan
// of pred_contains over the slab's labels (the first label >= handle
// decides).  The slab must not be the overflow form.
// `prange` is the row's range row; with one attribute column its value is
// passed as `r0`, loaded with the slab.
__device__ __forceinline__ bool slab_pred_matches(const gofann_predicate_view& v, uint32_t route,
                                                  uint32_t sample, const uint4& slab,
                                                  const float* prange, float r0)
{
    if (sample >= v.rows) return false;
    const uint32_t n = slab_count(slab);
    auto contains = [&](uint32_t handle) {
        if (v.csr_offsets == nullptr) return false;
        for (uint32_t k = 0; k < n; ++k) {
            const uint32_t label = slab_label(slab, k);
            if (label >= handle) return label == handle;
        }
        return false;
    };
    if (v.clauses) {
        for (uint32_t i = v.route_offsets[route]; i < v.route_offsets[route + 1]; ++i) {
            const gofann_clause cl = v.clauses[i];
            bool pass = true;
            for (uint32_t j = cl.label_begin; pass && j < cl.label_end; ++j)
                pass = contains(v.route_handles[j]);
            for (uint32_t j = cl.range_begin; pass && j < cl.range_end; ++j) {
                const gofann_range_atom a = v.ranges[j];
                pass = v.base_ranges != nullptr && a.dimension < range_columns(v) &&
                       range_matches(a.mode, a.lower, a.upper,
                                     !prange ? v.base_ranges[static_cast<uint64_t>(sample) *
                                                                 v.range_stride +
                                                             a.dimension]
                                     : range_columns(v) == 1 ? r0
                                                           : prange[a.dimension]);
            }
            if (pass) return true;
        }
        return false;
    }
    for (uint32_t i = v.route_offsets[route]; i < v.route_offsets[route + 1]; ++i)
        if (!contains(v.route_handles[i])) return false;
    return true;
}

__device__ __forceinline__ bool pair_le(float ad, uint32_t aid, float bd, uint32_t bid)
{
    return !pair_less(bd, bid, ad, aid);
}

// Entries of the ascending list (d, id)[0, n) that are <= (x, xid).
__device__ __forceinline__ int count_le(const float* d, const uint32_t* id, int n, float x,
                                        uint32_t xid)
{
    int lo = 0, hi = n;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (pair_le(d[mid], id[mid], x, xid))
            lo = mid + 1;
        else
            hi = mid;
    }
    return lo;
}

// Bitonic merge of [0, n): the first half ascending, the second half
// non-increasing; result ascending.
__device__ inline void bitonic_merge(float* d, uint32_t* id, int n, int tid, int nthreads)
{
    for (int stride = n >> 1; stride > 0; stride >>= 1) {
        for (int i = tid; i < n / 2; i += nthreads) {
            const int lo = 2 * i - (i & (stride - 1));
            const int hi = lo + stride;
            if (pair_less(d[hi], id[hi], d[lo], id[lo])) {
                const float td = d[lo];
                d[lo] = d[hi];
                d[hi] = td;
                const uint32_t ti = id[lo];
                id[lo] = id[hi];
                id[hi] = ti;
            }
        }
        __syncthreads();
    }
}

// Sort [base, base + n) descending (n a power of two).
__device__ inline void bitonic_sort_desc(float* d, uint32_t* id, int base, int n, int tid,
                                         int nthreads)
{
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = tid; i < n / 2; i += nthreads) {
                const int lo = base + 2 * i - (i & (stride - 1));
                const int hi = lo + stride;
                const bool descending = ((lo - base) & size) == 0;
                const bool swap = descending ? pair_less(d[lo], id[lo], d[hi], id[hi])
                                             : pair_less(d[hi], id[hi], d[lo], id[lo]);
                if (swap) {
                    const float td = d[lo];
                    d[lo] = d[hi];
                    d[hi] = td;
                    const uint32_t ti = id[lo];
                    id[lo] = id[hi];
                    id[hi] = ti;
                }
            }
            __syncthreads();
        }
    }
}

__device__ __forceinline__ int pow2_ceil(int x)
{
    int p = 1;
    while (p < x) p <<= 1;
    return p;
}

__global__ __launch_bounds__(kScanThreads) void range_scan_kernel(RangeScanArgs a,
                                                                  RabitqScanScorer sc)
{
    extern __shared__ __align__(16) unsigned char lds[];
    __shared__ uint32_t s_surv;
    __shared__ uint32_t s_pass;
    __shared__ uint32_t s_slot;
    const int tid = static_cast<int>(threadIdx.x);
    const uint32_t seg = blockIdx.x;
    if (seg >= a.segments) return;
    float* s_d = reinterpret_cast<float*>(lds + a.planes_bytes);
    uint32_t* s_id = reinterpret_cast<uint32_t*>(s_d + a.slots);

    const uint32_t route = a.seg_route[seg];
    sc.setup(a.routes.route_query[route], tid, lds);
    for (int i = tid; i < a.slots; i += kScanThreads) {
        s_d[i] = FLT_MAX;
        s_id[i] = UINT32_MAX;
    }
    if (tid == 0) s_pass = 0;

    // :5895-5902
    const uint64_t begin = a.seg_offset[seg];
    uint64_t count = a.seg_size[seg];
    if (begin > a.resident_rows)
        count = 0;
    else if (count > a.resident_rows - begin)
        count = a.resident_rows - begin;
    const uint32_t active = count_active_ranges(a.routes.range_modes, route, a.routes.range_count);
    if (active == 0) count = 0;  // :5917
    const bool enabled = pred_enabled(a.pred, route);
    const bool score_first = a.score_first != 0 && enabled;
    const int k = a.k, kp = a.k_pow2;
    const int chunk = a.chunk;
    uint32_t passes = 0;
    uint32_t surv_total = 0;  // s_surv only grows: a chunk's survivors are its increment
    if (tid == 0) s_surv = 0;
    __syncthreads();

    for (uint64_t base = 0; base < count; base += static_cast<uint64_t>(chunk)) {
        // Every read of the previous chunk (s_surv included) ends here, before
        // this chunk's survivors are counted into s_surv.
        __syncthreads();
        const float kth_d = s_d[k - 1];
        const uint32_t kth_id = s_id[k - 1];
        uint32_t surv = 0;
        for (int i = tid; i < chunk; i += kScanThreads) {
            const uint64_t j = base + static_cast<uint64_t>(i);
            float d = FLT_MAX;
            uint32_t id = UINT32_MAX;
            if (j < count) {
                const uint32_t s = a.posting[begin + j];
                bool ok = s < a.base_rows;
                if (ok) {
                    if (enabled) {
                        PredCounters c{0, 0};
                        ok = pred_matches(a.pred, route, s, c);
                    } else if (active > 1) {
                        ok = count_matching_ranges(a.routes, route, s) == active;
                    }
                }
                if (ok) {
                    if (!score_first) ++passes;
                    const float v = sc.score(s);
                    if (admissible(v, s) && pair_less(v, s, kth_d, kth_id)) {
                        d = v;
                        id = s;
                        ++surv;
                    }
                }
            }
            s_d[kp + i] = d;
            s_id[kp + i] = id;
        }
        if (surv) atomicAdd(&s_surv, surv);
        __syncthreads();
        const uint32_t now = s_surv;
        const int m = static_cast<int>(now - surv_total);
        surv_total = now;
        if (m == 0) continue;  // uniform: nothing can enter
        if (score_first) {
            for (int i = tid; i < chunk; i += kScanThreads) {
                const uint32_t xid = s_id[kp + i];
                if (xid == UINT32_MAX) continue;
                const float x = s_d[kp + i];
                int c = count_le(s_d, s_id, k, x, xid);
                for (int j = 0; j < i && c < k; ++j)
                    if (s_id[kp + j] != UINT32_MAX && pair_le(s_d[kp + j], s_id[kp + j], x, xid)) ++c;
                if (c < k) ++passes;
            }
            __syncthreads();  // the counts read LDS that the merge below reorders
        }
        const int mp = pow2_ceil(m);
        if (mp <= kp) {
            // Gather the survivors at the tail of [kp, 2kp), sort them
            // descending, then merge with the ascending running list.
            float keep_d[8];
            uint32_t keep_id[8];
            int nk = 0;
            const int per = chunk / kScanThreads;  // 4 or 8 (see the launcher)
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const int i = tid + t * kScanThreads;
                keep_d[t] = t < per ? s_d[kp + i] : FLT_MAX;
                keep_id[t] = t < per ? s_id[kp + i] : UINT32_MAX;
                nk += keep_id[t] != UINT32_MAX ? 1 : 0;
            }
            if (tid == 0) s_slot = 0;
            __syncthreads();
            for (int i = tid; i < kp; i += kScanThreads) {
                s_d[kp + i] = FLT_MAX;
                s_id[kp + i] = UINT32_MAX;
            }
            __syncthreads();
            if (nk) {
                uint32_t at = atomicAdd(&s_slot, static_cast<uint32_t>(nk));
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    if (keep_id[t] == UINT32_MAX) continue;
                    const int pos = 2 * kp - mp + static_cast<int>(at++);
                    s_d[pos] = keep_d[t];
                    s_id[pos] = keep_id[t];
                }
            }
            __syncthreads();
            bitonic_sort_desc(s_d, s_id, 2 * kp - mp, mp, tid, kScanThreads);
            bitonic_merge(s_d, s_id, 2 * kp, tid, kScanThreads);
        } else {
            bitonic_sort(s_d, s_id, a.slots, tid, kScanThreads);
        }
    }
    if (passes) atomicAdd(&s_pass, passes);
    __syncthreads();
    for (int i = tid; i < k; i += kScanThreads) {
        a.out_ids[static_cast<size_t>(seg) * k + i] = s_id[i];
        a.out_dists[static_cast<size_t>(seg) * k + i] = s_d[i];
    }
    if (tid == 0 && a.pass_counts) a.pass_counts[seg] = s_pass;
}

// ---------------------------------------------------------------------------
// Group-per-row scan.  A group of G lanes (G a power of two, <= 32) scores
// one code row: lane l of the group owns the 16-byte code vectors l, l + G,
// .. of the row (W of them, padded_dim / 128 = G * W), so one wave load
// reads 64 / G whole rows; the query bit planes are read from LDS.  The
// group's partial inner products are summed by a DPP butterfly.  Each
// chunk is first passed over one row per thread: the
// posting id, the filter, and the row's distance terms that need no code
// bits (f_add + g, f_rescale) are gathered into LDS; filter-first packs the
// passing rows (the shortlist does not depend on scan order), score-first
// keeps scan positions for its pass counts.  The group pass leaves only
// the integer inner product in LDS; a third pass, one row per thread again,
// forms the distance and drops rows that cannot beat the running k-th pair
// (lane-0 work inside the group pass would cost whole-wave issue per row).
// ---------------------------------------------------------------------------

// Rows in flight per group in the score pass (a build-time tuning knob).
#ifndef GOFANN_SCAN_ROW_UNROLL
#define GOFANN_SCAN_ROW_UNROLL 8
#endif
constexpr int kRowUnroll = GOFANN_SCAN_ROW_UNROLL;

// This lane's share of sum_d q8[d] * bit[d] over its W code vectors:
// sum_j 2^j popc(plane_j & code) for the seven low planes, minus 128 times
// the sign plane's count.  The planes sit in LDS plane-major,
// planes_t[j][word], so the lane's four words of plane j are one 16-byte
// read and a group's lanes read consecutive 16-byte blocks (no bank
// conflicts); registers stay free for rows in flight.
template <int G, int W>
__device__ __forceinline__ int lane_ip_lds(const uint4 (&c)[W], const uint4* planes_t,
                                           uint32_t vecs, int lg)
{
    uint32_t cnt[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int w = 0; w < W; ++w) {
        const uint32_t v = static_cast<uint32_t>(lg + G * w);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint4 p = planes_t[j * vecs + v];
            cnt[j] = bcnt_acc(p.x & c[w].x, cnt[j]);
            cnt[j] = bcnt_acc(p.y & c[w].y, cnt[j]);
            cnt[j] = bcnt_acc(p.z & c[w].z, cnt[j]);
            cnt[j] = bcnt_acc(p.w & c[w].w, cnt[j]);
        }
    }
    int ip = 0;
#pragma unroll
    for (int j = 0; j < 7; ++j) ip += static_cast<int>(cnt[j]) << j;
    return ip - 128 * static_cast<int>(cnt[7]);
}

template <int G, int W>
__global__ __launch_bounds__(kScanThreads) void range_scan_group_kernel(RangeScanArgs a,
                                                                        RabitqScanScorer sc)
{
    extern __shared__ __align__(16) unsigned char lds[];
    __shared__ uint32_t s_surv;
    __shared__ uint32_t s_rows;
    __shared__ uint32_t s_pass;
    __shared__ uint32_t s_slot;
    const int tid = static_cast<int>(threadIdx.x);
    const uint32_t seg = blockIdx.x;
    if (seg >= a.segments) return;
    float* s_d = reinterpret_cast<float*>(lds + a.planes_bytes);
    uint32_t* s_id = reinterpret_cast<uint32_t*>(s_d + a.slots);
    float* s_f1 = reinterpret_cast<float*>(s_id + a.slots);
    int* s_ip = reinterpret_cast<int*>(s_f1 + a.chunk);
    uint32_t* s_prow = reinterpret_cast<uint32_t*>(s_ip + a.chunk);  // segment-relative row

    const bool label_mode = a.label_mode != kRangeMode;
    const uint32_t route = a.label_mode == kLabelSlices ? seg / a.slices : a.seg_route[seg];
    const uint32_t query = a.routes.route_query[route];
    sc.setup(query, tid, lds);
    for (int i = tid; i < a.slots; i += kScanThreads) {
        s_d[i] = FLT_MAX;
        s_id[i] = UINT32_MAX;
    }
    if (tid == 0) {
        s_pass = 0;
        s_surv = 0;
        s_rows = 0;
    }
    __syncthreads();
    constexpr int kGroups = kScanThreads / G;
    const int lg = tid & (G - 1);
    const int grp = tid / G;
    // plane-major copy of the word-major planes sc.setup wrote
    const uint32_t words = sc.padded_dim / 32;
    uint32_t* planes_t = reinterpret_cast<uint32_t*>(s_prow + a.chunk);
    for (uint32_t e = tid; e < words * 8; e += kScanThreads)
        planes_t[(e & 7) * words + (e >> 3)] = sc.planes[e];
    __syncthreads();
    const uint4* planes_t4 = reinterpret_cast<const uint4*>(planes_t);
    const uint32_t vecs = words / 4;
    const uint4* codes = reinterpret_cast<const uint4*>(sc.codes);
    const size_t row_vecs = static_cast<size_t>(G) * W;

    uint64_t begin, count;
    uint32_t active = 0;
    if (a.label_mode == kLabelSlices) {
        // near-equal slices of the route's posting
        const uint64_t size = a.cand_sizes[route];
        const uint64_t part = (size + a.slices - 1) / a.slices;
        const uint64_t lo = std::min<uint64_t>(size, (seg % a.slices) * part);
        begin = static_cast<uint64_t>(a.cand_offsets[route]) + lo;
        count = std::min<uint64_t>(size, lo + part) - lo;
    } else if (a.label_mode == kLabelSegments) {
        begin = a.seg_offset[seg];
        count = a.seg_size[seg];
        if (begin > a.resident_rows)
            count = 0;
        else if (count > a.resident_rows - begin)
            count = a.resident_rows - begin;
    } else {
        // :5895-5902
        begin = a.seg_offset[seg];
        count = a.seg_size[seg];
        if (begin > a.resident_rows)
            count = 0;
        else if (count > a.resident_rows - begin)
            count = a.resident_rows - begin;
        active = count_active_ranges(a.routes.range_modes, route, a.routes.range_count);
        if (active == 0) count = 0;  // :5917
    }
    const bool enabled = pred_enabled(a.pred, route);
    const bool score_first = !label_mode && a.score_first != 0 && enabled;
    const bool cols = label_mode && enabled && a.pslab != nullptr;
    const int k = a.k, kp = a.k_pow2;
    const int chunk = a.chunk;
    const int per = chunk / kScanThreads;
    uint32_t passes = 0;
    uint32_t surv_total = 0;  // s_surv and s_rows only grow: a chunk's count is the increment
    uint32_t rows_total = 0;

    for (uint64_t base = 0; base < count; base += static_cast<uint64_t>(chunk)) {
        // Every read of the previous chunk ends here.
        __syncthreads();
        const float kth_d = s_d[k - 1];
        const uint32_t kth_id = s_id[k - 1];
        // Pass 1, one row per thread: posting id, filter, code-free terms,
        // in three rounds so that each round's loads are in flight together:
        // (1) sample ids and, with posting-order columns, the label slab
        // and range value; (2) the filter and the passing rows' aux terms;
        // (3) the LDS writes.
        uint32_t sv[8];
        uint4 slv[8];
        float r0v[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            sv[t] = UINT32_MAX;
            slv[t] = make_uint4(kSlabOverflow, 0, 0, 0);
            r0v[t] = 0.0f;
            if (t >= per) continue;
            const uint64_t j = base + static_cast<uint64_t>(tid + t * kScanThreads);
            if (j < count) {
                sv[t] = a.posting[begin + j];
                if (cols) {
                    slv[t] = a.pslab[begin + j];
                    if (a.pranges && range_columns(a.pred) == 1) r0v[t] = a.pranges[begin + j];
                }
            }
        }
        bool okv[8];
        float add0v[8], f1v[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            okv[t] = false;
            add0v[t] = FLT_MAX;
            f1v[t] = 0.0f;
            if (t >= per) continue;
            const uint64_t j = base + static_cast<uint64_t>(tid + t * kScanThreads);
            const uint32_t s = sv[t];
            bool ok = j < count && s < a.base_rows;  // UINT32_MAX never is
            if (ok) {
                if (cols && slab_count(slv[t]) != kSlabOverflow) {
                    const float* prange =
                        a.pranges && range_columns(a.pred) > 0
                            ? a.pranges + (begin + j) * range_columns(a.pred)
                            : nullptr;
                    ok = slab_pred_matches(a.pred, route, s, slv[t], prange, r0v[t]);
                } else if (enabled) {
                    PredCounters c{0, 0};
                    ok = pred_matches(a.pred, route, s, c);
                } else if (active > 1) {
                    ok = count_matching_ranges(a.routes, route, s) == active;
                }
            }
            okv[t] = ok;
            if (ok) {
                if (a.paux) {
                    const uint4 x = a.paux[begin + j];
                    add0v[t] = __uint_as_float(x.x) + sc.g_row[x.z];
                    f1v[t] = __uint_as_float(x.y);
                } else {
                    const uint32_t anchor = sc.anchor_ids[s];
                    add0v[t] = sc.factors[static_cast<size_t>(s) * 3] + sc.g_row[anchor];
                    f1v[t] = sc.factors[static_cast<size_t>(s) * 3 + 1];
                }
            }
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            if (t >= per) break;
            const int i = tid + t * kScanThreads;
            const uint64_t j = base + static_cast<uint64_t>(i);
            const bool ok = okv[t];
            // filter-first counts every passing row; a label posting
            // (backend_rabitq.cu:5494-5682) only predicate-checked ones
            if (ok && (label_mode ? enabled : !score_first)) ++passes;
            int pos = i;
            if (!score_first) {
                // pack the passing rows: a wave reserves its slots at once
                const uint64_t mask = __ballot(ok);
                uint32_t first = 0;
                if (__lane_id() == __ffsll(static_cast<unsigned long long>(mask)) - 1)
                    first = atomicAdd(&s_rows, static_cast<uint32_t>(__popcll(mask)));
                first = __shfl(first, __ffsll(static_cast<unsigned long long>(mask)) - 1, 64);
                pos = static_cast<int>(first - rows_total) +
                      __popcll(mask & ((1ull << __lane_id()) - 1ull));
            }
            if (ok || score_first) {
                s_id[kp + pos] = ok ? sv[t] : UINT32_MAX;
                s_d[kp + pos] = add0v[t];
                s_f1[pos] = f1v[t];
                s_prow[pos] = static_cast<uint32_t>(j);
            }
        }
        __syncthreads();
        int n_rows;
        if (score_first) {
            const uint64_t left = count - base;
            n_rows = left < static_cast<uint64_t>(chunk) ? static_cast<int>(left) : chunk;
        } else {
            const uint32_t now = s_rows;
            n_rows = static_cast<int>(now - rows_total);
            rows_total = now;
        }
        for (int i = n_rows + tid; i < chunk; i += kScanThreads) {
            s_d[kp + i] = FLT_MAX;
            s_id[kp + i] = UINT32_MAX;
        }
        // Pass 2, a group per row: the code bits' integer inner product.
        for (int i0 = grp; i0 < n_rows; i0 += kGroups * kRowUnroll) {
            uint32_t sid[kRowUnroll];
            uint4 c[kRowUnroll][W];
#pragma unroll
            for (int u = 0; u < kRowUnroll; ++u) {
                const int i = i0 + u * kGroups;
                sid[u] = i < n_rows ? s_id[kp + i] : UINT32_MAX;
                if (sid[u] != UINT32_MAX) {
                    const uint4* row = a.pcodes ? a.pcodes + (begin + s_prow[i]) * row_vecs
                                                : codes + static_cast<size_t>(sid[u]) * row_vecs;
#pragma unroll
                    for (int w = 0; w < W; ++w) c[u][w] = row[lg + G * w];
                }
            }
#pragma unroll
            for (int u = 0; u < kRowUnroll; ++u) {
                if (sid[u] == UINT32_MAX) continue;  // uniform over the group
                const int ip = group_sum<G>(lane_ip_lds<G, W>(c[u], planes_t4, vecs, lg));
                if (lg == 0) s_ip[i0 + u * kGroups] = ip;
            }
        }
        __syncthreads();
        // Pass 3, one row per thread: distance and survivor test.
        uint32_t surv = 0;
        for (int i = tid; i < n_rows; i += kScanThreads) {
            const uint32_t sid = s_id[kp + i];
            if (sid == UINT32_MAX) continue;
            const float short_ip = static_cast<float>(s_ip[i]) * sc.scale;
            const float tt = short_ip + sc.k1;
            const float v = fmaf(s_f1[i], tt, s_d[kp + i]);
            const bool in = admissible(v, sid) && pair_less(v, sid, kth_d, kth_id);
            s_d[kp + i] = in ? v : FLT_MAX;
            s_id[kp + i] = in ? sid : UINT32_MAX;
            surv += in ? 1u : 0u;
        }
        if (surv) atomicAdd(&s_surv, surv);
        __syncthreads();
        const uint32_t now = s_surv;
        const int m = static_cast<int>(now - surv_total);
        surv_total = now;
        if (m == 0) continue;  // uniform: nothing can enter
        if (score_first) {
            for (int i = tid; i < chunk; i += kScanThreads) {
                const uint32_t xid = s_id[kp + i];
                if (xid == UINT32_MAX) continue;
                const float x = s_d[kp + i];
                int cnt = count_le(s_d, s_id, k, x, xid);
                for (int j = 0; j < i && cnt < k; ++j)
                    if (s_id[kp + j] != UINT32_MAX && pair_le(s_d[kp + j], s_id[kp + j], x, xid))
                        ++cnt;
                if (cnt < k) ++passes;
            }
            __syncthreads();  // the counts read LDS that the merge below reorders
        }
        const int mp = pow2_ceil(m);
        if (mp <= kp) {
            // Gather the survivors at the tail of [kp, 2kp), sort them
            // descending, then merge with the ascending running list.
            float keep_d[8];
            uint32_t keep_id[8];
            int nk = 0;
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const int i = tid + t * kScanThreads;
                keep_d[t] = t < per ? s_d[kp + i] : FLT_MAX;
                keep_id[t] = t < per ? s_id[kp + i] : UINT32_MAX;
                nk += keep_id[t] != UINT32_MAX ? 1 : 0;
            }
            if (tid == 0) s_slot = 0;
            __syncthreads();
            for (int i = tid; i < kp; i += kScanThreads) {
                s_d[kp + i] = FLT_MAX;
                s_id[kp + i] = UINT32_MAX;
            }
            __syncthreads();
            if (nk) {
                uint32_t at = atomicAdd(&s_slot, static_cast<uint32_t>(nk));
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    if (keep_id[t] == UINT32_MAX) continue;
                    const int pos = 2 * kp - mp + static_cast<int>(at++);
                    s_d[pos] = keep_d[t];
                    s_id[pos] = keep_id[t];
                }
            }
            __syncthreads();
            bitonic_sort_desc(s_d, s_id, 2 * kp - mp, mp, tid, kScanThreads);
        } else {
            // More survivors than the list holds, so 2 kp <= chunk: sort the
            // chunk descending and move its kp least (its last kp) to
            // [kp, 2kp), which does not overlap [chunk, chunk + kp).
            bitonic_sort_desc(s_d, s_id, kp, chunk, tid, kScanThreads);
            for (int i = tid; i < kp; i += kScanThreads) {
                s_d[kp + i] = s_d[chunk + i];
                s_id[kp + i] = s_id[chunk + i];
            }
            __syncthreads();
        }
        bitonic_merge(s_d, s_id, 2 * kp, tid, kScanThreads);
    }
    if (passes) atomicAdd(&s_pass, passes);
    __syncthreads();
    for (int i = tid; i < k; i += kScanThreads) {
        a.out_ids[static_cast<size_t>(seg) * k + i] = s_id[i];
        a.out_dists[static_cast<size_t>(seg) * k + i] = s_d[i];
    }
    if (tid == 0 && a.pass_counts) a.pass_counts[seg] = s_pass;
}

// ---------------------------------------------------------------------------
// Label-shared posting scan (no counterpart in the reference, whose label
// postings are scanned route by route): the label-posting segments that scan
// the same posting rows -- the routes of one label -- share one workgroup.
// The workgroup loads a tile of the rows' posting-order columns (sample id,
// label slab, range value) into LDS once; each wave owns up to
// kShareRoutesPerWave of the routes and, per tile, filters the tile for
// each of them from LDS, queues the passing rows, scores them 64 at a time
// (one row per lane, codes and aux from the posting-order copies) and
// merges the survivors into the route's shortlist by rank, with no
// workgroup barrier per route.  Every route's output for the segment is the
// k least (distance, id) pairs of its passing rows and its pass count --
// the group kernel's output for that segment, bit for bit.
// ---------------------------------------------------------------------------
constexpr int kShareTile = 512;           // rows per LDS tile
constexpr int kShareRoutesPerWave = 4;
constexpr int kShareRoutes = kShareRoutesPerWave * (kScanThreads / kWave);  // 16 per item
constexpr int kShareMaxKp = 128;          // shortlist_k <= 128
constexpr int kShareHandles = 31;         // label handles of one pass held as row bits
constexpr uint32_t kBitsOverflow = 1u << 31;  // the row's slab overflows: read the CSR

struct ShareScanArgs {
    gofann_predicate_view pred;
    const uint32_t* route_query;
    const uint32_t* posting;
    uint64_t resident_rows;
    const uint32_t* seg_route;
    const uint64_t* item_offset;
    const uint64_t* item_size;
    const uint32_t* item_begin;  // [items + 1] into item_slots
    const uint32_t* item_slots;  // plan segment indices
    uint32_t items;
    uint32_t base_rows;
    int k;
    int k_pow2;
    const uint4* pcodes;
    const uint4* paux;
    const uint4* pslab;
    const float* pranges;
    uint32_t* out_ids;
    float* out_dists;
    uint32_t* pass_counts;
};

// A route predicate of one clause with at most 3 label and 2 range atoms,
// held in registers for the row loop (the clause walk of slab_pred_matches,
// unrolled); other predicates keep the general walk.
struct ShortClause {
    bool simple;
    int nl, nr;
    uint32_t h[3];
    gofann_range_atom r[2];
};

__device__ __forceinline__ ShortClause short_clause(const gofann_predicate_view& v, uint32_t route)
{
    ShortClause c{};
    c.simple = false;
    if (v.csr_offsets == nullptr) return c;
    uint32_t lb, le, rb = 0, re = 0;
    if (v.clauses) {
        if (v.route_offsets[route + 1] - v.route_offsets[route] != 1) return c;
        const gofann_clause cl = v.clauses[v.route_offsets[route]];
        lb = cl.label_begin;
        le = cl.label_end;
        rb = cl.range_begin;
        re = cl.range_end;
    } else {
        lb = v.route_offsets[route];
        le = v.route_offsets[route + 1];
    }
    if (le - lb > 3 || re - rb > 2) return c;
    c.nl = static_cast<int>(le - lb);
    c.nr = static_cast<int>(re - rb);
#pragma unroll
    for (int i = 0; i < 3; ++i) c.h[i] = i < c.nl ? v.route_handles[lb + i] : 0u;
#pragma unroll
    for (int i = 0; i < 2; ++i)
        if (i < c.nr) c.r[i] = v.ranges[rb + i];
    c.simple = true;
    return c;
}

// slab_pred_matches for a ShortClause route (same label scans and range
// tests, in the same order of evaluation results).
__device__ __forceinline__ bool short_clause_matches(const gofann_predicate_view& v,
                                                     const ShortClause& c, uint32_t sample,
                                                     const uint4& slab, const float* prange,
                                                     float r0)
{
    if (sample >= v.rows) return false;
    const uint32_t n = slab_count(slab);
    bool pass = true;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        if (i >= c.nl) break;
        bool hit = false;  // the first label >= handle decides
        for (uint32_t k = 0; k < n; ++k) {
            const uint32_t label = slab_label(slab, k);
            if (label >= c.h[i]) {
                hit = label == c.h[i];
                break;
            }
        }
        pass = pass && hit;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        if (i >= c.nr) break;
        const gofann_range_atom at = c.r[i];
        pass = pass && v.base_ranges != nullptr && at.dimension < range_columns(v) &&
               range_matches(at.mode, at.lower, at.upper,
                             !prange ? v.base_ranges[static_cast<uint64_t>(sample) * v.range_stride +
                                                     at.dimension]
                             : range_columns(v) == 1 ? r0
                                                   : prange[at.dimension]);
    }
    return pass;
}

// short_clause_matches with the label atoms given as the row's handle bits:
// every handle of the clause present ((bits & need) == need), then the same
// range tests.
__device__ __forceinline__ bool short_clause_bits_match(const gofann_predicate_view& v,
                                                        const ShortClause& c, uint32_t sample,
                                                        uint32_t bits, uint32_t need,
                                                        const float* prange, float r0)
{
    if (sample >= v.rows) return false;
    bool pass = (bits & need) == need;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        if (i >= c.nr) break;
        const gofann_range_atom at = c.r[i];
        pass = pass && v.base_ranges != nullptr && at.dimension < range_columns(v) &&
               range_matches(at.mode, at.lower, at.upper,
                             !prange ? v.base_ranges[static_cast<uint64_t>(sample) * v.range_stride +
                                                     at.dimension]
                             : range_columns(v) == 1 ? r0
                                                   : prange[at.dimension]);
    }
    return pass;
}

// What the tile loop and the flushes need of one route slot, read once per
// pass into LDS (64 bytes): the route, its query's scale and k1, and its
// predicate as a ShortClause (flags: bit 0 enabled, bit 1 simple, bits 2-3
// label atoms, bits 4-5 range atoms).  Otherwise every tile re-reads them
// through a chain of dependent global loads (slot -> route -> clause ->
// handles and ranges).
struct ShareSlot {
    uint32_t route;
    uint32_t query;
    float scale;
    float k1;
    uint32_t flags;
    uint32_t h[3];
    gofann_range_atom r[2];
};
static_assert(sizeof(ShareSlot) == 64, "one 64-byte record per route slot");

__device__ __forceinline__ ShareSlot share_slot(const gofann_predicate_view& v,
                                                const RabitqScanScorer& sc, uint32_t route,
                                                uint32_t query)
{
    ShareSlot o{};
    o.route = route;
    o.query = query;
    o.scale = sc.q_scale[query];
    o.k1 = sc.q_k1[query];
    const bool enabled = pred_enabled(v, route);
    const ShortClause c = enabled ? short_clause(v, route) : ShortClause{};
    o.flags = (enabled ? 1u : 0u) | (c.simple ? 2u : 0u) | (static_cast<uint32_t>(c.nl) << 2) |
              (static_cast<uint32_t>(c.nr) << 4);
#pragma unroll
    for (int i = 0; i < 3; ++i) o.h[i] = c.h[i];
#pragma unroll
    for (int i = 0; i < 2; ++i) o.r[i] = c.r[i];
    return o;
}

__device__ __forceinline__ ShortClause slot_clause(const ShareSlot& s)
{
    ShortClause c;
    c.simple = (s.flags & 2u) != 0;
    c.nl = static_cast<int>((s.flags >> 2) & 3u);
    c.nr = static_cast<int>((s.flags >> 4) & 3u);
#pragma unroll
    for (int i = 0; i < 3; ++i) c.h[i] = s.h[i];
#pragma unroll
    for (int i = 0; i < 2; ++i) c.r[i] = s.r[i];
    return c;
}

// Scores the queued rows of route slot q (lane i < qn takes queue[i], a row
// offset in the item) and merges the survivors into its shortlist by rank
// (the lists hold k pairs per slot).  All 64 lanes of the wave call it.
template <int V>
__device__ __forceinline__ void share_flush(const ShareScanArgs& a, const RabitqScanScorer& sc,
                                            const ShareSlot& slot, int q, const uint4* planes_all,
                                            float* lst_d_all, uint32_t* lst_id_all,
                                            const uint32_t* queue, int qn, uint64_t begin,
                                            int lane)
{
    const int k = a.k;
    const uint32_t query = slot.query;
    const float scale = slot.scale;
    const float k1 = slot.k1;
    const float* g_row = sc.centroid_dists + static_cast<size_t>(query) * sc.num_anchors;
    const uint4* planes = planes_all + q * 8 * V;
    float* ld = lst_d_all + q * k;
    uint32_t* lid = lst_id_all + q * k;
    const bool have = lane < qn;
    const uint64_t j = begin + (have ? queue[lane] : 0u);
    uint32_t sid = UINT32_MAX;
    float v = FLT_MAX;
    if (have) {
        sid = a.posting[j];
        const uint4 x = a.paux[j];
        uint4 c[V];
#pragma unroll
        for (int w = 0; w < V; ++w) c[w] = a.pcodes[j * V + w];
        const float add0 = __uint_as_float(x.x) + g_row[x.z];
        const int ip = lane_ip_lds<1, V>(c, planes, V, 0);
        const float short_ip = static_cast<float>(ip) * scale;
        const float tt = short_ip + k1;
        v = fmaf(__uint_as_float(x.y), tt, add0);
    }
    const float kd = ld[k - 1];
    const uint32_t kid = lid[k - 1];
    const bool in = have && admissible(v, sid) && pair_less(v, sid, kd, kid);
    const uint64_t sm = ballot(in);
    if (!sm) return;
    // ranks: list entry e moves up by the survivors below it; a survivor
    // lands after the list entries and survivors below it
    int c_self = 0;
    if (in) {
        int lo = 0, hi = k;
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (pair_less(ld[mid], lid[mid], v, sid))
                lo = mid + 1;
            else
                hi = mid;
        }
        c_self = lo;
    }
    const int e0 = lane, e1 = lane + kWave;
    const float d0 = e0 < k ? ld[e0] : FLT_MAX;
    const uint32_t i0 = e0 < k ? lid[e0] : UINT32_MAX;
    const float d1 = e1 < k ? ld[e1] : FLT_MAX;
    const uint32_t i1 = e1 < k ? lid[e1] : UINT32_MAX;
    int c0 = 0, c1 = 0;
    for (uint64_t m = sm; m; m &= m - 1) {
        const int src = __builtin_ctzll(m);
        const float sv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), src));
        const uint32_t si = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(sid), src));
        c0 += pair_less(sv, si, d0, i0) ? 1 : 0;
        c1 += pair_less(sv, si, d1, i1) ? 1 : 0;
        c_self += pair_less(sv, si, v, sid) ? 1 : 0;
    }
    // all reads of the old list precede these writes (one wave)
    if (e0 < k && e0 + c0 < k) {
        ld[e0 + c0] = d0;
        lid[e0 + c0] = i0;
    }
    if (e1 < k && e1 + c1 < k) {
        ld[e1 + c1] = d1;
        lid[e1 + c1] = i1;
    }
    if (in && c_self < k) {
        ld[c_self] = v;
        lid[c_self] = sid;
    }
}

// Waves per SIMD: 4 for query codes up to 512 bits (114-128 VGPRs, four
// workgroups per CU as LDS allows), 3 for longer codes (at 4 they spill).
template <int V>
__global__ __launch_bounds__(kScanThreads, (V <= 4 ? 4 : 3)) void label_share_scan_kernel(
    ShareScanArgs a, RabitqScanScorer sc)
{
    extern __shared__ __align__(16) unsigned char lds[];
    __shared__ uint32_t s_pass[kShareRoutes];
    __shared__ uint32_t s_h[kShareHandles];     // the pass's label handles, ascending
    __shared__ uint32_t s_need[kShareRoutes];   // per route slot: bits of its handles
    __shared__ int s_nh;
    __shared__ int s_use_bits;
    __shared__ int s_qn[kShareRoutes];
    __shared__ ShareSlot s_slot[kShareRoutes];
    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const uint32_t item = blockIdx.x;
    if (item >= a.items) return;
    const int k = a.k;
    // LDS: tile columns (sample ids, label slabs, first range value, label
    // bits), then per route slot its query planes (plane-major, 8 x V
    // 16-byte vectors), its shortlist (k pairs) and its queue of passing
    // rows still to score (kept across tiles, scored 64 at a time).
    uint32_t* t_ids = reinterpret_cast<uint32_t*>(lds);
    uint4* t_slab = reinterpret_cast<uint4*>(t_ids + kShareTile);
    float* t_r0 = reinterpret_cast<float*>(t_slab + kShareTile);
    uint32_t* t_bits = reinterpret_cast<uint32_t*>(t_r0 + kShareTile);
    uint4* planes_all = reinterpret_cast<uint4*>(t_bits + kShareTile);
    float* lst_d_all = reinterpret_cast<float*>(planes_all + kShareRoutes * 8 * V);
    uint32_t* lst_id_all = reinterpret_cast<uint32_t*>(lst_d_all + kShareRoutes * k);
    uint32_t* queue_all = lst_id_all + kShareRoutes * k;

    const uint32_t first_all = a.item_begin[item];
    const int n_all = static_cast<int>(a.item_begin[item + 1] - first_all);
    const uint64_t begin = a.item_offset[item];
    uint64_t count = a.item_size[item];
    if (begin > a.resident_rows)
        count = 0;
    else if (count > a.resident_rows - begin)
        count = a.resident_rows - begin;

    // An item of more than kShareRoutes routes is served in passes of
    // kShareRoutes slots, each re-reading the item's tiles, so every slot
    // is written whatever plan the caller built.
    for (int pass0 = 0; pass0 < n_all; pass0 += kShareRoutes) {
        const uint32_t first = first_all + static_cast<uint32_t>(pass0);
        const int n_routes = n_all - pass0 < kShareRoutes ? n_all - pass0 : kShareRoutes;
        // Route slots q = wave + 4 i: query planes and an empty shortlist.
        for (int i = 0; i < kShareRoutesPerWave; ++i) {
            const int q = wave + i * (kScanThreads / kWave);
            if (q >= n_routes) break;
            const uint32_t route = a.seg_route[a.item_slots[first + q]];
            const uint32_t query = a.route_query[route];
            uint32_t* pl = reinterpret_cast<uint32_t*>(planes_all + q * 8 * V);
            const int8_t* qrow = sc.q8 + static_cast<size_t>(query) * sc.padded_dim;
            const int words = 4 * V;  // padded_dim / 32
            if (lane < words) {
                uint32_t bits[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                for (int b = 0; b < 32; ++b) {
                    const uint32_t v = static_cast<uint8_t>(qrow[lane * 32 + b]);
    #pragma unroll
                    for (int j = 0; j < 8; ++j) bits[j] |= ((v >> j) & 1u) << (31 - b);
                }
    #pragma unroll
                for (int j = 0; j < 8; ++j) pl[j * words + lane] = bits[j];
            }
            for (int e = lane; e < k; e += kWave) {
                lst_d_all[q * k + e] = FLT_MAX;
                lst_id_all[q * k + e] = UINT32_MAX;
            }
            if (lane == 0) {
                s_pass[q] = 0;
                s_qn[q] = 0;
                s_slot[q] = share_slot(a.pred, sc, route, query);
            }
        }
        __syncthreads();
        // Label bits: when every enabled route of the pass is a short clause
        // and their label handles number at most kShareHandles, each tile row
        // gets one bit per handle it holds (found once per row), and a
        // route's label atoms reduce to (bits & need) == need -- the same
        // verdicts as the per-route slab walk (a row's slab labels are
        // distinct and ascending; a handle >= 0xFFFF is on no slab).
        if (tid == 0) {
            int nh = 0;
            int use = 1;
            for (int q = 0; q < n_routes && use; ++q) {
                if (!(s_slot[q].flags & 1u)) continue;
                const ShortClause c = slot_clause(s_slot[q]);
                if (!c.simple) {
                    use = 0;
                    break;
                }
                for (int i = 0; i < c.nl; ++i) {
                    int at = 0;
                    while (at < nh && s_h[at] < c.h[i]) ++at;
                    if (at < nh && s_h[at] == c.h[i]) continue;
                    if (nh == kShareHandles) {
                        use = 0;
                        break;
                    }
                    for (int m = nh; m > at; --m) s_h[m] = s_h[m - 1];
                    s_h[at] = c.h[i];
                    ++nh;
                }
            }
            for (int q = 0; q < n_routes && use; ++q) {
                uint32_t need = 0;
                if (s_slot[q].flags & 1u) {
                    const ShortClause c = slot_clause(s_slot[q]);
                    for (int i = 0; i < c.nl; ++i) {
                        int at = 0;
                        while (s_h[at] != c.h[i]) ++at;
                        need |= 1u << at;
                    }
                }
                s_need[q] = need;
            }
            s_nh = nh;
            s_use_bits = use;
        }
        __syncthreads();
        const bool use_bits = s_use_bits != 0;
        const int nh = s_nh;
        const bool r0_tile = a.pranges && range_columns(a.pred) == 1;

        for (uint64_t t0 = 0; t0 < count; t0 += kShareTile) {
            __syncthreads();  // the previous tile's reads end here
            const int n = static_cast<int>(count - t0 < kShareTile ? count - t0 : kShareTile);
            for (int r = tid; r < n; r += kScanThreads) {
                const uint64_t j = begin + t0 + static_cast<uint64_t>(r);
                t_ids[r] = a.posting[j];
                const uint4 slab = a.pslab[j];
                if (!use_bits) t_slab[r] = slab;
                if (r0_tile) t_r0[r] = a.pranges[j];
                if (use_bits) {
                    uint32_t bits = kBitsOverflow;
                    const uint32_t cnt = slab_count(slab);
                    if (cnt != kSlabOverflow) {
                        bits = 0;
                        for (uint32_t e = 0; e < cnt; ++e) {
                            const uint32_t label = slab_label(slab, e);
                            int lo = 0, hi = nh;  // first handle >= label
                            while (lo < hi) {
                                const int mid = (lo + hi) >> 1;
                                if (s_h[mid] < label)
                                    lo = mid + 1;
                                else
                                    hi = mid;
                            }
                            if (lo < nh && s_h[lo] == label) bits |= 1u << lo;
                        }
                    }
                    t_bits[r] = bits;
                }
            }
            __syncthreads();
            for (int i = 0; i < kShareRoutesPerWave; ++i) {
                const int q = wave + i * (kScanThreads / kWave);
                if (q >= n_routes) break;
                const ShareSlot& slot = s_slot[q];
                const uint32_t route = slot.route;
                const bool enabled = (slot.flags & 1u) != 0;
                const ShortClause sclause = slot_clause(slot);
                const uint32_t need = use_bits ? s_need[q] : 0u;
                uint32_t* queue = queue_all + q * kWave;
                int qn = s_qn[q];  // queued rows of this slot (uniform), kept across tiles
                uint32_t passes = 0;
                // Fast verdicts: label atoms as row bits and at most one range
                // atom, on the column held in the tile -- a row's verdict is
                // three LDS words and a few compares (rows whose slab
                // overflows still take the CSR walk).  Same verdicts as
                // short_clause_bits_match.
                const bool fast = use_bits && enabled && sclause.simple &&
                                  (sclause.nr == 0 || (sclause.nr == 1 && r0_tile));
                const gofann_range_atom fat = sclause.r[0];
                const bool fast_rng = sclause.nr != 0;
                const bool fast_live = !fast_rng || (a.pred.base_ranges != nullptr &&
                                                     fat.dimension < range_columns(a.pred));
                const uint32_t fast_rows = a.base_rows < a.pred.rows ? a.base_rows : a.pred.rows;
                for (int r0 = 0; r0 < n; r0 += kWave) {
                    const int r = r0 + lane;
                    bool ok = false;
                    if (fast) {
                        if (r < n) {
                            const uint32_t s = t_ids[r];
                            const uint32_t bits = t_bits[r];
                            if (!(bits & kBitsOverflow)) {
                                ok = s < fast_rows && (bits & need) == need && fast_live &&
                                     (!fast_rng ||
                                      range_matches(fat.mode, fat.lower, fat.upper, t_r0[r]));
                            } else if (s < a.base_rows) {
                                PredCounters pc{0, 0};
                                ok = pred_matches(a.pred, route, s, pc);
                            }
                        }
                    } else if (r < n) {
                        const uint32_t s = t_ids[r];
                        ok = s < a.base_rows;
                        if (ok && enabled && use_bits) {
                            const uint32_t bits = t_bits[r];
                            if (!(bits & kBitsOverflow)) {
                                const uint64_t j = begin + t0 + static_cast<uint64_t>(r);
                                const float* prange = a.pranges && range_columns(a.pred) > 0
                                                          ? a.pranges + j * range_columns(a.pred)
                                                          : nullptr;
                                const float rv = r0_tile ? t_r0[r] : 0.0f;
                                ok = short_clause_bits_match(a.pred, sclause, s, bits, need, prange,
                                                             rv);
                            } else {
                                PredCounters pc{0, 0};
                                ok = pred_matches(a.pred, route, s, pc);
                            }
                        } else if (ok && enabled) {
                            const uint4 slab = t_slab[r];
                            if (slab_count(slab) != kSlabOverflow) {
                                const uint64_t j = begin + t0 + static_cast<uint64_t>(r);
                                const float* prange = a.pranges && range_columns(a.pred) > 0
                                                          ? a.pranges + j * range_columns(a.pred)
                                                          : nullptr;
                                const float rv = r0_tile ? t_r0[r] : 0.0f;
                                ok = use_bits
                                         ? short_clause_bits_match(a.pred, sclause, s, t_bits[r],
                                                                   need, prange, rv)
                                     : sclause.simple
                                         ? short_clause_matches(a.pred, sclause, s, slab, prange, rv)
                                         : slab_pred_matches(a.pred, route, s, slab, prange, rv);
                            } else {
                                PredCounters pc{0, 0};
                                ok = pred_matches(a.pred, route, s, pc);
                            }
                        }
                    }
                    const uint64_t om = ballot(ok);
                    const int c = __popcll(om);
                    if (enabled) passes += static_cast<uint32_t>(c);
                    if (c == 0) continue;
                    if (qn + c > kWave) {
                        share_flush<V>(a, sc, slot, q, planes_all, lst_d_all, lst_id_all, queue,
                                       qn, begin, lane);
                        qn = 0;
                    }
                    // the row's offset in the item (items hold < 2^32 rows)
                    if (ok)
                        queue[qn + static_cast<int>(lanes_below(om))] =
                            static_cast<uint32_t>(t0) + static_cast<uint32_t>(r);
                    qn += c;
                }
                if (lane == 0) {
                    s_pass[q] += passes;
                    s_qn[q] = qn;
                }
            }
        }
        // the rows still queued
        __syncthreads();
        for (int i = 0; i < kShareRoutesPerWave; ++i) {
            const int q = wave + i * (kScanThreads / kWave);
            if (q >= n_routes) break;
            const int qn = s_qn[q];
            if (qn)
                share_flush<V>(a, sc, s_slot[q], q, planes_all,
                               lst_d_all, lst_id_all, queue_all + q * kWave, qn, begin, lane);
        }
        __syncthreads();
        for (int i = 0; i < kShareRoutesPerWave; ++i) {
            const int q = wave + i * (kScanThreads / kWave);
            if (q >= n_routes) break;
            const uint32_t slot = a.item_slots[first + q];
            for (int e = lane; e < k; e += kWave) {
                a.out_ids[static_cast<size_t>(slot) * k + e] = lst_id_all[q * k + e];
                a.out_dists[static_cast<size_t>(slot) * k + e] = lst_d_all[q * k + e];
            }
            if (lane == 0 && a.pass_counts) a.pass_counts[slot] = s_pass[q];
        }
    }
}

struct SegmentMergeArgs {
    const uint32_t* query_indptr;  // null: position p takes [p * stride, (p + 1) * stride)
    uint32_t stride;
    uint32_t positions;
    const uint32_t* seg_ids;
    const float* seg_dists;
    const uint32_t* seg_pass;
    int k;
    int k_pow2;
    uint32_t* out_ids;
    float* out_dists;
    uint32_t* out_pass;
};

__global__ __launch_bounds__(kScanThreads) void segment_merge_kernel(SegmentMergeArgs a)
{
    extern __shared__ __align__(16) unsigned char lds[];
    const int tid = static_cast<int>(threadIdx.x);
    const uint32_t p = blockIdx.x;
    if (p >= a.positions) return;
    const int k = a.k, kp = a.k_pow2;
    float* s_d = reinterpret_cast<float*>(lds);
    uint32_t* s_id = reinterpret_cast<uint32_t*>(s_d + 2 * kp);
    for (int i = tid; i < kp; i += kScanThreads) {
        s_d[i] = FLT_MAX;
        s_id[i] = UINT32_MAX;
    }
    __syncthreads();
    uint32_t passes = 0;
    const uint32_t first = a.query_indptr ? a.query_indptr[p] : p * a.stride;
    const uint32_t last = a.query_indptr ? a.query_indptr[p + 1] : (p + 1) * a.stride;
    for (uint32_t part = first; part < last; ++part) {
        passes += a.seg_pass[part];
        const size_t o = static_cast<size_t>(part) * k;
        // A segment's list is ascending: when its best pair cannot enter,
        // none of it can.
        const bool skip = !pair_less(a.seg_dists[o], a.seg_ids[o], s_d[k - 1], s_id[k - 1]);
        if (skip) continue;  // uniform
        for (int i = tid; i < kp; i += kScanThreads) {
            // reversed into [kp, 2kp): non-increasing, padding first
            const int src = kp - 1 - i;
            const bool in = src < k && admissible(a.seg_dists[o + src], a.seg_ids[o + src]);
            s_d[kp + i] = in ? a.seg_dists[o + src] : FLT_MAX;
            s_id[kp + i] = in ? a.seg_ids[o + src] : UINT32_MAX;
        }
        __syncthreads();
        bitonic_merge(s_d, s_id, 2 * kp, tid, kScanThreads);
    }
    for (int i = tid; i < k; i += kScanThreads) {
        a.out_ids[static_cast<size_t>(p) * k + i] = s_id[i];
        a.out_dists[static_cast<size_t>(p) * k + i] = s_d[i];
    }
    if (tid == 0 && a.out_pass) a.out_pass[p] = passes;
}

// Posting-order copies of the RaBitQ rows: one thread per 16-byte vector
// of a code row, and per aux record.
__global__ __launch_bounds__(256) void posting_rows_kernel(const uint4* codes, const float* factors,
                                                           const uint32_t* anchors,
                                                           const uint32_t* posting, uint64_t rows,
                                                           uint32_t vecs, uint32_t samples,
                                                           uint4* out_codes, uint4* out_aux)
{
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * 256u;
    const uint64_t total = rows * (vecs + 1u);
    for (uint64_t t = static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x; t < total;
         t += stride) {
        const uint64_t r = t / (vecs + 1u);
        const uint32_t v = static_cast<uint32_t>(t % (vecs + 1u));
        const uint32_t s = posting[r];
        const bool ok = s < samples;
        if (v < vecs) {
            out_codes[r * vecs + v] =
                ok ? codes[static_cast<uint64_t>(s) * vecs + v] : make_uint4(0, 0, 0, 0);
        } else {
            out_aux[r] = ok ? make_uint4(__float_as_uint(factors[static_cast<uint64_t>(s) * 3]),
                                         __float_as_uint(factors[static_cast<uint64_t>(s) * 3 + 1]),
                                         anchors[s], 0u)
                            : make_uint4(0, 0, 0, 0);
        }
    }
}

int rabitq_posting_rows(Context* ctx, const gofann_rabitq_view* rq, const uint32_t* posting,
                        uint64_t rows, uint8_t* out_codes, uint32_t* out_aux)
{
    if (!rq || !rq->codes || !rq->factors || !rq->anchor_ids || rq->padded_dim == 0 ||
        rq->padded_dim % 128 != 0)
        return ctx->fail(GOFANN_ERR_INVALID, "RaBitQ view invalid for posting rows");
    if (rows == 0) return GOFANN_OK;
    if (!posting || !out_codes || !out_aux)
        return ctx->fail(GOFANN_ERR_INVALID, "posting rows arrays missing");
    if ((reinterpret_cast<uintptr_t>(out_codes) | reinterpret_cast<uintptr_t>(out_aux) |
         reinterpret_cast<uintptr_t>(rq->codes)) & 15u)
        return ctx->fail(GOFANN_ERR_INVALID, "code and aux arrays must be 16-byte aligned");
    const uint32_t vecs = rq->padded_dim / 128;
    const uint64_t total = rows * (vecs + 1u);
    const uint32_t blocks = static_cast<uint32_t>(std::min<uint64_t>((total + 255) / 256, 1u << 20));
    hipLaunchKernelGGL(posting_rows_kernel, dim3(blocks), dim3(256), 0, ctx->stream,
                       reinterpret_cast<const uint4*>(rq->codes), rq->factors, rq->anchor_ids,
                       posting, rows, vecs, rq->samples, reinterpret_cast<uint4*>(out_codes),
                       reinterpret_cast<uint4*>(out_aux));
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("posting rows launch");
    return GOFANN_OK;
}

// Posting-order predicate columns: row r of the posting gets its sample's
// label slab -- u16 count, then the first labels of the CSR row in CSR
// order as u16 -- or the overflow form (count kSlabOverflow: the scan reads
// the CSR row) when the row has more than kSlabCapacity labels, a label
// above 0xFFFF, no CSR, or the sample is out of range; and its base range
// row (zeros without base ranges or for an out-of-range sample).
__global__ __launch_bounds__(256) void posting_pred_rows_kernel(gofann_predicate_view v,
                                                                const uint32_t* posting,
                                                                uint64_t rows, uint4* out_slab,
                                                                float* out_ranges)
{
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * 256u;
    for (uint64_t r = static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x; r < rows;
         r += stride) {
        const uint32_t s = posting[r];
        const bool in = s < v.rows;
        uint32_t w[4] = {kSlabOverflow, 0u, 0u, 0u};
        if (in && v.csr_offsets != nullptr) {
            const uint32_t b = v.csr_offsets[s];
            const uint32_t e = v.csr_offsets[s + 1];
            const uint32_t n = e - b;
            bool ok = e >= b && n <= kSlabCapacity;
            uint32_t x[4] = {n, 0u, 0u, 0u};
            for (uint32_t k = 0; ok && k < n; ++k) {
                const uint32_t label = v.csr_labels[b + k];
                ok = label <= 0xFFFFu;
                const uint32_t h = k + 1;  // u16 index
                x[h >> 1] |= (label & 0xFFFFu) << (16 * (h & 1));
            }
            if (ok) {
                w[0] = x[0];
                w[1] = x[1];
                w[2] = x[2];
                w[3] = x[3];
            }
        }
        out_slab[r] = make_uint4(w[0], w[1], w[2], w[3]);
        if (out_ranges) {
            const uint32_t cols = range_columns(v);
            for (uint32_t d = 0; d < cols; ++d)
                out_ranges[r * cols + d] =
                    in && v.base_ranges ? v.base_ranges[static_cast<uint64_t>(s) * v.range_stride + d]
                                        : 0.0f;
        }
    }
}

int posting_predicate_rows(Context* ctx, const gofann_predicate_view* pred,
                           const uint32_t* posting, uint64_t rows, uint32_t* out_slab,
                           float* out_ranges)
{
    if (!pred) return ctx->fail(GOFANN_ERR_INVALID, "predicate view missing");
    if (rows == 0) return GOFANN_OK;
    if (!posting || !out_slab)
        return ctx->fail(GOFANN_ERR_INVALID, "posting predicate rows arrays missing");
    if (pred->csr_offsets && !pred->csr_labels)
        return ctx->fail(GOFANN_ERR_INVALID, "CSR labels missing");
    if (reinterpret_cast<uintptr_t>(out_slab) & 15u)
        return ctx->fail(GOFANN_ERR_INVALID, "slab array must be 16-byte aligned");
    const uint32_t blocks = static_cast<uint32_t>(std::min<uint64_t>((rows + 255) / 256, 1u << 20));
    hipLaunchKernelGGL(posting_pred_rows_kernel, dim3(blocks), dim3(256), 0, ctx->stream, *pred,
                       posting, rows, reinterpret_cast<uint4*>(out_slab),
                       pred->range_stride ? out_ranges : nullptr);
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("posting predicate rows launch");
    return GOFANN_OK;
}

namespace {
int pow2_at_least(int x)
{
    int p = 1;
    while (p < x) p <<= 1;
    return p;
}

// The group-per-row kernel for a padded dimension: the row's 16-byte
// vectors split evenly over a power-of-two group of <= 32 lanes, two vectors
// per lane at most; null otherwise (the thread-per-row kernels remain).
const void* group_scan_kernel(uint32_t padded_dim)
{
    if (padded_dim == 0 || padded_dim % 128 != 0) return nullptr;
    switch (padded_dim / 128) {
        case 1: return reinterpret_cast<const void*>(range_scan_group_kernel<1, 1>);
        case 2: return reinterpret_cast<const void*>(range_scan_group_kernel<2, 1>);
        case 4: return reinterpret_cast<const void*>(range_scan_group_kernel<4, 1>);
        case 8: return reinterpret_cast<const void*>(range_scan_group_kernel<8, 1>);
        case 16: return reinterpret_cast<const void*>(range_scan_group_kernel<16, 1>);
        case 32: return reinterpret_cast<const void*>(range_scan_group_kernel<32, 1>);
        case 64: return reinterpret_cast<const void*>(range_scan_group_kernel<32, 2>);
        default: return nullptr;
    }
}

RabitqScanScorer scan_scorer(const gofann_rabitq_view* rq, const gofann_rabitq_queries* pre)
{
    RabitqScanScorer sc;
    sc.codes = rq->codes;
    sc.factors = rq->factors;
    sc.anchor_ids = rq->anchor_ids;
    sc.q8 = pre->q8;
    sc.q_scale = pre->scale;
    sc.q_k1 = pre->k1;
    sc.centroid_dists = pre->centroid_dists;
    sc.num_anchors = rq->num_anchors;
    sc.padded_dim = rq->padded_dim;
    sc.planes = nullptr;
    sc.scale = sc.k1 = 0.0f;
    sc.g_row = nullptr;
    return sc;
}

// Workgroups a label-posting launch aims for: enough to fill every CU
// several times over.
constexpr uint32_t kPostingTargetGroups = 4096;
constexpr uint32_t kPostingMaxSlices = 32;
}  // namespace

bool rabitq_posting_scan_grouped(uint32_t padded_dim)
{
    return group_scan_kernel(padded_dim) != nullptr;
}

// Label-posting scan (lowfreq_rabitq_resident_posting_kernel,
// backend_rabitq.cu:5494-5682) on the group-per-row kernel.  A route's
// posting is cut into `slices` near-equal parts so that few long routes
// still fill the chip; the parts' shortlists are merged per route (their
// union's k least pairs are the route's, pass counts add up).
int rabitq_posting_scan_group(Context* ctx, const gofann_rabitq_view* rq,
                              const gofann_rabitq_queries* pre, const gofann_predicate_view* pred,
                              const uint32_t* route_query, const uint32_t* cand_ids,
                              const uint32_t* cand_offsets, const uint32_t* cand_sizes,
                              uint32_t routes, int shortlist_k, uint32_t* out_ids,
                              float* out_dists, uint32_t* pass_counts)
{
    const void* kern = group_scan_kernel(rq->padded_dim);
    if (!kern) return ctx->fail(GOFANN_ERR_UNSUPPORTED, "padded_dim has no grouped posting scan");
    if (!pre->q8 || !pre->scale || !pre->k1 || !pre->centroid_dists || !rq->factors ||
        !rq->anchor_ids)
        return ctx->fail(GOFANN_ERR_INVALID, "RaBitQ view or prepared queries incomplete");
    if (!route_query || !cand_ids || !cand_offsets || !cand_sizes || !out_ids || !out_dists)
        return ctx->fail(GOFANN_ERR_INVALID, "posting scan arrays missing");
    uint32_t slices = (kPostingTargetGroups + routes - 1) / routes;
    slices = std::max(1u, std::min(slices, kPostingMaxSlices));
    const uint64_t segments = static_cast<uint64_t>(routes) * slices;
    if (segments > 0x7fffffffull)
        return ctx->fail(GOFANN_ERR_INVALID, "too many posting routes");

    uint32_t* scan_ids = out_ids;
    float* scan_dists = out_dists;
    uint32_t* scan_pass = pass_counts;
    if (slices > 1) {
        const size_t slots_out = static_cast<size_t>(segments) * static_cast<size_t>(shortlist_k);
        const size_t bytes = slots_out * 8 + static_cast<size_t>(segments) * 4 + 64;
        unsigned char* buf =
            static_cast<unsigned char*>(ctx->scratch(Context::kScratchRange, bytes));
        if (!buf) return ctx->fail(GOFANN_ERR_NOMEM, "posting slice scratch allocation failed");
        scan_ids = reinterpret_cast<uint32_t*>(buf);
        scan_dists = reinterpret_cast<float*>(buf + slots_out * 4);
        scan_pass = reinterpret_cast<uint32_t*>(buf + slots_out * 8);
    }

    RangeScanArgs a{};
    a.pred = pred ? *pred : gofann_predicate_view{};
    a.routes.route_query = route_query;
    a.posting = cand_ids;
    a.resident_rows = UINT64_MAX;
    a.segments = static_cast<uint32_t>(segments);
    a.base_rows = rq->samples ? rq->samples : UINT32_MAX;
    a.k = shortlist_k;
    a.k_pow2 = pow2_at_least(shortlist_k);
    a.chunk = a.k_pow2 <= 1024 ? 1024 : 2048;
    a.slots = std::max(2 * a.k_pow2, a.k_pow2 + a.chunk);
    a.planes_bytes = rq->padded_dim;
    a.score_first = 0;
    a.out_ids = scan_ids;
    a.out_dists = scan_dists;
    a.pass_counts = slices > 1 || pass_counts ? scan_pass : nullptr;
    a.label_mode = 1;
    a.cand_offsets = cand_offsets;
    a.cand_sizes = cand_sizes;
    a.slices = slices;
    a.pcodes = nullptr;
    a.paux = nullptr;
    const size_t lds = 2 * static_cast<size_t>(a.planes_bytes) + static_cast<size_t>(a.slots) * 8 +
                       static_cast<size_t>(a.chunk) * 12;
    if (lds > static_cast<size_t>(ctx->lds_per_block))
        return ctx->fail(GOFANN_ERR_UNSUPPORTED, "posting scan LDS exceeds the workgroup limit");
    if (hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(lds)) != hipSuccess)
        return ctx->fail_hip("hipFuncSetAttribute posting scan");
    RabitqScanScorer sc = scan_scorer(rq, pre);
    void* kargs[] = {&a, &sc};
    if (hipLaunchKernel(kern, dim3(a.segments), dim3(kScanThreads), kargs, lds, ctx->stream) !=
        hipSuccess)
        return ctx->fail_hip("posting scan launch");
    if (slices == 1) return GOFANN_OK;

    SegmentMergeArgs m;
    m.query_indptr = nullptr;
    m.stride = slices;
    m.positions = routes;
    m.seg_ids = scan_ids;
    m.seg_dists = scan_dists;
    m.seg_pass = scan_pass;
    m.k = shortlist_k;
    m.k_pow2 = a.k_pow2;
    m.out_ids = out_ids;
    m.out_dists = out_dists;
    m.out_pass = pass_counts;
    const size_t mlds = static_cast<size_t>(2 * a.k_pow2) * 8;
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(segment_merge_kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(mlds)) !=
        hipSuccess)
        return ctx->fail_hip("hipFuncSetAttribute posting merge");
    hipLaunchKernelGGL(segment_merge_kernel, dim3(routes), dim3(kScanThreads), mlds, ctx->stream,
                       m);
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("posting merge launch");
    return GOFANN_OK;
}

// Label-posting scan over an explicit segment plan: the results of
// rabitq_posting_scan_group for the routes whose postings the plan covers
// (a route's k least pairs over the union of its segments, pass counts
// summed), with long postings cut into many workgroups and, when given,
// the rows' codes and predicate columns read in posting order.
int rabitq_posting_scan_segments(Context* ctx, const gofann_rabitq_view* rq,
                                 const gofann_rabitq_queries* pre,
                                 const gofann_predicate_view* pred, const uint32_t* route_query,
                                 const uint32_t* posting, uint64_t posting_rows,
                                 const gofann_posting_segments* seg, int shortlist_k,
                                 const uint8_t* posting_codes, const uint32_t* posting_aux,
                                 const uint32_t* posting_slab, const float* posting_ranges,
                                 uint32_t* out_ids, float* out_dists, uint32_t* pass_counts)
{
    if ((posting_codes == nullptr) != (posting_aux == nullptr))
        return ctx->fail(GOFANN_ERR_INVALID, "posting codes and aux come together");
    if (posting_ranges && !posting_slab)
        return ctx->fail(GOFANN_ERR_INVALID, "posting ranges need the posting slab");
    if (!rq || !pre || !rq->codes || !rq->factors || !rq->anchor_ids || rq->padded_dim == 0 ||
        rq->padded_dim % 128 != 0)
        return ctx->fail(GOFANN_ERR_INVALID, "RaBitQ view invalid for posting scan");
    const void* kern = group_scan_kernel(rq->padded_dim);
    if (!kern) return ctx->fail(GOFANN_ERR_UNSUPPORTED, "padded_dim has no grouped posting scan");
    if (!pre->q8 || !pre->scale || !pre->k1 || !pre->centroid_dists)
        return ctx->fail(GOFANN_ERR_INVALID, "prepared RaBitQ queries incomplete");
    if (!seg) return ctx->fail(GOFANN_ERR_INVALID, "segment plan missing");
    if (shortlist_k < 1 || shortlist_k > kRangeMaxShortlist)
        return ctx->fail(GOFANN_ERR_INVALID, "shortlist_k must be in [1, 4096]");
    if (seg->count == 0) {
        if (seg->query_indptr && seg->positions)
            return ctx->fail(GOFANN_ERR_INVALID, "segment plan has positions but no segments");
        return GOFANN_OK;
    }
    if (!seg->route_ids || !seg->offsets || !seg->sizes || !posting || !route_query)
        return ctx->fail(GOFANN_ERR_INVALID, "segment plan or posting arrays missing");
    if (!out_ids || !out_dists) return ctx->fail(GOFANN_ERR_INVALID, "posting scan outputs missing");
    if ((reinterpret_cast<uintptr_t>(posting_codes) | reinterpret_cast<uintptr_t>(posting_aux) |
         reinterpret_cast<uintptr_t>(posting_slab)) & 15u)
        return ctx->fail(GOFANN_ERR_INVALID, "posting-order arrays must be 16-byte aligned");

    const bool merged = seg->query_indptr != nullptr;
    uint32_t* scan_ids = out_ids;
    float* scan_dists = out_dists;
    uint32_t* scan_pass = pass_counts;
    const size_t slots_out = static_cast<size_t>(seg->count) * static_cast<size_t>(shortlist_k);
    if (merged) {
        const size_t bytes = slots_out * 8 + static_cast<size_t>(seg->count) * 4 + 64;
        unsigned char* buf = static_cast<unsigned char*>(ctx->scratch(Context::kScratchRange, bytes));
        if (!buf) return ctx->fail(GOFANN_ERR_NOMEM, "posting segment scratch allocation failed");
        scan_ids = reinterpret_cast<uint32_t*>(buf);
        scan_dists = reinterpret_cast<float*>(buf + slots_out * 4);
        scan_pass = reinterpret_cast<uint32_t*>(buf + slots_out * 8);
    }

    RangeScanArgs a{};
    a.pred = pred ? *pred : gofann_predicate_view{};
    a.routes.route_query = route_query;
    a.posting = posting;
    a.resident_rows = posting_rows;
    a.seg_route = seg->route_ids;
    a.seg_offset = seg->offsets;
    a.seg_size = seg->sizes;
    a.segments = seg->count;
    a.base_rows = rq->samples ? rq->samples : UINT32_MAX;
    a.k = shortlist_k;
    a.k_pow2 = pow2_at_least(shortlist_k);
    a.chunk = a.k_pow2 <= 1024 ? 1024 : 2048;
    a.slots = std::max(2 * a.k_pow2, a.k_pow2 + a.chunk);
    a.planes_bytes = rq->padded_dim;
    a.score_first = 0;
    a.out_ids = scan_ids;
    a.out_dists = scan_dists;
    a.pass_counts = merged || pass_counts ? scan_pass : nullptr;
    a.label_mode = kLabelSegments;
    a.slices = 1;
    a.pcodes = reinterpret_cast<const uint4*>(posting_codes);
    a.paux = reinterpret_cast<const uint4*>(posting_aux);
    a.pslab = reinterpret_cast<const uint4*>(posting_slab);
    a.pranges = posting_ranges;
    const size_t lds = 2 * static_cast<size_t>(a.planes_bytes) + static_cast<size_t>(a.slots) * 8 +
                       static_cast<size_t>(a.chunk) * 12;
    if (lds > static_cast<size_t>(ctx->lds_per_block))
        return ctx->fail(GOFANN_ERR_UNSUPPORTED, "posting scan LDS exceeds the workgroup limit");
    if (hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(lds)) != hipSuccess)
        return ctx->fail_hip("hipFuncSetAttribute posting scan");
    RabitqScanScorer sc = scan_scorer(rq, pre);
    void* kargs[] = {&a, &sc};
    if (hipLaunchKernel(kern, dim3(seg->count), dim3(kScanThreads), kargs, lds, ctx->stream) !=
        hipSuccess)
        return ctx->fail_hip("posting scan launch");
    if (!merged || seg->positions == 0) return GOFANN_OK;

    SegmentMergeArgs m;
    m.query_indptr = seg->query_indptr;
    m.stride = 0;
    m.positions = seg->positions;
    m.seg_ids = scan_ids;
    m.seg_dists = scan_dists;
    m.seg_pass = scan_pass;
    m.k = shortlist_k;
    m.k_pow2 = a.k_pow2;
    m.out_ids = out_ids;
    m.out_dists = out_dists;
    m.out_pass = pass_counts;
    const size_t mlds = static_cast<size_t>(2 * a.k_pow2) * 8;
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(segment_merge_kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(mlds)) !=
        hipSuccess)
        return ctx->fail_hip("hipFuncSetAttribute posting merge");
    hipLaunchKernelGGL(segment_merge_kernel, dim3(seg->positions), dim3(kScanThreads), mlds,
                       ctx->stream, m);
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("posting merge launch");
    return GOFANN_OK;
}

// The label-shared variant of rabitq_posting_scan_segments: `share` lists
// the plan's segments by the rows they scan (items of segments with equal
// offset and size; kShareRoutes of them per pass over the item's rows).  Needs the posting-order codes, aux
// and slab; the outputs equal rabitq_posting_scan_segments' bit for bit.
int rabitq_posting_scan_shared(Context* ctx, const gofann_rabitq_view* rq,
                               const gofann_rabitq_queries* pre,
                               const gofann_predicate_view* pred, const uint32_t* route_query,
                               const uint32_t* posting, uint64_t posting_rows,
                               const gofann_posting_segments* seg,
                               const gofann_posting_share* share, int shortlist_k,
                               const uint8_t* posting_codes, const uint32_t* posting_aux,
                               const uint32_t* posting_slab, const float* posting_ranges,
                               uint32_t* out_ids, float* out_dists, uint32_t* pass_counts)
{
    if (!share) return ctx->fail(GOFANN_ERR_INVALID, "share plan missing");
    if (!posting_codes || !posting_aux || !posting_slab)
        return ctx->fail(GOFANN_ERR_INVALID, "the shared scan reads posting-order codes, aux and slab");
    if (posting_ranges && !posting_slab)
        return ctx->fail(GOFANN_ERR_INVALID, "posting ranges need the posting slab");
    if (!rq || !pre || !rq->codes || !rq->factors || !rq->anchor_ids || rq->padded_dim == 0 ||
        rq->padded_dim % 128 != 0)
        return ctx->fail(GOFANN_ERR_INVALID, "RaBitQ view invalid for posting scan");
    if (!pre->q8 || !pre->scale || !pre->k1 || !pre->centroid_dists)
        return ctx->fail(GOFANN_ERR_INVALID, "prepared RaBitQ queries incomplete");
    if (!seg) return ctx->fail(GOFANN_ERR_INVALID, "segment plan missing");
    if (shortlist_k < 1 || shortlist_k > kShareMaxKp)
        return ctx->fail(GOFANN_ERR_UNSUPPORTED, "the shared scan takes shortlist_k <= 128");
    const void* kern = nullptr;
    switch (rq->padded_dim / 128) {
        case 1: kern = reinterpret_cast<const void*>(label_share_scan_kernel<1>); break;
        case 2: kern = reinterpret_cast<const void*>(label_share_scan_kernel<2>); break;
        case 4: kern = reinterpret_cast<const void*>(label_share_scan_kernel<4>); break;
        case 8: kern = reinterpret_cast<const void*>(label_share_scan_kernel<8>); break;
        default: return ctx->fail(GOFANN_ERR_UNSUPPORTED, "the shared scan takes padded_dim <= 1024");
    }
    if (seg->count == 0) {
        if (seg->query_indptr && seg->positions)
            return ctx->fail(GOFANN_ERR_INVALID, "segment plan has positions but no segments");
        return GOFANN_OK;
    }
    if (!seg->route_ids || !posting || !route_query)
        return ctx->fail(GOFANN_ERR_INVALID, "segment plan or posting arrays missing");
    if (!share->item_offsets || !share->item_sizes || !share->item_begin || !share->item_slots ||
        share->items == 0)
        return ctx->fail(GOFANN_ERR_INVALID, "share plan arrays missing");
    if (!out_ids || !out_dists) return ctx->fail(GOFANN_ERR_INVALID, "posting scan outputs missing");
    if ((reinterpret_cast<uintptr_t>(posting_codes) | reinterpret_cast<uintptr_t>(posting_aux) |
         reinterpret_cast<uintptr_t>(posting_slab)) & 15u)
        return ctx->fail(GOFANN_ERR_INVALID, "posting-order arrays must be 16-byte aligned");

    const bool merged = seg->query_indptr != nullptr;
    uint32_t* scan_ids = out_ids;
    float* scan_dists = out_dists;
    uint32_t* scan_pass = pass_counts;
    const size_t slots_out = static_cast<size_t>(seg->count) * static_cast<size_t>(shortlist_k);
    if (merged) {
        const size_t bytes = slots_out * 8 + static_cast<size_t>(seg->count) * 4 + 64;
        unsigned char* buf = static_cast<unsigned char*>(ctx->scratch(Context::kScratchRange, bytes));
        if (!buf) return ctx->fail(GOFANN_ERR_NOMEM, "posting segment scratch allocation failed");
        scan_ids = reinterpret_cast<uint32_t*>(buf);
        scan_dists = reinterpret_cast<float*>(buf + slots_out * 4);
        scan_pass = reinterpret_cast<uint32_t*>(buf + slots_out * 8);
    }
    ShareScanArgs a{};
    a.pred = pred ? *pred : gofann_predicate_view{};
    a.route_query = route_query;
    a.posting = posting;
    a.resident_rows = posting_rows;
    a.seg_route = seg->route_ids;
    a.item_offset = share->item_offsets;
    a.item_size = share->item_sizes;
    a.item_begin = share->item_begin;
    a.item_slots = share->item_slots;
    a.items = share->items;
    a.base_rows = rq->samples ? rq->samples : UINT32_MAX;
    a.k = shortlist_k;
    a.k_pow2 = pow2_at_least(shortlist_k);
    a.pcodes = reinterpret_cast<const uint4*>(posting_codes);
    a.paux = reinterpret_cast<const uint4*>(posting_aux);
    a.pslab = reinterpret_cast<const uint4*>(posting_slab);
    a.pranges = posting_ranges;
    a.out_ids = scan_ids;
    a.out_dists = scan_dists;
    a.pass_counts = merged || pass_counts ? scan_pass : nullptr;
    const size_t vecs = rq->padded_dim / 128;
    const size_t lds = static_cast<size_t>(kShareTile) * 28 +
                       static_cast<size_t>(kShareRoutes) * 8 * vecs * 16 +
                       static_cast<size_t>(kShareRoutes) * a.k * 8 +
                       static_cast<size_t>(kShareRoutes) * kWave * 4;
    if (lds > static_cast<size_t>(ctx->lds_per_block))
        return ctx->fail(GOFANN_ERR_UNSUPPORTED, "shared posting scan LDS exceeds the workgroup limit");
    if (hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(lds)) != hipSuccess)
        return ctx->fail_hip("hipFuncSetAttribute shared posting scan");
    RabitqScanScorer sc = scan_scorer(rq, pre);
    void* kargs[] = {&a, &sc};
    if (hipLaunchKernel(kern, dim3(share->items), dim3(kScanThreads), kargs, lds, ctx->stream) !=
        hipSuccess)
        return ctx->fail_hip("shared posting scan launch");
    if (!merged || seg->positions == 0) return GOFANN_OK;

    SegmentMergeArgs m;
    m.query_indptr = seg->query_indptr;
    m.stride = 0;
    m.positions = seg->positions;
    m.seg_ids = scan_ids;
    m.seg_dists = scan_dists;
    m.seg_pass = scan_pass;
    m.k = shortlist_k;
    m.k_pow2 = a.k_pow2;
    m.out_ids = out_ids;
    m.out_dists = out_dists;
    m.out_pass = pass_counts;
    const size_t mlds = static_cast<size_t>(2 * a.k_pow2) * 8;
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(segment_merge_kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(mlds)) !=
        hipSuccess)
        return ctx->fail_hip("hipFuncSetAttribute posting merge");
    hipLaunchKernelGGL(segment_merge_kernel, dim3(seg->positions), dim3(kScanThreads), mlds,
                       ctx->stream, m);
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("posting merge launch");
    return GOFANN_OK;
}

int rabitq_range_scan(Context* ctx, const gofann_rabitq_view* rq,
                      const gofann_rabitq_queries* pre, const gofann_predicate_view* pred,
                      const gofann_routes* routes, const uint32_t* posting,
                      uint64_t resident_rows, const gofann_posting_segments* seg,
                      int shortlist_k, int score_first, uint32_t* out_ids, float* out_dists,
                      uint32_t* pass_counts, const uint8_t* posting_codes,
                      const uint32_t* posting_aux)
{
    if ((posting_codes == nullptr) != (posting_aux == nullptr))
        return ctx->fail(GOFANN_ERR_INVALID, "posting codes and aux come together");
    if (!rq || !pre || !rq->codes || !rq->factors || !rq->anchor_ids || rq->padded_dim == 0 ||
        rq->padded_dim % 128 != 0)
        return ctx->fail(GOFANN_ERR_INVALID, "RaBitQ view invalid for range scan");
    if (!pre->q8 || !pre->scale || !pre->k1 || !pre->centroid_dists)
        return ctx->fail(GOFANN_ERR_INVALID, "prepared RaBitQ queries incomplete");
    if (!routes || !routes->route_query || !seg)
        return ctx->fail(GOFANN_ERR_INVALID, "range scan routes or segments missing");
    if (shortlist_k < 1 || shortlist_k > kRangeMaxShortlist)
        return ctx->fail(GOFANN_ERR_INVALID, "shortlist_k must be in [1, 4096]");
    if (!out_ids || !out_dists)
        return ctx->fail(GOFANN_ERR_INVALID, "range scan outputs missing");
    if (seg->count == 0) {
        if (seg->query_indptr && seg->positions)
            return ctx->fail(GOFANN_ERR_INVALID, "segment plan has positions but no segments");
        return GOFANN_OK;
    }
    if (!seg->route_ids || !seg->offsets || !seg->sizes || (seg->count && !posting))
        return ctx->fail(GOFANN_ERR_INVALID, "segment plan arrays missing");

    const bool merged = seg->query_indptr != nullptr;
    uint32_t* scan_ids = out_ids;
    float* scan_dists = out_dists;
    uint32_t* scan_pass = pass_counts;
    const size_t slots_out = static_cast<size_t>(seg->count) * static_cast<size_t>(shortlist_k);
    if (merged) {
        const size_t bytes = slots_out * 8 + static_cast<size_t>(seg->count) * 4 + 64;
        unsigned char* buf = static_cast<unsigned char*>(ctx->scratch(Context::kScratchRange, bytes));
        if (!buf) return ctx->fail(GOFANN_ERR_NOMEM, "range segment scratch allocation failed");
        scan_ids = reinterpret_cast<uint32_t*>(buf);
        scan_dists = reinterpret_cast<float*>(buf + slots_out * 4);
        scan_pass = reinterpret_cast<uint32_t*>(buf + slots_out * 8);
    }

    RangeScanArgs a;
    a.pred = pred ? *pred : gofann_predicate_view{};
    a.routes = *routes;
    a.posting = posting;
    a.resident_rows = resident_rows;
    a.seg_route = seg->route_ids;
    a.seg_offset = seg->offsets;
    a.seg_size = seg->sizes;
    a.segments = seg->count;
    a.base_rows = rq->samples;
    a.k = shortlist_k;
    a.k_pow2 = pow2_at_least(shortlist_k);
    // LDS pairs [0, k_pow2) hold the running list, [k_pow2, k_pow2 + chunk)
    // the chunk being scored; the rest stays padding.  At most 8 rows per
    // thread (the survivor gather keeps them in registers).
    a.chunk = a.k_pow2 <= 1024 ? 1024 : 2048;
    a.slots = pow2_at_least(a.k_pow2 + a.chunk);
    a.planes_bytes = rq->padded_dim;  // 8 bit planes of padded_dim bits
    a.score_first = score_first ? 1 : 0;
    a.out_ids = scan_ids;
    a.out_dists = scan_dists;
    a.pass_counts = scan_pass;
    a.label_mode = 0;
    a.cand_offsets = nullptr;
    a.cand_sizes = nullptr;
    a.slices = 1;
    // The thread-per-row kernel gathers (same results); the group kernel
    // streams the copies when given.
    a.pcodes = reinterpret_cast<const uint4*>(posting_codes);
    a.paux = reinterpret_cast<const uint4*>(posting_aux);
    a.pslab = nullptr;
    a.pranges = nullptr;
    if (a.chunk % kScanThreads != 0 || a.chunk / kScanThreads > 8 || a.slots < 2 * a.k_pow2 ||
        a.slots < a.k_pow2 + a.chunk)
        return ctx->fail(GOFANN_ERR_INVALID, "range scan chunk layout invalid");

    RabitqScanScorer sc = scan_scorer(rq, pre);

    // Group-per-row kernel when the row's 16-byte vectors split evenly over
    // a power-of-two group of <= 32 lanes, two vectors per lane at most;
    // thread-per-row kernel otherwise.
    const void* kern = group_scan_kernel(rq->padded_dim);
    size_t lds;
    if (kern) {
        // [0, kp) running list, [kp, kp + chunk) the chunk; the merges use
        // [0, 2 kp); then per chunk row f_rescale and the inner product.
        a.slots = std::max(2 * a.k_pow2, a.k_pow2 + a.chunk);
        lds = 2 * static_cast<size_t>(a.planes_bytes) + static_cast<size_t>(a.slots) * 8 +
              static_cast<size_t>(a.chunk) * 12;
    } else {
        kern = reinterpret_cast<const void*>(range_scan_kernel);
        lds = a.planes_bytes + static_cast<size_t>(a.slots) * 8;
    }
    if (lds > static_cast<size_t>(ctx->lds_per_block))
        return ctx->fail(GOFANN_ERR_UNSUPPORTED, "range scan LDS exceeds the workgroup limit");
    if (hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(lds)) != hipSuccess)
        return ctx->fail_hip("hipFuncSetAttribute range scan");
    void* kargs[] = {&a, &sc};
    if (hipLaunchKernel(kern, dim3(seg->count), dim3(kScanThreads), kargs, lds, ctx->stream) !=
        hipSuccess)
        return ctx->fail_hip("range scan launch");
    if (!merged) return GOFANN_OK;

    SegmentMergeArgs m;
    m.query_indptr = seg->query_indptr;
    m.stride = 0;
    m.positions = seg->positions;
    m.seg_ids = scan_ids;
    m.seg_dists = scan_dists;
    m.seg_pass = scan_pass;
    m.k = shortlist_k;
    m.k_pow2 = a.k_pow2;
    m.out_ids = out_ids;
    m.out_dists = out_dists;
    m.out_pass = pass_counts;
    if (seg->positions == 0) return GOFANN_OK;
    const size_t mlds = static_cast<size_t>(2 * a.k_pow2) * 8;
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(segment_merge_kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(mlds)) !=
        hipSuccess)
        return ctx->fail_hip("hipFuncSetAttribute segment merge");
    hipLaunchKernelGGL(segment_merge_kernel, dim3(seg->positions), dim3(kScanThreads), mlds,
                       ctx->stream, m);
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("segment merge launch");
    return GOFANN_OK;
}

}  // namespace gofann
