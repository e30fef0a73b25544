// range_posting.cpp -- host-side planning for range postings: the posting
// segment plan and the smallest-slice choice over an ordered range posting
// index.  Plain C++ over host arrays; no device calls.
//
// Segment plan: posting_segments::make_plan (src/execution/
// posting_segment_plan.h:20-51).  A posting of `rows` rows becomes
// max(1, ceil(rows / target_rows)) segments of near-equal length, the first
// rows % count of them one row longer, in posting order; query_indptr marks
// each posting's run of segments.
//
// Slice choice: range_posting::choose_smallest_slice (src/index/
// range_posting_index.cpp:277-312) with slice_bounds (:49-75).  For every
// active range (mode != 0) of a query row the slice of the dimension's
// ordered sample ids that satisfies it is found by binary search on the
// dimension's unique values (mode 1: values > lower, 2: values < upper,
// 3: lower <= value < upper); the smallest slice wins, ties to the lower
// range index.
#include <algorithm>
#include <cstdint>
#include <limits>

#include "gofann_hip.h"

namespace {

struct SliceBounds {
    uint64_t begin, end;
    bool ok;
};

SliceBounds slice_bounds(const float* values, const uint64_t* offsets, uint64_t unique,
                         uint8_t mode, float lower, float upper)
{
    const float* first = values;
    const float* last = values + unique;
    switch (mode) {
    case 1: first = std::upper_bound(values, values + unique, lower); break;
    case 2: last = std::lower_bound(values, values + unique, upper); break;
    case 3:
        first = std::lower_bound(values, values + unique, lower);
        last = std::lower_bound(first, values + unique, upper);
        break;
    default: return {0, 0, false};
    }
    return {offsets[first - values], offsets[last - values], true};
}

}  // namespace

extern "C" {

int gofann_posting_segment_plan(const uint32_t* route_ids, const uint64_t* offsets,
                                const uint64_t* sizes, uint32_t n, uint32_t target_rows,
                                uint32_t capacity, uint32_t* seg_route_ids,
                                uint32_t* seg_positions, uint64_t* seg_offsets,
                                uint64_t* seg_sizes, uint32_t* query_indptr,
                                uint32_t* out_count)
{
    if (target_rows == 0 || (n > 0 && (!route_ids || !offsets || !sizes)))
        return GOFANN_ERR_INVALID;
    uint64_t total = 0;
    for (uint32_t q = 0; q < n; ++q) {
        if (offsets[q] > std::numeric_limits<uint64_t>::max() - sizes[q])
            return GOFANN_ERR_UNSUPPORTED;
        const uint64_t parts = sizes[q] == 0 ? 1 : 1 + (sizes[q] - 1) / target_rows;
        total += parts;
        if (total > std::numeric_limits<uint32_t>::max()) return GOFANN_ERR_UNSUPPORTED;
    }
    if (out_count) *out_count = static_cast<uint32_t>(total);
    if (total > capacity || !seg_route_ids || !seg_positions || !seg_offsets || !seg_sizes ||
        !query_indptr)
        return GOFANN_ERR_INVALID;
    uint32_t at = 0;
    query_indptr[0] = 0;
    for (uint32_t q = 0; q < n; ++q) {
        const uint64_t rows = sizes[q];
        const uint64_t parts = rows == 0 ? 1 : 1 + (rows - 1) / target_rows;
        const uint64_t base_len = rows / parts;
        const uint64_t longer = rows % parts;  // the first `longer` parts get one more row
        uint64_t pos = offsets[q];
        for (uint64_t part = 0; part < parts; ++part) {
            const uint64_t len = base_len + (part < longer ? 1 : 0);
            seg_route_ids[at] = route_ids[q];
            seg_positions[at] = q;
            seg_offsets[at] = pos;
            seg_sizes[at] = len;
            pos += len;
            ++at;
        }
        query_indptr[q + 1] = at;
    }
    return GOFANN_OK;
}

int gofann_range_slices(const float* const* unique_values, const uint64_t* const* offsets,
                        const uint64_t* unique_counts, uint32_t range_count,
                        const uint8_t* modes, const float* lower, const float* upper,
                        uint32_t n, uint64_t* out)
{
    if (n == 0) return GOFANN_OK;
    if (!out || (range_count > 0 && (!unique_values || !offsets || !unique_counts || !modes ||
                                     !lower || !upper)))
        return GOFANN_ERR_INVALID;
    for (uint32_t q = 0; q < n; ++q) {
        uint64_t has = 0, active = 0, best_r = UINT32_MAX, best_begin = 0;
        uint64_t best_count = std::numeric_limits<uint64_t>::max();
        for (uint32_t r = 0; r < range_count; ++r) {
            const size_t f = static_cast<size_t>(q) * range_count + r;
            if (modes[f] == 0) continue;
            has = 1;
            ++active;
            if (!unique_values[r] || !offsets[r]) return GOFANN_ERR_INVALID;
            const SliceBounds b = slice_bounds(unique_values[r], offsets[r], unique_counts[r],
                                               modes[f], lower[f], upper[f]);
            if (!b.ok) return GOFANN_ERR_INVALID;  // unknown active mode
            const uint64_t cnt = b.end - b.begin;
            if (cnt < best_count || (cnt == best_count && r < best_r)) {
                best_r = r;
                best_begin = b.begin;
                best_count = cnt;
            }
        }
        uint64_t* o = out + static_cast<size_t>(q) * 5;
        o[0] = has;
        o[1] = active;
        o[2] = has ? best_r : UINT32_MAX;
        o[3] = has ? best_begin : 0;
        o[4] = has ? best_count : 0;
    }
    return GOFANN_OK;
}

}  // extern "C"
