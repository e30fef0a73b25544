// ref_shim.cpp -- C entry points over the reference's own host-compilable
// headers, compiled where they lie under the GO-FANN source tree (never
// copied).  TEST INFRASTRUCTURE ONLY: the resulting oracle/_ref library is a
// second checker for the oracle restatement; the product never loads it.
//
// Headers used (all plain C++ when not compiled by nvcc):
//   src/predicates/gpu_predicate_index.cuh   (View, contains, matches, priority)
//   src/predicates/range_filter.cuh          (range counting, filter bonuses)
//   src/search/common/posting_shortlist_heap.cuh
//   src/search/pq/pq_resident_posting.cuh    (bounds, candidate)
//   src/search/rabitq/rabitq_lowfreq_merge.h (merge_route_results_to_original)
//   src/data/fp16_l2.h                       (decode, scalar L2)
//   src/execution/posting_segment_plan.h     (posting segment plan)
//   src/index/range_posting_index.{h,cpp}    (FARPIDX1 loader, smallest slice)
//   src/index/graph_file_format.{h,cpp}      (FDRG graph file reader/writer)
//   include/smmh2.h                          (symmetric min-max heap)
//   include/bin_heap.h                       (binary max-heap push/pop)
//   src/search/common/native_visited_hash.cuh (visited hash)
//   src/planning/route_predicate_plan.h      (route residual compile; with
//                                             src/data/dataloader.h's inline
//                                             runtime and clause-table types)
// range_filter.cuh comes first: it defines __host__/__device__/__forceinline__
// for a host compiler, which the three device headers above need.
#include <cstdio>

#include "predicates/range_filter.cuh"
#include "predicates/gpu_predicate_index.cuh"
#include "smmh2.h"
#include "bin_heap.h"
#include "search/common/native_visited_hash.cuh"
#include "search/common/posting_shortlist_heap.cuh"
#include "search/pq/pq_resident_posting.cuh"
#include "search/rabitq/rabitq_lowfreq_merge.h"
#include "data/fp16_l2.h"
#include "execution/posting_segment_plan.h"
#include "index/range_posting_index.h"
#include "index/graph_file_format.h"
#include "planning/route_predicate_plan.h"

#include <cstdint>
#include <cstring>
#include <exception>
#include <string>
#include <vector>

namespace gp = go_fann::gpu_predicate;

namespace {
gp::View make_view(const uint32_t* route_offsets, const uint32_t* route_handles,
                   const void* clauses, const void* ranges, const uint8_t* route_enabled,
                   const float* base_ranges, uint32_t range_stride,
                   const uint32_t* csr_offsets, const uint32_t* csr_labels, uint32_t rows)
{
    gp::View v;
    v.route_offsets = route_offsets;
    v.route_handles = route_handles;
    v.clauses = static_cast<const gp::Clause*>(clauses);
    v.ranges = static_cast<const gp::RangeAtom*>(ranges);
    v.route_enabled = route_enabled;
    v.base_ranges = base_ranges;
    v.range_stride = range_stride;
    v.csr_offsets = csr_offsets;
    v.csr_labels = csr_labels;
    v.rows = rows;
    return v;
}
}  // namespace

namespace {

// Result-heap entry: KernelPair<float, uint32_t> (warp_kernel.cuh:18-26)
// orders on `first` only; warp_kernel.cuh itself needs the CUDA runtime, so
// the pair type is written out here with that comparison.
struct RefResultPair {
    float first;
    uint32_t second;
    bool operator<(const RefResultPair& o) const { return first < o.first; }
    bool operator>(const RefResultPair& o) const { return first > o.first; }
};
static_assert(sizeof(RefResultPair) == 8, "result pair layout");

constexpr int kRefHashCapacity = 4096;  // backend_pq.cu:194

}  // namespace

extern "C" {

// smmh2 over the reference's 12-byte BiasedPair (first, second, base),
// the frontier entry of the biased PQ/RaBitQ kernels.
void ref_smmh2_insert(void* heap, int* size, const void* entry)
{
    gp::BiasedPair e = *static_cast<const gp::BiasedPair*>(entry);
    smmh2::insert(static_cast<gp::BiasedPair*>(heap), *size, e);
}

void ref_smmh2_pop_max(void* heap, int* size, void* out)
{
    *static_cast<gp::BiasedPair*>(out) = smmh2::pop_max(static_cast<gp::BiasedPair*>(heap), *size);
}

void ref_smmh2_pop_min(void* heap, int* size, void* out)
{
    *static_cast<gp::BiasedPair*>(out) = smmh2::pop_min(static_cast<gp::BiasedPair*>(heap), *size);
}

// bin_heap.h over [begin, begin + size): push after appending, pop.
void ref_bin_heap_push(void* begin, int size_after_append)
{
    auto* b = static_cast<RefResultPair*>(begin);
    ::push_heap(b, b + size_after_append);
}

void ref_bin_heap_pop(void* begin, int size, void* out)
{
    auto* b = static_cast<RefResultPair*>(begin);
    *static_cast<RefResultPair*>(out) = ::pop_heap(b, b + size);
}

uint32_t ref_hash_code(uint32_t value)
{
    return go_fann::native_visited_hash::code<kRefHashCapacity>(value);
}

// clear as a 32-lane warp runs it: lanes 0..31 each stride by 32.
void ref_hash_clear(uint32_t* table)
{
    for (int lane = 0; lane < 32; ++lane)
        go_fann::native_visited_hash::clear<kRefHashCapacity>(table, lane);
}

int ref_hash_test(const uint32_t* table, uint32_t value)
{
    return go_fann::native_visited_hash::test<kRefHashCapacity>(table, value) ? 1 : 0;
}

void ref_hash_add(uint32_t* table, uint32_t value)
{
    go_fann::native_visited_hash::add<kRefHashCapacity>(table, value);
}

int ref_pred_matches(const uint32_t* route_offsets, const uint32_t* route_handles,
                     const void* clauses, const void* ranges, const uint8_t* route_enabled,
                     const float* base_ranges, uint32_t range_stride,
                     const uint32_t* csr_offsets, const uint32_t* csr_labels, uint32_t rows,
                     uint32_t route, uint32_t sample)
{
    const gp::View v = make_view(route_offsets, route_handles, clauses, ranges, route_enabled,
                                 base_ranges, range_stride, csr_offsets, csr_labels, rows);
    return gp::matches(v, route, sample) ? 1 : 0;
}

int ref_pred_enabled(const uint32_t* route_offsets, const uint8_t* route_enabled,
                     const uint32_t* csr_offsets, uint32_t route)
{
    gp::View v;
    v.route_offsets = route_offsets;
    v.route_enabled = route_enabled;
    v.csr_offsets = csr_offsets;
    return gp::enabled(v, route) ? 1 : 0;
}

int ref_csr_contains(const uint32_t* csr_offsets, const uint32_t* csr_labels, uint32_t rows,
                     uint32_t handle, uint32_t sample)
{
    gp::View v;
    v.csr_offsets = csr_offsets;
    v.csr_labels = csr_labels;
    v.rows = rows;
    return gp::contains(v, handle, sample) ? 1 : 0;
}

float ref_priority(float base, float penalty, int pass, int* saturated)
{
    bool s = false;
    const float r = gp::priority(base, penalty, pass != 0, s);
    if (saturated) *saturated = s ? 1 : 0;
    return r;
}

// Pool entries are {first, second, base} triples (gp::BiasedPair layout).
float ref_minimum_pending_base(const void* pool, int size, const void* current,
                               const void* next, int current_valid, int next_valid)
{
    const auto* p = static_cast<const gp::BiasedPair*>(pool);
    return gp::minimum_pending_base(p, size, *static_cast<const gp::BiasedPair*>(current),
                                    *static_cast<const gp::BiasedPair*>(next),
                                    current_valid != 0, next_valid != 0,
                                    [](uint32_t payload) { return (payload & 0x80000000u) == 0; });
}

uint32_t ref_count_matching_ranges(const uint8_t* modes, const float* lower, const float* upper,
                                   const float* base_values, uint32_t route, uint32_t sample,
                                   uint32_t count)
{
    return go_fann::range_filter::count_matching_active_ranges(modes, lower, upper, base_values,
                                                               route, sample, count);
}

uint32_t ref_count_active_ranges(const uint8_t* modes, uint32_t route, uint32_t count)
{
    return go_fann::range_filter::count_active_ranges(modes, route, count);
}

float ref_apply_filter_bonuses(float dist, int bit_match, uint32_t matched, float bit_bonus,
                               float range_bonus)
{
    return go_fann::range_filter::apply_filter_bonuses(dist, bit_match != 0, matched, bit_bonus,
                                                       range_bonus);
}

int ref_shortlist_can_enter(float dist, uint32_t id, const float* d, const uint32_t* ids, int k)
{
    return go_fann::posting_shortlist_heap::can_enter<uint32_t>(dist, id, d, ids, k) ? 1 : 0;
}

void ref_shortlist_insert(float dist, uint32_t id, float* d, uint32_t* ids, int k)
{
    go_fann::posting_shortlist_heap::insert<uint32_t>(dist, id, d, ids, k);
}

void ref_shortlist_sort(float* d, uint32_t* ids, int k)
{
    go_fann::posting_shortlist_heap::sort<uint32_t>(d, ids, k);
}

// pq_resident_posting::View fields in declaration order.
int ref_pq_resident_probe(const uint32_t* group_offsets, const uint32_t* group_sizes,
                          const uint32_t* sample_ids, const uint64_t* row_masks,
                          const uint32_t* query_groups, const uint64_t* query_masks,
                          const uint8_t* range_modes, const float* range_lower,
                          const float* range_upper, const float* base_ranges, uint32_t groups,
                          uint32_t rows, uint32_t samples, uint32_t routes,
                          uint32_t range_count, uint32_t route, uint32_t index,
                          uint32_t* out_begin, uint32_t* out_count)
{
    go_fann::pq_resident_posting::View v{group_offsets, group_sizes, sample_ids, row_masks,
                                         query_groups, query_masks, range_modes, range_lower,
                                         range_upper, base_ranges, groups, rows, samples,
                                         routes, range_count, true};
    uint32_t begin = 0, count = 0;
    go_fann::pq_resident_posting::bounds(v, route, begin, count);
    *out_begin = begin;
    *out_count = count;
    return index < count ? static_cast<int>(go_fann::pq_resident_posting::candidate(
                               v, route, begin + index))
                         : -1;
}

float ref_fp16_decode(uint16_t h) { return go_fann::fp16_l2::decode(h); }

float ref_fp16_l2_scalar(const uint16_t* base, const float* query, uint32_t cols)
{
    return go_fann::fp16_l2::scalar(base, query, cols);
}

// Route merge over dense [routes][width] results; outputs [queries][topk].
int ref_merge_routes(const uint32_t* route_to_query, uint32_t routes, uint32_t queries,
                     const uint32_t* route_ids, const float* route_dists, uint32_t width,
                     uint32_t topk, uint32_t* out_ids, float* out_dists)
{
    std::vector<uint32_t> r2q(route_to_query, route_to_query + routes);
    std::vector<std::vector<uint32_t>> ids(routes);
    std::vector<std::vector<float>> dists(routes);
    std::vector<int> steps(routes, 1);
    for (uint32_t r = 0; r < routes; ++r) {
        ids[r].assign(route_ids + size_t(r) * width, route_ids + size_t(r + 1) * width);
        dists[r].assign(route_dists + size_t(r) * width, route_dists + size_t(r + 1) * width);
    }
    std::vector<std::vector<uint32_t>> merged;
    std::vector<int> merged_steps;
    std::vector<std::vector<float>> merged_d;
    const auto strategy = go_fann::backend_rabitq::lowfreq_merge::merge_route_results_to_original(
        r2q, queries, ids, dists, steps, topk, merged, merged_steps, &merged_d);
    for (uint32_t q = 0; q < queries; ++q) {
        for (uint32_t i = 0; i < topk; ++i) {
            out_ids[size_t(q) * topk + i] = i < merged[q].size() ? merged[q][i] : UINT32_MAX;
            out_dists[size_t(q) * topk + i] = i < merged_d[q].size() ? merged_d[q][i] : 3.402823466e+38f;
        }
    }
    return static_cast<int>(strategy);
}

// posting_segments::make_plan; returns the segment count or -1 when it throws.
int ref_segment_plan(const uint32_t* route_ids, const uint64_t* offsets, const uint64_t* sizes,
                     uint32_t n, uint32_t target_rows, uint32_t capacity, uint32_t* seg_routes,
                     uint32_t* seg_positions, uint64_t* seg_offsets, uint64_t* seg_sizes,
                     uint32_t* query_indptr)
{
    try {
        const auto plan = go_fann::posting_segments::make_plan(
            std::vector<uint32_t>(route_ids, route_ids + n),
            std::vector<uint64_t>(offsets, offsets + n), std::vector<uint64_t>(sizes, sizes + n),
            target_rows);
        const size_t count = plan.route_ids.size();
        if (count > capacity) return static_cast<int>(count);
        std::memcpy(seg_routes, plan.route_ids.data(), count * sizeof(uint32_t));
        std::memcpy(seg_positions, plan.query_positions.data(), count * sizeof(uint32_t));
        std::memcpy(seg_offsets, plan.offsets.data(), count * sizeof(uint64_t));
        std::memcpy(seg_sizes, plan.sizes.data(), count * sizeof(uint64_t));
        std::memcpy(query_indptr, plan.query_indptr.data(), (n + 1) * sizeof(uint32_t));
        return static_cast<int>(count);
    } catch (const std::exception&) {
        return -1;
    }
}

// Loads a FARPIDX1 file with the reference loader (all of its validation)
// and chooses the smallest slice for each query row of the range table.
// out[q] = {has_active, active_dims, range_index, begin, count}.  Returns 0,
// or -1 with the loader's message in `error` (NUL-terminated, truncated).
int ref_range_slices(const char* path, const uint8_t* modes, const float* lower,
                     const float* upper, uint32_t rows, uint32_t range_count, uint64_t* out,
                     uint64_t* row_count, char* error, uint32_t error_bytes)
{
    namespace rp = go_fann::range_posting;
    try {
        const rp::Index index = rp::Index::load(path);
        *row_count = index.row_count();
        ::QueryRangeTable table;
        table.rows = rows;
        table.range_count = range_count;
        const size_t n = static_cast<size_t>(rows) * range_count;
        table.modes.assign(modes, modes + n);
        table.lower_bounds.assign(lower, lower + n);
        table.upper_bounds.assign(upper, upper + n);
        for (uint32_t q = 0; q < rows; ++q) {
            const rp::Slice s = rp::choose_smallest_slice(index, table, q);
            out[q * 5 + 0] = s.has_active_range ? 1 : 0;
            out[q * 5 + 1] = s.active_dimension_count;
            out[q * 5 + 2] = s.range_index;
            out[q * 5 + 3] = s.begin;
            out[q * 5 + 4] = s.count;
        }
        return 0;
    } catch (const std::exception& e) {
        if (error && error_bytes) {
            std::strncpy(error, e.what(), error_bytes - 1);
            error[error_bytes - 1] = 0;
        }
        return -1;
    }
}

namespace {
int ref_error(const std::exception& e, char* error, uint32_t error_bytes)
{
    if (error && error_bytes) {
        std::strncpy(error, e.what(), error_bytes - 1);
        error[error_bytes - 1] = 0;
    }
    return -1;
}
}  // namespace

// FDRG: the header as read_graph_file_header returns it (40 bytes).
int ref_graph_file_header(const char* path, void* out, char* error, uint32_t error_bytes)
{
    try {
        const go_fann::graph_file::GraphFileHeader h = go_fann::graph_file::read_graph_file_header(path);
        std::memcpy(out, &h, sizeof(h));
        return 0;
    } catch (const std::exception& e) {
        return ref_error(e, error, error_bytes);
    }
}

// FDRG: load_graph_file_as_contiguous_matrix into out (capacity words);
// *rows/*cols receive the shape.
int ref_graph_file_load(const char* path, uint32_t* out, uint64_t capacity, uint64_t* rows,
                        uint64_t* cols, char* error, uint32_t error_bytes)
{
    try {
        const auto m = go_fann::graph_file::load_graph_file_as_contiguous_matrix(path);
        *rows = m.rows;
        *cols = m.cols;
        if (m.data.size() > capacity) return -2;
        if (!m.data.empty()) std::memcpy(out, m.data.data(), m.data.size() * sizeof(uint32_t));
        return 0;
    } catch (const std::exception& e) {
        return ref_error(e, error, error_bytes);
    }
}

// FDRG: GraphFileSequentialWriter, rows appended in chunks of `chunk`.
int ref_graph_file_write(const char* path, const uint32_t* rows, uint64_t row_count, uint32_t degree,
                         uint64_t chunk, char* error, uint32_t error_bytes)
{
    try {
        go_fann::graph_file::GraphFileSequentialWriter w(path, row_count, degree);
        for (uint64_t r = 0; r < row_count; r += chunk) {
            const uint64_t n = row_count - r < chunk ? row_count - r : chunk;
            w.append_rows(rows + r * degree, n);
        }
        w.close();
        return 0;
    } catch (const std::exception& e) {
        return ref_error(e, error, error_bytes);
    }
}

int ref_graph_file_convert_legacy(const char* legacy_path, const char* path, char* error,
                                  uint32_t error_bytes)
{
    try {
        go_fann::graph_file::convert_legacy_graph_file(legacy_path, path);
        return 0;
    } catch (const std::exception& e) {
        return ref_error(e, error, error_bytes);
    }
}

// route_predicate::compile (route_predicate_plan.h:175-315) for graph routes
// (producer 0) or label-posting routes (producer 1) that own DNF clauses of
// their original query, on an ungrouped label layout (group g is label g).
// Query q owns clauses [q_indptr[q], q_indptr[q+1]); clause c has labels
// [label_indptr[c], label_indptr[c+1]) and uses the query's range row when
// uses_range[c].  Route r: original query route_query[r], anchor label
// route_anchor[r] (its group), owned clauses [route_clause_indptr[r], +1).
// label_rows[l]: posting size of label l (label-posting producer).
//
// Output, u32 words per route: available, entailed, clause count, then per
// clause: label count, labels, range count, then per atom: dimension,
// mode, lower bits, upper bits.  *out_words receives the length; returns
// -2 when it exceeds `capacity`, -1 on a reference exception.
int ref_route_compile(int producer, uint32_t queries, const uint64_t* q_indptr,
                      const uint64_t* label_indptr, const uint32_t* labels,
                      const uint8_t* uses_range, uint32_t range_count, const uint8_t* modes,
                      const float* lower, const float* upper, uint32_t num_labels,
                      uint32_t samples, const uint32_t* label_rows, uint32_t routes,
                      const uint32_t* route_query, const uint32_t* route_anchor,
                      const uint64_t* route_clause_indptr, const uint32_t* route_clause_ids,
                      uint32_t* out, uint64_t capacity, uint64_t* out_words, char* error,
                      uint32_t error_bytes)
{
    try {
        namespace rp = go_fann::route_predicate;
        GraphRuntime rt;
        const uint64_t clauses = q_indptr[queries];
        rt.original_query_count = queries;
        rt.base_range_count = range_count;
        rt.base_vectors.rows = samples;
        rt.data_labels.rows = samples;
        rt.data_labels.cols = num_labels;
        rt.query_vectors.rows = routes;
        auto& t = rt.original_query_clauses;
        t.rows = queries;
        t.query_indptr.assign(q_indptr, q_indptr + queries + 1);
        t.label_indptr.assign(label_indptr, label_indptr + clauses + 1);
        t.labels.assign(labels, labels + label_indptr[clauses]);
        t.top_branch_ids.assign(clauses, 0u);
        t.uses_original_range.assign(uses_range, uses_range + clauses);
        auto& qr = rt.original_query_ranges;
        qr.rows = queries;
        qr.range_count = range_count;
        qr.modes.assign(modes, modes + static_cast<size_t>(queries) * range_count);
        qr.lower_bounds.assign(lower, lower + static_cast<size_t>(queries) * range_count);
        qr.upper_bounds.assign(upper, upper + static_cast<size_t>(queries) * range_count);
        rt.group_layout.groups.resize(num_labels);
        rt.group_layout.label_to_group.resize(num_labels);
        for (uint32_t l = 0; l < num_labels; ++l) {
            rt.group_layout.groups[l] = {l};
            rt.group_layout.label_to_group[l] = l;
        }
        rt.route_to_original_query.assign(route_query, route_query + routes);
        rt.query_group_ids.assign(route_anchor, route_anchor + routes);
        rt.query_filter_labels.assign(route_anchor, route_anchor + routes);
        rt.route_clause_indptr.assign(route_clause_indptr, route_clause_indptr + routes + 1);
        rt.route_clause_ids.assign(route_clause_ids, route_clause_ids + route_clause_indptr[routes]);
        rp::Producer prod = rp::Producer::Graph;
        if (producer == 0) {
            rt.high_query_indices.resize(routes);
            for (uint32_t r = 0; r < routes; ++r) rt.high_query_indices[r] = r;
        } else {
            prod = rp::Producer::LabelPosting;
            rt.query_is_lowfreq.assign(routes, 1);
            rt.route_providers.assign(routes, QueryRouteProvider::Label);
            rt.route_candidate_sources.assign(routes, QueryCandidateSource::LabelPosting);
            rt.route_execution_modes.assign(routes, QueryRouteExecution::GpuResidentScan);
            auto& ix = rt.lowfreq_index;
            ix.group_count = num_labels;
            ix.label_size.assign(label_rows, label_rows + num_labels);
            ix.label_offset.resize(num_labels);
            uint64_t total = 0;
            for (uint32_t l = 0; l < num_labels; ++l) {
                ix.label_offset[l] = static_cast<uint32_t>(total);
                total += label_rows[l];
            }
            ix.total_rows = static_cast<uint32_t>(total);
            ix.sample_ids.assign(total, 0u);
            ix.row_filter_mask.assign(total, 0ull);
        }
        const rp::Plan plan = rp::compile(rt, prod);
        std::vector<uint32_t> w;
        for (const rp::Route& route : plan.routes) {
            w.push_back(route.available ? 1u : 0u);
            w.push_back(route.entailed ? 1u : 0u);
            w.push_back(static_cast<uint32_t>(route.clauses.size()));
            for (const rp::Clause& c : route.clauses) {
                w.push_back(static_cast<uint32_t>(c.labels.size()));
                w.insert(w.end(), c.labels.begin(), c.labels.end());
                w.push_back(static_cast<uint32_t>(c.ranges.size()));
                for (const rp::RangeAtom& a : c.ranges) {
                    uint32_t lo, hi;
                    std::memcpy(&lo, &a.lower, 4);
                    std::memcpy(&hi, &a.upper, 4);
                    w.push_back(a.dimension);
                    w.push_back(a.mode);
                    w.push_back(lo);
                    w.push_back(hi);
                }
            }
        }
        *out_words = w.size();
        if (w.size() > capacity) return -2;
        std::memcpy(out, w.data(), w.size() * 4);
        return 0;
    } catch (const std::exception& e) {
        return ref_error(e, error, error_bytes);
    }
}

}  // extern "C"
