// gofann_abi.cpp -- extern "C" entry points of gofann_hip.h.  Validates
// arguments, maps them to the kernel launchers and converts every failure
// into a status code plus a message (no exception crosses the ABI).
#include <hip/hip_runtime.h>

#include <new>
#include <string>

#include "gofann_hip.h"
#include "gofann_internal.hpp"

namespace gofann {

void* Context::scratch(int slot, size_t bytes)
{
    if (slot < 0 || slot >= kScratchCount) return nullptr;
    if (scratch_bytes[slot] >= bytes && scratch_ptr[slot] != nullptr) return scratch_ptr[slot];
    if (scratch_ptr[slot] != nullptr) {
        // The stream may still read the old buffer.
        if (hipStreamSynchronize(stream) != hipSuccess) return nullptr;
        (void)hipFree(scratch_ptr[slot]);
        scratch_ptr[slot] = nullptr;
        scratch_bytes[slot] = 0;
    }
    void* p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    scratch_ptr[slot] = p;
    scratch_bytes[slot] = bytes;
    return p;
}

}  // namespace gofann

using gofann::Context;

namespace {
Context* as_ctx(gofann_ctx* c) { return reinterpret_cast<Context*>(c); }

template <class F>
int guarded(gofann_ctx* c, F&& f)
{
    if (c == nullptr) return GOFANN_ERR_INVALID;
    try {
        return f(as_ctx(c));
    } catch (const std::bad_alloc&) {
        return as_ctx(c)->fail(GOFANN_ERR_NOMEM, "host allocation failed");
    } catch (const std::exception& e) {
        return as_ctx(c)->fail(GOFANN_ERR_INVALID, e.what());
    }
}
}  // namespace

extern "C" {

int gofann_create(int device, gofann_ctx** out)
{
    if (out == nullptr) return GOFANN_ERR_INVALID;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) return GOFANN_ERR_HIP;
    if (hipSetDevice(device) != hipSuccess) return GOFANN_ERR_HIP;
    Context* ctx = new (std::nothrow) Context();
    if (ctx == nullptr) return GOFANN_ERR_NOMEM;
    ctx->device = device;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) {
        delete ctx;
        return GOFANN_ERR_HIP;
    }
    ctx->compute_units = prop.multiProcessorCount;
    ctx->lds_per_block = static_cast<int>(prop.sharedMemPerBlock);
    int per_cu = 0;
    if (hipDeviceGetAttribute(&per_cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, device) !=
            hipSuccess ||
        per_cu <= 0)
        per_cu = ctx->lds_per_block;
    ctx->lds_per_cu = per_cu;
    gofann::noalloc_setup(device);
    *out = reinterpret_cast<gofann_ctx*>(ctx);
    return GOFANN_OK;
}

void gofann_destroy(gofann_ctx* c)
{
    if (c == nullptr) return;
    Context* ctx = as_ctx(c);
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    gofann::destroy_blas(ctx);
    for (int i = 0; i < Context::kScratchCount; ++i)
        if (ctx->scratch_ptr[i]) (void)hipFree(ctx->scratch_ptr[i]);
    delete ctx;
}

const char* gofann_last_error(const gofann_ctx* c)
{
    if (c == nullptr) return "null context";
    return reinterpret_cast<const Context*>(c)->error.c_str();
}

int gofann_set_stream(gofann_ctx* c, void* stream)
{
    return guarded(c, [&](Context* ctx) {
        // Work queued on the previous stream may still read the context's
        // scratch buffers, which later calls (on the new stream) may free
        // when they grow; drain it before switching.
        if (ctx->stream != static_cast<hipStream_t>(stream) &&
            hipStreamSynchronize(ctx->stream) != hipSuccess)
            return ctx->fail_hip("set_stream: synchronize the previous stream");
        ctx->stream = static_cast<hipStream_t>(stream);
        return GOFANN_OK;
    });
}

int gofann_synchronize(gofann_ctx* c)
{
    return guarded(c, [&](Context* ctx) {
        if (hipStreamSynchronize(ctx->stream) != hipSuccess) return ctx->fail_hip("synchronize");
        return GOFANN_OK;
    });
}

int gofann_device_info(gofann_ctx* c, int* compute_units, int* lds_bytes)
{
    return guarded(c, [&](Context* ctx) {
        if (compute_units) *compute_units = ctx->compute_units;
        if (lds_bytes) *lds_bytes = ctx->lds_per_cu;
        return GOFANN_OK;
    });
}

int gofann_last_placement(gofann_ctx* c, int* table_in_lds, int* hash_in_lds, int* lds_bytes,
                          int* resident_per_cu)
{
    return guarded(c, [&](Context* ctx) {
        if (table_in_lds) *table_in_lds = ctx->last_table_in_lds;
        if (hash_in_lds) *hash_in_lds = ctx->last_hash_in_lds;
        if (lds_bytes) *lds_bytes = ctx->last_lds_bytes;
        if (resident_per_cu) *resident_per_cu = ctx->last_resident;
        return GOFANN_OK;
    });
}

int gofann_pq_search(gofann_ctx* c, const gofann_pq_view* pq, const void* queries, int query_elem,
                     const gofann_graph_view* graph, const gofann_predicate_view* predicate,
                     const gofann_routes* routes, const gofann_search_params* params,
                     uint32_t* out_ids, float* out_dists, gofann_route_stats* stats)
{
    return guarded(c, [&](Context* ctx) {
        if (!out_ids || !out_dists) return ctx->fail(GOFANN_ERR_INVALID, "null outputs");
        return gofann::pq_search(ctx, pq, queries, query_elem, graph, predicate, routes, params,
                                 out_ids, out_dists, stats);
    });
}

int gofann_rabitq_prepare_queries(gofann_ctx* c, const gofann_rabitq_view* rq,
                                  const float* queries, uint32_t count, const float* rotation,
                                  gofann_rabitq_queries* out)
{
    return guarded(c, [&](Context* ctx) {
        return gofann::rabitq_prepare(ctx, rq, queries, count, rotation, out);
    });
}

int gofann_rabitq_search(gofann_ctx* c, const gofann_rabitq_view* rq,
                         const gofann_rabitq_queries* prepared, const gofann_graph_view* graph,
                         const gofann_predicate_view* predicate, const gofann_routes* routes,
                         const gofann_search_params* params, uint32_t* out_ids, float* out_dists,
                         gofann_route_stats* stats)
{
    return guarded(c, [&](Context* ctx) {
        if (!out_ids || !out_dists) return ctx->fail(GOFANN_ERR_INVALID, "null outputs");
        return gofann::rabitq_search(ctx, rq, prepared, graph, predicate, routes, params, out_ids,
                                     out_dists, stats);
    });
}

int gofann_pq_posting_scan(gofann_ctx* c, const gofann_pq_view* pq, const void* queries,
                           int query_elem, const gofann_predicate_view* predicate,
                           const uint32_t* route_query, const uint32_t* cand_ids,
                           const uint32_t* cand_offsets, const uint32_t* cand_sizes,
                           uint32_t routes, int shortlist_k, uint32_t* out_ids, float* out_dists,
                           uint32_t* pass_counts)
{
    return guarded(c, [&](Context* ctx) {
        if (routes > 0 && (!route_query || !cand_ids || !cand_offsets || !cand_sizes || !out_ids ||
                           !out_dists))
            return ctx->fail(GOFANN_ERR_INVALID, "posting scan arrays missing");
        return gofann::pq_posting_scan(ctx, pq, queries, query_elem, predicate, route_query,
                                       cand_ids, cand_offsets, cand_sizes, routes, shortlist_k,
                                       out_ids, out_dists, pass_counts);
    });
}

int gofann_rabitq_posting_scan(gofann_ctx* c, const gofann_rabitq_view* rq,
                               const gofann_rabitq_queries* prepared,
                               const gofann_predicate_view* predicate,
                               const uint32_t* route_query, const uint32_t* cand_ids,
                               const uint32_t* cand_offsets, const uint32_t* cand_sizes,
                               uint32_t routes, int shortlist_k, uint32_t* out_ids,
                               float* out_dists, uint32_t* pass_counts)
{
    return guarded(c, [&](Context* ctx) {
        if (routes > 0 && (!route_query || !cand_ids || !cand_offsets || !cand_sizes || !out_ids ||
                           !out_dists))
            return ctx->fail(GOFANN_ERR_INVALID, "posting scan arrays missing");
        return gofann::rabitq_posting_scan(ctx, rq, prepared, predicate, route_query, cand_ids,
                                           cand_offsets, cand_sizes, routes, shortlist_k, out_ids,
                                           out_dists, pass_counts);
    });
}

int gofann_exact_search(gofann_ctx* c, const void* base, int base_elem, uint32_t dim,
                        uint32_t samples, const void* queries, const gofann_graph_view* graph,
                        const uint32_t* label_size, const gofann_predicate_view* predicate,
                        const gofann_routes* routes, const gofann_exact_params* params,
                        uint32_t* out_ids, float* out_dists, gofann_route_stats* stats)
{
    return guarded(c, [&](Context* ctx) {
        return gofann::exact_search(ctx, base, base_elem, dim, samples, queries, graph,
                                    label_size, predicate, routes, params, out_ids, out_dists,
                                    stats);
    });
}

int gofann_exact_search_noalloc(gofann_ctx* c, const void* base, int base_elem, uint32_t dim,
                                uint32_t samples, const void* queries,
                                const gofann_graph_view* graph, const uint32_t* label_size,
                                const gofann_predicate_view* predicate,
                                const gofann_routes* routes, const gofann_exact_params* params,
                                uint32_t* out_ids, float* out_dists, gofann_route_stats* stats)
{
    return guarded(c, [&](Context* ctx) {
        return gofann::exact_search_noalloc(ctx, base, base_elem, dim, samples, queries, graph,
                                            label_size, predicate, routes, params, out_ids,
                                            out_dists, stats);
    });
}

int gofann_rabitq_range_scan(gofann_ctx* c, const gofann_rabitq_view* rq,
                             const gofann_rabitq_queries* prepared,
                             const gofann_predicate_view* predicate, const gofann_routes* routes,
                             const uint32_t* posting_sample_ids, uint64_t resident_rows,
                             const gofann_posting_segments* segments, int shortlist_k,
                             int score_first, uint32_t* out_ids, float* out_dists,
                             uint32_t* pass_counts)
{
    return guarded(c, [&](Context* ctx) {
        return gofann::rabitq_range_scan(ctx, rq, prepared, predicate, routes, posting_sample_ids,
                                         resident_rows, segments, shortlist_k, score_first,
                                         out_ids, out_dists, pass_counts);
    });
}

int gofann_rabitq_posting_rows(gofann_ctx* c, const gofann_rabitq_view* rq,
                               const uint32_t* posting_sample_ids, uint64_t rows,
                               uint8_t* out_codes, uint32_t* out_aux)
{
    return guarded(c, [&](Context* ctx) {
        return gofann::rabitq_posting_rows(ctx, rq, posting_sample_ids, rows, out_codes, out_aux);
    });
}

int gofann_rabitq_range_scan_resident(gofann_ctx* c, const gofann_rabitq_view* rq,
                                      const gofann_rabitq_queries* prepared,
                                      const gofann_predicate_view* predicate,
                                      const gofann_routes* routes,
                                      const uint32_t* posting_sample_ids, uint64_t resident_rows,
                                      const uint8_t* posting_codes, const uint32_t* posting_aux,
                                      const gofann_posting_segments* segments, int shortlist_k,
                                      int score_first, uint32_t* out_ids, float* out_dists,
                                      uint32_t* pass_counts)
{
    return guarded(c, [&](Context* ctx) {
        if (!posting_codes || !posting_aux)
            return ctx->fail(GOFANN_ERR_INVALID, "posting codes and aux required");
        return gofann::rabitq_range_scan(ctx, rq, prepared, predicate, routes, posting_sample_ids,
                                         resident_rows, segments, shortlist_k, score_first,
                                         out_ids, out_dists, pass_counts, posting_codes,
                                         posting_aux);
    });
}

int gofann_posting_predicate_rows(gofann_ctx* c, const gofann_predicate_view* predicate,
                                  const uint32_t* posting_sample_ids, uint64_t rows,
                                  uint32_t* out_slab, float* out_ranges)
{
    return guarded(c, [&](Context* ctx) {
        return gofann::posting_predicate_rows(ctx, predicate, posting_sample_ids, rows, out_slab,
                                              out_ranges);
    });
}

int gofann_rabitq_posting_scan_segments(gofann_ctx* c, const gofann_rabitq_view* rq,
                                        const gofann_rabitq_queries* prepared,
                                        const gofann_predicate_view* predicate,
                                        const uint32_t* route_query,
                                        const uint32_t* posting_sample_ids, uint64_t posting_rows,
                                        const gofann_posting_segments* segments, int shortlist_k,
                                        const uint8_t* posting_codes, const uint32_t* posting_aux,
                                        const uint32_t* posting_slab,
                                        const float* posting_ranges, uint32_t* out_ids,
                                        float* out_dists, uint32_t* pass_counts)
{
    return guarded(c, [&](Context* ctx) {
        return gofann::rabitq_posting_scan_segments(
            ctx, rq, prepared, predicate, route_query, posting_sample_ids, posting_rows, segments,
            shortlist_k, posting_codes, posting_aux, posting_slab, posting_ranges, out_ids,
            out_dists, pass_counts);
    });
}

int gofann_rabitq_posting_scan_shared(gofann_ctx* c, const gofann_rabitq_view* rq,
                                      const gofann_rabitq_queries* prepared,
                                      const gofann_predicate_view* predicate,
                                      const uint32_t* route_query,
                                      const uint32_t* posting_sample_ids, uint64_t posting_rows,
                                      const gofann_posting_segments* segments,
                                      const gofann_posting_share* share, int shortlist_k,
                                      const uint8_t* posting_codes, const uint32_t* posting_aux,
                                      const uint32_t* posting_slab,
                                      const float* posting_ranges, uint32_t* out_ids,
                                      float* out_dists, uint32_t* pass_counts)
{
    return guarded(c, [&](Context* ctx) {
        return gofann::rabitq_posting_scan_shared(
            ctx, rq, prepared, predicate, route_query, posting_sample_ids, posting_rows, segments,
            share, shortlist_k, posting_codes, posting_aux, posting_slab, posting_ranges, out_ids,
            out_dists, pass_counts);
    });
}

int gofann_exact_rerank(gofann_ctx* c, const void* base, int base_elem, uint32_t dim,
                        uint32_t samples, const void* queries, const uint32_t* route_query,
                        const uint32_t* shortlist, uint32_t width, uint32_t routes, uint32_t topk,
                        uint32_t* out_ids, float* out_dists)
{
    return guarded(c, [&](Context* ctx) {
        if (routes > 0 && (!out_ids || !out_dists))
            return ctx->fail(GOFANN_ERR_INVALID, "null outputs");
        return gofann::exact_rerank(ctx, base, base_elem, dim, samples, queries, route_query,
                                    shortlist, width, routes, topk, out_ids, out_dists);
    });
}

int gofann_exact_posting_scan(gofann_ctx* c, const void* base, int base_elem, uint32_t dim,
                              uint32_t samples, const void* queries,
                              const gofann_predicate_view* predicate,
                              const uint32_t* route_query, const uint32_t* cand_ids,
                              const uint32_t* cand_offsets, const uint32_t* cand_sizes,
                              uint32_t routes, int topk, int order, uint32_t* out_ids,
                              float* out_dists, uint32_t* pass_counts)
{
    return guarded(c, [&](Context* ctx) {
        return gofann::exact_posting_scan(ctx, base, base_elem, dim, samples, queries, predicate,
                                          route_query, cand_ids, cand_offsets, cand_sizes, routes,
                                          topk, order, out_ids, out_dists, pass_counts);
    });
}

int gofann_predicate_masks(gofann_ctx* c, const gofann_predicate_view* predicate,
                           const uint32_t* route_ids, const uint32_t* sample_ids, uint32_t n,
                           uint32_t* masks)
{
    return guarded(c, [&](Context* ctx) {
        return gofann::predicate_masks(ctx, predicate, route_ids, sample_ids, n, masks);
    });
}

int gofann_merge_routes(gofann_ctx* c, const uint32_t* query_route_offsets,
                        const uint32_t* query_routes, const uint32_t* route_ids,
                        const float* route_dists, uint32_t width, uint32_t queries, uint32_t topk,
                        uint32_t* out_ids, float* out_dists)
{
    return guarded(c, [&](Context* ctx) {
        return gofann::merge_routes(ctx, query_route_offsets, query_routes, route_ids,
                                    route_dists, width, queries, topk, out_ids, out_dists);
    });
}

int gofann_pq_score(gofann_ctx* c, const gofann_pq_view* pq, const void* queries, int query_elem,
                    const uint32_t* q_idx, const uint32_t* s_idx, uint32_t n, float* out)
{
    return guarded(c, [&](Context* ctx) {
        if (n > 0 && (!q_idx || !s_idx || !out))
            return ctx->fail(GOFANN_ERR_INVALID, "score arrays missing");
        return gofann::pq_score(ctx, pq, queries, query_elem, q_idx, s_idx, n, out);
    });
}

int gofann_rabitq_score(gofann_ctx* c, const gofann_rabitq_view* rq,
                        const gofann_rabitq_queries* prepared, const uint32_t* q_idx,
                        const uint32_t* s_idx, uint32_t n, float* out, int32_t* ip_int)
{
    return guarded(c, [&](Context* ctx) {
        if (n > 0 && (!q_idx || !s_idx || !out))
            return ctx->fail(GOFANN_ERR_INVALID, "score arrays missing");
        return gofann::rabitq_score(ctx, rq, prepared, q_idx, s_idx, n, out, ip_int);
    });
}

int gofann_build_assign(gofann_ctx* c, const void* rows, int elem, uint32_t dim, uint64_t n,
                        const float* centres, uint32_t k, uint32_t* out_idx, float* out_score)
{
    return guarded(c, [&](Context* ctx) {
        return gofann::build_assign(ctx, rows, elem, dim, n, centres, k, out_idx, out_score);
    });
}

int gofann_build_kmeanspp(gofann_ctx* c, const void* rows, int elem, uint32_t dim, uint64_t n,
                          uint32_t k, uint64_t seed, float* centres)
{
    return guarded(c, [&](Context* ctx) {
        return gofann::build_kmeanspp(ctx, rows, elem, dim, n, k, seed, centres);
    });
}

int gofann_build_kmeans(gofann_ctx* c, const void* rows, int elem, uint32_t dim, uint64_t n,
                        uint32_t k, uint32_t iters, float* centres)
{
    return guarded(c, [&](Context* ctx) {
        return gofann::build_kmeans(ctx, rows, elem, dim, n, k, iters, centres);
    });
}

int gofann_build_knn(gofann_ctx* c, const void* rows, int elem, uint32_t dim,
                     const gofann_build_buckets* buckets, uint32_t k, uint32_t* out_ids,
                     float* out_dists)
{
    return guarded(c, [&](Context* ctx) {
        return gofann::build_knn(ctx, rows, elem, dim, buckets, k, out_ids, out_dists);
    });
}

int gofann_build_pq_train(gofann_ctx* c, const void* rows, int elem, uint32_t dim, uint64_t n,
                          uint32_t pq_dim, uint32_t iters, float* centroids)
{
    return guarded(c, [&](Context* ctx) {
        return gofann::build_pq_train(ctx, rows, elem, dim, n, pq_dim, iters, centroids);
    });
}

int gofann_build_pq_encode(gofann_ctx* c, const void* rows, int elem, uint32_t dim, uint64_t n,
                           uint32_t pq_dim, const float* centroids, uint8_t* codes,
                           uint32_t code_stride)
{
    return guarded(c, [&](Context* ctx) {
        return gofann::build_pq_encode(ctx, rows, elem, dim, n, pq_dim, centroids, codes,
                                       code_stride);
    });
}

int gofann_build_rotate(gofann_ctx* c, const void* rows, int elem, uint32_t dim, uint32_t n,
                        const float* rotation, uint32_t padded_dim, float* out)
{
    return guarded(c, [&](Context* ctx) {
        return gofann::build_rotate(ctx, rows, elem, dim, n, rotation, padded_dim, out);
    });
}

int gofann_build_rabitq_encode(gofann_ctx* c, const float* rotated, uint32_t n,
                               uint32_t padded_dim, const float* anchors, uint32_t num_anchors,
                               uint32_t* anchor_ids, uint8_t* codes, float* factors)
{
    return guarded(c, [&](Context* ctx) {
        return gofann::build_rabitq_encode(ctx, rotated, n, padded_dim, anchors, num_anchors,
                                           anchor_ids, codes, factors);
    });
}

int gofann_build_medoid(gofann_ctx* c, const void* rows, int elem, uint32_t dim, uint64_t n,
                        uint32_t* out_row)
{
    return guarded(c, [&](Context* ctx) {
        return gofann::build_medoid(ctx, rows, elem, dim, n, out_row);
    });
}

int gofann_build_bucket_reps(gofann_ctx* c, const void* rows, int elem, uint32_t dim,
                             const uint32_t* bucket_offsets, uint32_t buckets, float* means,
                             uint32_t* reps)
{
    return guarded(c, [&](Context* ctx) {
        return gofann::build_bucket_reps(ctx, rows, elem, dim, bucket_offsets, buckets, means, reps);
    });
}

int gofann_build_links(gofann_ctx* c, const gofann_build_link_inputs* inputs,
                       const gofann_build_link_params* params, uint32_t* out_graph)
{
    return guarded(c, [&](Context* ctx) {
        return gofann::build_links(ctx, inputs, params, out_graph);
    });
}

int gofann_build_cagra_optimize(gofann_ctx* c, const uint32_t* knn, uint32_t n, uint32_t kin,
                                uint32_t degree, uint32_t* pruned, uint32_t* out_graph)
{
    return guarded(c, [&](Context* ctx) {
        return gofann::build_cagra_optimize(ctx, knn, n, kin, degree, pruned, out_graph);
    });
}

int gofann_build_reach(gofann_ctx* c, const uint32_t* graph, uint32_t n, uint32_t degree,
                       uint32_t entry_row, uint32_t* reached, uint32_t* reached_count)
{
    return guarded(c, [&](Context* ctx) {
        return gofann::build_reach(ctx, graph, n, degree, entry_row, reached, reached_count);
    });
}

}  // extern "C"
