// gofann_internal.hpp -- context object behind the C ABI (gofann_hip.h) and
// the internal entry points each kernel file implements.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "gofann_hip.h"

namespace gofann {

// Owns the stream binding, device properties, the last error message and
// the grow-only device scratch buffers of one host thread's search state
// (the reference's per-context buffers, backend_pq.cu:6753-6990).
struct Context {
    enum ScratchSlot {
        kScratchHash = 0,
        kScratchSegments = 1,
        kScratchMisc = 2,
        kScratchRange = 3,  // per-segment range-scan shortlists before the merge
        kScratchBuild = 4,  // index construction (k-means, kNN, graph optimisation)
        kScratchCount = 5
    };

    int device = 0;
    hipStream_t stream = nullptr;
    int compute_units = 0;
    int lds_per_block = 0;
    int lds_per_cu = 0;
    std::string error;
    void* scratch_ptr[kScratchCount] = {};
    size_t scratch_bytes[kScratchCount] = {};
    // Placement chosen by the last traversal launch (diagnostics).
    int last_hash_in_lds = 0;
    int last_table_in_lds = 0;
    int last_lds_bytes = 0;
    int last_resident = 0;
    void* blas = nullptr;  // rocblas_handle of the query-rotation GEMM (lazy)

    int fail(int code, const std::string& msg)
    {
        error = msg;
        return code;
    }
    int fail_hip(const std::string& what)
    {
        const hipError_t e = hipGetLastError();
        error = what + ": " + hipGetErrorString(e);
        return GOFANN_ERR_HIP;
    }
    // Returns a device buffer of at least `bytes` for `slot` (grows, never
    // shrinks; freed by gofann_destroy).  nullptr on allocation failure.
    void* scratch(int slot, size_t bytes);
};

int pq_search(Context* ctx, const gofann_pq_view* pq, const void* queries, int query_elem,
              const gofann_graph_view* g, const gofann_predicate_view* pred,
              const gofann_routes* r, const gofann_search_params* p, uint32_t* out_ids,
              float* out_dists, gofann_route_stats* stats);
int rabitq_search(Context* ctx, const gofann_rabitq_view* rq, const gofann_rabitq_queries* pre,
                  const gofann_graph_view* g, const gofann_predicate_view* pred,
                  const gofann_routes* r, const gofann_search_params* p, uint32_t* out_ids,
                  float* out_dists, gofann_route_stats* stats);
int pq_score(Context* ctx, const gofann_pq_view* pq, const void* queries, int query_elem,
             const uint32_t* q_idx, const uint32_t* s_idx, uint32_t n, float* out);
int rabitq_score(Context* ctx, const gofann_rabitq_view* rq, const gofann_rabitq_queries* pre,
                 const uint32_t* q_idx, const uint32_t* s_idx, uint32_t n, float* out,
                 int32_t* ip_int);
int pq_posting_scan(Context* ctx, const gofann_pq_view* pq, const void* queries, int query_elem,
                    const gofann_predicate_view* pred, const uint32_t* route_query,
                    const uint32_t* cand_ids, const uint32_t* cand_offsets,
                    const uint32_t* cand_sizes, uint32_t routes, int shortlist_k,
                    uint32_t* out_ids, float* out_dists, uint32_t* pass_counts);
int rabitq_posting_scan(Context* ctx, const gofann_rabitq_view* rq,
                        const gofann_rabitq_queries* pre, const gofann_predicate_view* pred,
                        const uint32_t* route_query, const uint32_t* cand_ids,
                        const uint32_t* cand_offsets, const uint32_t* cand_sizes,
                        uint32_t routes, int shortlist_k, uint32_t* out_ids, float* out_dists,
                        uint32_t* pass_counts);
bool rabitq_posting_scan_grouped(uint32_t padded_dim);
int rabitq_posting_scan_group(Context* ctx, const gofann_rabitq_view* rq,
                              const gofann_rabitq_queries* pre, const gofann_predicate_view* pred,
                              const uint32_t* route_query, const uint32_t* cand_ids,
                              const uint32_t* cand_offsets, const uint32_t* cand_sizes,
                              uint32_t routes, int shortlist_k, uint32_t* out_ids,
                              float* out_dists, uint32_t* pass_counts);
int exact_rerank(Context* ctx, const void* base, int base_elem, uint32_t dim, uint32_t samples,
                 const void* queries, const uint32_t* route_query, const uint32_t* shortlist,
                 uint32_t width, uint32_t routes, uint32_t topk, uint32_t* out_ids,
                 float* out_dists);
int exact_posting_scan(Context* ctx, const void* base, int base_elem, uint32_t dim,
                       uint32_t samples, const void* queries, const gofann_predicate_view* pred,
                       const uint32_t* route_query, const uint32_t* cand_ids,
                       const uint32_t* cand_offsets, const uint32_t* cand_sizes, uint32_t routes,
                       int topk, int order, uint32_t* out_ids, float* out_dists,
                       uint32_t* pass_counts);
int predicate_masks(Context* ctx, const gofann_predicate_view* pred, const uint32_t* route_ids,
                    const uint32_t* sample_ids, uint32_t n, uint32_t* masks);
int merge_routes(Context* ctx, const uint32_t* q_route_offsets, const uint32_t* q_routes,
                 const uint32_t* route_ids, const float* route_dists, uint32_t width,
                 uint32_t queries, uint32_t topk, uint32_t* out_ids, float* out_dists);
int rabitq_range_scan(Context* ctx, const gofann_rabitq_view* rq,
                      const gofann_rabitq_queries* pre, const gofann_predicate_view* pred,
                      const gofann_routes* routes, const uint32_t* posting,
                      uint64_t resident_rows, const gofann_posting_segments* seg,
                      int shortlist_k, int score_first, uint32_t* out_ids, float* out_dists,
                      uint32_t* pass_counts, const uint8_t* posting_codes = nullptr,
                      const uint32_t* posting_aux = nullptr);
int rabitq_posting_rows(Context* ctx, const gofann_rabitq_view* rq, const uint32_t* posting,
                        uint64_t rows, uint8_t* out_codes, uint32_t* out_aux);
int posting_predicate_rows(Context* ctx, const gofann_predicate_view* pred,
                           const uint32_t* posting, uint64_t rows, uint32_t* out_slab,
                           float* out_ranges);
int rabitq_posting_scan_segments(Context* ctx, const gofann_rabitq_view* rq,
                                 const gofann_rabitq_queries* pre,
                                 const gofann_predicate_view* pred, const uint32_t* route_query,
                                 const uint32_t* posting, uint64_t posting_rows,
                                 const gofann_posting_segments* seg, int shortlist_k,
                                 const uint8_t* posting_codes, const uint32_t* posting_aux,
                                 const uint32_t* posting_slab, const float* posting_ranges,
                                 uint32_t* out_ids, float* out_dists, uint32_t* pass_counts);
int rabitq_posting_scan_shared(Context* ctx, const gofann_rabitq_view* rq,
                               const gofann_rabitq_queries* pre,
                               const gofann_predicate_view* pred, const uint32_t* route_query,
                               const uint32_t* posting, uint64_t posting_rows,
                               const gofann_posting_segments* seg,
                               const gofann_posting_share* share, int shortlist_k,
                               const uint8_t* posting_codes, const uint32_t* posting_aux,
                               const uint32_t* posting_slab, const float* posting_ranges,
                               uint32_t* out_ids, float* out_dists, uint32_t* pass_counts);
int exact_search(Context* ctx, const void* base, int base_elem, uint32_t dim, uint32_t samples,
                 const void* queries, const gofann_graph_view* g, const uint32_t* label_size,
                 const gofann_predicate_view* pred, const gofann_routes* r,
                 const gofann_exact_params* p, uint32_t* out_ids, float* out_dists,
                 gofann_route_stats* stats);
int exact_search_noalloc(Context* ctx, const void* base, int base_elem, uint32_t dim,
                         uint32_t samples, const void* queries, const gofann_graph_view* g,
                         const uint32_t* label_size, const gofann_predicate_view* pred,
                         const gofann_routes* r, const gofann_exact_params* p,
                         uint32_t* out_ids, float* out_dists, gofann_route_stats* stats);
// Per-device lookup of the no-alloc entry point's fixed scratch (called by
// gofann_create with the device current).
void noalloc_setup(int device);
void destroy_blas(Context* ctx);
int build_assign(Context* ctx, const void* rows, int elem, uint32_t dim, uint64_t n,
                 const float* centres, uint32_t k, uint32_t* out_idx, float* out_score);
int build_kmeanspp(Context* ctx, const void* rows, int elem, uint32_t dim, uint64_t n, uint32_t k,
                   uint64_t seed, float* centres);
int build_kmeans(Context* ctx, const void* rows, int elem, uint32_t dim, uint64_t n, uint32_t k,
                 uint32_t iters, float* centres);
int build_knn(Context* ctx, const void* rows, int elem, uint32_t dim,
              const gofann_build_buckets* b, uint32_t k, uint32_t* out_ids, float* out_dists);
int build_pq_train(Context* ctx, const void* rows, int elem, uint32_t dim, uint64_t n,
                   uint32_t pq_dim, uint32_t iters, float* centroids);
int build_pq_encode(Context* ctx, const void* rows, int elem, uint32_t dim, uint64_t n,
                    uint32_t pq_dim, const float* centroids, uint8_t* codes, uint32_t code_stride);
int build_rotate(Context* ctx, const void* rows, int elem, uint32_t dim, uint32_t n,
                 const float* rotation, uint32_t padded_dim, float* out);
int build_rabitq_encode(Context* ctx, const float* rotated, uint32_t n, uint32_t padded_dim,
                        const float* anchors, uint32_t num_anchors, uint32_t* anchor_ids,
                        uint8_t* codes, float* factors);
int build_medoid(Context* ctx, const void* rows, int elem, uint32_t dim, uint64_t n, uint32_t* out);
int build_bucket_reps(Context* ctx, const void* rows, int elem, uint32_t dim,
                      const uint32_t* bucket_offsets, uint32_t buckets, float* means, uint32_t* reps);
int build_links(Context* ctx, const gofann_build_link_inputs* in, const gofann_build_link_params* p,
                uint32_t* out_graph);
int build_cagra_optimize(Context* ctx, const uint32_t* knn, uint32_t n, uint32_t kin, uint32_t degree,
                         uint32_t* pruned, uint32_t* out_graph);
int build_reach(Context* ctx, const uint32_t* graph, uint32_t n, uint32_t degree, uint32_t entry,
                uint32_t* reached, uint32_t* out_count);
int rabitq_prepare(Context* ctx, const gofann_rabitq_view* rq, const float* queries,
                   uint32_t count, const float* rotation, gofann_rabitq_queries* out);

}  // namespace gofann
