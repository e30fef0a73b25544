/* cpu_baseline.c -- the oracle's batch drivers run over all host cores.
 *
 * TEST INFRASTRUCTURE ONLY (the CPU baseline that bench.py times next to the
 * GPU): routes are independent, so each OpenMP thread runs the
 * single-threaded oracle (gofann_oracle.c) on its own chunk of routes, with
 * every per-route array offset to the chunk.  Built -O3 with OpenMP and
 * -ffp-contract=off, so the results are those of the oracle bit for bit
 * (the tests check it); only the wall time differs.  The product never
 * loads this library.
 *
 * The reference's own CPU-side structure is the same: a pool of host
 * workers, one route (or a few) at a time (rabitq_cpu_worker_pool.h,
 * cpu_rerank_schedule.h:10-44).
 */
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#include <omp.h>

#include "gofann_oracle.h"

#define CBL_CHUNK 16u

static int threads_or_default(int threads)
{
    return threads > 0 ? threads : omp_get_max_threads();
}

int cbl_max_threads(void) { return omp_get_max_threads(); }

/* The graph view and predicate view of routes [r0, ...). */
static orc_graph graph_at(const orc_graph* g, uint32_t r0)
{
    orc_graph s = *g;
    if (s.route_group) s.route_group += r0;
    if (s.route_start) s.route_start += r0;
    if (s.query_filter_bits) s.query_filter_bits += r0;
    if (s.range_modes) s.range_modes += (size_t)r0 * s.range_count;
    if (s.range_lower) s.range_lower += (size_t)r0 * s.range_count;
    if (s.range_upper) s.range_upper += (size_t)r0 * s.range_count;
    return s;
}

static orc_predicate pred_at(const orc_predicate* p, uint32_t r0)
{
    orc_predicate s = *p;
    if (s.route_offsets) s.route_offsets += r0;
    if (s.route_enabled) s.route_enabled += r0;
    if (s.route_compiled) s.route_compiled += r0;
    return s;
}

int cbl_exact_search(const orc_graph* g, const uint32_t* label_size, const orc_predicate* pred,
                     const orc_exact_params* p, const void* base, int elem, uint32_t dim,
                     uint32_t samples, const void* queries, const uint32_t* route_query,
                     uint32_t routes, uint32_t* out_ids, float* out_dists,
                     orc_route_stats* stats, int threads)
{
    int rc = 0;
    const uint32_t K = (uint32_t)p->topk;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads_or_default(threads)) reduction(| : rc)
    for (uint32_t r0 = 0; r0 < routes; r0 += CBL_CHUNK) {
        const uint32_t n = routes - r0 < CBL_CHUNK ? routes - r0 : CBL_CHUNK;
        orc_graph gs = graph_at(g, r0);
        orc_predicate ps;
        if (pred) ps = pred_at(pred, r0);
        rc |= orc_exact_search(&gs, label_size, pred ? &ps : NULL, p, base, elem, dim, samples,
                               queries,
                               route_query + r0, n, out_ids + (size_t)r0 * K,
                               out_dists + (size_t)r0 * K, stats ? stats + r0 : NULL) != 0;
    }
    return rc ? -1 : 0;
}

int cbl_pq_search_batch(const orc_graph* g, const orc_predicate* pred,
                        const orc_search_params* p, const uint8_t* codes,
                        const float* centroids, const void* queries, int query_is_float,
                        const void* exact_base, const uint32_t* route_query, int dim,
                        int pq_dim, uint32_t routes, uint32_t* out_ids, float* out_dists,
                        orc_route_stats* stats, int threads)
{
    int rc = 0;
    const size_t W = (size_t)p->result_width;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads_or_default(threads)) reduction(| : rc)
    for (uint32_t r0 = 0; r0 < routes; r0 += CBL_CHUNK) {
        const uint32_t n = routes - r0 < CBL_CHUNK ? routes - r0 : CBL_CHUNK;
        orc_graph gs = graph_at(g, r0);
        orc_predicate ps;
        if (pred) ps = pred_at(pred, r0);
        rc |= orc_pq_search_batch(&gs, pred ? &ps : NULL, p, codes, centroids, queries,
                                  query_is_float, exact_base, route_query + r0, dim, pq_dim, n,
                                  out_ids + r0 * W, out_dists + r0 * W,
                                  stats ? stats + r0 : NULL) != 0;
    }
    return rc ? -1 : 0;
}

int cbl_rabitq_search_batch(const orc_graph* g, const orc_predicate* pred,
                            const orc_search_params* p, const uint8_t* codes,
                            uint32_t code_bytes, const float* factors,
                            const uint32_t* anchor_ids, const int8_t* q8, const float* q_scale,
                            const float* q_k1, const float* centroid_dists, uint32_t num_anchors,
                            uint32_t padded_dim, const uint32_t* route_query, uint32_t routes,
                            uint32_t* out_ids, float* out_dists, orc_route_stats* stats,
                            int threads)
{
    int rc = 0;
    const size_t W = (size_t)p->result_width;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads_or_default(threads)) reduction(| : rc)
    for (uint32_t r0 = 0; r0 < routes; r0 += CBL_CHUNK) {
        const uint32_t n = routes - r0 < CBL_CHUNK ? routes - r0 : CBL_CHUNK;
        orc_graph gs = graph_at(g, r0);
        orc_predicate ps;
        if (pred) ps = pred_at(pred, r0);
        rc |= orc_rabitq_search_batch(&gs, pred ? &ps : NULL, p, codes, code_bytes, factors,
                                      anchor_ids, q8, q_scale, q_k1, centroid_dists, num_anchors,
                                      padded_dim, route_query + r0, n, out_ids + r0 * W,
                                      out_dists + r0 * W, stats ? stats + r0 : NULL) != 0;
    }
    return rc ? -1 : 0;
}

int cbl_pq_posting_scan(const orc_predicate* pred, const uint8_t* codes, const float* centroids,
                        const void* queries, int query_is_float, const uint32_t* route_query,
                        const uint32_t* cand_ids, const uint32_t* cand_offsets,
                        const uint32_t* cand_sizes, uint32_t routes, int dim, int pq_dim,
                        int shortlist_k, int score_first, uint32_t* out_ids, float* out_dists,
                        uint32_t* pass_counts, int threads)
{
    int rc = 0;
    const size_t k = (size_t)shortlist_k;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads_or_default(threads)) reduction(| : rc)
    for (uint32_t r0 = 0; r0 < routes; r0 += CBL_CHUNK) {
        const uint32_t n = routes - r0 < CBL_CHUNK ? routes - r0 : CBL_CHUNK;
        orc_predicate ps;
        if (pred) ps = pred_at(pred, r0);
        rc |= orc_pq_posting_scan(pred ? &ps : NULL, codes, centroids, queries, query_is_float,
                                  route_query + r0, cand_ids, cand_offsets + r0, cand_sizes + r0,
                                  n, dim, pq_dim, shortlist_k, score_first, out_ids + r0 * k,
                                  out_dists + r0 * k, pass_counts ? pass_counts + r0 : NULL) != 0;
    }
    return rc ? -1 : 0;
}

int cbl_rabitq_posting_scan(const orc_predicate* pred, const uint8_t* codes, uint32_t code_bytes,
                            const float* factors, const uint32_t* anchor_ids, const int8_t* q8,
                            const float* q_scale, const float* q_k1, const float* centroid_dists,
                            uint32_t num_anchors, uint32_t padded_dim, const uint32_t* route_query,
                            const uint32_t* cand_ids, const uint32_t* cand_offsets,
                            const uint32_t* cand_sizes, uint32_t routes, int shortlist_k,
                            uint32_t* out_ids, float* out_dists, uint32_t* pass_counts,
                            int threads)
{
    int rc = 0;
    const size_t k = (size_t)shortlist_k;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads_or_default(threads)) reduction(| : rc)
    for (uint32_t r0 = 0; r0 < routes; r0 += CBL_CHUNK) {
        const uint32_t n = routes - r0 < CBL_CHUNK ? routes - r0 : CBL_CHUNK;
        orc_predicate ps;
        if (pred) ps = pred_at(pred, r0);
        rc |= orc_rabitq_posting_scan(pred ? &ps : NULL, codes, code_bytes, factors, anchor_ids, q8,
                                      q_scale, q_k1, centroid_dists, num_anchors, padded_dim,
                                      route_query + r0, cand_ids, cand_offsets + r0,
                                      cand_sizes + r0, n, shortlist_k, out_ids + r0 * k,
                                      out_dists + r0 * k,
                                      pass_counts ? pass_counts + r0 : NULL) != 0;
    }
    return rc ? -1 : 0;
}

/* Segments are independent: each thread scans a chunk of them (segment s
 * still names its route through seg_routes[s]). */
int cbl_rabitq_range_scan(const orc_predicate* pred, const orc_range_table* rt,
                          const uint8_t* codes, uint32_t code_bytes, const float* factors,
                          const uint32_t* anchor_ids, const int8_t* q8, const float* q_scale,
                          const float* q_k1, const float* centroid_dists, uint32_t num_anchors,
                          uint32_t padded_dim, const uint32_t* route_query,
                          const uint32_t* posting, uint64_t resident_rows, uint32_t base_rows,
                          const uint32_t* seg_routes, const uint64_t* seg_offsets,
                          const uint64_t* seg_sizes, uint32_t segments, int shortlist_k,
                          int score_first, uint32_t* out_ids, float* out_dists,
                          uint32_t* pass_counts, int threads)
{
    int rc = 0;
    const size_t k = (size_t)shortlist_k;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads_or_default(threads)) reduction(| : rc)
    for (uint32_t s0 = 0; s0 < segments; s0 += CBL_CHUNK) {
        const uint32_t n = segments - s0 < CBL_CHUNK ? segments - s0 : CBL_CHUNK;
        rc |= orc_rabitq_range_scan(pred, rt, codes, code_bytes, factors, anchor_ids, q8, q_scale,
                                    q_k1, centroid_dists, num_anchors, padded_dim, route_query,
                                    posting, resident_rows, base_rows, seg_routes + s0,
                                    seg_offsets + s0, seg_sizes + s0, n, shortlist_k, score_first,
                                    out_ids + s0 * k, out_dists + s0 * k,
                                    pass_counts ? pass_counts + s0 : NULL) != 0;
    }
    return rc ? -1 : 0;
}

int cbl_rerank(const void* base, int elem_type, uint32_t dim, uint32_t samples,
               const void* queries, const uint32_t* route_query, const uint32_t* shortlist,
               uint32_t width, uint32_t routes, uint32_t topk, uint32_t* out_ids,
               float* out_dists, int threads)
{
    int rc = 0;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads_or_default(threads)) reduction(| : rc)
    for (uint32_t r0 = 0; r0 < routes; r0 += CBL_CHUNK) {
        const uint32_t n = routes - r0 < CBL_CHUNK ? routes - r0 : CBL_CHUNK;
        rc |= orc_rerank(base, elem_type, dim, samples, queries, route_query + r0,
                         shortlist + (size_t)r0 * width, width, n, topk,
                         out_ids + (size_t)r0 * topk, out_dists + (size_t)r0 * topk) != 0;
    }
    return rc ? -1 : 0;
}
