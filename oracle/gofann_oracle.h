/*
 * gofann_oracle.h -- CPU restatement of GO-FANN's GPU filtered graph-search
 * hot path.  TEST INFRASTRUCTURE ONLY: this library is the checker that the
 * HIP product path is compared against.  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load it; the product never links it.
 *
 * Every function restates the reference algorithm from its mathematics and
 * cites the reference file:line it follows (paths relative to the GO-FANN
 * source tree).  Floating-point operation order is spelled out explicitly
 * (the file is compiled with -ffp-contract=off; fused multiply-adds are
 * written as fmaf where the reference's nvcc build contracts them), so the
 * HIP kernels can reproduce every float bit for bit.
 *
 * Pinning of each function (golden vectors, closed forms, brute force) lives
 * in tests/test_oracle_*.py.  Functions without such a check say
 * "parity unpinned" in their comment.
 */
#ifndef GOFANN_ORACLE_H
#define GOFANN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_HASH_CAPACITY 4096u   /* backend_pq.cu:194 kHashTableCapacity */
#define ORC_FIXED_DEGREE 64       /* include/config1B.h:29 FIXED_DEGREE */
#define ORC_POOL_USED 0x80000000u /* backend_pq.cu:713 kPoolUsedMask */
#define ORC_EARLY_STOP_FIXED 0    /* backend_pq.cu:1615-1617 */
#define ORC_EARLY_STOP_OFF 1
#define ORC_EARLY_STOP_ADAPTIVE 2

/* Frontier entry.  `base` is the unbiased score (gpu_predicate::BiasedPair,
 * gpu_predicate_index.cuh:137-144); for the plain PoolPair (backend_pq.cu:521)
 * base always equals first. */
typedef struct {
    float first;
    uint32_t second;
    float base;
} orc_pair;

/* Stop heap entry: KernelPair<dist_t, idx_t> (backend_pq.cu:523). */
typedef struct {
    float first;
    uint64_t second;
} orc_stop_pair;

/* Result heap entry: KernelPair<dist_t, uint32_t> (backend_pq.cu:522). */
typedef struct {
    float first;
    uint32_t second;
} orc_result_pair;

/* gpu_predicate::Clause / RangeAtom (gpu_predicate_index.cuh:23-24). */
typedef struct {
    uint32_t label_begin, label_end, range_begin, range_end;
} orc_clause;
typedef struct {
    uint32_t dimension, mode;
    float lower, upper;
} orc_range_atom;

/* gpu_predicate::View, CSR storage (gpu_predicate_index.cuh:25-48). */
typedef struct {
    const uint32_t* route_offsets; /* [routes+1] into clauses (or handles) */
    const uint32_t* route_handles; /* original label ids */
    const orc_clause* clauses;     /* NULL: legacy conjunction of handles */
    const orc_range_atom* ranges;
    const uint8_t* route_enabled;  /* NULL: enabled iff csr_offsets != NULL */
    const uint8_t* route_compiled; /* NULL: no route compiled */
    const float* base_ranges;      /* [rows][range_stride] */
    const uint32_t* csr_offsets;   /* [rows+1] */
    const uint32_t* csr_labels;    /* strictly sorted per row */
    uint32_t rows;
    uint32_t range_stride;
    float alpha;
    int pending_base_stop;
} orc_predicate;

/* Counters of the work one predicate evaluation did (bytes model). */
typedef struct {
    uint64_t rows_checked;  /* CSR rows opened (2 offsets read each) */
    uint64_t label_words;   /* CSR label words read */
    uint64_t range_values;  /* base range values read */
} orc_pred_counters;

/* Label-partitioned graph + legacy (uncompiled) route filters. */
typedef struct {
    const uint32_t* graph;          /* [rows][degree] label-local ids */
    uint32_t degree;                /* row stride (<= 64 are read) */
    const uint32_t* row_to_sample;  /* [rows] */
    const uint32_t* label_offset;   /* [groups] */
    const uint32_t* route_group;    /* [routes] */
    const uint32_t* route_start;    /* [routes] label-local seed row */
    const uint64_t* row_filter_mask;   /* [rows] or NULL (all ones) */
    const uint64_t* query_filter_bits; /* [routes] or NULL (all ones) */
    const uint8_t* range_modes;        /* [routes][range_count] or NULL */
    const float* range_lower;
    const float* range_upper;
    const float* base_range_values;    /* [samples][range_count] */
    uint32_t range_count;
} orc_graph;

typedef struct {
    int queue_limit;
    int finish_limit;
    int early_stop_mode;
    int max_steps;
    int stop_width;
    int result_width;
    float bit_filter_bonus;
    float range_filter_bonus;
    int bias;          /* kPredicateBias: frontier orders by biased priority */
    int rabitq_verdict; /* 1: backend_rabitq.cu:3873-3894 verdict chain */
    int inline_exact;   /* enable_true_distance_rerank (backend_pq.cu:4507-4546) */
} orc_search_params;

typedef struct {
    int32_t steps;
    int32_t expanded;
    int32_t passed;
    int32_t scored;        /* distance evaluations incl. the seed */
    int32_t pred_rows;     /* predicate CSR rows opened */
    int32_t pred_labels;   /* predicate CSR label words read */
    int32_t admitted;      /* frontier insertions */
    int32_t exhausted;
} orc_route_stats;

/* ---------------- visited hash (native_visited_hash.cuh:10-60) ---------- */
uint32_t orc_hash_code(uint32_t value);
void orc_hash_clear(uint32_t* table);
int orc_hash_test(const uint32_t* table, uint32_t value);
void orc_hash_add(uint32_t* table, uint32_t value);

/* ---------------- heaps (include/smmh2.h, include/bin_heap.h) ----------- */
void orc_smmh2_insert(orc_pair* heap, int* size, orc_pair entry);
orc_pair orc_smmh2_pop_max(orc_pair* heap, int* size);
orc_pair orc_smmh2_pop_min(orc_pair* heap, int* size);
int orc_pickup_unused(orc_pair* pool, int size, orc_pair* out);
void orc_result_push(orc_result_pair* begin, int size_after_append);
orc_result_pair orc_result_pop(orc_result_pair* begin, int size);

/* ---------------- posting shortlist heap (posting_shortlist_heap.cuh) ---- */
int orc_shortlist_can_enter(float dist, uint32_t id, const float* dists,
                            const uint32_t* ids, int k);
void orc_shortlist_insert(float dist, uint32_t id, float* dists, uint32_t* ids, int k);
void orc_shortlist_sort(float* dists, uint32_t* ids, int k);

/* ---------------- early stop (backend_pq.cu:2822-2873) ------------------- */
int orc_adaptive_early_stop_limit(int queue_limit, int expanded, int passed, int stop_width);
int orc_early_stop_reached(int mode, int bad, int fixed_limit, int queue_limit,
                           int expanded, int passed, int stop_width);

/* ---------------- predicates (gpu_predicate_index.cuh, range_filter.cuh) - */
int orc_csr_contains(const uint32_t* labels, uint32_t begin, uint32_t end,
                     uint32_t handle, uint64_t* words_read);
int orc_pred_enabled(const orc_predicate* v, uint32_t route);
int orc_pred_matches(const orc_predicate* v, uint32_t route, uint32_t sample,
                     orc_pred_counters* counters);
int orc_range_matches(uint32_t mode, float lower, float upper, float value);
float orc_priority(float base, float penalty, int pass, int* saturated);
float orc_minimum_pending_base(const orc_pair* pool, int size, orc_pair current,
                               orc_pair next, int current_valid, int next_valid);
float orc_bias_penalty(float alpha, float start_distance);
uint32_t orc_count_active_ranges(const uint8_t* modes, uint32_t route, uint32_t count);
uint32_t orc_count_matching_ranges(const uint8_t* modes, const float* lower,
                                   const float* upper, const float* base_values,
                                   uint32_t route, uint32_t sample, uint32_t count);
float orc_apply_filter_bonuses(float dist, int bit_match, uint32_t matched,
                               float bit_bonus, float range_bonus);

/* ---------------- PQ (backend_pq.cu:1999-2022, 4164-4187, 4711-4725) ----- */
void orc_pq_lut_u8(const float* centroids, const uint8_t* query, int dim,
                   int pq_dim, float* lut);
void orc_pq_lut_f32(const float* centroids, const float* query, int dim,
                    int pq_dim, float* lut);
float orc_pq_adc(const float* lut, const uint8_t* code, int pq_dim);

/* ---------------- RaBitQ (backend_rabitq.cu:2898-2964, 3070-3200) -------- */
void orc_rabitq_query_factors(const float* rotated, uint32_t padded_dim,
                              float* k1, float* kb);
void orc_rabitq_quantize(const float* rotated, uint32_t padded_dim, int8_t* q8,
                         float* scale);
int32_t orc_rabitq_ip_int(const int8_t* q8, const uint8_t* code, uint32_t padded_dim);
int32_t orc_rabitq_ip_popcount(const int8_t* q8, const uint8_t* code,
                               uint32_t padded_dim);
int32_t orc_rabitq_ip_dp4a(const int8_t* q8, const uint8_t* code, uint32_t padded_dim);
float orc_rabitq_score_b1(int32_t ip_int, float scale, float k1, float f_add,
                          float f_rescale, float g_add);

/* ---------------- traversal (backend_pq.cu:3980-5013) --------------------- */
typedef float (*orc_scorer)(void* ctx, uint32_t route, uint32_t sample);
/* Exact distance of the expanded node (may be NULL when inline_exact = 0). */
typedef float (*orc_exact)(void* ctx, uint32_t route, uint32_t sample);

int orc_beam_search_route(const orc_graph* g, const orc_predicate* pred,
                          const orc_search_params* p, uint32_t route,
                          orc_scorer scorer, orc_exact exact, void* scorer_ctx,
                          uint32_t* out_ids, float* out_dists,
                          orc_route_stats* stats);
/* Inline exact distance in the reference's 32-lane order: partial j sums
 * 4-element words j, j+32, ... (elements in order), xor butterfly 16..1. */
float orc_exact_inline_u8(const uint8_t* q, const uint8_t* b, uint32_t dim);
float orc_exact_inline_f32(const float* q, const float* b, uint32_t dim);

/* Batch drivers: one call runs every route.  Queries are per route
 * (route_query[route] selects the query vector row). */
int orc_pq_search_batch(const orc_graph* g, const orc_predicate* pred,
                        const orc_search_params* p, const uint8_t* codes,
                        const float* centroids, const void* queries,
                        int query_is_float, const void* exact_base,
                        const uint32_t* route_query,
                        int dim, int pq_dim, uint32_t routes, uint32_t* out_ids,
                        float* out_dists, orc_route_stats* stats);

int orc_rabitq_search_batch(const orc_graph* g, const orc_predicate* pred,
                            const orc_search_params* p, const uint8_t* codes,
                            uint32_t code_bytes, const float* factors,
                            const uint32_t* anchor_ids, const int8_t* q8,
                            const float* q_scale, const float* q_k1,
                            const float* centroid_dists, uint32_t num_anchors,
                            uint32_t padded_dim, const uint32_t* route_query,
                            uint32_t routes, uint32_t* out_ids, float* out_dists,
                            orc_route_stats* stats);

/* ---------------- full-GPU exact route (backend_full_gpu.cu:1682-2042) ----
 * Exact-distance beam over u8 vectors: frontier keys are the integer squared
 * L2 (l2_distance_device :1199-1244) as float; each expanded node that passes
 * the filter enters a sorted best-k with sample dedup (insert_best_result
 * :1342-1375).  Filter of an expanded node: row mask & route bits non-zero,
 * every active legacy range matches, and the route predicate when enabled
 * (candidate_passes_device :1015-1092 over the same label/range sets). */
typedef struct {
    int queue_limit;
    int finish_limit;
    int early_stop_mode;
    int max_steps;
    int topk; /* <= 10 (defaults::max_topk) */
} orc_exact_params;

uint32_t orc_l2_u8_int(const uint8_t* a, const uint8_t* b, uint32_t dim);
int orc_insert_best(float dist, uint32_t id, uint32_t topk, float* best_d, uint32_t* best_i,
                    uint32_t* best_size);
/* label_size [groups] (NULL: adjacency entries are taken as valid); stats
 * may be NULL; out [routes][topk] ascending by (distance, id). */
/* base/queries of element type elem (0 u8, 1 f32, 2 f16 as uint16 bits);
 * distances in the warp order (orc_l2_w32). */
int orc_exact_search(const orc_graph* g, const uint32_t* label_size, const orc_predicate* pred,
                     const orc_exact_params* p, const void* base, int elem, uint32_t dim,
                     uint32_t samples, const void* queries, const uint32_t* route_query,
                     uint32_t routes, uint32_t* out_ids, float* out_dists,
                     orc_route_stats* stats);
float orc_l2_w32(const void* row, const void* q, int elem, uint32_t dim);
float orc_l2_serial(const void* row, const void* q, int elem, uint32_t dim);

/* ---- exact posting scans (backend_full_gpu.cu:1383-1493, 2124-2262) ---- */
#define ORC_EXACT_ORDER_SERIAL 0
#define ORC_EXACT_ORDER_W32 1
#define ORC_EXACT_SCAN_MAX_TOPK 64
int orc_exact_posting_scan(const orc_predicate* pred, const void* base, int elem,
                           uint32_t dim, uint32_t samples, const void* queries,
                           const uint32_t* route_query, const uint32_t* cand_ids,
                           const uint32_t* cand_offsets, const uint32_t* cand_sizes,
                           uint32_t routes, int topk, int order, uint32_t* out_ids,
                           float* out_dists, uint32_t* pass_counts);

/* ---------------- posting scans (backend_pq.cu:2046-2133) ---------------- */
int orc_pq_posting_scan(const orc_predicate* pred, const uint8_t* codes,
                        const float* centroids, const void* queries,
                        int query_is_float, const uint32_t* route_query,
                        const uint32_t* cand_ids, const uint32_t* cand_offsets,
                        const uint32_t* cand_sizes, uint32_t routes, int dim,
                        int pq_dim, int shortlist_k, int score_first,
                        uint32_t* out_ids, float* out_dists, uint32_t* pass_counts);

int orc_rabitq_posting_scan(const orc_predicate* pred, const uint8_t* codes,
                            uint32_t code_bytes, const float* factors,
                            const uint32_t* anchor_ids, const int8_t* q8,
                            const float* q_scale, const float* q_k1,
                            const float* centroid_dists, uint32_t num_anchors,
                            uint32_t padded_dim, const uint32_t* route_query,
                            const uint32_t* cand_ids, const uint32_t* cand_offsets,
                            const uint32_t* cand_sizes, uint32_t routes,
                            int shortlist_k, uint32_t* out_ids, float* out_dists,
                            uint32_t* pass_counts);

/* ---------------- range posting segments and scan ----------------------
 * Segment plan: posting_segments::make_plan (src/execution/
 * posting_segment_plan.h:20-51).  Returns 0 and fills the arrays when
 * capacity >= the segment count, 1 when capacity is short (out_count still
 * receives the count), -1 on invalid input, -2 on overflow. */
int orc_segment_plan(const uint32_t* route_ids, const uint64_t* offsets, const uint64_t* sizes,
                     uint32_t n, uint32_t target_rows, uint32_t capacity, uint32_t* seg_routes,
                     uint32_t* seg_positions, uint64_t* seg_offsets, uint64_t* seg_sizes,
                     uint32_t* query_indptr, uint32_t* out_count);

/* Per-route range table of the query (QueryRangeTable, dataloader.h:545). */
typedef struct {
    const uint8_t* modes;       /* [routes][count] */
    const float* lower;
    const float* upper;
    const float* base_values;   /* [samples][count] */
    uint32_t count;
} orc_range_table;

/* range_posting_rabitq_scan_kernel (backend_rabitq.cu:5846-6015): segment
 * s scans posting[offsets[s] .. + sizes[s]) (clipped to resident_rows) for
 * route seg_routes[s].  Outputs [segments][shortlist_k] ascending by
 * (distance, id) (the kernel's heap holds the same multiset) and the
 * per-segment exact pass count. */
int orc_rabitq_range_scan(const orc_predicate* pred, const orc_range_table* ranges,
                          const uint8_t* codes, uint32_t code_bytes, const float* factors,
                          const uint32_t* anchor_ids, const int8_t* q8, const float* q_scale,
                          const float* q_k1, const float* centroid_dists, uint32_t num_anchors,
                          uint32_t padded_dim, const uint32_t* route_query,
                          const uint32_t* posting, uint64_t resident_rows, uint32_t base_rows,
                          const uint32_t* seg_routes, const uint64_t* seg_offsets,
                          const uint64_t* seg_sizes, uint32_t segments, int shortlist_k,
                          int score_first, uint32_t* out_ids, float* out_dists,
                          uint32_t* pass_counts);

/* merge_one_query (src/search/common/posting_segment_merge.cuh:12-46):
 * position p merges segments [query_indptr[p], query_indptr[p+1]) through
 * the shortlist heap and sums their pass counts; output ascending. */
int orc_merge_segments(const uint32_t* query_indptr, uint32_t positions,
                       const uint32_t* seg_ids, const float* seg_dists,
                       const uint32_t* seg_pass, int shortlist_k, uint32_t* out_ids,
                       float* out_dists, uint32_t* out_pass);

/* ---------------- resident posting view (pq_resident_posting.cuh:27-58) */
int orc_resident_bounds(const uint32_t* group_offsets, const uint32_t* group_sizes,
                        const uint32_t* query_groups, uint32_t groups, uint32_t rows,
                        uint32_t routes, uint32_t route, uint32_t* begin, uint32_t* count);
uint32_t orc_resident_candidate(const uint32_t* sample_ids, const uint64_t* row_masks,
                                const uint64_t* query_masks, const uint8_t* range_modes,
                                const float* range_lower, const float* range_upper,
                                const float* base_ranges, uint32_t rows, uint32_t samples,
                                uint32_t routes, uint32_t range_count, uint32_t route,
                                uint32_t row);

/* ---------------- exact rerank (backend_pq.cu:2187-2195, 2479-2592) ------ */
float orc_l2_u8(const uint8_t* a, const uint8_t* b, uint32_t dim);
float orc_l2_f32(const float* a, const float* b, uint32_t dim);
float orc_half_to_float(uint16_t h);
float orc_l2_f16(const float* q, const uint16_t* b, uint32_t dim);
/* elem_type: 0 = u8, 1 = f32, 2 = f16 (queries are f32 for f16 bases). */
int orc_rerank(const void* base, int elem_type, uint32_t dim, uint32_t samples,
               const void* queries, const uint32_t* route_query,
               const uint32_t* shortlist, uint32_t width, uint32_t routes,
               uint32_t topk, uint32_t* out_ids, float* out_dists);

/* ---------------- route merge (rabitq_lowfreq_merge.h:709-815) ----------- */
int orc_merge_routes(const uint32_t* route_to_query, uint32_t routes,
                     uint32_t queries, const uint32_t* route_ids,
                     const float* route_dists, uint32_t width, uint32_t topk,
                     uint32_t* out_ids, float* out_dists);


/* ---- index construction (oracle/build_oracle.c): the GPU build's
 * definitions (include/gofann_hip.h gofann_build_*), restated.  elem: 0 u8,
 * 1 f32, 2 f16 (as uint16 bits). */
uint64_t orc_build_draw64(uint64_t seed, uint64_t stream, uint64_t index);
double orc_build_draw_unit(uint64_t seed, uint64_t stream, uint64_t index);
void orc_build_assign(const void* rows, int elem, uint32_t dim, uint64_t n, const float* centres,
                      uint32_t k, uint32_t* out_idx, float* out_score);
void orc_build_kmeanspp(const void* rows, int elem, uint32_t dim, uint64_t n, uint32_t k,
                        uint64_t seed, float* centres);
void orc_build_kmeans(const void* rows, int elem, uint32_t dim, uint64_t n, uint32_t k,
                      uint32_t iters, float* centres);
void orc_build_knn(const void* rows, int elem, uint32_t dim, const uint32_t* bucket_off,
                   uint32_t buckets, const uint32_t* probe_off, const uint32_t* probe, uint32_t k,
                   uint32_t* out_ids, float* out_d);
void orc_build_pq_encode(const void* rows, int elem, uint32_t dim, uint64_t n, uint32_t pq_dim,
                         const float* centroids, uint8_t* codes, uint32_t code_stride);
void orc_build_pq_train(const void* rows, int elem, uint32_t dim, uint64_t n, uint32_t pq_dim,
                        uint32_t iters, float* centroids);
void orc_build_rabitq_encode(const float* xr, uint32_t n, uint32_t P, const float* anchors,
                             uint32_t A, uint32_t* aid, uint8_t* codes, float* factors);
uint32_t orc_build_medoid(const void* rows, int elem, uint32_t dim, uint64_t n);
void orc_build_bucket_reps(const void* rows, int elem, uint32_t dim, const uint32_t* bucket_off,
                           uint32_t buckets, float* means, uint32_t* reps);
void orc_build_links(uint32_t n, const uint32_t* knn, uint32_t knn_width, const uint32_t* bucket_of,
                     const uint32_t* reps, const uint32_t* near, uint32_t near_width, uint32_t buckets,
                     const uint32_t* order, uint32_t degree, uint32_t local, uint32_t near_links,
                     uint32_t rep_local, uint32_t rep_near, uint32_t entry, uint64_t seed,
                     uint32_t* out);
void orc_build_cagra_optimize(const uint32_t* knn, uint32_t n, uint32_t kin, uint32_t degree,
                              uint32_t* pruned, uint32_t* out);
uint32_t orc_build_reach(const uint32_t* graph, uint32_t n, uint32_t degree, uint32_t entry,
                         uint32_t* reached);

#ifdef __cplusplus
}
#endif
#endif
