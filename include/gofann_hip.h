/*
 * gofann_hip.h -- C ABI of the MI355X (gfx950) GPU stage of GO-FANN's
 * filtered graph search.  Plain C: opaque context, POD views of
 * caller-owned device arrays, int status codes, no exceptions and no
 * framework types cross this boundary.
 *
 * Reference interfaces replaced (paths relative to the GO-FANN tree):
 *   - kernel launch of native_warp_independent_search_kernel_impl
 *     (src/search/pq/backend_pq.cu:5015-5199, launched :9863-9960)
 *       -> gofann_pq_search
 *   - native_rabitq_search_kernel (src/search/rabitq/backend_rabitq.cu:
 *     4293-4470, launched :10874-10988)              -> gofann_rabitq_search
 *   - lowfreq_pq_scan_kernel (backend_pq.cu:2136-2185) -> gofann_pq_posting_scan
 *   - lowfreq_rabitq_resident_posting_kernel (backend_rabitq.cu:5751)
 *                                                     -> gofann_rabitq_posting_scan
 *   - init_prepared_query_state query preparation (backend_rabitq.cu:
 *     7800-8084; RabitqQueryRotation src/search/rabitq/
 *     rabitq_query_rotation.cuh:51-113)             -> gofann_rabitq_prepare_queries
 *   - resident_pq_batch_exact_rerank_kernel (backend_pq.cu:5201-5310) and
 *     highfreq_float_gpu_l2_kernel/_topk_kernel (backend_rabitq.cu:
 *     6173-6270)                                     -> gofann_exact_rerank
 *
 * Conventions (mirroring check_cuda/fail_pq, backend_pq.cu:1015, 1338-1343):
 * every call returns GOFANN_OK or a negative status and records a message
 * retrievable with gofann_last_error(ctx).  All array pointers are device
 * pointers unless a field says otherwise; the library never frees them.
 * Calls are asynchronous on the context's stream; outputs are valid after
 * gofann_synchronize (or an event recorded on that stream).  One context
 * per host thread; contexts never share scratch memory.
 */
#ifndef GOFANN_HIP_H
#define GOFANN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GOFANN_OK 0
#define GOFANN_ERR_INVALID -1
#define GOFANN_ERR_HIP -2
#define GOFANN_ERR_UNSUPPORTED -3
#define GOFANN_ERR_NOMEM -4

#define GOFANN_EARLY_STOP_FIXED 0 /* backend_pq.cu:1615-1617 */
#define GOFANN_EARLY_STOP_OFF 1
#define GOFANN_EARLY_STOP_ADAPTIVE 2

#define GOFANN_ELEM_U8 0
#define GOFANN_ELEM_F32 1
#define GOFANN_ELEM_F16 2

#define GOFANN_PLACE_AUTO 0
#define GOFANN_PLACE_LDS 1
#define GOFANN_PLACE_GLOBAL 2
#define GOFANN_PLACE_SPILL 3 /* visited set: 1024-slot LDS table moved to the global slab when 3/4 full */

typedef struct gofann_ctx gofann_ctx;

/* ---- context (replaces init_graph_context / cleanup, backend_pq.cu:6753) */
int gofann_create(int device, gofann_ctx** out);
void gofann_destroy(gofann_ctx* ctx);
const char* gofann_last_error(const gofann_ctx* ctx);
/* Use a caller-created hipStream_t (passed as void*); NULL = default. */
int gofann_set_stream(gofann_ctx* ctx, void* hip_stream);
int gofann_synchronize(gofann_ctx* ctx);
/* Number of the device's compute units and its LDS per workgroup. */
int gofann_device_info(gofann_ctx* ctx, int* compute_units, int* lds_bytes);
/* Placement the last traversal launch chose (no reference counterpart;
 * diagnostics): ADC table in LDS (1) or on demand (0); visited set global
 * (0), LDS (1) or spilling LDS (2); dynamic LDS bytes per route; resident
 * routes per CU.  Any pointer may be NULL. */
int gofann_last_placement(gofann_ctx* ctx, int* table_in_lds, int* hash_in_lds, int* lds_bytes,
                          int* resident_per_cu);

/* ---- device arrays -------------------------------------------------------
 * Label-partitioned graph (GraphMetadata + resident graph, src/data/
 * dataloader.h:583-602, backend_pq.cu:1516-1523).  Group g owns global rows
 * [label_offset[g], label_offset[g] + label_size[g]); adjacency entries are
 * label-local rows, UINT32_MAX = empty slot. */
typedef struct {
    const uint32_t* graph;          /* [rows][degree] */
    const uint32_t* row_to_sample;  /* [rows] */
    const uint32_t* label_offset;   /* [groups] */
    uint32_t rows;
    uint32_t degree;                /* row stride, in [1, 64]; a larger degree is
                                       GOFANN_ERR_UNSUPPORTED (backend_pq.cu:11486) */
    uint32_t groups;
    uint32_t samples;
    /* Optional [rows][degree] sample id of each adjacency entry
     * (row_to_sample[label_offset + graph[r][j]]; the reference ships the
     * same "neighbor samples" words in its graph-row payload,
     * src/execution/async_io.cpp:1025-1047).  NULL: gathered through
     * row_to_sample.  Results are identical either way. */
    const uint32_t* neighbor_samples;
} gofann_graph_view;

/* Device predicate (gpu_predicate::View, src/predicates/
 * gpu_predicate_index.cuh:25-48), CSR storage, DNF clauses per route. */
typedef struct {
    uint32_t label_begin, label_end, range_begin, range_end;
} gofann_clause;
typedef struct {
    uint32_t dimension, mode; /* mode 0 any, 1 (>lo), 2 (<hi), 3 [lo,hi) */
    float lower, upper;
} gofann_range_atom;
typedef struct {
    const uint32_t* route_offsets;     /* [routes+1] -> clauses */
    const uint32_t* route_handles;     /* clause labels */
    const gofann_clause* clauses;      /* NULL: conjunction of handles */
    const gofann_range_atom* ranges;
    const uint8_t* route_enabled;      /* NULL: enabled iff csr_offsets */
    const uint8_t* route_compiled;     /* NULL: none compiled */
    const float* base_ranges;          /* [samples][range_stride] */
    const uint32_t* csr_offsets;       /* [samples+1] sample-major labels */
    const uint32_t* csr_labels;        /* strictly increasing per row */
    uint32_t rows;                     /* samples */
    uint32_t range_stride;
    float alpha;                       /* bias penalty factor */
    int pending_base_stop;
    /* Optional 16-byte label slab per sample at label_slab + s*slab_stride
     * (16-byte aligned): u16 count, then up to 7 u16 labels, ascending --
     * the sample's CSR row inline, typically beside its PQ codes so one
     * cache line serves both.  count 0xFFFF: row too long, read the CSR.
     * Labels must be < 0xFFFF.  NULL: CSR only.  Results are identical. */
    const uint8_t* label_slab;
    uint32_t slab_stride;
    /* Attribute columns of base_ranges; 0: range_stride.  Set when the
     * values sit inside wider per-sample records (range_stride is then the
     * record stride in floats), so a range atom on a column past the last
     * still fails as it does with the plain array. */
    uint32_t range_columns;
} gofann_predicate_view;

/* Routes of one batch.  Route r searches group route_group[r] from the
 * label-local seed route_start[r] with query vector route_query[r].  The
 * legacy filter arrays (uncompiled routes) may be NULL = pass. */
typedef struct {
    const uint32_t* route_query;
    const uint32_t* route_group;
    const uint32_t* route_start;
    const uint64_t* row_filter_mask;   /* [rows] */
    const uint64_t* query_filter_bits; /* [routes] */
    const uint8_t* range_modes;        /* [routes][range_count] */
    const float* range_lower;
    const float* range_upper;
    const float* base_range_values;    /* [samples][range_count] */
    uint32_t range_count;
    uint32_t count;
    /* Optional host-side hint: launch order (device array of route ids);
     * NULL = identity.  Results stay indexed by route id. */
    const uint32_t* launch_order;
} gofann_routes;

typedef struct {
    int queue_limit;    /* beam Q */
    int finish_limit;   /* fixed early stop limit */
    int early_stop_mode;
    int max_steps;      /* 0 = unlimited */
    int stop_width;     /* <= 10 */
    int result_width;   /* W, shortlist handed to rerank, <= 512 */
    float bit_filter_bonus;
    float range_filter_bonus;
    int predicate_bias; /* kPredicateBias */
    /* Exact distance of every expanded predicate-passing node ranks the
     * result/stop heaps (enable_true_distance_rerank, backend_pq.cu:
     * 4507-4546, 4566-4572); needs gofann_pq_view.exact_base. */
    int inline_exact_rerank;
    /* Placement of per-route state; results are identical in every mode.
     * table_mode (PQ): 0 auto, 1 ADC table in LDS (computePQTable layout,
     * M x 256 fp32), 2 table entries computed on demand from the
     * L2-resident centroid table (same fma chain, so the same bits).
     * hash_mode (visited set): 0 auto, 1 the 4096-slot table in LDS, 2 the
     * same table in a per-route global slab, 3 a 1024-slot LDS table moved
     * into the global slab before it passes 3/4 load.
     * Auto picks the placement with the most resident routes per CU. */
    int table_mode;
    int hash_mode;
} gofann_search_params;

/* Per-route counters emitted by the traversal kernels (bytes model). */
typedef struct {
    int32_t steps;
    int32_t expanded;
    int32_t passed;
    int32_t scored;
    int32_t pred_rows;
    int32_t pred_labels;
    int32_t admitted;
    int32_t exhausted;
} gofann_route_stats;

typedef struct {
    const uint8_t* codes;     /* [samples][pq_dim] */
    const float* centroids;   /* [256][dim] */
    uint32_t dim;
    uint32_t pq_dim;
    uint32_t samples;
    const void* exact_base;   /* [samples][dim] u8 or f32 (matches the queries); may be NULL */
    uint32_t code_stride;     /* bytes between code rows; 0 = pq_dim (codes inside wider
                                 per-sample records); multiple of 16 when pq_dim % 16 == 0 */
} gofann_pq_view;

typedef struct {
    const uint8_t* codes;          /* [samples][padded_dim/8], MSB-first u32 words */
    const float* factors;          /* [samples][3] f_add, f_rescale, f_err */
    const uint32_t* anchor_ids;    /* [samples] */
    const float* anchors;          /* [anchors][padded_dim], rotated centroids */
    uint32_t dim;
    uint32_t padded_dim;
    uint32_t num_anchors;
    uint32_t samples;
    /* Optional per-sample records read by the graph traversal in place of
     * the three arrays above (no counterpart in the reference, which keeps
     * them apart): record s at records + s * record_stride holds the code
     * row (padded_dim/8 bytes) at offset 0, then f_add and f_rescale (f32)
     * and the anchor id (u32), so one memory line serves a scored
     * candidate; the predicate view's label_slab and base_ranges may point
     * into the same records.  record_stride: multiple of 16, at least
     * padded_dim/8 + 12; records 16-byte aligned.  NULL: the arrays.
     * Results are identical either way; the arrays stay required (the
     * posting scans and the row builders read them). */
    const uint8_t* records;
    uint32_t record_stride;
} gofann_rabitq_view;

/* Prepared RaBitQ queries (init_prepared_query_state outputs). */
typedef struct {
    float* rotated;          /* [queries][padded_dim] */
    int8_t* q8;              /* [queries][padded_dim] */
    float* scale;            /* [queries] */
    float* k1;               /* [queries] */
    float* centroid_dists;   /* [queries][num_anchors] */
    uint32_t count;
} gofann_rabitq_queries;

/* ---- PQ traversal (backend_pq.cu:3980-5199, device-resident transport).
 * queries: [n][dim] u8 (query_elem GOFANN_ELEM_U8) or f32.  Outputs per
 * route: out_ids/out_dists [routes][result_width] ascending, sample ids,
 * UINT32_MAX / FLT_MAX padding; stats may be NULL. */
int gofann_pq_search(gofann_ctx* ctx, const gofann_pq_view* pq,
                     const void* queries, int query_elem,
                     const gofann_graph_view* graph,
                     const gofann_predicate_view* predicate,
                     const gofann_routes* routes,
                     const gofann_search_params* params,
                     uint32_t* out_ids, float* out_dists,
                     gofann_route_stats* stats);

/* ---- RaBitQ query preparation: rotation GEMM on MFMA (FP32 operands),
 * int8 quantization, query factors, centroid distances.  queries [n][dim]
 * f32; rotation [dim][padded_dim] row-major (y = q R). */
int gofann_rabitq_prepare_queries(gofann_ctx* ctx, const gofann_rabitq_view* rq,
                                  const float* queries, uint32_t count,
                                  const float* rotation,
                                  gofann_rabitq_queries* out);

/* ---- RaBitQ traversal (backend_rabitq.cu:3487-4470). */
int gofann_rabitq_search(gofann_ctx* ctx, const gofann_rabitq_view* rq,
                         const gofann_rabitq_queries* prepared,
                         const gofann_graph_view* graph,
                         const gofann_predicate_view* predicate,
                         const gofann_routes* routes,
                         const gofann_search_params* params,
                         uint32_t* out_ids, float* out_dists,
                         gofann_route_stats* stats);

/* ---- posting scans (backend_pq.cu:2046-2185; backend_rabitq.cu:5494-5682).
 * Route r scans sample ids cand_ids[cand_offsets[r] .. + cand_sizes[r]).
 * Outputs [routes][shortlist_k] ascending by (distance, id); pass_counts
 * (may be NULL) receives the predicate passes per route. */
int gofann_pq_posting_scan(gofann_ctx* ctx, const gofann_pq_view* pq,
                           const void* queries, int query_elem,
                           const gofann_predicate_view* predicate,
                           const uint32_t* route_query, const uint32_t* cand_ids,
                           const uint32_t* cand_offsets, const uint32_t* cand_sizes,
                           uint32_t routes, int shortlist_k,
                           uint32_t* out_ids, float* out_dists,
                           uint32_t* pass_counts);

int gofann_rabitq_posting_scan(gofann_ctx* ctx, const gofann_rabitq_view* rq,
                               const gofann_rabitq_queries* prepared,
                               const gofann_predicate_view* predicate,
                               const uint32_t* route_query, const uint32_t* cand_ids,
                               const uint32_t* cand_offsets, const uint32_t* cand_sizes,
                               uint32_t routes, int shortlist_k,
                               uint32_t* out_ids, float* out_dists,
                               uint32_t* pass_counts);

/* ---- full-GPU exact route (run_full_gpu_highfreq_route, src/search/
 * full_gpu/backend_full_gpu.cu:1682-2042, launched by full_gpu_highfreq_kernel
 * :2045-2122).  Beam search keyed by the exact squared L2 (u8: the integer,
 * returned as float; f32 and f16: l2_distance_device's warp order,
 * :1107-1160, as GOFANN_EXACT_ORDER_WARP below); every expanded node is
 * filtered (row mask & route bits, all active legacy ranges of `routes`,
 * the route predicate when enabled) and a passing node enters a sorted
 * best-topk with sample dedup.  base [samples][dim] and queries [n][dim]
 * both of base_elem (u8, f32 or f16 -- the reference's template T for both;
 * base 16-byte aligned).  label_size
 * [groups] (device; NULL: adjacency entries are trusted) bounds each group's
 * local ids.  Outputs [routes][topk] ascending by (distance, id), padded
 * UINT32_MAX / FLT_MAX; stats (may be NULL) per route. */
typedef struct {
    int queue_limit;     /* [2, 1024] */
    int finish_limit;    /* fixed early stop limit */
    int early_stop_mode;
    int max_steps;       /* 0 = unlimited */
    int topk;            /* [1, 10] */
    int hash_mode;       /* visited-set placement, as gofann_search_params.hash_mode */
} gofann_exact_params;

int gofann_exact_search(gofann_ctx* ctx, const void* base, int base_elem, uint32_t dim,
                        uint32_t samples, const void* queries, const gofann_graph_view* graph,
                        const uint32_t* label_size, const gofann_predicate_view* predicate,
                        const gofann_routes* routes, const gofann_exact_params* params,
                        uint32_t* out_ids, float* out_dists, gofann_route_stats* stats);

/* ---- full-GPU exact route that allocates nothing.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Arguments, results and placement choice are those of
 * gofann_exact_search, but a visited set outside LDS (hash_mode 2 or 3, or
 * auto choosing one) lives in a fixed per-GPU device array of
 * GOFANN_EXACT_NOALLOC_MAX_ROUTES x 4096 u32 (64 MiB, held by each GPU the
 * library runs on until the process ends) instead of context scratch; such
 * a call takes at most GOFANN_EXACT_NOALLOC_MAX_ROUTES routes, and a larger
 * batch is GOFANN_ERR_INVALID before anything is launched.  No hipMalloc,
 * hipFree or allocating library routine is called.  Every call on one GPU
 * shares the array (each route clears its slab before use): calls that
 * overlap on one GPU, from any context or stream, race. */
#define GOFANN_EXACT_NOALLOC_MAX_ROUTES 4096
int gofann_exact_search_noalloc(gofann_ctx* ctx, const void* base, int base_elem, uint32_t dim,
                                uint32_t samples, const void* queries,
                                const gofann_graph_view* graph, const uint32_t* label_size,
                                const gofann_predicate_view* predicate,
                                const gofann_routes* routes, const gofann_exact_params* params,
                                uint32_t* out_ids, float* out_dists, gofann_route_stats* stats);

/* ---- exact posting scans of the full-GPU backend (full_gpu_range_posting_
 * kernel, src/search/full_gpu/backend_full_gpu.cu:1383-1493, and
 * full_gpu_lowfreq_kernel :2124-2262).  Route r scans the sample ids
 * cand_ids[cand_offsets[r] .. + cand_sizes[r]) against query
 * route_query[r]; ids UINT32_MAX or >= samples are skipped, and with the
 * route predicate enabled only passing samples count.  Each is scored by
 * exact squared L2 (base [samples][dim] and queries [n][dim] both of
 * base_elem: u8, f32 or f16; base 16-byte aligned) in `order`:
 *   GOFANN_EXACT_ORDER_SERIAL -- one chain over d ascending, the range
 *     posting kernel's order (:1443-1469);
 *   GOFANN_EXACT_ORDER_WARP -- l2_distance_device's warp order (:1107-1160;
 *     u8: the integer sum), the low-frequency group kernel's.
 * Outputs [routes][topk] (topk <= 64): the topk least (distance, id) pairs
 * over the distinct passing samples (insert_best_result's sample dedup,
 * :1333-1375), ascending, padded UINT32_MAX / FLT_MAX; a NaN distance is
 * dropped.  pass_counts (may be NULL): passing listed samples per route,
 * duplicates included. */
#define GOFANN_EXACT_ORDER_SERIAL 0
#define GOFANN_EXACT_ORDER_WARP 1
int gofann_exact_posting_scan(gofann_ctx* ctx, const void* base, int base_elem, uint32_t dim,
                              uint32_t samples, const void* queries,
                              const gofann_predicate_view* predicate,
                              const uint32_t* route_query, const uint32_t* cand_ids,
                              const uint32_t* cand_offsets, const uint32_t* cand_sizes,
                              uint32_t routes, int topk, int order,
                              uint32_t* out_ids, float* out_dists, uint32_t* pass_counts);

/* ---- range postings ------------------------------------------------------
 * Posting segments (posting_segments::Plan, src/execution/
 * posting_segment_plan.h:12-18).  Segment s scans posting rows
 * [offsets[s], offsets[s] + sizes[s]) for route route_ids[s].  With
 * query_indptr, output row p merges segments [query_indptr[p],
 * query_indptr[p+1]); without it (NULL) segment s is output row s. */
typedef struct {
    const uint32_t* route_ids;     /* [count] */
    const uint64_t* offsets;       /* [count] */
    const uint64_t* sizes;         /* [count] */
    uint32_t count;
    const uint32_t* query_indptr;  /* [positions + 1] or NULL */
    uint32_t positions;
} gofann_posting_segments;

/* Host: posting_segments::make_plan (posting_segment_plan.h:20-51) over
 * host arrays -- each posting of n split into ceil(size / target_rows)
 * near-equal segments (one empty segment for an empty posting).  Fills the
 * outputs when capacity covers the plan; *out_count always receives the
 * segment count.  Returns GOFANN_OK, or GOFANN_ERR_INVALID (target_rows 0,
 * missing arrays, capacity short) / GOFANN_ERR_UNSUPPORTED (overflow). */
int gofann_posting_segment_plan(const uint32_t* route_ids, const uint64_t* offsets,
                                const uint64_t* sizes, uint32_t n, uint32_t target_rows,
                                uint32_t capacity, uint32_t* seg_route_ids,
                                uint32_t* seg_positions, uint64_t* seg_offsets,
                                uint64_t* seg_sizes, uint32_t* query_indptr,
                                uint32_t* out_count);

/* Host: range_posting::choose_smallest_slice (src/index/
 * range_posting_index.cpp:277-312) for rows [0, n) of a query range table
 * (modes/lower/upper [n][range_count], host).  Dimension r of the ordered
 * range posting index has unique_counts[r] strictly increasing values
 * unique_values[r] and offsets[r] ([unique_counts[r] + 1] row offsets).
 * out[q] = {has_active_range, active_dimension_count, range_index, begin,
 * count} (begin dimension-local; range_index UINT32_MAX when none). */
int gofann_range_slices(const float* const* unique_values, const uint64_t* const* offsets,
                        const uint64_t* unique_counts, uint32_t range_count,
                        const uint8_t* modes, const float* lower, const float* upper,
                        uint32_t n, uint64_t* out);

/* ---- RaBitQ range-posting scan (range_posting_rabitq_scan_kernel,
 * backend_rabitq.cu:5846-6015) with the segment merge (merge_one_query,
 * posting_segment_merge.cuh:12-46).  posting: [resident_rows] sample ids
 * (device).  routes: route_query and the query range table (range_modes,
 * range_lower, range_upper, base_range_values, range_count).  Rows with a
 * sample >= rq->samples are skipped.  score_first: consult an enabled
 * predicate only for rows that can enter the shortlist (results are the
 * same; pass counts follow that order).  Outputs [rows][shortlist_k]
 * ascending by (distance, id), padding UINT32_MAX / FLT_MAX; pass_counts
 * [rows] (may be NULL); rows = positions with query_indptr, else
 * segments.  shortlist_k <= 4096. */
int gofann_rabitq_range_scan(gofann_ctx* ctx, const gofann_rabitq_view* rq,
                             const gofann_rabitq_queries* prepared,
                             const gofann_predicate_view* predicate,
                             const gofann_routes* routes, const uint32_t* posting_sample_ids,
                             uint64_t resident_rows, const gofann_posting_segments* segments,
                             int shortlist_k, int score_first, uint32_t* out_ids,
                             float* out_dists, uint32_t* pass_counts);

/* ---- posting-resident RaBitQ rows: no counterpart in the reference, whose
 * range scan gathers every row by sample id (backend_rabitq.cu:5920-5960).
 * A copy of each posting row's RaBitQ row in posting order lets the scan
 * stream both arrays instead of gathering: codes [rows][padded_dim/8] and
 * aux [rows][4] u32 = {f_add bits, f_rescale bits, anchor id, 0}.  Rows
 * whose sample is >= rq->samples are zero.  gofann_rabitq_posting_rows
 * fills them from rq (device gather); gofann_rabitq_range_scan_resident is
 * gofann_rabitq_range_scan reading row r of every segment from the copies
 * (the same results, bit for bit). */
int gofann_rabitq_posting_rows(gofann_ctx* ctx, const gofann_rabitq_view* rq,
                               const uint32_t* posting_sample_ids, uint64_t rows,
                               uint8_t* out_codes, uint32_t* out_aux);

int gofann_rabitq_range_scan_resident(gofann_ctx* ctx, const gofann_rabitq_view* rq,
                                      const gofann_rabitq_queries* prepared,
                                      const gofann_predicate_view* predicate,
                                      const gofann_routes* routes,
                                      const uint32_t* posting_sample_ids, uint64_t resident_rows,
                                      const uint8_t* posting_codes, const uint32_t* posting_aux,
                                      const gofann_posting_segments* segments, int shortlist_k,
                                      int score_first, uint32_t* out_ids, float* out_dists,
                                      uint32_t* pass_counts);

/* ---- label postings in posting order: gofann_rabitq_posting_scan
 * (lowfreq_rabitq_resident_posting_kernel, backend_rabitq.cu:5494-5682)
 * over an explicit segment plan, so that a long posting is scanned by many
 * workgroups, with optional posting-order copies of what each row's filter
 * and score read.  No counterpart in the reference, whose scan gathers the
 * label row, range value and code of every posting row by sample id.
 *
 * gofann_posting_predicate_rows fills, for rows [0, rows) of a posting
 * array: out_slab [rows][4] u32 -- the sample's label row as a 16-byte slab
 * (u16 count, then up to 7 u16 labels in CSR order; count 0xFFFF when the
 * row has more labels, a label above 0xFFFF, no CSR, or the sample is
 * >= predicate->rows) -- and out_ranges [rows][predicate->range_stride]
 * (the sample's base range row; zeros without base ranges; may be NULL).
 *
 * gofann_rabitq_posting_scan_segments: segment s scans
 * posting_sample_ids[offsets[s] .. + sizes[s]) (clipped to posting_rows)
 * for route route_ids[s], filtered by the route's predicate alone, as
 * gofann_rabitq_posting_scan does; with segments->query_indptr, output row
 * p is route p's merge of segments [query_indptr[p], query_indptr[p+1]).
 * With a plan from gofann_posting_segment_plan over (cand_offsets,
 * cand_sizes) the outputs equal gofann_rabitq_posting_scan's bit for bit.
 * posting_codes/posting_aux (gofann_rabitq_posting_rows over the same
 * posting array, together or both NULL) and posting_slab/posting_ranges
 * (gofann_posting_predicate_rows; ranges need the slab) are read at the
 * row's posting position instead of gathered by sample id; any may be
 * NULL.  shortlist_k <= 4096. */
int gofann_posting_predicate_rows(gofann_ctx* ctx, const gofann_predicate_view* predicate,
                                  const uint32_t* posting_sample_ids, uint64_t rows,
                                  uint32_t* out_slab, float* out_ranges);

int gofann_rabitq_posting_scan_segments(gofann_ctx* ctx, const gofann_rabitq_view* rq,
                                        const gofann_rabitq_queries* prepared,
                                        const gofann_predicate_view* predicate,
                                        const uint32_t* route_query,
                                        const uint32_t* posting_sample_ids, uint64_t posting_rows,
                                        const gofann_posting_segments* segments, int shortlist_k,
                                        const uint8_t* posting_codes, const uint32_t* posting_aux,
                                        const uint32_t* posting_slab,
                                        const float* posting_ranges, uint32_t* out_ids,
                                        float* out_dists, uint32_t* pass_counts);

/* ---- label-shared posting scan: no counterpart in the reference, which
 * scans every label posting route by route (the label-posting scan of
 * backend_rabitq.cu:5494-5682, which gofann_rabitq_posting_scan_segments
 * restates).  The segments of a plan that scan the same posting rows (the
 * routes of one label) are listed together in a share plan: item i covers
 * posting rows [item_offsets[i], + item_sizes[i]) for the plan segments
 * item_slots[item_begin[i] .. item_begin[i+1]) (each with exactly that
 * offset and size).  One workgroup per item reads the rows' posting-order
 * columns once and filters and scores them for every route of the item, 16
 * route slots per pass over the rows: items of at most 16 routes take one
 * pass, larger items re-read their rows once per further 16.  Takes posting_codes, posting_aux and posting_slab
 * (posting_ranges optional), shortlist_k <= 128 and padded_dim <= 1024
 * (GOFANN_ERR_UNSUPPORTED otherwise); every output equals
 * gofann_rabitq_posting_scan_segments' for the same plan, bit for bit. */
typedef struct {
    const uint64_t* item_offsets; /* [items] */
    const uint64_t* item_sizes;   /* [items] */
    const uint32_t* item_begin;   /* [items + 1] into item_slots */
    const uint32_t* item_slots;   /* plan segment indices */
    uint32_t items;
} gofann_posting_share;

int gofann_rabitq_posting_scan_shared(gofann_ctx* ctx, const gofann_rabitq_view* rq,
                                      const gofann_rabitq_queries* prepared,
                                      const gofann_predicate_view* predicate,
                                      const uint32_t* route_query,
                                      const uint32_t* posting_sample_ids, uint64_t posting_rows,
                                      const gofann_posting_segments* segments,
                                      const gofann_posting_share* share, int shortlist_k,
                                      const uint8_t* posting_codes, const uint32_t* posting_aux,
                                      const uint32_t* posting_slab,
                                      const float* posting_ranges, uint32_t* out_ids,
                                      float* out_dists, uint32_t* pass_counts);

/* ---- exact rerank on the GPU: per route, unique valid candidates of the
 * shortlist, exact L2 against base[samples][dim] (u8 / f32 / f16 with f32
 * queries for f32 and f16, u8 queries for u8), top-k by (distance, id). */
int gofann_exact_rerank(gofann_ctx* ctx, const void* base, int base_elem,
                        uint32_t dim, uint32_t samples, const void* queries,
                        const uint32_t* route_query, const uint32_t* shortlist,
                        uint32_t width, uint32_t routes, uint32_t topk,
                        uint32_t* out_ids, float* out_dists);

/* ---- route -> original query merge (merge_route_results_to_original,
 * src/search/rabitq/rabitq_lowfreq_merge.h:709-815): query q owns routes
 * query_routes[query_route_offsets[q] .. [q+1]); per query, minimum
 * distance per sample, (distance, id) order, first topk (<= 64). */
int gofann_merge_routes(gofann_ctx* ctx, const uint32_t* query_route_offsets,
                        const uint32_t* query_routes, const uint32_t* route_ids,
                        const float* route_dists, uint32_t width, uint32_t queries,
                        uint32_t topk, uint32_t* out_ids, float* out_dists);

/* ---- device predicate bitsets (prepare_candidate_pass_masks,
 * src/predicates/gpu_predicate_parallel.cuh:21-42): bit i % 32 of
 * masks[i / 32] = matches(route_ids[i], sample_ids[i]); ceil(n/32) words. */
int gofann_predicate_masks(gofann_ctx* ctx, const gofann_predicate_view* predicate,
                           const uint32_t* route_ids, const uint32_t* sample_ids,
                           uint32_t n, uint32_t* masks);

/* ---- batched scoring of explicit candidate lists (minimum-slice entry
 * points): out[i] = ADC / RaBitQ estimate of (query q_idx[i], sample s[i]).
 * PQ uses the traversal's summation order; RaBitQ also returns the exact
 * integer dot product ip_int[i] (may be NULL). */
int gofann_pq_score(gofann_ctx* ctx, const gofann_pq_view* pq, const void* queries,
                    int query_elem, const uint32_t* q_idx, const uint32_t* s_idx,
                    uint32_t n, float* out);
int gofann_rabitq_score(gofann_ctx* ctx, const gofann_rabitq_view* rq,
                        const gofann_rabitq_queries* prepared, const uint32_t* q_idx,
                        const uint32_t* s_idx, uint32_t n, float* out, int32_t* ip_int);

/* ---- streamed CPU exact rerank (run_highfreq_streaming_rerank and
 * highfreq_host_batch_rerank_range, backend_pq.cu:9646-9738, 2479-2592;
 * exact_l2_u8 :2187-2195).  A host worker pool over caller-owned host
 * arrays: base [samples][dim] (u8 / f32 / f16) and queries [n][dim] (u8 for
 * a u8 base, else f32).  Per route: valid unique shortlist ids, exact fp32
 * L2 with dimensions in order, top-k by (distance, id), ascending, padded
 * with UINT32_MAX / FLT_MAX.  The shortlist is taken as predicate-verified
 * (device predicates admit only passing nodes to the result heap). */
typedef struct gofann_host_rerank gofann_host_rerank;
int gofann_host_rerank_create(const void* base, int base_elem, uint32_t dim, uint32_t samples,
                              const void* queries, uint32_t threads, gofann_host_rerank** out);
void gofann_host_rerank_destroy(gofann_host_rerank* hr);
const char* gofann_host_rerank_last_error(const gofann_host_rerank* hr);
/* fp16 rows: the L2 kernel chosen at create, as the reference chooses it
 * (fp16_l2::select, src/data/fp16_l2.h:53-70): environment variable
 * GOFANN_FP16_RERANK_KERNEL (or, when that is unset, the reference's
 * GO_FANN_FP16_RERANK_KERNEL) = auto (AVX-512 if the CPU has it, else AVX2,
 * else scalar) | scalar | avx2 | avx512, each with the reference kernel's
 * summation order.  Read only when base_elem is GOFANN_ELEM_F16, as the
 * reference reads it only for fp16 sources (dataloader.cpp:2132): for those
 * an unknown name makes create return GOFANN_ERR_INVALID, an ISA the CPU
 * lacks GOFANN_ERR_UNSUPPORTED.  Returns "scalar", "avx2" or "avx512"
 * ("scalar" for u8 and f32 rows, which take no fp16 kernel). */
const char* gofann_host_rerank_fp16_kernel(const gofann_host_rerank* hr);
/* Host arrays only: shortlist [routes][width], route_query [routes],
 * outputs [routes][topk]. */
int gofann_host_rerank_routes(gofann_host_rerank* hr, const uint32_t* shortlist, uint32_t width,
                              const uint32_t* route_query, uint32_t routes, uint32_t topk,
                              uint32_t* out_ids, float* out_dists);
/* PQ traversal (as gofann_pq_search, routes in id order, launch_order
 * NULL) in chunks of chunk_routes on the context's stream; each chunk's
 * shortlist (params->result_width ids) is copied to pinned host memory on a
 * copy stream after the chunk's event and reranked on the host while later
 * chunks search.  route_query_host: host copy of routes->route_query;
 * out_ids / out_dists: host [routes][topk].  Returns when every route is
 * reranked. */
int gofann_pq_search_host_rerank(gofann_ctx* ctx, gofann_host_rerank* hr, const gofann_pq_view* pq,
                                 const void* queries, int query_elem,
                                 const gofann_graph_view* graph,
                                 const gofann_predicate_view* predicate,
                                 const gofann_routes* routes, const gofann_search_params* params,
                                 const uint32_t* route_query_host, uint32_t chunk_routes,
                                 uint32_t topk, uint32_t* out_ids, float* out_dists,
                                 gofann_route_stats* stats);
/* Host route -> query merge (merge_route_results_to_original,
 * rabitq_lowfreq_merge.h:709-815); host arrays, as gofann_merge_routes. */
int gofann_host_merge_routes(const uint32_t* query_route_offsets, const uint32_t* query_routes,
                             const uint32_t* route_ids, const float* route_dists, uint32_t width,
                             uint32_t queries, uint32_t topk, uint32_t* out_ids, float* out_dists);

/* ---- Reference artifacts on disk (host only).  Readers validate what the
 * reference's loaders validate; each returns GOFANN_OK or a negative status
 * with a message from gofann_io_last_error() (per host thread).  Outputs are
 * caller-allocated host arrays sized from the matching *_read_header call;
 * pinned buffers stream straight into device memory.  Output pointers noted
 * "may be NULL" skip that array. */
const char* gofann_io_last_error(void);

/* FDRG graph file (src/index/graph_file_format.h:16-25): 4096-byte header
 * block, rows of `degree` u32 packed 4096/(4*degree) to a 4096-byte block,
 * block tails zero. */
typedef struct {
    uint32_t magic;          /* 0x47524446 "FDRG" */
    uint32_t version;        /* 1 */
    uint32_t block_size;     /* 4096 */
    uint32_t header_size;    /* 4096 */
    uint64_t rows;
    uint32_t degree;
    uint32_t row_size_bytes; /* 4 * degree */
    uint64_t rows_per_block; /* 4096 / row_size_bytes */
} gofann_graph_file_header;

/* has_graph_file_magic (graph_file_format.cpp): 1 / 0, or a negative status
 * when the file has no 4-byte marker. */
int gofann_graph_file_has_magic(const char* path);
/* read_graph_file_header (graph_file_format.cpp) with all of its checks. */
int gofann_graph_file_read_header(const char* path, gofann_graph_file_header* out);
/* Rows [row_begin, row_begin + row_count) as a row-major [row_count][degree]
 * matrix (load_graph_file_as_contiguous_matrix over a window). */
int gofann_graph_file_read_rows(const char* path, uint64_t row_begin, uint64_t row_count,
                                uint32_t* out);
/* GraphFileSequentialWriter (graph_file_format.h:40-55) over a whole
 * [row_count][degree] matrix; byte-identical to the reference's file. */
int gofann_graph_file_write(const char* path, const uint32_t* rows, uint64_t row_count,
                            uint32_t degree);
/* convert_legacy_graph_file (graph_file_format.cpp): u64 rows, u64 cols,
 * then rows*cols u32 -> FDRG. */
int gofann_graph_file_convert_legacy(const char* legacy_path, const char* path);

/* Graph metadata sidecar (GraphMetadataSidecarHeader, src/data/
 * dataloader.h:630-644; payload dataloader.cpp:7782-7821): the arrays a
 * gofann_graph_view and gofann_routes take (label_offset, row_to_sample,
 * row_filter_mask) with label_size, cat_freq and label_filter_bit. */
typedef struct {
    uint32_t version;  /* 1 */
    uint32_t reserved;
    uint64_t label_count;  /* groups */
    uint64_t group_count;
    uint64_t original_label_count;
    uint64_t num_points;
    uint64_t row_limit;
    uint64_t graph_rows;
    uint64_t total_rows;
    uint64_t graph_degree;
    uint64_t specificity_threshold;
    uint64_t group_layout_checksum;
} gofann_graph_metadata_header;

int gofann_graph_metadata_read_header(const char* path, gofann_graph_metadata_header* out);
/* [label_count] u32 x4, row_to_sample [total_rows] u32, row_filter_mask
 * [total_rows] u64, label_filter_bit [original_label_count] u64; any output
 * may be NULL.  Checks load_metadata_sidecar's vector rules
 * (dataloader.cpp:7612-7690) that need no group layout. */
int gofann_graph_metadata_read(const char* path, uint32_t* cat_freq, uint32_t* group_posting_size,
                               uint32_t* label_size, uint32_t* label_offset,
                               uint32_t* row_to_sample, uint64_t* row_filter_mask,
                               uint64_t* label_filter_bit);
/* save_metadata_sidecar (dataloader.cpp:7782-7821); row_filter_mask NULL
 * writes all-ones (one label per group). */
int gofann_graph_metadata_write(const char* path, const gofann_graph_metadata_header* header,
                                const uint32_t* cat_freq, const uint32_t* group_posting_size,
                                const uint32_t* label_size, const uint32_t* label_offset,
                                const uint32_t* row_to_sample, const uint64_t* row_filter_mask,
                                const uint64_t* label_filter_bit);
/* group_layout_checksum (dataloader.cpp:320-332) of groups given as CSR
 * (group_offsets [groups+1], group_labels); both NULL = one label per group. */
uint64_t gofann_group_layout_checksum(const uint32_t* group_offsets, const uint32_t* group_labels,
                                      uint32_t groups, uint32_t label_count);

/* Seed sidecar (GraphSeedFileHeader, dataloader.h:609-617): label-local
 * seed row per group, UINT32_MAX for an empty group. */
typedef struct {
    uint32_t version;  /* 2 */
    uint32_t reserved;
    uint64_t label_count;
    uint64_t num_points;
    uint64_t graph_rows;
    uint64_t graph_degree;
    uint64_t specificity_threshold;
} gofann_graph_seed_header;

int gofann_graph_seeds_read_header(const char* path, gofann_graph_seed_header* out);
/* seeds [label_count]; label_size (may be NULL) enables load_seed_sidecar's
 * per-label check (dataloader.cpp:7538-7550). */
int gofann_graph_seeds_read(const char* path, const uint32_t* label_size, uint32_t* seeds);
int gofann_graph_seeds_write(const char* path, const gofann_graph_seed_header* header,
                             const uint32_t* seeds);

/* .spmat label matrix (load_spmat_labels, dataloader.cpp:6663-6760): u64
 * rows, cols, nnz, indptr [rows+1] u64, indices [nnz] u32. */
int gofann_spmat_read_header(const char* path, uint64_t* rows, uint64_t* cols, uint64_t* nnz);
/* First min(row_limit, rows) rows (row_limit 0 = all) as CSR with each row
 * sorted and de-duplicated: indptr [rows'+1], indices capacity >= header
 * nnz; *out_nnz receives the compacted count. */
int gofann_spmat_read(const char* path, uint32_t row_limit, uint64_t* indptr, uint32_t* indices,
                      uint64_t capacity, uint64_t* out_nnz);

/* query_range.bin (load_query_range_binary, dataloader.cpp:6780-6880):
 * u32 query_count, [u32 range_count], records {u8 mode, f32 upper, f32
 * lower} packed (9 bytes) or aligned (12).  path NULL or "" = one zero range
 * per query.  *record_bytes receives 9, 12 or 0 (no file). */
int gofann_query_range_read_header(const char* path, uint32_t expected_queries,
                                   uint32_t* range_count, uint32_t* record_bytes);
/* modes/lower/upper [expected_queries][range_count]: the layout of
 * gofann_routes' range table. */
int gofann_query_range_read(const char* path, uint32_t expected_queries, uint8_t* modes,
                            float* lower, float* upper);

/* rabitq.b1.bin v2 (RabitqArtifactHeader + RabitqCodecSpec, backend_rabitq.
 * cuh:16-32; arrays backend_rabitq.cu:2748-2845).  The rotation on disk is
 * [padded_dim][padded_dim]; its first dim rows are the [dim][padded_dim]
 * matrix gofann_rabitq_prepare_queries takes.  anchors, anchor_ids, codes
 * and factors are gofann_rabitq_view's arrays as they lie. */
typedef struct {
    uint32_t version;  /* 2 */
    uint32_t dim;
    uint32_t num_anchors;
    uint32_t code_bytes;  /* 4 * short_code_words */
    uint64_t num_points;
    uint32_t padded_dim;  /* multiple of 64, >= dim */
    uint32_t bits_per_dim;
    uint32_t short_code_words;
    uint32_t long_code_bytes;
    uint32_t layout_flags;  /* bits 0..2 set */
    uint32_t short_factor_count;  /* 3 */
    uint32_t ex_factor_count;     /* 2 */
} gofann_rabitq_file_header;

/* load_rabitq_index's header, codec and payload-size checks. */
int gofann_rabitq_file_read_header(const char* path, gofann_rabitq_file_header* out);
/* Arrays in file order; every output may be NULL (anchor ids are range
 * checked either way). */
int gofann_rabitq_file_read(const char* path, float* anchors, float* rotation,
                            float* query_scaling_factors, uint32_t* anchor_ids, uint8_t* codes,
                            uint8_t* long_codes, float* factors, float* ex_factors);
/* save_rabitq_index; rotation, query_scaling_factors and ex_factors may be
 * NULL (written as zeros). */
int gofann_rabitq_file_write(const char* path, const gofann_rabitq_file_header* header,
                             const float* anchors, const float* rotation,
                             const float* query_scaling_factors, const uint32_t* anchor_ids,
                             const uint8_t* codes, const uint8_t* long_codes, const float* factors,
                             const float* ex_factors);

/* DiskANN-style PQ files (writer tools/quantization/pq_builder.cu:110-122;
 * loader load_pq_pivots_local / load_pq_index, backend_pq.cu:1716-1823). */
int gofann_pq_pivots_read_header(const char* path, uint32_t* dim, uint32_t* pq_dim);
/* centroids [256][dim] = centre + mean (one f32 add, as load_pq_index);
 * pq_dim 0 accepts the file's.  Non-uniform chunk boundaries are
 * GOFANN_ERR_UNSUPPORTED. */
int gofann_pq_pivots_read(const char* path, uint32_t pq_dim, float* centroids);
int gofann_pq_codes_read_header(const char* path, uint64_t* rows, uint32_t* pq_dim);
/* Code rows [row_begin, row_begin + row_count); out_stride 0 = pq_dim, or
 * the byte stride of wider per-sample records (gofann_pq_view.code_stride). */
int gofann_pq_codes_read(const char* path, uint64_t row_begin, uint64_t row_count, uint8_t* out,
                         uint32_t out_stride);
/* Both files, with a zero mean and uniform boundaries, as pq_builder. */
int gofann_pq_files_write(const char* pivots_path, const char* codes_path, const float* centroids,
                          uint32_t dim, uint32_t pq_dim, const uint8_t* codes, uint64_t rows);

/* ---- index construction on the GPU (offline build).  The reference builds
 * its per-label graphs with cuVS CAGRA (build_cagra_graph_chunk,
 * src/index/graph_builder.cu:1279-1315: graph_degree R, intermediate degree
 * 2R, guarantee_connectivity), its PQ codebooks and codes with cuVS PQ
 * (tools/quantization/pq_builder.cu:49-153) and its RaBitQ codes with the
 * vendored IVF-RaBitQ encoder (third_party/cuvs_rabitq/src/neighbors/
 * ivf_rabitq/gpu_index/quantizer_gpu_fast.cu:39-101, 180-265).  These entry
 * points replace those calls.  Every output is defined by a fixed
 * arithmetic order and is deterministic:
 *   score of a row x against a centre c: |c|^2 - 2 <x, c>, both sums in
 *     fp32 with fmaf over d ascending; the nearest centre is the least
 *     (score, index);
 *   distance between two rows: sum_d (x_d - y_d)^2, fmaf over d ascending;
 *   ties always go to the lower index.
 * All arrays are device memory unless stated; rows are [n][dim] of
 * elem (GOFANN_ELEM_U8 / F32 / F16), centres f32. */

/* Nearest centre of each row: out_idx[i] = the least (score, k) over the k
 * centres [k][dim]; out_score (optional) = that score. */
int gofann_build_assign(gofann_ctx* ctx, const void* rows, int elem, uint32_t dim, uint64_t n,
                        const float* centres, uint32_t k, uint32_t* out_idx, float* out_score);

/* k-means++ seeding (D^2 sampling) of k centres from the rows: the first
 * centre is row floor(u_0 n); centre j is the first row whose running sum
 * of best distances (fp64, rows ascending, in 1024 chunks whose sums are
 * added in order) reaches u_j times the total, where best is each row's
 * distance to its nearest chosen centre (lane-strided fmaf sums over 64
 * lanes, then an xor butterfly) and u_j the j-th uniform draw of SplitMix64
 * under `seed`.  Writes centres [k][dim]. */
int gofann_build_kmeanspp(gofann_ctx* ctx, const void* rows, int elem, uint32_t dim, uint64_t n,
                          uint32_t k, uint64_t seed, float* centres);

/* `iters` Lloyd iterations on centres [k][dim] in place: assign each row to
 * its nearest centre, then each centre becomes the mean of its rows (fp64
 * sums over its rows in ascending order, rounded to fp32); a centre with no
 * row keeps its value.  n < 2^31. */
int gofann_build_kmeans(gofann_ctx* ctx, const void* rows, int elem, uint32_t dim, uint64_t n,
                        uint32_t k, uint32_t iters, float* centres);

/* Rows sorted by bucket: bucket b holds rows [bucket_offsets[b],
 * bucket_offsets[b+1]) and bucket_offsets[buckets] == rows.  A row's
 * candidates are the rows of every bucket on its bucket's probe list
 * (probe_buckets[probe_offsets[b] .. probe_offsets[b+1]), no repeats), or of
 * its own bucket when probe_offsets is NULL. */
typedef struct {
    const uint32_t* bucket_offsets; /* [buckets + 1] */
    uint32_t buckets;
    uint32_t rows;
    const uint32_t* probe_offsets;  /* [buckets + 1] or NULL */
    const uint32_t* probe_buckets;
} gofann_build_buckets;

/* Exact k nearest candidates of every row (the row itself excluded), as
 * (distance, row) pairs ascending: out_ids [rows][k] rows of the sorted
 * space (UINT32_MAX past the candidates), out_dists [rows][k] (optional;
 * FLT_MAX past them).  k <= 128.  Replaces the kNN stage of the CAGRA build
 * (intermediate_graph_degree, graph_builder.cu:1293). */
int gofann_build_knn(gofann_ctx* ctx, const void* rows, int elem, uint32_t dim,
                     const gofann_build_buckets* buckets, uint32_t k, uint32_t* out_ids,
                     float* out_dists);

/* PQ codebook training: `iters` Lloyd iterations per subspace on
 * centroids [256][dim] in place (subspace m owns dims [m dim/pq_dim,
 * (m+1) dim/pq_dim)); codes by the rule of gofann_build_pq_encode, means as
 * gofann_build_kmeans.  Replaces pq::build (pq_builder.cu:92). */
int gofann_build_pq_train(gofann_ctx* ctx, const void* rows, int elem, uint32_t dim, uint64_t n,
                          uint32_t pq_dim, uint32_t iters, float* centroids);

/* PQ codes: codes[i * code_stride + m] = the least (sum_t (x - c)^2 over the
 * subspace's dims, fmaf ascending; centre index) over the 256 centres.
 * Replaces pq::transform (pq_builder.cu:129). */
int gofann_build_pq_encode(gofann_ctx* ctx, const void* rows, int elem, uint32_t dim, uint64_t n,
                           uint32_t pq_dim, const float* centroids, uint8_t* codes,
                           uint32_t code_stride);

/* Rotation of base rows for RaBitQ: out [n][padded_dim] = rows [n][dim]
 * (as f32) times rotation [dim][padded_dim] (FP32 SGEMM through rocBLAS, as
 * the query rotation).  The caller takes rows in chunks. */
int gofann_build_rotate(gofann_ctx* ctx, const void* rows, int elem, uint32_t dim, uint32_t n,
                        const float* rotation, uint32_t padded_dim, float* out);

/* One-bit RaBitQ encoding of rotated rows [n][padded_dim] against anchors
 * [num_anchors][padded_dim] (the rotated centres): anchor_ids = nearest
 * anchor (gofann_build_assign's rule); r = row - anchor; codes [n][P/8]
 * MSB-first u32 words (dim d is bit 31 - d % 32 of word d / 32, bit = r > 0);
 * factors [n][3] = f_add, f_rescale, f_err by the reference encoder's
 * formulas (quantizer_gpu_fast.cu:200-245), the sums over lanes d % 64
 * (fmaf) followed by an xor butterfly. */
int gofann_build_rabitq_encode(gofann_ctx* ctx, const float* rotated, uint32_t n,
                               uint32_t padded_dim, const float* anchors, uint32_t num_anchors,
                               uint32_t* anchor_ids, uint8_t* codes, float* factors);

/* The row nearest the rows' mean (the graph seed of a label group,
 * build_seed_local_ids_typed, dataloader.cpp:7361-7406): the mean in fp64
 * (sums over blocks of 4096 rows, rows ascending, blocks added in order,
 * divided by n), distances in fp64 (fma over d ascending), the least
 * (distance, row).  *out_row is a host pointer. */
int gofann_build_medoid(gofann_ctx* ctx, const void* rows, int elem, uint32_t dim, uint64_t n,
                        uint32_t* out_row);

/* Per bucket of bucket-sorted rows: means [buckets][dim] (fp64 sums over the
 * bucket's rows ascending, rounded to fp32) and reps [buckets], the row
 * nearest the mean (fp32 distance, least (distance, row); UINT32_MAX for an
 * empty bucket). */
int gofann_build_bucket_reps(gofann_ctx* ctx, const void* rows, int elem, uint32_t dim,
                             const uint32_t* bucket_offsets, uint32_t buckets, float* means,
                             uint32_t* reps);

/* This repo's graph (no counterpart in the reference, whose CAGRA graphs
 * it replaces): for row i of the bucket-sorted space, the candidate
 * sequence is
 *   ordinary row: knn[i][0 .. local), reps[bucket_of[i]], reps of
 *     near_buckets[b][0 .. near_links), then R draws;
 *   bucket representative: knn[i][0 .. rep_local), reps of
 *     near_buckets[b][0 .. rep_near), then R draws;
 *   entry_row: 4 R draws;
 * where draw j of row i is SplitMix64(seed, stream, i * 256 + j) mod rows
 * (streams 1, 2 and 3 for the three kinds).  The row keeps the first
 * `degree` distinct valid candidates other than itself; UINT32_MAX pads.
 * out_graph [rows][degree] is in the caller's row order: row order[i] of
 * out_graph holds order[candidate]. */
typedef struct {
    uint32_t rows;
    const uint32_t* knn;          /* [rows][knn_width] sorted-space rows */
    uint32_t knn_width;
    const uint32_t* bucket_of;    /* [rows] */
    const uint32_t* reps;         /* [buckets] */
    const uint32_t* near_buckets; /* [buckets][near_width] */
    uint32_t near_width;
    uint32_t buckets;
    const uint32_t* order;        /* [rows] caller row of each sorted row */
} gofann_build_link_inputs;
typedef struct {
    uint32_t degree;
    uint32_t local;
    uint32_t near_links;
    uint32_t rep_local;
    uint32_t rep_near;
    uint32_t entry_row;  /* sorted space; UINT32_MAX: none */
    uint64_t seed;
} gofann_build_link_params;
int gofann_build_links(gofann_ctx* ctx, const gofann_build_link_inputs* inputs,
                       const gofann_build_link_params* params, uint32_t* out_graph);

/* CAGRA's graph optimisation, written from the published method (Ootomo
 * et al., ICDE 2024, sec. IV-B) for the reference's graph_degree /
 * intermediate_graph_degree recipe (graph_builder.cu:1291-1293): knn
 * [n][kin] lists ascending by (distance, row); pruned [n][degree] = each
 * row's entries of least (detour count, rank), where the entry at rank j
 * counts a detour for every entry u at rank m whose own list holds it at
 * rank r with max(m, r) < j; out_graph [n][degree] = the first degree / 2
 * pruned edges, then reverse edges in order of (rank in the source's
 * pruned list, source row), then the remaining pruned edges, without
 * repeats (at most 2 degree reverse edges are considered).  n < 2^27,
 * degree <= kin <= 128. */
int gofann_build_cagra_optimize(gofann_ctx* ctx, const uint32_t* knn, uint32_t n, uint32_t kin,
                                uint32_t degree, uint32_t* pruned, uint32_t* out_graph);

/* Rows reachable from entry_row by the graph's edges: reached [n] u32 flags
 * (device), *reached_count (host) their number.  The connectivity check of
 * guarantee_connectivity (graph_builder.cu:1295). */
int gofann_build_reach(gofann_ctx* ctx, const uint32_t* graph, uint32_t n, uint32_t degree,
                       uint32_t entry_row, uint32_t* reached, uint32_t* reached_count);

#ifdef __cplusplus
}
#endif
#endif
