/*
 * gofann_oracle.c -- CPU restatement of GO-FANN's GPU filtered graph-search
 * hot path.  TEST INFRASTRUCTURE ONLY (see gofann_oracle.h).  Built with
 * -O2 -ffp-contract=off; every fused multiply-add is an explicit fmaf.
 */
#include "gofann_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ======================================================================
 * Visited hash -- src/search/common/native_visited_hash.cuh:10-60.
 * Open addressing with linear probing over 4096 u32 slots, empty slot =
 * UINT32_MAX; add drops the value silently when every slot is taken.
 * ====================================================================== */
uint32_t orc_hash_code(uint32_t value)
{
    /* native_visited_hash.cuh:13-18 */
    const uint64_t mixed = (uint64_t)value ^
                           ((uint64_t)(value >> 16) * 0x4bcb391f924ed183ULL) ^
                           0xa0ab69ccd854fc0aULL;
    return (uint32_t)(mixed % ORC_HASH_CAPACITY);
}

void orc_hash_clear(uint32_t* table)
{
    for (uint32_t i = 0; i < ORC_HASH_CAPACITY; ++i) table[i] = UINT32_MAX;
}

int orc_hash_test(const uint32_t* table, uint32_t value)
{
    /* native_visited_hash.cuh:28-41 */
    uint32_t slot = orc_hash_code(value);
    for (uint32_t probes = 0; probes < ORC_HASH_CAPACITY; ++probes) {
        if (table[slot] == UINT32_MAX) return 0;
        if (table[slot] == value) return 1;
        slot = (slot + 1) % ORC_HASH_CAPACITY;
    }
    return 0;
}

void orc_hash_add(uint32_t* table, uint32_t value)
{
    /* native_visited_hash.cuh:43-58 */
    uint32_t slot = orc_hash_code(value);
    for (uint32_t probes = 0; probes < ORC_HASH_CAPACITY; ++probes) {
        if (table[slot] == value) return;
        if (table[slot] == UINT32_MAX) {
            table[slot] = value;
            return;
        }
        slot = (slot + 1) % ORC_HASH_CAPACITY;
    }
}

/* ======================================================================
 * Symmetric min-max heap -- include/smmh2.h:1-147.  Slot 0 is the empty
 * root; slot 1 holds the minimum and slot 2 the maximum.  Entries compare
 * on `first` only (KernelPair operator<, warp_kernel.cuh:20-27; BiasedPair
 * gpu_predicate_index.cuh:137-144).
 * ====================================================================== */
static void pair_swap(orc_pair* a, orc_pair* b)
{
    orc_pair t = *a;
    *a = *b;
    *b = t;
}

static int smmh_adjust_sibling(orc_pair* h, int y, int size)
{
    /* smmh2.h:12-31 */
    if (y & 1) {
        const int s = y + 1;
        if (s >= size) return y;
        if (h[y].first > h[s].first) {
            pair_swap(&h[y], &h[s]);
            return s;
        }
    } else {
        const int s = y - 1;
        if (h[y].first < h[s].first) {
            pair_swap(&h[y], &h[s]);
            return s;
        }
    }
    return y;
}

static int smmh_adjust_grandparent(orc_pair* h, int y)
{
    /* smmh2.h:58-72 */
    if (y <= 2) return y;
    const int g = (y - 3) >> 2;
    const int gl = (g << 1) + 1;
    const int gr = (g << 1) + 2;
    if (h[gl].first > h[y].first) {
        pair_swap(&h[gl], &h[y]);
        return gl;
    } else if (h[gr].first < h[y].first) {
        pair_swap(&h[gr], &h[y]);
        return gr;
    }
    return y;
}

void orc_smmh2_insert(orc_pair* h, int* size, orc_pair entry)
{
    /* smmh2.h:76-89 */
    int y = *size;
    h[(*size)++] = entry;
    for (;;) {
        y = smmh_adjust_sibling(h, y, *size);
        const int x = smmh_adjust_grandparent(h, y);
        if (x == y) break;
        y = x;
    }
}

static int smmh_adjust_grandchild(orc_pair* h, int y, int size)
{
    /* smmh2.h:91-118 */
    if (y & 1) {
        if ((y << 1) + 1 >= size) return y; /* is_leaf */
        const int cl = (y << 1) + 1;
        const int cr = ((y + 1) << 1) + 1;
        int c = cl;
        if (cr < size && h[cr].first < h[cl].first) c = cr;
        if (h[c].first < h[y].first) {
            pair_swap(&h[c], &h[y]);
            return c;
        }
    } else {
        const int cl = ((y - 1) << 1) + 2;
        const int cr = (y << 1) + 2;
        if (cl >= size) return y;
        int c = cl;
        if (cr < size && h[cr].first > h[cl].first) c = cr;
        if (h[c].first > h[y].first) {
            pair_swap(&h[c], &h[y]);
            return c;
        }
    }
    return y;
}

static void smmh_deletion(orc_pair* h, int idx, int* size)
{
    /* smmh2.h:120-131: the sibling adjustment's return value is ignored. */
    h[idx] = h[--(*size)];
    int y = idx;
    for (;;) {
        (void)smmh_adjust_sibling(h, y, *size);
        const int x = smmh_adjust_grandchild(h, y, *size);
        if (x == y) break;
        y = x;
    }
}

orc_pair orc_smmh2_pop_min(orc_pair* h, int* size)
{
    orc_pair ret = h[1];
    smmh_deletion(h, 1, size);
    return ret;
}

orc_pair orc_smmh2_pop_max(orc_pair* h, int* size)
{
    orc_pair ret = h[2];
    smmh_deletion(h, 2, size);
    return ret;
}

int orc_pickup_unused(orc_pair* pool, int size, orc_pair* out)
{
    /* backend_pq.cu:824-842 (serial) == :844-892 (cooperative): the unused
     * entry of minimum `first`, lowest index on ties, is marked used. */
    int best = -1;
    for (int i = 1; i < size; ++i) {
        if (pool[i].second & ORC_POOL_USED) continue;
        if (best < 0 || pool[i].first < pool[best].first) best = i;
    }
    if (best < 0) return 0;
    *out = pool[best];
    pool[best].second |= ORC_POOL_USED;
    return 1;
}

/* Binary max-heap of bin_heap.h:4-64 over [begin, begin+size). */
#define ORC_DEFINE_BIN_HEAP(NAME, T)                                          \
    static void NAME##_push(T* begin, int size)                               \
    {                                                                         \
        int now = size - 1;                                                   \
        int parent = (now - 1) / 2;                                           \
        while (now > 0 && begin[parent].first < begin[now].first) {           \
            T tmp = begin[now];                                               \
            begin[now] = begin[parent];                                       \
            begin[parent] = tmp;                                              \
            now = parent;                                                     \
            parent = (now - 1) / 2;                                           \
        }                                                                     \
    }                                                                         \
    static T NAME##_pop(T* begin, int size)                                   \
    {                                                                         \
        T ret = begin[0];                                                     \
        const int len = size - 1;                                             \
        if (len <= 0) return ret;                                             \
        begin[0] = begin[size - 1];                                           \
        int now = 0;                                                          \
        while (now * 2 + 1 < len) {                                           \
            const int left = now * 2 + 1;                                     \
            const int right = now * 2 + 2;                                    \
            int next = left;                                                  \
            if (right < len && begin[left].first < begin[right].first)        \
                next = right;                                                 \
            if (!(begin[now].first < begin[next].first)) break;               \
            T tmp = begin[now];                                               \
            begin[now] = begin[next];                                         \
            begin[next] = tmp;                                                \
            now = next;                                                       \
        }                                                                     \
        return ret;                                                           \
    }

ORC_DEFINE_BIN_HEAP(stopheap, orc_stop_pair)
ORC_DEFINE_BIN_HEAP(resheap, orc_result_pair)

void orc_result_push(orc_result_pair* begin, int size_after_append)
{
    resheap_push(begin, size_after_append);
}

orc_result_pair orc_result_pop(orc_result_pair* begin, int size)
{
    return resheap_pop(begin, size);
}

/* ======================================================================
 * Posting shortlist heap -- src/search/common/posting_shortlist_heap.cuh.
 * A fixed-size max-heap of k (dist, id) pairs pre-filled with
 * (FLT_MAX, UINT32_MAX); worse = larger dist, then larger id.
 * ====================================================================== */
static int pair_is_worse(float ld, uint32_t lid, float rd, uint32_t rid)
{
    return ld > rd || (ld == rd && lid > rid); /* :15-21 */
}

static void shortlist_sift_down(float* d, uint32_t* ids, int heap_size, int root)
{
    /* :23-53 */
    for (;;) {
        const int left = root * 2 + 1;
        if (left >= heap_size) break;
        const int right = left + 1;
        int worse = left;
        if (right < heap_size && pair_is_worse(d[right], ids[right], d[left], ids[left]))
            worse = right;
        if (!pair_is_worse(d[worse], ids[worse], d[root], ids[root])) break;
        const float td = d[root];
        const uint32_t ti = ids[root];
        d[root] = d[worse];
        ids[root] = ids[worse];
        d[worse] = td;
        ids[worse] = ti;
        root = worse;
    }
}

int orc_shortlist_can_enter(float dist, uint32_t id, const float* d, const uint32_t* ids, int k)
{
    /* :57-65 */
    return id != UINT32_MAX && k > 0 && pair_is_worse(d[0], ids[0], dist, id);
}

void orc_shortlist_insert(float dist, uint32_t id, float* d, uint32_t* ids, int k)
{
    /* :67-80 */
    if (!orc_shortlist_can_enter(dist, id, d, ids, k)) return;
    d[0] = dist;
    ids[0] = id;
    shortlist_sift_down(d, ids, k, 0);
}

void orc_shortlist_sort(float* d, uint32_t* ids, int k)
{
    /* :82-99 */
    for (int heap_size = k; heap_size > 1; --heap_size) {
        const int tail = heap_size - 1;
        const float td = d[0];
        const uint32_t ti = ids[0];
        d[0] = d[tail];
        ids[0] = ids[tail];
        d[tail] = td;
        ids[tail] = ti;
        shortlist_sift_down(d, ids, tail, 0);
    }
}

/* ======================================================================
 * Early stop -- backend_pq.cu:2822-2873 (same in backend_rabitq.cu).
 * ====================================================================== */
int orc_adaptive_early_stop_limit(int queue_limit, int expanded, int passed, int stop_width)
{
    const int prior_pass = 8, prior_total = 16, max_extra = 32;
    const int queue_base = queue_limit > 1 ? queue_limit : 1;
    int base_limit = (queue_base * 1 + 2 - 1) / 2;
    const int min_base = stop_width > 0 ? stop_width * 2 : 1;
    base_limit = base_limit > min_base ? base_limit : min_base;
    const int denom = (expanded + prior_total) > 1 ? (expanded + prior_total) : 1;
    const int pass_with_prior = passed + prior_pass;
    const int pass_estimate = pass_with_prior < denom ? pass_with_prior : denom;
    const int reject_estimate = (denom - pass_estimate) > 0 ? (denom - pass_estimate) : 0;
    const int64_t numerator = (int64_t)queue_limit * 1 * reject_estimate;
    int extra = (int)((numerator + (2 * denom - 1)) / (2 * denom));
    extra = extra > 0 ? extra : 0;
    extra = extra < max_extra ? extra : max_extra;
    return base_limit + extra;
}

int orc_early_stop_reached(int mode, int bad, int fixed_limit, int queue_limit,
                           int expanded, int passed, int stop_width)
{
    if (mode == ORC_EARLY_STOP_OFF) return 0;
    if (mode == ORC_EARLY_STOP_ADAPTIVE)
        return bad >= orc_adaptive_early_stop_limit(queue_limit, expanded, passed, stop_width);
    return bad >= fixed_limit;
}

/* ======================================================================
 * Device predicates -- src/predicates/gpu_predicate_index.cuh:52-166 and
 * src/predicates/range_filter.cuh:23-124 (CSR storage, threshold 0).
 * ====================================================================== */
int orc_csr_contains(const uint32_t* labels, uint32_t begin, uint32_t end,
                     uint32_t handle, uint64_t* words_read)
{
    /* gpu_predicate_index.cuh:55-78, linear scan of a sorted row */
    for (uint32_t i = begin; i < end; ++i) {
        const uint32_t label = labels[i];
        if (words_read) ++*words_read;
        if (label >= handle) return label == handle;
    }
    return 0;
}

static int pred_contains(const orc_predicate* v, uint32_t handle, uint32_t sample,
                         orc_pred_counters* c)
{
    /* gpu_predicate_index.cuh:79-96 (CSR branch) */
    if (sample >= v->rows) return 0;
    if (v->csr_offsets == NULL) return 0;
    if (c) ++c->rows_checked;
    return orc_csr_contains(v->csr_labels, v->csr_offsets[sample], v->csr_offsets[sample + 1],
                            handle, c ? &c->label_words : NULL);
}

int orc_pred_enabled(const orc_predicate* v, uint32_t route)
{
    /* gpu_predicate_index.cuh:97-99 */
    if (v == NULL) return 0;
    return v->route_enabled ? v->route_enabled[route] != 0 : (v->csr_offsets != NULL);
}

int orc_range_matches(uint32_t mode, float lower, float upper, float value)
{
    /* gpu_predicate_index.cuh:100-108 == range_filter.cuh:28-45 */
    switch (mode) {
    case 0: return 1;
    case 1: return value > lower;
    case 2: return value < upper;
    case 3: return value >= lower && value < upper;
    default: return 0;
    }
}

int orc_pred_matches(const orc_predicate* v, uint32_t route, uint32_t sample,
                     orc_pred_counters* c)
{
    /* gpu_predicate_index.cuh:109-136 */
    if (sample >= v->rows) return 0;
    if (v->clauses) {
        for (uint32_t i = v->route_offsets[route]; i < v->route_offsets[route + 1]; ++i) {
            const orc_clause cl = v->clauses[i];
            int pass = 1;
            for (uint32_t j = cl.label_begin; pass && j < cl.label_end; ++j)
                pass = pred_contains(v, v->route_handles[j], sample, c);
            for (uint32_t j = cl.range_begin; pass && j < cl.range_end; ++j) {
                const orc_range_atom a = v->ranges[j];
                if (c) ++c->range_values;
                pass = v->base_ranges != NULL && a.dimension < v->range_stride &&
                       orc_range_matches(a.mode, a.lower, a.upper,
                                         v->base_ranges[(uint64_t)sample * v->range_stride +
                                                        a.dimension]);
            }
            if (pass) return 1;
        }
        return 0;
    }
    for (uint32_t i = v->route_offsets[route]; i < v->route_offsets[route + 1]; ++i)
        if (!pred_contains(v, v->route_handles[i], sample, c)) return 0;
    return 1;
}

float orc_priority(float base, float penalty, int pass, int* saturated)
{
    /* gpu_predicate_index.cuh:161-166 */
    if (pass || penalty == 0 || !isfinite(base) || base == FLT_MAX) return base;
    if (base > FLT_MAX - penalty) {
        if (saturated) *saturated = 1;
        return FLT_MAX;
    }
    return base + penalty;
}

float orc_minimum_pending_base(const orc_pair* pool, int size, orc_pair current,
                               orc_pair next, int current_valid, int next_valid)
{
    /* gpu_predicate_index.cuh:147-160 with the "unused" pending test of
     * backend_pq.cu:4273 */
    float minimum = FLT_MAX;
    if (current_valid) minimum = fminf(minimum, current.base);
    if (next_valid) minimum = fminf(minimum, next.base);
    for (int i = 1; i < size; ++i)
        if (!(pool[i].second & ORC_POOL_USED)) minimum = fminf(minimum, pool[i].base);
    return minimum;
}

float orc_bias_penalty(float alpha, float start_distance)
{
    /* backend_pq.cu:4190-4194 */
    const double wide = (double)alpha * fmax((double)fabsf(start_distance), 1e-6);
    return isfinite(wide) ? (float)fmin(wide, (double)FLT_MAX) : 0.0f;
}

uint32_t orc_count_active_ranges(const uint8_t* modes, uint32_t route, uint32_t count)
{
    /* range_filter.cuh:76-90 */
    if (modes == NULL) return 0;
    uint32_t active = 0;
    for (uint32_t r = 0; r < count; ++r)
        if (modes[(size_t)route * count + r] != 0) ++active;
    return active;
}

uint32_t orc_count_matching_ranges(const uint8_t* modes, const float* lower,
                                   const float* upper, const float* base_values,
                                   uint32_t route, uint32_t sample, uint32_t count)
{
    /* range_filter.cuh:47-74 */
    if (modes == NULL || lower == NULL || upper == NULL) return 0;
    uint32_t matched = 0;
    for (uint32_t r = 0; r < count; ++r) {
        const size_t qf = (size_t)route * count + r;
        const uint8_t mode = modes[qf];
        if (mode == 0) continue;
        if (base_values == NULL) return 0;
        if (orc_range_matches(mode, lower[qf], upper[qf], base_values[(size_t)sample * count + r]))
            ++matched;
    }
    return matched;
}

float orc_apply_filter_bonuses(float dist, int bit_match, uint32_t matched,
                               float bit_bonus, float range_bonus)
{
    /* range_filter.cuh:107-120 */
    if (bit_match) dist *= bit_bonus;
    for (uint32_t i = 0; i < matched; ++i) dist *= range_bonus;
    return dist;
}

/* ======================================================================
 * PQ -- backend_pq.cu:1999-2022 (LUT), 4164-4187 and 4711-4725 (ADC).
 * ====================================================================== */
void orc_pq_lut_u8(const float* centroids, const uint8_t* query, int dim, int pq_dim, float* lut)
{
    /* computePQTable: LUT[m][k] = sum_t (q - C[k])^2 accumulated in t order;
     * nvcc contracts `distance += diff * diff` into an FMA. */
    const int sub = dim / pq_dim;
    for (int m = 0; m < pq_dim; ++m) {
        for (int k = 0; k < 256; ++k) {
            float acc = 0.0f;
            for (int t = 0; t < sub; ++t) {
                const float diff = (float)query[m * sub + t] - centroids[(size_t)k * dim + m * sub + t];
                acc = fmaf(diff, diff, acc);
            }
            lut[m * 256 + k] = acc;
        }
    }
}

void orc_pq_lut_f32(const float* centroids, const float* query, int dim, int pq_dim, float* lut)
{
    /* Same table for fp32 queries (the reference instantiates u8 only). */
    const int sub = dim / pq_dim;
    for (int m = 0; m < pq_dim; ++m) {
        for (int k = 0; k < 256; ++k) {
            float acc = 0.0f;
            for (int t = 0; t < sub; ++t) {
                const float diff = query[m * sub + t] - centroids[(size_t)k * dim + m * sub + t];
                acc = fmaf(diff, diff, acc);
            }
            lut[m * 256 + k] = acc;
        }
    }
}

float orc_pq_adc(const float* lut, const uint8_t* code, int pq_dim)
{
    /* Lane j of a 32-lane warp sums subspaces m = j, j+32, ... in order,
     * then an xor butterfly over offsets 16, 8, 4, 2, 1 (backend_pq.cu:
     * 4716-4722).  Float addition commutes, so the butterfly equals this
     * fixed pairwise tree. */
    float s[32];
    for (int j = 0; j < 32; ++j) {
        float acc = 0.0f;
        for (int m = j; m < pq_dim; m += 32) acc += lut[m * 256 + code[m]];
        s[j] = acc;
    }
    for (int off = 16; off > 0; off >>= 1)
        for (int j = 0; j < off; ++j) s[j] = s[j] + s[j + off];
    return s[0];
}

static float pq_adc_serial(const float* lut, const uint8_t* code, int pq_dim)
{
    /* Posting scan order, backend_pq.cu:2102-2106: one thread, m ascending. */
    float dist = 0.0f;
    for (int m = 0; m < pq_dim; ++m) dist += lut[m * 256 + code[m]];
    return dist;
}

/* ======================================================================
 * RaBitQ -- backend_rabitq.cu:2898-2964 (query prep), 3070-3200 (score).
 * ====================================================================== */
static float block256_sum(const float* row, uint32_t n)
{
    /* 256-thread strided partial sums, then a shared-memory tree with
     * strides 128..1 (backend_rabitq.cu:2908-2922). */
    float partial[256];
    for (uint32_t t = 0; t < 256; ++t) {
        float acc = 0.0f;
        for (uint32_t d = t; d < n; d += 256) acc += row[d];
        partial[t] = acc;
    }
    for (uint32_t stride = 128; stride > 0; stride >>= 1)
        for (uint32_t t = 0; t < stride; ++t) partial[t] += partial[t + stride];
    return partial[0];
}

void orc_rabitq_query_factors(const float* rotated, uint32_t padded_dim, float* k1, float* kb)
{
    /* compute_rabitq_query_factors_kernel for bits_per_dim = 1 */
    const float sum = block256_sum(rotated, padded_dim);
    if (k1) *k1 = sum * -0.5f;
    if (kb) *kb = sum * (-(float)((1u << 1) - 1u) * 0.5f);
}

void orc_rabitq_quantize(const float* rotated, uint32_t padded_dim, int8_t* q8, float* scale)
{
    /* quantize_rabitq_queries_int8_kernel: scale = max|q|/127 (1 when the
     * query is zero), q8 = clamp(round-half-even(q / scale), -127, 127). */
    float max_abs = 0.0f;
    for (uint32_t d = 0; d < padded_dim; ++d) max_abs = fmaxf(max_abs, fabsf(rotated[d]));
    const float s = max_abs > 0.0f ? max_abs / 127.0f : 1.0f;
    for (uint32_t d = 0; d < padded_dim; ++d) {
        long v = lrintf(rotated[d] / s);
        if (v < -127) v = -127;
        if (v > 127) v = 127;
        q8[d] = (int8_t)v;
    }
    *scale = s;
}

int32_t orc_rabitq_ip_int(const int8_t* q8, const uint8_t* code, uint32_t padded_dim)
{
    /* Closed form of rabitq_dp4a_binary_dot_lane (backend_rabitq.cu:3070-3098):
     * sum_d q8[d] * bit[d]; bit d is bit (31 - d%32) of little-endian u32
     * word d/32 (MSB-first packing, quantizer_gpu_fast.cu:254-262). */
    int32_t acc = 0;
    for (uint32_t d = 0; d < padded_dim; ++d) {
        const uint32_t w = (uint32_t)code[(d / 32) * 4] | ((uint32_t)code[(d / 32) * 4 + 1] << 8) |
                           ((uint32_t)code[(d / 32) * 4 + 2] << 16) |
                           ((uint32_t)code[(d / 32) * 4 + 3] << 24);
        if ((w >> (31u - (d % 32u))) & 1u) acc += q8[d];
    }
    return acc;
}

static int32_t dp4a(int32_t a, int32_t b, int32_t c)
{
    for (int k = 0; k < 4; ++k)
        c += (int32_t)(int8_t)(a >> (8 * k)) * (int32_t)(int8_t)(b >> (8 * k));
    return c;
}

int32_t orc_rabitq_ip_popcount(const int8_t* q8, const uint8_t* code, uint32_t padded_dim)
{
    /* Bit-plane restatement: q8 = sum_j w_j * plane_j with w_j = 2^j (j<7)
     * and w_7 = -128 (two's complement), so sum_d q8[d]*bit[d] =
     * sum_j w_j * popcount(plane_j & code). */
    const uint32_t words = padded_dim / 32;
    int32_t total = 0;
    for (uint32_t w = 0; w < words; ++w) {
        const uint32_t cw = (uint32_t)code[w * 4] | ((uint32_t)code[w * 4 + 1] << 8) |
                            ((uint32_t)code[w * 4 + 2] << 16) | ((uint32_t)code[w * 4 + 3] << 24);
        for (int j = 0; j < 8; ++j) {
            uint32_t plane = 0;
            for (uint32_t b = 0; b < 32; ++b)
                if (((uint8_t)q8[w * 32 + b] >> j) & 1u) plane |= 1u << (31u - b);
            const int32_t cnt = __builtin_popcount(plane & cw);
            total += (j == 7) ? -128 * cnt : (1 << j) * cnt;
        }
    }
    return total;
}

int32_t orc_rabitq_ip_dp4a(const int8_t* q8, const uint8_t* code, uint32_t padded_dim)
{
    /* Literal restatement of the dp4a + nibble-mask path
     * (backend_rabitq.cu:204-209, 3070-3098): mask[p] has byte 3-i set to 1
     * iff bit i of nibble p is set; code bytes are read byte-reversed within
     * each u32 word. */
    int32_t mask[16];
    for (int p = 0; p < 16; ++p) {
        uint32_t m = 0;
        for (int i = 0; i < 4; ++i)
            if ((p >> i) & 1) m |= 1u << (8 * (3 - i));
        mask[p] = (int32_t)m;
    }
    int32_t partial = 0;
    for (uint32_t chunk = 0; chunk < padded_dim / 8; ++chunk) {
        const uint8_t pattern = code[(chunk >> 2) * 4 + (3 - (chunk & 3))];
        int32_t w0, w1;
        memcpy(&w0, q8 + chunk * 8, 4);
        memcpy(&w1, q8 + chunk * 8 + 4, 4);
        partial = dp4a(w0, mask[pattern >> 4], partial);
        partial = dp4a(w1, mask[pattern & 15], partial);
    }
    return partial;
}

float orc_rabitq_score_b1(int32_t ip_int, float scale, float k1, float f_add,
                          float f_rescale, float g_add)
{
    /* score_rabitq_code_device, ex_bits == 0 (backend_rabitq.cu:3176-3190):
     * f_add + g + f_rescale * (ip * scale + k1), the trailing product-sum
     * fused as nvcc contracts it. */
    const float short_ip = (float)ip_int * scale;
    const float t = short_ip + k1;
    return fmaf(f_rescale, t, f_add + g_add);
}

/* ======================================================================
 * Label-partitioned beam search -- backend_pq.cu:3980-5013 (device-resident
 * graph transport, :1516-1523 and :4642-4650), shared with
 * backend_rabitq.cu:3487-4291 (score and verdict differences flagged).
 * ====================================================================== */
static uint32_t float_bits(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static float bits_float(uint32_t u)
{
    float f;
    memcpy(&f, &u, 4);
    return f;
}

int orc_beam_search_route(const orc_graph* g, const orc_predicate* pred,
                          const orc_search_params* p, uint32_t route,
                          orc_scorer scorer, orc_exact exact, void* sctx, uint32_t* out_ids,
                          float* out_dists, orc_route_stats* st)
{
    const int Q = p->queue_limit;
    const int W = p->result_width;
    const int stop_width = p->stop_width;
    uint32_t* hash = (uint32_t*)malloc(ORC_HASH_CAPACITY * sizeof(uint32_t));
    orc_pair* frontier = (orc_pair*)malloc((size_t)(Q + 2) * sizeof(orc_pair));
    orc_result_pair* topk = (orc_result_pair*)malloc((size_t)(W + 1) * sizeof(orc_result_pair));
    orc_stop_pair stop[16];
    uint32_t list[ORC_FIXED_DEGREE];
    float dist_list[ORC_FIXED_DEGREE];
    uint8_t pass_list[ORC_FIXED_DEGREE];
    orc_pred_counters pc = {0, 0, 0};
    orc_route_stats local;
    memset(&local, 0, sizeof(local));
    if (!hash || !frontier || !topk || stop_width > 15) {
        free(hash);
        free(frontier);
        free(topk);
        return -1;
    }

    const uint32_t group = g->route_group[route];
    const uint32_t label_offset = g->label_offset[group];
    const uint64_t qfbit = g->query_filter_bits ? g->query_filter_bits[route] : ~0ULL;
    const uint32_t active_ranges = orc_count_active_ranges(g->range_modes, route, g->range_count);
    const uint32_t begin_id = g->route_start[route];
    const int enabled = orc_pred_enabled(pred, route);
    const int compiled = pred && pred->route_compiled && pred->route_compiled[route];
    const uint32_t degree = g->degree < ORC_FIXED_DEGREE ? g->degree : ORC_FIXED_DEGREE;

    orc_hash_clear(hash);
    /* Seed score (:4164-4187). */
    const uint32_t begin_sample = g->row_to_sample[label_offset + begin_id];
    const float start_distance = scorer(sctx, route, begin_sample);
    local.scored = 1;
    float penalty = 0.0f;
    if (p->bias) penalty = orc_bias_penalty(pred ? pred->alpha : 0.0f, start_distance);

    /* State init (:4195-4228). */
    int heap_size = 1;
    int stop_size = 0;
    float stop_worst = -FLT_MAX;
    int topk_size = 0;
    int finished = 0, exhausted = 0, expanded = 0, passed = 0;
    orc_pair now, next;
    const orc_pair sentinel = {FLT_MAX, UINT32_MAX, FLT_MAX};
    {
        orc_pair kp = {start_distance, begin_id, start_distance};
        orc_smmh2_insert(frontier, &heap_size, kp);
        orc_hash_add(hash, begin_id);
    }
    if (!orc_pickup_unused(frontier, heap_size, &now)) {
        exhausted = 1;
        now = sentinel;
    }
    next = sentinel;

    int step = 0;
    while (step == 0 || heap_size > 1) {
        const uint32_t now_local = now.second & ~ORC_POOL_USED;
        ++step;
        int list_len = 0;

        if (step != 1) {
            /* Pick up `next` before expanding `now` (:4266-4287). */
            const int found = orc_pickup_unused(frontier, heap_size, &next);
            if (!found) {
                exhausted = 1;
                next = sentinel;
            } else if (stop_size == stop_width) {
                float pending = next.first;
                if (pred && pred->pending_base_stop && enabled)
                    pending = orc_minimum_pending_base(frontier, heap_size, now, next, 1, found);
                if (p->early_stop_mode != ORC_EARLY_STOP_OFF && stop_worst <= pending) ++finished;
            }
        }

        /* Verdict of the expanded node (:4393-4441; RaBitQ :3855-3894).
         * When the pool is exhausted the loop breaks below before the
         * verdict is read, so it is not evaluated here. */
        int filt = 1;
        float rank = now.base;
        if (!exhausted) {
            const uint32_t global_row = label_offset + now_local;
            const uint32_t sample = g->row_to_sample[global_row];
            const uint64_t rmask = g->row_filter_mask ? g->row_filter_mask[global_row] : ~0ULL;
            const int bit_match = (rmask & qfbit) != 0;
            const uint32_t matched = orc_count_matching_ranges(
                g->range_modes, g->range_lower, g->range_upper, g->base_range_values, route,
                sample, g->range_count);
            const int exact_range = active_ranges == 0 || matched == active_ranges;
            if (enabled) filt = orc_pred_matches(pred, route, sample, &pc) ? 1 : 2;
            if (p->rabitq_verdict) {
                if (!compiled) filt = (filt == 1 && bit_match && exact_range) ? 1 : 2;
            } else if (!enabled && !compiled) {
                filt = (filt == 1 && bit_match && exact_range) ? 1 : 2;
            }
            /* Inline exact distance of a passing node (:4507-4546). */
            if (filt == 1 && p->inline_exact && exact) rank = exact(sctx, route, sample);
        }
        const float current_dist = now.base;

        if (exhausted ||
            orc_early_stop_reached(p->early_stop_mode, finished, p->finish_limit, Q, expanded,
                                   passed, stop_width) ||
            (p->max_steps > 0 && step >= p->max_steps))
            break;

        /* Result and stop heaps (:4558-4631). */
        ++expanded;
        if (filt == 1) {
            ++passed;
            /* ranked by the exact distance when inline rerank is on; the
             * stop payload keeps the approximate distance (:4566-4579) */
            orc_result_pair te = {rank, now_local};
            orc_stop_pair se = {rank,
                                ((uint64_t)float_bits(current_dist) << 32) | (uint64_t)now_local};
            int improved = 0;
            if (stop_size < stop_width) {
                stop[stop_size++] = se;
                stopheap_push(stop, stop_size);
                improved = 1;
                if (stop_size == 1 || current_dist > stop_worst) stop_worst = current_dist;
            } else if (se.first < stop[0].first) {
                stop[stop_size++] = se;
                stopheap_push(stop, stop_size);
                const orc_stop_pair removed = stopheap_pop(stop, stop_size);
                --stop_size;
                improved = 1;
                const uint32_t removed_bits = (uint32_t)(removed.second >> 32);
                if (current_dist > stop_worst) {
                    stop_worst = current_dist;
                } else if (removed_bits == float_bits(stop_worst)) {
                    stop_worst = -FLT_MAX;
                    for (int ii = 0; ii < stop_size; ++ii) {
                        const float d = bits_float((uint32_t)(stop[ii].second >> 32));
                        if (d > stop_worst) stop_worst = d;
                    }
                }
            }
            if (p->early_stop_mode == ORC_EARLY_STOP_ADAPTIVE && improved) finished = 0;
            if (topk_size < W) {
                topk[topk_size++] = te;
                resheap_push(topk, topk_size);
            } else if (te.first < topk[0].first) {
                topk[topk_size++] = te;
                resheap_push(topk, topk_size);
                (void)resheap_pop(topk, topk_size);
                --topk_size;
            }
        }

        /* Unvisited neighbours, in adjacency order (:4636-4684). */
        const uint32_t* row = g->graph + (size_t)(label_offset + now_local) * g->degree;
        for (uint32_t i = 0; i < degree; ++i) {
            const uint32_t idx = row[i];
            if (idx == UINT32_MAX) continue;
            if (orc_hash_test(hash, idx)) continue;
            list[list_len++] = idx;
        }

        if (orc_early_stop_reached(p->early_stop_mode, finished, p->finish_limit, Q, expanded,
                                   passed, stop_width) ||
            (p->max_steps > 0 && step >= p->max_steps))
            break;

        /* Score (:4704-4725) and predicate pass bits (:4738-4747). */
        for (int i = 0; i < list_len; ++i) {
            const uint32_t sample = g->row_to_sample[label_offset + list[i]];
            dist_list[i] = scorer(sctx, route, sample);
            pass_list[i] = 1;
            if (p->bias && enabled) pass_list[i] = (uint8_t)orc_pred_matches(pred, route, sample, &pc);
        }
        local.scored += list_len;

        /* Ordered frontier admission (:4826-4910). */
        for (int i = 0; i < list_len; ++i) {
            const uint32_t local_row = list[i];
            orc_pair kp;
            kp.first = dist_list[i];
            if (p->bit_filter_bonus != 1.0f || p->range_filter_bonus != 1.0f) {
                const uint32_t global_row = label_offset + local_row;
                const uint32_t sample = g->row_to_sample[global_row];
                const uint64_t rmask = g->row_filter_mask ? g->row_filter_mask[global_row] : ~0ULL;
                const uint32_t matched = orc_count_matching_ranges(
                    g->range_modes, g->range_lower, g->range_upper, g->base_range_values, route,
                    sample, g->range_count);
                kp.first = orc_apply_filter_bonuses(dist_list[i], (rmask & qfbit) != 0, matched,
                                                    p->bit_filter_bonus, p->range_filter_bonus);
            }
            kp.base = kp.first;
            if (p->bias && enabled) kp.first = orc_priority(kp.base, penalty, pass_list[i], NULL);
            kp.second = local_row;
            if (heap_size >= Q + 1 && frontier[2].first < kp.first) continue;
            orc_smmh2_insert(frontier, &heap_size, kp);
            orc_hash_add(hash, local_row);
            ++local.admitted;
            if (heap_size >= Q + 2) (void)orc_smmh2_pop_max(frontier, &heap_size);
        }

        if (step == 1) {
            if (!orc_pickup_unused(frontier, heap_size, &next)) {
                exhausted = 1;
                next = sentinel;
            }
        }
        now = next;
    }

    /* Sorted output (:4961-4982). */
    const int valid = topk_size < W ? topk_size : W;
    for (int i = 0; i < W; ++i) {
        out_ids[i] = UINT32_MAX;
        out_dists[i] = FLT_MAX;
    }
    for (int i = 0; i < valid; ++i) {
        const orc_result_pair res = resheap_pop(topk, topk_size - i);
        const int slot = valid - 1 - i;
        if (res.second == UINT32_MAX) continue;
        out_ids[slot] = g->row_to_sample[label_offset + res.second];
        out_dists[slot] = res.first;
    }
    local.steps = step;
    local.expanded = expanded;
    local.passed = passed;
    local.pred_rows = (int32_t)pc.rows_checked;
    local.pred_labels = (int32_t)pc.label_words;
    local.exhausted = exhausted;
    if (st) *st = local;
    free(hash);
    free(frontier);
    free(topk);
    return 0;
}

/* ---------------------------------------------------------------------- */
float orc_exact_inline_u8(const uint8_t* q, const uint8_t* b, uint32_t dim)
{
    /* backend_pq.cu:4507-4536: integer squares of (u8 - u8), added as float */
    float s[32];
    const uint32_t words = dim / 4;
    for (uint32_t j = 0; j < 32; ++j) {
        float acc = 0.0f;
        for (uint32_t w = j; w < words; w += 32)
            for (uint32_t t = 0; t < 4; ++t) {
                const int diff = (int)b[4 * w + t] - (int)q[4 * w + t];
                acc += (float)(diff * diff);
            }
        s[j] = acc;
    }
    for (int off = 16; off > 0; off >>= 1)
        for (int j = 0; j < off; ++j) s[j] = s[j] + s[j + off];
    return s[0];
}

float orc_exact_inline_f32(const float* q, const float* b, uint32_t dim)
{
    /* fp32 payload variant (backend_rabitq.cu:3936-3944 per element, fma) in
     * the same 32-lane word order */
    float s[32];
    const uint32_t words = dim / 4;
    for (uint32_t j = 0; j < 32; ++j) {
        float acc = 0.0f;
        for (uint32_t w = j; w < words; w += 32)
            for (uint32_t t = 0; t < 4; ++t) {
                const float diff = b[4 * w + t] - q[4 * w + t];
                acc = fmaf(diff, diff, acc);
            }
        s[j] = acc;
    }
    for (int off = 16; off > 0; off >>= 1)
        for (int j = 0; j < off; ++j) s[j] = s[j] + s[j + off];
    return s[0];
}

typedef struct {
    const uint8_t* codes;
    int pq_dim;
    const float* lut; /* current route's table */
    const void* base; /* exact vectors (inline rerank) */
    const void* query;
    int is_float;
    int dim;
} pq_ctx;

static float pq_score(void* ctx, uint32_t route, uint32_t sample)
{
    (void)route;
    const pq_ctx* c = (const pq_ctx*)ctx;
    return orc_pq_adc(c->lut, c->codes + (size_t)sample * c->pq_dim, c->pq_dim);
}

static float pq_exact(void* ctx, uint32_t route, uint32_t sample)
{
    (void)route;
    const pq_ctx* c = (const pq_ctx*)ctx;
    if (c->is_float)
        return orc_exact_inline_f32((const float*)c->query,
                                    (const float*)c->base + (size_t)sample * c->dim, c->dim);
    return orc_exact_inline_u8((const uint8_t*)c->query,
                               (const uint8_t*)c->base + (size_t)sample * c->dim, c->dim);
}

int orc_pq_search_batch(const orc_graph* g, const orc_predicate* pred,
                        const orc_search_params* p, const uint8_t* codes,
                        const float* centroids, const void* queries, int query_is_float,
                        const void* exact_base, const uint32_t* route_query, int dim,
                        int pq_dim, uint32_t routes, uint32_t* out_ids, float* out_dists,
                        orc_route_stats* stats)
{
    float* lut = (float*)malloc((size_t)pq_dim * 256 * sizeof(float));
    if (!lut) return -1;
    pq_ctx ctx = {codes, pq_dim, lut, exact_base, NULL, query_is_float, dim};
    for (uint32_t r = 0; r < routes; ++r) {
        const uint32_t q = route_query[r];
        if (query_is_float) {
            ctx.query = (const float*)queries + (size_t)q * dim;
            orc_pq_lut_f32(centroids, (const float*)queries + (size_t)q * dim, dim, pq_dim, lut);
        } else {
            ctx.query = (const uint8_t*)queries + (size_t)q * dim;
            orc_pq_lut_u8(centroids, (const uint8_t*)queries + (size_t)q * dim, dim, pq_dim, lut);
        }
        if (orc_beam_search_route(g, pred, p, r, pq_score, exact_base ? pq_exact : NULL, &ctx,
                                  out_ids + (size_t)r * p->result_width,
                                  out_dists + (size_t)r * p->result_width,
                                  stats ? stats + r : NULL) != 0) {
            free(lut);
            return -1;
        }
    }
    free(lut);
    return 0;
}

typedef struct {
    const uint8_t* codes;
    uint32_t code_bytes;
    const float* factors;
    const uint32_t* anchor_ids;
    const int8_t* q8;
    const float* q_scale;
    const float* q_k1;
    const float* centroid_dists;
    uint32_t num_anchors;
    uint32_t padded_dim;
    uint32_t query;
} rq_ctx;

static float rabitq_score(void* ctx, uint32_t route, uint32_t sample)
{
    (void)route;
    const rq_ctx* c = (const rq_ctx*)ctx;
    const int32_t ip = orc_rabitq_ip_int(c->q8 + (size_t)c->query * c->padded_dim,
                                         c->codes + (size_t)sample * c->code_bytes, c->padded_dim);
    const uint32_t anchor = c->anchor_ids[sample];
    return orc_rabitq_score_b1(ip, c->q_scale[c->query], c->q_k1[c->query],
                               c->factors[(size_t)sample * 3], c->factors[(size_t)sample * 3 + 1],
                               c->centroid_dists[(size_t)c->query * c->num_anchors + anchor]);
}

int orc_rabitq_search_batch(const orc_graph* g, const orc_predicate* pred,
                            const orc_search_params* p, const uint8_t* codes,
                            uint32_t code_bytes, const float* factors,
                            const uint32_t* anchor_ids, const int8_t* q8, const float* q_scale,
                            const float* q_k1, const float* centroid_dists, uint32_t num_anchors,
                            uint32_t padded_dim, const uint32_t* route_query, uint32_t routes,
                            uint32_t* out_ids, float* out_dists, orc_route_stats* stats)
{
    rq_ctx ctx = {codes, code_bytes, factors, anchor_ids, q8, q_scale, q_k1,
                  centroid_dists, num_anchors, padded_dim, 0};
    for (uint32_t r = 0; r < routes; ++r) {
        ctx.query = route_query[r];
        if (orc_beam_search_route(g, pred, p, r, rabitq_score, NULL, &ctx,
                                  out_ids + (size_t)r * p->result_width,
                                  out_dists + (size_t)r * p->result_width,
                                  stats ? stats + r : NULL) != 0)
            return -1;
    }
    return 0;
}

/* ======================================================================
 * Full-GPU exact route -- backend_full_gpu.cu:1682-2042.
 * ====================================================================== */
uint32_t orc_l2_u8_int(const uint8_t* a, const uint8_t* b, uint32_t dim)
{
    /* :1235-1243: integer squared differences (the dp4a form :1209-1232,
     * |b|^2 + |q|^2 - 2 b.q in u32, is the same integer) */
    uint32_t acc = 0;
    for (uint32_t d = 0; d < dim; ++d) {
        const int diff = (int)a[d] - (int)b[d];
        acc += (uint32_t)(diff * diff);
    }
    return acc;
}

static int better_result(float ld, uint32_t lid, float rd, uint32_t rid)
{
    return ld < rd || (ld == rd && lid < rid); /* :1337-1340 */
}

int orc_insert_best(float dist, uint32_t id, uint32_t topk, float* bd, uint32_t* bi,
                    uint32_t* size)
{
    /* :1342-1375 */
    int changed = 0;
    for (uint32_t i = 0; i < *size; ++i) {
        if (bi[i] != id) continue;
        if (dist >= bd[i]) return 0;
        for (uint32_t j = i; j + 1 < *size; ++j) {
            bd[j] = bd[j + 1];
            bi[j] = bi[j + 1];
        }
        --*size;
        changed = 1;
        break;
    }
    if (*size == topk && !better_result(dist, id, bd[topk - 1], bi[topk - 1])) return changed;
    uint32_t pos = *size;
    if (*size < topk)
        ++*size;
    else
        pos = topk - 1;
    while (pos > 0 && better_result(dist, id, bd[pos - 1], bi[pos - 1])) {
        bd[pos] = bd[pos - 1];
        bi[pos] = bi[pos - 1];
        --pos;
    }
    bd[pos] = dist;
    bi[pos] = id;
    return 1;
}

/* Squared L2 in the order of the reference's cooperative warp distance
 * (l2_distance_device, backend_full_gpu.cu:1107-1160): 32 partial sums,
 * partial j a fused multiply-add chain over the elements j, j + 32, ...
 * (f16 rows of even dim: over the element pairs j, j + 32, ..., each pair
 * adding fma(dx, dx, dy * dy) -- the reference writes dx*dx + dy*dy and
 * leaves its contraction to nvcc, so this grouping is the one restated
 * here), then the shfl_down halving tree: p[j] += p[j + 16] for j < 16,
 * then + 8, + 4, + 2, + 1; the result is p[0].  diff = base - query.  u8
 * rows: the integer sum (the dp4a form :1199-1244), exact in any order.
 * row and q have element type elem (0 u8, 1 f32, 2 f16 as uint16 bits). */
static float elem_at(const void* v, int elem, uint32_t i)
{
    if (elem == 1) return ((const float*)v)[i];
    if (elem == 2) return orc_half_to_float(((const uint16_t*)v)[i]);
    return (float)((const uint8_t*)v)[i];
}

float orc_l2_w32(const void* row, const void* q, int elem, uint32_t dim)
{
    if (elem == 0) return (float)orc_l2_u8_int((const uint8_t*)row, (const uint8_t*)q, dim);
    float p[32];
    for (uint32_t j = 0; j < 32; ++j) {
        float acc = 0.0f;
        if (elem == 2 && (dim & 1u) == 0) {
            for (uint32_t d2 = j; d2 < dim / 2; d2 += 32) {
                const float dx = elem_at(row, 2, 2 * d2) - elem_at(q, 2, 2 * d2);
                const float dy = elem_at(row, 2, 2 * d2 + 1) - elem_at(q, 2, 2 * d2 + 1);
                acc = acc + fmaf(dx, dx, dy * dy);
            }
        } else {
            for (uint32_t d = j; d < dim; d += 32) {
                const float diff = elem_at(row, elem, d) - elem_at(q, elem, d);
                acc = fmaf(diff, diff, acc);
            }
        }
        p[j] = acc;
    }
    for (uint32_t off = 16; off > 0; off >>= 1)
        for (uint32_t j = 0; j < off; ++j) p[j] = p[j] + p[j + off];
    return p[0];
}

/* Squared L2 in the order of the reference's range-posting scan
 * (full_gpu_range_posting_kernel, backend_full_gpu.cu:1443-1469): one
 * fused multiply-add chain over d ascending (f16 rows of even dim: over
 * the pairs, dist + fma(dx, dx, dy * dy) as above); u8 elements are
 * converted to float first (T = uint8_t there), which equals the integer
 * sum while every partial sum stays below 2^24 (dim <= 258). */
float orc_l2_serial(const void* row, const void* q, int elem, uint32_t dim)
{
    float acc = 0.0f;
    if (elem == 2 && (dim & 1u) == 0) {
        for (uint32_t d2 = 0; d2 < dim / 2; ++d2) {
            const float dx = elem_at(row, 2, 2 * d2) - elem_at(q, 2, 2 * d2);
            const float dy = elem_at(row, 2, 2 * d2 + 1) - elem_at(q, 2, 2 * d2 + 1);
            acc = acc + fmaf(dx, dx, dy * dy);
        }
        return acc;
    }
    for (uint32_t d = 0; d < dim; ++d) {
        const float diff = elem_at(row, elem, d) - elem_at(q, elem, d);
        acc = fmaf(diff, diff, acc);
    }
    return acc;
}

static size_t elem_size(int elem) { return elem == 1 ? 4u : (elem == 2 ? 2u : 1u); }

int orc_exact_search(const orc_graph* g, const uint32_t* label_size, const orc_predicate* pred,
                     const orc_exact_params* p, const void* base, int elem, uint32_t dim,
                     uint32_t samples, const void* queries, const uint32_t* route_query,
                     uint32_t routes, uint32_t* out_ids, float* out_dists,
                     orc_route_stats* stats)
{
    if (elem < 0 || elem > 2) return -1;
    const size_t es = elem_size(elem);
    const int Q = p->queue_limit;
    const uint32_t K = (uint32_t)p->topk;
    if (Q < 2 || K == 0 || K > 10) return -1;
    uint32_t* hash = (uint32_t*)malloc(ORC_HASH_CAPACITY * sizeof(uint32_t));
    orc_pair* pool = (orc_pair*)malloc((size_t)(Q + 2) * sizeof(orc_pair));
    if (!hash || !pool) {
        free(hash);
        free(pool);
        return -1;
    }
    const uint32_t degree = g->degree < ORC_FIXED_DEGREE ? g->degree : ORC_FIXED_DEGREE;
    for (uint32_t r = 0; r < routes; ++r) {
        orc_route_stats st;
        memset(&st, 0, sizeof(st));
        float bd[10];
        uint32_t bi[10];
        uint32_t bsize = 0;
        for (int i = 0; i < 10; ++i) {
            bd[i] = FLT_MAX;
            bi[i] = UINT32_MAX;
        }
        orc_pred_counters pc = {0, 0, 0};
        const uint32_t group = g->route_group[r];
        const uint32_t seed = g->route_start[r];
        const uint32_t gsize = label_size ? label_size[group] : UINT32_MAX;
        const void* q = (const char*)queries + (size_t)route_query[r] * dim * es;
        const uint32_t off = g->label_offset[group];
        const uint64_t qfbit = g->query_filter_bits ? g->query_filter_bits[r] : ~0ULL;
        const uint32_t active = orc_count_active_ranges(g->range_modes, r, g->range_count);
        const int enabled = orc_pred_enabled(pred, r);
        int heap_size = 1;
        int done = 0;
        orc_pair now, next;
        /* :1793-1850: the seed (visited is empty, so it is always fresh) */
        if (gsize == 0 || seed == UINT32_MAX || seed >= gsize) {
            done = 1;
        } else {
            orc_hash_clear(hash);
            const uint32_t s0 = g->row_to_sample[off + seed];
            if (s0 < samples && !orc_hash_test(hash, seed)) {
                const float d0 = orc_l2_w32((const char*)base + (size_t)s0 * dim * es, q, elem, dim);
                ++st.scored;
                orc_pair kp = {d0, seed, d0};
                orc_smmh2_insert(pool, &heap_size, kp);
                if (heap_size >= Q + 2) orc_smmh2_pop_max(pool, &heap_size);
                orc_hash_add(hash, seed);
            } else {
                done = 1;
            }
        }
        if (!done && !orc_pickup_unused(pool, heap_size, &now)) done = 1;
        if (done) st.exhausted = 1;
        uint32_t steps = 0, finished = 0;
        int first_step = 1;
        while (!done) {
            if (p->max_steps != 0 && steps >= (uint32_t)p->max_steps) break; /* :1878-1883 */
            /* :1885-1918: the expanded node's filter and best-k */
            const uint32_t cur = now.second & ~ORC_POOL_USED;
            const uint32_t grow = off + cur;
            const uint32_t sample = g->row_to_sample[grow];
            const uint64_t rmask = g->row_filter_mask ? g->row_filter_mask[grow] : ~0ULL;
            int pass = (rmask & qfbit) != 0;
            if (pass && active != 0)
                pass = orc_count_matching_ranges(g->range_modes, g->range_lower, g->range_upper,
                                                 g->base_range_values, r, sample,
                                                 g->range_count) == active;
            if (pass && enabled) pass = orc_pred_matches(pred, r, sample, &pc);
            ++st.expanded;
            int improved = 0;
            if (pass) {
                ++st.passed;
                improved = orc_insert_best(now.first, sample, K, bd, bi, &bsize);
            }
            ++steps;
            /* :1920-1958: neighbours, then ordered admission :1962-1981 */
            uint32_t cl[ORC_FIXED_DEGREE];
            float cd[ORC_FIXED_DEGREE];
            int nc = 0;
            for (uint32_t e = 0; e < degree; ++e) {
                const uint32_t local = g->graph[(size_t)grow * g->degree + e];
                if (local == UINT32_MAX || local >= gsize || orc_hash_test(hash, local)) continue;
                const uint32_t s = g->row_to_sample[off + local];
                if (s >= samples) continue;
                cl[nc] = local;
                cd[nc] = orc_l2_w32((const char*)base + (size_t)s * dim * es, q, elem, dim);
                ++nc;
            }
            st.scored += nc;
            for (int i = 0; i < nc; ++i) {
                orc_pair kp = {cd[i], cl[i], cd[i]};
                if (heap_size > 2 && heap_size >= Q + 1 && pool[2].first < kp.first) continue;
                orc_smmh2_insert(pool, &heap_size, kp);
                ++st.admitted;
                orc_hash_add(hash, cl[i]);
                if (heap_size >= Q + 2) orc_smmh2_pop_max(pool, &heap_size);
            }
            /* :1985-2030: pickup and early stop */
            if (!orc_pickup_unused(pool, heap_size, &next)) {
                st.exhausted = 1;
                break;
            }
            if (!first_step) {
                const uint32_t ns = g->row_to_sample[off + (next.second & ~ORC_POOL_USED)];
                if (p->early_stop_mode == ORC_EARLY_STOP_ADAPTIVE && improved) {
                    finished = 0;
                } else if (bsize == K && !better_result(next.first, ns, bd[K - 1], bi[K - 1])) {
                    ++finished;
                    if (orc_early_stop_reached(p->early_stop_mode, (int)finished, p->finish_limit,
                                               Q, st.expanded, st.passed, (int)K))
                        break;
                } else {
                    finished = 0;
                }
            }
            now = next;
            first_step = 0;
        }
        st.steps = (int32_t)steps;
        st.pred_rows = (int32_t)pc.rows_checked;
        st.pred_labels = (int32_t)pc.label_words;
        for (uint32_t i = 0; i < K; ++i) {
            out_ids[(size_t)r * K + i] = i < bsize ? bi[i] : UINT32_MAX;
            out_dists[(size_t)r * K + i] = i < bsize ? bd[i] : FLT_MAX;
        }
        if (stats) stats[r] = st;
    }
    free(hash);
    free(pool);
    return 0;
}

/* Exact posting scan: the full-GPU backend's posting routes
 * (full_gpu_range_posting_kernel, backend_full_gpu.cu:1383-1493, order
 * ORC_EXACT_ORDER_SERIAL; full_gpu_lowfreq_kernel :2124-2262, the warp
 * order ORC_EXACT_ORDER_W32).  Per route: every listed sample s (skipped:
 * UINT32_MAX, s >= samples, the route predicate fails when enabled) is
 * scored by exact squared L2 and enters the best-topk with sample dedup
 * (insert_best_result :1333-1375), so the output is the topk least
 * (distance, id) pairs over the distinct samples, ascending, padded
 * (FLT_MAX, UINT32_MAX).  A NaN distance (only from NaN or infinite
 * inputs) is skipped: the reference's insertion of one depends on which
 * thread met it first.  pass_counts: predicate passes (all listed valid
 * samples when the predicate is off). */
int orc_exact_posting_scan(const orc_predicate* pred, const void* base, int elem,
                           uint32_t dim, uint32_t samples, const void* queries,
                           const uint32_t* route_query, const uint32_t* cand_ids,
                           const uint32_t* cand_offsets, const uint32_t* cand_sizes,
                           uint32_t routes, int topk, int order, uint32_t* out_ids,
                           float* out_dists, uint32_t* pass_counts)
{
    if (elem < 0 || elem > 2 || topk < 1 || topk > ORC_EXACT_SCAN_MAX_TOPK) return -1;
    const size_t es = elem_size(elem);
    const uint32_t K = (uint32_t)topk;
    float* bd = (float*)malloc(K * sizeof(float));
    uint32_t* bi = (uint32_t*)malloc(K * sizeof(uint32_t));
    if (!bd || !bi) {
        free(bd);
        free(bi);
        return -1;
    }
    for (uint32_t r = 0; r < routes; ++r) {
        const void* q = (const char*)queries + (size_t)route_query[r] * dim * es;
        const int enabled = orc_pred_enabled(pred, r);
        orc_pred_counters pc = {0, 0, 0};
        uint32_t bsize = 0, passes = 0;
        for (uint32_t i = 0; i < K; ++i) {
            bd[i] = FLT_MAX;
            bi[i] = UINT32_MAX;
        }
        for (uint32_t j = 0; j < cand_sizes[r]; ++j) {
            const uint32_t s = cand_ids[cand_offsets[r] + j];
            if (s == UINT32_MAX || s >= samples) continue;
            if (enabled && !orc_pred_matches(pred, r, s, &pc)) continue;
            ++passes;
            const void* row = (const char*)base + (size_t)s * dim * es;
            const float d = order == ORC_EXACT_ORDER_W32 ? orc_l2_w32(row, q, elem, dim)
                                                         : orc_l2_serial(row, q, elem, dim);
            if (d != d) continue;
            orc_insert_best(d, s, K, bd, bi, &bsize);
        }
        for (uint32_t i = 0; i < K; ++i) {
            out_ids[(size_t)r * K + i] = i < bsize ? bi[i] : UINT32_MAX;
            out_dists[(size_t)r * K + i] = i < bsize ? bd[i] : FLT_MAX;
        }
        if (pass_counts) pass_counts[r] = passes;
    }
    free(bd);
    free(bi);
    return 0;
}

/* ======================================================================
 * Posting scans -- backend_pq.cu:2046-2133 (PQ, serial ADC order) and
 * backend_rabitq.cu:5494-5682 (RaBitQ).
 * ====================================================================== */
int orc_pq_posting_scan(const orc_predicate* pred, const uint8_t* codes,
                        const float* centroids, const void* queries, int query_is_float,
                        const uint32_t* route_query, const uint32_t* cand_ids,
                        const uint32_t* cand_offsets, const uint32_t* cand_sizes,
                        uint32_t routes, int dim, int pq_dim, int shortlist_k,
                        int score_first, uint32_t* out_ids, float* out_dists,
                        uint32_t* pass_counts)
{
    float* lut = (float*)malloc((size_t)pq_dim * 256 * sizeof(float));
    if (!lut) return -1;
    for (uint32_t r = 0; r < routes; ++r) {
        float* bd = out_dists + (size_t)r * shortlist_k;
        uint32_t* bi = out_ids + (size_t)r * shortlist_k;
        for (int i = 0; i < shortlist_k; ++i) {
            bd[i] = FLT_MAX;
            bi[i] = UINT32_MAX;
        }
        const uint32_t q = route_query[r];
        if (query_is_float)
            orc_pq_lut_f32(centroids, (const float*)queries + (size_t)q * dim, dim, pq_dim, lut);
        else
            orc_pq_lut_u8(centroids, (const uint8_t*)queries + (size_t)q * dim, dim, pq_dim, lut);
        const int enabled = orc_pred_enabled(pred, r);
        uint32_t passes = 0;
        for (uint32_t i = 0; i < cand_sizes[r]; ++i) {
            const uint32_t s = cand_ids[cand_offsets[r] + i];
            if (s == UINT32_MAX) continue;
            if (!score_first && enabled) {
                if (!orc_pred_matches(pred, r, s, NULL)) continue;
                ++passes;
            }
            const float d = pq_adc_serial(lut, codes + (size_t)s * pq_dim, pq_dim);
            if (score_first) {
                if (!orc_shortlist_can_enter(d, s, bd, bi, shortlist_k)) continue;
                if (enabled && !orc_pred_matches(pred, r, s, NULL)) continue;
            }
            orc_shortlist_insert(d, s, bd, bi, shortlist_k);
        }
        orc_shortlist_sort(bd, bi, shortlist_k);
        if (pass_counts) pass_counts[r] = passes;
    }
    free(lut);
    return 0;
}

int orc_rabitq_posting_scan(const orc_predicate* pred, const uint8_t* codes,
                            uint32_t code_bytes, const float* factors,
                            const uint32_t* anchor_ids, const int8_t* q8, const float* q_scale,
                            const float* q_k1, const float* centroid_dists,
                            uint32_t num_anchors, uint32_t padded_dim,
                            const uint32_t* route_query, const uint32_t* cand_ids,
                            const uint32_t* cand_offsets, const uint32_t* cand_sizes,
                            uint32_t routes, int shortlist_k, uint32_t* out_ids,
                            float* out_dists, uint32_t* pass_counts)
{
    rq_ctx ctx = {codes, code_bytes, factors, anchor_ids, q8, q_scale, q_k1,
                  centroid_dists, num_anchors, padded_dim, 0};
    const uint32_t rows = pred ? pred->rows : UINT32_MAX;
    for (uint32_t r = 0; r < routes; ++r) {
        float* bd = out_dists + (size_t)r * shortlist_k;
        uint32_t* bi = out_ids + (size_t)r * shortlist_k;
        for (int i = 0; i < shortlist_k; ++i) {
            bd[i] = FLT_MAX;
            bi[i] = UINT32_MAX;
        }
        ctx.query = route_query[r];
        const int enabled = orc_pred_enabled(pred, r);
        uint32_t passes = 0;
        for (uint32_t i = 0; i < cand_sizes[r]; ++i) {
            const uint32_t s = cand_ids[cand_offsets[r] + i];
            if (s >= rows) continue;
            if (enabled) {
                if (!orc_pred_matches(pred, r, s, NULL)) continue;
                ++passes;
            }
            const float d = rabitq_score(&ctx, r, s);
            orc_shortlist_insert(d, s, bd, bi, shortlist_k);
        }
        orc_shortlist_sort(bd, bi, shortlist_k);
        if (pass_counts) pass_counts[r] = passes;
    }
    return 0;
}

/* ======================================================================
 * Range postings -- segment plan (posting_segment_plan.h:20-51), range
 * scan (backend_rabitq.cu:5846-6015) and segment merge
 * (posting_segment_merge.cuh:12-46).
 * ====================================================================== */
int orc_segment_plan(const uint32_t* route_ids, const uint64_t* offsets, const uint64_t* sizes,
                     uint32_t n, uint32_t target_rows, uint32_t capacity, uint32_t* seg_routes,
                     uint32_t* seg_positions, uint64_t* seg_offsets, uint64_t* seg_sizes,
                     uint32_t* query_indptr, uint32_t* out_count)
{
    if (target_rows == 0 || (n > 0 && (!route_ids || !offsets || !sizes))) return -1;
    /* :30-38: an empty posting still yields one (empty) segment */
    uint64_t total = 0;
    for (uint32_t q = 0; q < n; ++q) {
        if (offsets[q] > UINT64_MAX - sizes[q]) return -2;
        const uint64_t count = sizes[q] == 0 ? 1 : 1 + (sizes[q] - 1) / target_rows;
        if (count > (uint64_t)UINT32_MAX - total) return -2;
        total += count;
    }
    if (out_count) *out_count = (uint32_t)total;
    if (capacity < total || !seg_routes || !seg_positions || !seg_offsets || !seg_sizes ||
        !query_indptr)
        return 1;
    uint32_t s = 0;
    query_indptr[0] = 0;
    for (uint32_t q = 0; q < n; ++q) {
        const uint64_t rows = sizes[q];
        const uint64_t count = rows == 0 ? 1 : 1 + (rows - 1) / target_rows;
        /* :39-49: near-equal parts, the first `rows % count` one row longer */
        const uint64_t width = rows / count, extra = rows % count;
        for (uint64_t part = 0; part < count; ++part, ++s) {
            seg_routes[s] = route_ids[q];
            seg_positions[s] = q;
            seg_offsets[s] = offsets[q] + part * width + (part < extra ? part : extra);
            seg_sizes[s] = width + (part < extra ? 1 : 0);
        }
        query_indptr[q + 1] = s;
    }
    return 0;
}

int orc_rabitq_range_scan(const orc_predicate* pred, const orc_range_table* rt,
                          const uint8_t* codes, uint32_t code_bytes, const float* factors,
                          const uint32_t* anchor_ids, const int8_t* q8, const float* q_scale,
                          const float* q_k1, const float* centroid_dists, uint32_t num_anchors,
                          uint32_t padded_dim, const uint32_t* route_query,
                          const uint32_t* posting, uint64_t resident_rows, uint32_t base_rows,
                          const uint32_t* seg_routes, const uint64_t* seg_offsets,
                          const uint64_t* seg_sizes, uint32_t segments, int shortlist_k,
                          int score_first, uint32_t* out_ids, float* out_dists,
                          uint32_t* pass_counts)
{
    rq_ctx ctx = {codes, code_bytes, factors, anchor_ids, q8, q_scale, q_k1,
                  centroid_dists, num_anchors, padded_dim, 0};
    for (uint32_t sg = 0; sg < segments; ++sg) {
        float* bd = out_dists + (size_t)sg * shortlist_k;
        uint32_t* bi = out_ids + (size_t)sg * shortlist_k;
        for (int i = 0; i < shortlist_k; ++i) {
            bd[i] = FLT_MAX;
            bi[i] = UINT32_MAX;
        }
        const uint32_t route = seg_routes[sg];
        ctx.query = route_query[route];
        /* :5895-5902 clip to the resident rows */
        const uint64_t begin = seg_offsets[sg];
        uint64_t count = seg_sizes[sg];
        if (begin > resident_rows)
            count = 0;
        else if (count > resident_rows - begin)
            count = resident_rows - begin;
        /* :5903-5913 */
        const uint32_t active =
            rt ? orc_count_active_ranges(rt->modes, route, rt->count) : 0;
        const int enabled = orc_pred_enabled(pred, route);
        const int sf = score_first && enabled;
        uint32_t passes = 0;
        for (uint64_t i = 0; i < count; ++i) {
            const uint32_t s = posting[begin + i];
            if (s >= base_rows || active == 0) continue;                    /* :5917 */
            if (!sf && enabled) {                                            /* :5921-5923 */
                if (!orc_pred_matches(pred, route, s, NULL)) continue;
            } else if (!sf && active > 1) {                                  /* :5924-5934 */
                if (orc_count_matching_ranges(rt->modes, rt->lower, rt->upper, rt->base_values,
                                              route, s, rt->count) != active)
                    continue;
            }
            const float d = rabitq_score(&ctx, route, s);
            if (sf) {                                                        /* :5960-5970 */
                if (!orc_shortlist_can_enter(d, s, bd, bi, shortlist_k)) continue;
                if (!orc_pred_matches(pred, route, s, NULL)) continue;
            }
            ++passes;                                                        /* :5971-5975 */
            orc_shortlist_insert(d, s, bd, bi, shortlist_k);
        }
        orc_shortlist_sort(bd, bi, shortlist_k);
        if (pass_counts) pass_counts[sg] = passes;
    }
    return 0;
}

int orc_merge_segments(const uint32_t* query_indptr, uint32_t positions,
                       const uint32_t* seg_ids, const float* seg_dists,
                       const uint32_t* seg_pass, int shortlist_k, uint32_t* out_ids,
                       float* out_dists, uint32_t* out_pass)
{
    for (uint32_t p = 0; p < positions; ++p) {
        float* bd = out_dists + (size_t)p * shortlist_k;
        uint32_t* bi = out_ids + (size_t)p * shortlist_k;
        for (int i = 0; i < shortlist_k; ++i) {
            bd[i] = FLT_MAX;
            bi[i] = UINT32_MAX;
        }
        uint32_t passes = 0;
        for (uint32_t part = query_indptr[p]; part < query_indptr[p + 1]; ++part) {
            passes += seg_pass[part];
            const size_t o = (size_t)part * shortlist_k;
            for (int i = 0; i < shortlist_k; ++i)
                orc_shortlist_insert(seg_dists[o + i], seg_ids[o + i], bd, bi, shortlist_k);
        }
        orc_shortlist_sort(bd, bi, shortlist_k);
        if (out_pass) out_pass[p] = passes;
    }
    return 0;
}

/* ======================================================================
 * Resident posting producer -- src/search/pq/pq_resident_posting.cuh:27-58:
 * a route's posting slice is its group's [offset, offset + size) when it
 * fits the table; a row yields its sample only when the row mask shares a
 * bit with the route mask, the sample is in range and every active range
 * atom of the route matches.
 * ====================================================================== */
int orc_resident_bounds(const uint32_t* group_offsets, const uint32_t* group_sizes,
                        const uint32_t* query_groups, uint32_t groups, uint32_t rows,
                        uint32_t routes, uint32_t route, uint32_t* begin, uint32_t* count)
{
    *begin = *count = 0;
    if (route >= routes) return 0;
    const uint32_t group = query_groups[route];
    if (group >= groups) return 0;
    *begin = group_offsets[group];
    *count = group_sizes[group];
    if (*begin > rows || *count > rows - *begin) {
        *begin = *count = 0;
        return 0;
    }
    return 1;
}

uint32_t orc_resident_candidate(const uint32_t* sample_ids, const uint64_t* row_masks,
                                const uint64_t* query_masks, const uint8_t* range_modes,
                                const float* range_lower, const float* range_upper,
                                const float* base_ranges, uint32_t rows, uint32_t samples,
                                uint32_t routes, uint32_t range_count, uint32_t route,
                                uint32_t row)
{
    if (route >= routes || row >= rows || (row_masks[row] & query_masks[route]) == 0)
        return UINT32_MAX;
    const uint32_t sample = sample_ids[row];
    if (sample >= samples) return UINT32_MAX;
    if (base_ranges != NULL &&
        orc_count_matching_ranges(range_modes, range_lower, range_upper, base_ranges, route,
                                  sample, range_count) !=
            orc_count_active_ranges(range_modes, route, range_count))
        return UINT32_MAX;
    return sample;
}

/* ======================================================================
 * Exact rerank -- exact_l2_u8 (backend_pq.cu:2187-2195) and the host batch
 * reranker (backend_pq.cu:2479-2592): unique valid candidates, exact L2,
 * top-k by (distance, sample id) ascending.  The exact L2 is accumulated
 * by 64 interleaved partial sums (lane j takes d = j mod 64, fmaf) folded
 * by an xor butterfly 32..1; for u8 data every partial is an exact
 * integer, so any order gives the reference's value.
 * ====================================================================== */
static float fold64(float* s)
{
    for (int off = 32; off > 0; off >>= 1)
        for (int j = 0; j < off; ++j) s[j] = s[j] + s[j + off];
    return s[0];
}

float orc_l2_u8(const uint8_t* a, const uint8_t* b, uint32_t dim)
{
    float s[64];
    for (int j = 0; j < 64; ++j) {
        float acc = 0.0f;
        for (uint32_t d = (uint32_t)j; d < dim; d += 64) {
            const float diff = (float)a[d] - (float)b[d];
            acc = fmaf(diff, diff, acc);
        }
        s[j] = acc;
    }
    return fold64(s);
}

float orc_l2_f32(const float* a, const float* b, uint32_t dim)
{
    float s[64];
    for (int j = 0; j < 64; ++j) {
        float acc = 0.0f;
        for (uint32_t d = (uint32_t)j; d < dim; d += 64) {
            const float diff = a[d] - b[d];
            acc = fmaf(diff, diff, acc);
        }
        s[j] = acc;
    }
    return fold64(s);
}

float orc_half_to_float(uint16_t h)
{
    /* IEEE 754 binary16 -> binary32 (fp16_l2.h:21-60 decodes the same). */
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t exp = (h >> 10) & 0x1f;
    uint32_t mant = h & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else {
            int e = -1;
            do {
                ++e;
                mant <<= 1;
            } while ((mant & 0x400) == 0);
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((mant & 0x3ff) << 13);
        }
    } else if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (mant << 13);
    }
    return bits_float(bits);
}

float orc_l2_f16(const float* q, const uint16_t* b, uint32_t dim)
{
    float s[64];
    for (int j = 0; j < 64; ++j) {
        float acc = 0.0f;
        for (uint32_t d = (uint32_t)j; d < dim; d += 64) {
            const float diff = q[d] - orc_half_to_float(b[d]);
            acc = fmaf(diff, diff, acc);
        }
        s[j] = acc;
    }
    return fold64(s);
}

static int cmp_u32(const void* a, const void* b)
{
    const uint32_t x = *(const uint32_t*)a, y = *(const uint32_t*)b;
    return x < y ? -1 : x > y;
}

int orc_rerank(const void* base, int elem_type, uint32_t dim, uint32_t samples,
               const void* queries, const uint32_t* route_query, const uint32_t* shortlist,
               uint32_t width, uint32_t routes, uint32_t topk, uint32_t* out_ids,
               float* out_dists)
{
    uint32_t* cand = (uint32_t*)malloc((size_t)(width ? width : 1) * sizeof(uint32_t));
    float* hd = (float*)malloc((size_t)(topk + 1) * sizeof(float));
    uint32_t* hi = (uint32_t*)malloc((size_t)(topk + 1) * sizeof(uint32_t));
    if (!cand || !hd || !hi) {
        free(cand);
        free(hd);
        free(hi);
        return -1;
    }
    for (uint32_t r = 0; r < routes; ++r) {
        uint32_t n = 0;
        for (uint32_t i = 0; i < width; ++i) {
            const uint32_t s = shortlist[(size_t)r * width + i];
            if (s == UINT32_MAX || s >= samples) continue;
            cand[n++] = s;
        }
        qsort(cand, n, sizeof(uint32_t), cmp_u32);
        for (uint32_t i = 0; i < topk; ++i) {
            hd[i] = FLT_MAX;
            hi[i] = UINT32_MAX;
        }
        const uint32_t q = route_query[r];
        for (uint32_t i = 0; i < n; ++i) {
            if (i > 0 && cand[i] == cand[i - 1]) continue;
            const uint32_t s = cand[i];
            float d;
            if (elem_type == 0)
                d = orc_l2_u8((const uint8_t*)queries + (size_t)q * dim,
                              (const uint8_t*)base + (size_t)s * dim, dim);
            else if (elem_type == 1)
                d = orc_l2_f32((const float*)queries + (size_t)q * dim,
                               (const float*)base + (size_t)s * dim, dim);
            else
                d = orc_l2_f16((const float*)queries + (size_t)q * dim,
                               (const uint16_t*)base + (size_t)s * dim, dim);
            /* Top-k by (dist, id); identical to the std::push_heap/pop_heap
             * max-heap on std::pair of backend_pq.cu:2546-2554. */
            orc_shortlist_insert(d, s, hd, hi, (int)topk);
        }
        orc_shortlist_sort(hd, hi, (int)topk);
        for (uint32_t i = 0; i < topk; ++i) {
            out_ids[(size_t)r * topk + i] = hi[i];
            out_dists[(size_t)r * topk + i] = hd[i];
        }
    }
    free(cand);
    free(hd);
    free(hi);
    return 0;
}

/* ======================================================================
 * Route merge -- rabitq_lowfreq_merge.h:709-815 (hash/dedup/sort path):
 * per original query keep each sample's minimum distance over its routes,
 * sort by (distance, id), take topk; padding UINT32_MAX / FLT_MAX.
 * ====================================================================== */
typedef struct {
    float d;
    uint32_t id;
} dpair;

static int cmp_dpair(const void* a, const void* b)
{
    const dpair* x = (const dpair*)a;
    const dpair* y = (const dpair*)b;
    if (x->d != y->d) return x->d < y->d ? -1 : 1;
    return x->id < y->id ? -1 : x->id > y->id;
}

static int cmp_dpair_id(const void* a, const void* b)
{
    const dpair* x = (const dpair*)a;
    const dpair* y = (const dpair*)b;
    return x->id < y->id ? -1 : x->id > y->id;
}

int orc_merge_routes(const uint32_t* route_to_query, uint32_t routes, uint32_t queries,
                     const uint32_t* route_ids, const float* route_dists, uint32_t width,
                     uint32_t topk, uint32_t* out_ids, float* out_dists)
{
    uint32_t* count = (uint32_t*)calloc(queries + 1, sizeof(uint32_t));
    if (!count) return -1;
    for (uint32_t r = 0; r < routes; ++r)
        if (route_to_query[r] < queries) ++count[route_to_query[r] + 1];
    for (uint32_t q = 0; q < queries; ++q) count[q + 1] += count[q];
    uint32_t* order = (uint32_t*)malloc((size_t)(routes ? routes : 1) * sizeof(uint32_t));
    uint32_t* fill = (uint32_t*)calloc(queries ? queries : 1, sizeof(uint32_t));
    dpair* buf = (dpair*)malloc((size_t)(width ? width : 1) * (routes ? routes : 1) * sizeof(dpair));
    if (!order || !fill || !buf) {
        free(count);
        free(order);
        free(fill);
        free(buf);
        return -1;
    }
    for (uint32_t r = 0; r < routes; ++r) {
        const uint32_t q = route_to_query[r];
        if (q < queries) order[count[q] + fill[q]++] = r;
    }
    for (uint32_t q = 0; q < queries; ++q) {
        size_t n = 0;
        for (uint32_t k = count[q]; k < count[q + 1]; ++k) {
            const uint32_t r = order[k];
            for (uint32_t i = 0; i < width; ++i) {
                const uint32_t id = route_ids[(size_t)r * width + i];
                if (id == UINT32_MAX) continue;
                buf[n].d = route_dists[(size_t)r * width + i];
                buf[n].id = id;
                ++n;
            }
        }
        /* keep the minimum distance per sample */
        qsort(buf, n, sizeof(dpair), cmp_dpair_id);
        size_t u = 0;
        for (size_t i = 0; i < n; ++i) {
            if (u > 0 && buf[u - 1].id == buf[i].id) {
                if (buf[i].d < buf[u - 1].d) buf[u - 1].d = buf[i].d;
            } else {
                buf[u++] = buf[i];
            }
        }
        qsort(buf, u, sizeof(dpair), cmp_dpair);
        for (uint32_t i = 0; i < topk; ++i) {
            out_ids[(size_t)q * topk + i] = i < u ? buf[i].id : UINT32_MAX;
            out_dists[(size_t)q * topk + i] = i < u ? buf[i].d : FLT_MAX;
        }
    }
    free(count);
    free(order);
    free(fill);
    free(buf);
    return 0;
}
