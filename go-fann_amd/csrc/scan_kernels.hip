// scan_kernels.hip -- posting-list scans and exact rerank on gfx950.
//
// Posting scans (lowfreq_pq_scan_kernel, src/search/pq/backend_pq.cu:
// 2046-2185; lowfreq_rabitq_resident_posting_kernel, src/search/rabitq/
// backend_rabitq.cu:5494-5682) keep the `shortlist_k` best predicate-valid
// candidates by (distance, id) through posting_shortlist_heap
// (src/search/common/posting_shortlist_heap.cuh).  That heap keeps exactly
// the k least admissible pairs of the scanned multiset (admissible: id !=
// UINT32_MAX and distance <= FLT_MAX, so NaN and +inf never enter) and
// emits them sorted, padded with (FLT_MAX, UINT32_MAX).  Here a 256-thread
// workgroup scores a chunk of candidates in parallel into LDS and a bitonic
// sort on the (distance, id) order merges the chunk with the running top-k,
// which yields the same sorted multiset.
//
// Exact rerank: one wave per candidate (lane j accumulates dimensions
// j mod 64 with fma, xor butterfly 32..1), unique valid candidates, top-k
// by (distance, id) -- the host reranker's order (backend_pq.cu:2479-2592)
// and resident_pq_batch_exact_rerank_kernel (backend_pq.cu:5201-5310).
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cfloat>
#include <cstdint>

#include "device_common.hpp"
#include "gofann_internal.hpp"
#include "scan_common.hpp"

namespace gofann {

struct ScanArgs {
    gofann_predicate_view pred;
    const uint32_t* route_query;
    const uint32_t* cand_ids;
    const uint32_t* cand_offsets;
    const uint32_t* cand_sizes;
    uint32_t routes;
    int k;
    int k_pow2;  // running-top-k region (power of two >= k)
    uint32_t* out_ids;
    float* out_dists;
    uint32_t* pass_counts;
    uint32_t table_bytes;
    uint32_t samples;  // ids >= samples are skipped (RaBitQ scan)
};

template <class Scorer>
__global__ __launch_bounds__(kScanThreads) void posting_scan_kernel(ScanArgs a, Scorer sc)
{
    extern __shared__ __align__(16) unsigned char lds[];
    __shared__ float s_d[kScanSlots];
    __shared__ uint32_t s_id[kScanSlots];
    __shared__ uint32_t s_pass;
    const int tid = static_cast<int>(threadIdx.x);
    const uint32_t route = blockIdx.x;
    if (route >= a.routes) return;

    sc.setup(a.route_query[route], tid, lds);
    for (int i = tid; i < kScanSlots; i += kScanThreads) {
        s_d[i] = FLT_MAX;
        s_id[i] = UINT32_MAX;
    }
    if (tid == 0) s_pass = 0;
    __syncthreads();

    const bool enabled = pred_enabled(a.pred, route);
    const uint32_t begin = a.cand_offsets[route];
    const uint32_t count = a.cand_sizes[route];
    const int chunk = kScanSlots - a.k_pow2;
    uint32_t passes = 0;
    for (uint32_t base = 0; base < count; base += static_cast<uint32_t>(chunk)) {
        for (int i = tid; i < chunk; i += kScanThreads) {
            const uint32_t j = base + static_cast<uint32_t>(i);
            float d = FLT_MAX;
            uint32_t id = UINT32_MAX;
            if (j < count) {
                const uint32_t s = a.cand_ids[begin + j];
                bool ok = s != UINT32_MAX && s < a.samples;
                if (ok && enabled) {
                    PredCounters c{0, 0};
                    ok = pred_matches(a.pred, route, s, c);
                    passes += ok ? 1u : 0u;
                }
                if (ok) {
                    const float v = sc.score(s);
                    if (admissible(v, s)) {
                        d = v;
                        id = s;
                    }
                }
            }
            s_d[a.k_pow2 + i] = d;
            s_id[a.k_pow2 + i] = id;
        }
        __syncthreads();
        bitonic_sort(s_d, s_id, kScanSlots, tid, kScanThreads);
    }
    atomicAdd(&s_pass, passes);
    __syncthreads();
    for (int i = tid; i < a.k; i += kScanThreads) {
        a.out_ids[static_cast<size_t>(route) * a.k + i] = s_id[i];
        a.out_dists[static_cast<size_t>(route) * a.k + i] = s_d[i];
    }
    if (tid == 0 && a.pass_counts) a.pass_counts[route] = s_pass;
}

// Exact rerank: one workgroup of 4 waves per route.
struct RerankArgs {
    const void* base;
    int base_elem;
    uint32_t dim;
    uint32_t samples;
    const void* queries;
    const uint32_t* route_query;
    const uint32_t* shortlist;
    uint32_t width;
    uint32_t width_pow2;
    uint32_t routes;
    uint32_t topk;
    uint32_t* out_ids;
    float* out_dists;
};

constexpr int kRerankThreads = 256;

// One lane's chain of the rerank distance: acc = fma(diff, diff, acc) over
// d = lane, lane + 64, ... in d order, with kRerankBatch row elements
// loaded before the first of them is used (the compiler's unrolling of the
// plain loop kept the loads in small groups).  load(d): the base element as
// float; diff(d, b): query minus base, in the element type's form.
constexpr int kRerankBatch = 16;

template <class Load, class Diff>
__device__ __forceinline__ float lane_chain(uint32_t dim, int lane, Load load, Diff diff)
{
    float acc = 0.0f;
    uint32_t d = static_cast<uint32_t>(lane);
    for (; d + kWave * (kRerankBatch - 1) < dim; d += kWave * kRerankBatch) {
        float bv[kRerankBatch];
#pragma unroll
        for (int t = 0; t < kRerankBatch; ++t) bv[t] = load(d + kWave * t);
#pragma unroll
        for (int t = 0; t < kRerankBatch; ++t) {
            const float x = diff(d + kWave * t, bv[t]);
            acc = fmaf(x, x, acc);
        }
    }
    // the rest (whole rows under kRerankBatch * 64 elements): unrolled so
    // that 8 steps' loads are in flight
#pragma unroll 8
    for (; d < dim; d += kWave) {
        const float x = diff(d, load(d));
        acc = fmaf(x, x, acc);
    }
    return acc;
}

__global__ __launch_bounds__(kRerankThreads) void exact_rerank_kernel(RerankArgs a)
{
    __shared__ float s_d[kMaxShortlist];
    __shared__ uint32_t s_id[kMaxShortlist];
    __shared__ uint32_t s_keep[kMaxShortlist];
    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const uint32_t route = blockIdx.x;
    if (route >= a.routes) return;
    const uint32_t q = a.route_query[route];

    for (uint32_t i = tid; i < a.width_pow2; i += kRerankThreads) {
        s_d[i] = FLT_MAX;
        s_id[i] = UINT32_MAX;
    }
    __syncthreads();
    for (uint32_t c = wave; c < a.width; c += kRerankThreads / kWave) {
        const uint32_t s = a.shortlist[static_cast<size_t>(route) * a.width + c];
        if (s == UINT32_MAX || s >= a.samples) continue;  // uniform per wave
        float acc = 0.0f;
        if (a.base_elem == GOFANN_ELEM_U8) {
            const uint8_t* b = static_cast<const uint8_t*>(a.base) + static_cast<size_t>(s) * a.dim;
            const uint8_t* qq = static_cast<const uint8_t*>(a.queries) + static_cast<size_t>(q) * a.dim;
            acc = lane_chain(a.dim, lane, [&](uint32_t d) { return static_cast<float>(b[d]); },
                             [&](uint32_t d, float bv) { return static_cast<float>(qq[d]) - bv; });
        } else if (a.base_elem == GOFANN_ELEM_F32) {
            const float* b = static_cast<const float*>(a.base) + static_cast<size_t>(s) * a.dim;
            const float* qq = static_cast<const float*>(a.queries) + static_cast<size_t>(q) * a.dim;
            acc = lane_chain(a.dim, lane, [&](uint32_t d) { return b[d]; },
                             [&](uint32_t d, float bv) { return qq[d] - bv; });
        } else {
            const __half* b = static_cast<const __half*>(a.base) + static_cast<size_t>(s) * a.dim;
            const float* qq = static_cast<const float*>(a.queries) + static_cast<size_t>(q) * a.dim;
            acc = lane_chain(a.dim, lane, [&](uint32_t d) { return __half2float(b[d]); },
                             [&](uint32_t d, float bv) { return qq[d] - bv; });
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) acc = acc + __shfl_xor(acc, off, kWave);
        if (lane == 0) {
            s_d[c] = acc;
            s_id[c] = s;
        }
    }
    __syncthreads();
    bitonic_sort(s_d, s_id, static_cast<int>(a.width_pow2), tid, kRerankThreads);
    // Unique valid ids (a duplicate has the same distance, so it is adjacent).
    for (uint32_t i = tid; i < a.width_pow2; i += kRerankThreads)
        s_keep[i] = (s_id[i] != UINT32_MAX && (i == 0 || s_id[i - 1] != s_id[i])) ? 1u : 0u;
    __syncthreads();
    if (tid == 0) {
        uint32_t o = 0;
        for (uint32_t i = 0; i < a.width_pow2 && o < a.topk; ++i) {
            if (!s_keep[i]) continue;
            a.out_ids[static_cast<size_t>(route) * a.topk + o] = s_id[i];
            a.out_dists[static_cast<size_t>(route) * a.topk + o] = s_d[i];
            ++o;
        }
        for (; o < a.topk; ++o) {
            a.out_ids[static_cast<size_t>(route) * a.topk + o] = UINT32_MAX;
            a.out_dists[static_cast<size_t>(route) * a.topk + o] = FLT_MAX;
        }
    }
}

// Candidate pass bitsets: each lane evaluates one (route, sample) pair; the
// wave ballot is split into the reference's 32-bit words.
__global__ __launch_bounds__(64) void predicate_masks_kernel(gofann_predicate_view pred,
                                                            const uint32_t* route_ids,
                                                            const uint32_t* sample_ids, uint32_t n,
                                                            uint32_t* masks)
{
    const uint32_t i = blockIdx.x * kWave + threadIdx.x;
    bool pass = false;
    if (i < n) {
        PredCounters c{0, 0};
        pass = pred_enabled(pred, route_ids[i]) &&
               pred_matches(pred, route_ids[i], sample_ids[i], c);
    }
    const uint64_t b = ballot(pass);
    const uint32_t w0 = blockIdx.x * 2;
    const uint32_t words = (n + 31) / 32;
    if (threadIdx.x == 0 && w0 < words) masks[w0] = static_cast<uint32_t>(b);
    if (threadIdx.x == 0 && w0 + 1 < words) masks[w0 + 1] = static_cast<uint32_t>(b >> 32);
}

int predicate_masks(Context* ctx, const gofann_predicate_view* pred, const uint32_t* route_ids,
                    const uint32_t* sample_ids, uint32_t n, uint32_t* masks)
{
    if (!pred || !route_ids || !sample_ids || !masks)
        return ctx->fail(GOFANN_ERR_INVALID, "predicate mask inputs incomplete");
    if (n == 0) return GOFANN_OK;
    hipLaunchKernelGGL(predicate_masks_kernel, dim3((n + kWave - 1) / kWave), dim3(kWave), 0,
                       ctx->stream, *pred, route_ids, sample_ids, n, masks);
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("predicate masks launch");
    return GOFANN_OK;
}

// Route -> original query merge (merge_route_results_to_original,
// src/search/rabitq/rabitq_lowfreq_merge.h:709-815): for each query the
// minimum distance per sample over its routes, ordered by (distance, id),
// first topk.  One thread per query keeps a sorted top-k with dedup: a
// sample already held is replaced only by a smaller distance, and a sample
// evicted earlier can never re-enter with a larger one (the k-th distance
// only falls), so the streamed result equals the hash/dedup/sort of the
// reference.
constexpr int kMaxMergeTopk = 64;

__global__ __launch_bounds__(256) void merge_routes_kernel(const uint32_t* q_route_offsets,
                                                          const uint32_t* q_routes,
                                                          const uint32_t* route_ids,
                                                          const float* route_dists, uint32_t width,
                                                          uint32_t queries, uint32_t topk,
                                                          uint32_t* out_ids, float* out_dists)
{
    const uint32_t q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= queries) return;
    float bd[kMaxMergeTopk];
    uint32_t bi[kMaxMergeTopk];
    uint32_t n = 0;
    for (uint32_t k = q_route_offsets[q]; k < q_route_offsets[q + 1]; ++k) {
        const uint32_t r = q_routes[k];
        for (uint32_t i = 0; i < width; ++i) {
            const uint32_t id = route_ids[static_cast<size_t>(r) * width + i];
            if (id == UINT32_MAX) continue;
            const float d = route_dists[static_cast<size_t>(r) * width + i];
            uint32_t have = n;
            for (uint32_t j = 0; j < n; ++j)
                if (bi[j] == id) have = j;
            if (have < n) {
                if (!(d < bd[have])) continue;
                for (uint32_t j = have; j + 1 < n; ++j) {  // drop the old entry
                    bd[j] = bd[j + 1];
                    bi[j] = bi[j + 1];
                }
                --n;
            }
            if (n == topk && !pair_less(d, id, bd[n - 1], bi[n - 1])) continue;
            uint32_t pos = n < topk ? n : topk - 1;
            while (pos > 0 && pair_less(d, id, bd[pos - 1], bi[pos - 1])) {
                bd[pos] = bd[pos - 1];
                bi[pos] = bi[pos - 1];
                --pos;
            }
            bd[pos] = d;
            bi[pos] = id;
            if (n < topk) ++n;
        }
    }
    for (uint32_t j = 0; j < topk; ++j) {
        out_ids[static_cast<size_t>(q) * topk + j] = j < n ? bi[j] : UINT32_MAX;
        out_dists[static_cast<size_t>(q) * topk + j] = j < n ? bd[j] : FLT_MAX;
    }
}

int merge_routes(Context* ctx, const uint32_t* q_route_offsets, const uint32_t* q_routes,
                 const uint32_t* route_ids, const float* route_dists, uint32_t width,
                 uint32_t queries, uint32_t topk, uint32_t* out_ids, float* out_dists)
{
    if (!q_route_offsets || !q_routes || !route_ids || !route_dists || !out_ids || !out_dists)
        return ctx->fail(GOFANN_ERR_INVALID, "merge inputs incomplete");
    if (topk == 0 || topk > static_cast<uint32_t>(kMaxMergeTopk))
        return ctx->fail(GOFANN_ERR_INVALID, "merge topk must be in [1, 64]");
    if (queries == 0) return GOFANN_OK;
    hipLaunchKernelGGL(merge_routes_kernel, dim3((queries + 255) / 256), dim3(256), 0, ctx->stream,
                       q_route_offsets, q_routes, route_ids, route_dists, width, queries, topk,
                       out_ids, out_dists);
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("merge launch");
    return GOFANN_OK;
}

namespace {
uint32_t pow2_at_least(uint32_t x)
{
    uint32_t p = 1;
    while (p < x) p <<= 1;
    return p;
}
}  // namespace

int pq_posting_scan(Context* ctx, const gofann_pq_view* pq, const void* queries, int query_elem,
                    const gofann_predicate_view* pred, const uint32_t* route_query,
                    const uint32_t* cand_ids, const uint32_t* cand_offsets,
                    const uint32_t* cand_sizes, uint32_t routes, int shortlist_k,
                    uint32_t* out_ids, float* out_dists, uint32_t* pass_counts)
{
    if (!pq || !pq->codes || !pq->centroids || !queries || pq->pq_dim == 0 ||
        pq->dim % pq->pq_dim != 0 || pq->pq_dim > 64)
        return ctx->fail(GOFANN_ERR_INVALID, "PQ view invalid for posting scan (pq_dim <= 64)");
    if (shortlist_k < 1 || shortlist_k > kMaxShortlist)
        return ctx->fail(GOFANN_ERR_INVALID, "shortlist_k must be in [1, 512]");
    if (routes == 0) return GOFANN_OK;
    ScanArgs a;
    a.pred = pred ? *pred : gofann_predicate_view{};
    a.route_query = route_query;
    a.cand_ids = cand_ids;
    a.cand_offsets = cand_offsets;
    a.cand_sizes = cand_sizes;
    a.routes = routes;
    a.k = shortlist_k;
    a.k_pow2 = static_cast<int>(pow2_at_least(static_cast<uint32_t>(shortlist_k)));
    a.out_ids = out_ids;
    a.out_dists = out_dists;
    a.pass_counts = pass_counts;
    a.samples = pq->samples ? pq->samples : UINT32_MAX;
    PqScanScorer sc;
    sc.codes = pq->codes;
    sc.centroids = pq->centroids;
    sc.queries = queries;
    sc.query_f32 = query_elem == GOFANN_ELEM_F32 ? 1 : 0;
    sc.dim = pq->dim;
    sc.pq_dim = pq->pq_dim;
    sc.stride = pq->code_stride ? pq->code_stride : pq->pq_dim;
    sc.lut = nullptr;
    const uint32_t lds = pq->pq_dim * 256u * 4u;
    a.table_bytes = lds;
    auto kern = posting_scan_kernel<PqScanScorer>;
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)) !=
        hipSuccess)
        return ctx->fail_hip("hipFuncSetAttribute posting scan");
    hipLaunchKernelGGL(kern, dim3(routes), dim3(kScanThreads), lds, ctx->stream, a, sc);
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("pq posting scan launch");
    return GOFANN_OK;
}

int rabitq_posting_scan(Context* ctx, const gofann_rabitq_view* rq,
                        const gofann_rabitq_queries* pre, const gofann_predicate_view* pred,
                        const uint32_t* route_query, const uint32_t* cand_ids,
                        const uint32_t* cand_offsets, const uint32_t* cand_sizes,
                        uint32_t routes, int shortlist_k, uint32_t* out_ids, float* out_dists,
                        uint32_t* pass_counts)
{
    if (!rq || !pre || !rq->codes || rq->padded_dim == 0 || rq->padded_dim % 128 != 0)
        return ctx->fail(GOFANN_ERR_INVALID, "RaBitQ view invalid for posting scan");
    if (shortlist_k < 1 || shortlist_k > kMaxShortlist)
        return ctx->fail(GOFANN_ERR_INVALID, "shortlist_k must be in [1, 512]");
    if (routes == 0) return GOFANN_OK;
    // Code rows that split over a lane group take the group-per-row scan
    // (range_scan.hip); the thread-per-row kernel below takes the rest.
    if (rabitq_posting_scan_grouped(rq->padded_dim))
        return rabitq_posting_scan_group(ctx, rq, pre, pred, route_query, cand_ids, cand_offsets,
                                         cand_sizes, routes, shortlist_k, out_ids, out_dists,
                                         pass_counts);
    ScanArgs a;
    a.pred = pred ? *pred : gofann_predicate_view{};
    a.route_query = route_query;
    a.cand_ids = cand_ids;
    a.cand_offsets = cand_offsets;
    a.cand_sizes = cand_sizes;
    a.routes = routes;
    a.k = shortlist_k;
    a.k_pow2 = static_cast<int>(pow2_at_least(static_cast<uint32_t>(shortlist_k)));
    a.out_ids = out_ids;
    a.out_dists = out_dists;
    a.pass_counts = pass_counts;
    a.samples = rq->samples ? rq->samples : UINT32_MAX;
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
    const uint32_t lds = rq->padded_dim;
    a.table_bytes = lds;
    hipLaunchKernelGGL(posting_scan_kernel<RabitqScanScorer>, dim3(routes), dim3(kScanThreads), lds,
                       ctx->stream, a, sc);
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("rabitq posting scan launch");
    return GOFANN_OK;
}

int exact_rerank(Context* ctx, const void* base, int base_elem, uint32_t dim, uint32_t samples,
                 const void* queries, const uint32_t* route_query, const uint32_t* shortlist,
                 uint32_t width, uint32_t routes, uint32_t topk, uint32_t* out_ids,
                 float* out_dists)
{
    if (!base || !queries || !route_query || !shortlist || dim == 0)
        return ctx->fail(GOFANN_ERR_INVALID, "rerank inputs incomplete");
    if (base_elem < GOFANN_ELEM_U8 || base_elem > GOFANN_ELEM_F16)
        return ctx->fail(GOFANN_ERR_INVALID, "unknown base element type");
    if (width == 0 || width > static_cast<uint32_t>(kMaxShortlist) || topk == 0 || topk > width)
        return ctx->fail(GOFANN_ERR_INVALID, "rerank width must be in [1, 512], topk in [1, width]");
    if (routes == 0) return GOFANN_OK;
    RerankArgs a;
    a.base = base;
    a.base_elem = base_elem;
    a.dim = dim;
    a.samples = samples;
    a.queries = queries;
    a.route_query = route_query;
    a.shortlist = shortlist;
    a.width = width;
    a.width_pow2 = pow2_at_least(width);
    a.routes = routes;
    a.topk = topk;
    a.out_ids = out_ids;
    a.out_dists = out_dists;
    hipLaunchKernelGGL(exact_rerank_kernel, dim3(routes), dim3(kRerankThreads), 0, ctx->stream, a);
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("exact rerank launch");
    return GOFANN_OK;
}

}  // namespace gofann
