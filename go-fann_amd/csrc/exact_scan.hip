// exact_scan.hip -- exact-distance posting scans of the full-GPU backend on
// gfx950.
//
// Reference: full_gpu_range_posting_kernel (src/search/full_gpu/
// backend_full_gpu.cu:1383-1493; a thread per posting row, the distance a
// serial chain over d) and full_gpu_lowfreq_kernel (:2124-2262; a warp per
// route, each row's distance in l2_distance_device's warp order).  Both keep
// a best-topk with sample dedup (insert_best_result :1333-1375), so per
// route the result is the topk least (distance, id) pairs over the distinct
// listed samples that pass the filter.
//
// Here one 256-thread workgroup scans one route in chunks of the 2048-slot
// LDS pair array (running top-k + chunk):
//  * the chunk's valid, predicate-passing samples are compacted into the
//    chunk slots (order is free: the (distance, id) sort fixes it);
//  * serial order: a thread per row (16-byte loads, the chain in d order);
//    warp order: a 32-lane half per row (exact_dist.hpp);
//  * a bitonic sort on (distance, id) merges the chunk with the running
//    top-k, and one lane keeps the first topk distinct ids (a duplicate has
//    the same distance, so it sits next to its twin).
// Empty slots hold (+inf, UINT32_MAX), so a row of infinite distance still
// ranks before them, as it enters the reference's list.  A NaN distance
// (only from NaN or infinite inputs) is dropped.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>
#include <string>

#include "device_common.hpp"
#include "exact_dist.hpp"
#include "gofann_internal.hpp"
#include "scan_common.hpp"

namespace gofann {

struct ExactScanArgs {
    gofann_predicate_view pred;
    const uint8_t* base;
    const uint8_t* queries;
    uint32_t dim;
    uint32_t samples;
    const uint32_t* route_query;
    const uint32_t* cand_ids;
    const uint32_t* cand_offsets;
    const uint32_t* cand_sizes;
    uint32_t routes;
    int k;
    int k_pow2;
    uint32_t* out_ids;
    float* out_dists;
    uint32_t* pass_counts;
};

constexpr int kExactScanMaxTopk = 64;

template <int kElem, int kOrder>
__global__ __launch_bounds__(kScanThreads) void exact_scan_kernel(ExactScanArgs a)
{
    extern __shared__ __align__(16) unsigned char lds[];  // query as f32 [dim]
    __shared__ float s_d[kScanSlots];
    __shared__ uint32_t s_id[kScanSlots];
    __shared__ uint32_t s_n;
    __shared__ uint32_t s_pass;
    const int tid = static_cast<int>(threadIdx.x);
    const uint32_t route = blockIdx.x;
    if (route >= a.routes) return;
    const float inf = __builtin_inff();

    float* q = reinterpret_cast<float*>(lds);
    const uint8_t* qrow =
        a.queries + static_cast<size_t>(a.route_query[route]) * a.dim * elem_bytes(kElem);
    for (uint32_t d = tid; d < a.dim; d += kScanThreads) q[d] = elem_to_float<kElem>(qrow, d);
    for (int i = tid; i < kScanSlots; i += kScanThreads) {
        s_d[i] = inf;
        s_id[i] = UINT32_MAX;
    }
    if (tid == 0) s_pass = 0;
    __syncthreads();

    const bool enabled = pred_enabled(a.pred, route);
    const uint32_t begin = a.cand_offsets[route];
    const uint32_t count = a.cand_sizes[route];
    const size_t row_bytes = static_cast<size_t>(a.dim) * elem_bytes(kElem);
    const int chunk = kScanSlots - a.k_pow2;
    uint32_t passes = 0;
    for (uint32_t b0 = 0; b0 < count; b0 += static_cast<uint32_t>(chunk)) {
        if (tid == 0) s_n = 0;
        __syncthreads();
        for (int i = tid; i < chunk; i += kScanThreads) {
            const uint32_t j = b0 + static_cast<uint32_t>(i);
            if (j >= count) break;
            const uint32_t s = a.cand_ids[begin + j];
            bool ok = s != UINT32_MAX && s < a.samples;
            if (ok && enabled) {
                PredCounters c{0, 0};
                ok = pred_matches(a.pred, route, s, c);
            }
            if (ok) {
                ++passes;
                const uint32_t pos = atomicAdd(&s_n, 1u);
                s_id[a.k_pow2 + static_cast<int>(pos)] = s;
            }
        }
        __syncthreads();
        const int n = static_cast<int>(s_n);
        if constexpr (kOrder == GOFANN_EXACT_ORDER_SERIAL) {
            for (int i = tid; i < n; i += kScanThreads) {
                const int slot = a.k_pow2 + i;
                const uint32_t s = s_id[slot];
                const float d = l2_serial<kElem>(a.base + static_cast<size_t>(s) * row_bytes, q, a.dim);
                const bool nan = d != d;
                s_d[slot] = nan ? inf : d;
                if (nan) s_id[slot] = UINT32_MAX;
            }
        } else {
            const uint32_t j = static_cast<uint32_t>(tid) & 31u;
            for (int i = tid >> 5; i < n; i += kScanThreads / 32) {
                const int slot = a.k_pow2 + i;
                const uint32_t s = s_id[slot];
                const float d = w32_tree<kElem>(
                    l2_w32_partial<kElem>(a.base + static_cast<size_t>(s) * row_bytes, q, a.dim, j));
                if (j == 0) {
                    const bool nan = d != d;
                    s_d[slot] = nan ? inf : d;
                    if (nan) s_id[slot] = UINT32_MAX;
                }
            }
        }
        for (int i = a.k_pow2 + n + tid; i < kScanSlots; i += kScanThreads) {
            s_d[i] = inf;
            s_id[i] = UINT32_MAX;
        }
        __syncthreads();
        bitonic_sort(s_d, s_id, kScanSlots, tid, kScanThreads);
        if (tid == 0) {
            int o = 0;
            uint32_t prev = UINT32_MAX;
            for (int i = 0; i < kScanSlots && o < a.k; ++i) {
                const uint32_t id = s_id[i];
                if (id == UINT32_MAX) break;
                if (id == prev) continue;
                prev = id;
                s_d[o] = s_d[i];
                s_id[o] = id;
                ++o;
            }
            for (; o < a.k_pow2; ++o) {
                s_d[o] = inf;
                s_id[o] = UINT32_MAX;
            }
        }
        __syncthreads();
    }
    atomicAdd(&s_pass, passes);
    __syncthreads();
    for (int i = tid; i < a.k; i += kScanThreads) {
        const uint32_t id = s_id[i];
        a.out_ids[static_cast<size_t>(route) * a.k + i] = id;
        a.out_dists[static_cast<size_t>(route) * a.k + i] = id == UINT32_MAX ? FLT_MAX : s_d[i];
    }
    if (tid == 0 && a.pass_counts) a.pass_counts[route] = s_pass;
}

namespace {

int pow2_ceil(int x)
{
    int p = 1;
    while (p < x) p <<= 1;
    return p;
}

template <int kElem, int kOrder>
int launch_exact_scan(Context* ctx, const ExactScanArgs& a, uint32_t lds)
{
    const void* k = reinterpret_cast<const void*>(exact_scan_kernel<kElem, kOrder>);
    if (hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)) !=
        hipSuccess)
        return ctx->fail_hip("hipFuncSetAttribute exact posting scan");
    hipLaunchKernelGGL((exact_scan_kernel<kElem, kOrder>), dim3(a.routes), dim3(kScanThreads), lds,
                       ctx->stream, a);
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("exact posting scan launch");
    return GOFANN_OK;
}

template <int kElem>
int launch_exact_scan_order(Context* ctx, const ExactScanArgs& a, uint32_t lds, int order)
{
    return order == GOFANN_EXACT_ORDER_WARP
               ? launch_exact_scan<kElem, GOFANN_EXACT_ORDER_WARP>(ctx, a, lds)
               : launch_exact_scan<kElem, GOFANN_EXACT_ORDER_SERIAL>(ctx, a, lds);
}

}  // namespace

int exact_posting_scan(Context* ctx, const void* base, int base_elem, uint32_t dim,
                       uint32_t samples, const void* queries, const gofann_predicate_view* pred,
                       const uint32_t* route_query, const uint32_t* cand_ids,
                       const uint32_t* cand_offsets, const uint32_t* cand_sizes, uint32_t routes,
                       int topk, int order, uint32_t* out_ids, float* out_dists,
                       uint32_t* pass_counts)
{
    if (base_elem != GOFANN_ELEM_U8 && base_elem != GOFANN_ELEM_F32 && base_elem != GOFANN_ELEM_F16)
        return ctx->fail(GOFANN_ERR_INVALID, "base_elem must be u8, f32 or f16");
    if (order != GOFANN_EXACT_ORDER_SERIAL && order != GOFANN_EXACT_ORDER_WARP)
        return ctx->fail(GOFANN_ERR_INVALID, "order must be GOFANN_EXACT_ORDER_SERIAL or _WARP");
    if (topk < 1 || topk > kExactScanMaxTopk)
        return ctx->fail(GOFANN_ERR_INVALID, "topk must be in [1, 64]");
    if (!base || !queries || dim == 0)
        return ctx->fail(GOFANN_ERR_INVALID, "exact posting scan vectors missing");
    if (dim > 65536) return ctx->fail(GOFANN_ERR_INVALID, "dim must be <= 65536");
    if ((reinterpret_cast<uintptr_t>(base) & 15u) != 0)
        return ctx->fail(GOFANN_ERR_INVALID, "base must be 16-byte aligned");
    if (routes == 0) return GOFANN_OK;
    if (!route_query || !cand_ids || !cand_offsets || !cand_sizes || !out_ids || !out_dists)
        return ctx->fail(GOFANN_ERR_INVALID, "route arrays or outputs missing");
    const uint32_t lds = (dim * 4u + 15u) & ~15u;
    const uint32_t fixed = kScanSlots * 8u + 8u;
    if (lds + fixed > static_cast<uint32_t>(ctx->lds_per_block))
        return ctx->fail(GOFANN_ERR_UNSUPPORTED,
                         "the query row (" + std::to_string(dim) + " f32) does not fit in LDS");
    ExactScanArgs a;
    a.pred = pred ? *pred : gofann_predicate_view{};
    a.base = static_cast<const uint8_t*>(base);
    a.queries = static_cast<const uint8_t*>(queries);
    a.dim = dim;
    a.samples = samples;
    a.route_query = route_query;
    a.cand_ids = cand_ids;
    a.cand_offsets = cand_offsets;
    a.cand_sizes = cand_sizes;
    a.routes = routes;
    a.k = topk;
    a.k_pow2 = pow2_ceil(topk);
    a.out_ids = out_ids;
    a.out_dists = out_dists;
    a.pass_counts = pass_counts;
    switch (base_elem) {
    case GOFANN_ELEM_F32: return launch_exact_scan_order<GOFANN_ELEM_F32>(ctx, a, lds, order);
    case GOFANN_ELEM_F16: return launch_exact_scan_order<GOFANN_ELEM_F16>(ctx, a, lds, order);
    default: return launch_exact_scan_order<GOFANN_ELEM_U8>(ctx, a, lds, order);
    }
}

}  // namespace gofann
