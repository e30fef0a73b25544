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
//  * serial order: a lane per row, the chain in d order, rows read through
//    per-wave LDS tiles so that loads cover whole lines (a thread reading
//    its own row where the row length does not allow 16-byte words); warp
//    order: a quad of lanes per row (exact_dist.hpp);
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
    uint32_t tile_offset;  // bytes from the LDS base to the tiles
};

constexpr int kExactScanMaxTopk = 64;

// kTile: 0 -- the serial order one thread per row reading its own row (any
// row length); 16 or 32 -- the serial order through LDS tiles of that many
// words per row (l2_serial_tiled; row bytes % 16 == 0).  The warp order
// takes a quad of lanes per row (l2_w32_quad) and ignores kTile.
template <int kElem, int kOrder, int kTile>
__global__ __launch_bounds__(kScanThreads) void exact_scan_kernel(ExactScanArgs a)
{
    // dynamic LDS: the query as f32 [dim], then (tiled) one tile per wave
    extern __shared__ __align__(16) unsigned char lds[];
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
        if constexpr (kOrder == GOFANN_EXACT_ORDER_SERIAL && kTile > 0) {
            const int wave = tid / kWave;
            const int lane = tid % kWave;
            uint32_t* tile = reinterpret_cast<uint32_t*>(lds + a.tile_offset) +
                             wave * kWave * (kTile + 1);
            for (int i0 = wave * kWave; i0 < n; i0 += kScanThreads) {
                const int rows = n - i0 < kWave ? n - i0 : kWave;
                const float d = l2_serial_tiled<kElem, kTile>(a.base, row_bytes, q,
                                                              &s_id[a.k_pow2 + i0], rows, tile,
                                                              lane);
                if (lane < rows) {
                    const int slot = a.k_pow2 + i0 + lane;
                    const bool nan = d != d;
                    s_d[slot] = nan ? inf : d;
                    if (nan) s_id[slot] = UINT32_MAX;
                }
            }
        } else if constexpr (kOrder == GOFANN_EXACT_ORDER_SERIAL) {
            for (int i = tid; i < n; i += kScanThreads) {
                const int slot = a.k_pow2 + i;
                const uint32_t s = s_id[slot];
                const float d = l2_serial<kElem>(a.base + static_cast<size_t>(s) * row_bytes, q, a.dim);
                const bool nan = d != d;
                s_d[slot] = nan ? inf : d;
                if (nan) s_id[slot] = UINT32_MAX;
            }
        } else {
            const uint32_t g = static_cast<uint32_t>(tid) & 3u;
            for (int i = tid >> 2; i - (tid >> 2) < n; i += kScanThreads / 4) {
                if (i < n) {
                    const int slot = a.k_pow2 + i;
                    const uint32_t s = s_id[slot];
                    const float d =
                        l2_w32_quad<kElem>(a.base + static_cast<size_t>(s) * row_bytes, q, a.dim, g);
                    if (g == 0) {
                        const bool nan = d != d;
                        s_d[slot] = nan ? inf : d;
                        if (nan) s_id[slot] = UINT32_MAX;
                    }
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

template <int kElem, int kOrder, int kTile>
int launch_exact_scan(Context* ctx, const ExactScanArgs& a, uint32_t lds)
{
    const void* k = reinterpret_cast<const void*>(exact_scan_kernel<kElem, kOrder, kTile>);
    if (hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)) !=
        hipSuccess)
        return ctx->fail_hip("hipFuncSetAttribute exact posting scan");
    hipLaunchKernelGGL((exact_scan_kernel<kElem, kOrder, kTile>), dim3(a.routes),
                       dim3(kScanThreads), lds, ctx->stream, a);
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("exact posting scan launch");
    return GOFANN_OK;
}

// Serial order: LDS tiles of 32 words per row where the row allows them and
// the workgroup's LDS holds them, else of 16, else a thread per row.
template <int kElem>
int launch_exact_scan_order(Context* ctx, ExactScanArgs& a, uint32_t q_lds, uint32_t fixed,
                            int order)
{
    if (order == GOFANN_EXACT_ORDER_WARP)
        return launch_exact_scan<kElem, GOFANN_EXACT_ORDER_WARP, 0>(ctx, a, q_lds);
    const size_t row_bytes = static_cast<size_t>(a.dim) * elem_bytes(kElem);
    const uint32_t limit = static_cast<uint32_t>(ctx->lds_per_block);
    a.tile_offset = q_lds;
    const uint32_t waves = kScanThreads / kWave;
    const uint32_t t32 = q_lds + waves * kWave * 33u * 4u;
    const uint32_t t16 = q_lds + waves * kWave * 17u * 4u;
    if (row_bytes % 16 == 0 && t32 + fixed <= limit)
        return launch_exact_scan<kElem, GOFANN_EXACT_ORDER_SERIAL, 32>(ctx, a, t32);
    if (row_bytes % 16 == 0 && t16 + fixed <= limit)
        return launch_exact_scan<kElem, GOFANN_EXACT_ORDER_SERIAL, 16>(ctx, a, t16);
    return launch_exact_scan<kElem, GOFANN_EXACT_ORDER_SERIAL, 0>(ctx, a, q_lds);
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
    a.tile_offset = 0;
    switch (base_elem) {
    case GOFANN_ELEM_F32:
        return launch_exact_scan_order<GOFANN_ELEM_F32>(ctx, a, lds, fixed, order);
    case GOFANN_ELEM_F16:
        return launch_exact_scan_order<GOFANN_ELEM_F16>(ctx, a, lds, fixed, order);
    default: return launch_exact_scan_order<GOFANN_ELEM_U8>(ctx, a, lds, fixed, order);
    }
}

}  // namespace gofann
