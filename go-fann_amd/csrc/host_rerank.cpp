// host_rerank.cpp -- CPU exact rerank of GPU graph shortlists, streamed so
// the host reranks finished route chunks while the GPU searches the next
// ones (the reference's streaming CPU rerank schedule).
//
//   * exact distances follow highfreq_host_batch_rerank_range and
//     exact_l2_u8 (src/search/pq/backend_pq.cu:2187-2195, 2479-2592) and the
//     float base path compute_base_float_vector_l2 (src/data/dataloader.cpp:
//     2746-2772): fp32, dimensions in order;
//   * per route: valid unique shortlist ids (sorted, UINT32_MAX and ids past
//     the base skipped), top-k by (distance, id) with the smaller id winning a
//     tie, output ascending and padded with (UINT32_MAX, FLT_MAX);
//   * the shortlist is predicate-verified on the device (only passing nodes
//     enter the result heap), as the reference assumes for its GPU predicate
//     mode (shortlist_verified, backend_pq.cu:9725), so labels are not
//     re-checked here;
//   * fp16 rows: the reference picks its fp16 L2 kernel at run time
//     (fp16_l2::select, src/data/fp16_l2.h:53-70; GO_FANN_FP16_RERANK_KERNEL,
//     dataloader.cpp:2131-2133): AVX-512 when the CPU has it, else AVX2, else
//     scalar, and each kernel has its own summation order (16 or 8 lane
//     partial sums, then the lanes in order, then the tail; scalar: the
//     dimensions in order).  The same choice and the same orders are made
//     here (GOFANN_FP16_RERANK_KERNEL = auto | scalar | avx2 | avx512), so a
//     distance equals the reference's on the same machine;
//   * streaming (run_highfreq_streaming_rerank, backend_pq.cu:9646-9738):
//     the reference polls per-route mapped status flags; here routes run in
//     chunks on the compute stream, each chunk's shortlist is copied into
//     pinned host memory on a copy stream once an event says the chunk is
//     done, and a host worker pool reranks it while later chunks search.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#if defined(__x86_64__) && !defined(__HIP_DEVICE_COMPILE__)
#include <immintrin.h>
#endif

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <cfloat>
#include <condition_variable>
#include <cstdint>
#include <cstring>
#include <deque>
#include <functional>
#include <mutex>
#include <new>
#include <string>
#include <thread>
#include <vector>

#include "gofann_hip.h"
#include "gofann_internal.hpp"

struct gofann_host_rerank {
    const void* base = nullptr;      // host [samples][dim]
    int elem = GOFANN_ELEM_U8;
    uint32_t dim = 0;
    uint32_t samples = 0;
    const void* queries = nullptr;   // host [queries][dim] (u8 for u8 base, else f32)
    uint32_t threads = 1;
    int fp16_kernel = 0;             // kFp16Scalar / kFp16Avx2 / kFp16Avx512
    std::string error;

    // Worker pool: a queue of jobs, each a half-open route range.
    std::vector<std::thread> workers;
    std::mutex mu;
    std::condition_variable cv;
    std::condition_variable done_cv;
    std::deque<std::function<void()>> jobs;
    size_t pending = 0;
    bool stop = false;

    // Pinned staging of the current streamed search (grows, never shrinks).
    uint32_t* pinned_ids = nullptr;
    size_t pinned_slots = 0;
    hipStream_t copy_stream = nullptr;
    int device = -1;
};

namespace {

float l2_u8(const uint8_t* q, const uint8_t* b, uint32_t dim)
{
    // Every partial sum of squared u8 differences is an integer below 2^24
    // for dim <= 258, so the reference's float loop is exact; the integer
    // form gives the same value and vectorises.
    if (dim <= 258) {
        int32_t acc = 0;
        for (uint32_t d = 0; d < dim; ++d) {
            const int32_t diff = static_cast<int32_t>(q[d]) - static_cast<int32_t>(b[d]);
            acc += diff * diff;
        }
        return static_cast<float>(acc);
    }
    float dist = 0.0f;
    for (uint32_t d = 0; d < dim; ++d) {
        const float diff = static_cast<float>(q[d]) - static_cast<float>(b[d]);
        dist += diff * diff;
    }
    return dist;
}

float l2_f32(const float* q, const float* b, uint32_t dim)
{
    float dist = 0.0f;
    for (uint32_t d = 0; d < dim; ++d) {
        const float diff = q[d] - b[d];
        dist += diff * diff;
    }
    return dist;
}

constexpr int kFp16Scalar = 0;
constexpr int kFp16Avx2 = 1;
constexpr int kFp16Avx512 = 2;

const char* fp16_kernel_name(int k)
{
    return k == kFp16Avx512 ? "avx512" : (k == kFp16Avx2 ? "avx2" : "scalar");
}

// The x86 kernels exist in the host pass only (hipcc also compiles this
// file for the device, where there is no CPU to ask).
#if defined(__x86_64__) && !defined(__HIP_DEVICE_COMPILE__)
#define GOFANN_HOST_X86 1
#else
#define GOFANN_HOST_X86 0
#endif

bool fp16_kernel_supported(int k)
{
    if (k == kFp16Scalar) return true;
#if GOFANN_HOST_X86
    __builtin_cpu_init();
    return __builtin_cpu_supports("f16c") && __builtin_cpu_supports("avx2") &&
           (k != kFp16Avx512 || __builtin_cpu_supports("avx512f"));
#else
    return false;
#endif
}

float l2_f16(const float* q, const __half* b, uint32_t dim)
{
    float dist = 0.0f;
    for (uint32_t d = 0; d < dim; ++d) {
        const float diff = q[d] - __half2float(b[d]);
        dist += diff * diff;
    }
    return dist;
}

#if GOFANN_HOST_X86
// Lane-partial sums: lane l accumulates the squared differences of the
// dimensions d = l (mod lanes) of the whole blocks, in block order; the lane
// sums are then added in lane order, then the tail dimensions in order.
// Products and sums are separate roundings (no fused multiply-add).
__attribute__((target("avx2,f16c"))) float l2_f16_avx2(const float* q, const __half* b,
                                                        uint32_t dim)
{
    __m256 acc = _mm256_setzero_ps();
    const uint16_t* h = reinterpret_cast<const uint16_t*>(b);
    uint32_t d = 0;
    for (; d + 8 <= dim; d += 8) {
        const __m256 x = _mm256_cvtph_ps(_mm_loadu_si128(reinterpret_cast<const __m128i*>(h + d)));
        const __m256 diff = _mm256_sub_ps(_mm256_loadu_ps(q + d), x);
        acc = _mm256_add_ps(acc, _mm256_mul_ps(diff, diff));
    }
    alignas(32) float lane[8];
    _mm256_store_ps(lane, acc);
    float dist = 0.0f;
    for (int l = 0; l < 8; ++l) dist += lane[l];
    for (; d < dim; ++d) {
        const float diff = q[d] - __half2float(b[d]);
        dist += diff * diff;
    }
    return dist;
}

__attribute__((target("avx512f,avx2,f16c"))) float l2_f16_avx512(const float* q,
                                                                   const __half* b,
                                                                   uint32_t dim)
{
    __m512 acc = _mm512_setzero_ps();
    const uint16_t* h = reinterpret_cast<const uint16_t*>(b);
    uint32_t d = 0;
    for (; d + 16 <= dim; d += 16) {
        const __m512 x =
            _mm512_cvtph_ps(_mm256_loadu_si256(reinterpret_cast<const __m256i*>(h + d)));
        const __m512 diff = _mm512_sub_ps(_mm512_loadu_ps(q + d), x);
        acc = _mm512_add_ps(acc, _mm512_mul_ps(diff, diff));
    }
    alignas(64) float lane[16];
    _mm512_store_ps(lane, acc);
    float dist = 0.0f;
    for (int l = 0; l < 16; ++l) dist += lane[l];
    for (; d < dim; ++d) {
        const float diff = q[d] - __half2float(b[d]);
        dist += diff * diff;
    }
    return dist;
}
#endif

float exact_distance(const gofann_host_rerank* hr, uint32_t query, uint32_t sample)
{
    const size_t qo = static_cast<size_t>(query) * hr->dim;
    const size_t bo = static_cast<size_t>(sample) * hr->dim;
    if (hr->elem == GOFANN_ELEM_U8)
        return l2_u8(static_cast<const uint8_t*>(hr->queries) + qo,
                     static_cast<const uint8_t*>(hr->base) + bo, hr->dim);
    if (hr->elem == GOFANN_ELEM_F32)
        return l2_f32(static_cast<const float*>(hr->queries) + qo,
                      static_cast<const float*>(hr->base) + bo, hr->dim);
    const float* qf = static_cast<const float*>(hr->queries) + qo;
    const __half* bh = static_cast<const __half*>(hr->base) + bo;
#if GOFANN_HOST_X86
    if (hr->fp16_kernel == kFp16Avx512) return l2_f16_avx512(qf, bh, hr->dim);
    if (hr->fp16_kernel == kFp16Avx2) return l2_f16_avx2(qf, bh, hr->dim);
#endif
    return l2_f16(qf, bh, hr->dim);
}

bool pair_less(float ad, uint32_t ai, float bd, uint32_t bi)
{
    return ad < bd || (ad == bd && ai < bi);
}

// Routes [r0, r1): exact top-k of each shortlist row.
void rerank_range(const gofann_host_rerank* hr, const uint32_t* shortlist, uint32_t width,
                  const uint32_t* route_query, uint32_t r0, uint32_t r1, uint32_t topk,
                  uint32_t* out_ids, float* out_dists)
{
    std::vector<uint32_t> cand(width);
    std::vector<std::pair<float, uint32_t>> heap;
    heap.reserve(topk + 1);
    const auto worse = [](const std::pair<float, uint32_t>& x, const std::pair<float, uint32_t>& y) {
        return pair_less(x.first, x.second, y.first, y.second);  // max-heap on (dist, id)
    };
    for (uint32_t r = r0; r < r1; ++r) {
        uint32_t n = 0;
        const uint32_t* row = shortlist + static_cast<size_t>(r) * width;
        for (uint32_t i = 0; i < width; ++i)
            if (row[i] != UINT32_MAX && row[i] < hr->samples) cand[n++] = row[i];
        std::sort(cand.begin(), cand.begin() + n);
        n = static_cast<uint32_t>(std::unique(cand.begin(), cand.begin() + n) - cand.begin());
        heap.clear();
        const uint32_t q = route_query[r];
        for (uint32_t i = 0; i < n; ++i) {
            const float d = exact_distance(hr, q, cand[i]);
            if (heap.size() < topk) {
                heap.emplace_back(d, cand[i]);
                std::push_heap(heap.begin(), heap.end(), worse);
            } else if (pair_less(d, cand[i], heap.front().first, heap.front().second)) {
                std::pop_heap(heap.begin(), heap.end(), worse);
                heap.back() = {d, cand[i]};
                std::push_heap(heap.begin(), heap.end(), worse);
            }
        }
        std::sort_heap(heap.begin(), heap.end(), worse);
        for (uint32_t k = 0; k < topk; ++k) {
            const bool have = k < heap.size();
            out_ids[static_cast<size_t>(r) * topk + k] = have ? heap[k].second : UINT32_MAX;
            out_dists[static_cast<size_t>(r) * topk + k] = have ? heap[k].first : FLT_MAX;
        }
    }
}

void worker_loop(gofann_host_rerank* hr)
{
    for (;;) {
        std::function<void()> job;
        {
            std::unique_lock<std::mutex> lk(hr->mu);
            hr->cv.wait(lk, [&] { return hr->stop || !hr->jobs.empty(); });
            if (hr->stop && hr->jobs.empty()) return;
            job = std::move(hr->jobs.front());
            hr->jobs.pop_front();
        }
        job();
        {
            std::lock_guard<std::mutex> lk(hr->mu);
            if (--hr->pending == 0) hr->done_cv.notify_all();
        }
    }
}

// Splits [r0, r1) into jobs of `grain` routes.
void submit_routes(gofann_host_rerank* hr, const uint32_t* shortlist, uint32_t width,
                   const uint32_t* route_query, uint32_t r0, uint32_t r1, uint32_t topk,
                   uint32_t* out_ids, float* out_dists, uint32_t grain)
{
    std::lock_guard<std::mutex> lk(hr->mu);
    for (uint32_t a = r0; a < r1; a += grain) {
        const uint32_t b = std::min(r1, a + grain);
        hr->jobs.emplace_back([=] {
            rerank_range(hr, shortlist, width, route_query, a, b, topk, out_ids, out_dists);
        });
        ++hr->pending;
    }
    hr->cv.notify_all();
}

void wait_all(gofann_host_rerank* hr)
{
    std::unique_lock<std::mutex> lk(hr->mu);
    hr->done_cv.wait(lk, [&] { return hr->pending == 0; });
}

int fail(gofann_host_rerank* hr, int code, const std::string& msg)
{
    hr->error = msg;
    return code;
}

}  // namespace

extern "C" {

int gofann_host_rerank_create(const void* base, int base_elem, uint32_t dim, uint32_t samples,
                              const void* queries, uint32_t threads, gofann_host_rerank** out)
{
    if (out == nullptr) return GOFANN_ERR_INVALID;
    *out = nullptr;
    if (!base || !queries || dim == 0 || base_elem < GOFANN_ELEM_U8 || base_elem > GOFANN_ELEM_F16)
        return GOFANN_ERR_INVALID;
    gofann_host_rerank* hr = new (std::nothrow) gofann_host_rerank();
    if (hr == nullptr) return GOFANN_ERR_NOMEM;
    hr->base = base;
    hr->elem = base_elem;
    hr->dim = dim;
    hr->samples = samples;
    hr->queries = queries;
    hr->threads = threads == 0 ? 1 : threads;
    hr->fp16_kernel = kFp16Scalar;
    if (base_elem == GOFANN_ELEM_F16) {
        // the reference's fp16 kernel choice (fp16_l2::select), read only
        // for fp16 rows as the reference reads it only when it opens an fp16
        // source (dataloader.cpp:2132); the reference's own variable name is
        // taken when this library's is unset
        const char* env = std::getenv("GOFANN_FP16_RERANK_KERNEL");
        if (env == nullptr) env = std::getenv("GO_FANN_FP16_RERANK_KERNEL");
        const std::string req = env ? env : "auto";
        int k;
        if (req.empty() || req == "auto") {
            k = fp16_kernel_supported(kFp16Avx512)
                    ? kFp16Avx512
                    : (fp16_kernel_supported(kFp16Avx2) ? kFp16Avx2 : kFp16Scalar);
        } else if (req == "scalar") {
            k = kFp16Scalar;
        } else if (req == "avx2") {
            k = kFp16Avx2;
        } else if (req == "avx512") {
            k = kFp16Avx512;
        } else {
            delete hr;
            return GOFANN_ERR_INVALID;  // unknown kernel name
        }
        if (!fp16_kernel_supported(k)) {
            delete hr;
            return GOFANN_ERR_UNSUPPORTED;  // the CPU lacks the requested ISA
        }
        hr->fp16_kernel = k;
    }
    try {
        for (uint32_t t = 0; t < hr->threads; ++t) hr->workers.emplace_back(worker_loop, hr);
    } catch (...) {
        {
            std::lock_guard<std::mutex> lk(hr->mu);
            hr->stop = true;
        }
        hr->cv.notify_all();
        for (auto& w : hr->workers) w.join();
        delete hr;
        return GOFANN_ERR_NOMEM;
    }
    *out = hr;
    return GOFANN_OK;
}

void gofann_host_rerank_destroy(gofann_host_rerank* hr)
{
    if (hr == nullptr) return;
    {
        std::lock_guard<std::mutex> lk(hr->mu);
        hr->stop = true;
    }
    hr->cv.notify_all();
    for (auto& w : hr->workers) w.join();
    if (hr->device >= 0) {
        (void)hipSetDevice(hr->device);
        if (hr->copy_stream) (void)hipStreamDestroy(hr->copy_stream);
        if (hr->pinned_ids) (void)hipHostFree(hr->pinned_ids);
    }
    delete hr;
}

const char* gofann_host_rerank_last_error(const gofann_host_rerank* hr)
{
    return hr ? hr->error.c_str() : "null rerank handle";
}

const char* gofann_host_rerank_fp16_kernel(const gofann_host_rerank* hr)
{
    return hr ? fp16_kernel_name(hr->fp16_kernel) : "";
}

int gofann_host_rerank_routes(gofann_host_rerank* hr, const uint32_t* shortlist, uint32_t width,
                              const uint32_t* route_query, uint32_t routes, uint32_t topk,
                              uint32_t* out_ids, float* out_dists)
{
    if (hr == nullptr) return GOFANN_ERR_INVALID;
    if (routes == 0) return GOFANN_OK;
    if (!shortlist || !route_query || !out_ids || !out_dists || width == 0 || topk == 0)
        return fail(hr, GOFANN_ERR_INVALID, "rerank arrays missing or empty width / topk");
    try {
        const uint32_t grain = std::max<uint32_t>(16, routes / (hr->threads * 8) + 1);
        submit_routes(hr, shortlist, width, route_query, 0, routes, topk, out_ids, out_dists,
                      grain);
        wait_all(hr);
    } catch (const std::exception& e) {
        return fail(hr, GOFANN_ERR_NOMEM, e.what());
    }
    return GOFANN_OK;
}

int gofann_pq_search_host_rerank(gofann_ctx* c, gofann_host_rerank* hr, const gofann_pq_view* pq,
                                 const void* queries, int query_elem,
                                 const gofann_graph_view* graph,
                                 const gofann_predicate_view* predicate,
                                 const gofann_routes* routes, const gofann_search_params* params,
                                 const uint32_t* route_query_host, uint32_t chunk_routes,
                                 uint32_t topk, uint32_t* out_ids, float* out_dists,
                                 gofann_route_stats* stats)
{
    if (c == nullptr || hr == nullptr) return GOFANN_ERR_INVALID;
    auto* ctx = reinterpret_cast<gofann::Context*>(c);
    if (!routes || !params || !route_query_host || !out_ids || !out_dists || topk == 0)
        return ctx->fail(GOFANN_ERR_INVALID, "host rerank search arguments missing");
    if (routes->launch_order != nullptr)
        return ctx->fail(GOFANN_ERR_INVALID, "streamed search runs routes in id order (no launch_order)");
    const uint32_t n = routes->count;
    const uint32_t W = static_cast<uint32_t>(params->result_width);
    if (n == 0) return GOFANN_OK;
    if (chunk_routes == 0) chunk_routes = n;
    try {
        // Device shortlist + pinned host staging.
        const size_t slots = static_cast<size_t>(n) * W;
        void* dbuf = ctx->scratch(gofann::Context::kScratchMisc, slots * 8);
        if (dbuf == nullptr) return ctx->fail(GOFANN_ERR_NOMEM, "device shortlist");
        uint32_t* d_ids = static_cast<uint32_t*>(dbuf);
        float* d_dists = reinterpret_cast<float*>(d_ids + slots);
        if (hr->device != ctx->device) {
            if (hr->copy_stream) (void)hipStreamDestroy(hr->copy_stream);
            if (hr->pinned_ids) (void)hipHostFree(hr->pinned_ids);
            hr->copy_stream = nullptr;
            hr->pinned_ids = nullptr;
            hr->pinned_slots = 0;
            hr->device = ctx->device;
            if (hipStreamCreateWithFlags(&hr->copy_stream, hipStreamNonBlocking) != hipSuccess)
                return ctx->fail_hip("copy stream");
        }
        if (hr->pinned_slots < slots) {
            if (hr->pinned_ids) (void)hipHostFree(hr->pinned_ids);
            hr->pinned_ids = nullptr;
            hr->pinned_slots = 0;
            if (hipHostMalloc(reinterpret_cast<void**>(&hr->pinned_ids), slots * 4,
                              hipHostMallocDefault) != hipSuccess)
                return ctx->fail_hip("pinned shortlist");
            hr->pinned_slots = slots;
        }
        const uint32_t chunks = (n + chunk_routes - 1) / chunk_routes;
        std::vector<hipEvent_t> searched(chunks, nullptr), copied(chunks, nullptr);
        auto release = [&] {
            for (auto& e : searched)
                if (e) (void)hipEventDestroy(e);
            for (auto& e : copied)
                if (e) (void)hipEventDestroy(e);
        };
        for (uint32_t k = 0; k < chunks; ++k) {
            if (hipEventCreateWithFlags(&searched[k], hipEventDisableTiming) != hipSuccess ||
                hipEventCreateWithFlags(&copied[k], hipEventDisableTiming) != hipSuccess) {
                release();
                return ctx->fail_hip("events");
            }
        }
        // Identity launch order per chunk: a device array of route ids.
        void* obuf = ctx->scratch(gofann::Context::kScratchSegments, static_cast<size_t>(n) * 4);
        if (obuf == nullptr) {
            release();
            return ctx->fail(GOFANN_ERR_NOMEM, "launch order");
        }
        std::vector<uint32_t> order(n);
        for (uint32_t i = 0; i < n; ++i) order[i] = i;
        if (hipMemcpyAsync(obuf, order.data(), static_cast<size_t>(n) * 4, hipMemcpyHostToDevice,
                           ctx->stream) != hipSuccess ||
            hipStreamSynchronize(ctx->stream) != hipSuccess) {
            release();
            return ctx->fail_hip("launch order upload");
        }
        const uint32_t* d_order = static_cast<const uint32_t*>(obuf);
        // Enqueue every chunk: search on the compute stream, copy on the
        // copy stream after the chunk's event.
        for (uint32_t k = 0; k < chunks; ++k) {
            const uint32_t r0 = k * chunk_routes;
            const uint32_t r1 = std::min(n, r0 + chunk_routes);
            gofann_routes sub = *routes;
            sub.launch_order = d_order + r0;
            sub.count = r1 - r0;
            int rc = gofann::pq_search(ctx, pq, queries, query_elem, graph, predicate, &sub, params,
                                       d_ids, d_dists, stats);
            if (rc != GOFANN_OK) {
                (void)hipStreamSynchronize(ctx->stream);
                release();
                return rc;
            }
            if (hipEventRecord(searched[k], ctx->stream) != hipSuccess ||
                hipStreamWaitEvent(hr->copy_stream, searched[k], 0) != hipSuccess ||
                hipMemcpyAsync(hr->pinned_ids + static_cast<size_t>(r0) * W,
                               d_ids + static_cast<size_t>(r0) * W,
                               static_cast<size_t>(r1 - r0) * W * 4, hipMemcpyDeviceToHost,
                               hr->copy_stream) != hipSuccess ||
                hipEventRecord(copied[k], hr->copy_stream) != hipSuccess) {
                (void)hipStreamSynchronize(ctx->stream);
                release();
                return ctx->fail_hip("chunk hand-off");
            }
        }
        // Host side: rerank each chunk as soon as its copy lands.
        const uint32_t grain = std::max<uint32_t>(16, chunk_routes / (hr->threads * 4) + 1);
        for (uint32_t k = 0; k < chunks; ++k) {
            if (hipEventSynchronize(copied[k]) != hipSuccess) {
                wait_all(hr);
                release();
                return ctx->fail_hip("chunk copy");
            }
            const uint32_t r0 = k * chunk_routes;
            const uint32_t r1 = std::min(n, r0 + chunk_routes);
            submit_routes(hr, hr->pinned_ids, W, route_query_host, r0, r1, topk, out_ids,
                          out_dists, grain);
        }
        wait_all(hr);
        release();
    } catch (const std::exception& e) {
        wait_all(hr);
        return ctx->fail(GOFANN_ERR_NOMEM, e.what());
    }
    return GOFANN_OK;
}

// Route -> original query merge on the host (merge_route_results_to_original,
// src/search/rabitq/rabitq_lowfreq_merge.h:709-815): per query the minimum
// distance per sample over its routes, (distance, id) order, first topk.
int gofann_host_merge_routes(const uint32_t* query_route_offsets, const uint32_t* query_routes,
                             const uint32_t* route_ids, const float* route_dists, uint32_t width,
                             uint32_t queries, uint32_t topk, uint32_t* out_ids, float* out_dists)
{
    if (queries == 0) return GOFANN_OK;
    if (!query_route_offsets || !query_routes || !route_ids || !route_dists || !out_ids ||
        !out_dists || topk == 0)
        return GOFANN_ERR_INVALID;
    std::vector<std::pair<float, uint32_t>> all;
    for (uint32_t q = 0; q < queries; ++q) {
        all.clear();
        for (uint32_t k = query_route_offsets[q]; k < query_route_offsets[q + 1]; ++k) {
            const uint32_t r = query_routes[k];
            for (uint32_t i = 0; i < width; ++i) {
                const uint32_t id = route_ids[static_cast<size_t>(r) * width + i];
                if (id == UINT32_MAX) continue;
                all.emplace_back(route_dists[static_cast<size_t>(r) * width + i], id);
            }
        }
        // minimum distance per sample, then (distance, id) order
        std::sort(all.begin(), all.end(), [](const auto& a, const auto& b) {
            return a.second < b.second || (a.second == b.second && a.first < b.first);
        });
        size_t m = 0;
        for (size_t i = 0; i < all.size(); ++i)
            if (i == 0 || all[i].second != all[i - 1].second) all[m++] = all[i];
        all.resize(m);
        std::sort(all.begin(), all.end(), [](const auto& a, const auto& b) {
            return pair_less(a.first, a.second, b.first, b.second);
        });
        for (uint32_t k = 0; k < topk; ++k) {
            const bool have = k < all.size();
            out_ids[static_cast<size_t>(q) * topk + k] = have ? all[k].second : UINT32_MAX;
            out_dists[static_cast<size_t>(q) * topk + k] = have ? all[k].first : FLT_MAX;
        }
    }
    return GOFANN_OK;
}

}  // extern "C"
