// exact_route.hip -- the full-GPU exact-distance route on gfx950.
//
// Reference: run_full_gpu_highfreq_route (src/search/full_gpu/
// backend_full_gpu.cu:1682-2042) launched by full_gpu_highfreq_kernel
// (:2045-2122).  A beam search whose frontier is keyed by the exact squared
// L2 distance of u8 vectors (l2_distance_device :1199-1244: an integer, here
// |b|^2 + |q|^2 - 2 b.q in u32 through v_dot4_u32_u8, converted to float),
// with the route filter applied to every expanded node and a sorted best-k
// with sample dedup (insert_best_result :1342-1375).
//
// Per step (one wave64 per route):
//  * lane 0: filter of the expanded node (row mask & route bits, every active
//    legacy range, the route predicate when enabled) and its best-k insert;
//  * lane j: adjacency entry j of the node (prefetched at pickup), its
//    visited test, group bound and sample id, then the exact distance of its
//    own base row -- every lane streams a different row, 16 bytes a load;
//  * candidates that cannot enter a full frontier are dropped in parallel,
//    the rest are admitted by lane 0 in adjacency order (smmh2 insert,
//    pop_max at Q+2), and the admitted rows enter the visited set;
//  * pickup of the next entry and the reference's early-stop rule (skipped on
//    the first transition): adaptive mode resets on an improved best-k,
//    otherwise a full best-k that the next entry cannot improve counts
//    towards early_stop_reached(mode, hits, finish, Q, expanded, passed, K).
//
// A route with no group rows, an invalid seed, or a seed sample past the
// base emits padding (UINT32_MAX / FLT_MAX) and zero steps.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>

#include "device_common.hpp"
#include "gofann_internal.hpp"

namespace gofann {

constexpr int kExactMaxTopk = 10;  // defaults::max_topk

struct ExactArgs {
    gofann_graph_view graph;
    const uint32_t* label_size;
    gofann_predicate_view pred;
    gofann_routes routes;
    const uint8_t* base;
    const uint8_t* queries;
    uint32_t dim;
    uint32_t samples;
    gofann_exact_params params;
    uint32_t* out_ids;
    float* out_dists;
    gofann_route_stats* stats;
    uint32_t* hash_global;
    uint32_t off_frontier;
    uint32_t off_hash;
};

// Squared L2 of a u8 row against the query held in LDS (q, |q|^2).
__device__ __forceinline__ uint32_t l2_u8_row(const uint8_t* row, const uint32_t* q,
                                              uint32_t dim, uint32_t qnorm)
{
    uint32_t nb = 0, dot = 0;
    if ((dim & 15u) == 0) {
        const uint4* r4 = reinterpret_cast<const uint4*>(row);
        const uint4* q4 = reinterpret_cast<const uint4*>(q);
        for (uint32_t i = 0; i < dim / 16; ++i) {
            const uint4 b = r4[i];
            const uint4 w = q4[i];
            nb = __builtin_amdgcn_udot4(b.x, b.x, nb, false);
            nb = __builtin_amdgcn_udot4(b.y, b.y, nb, false);
            nb = __builtin_amdgcn_udot4(b.z, b.z, nb, false);
            nb = __builtin_amdgcn_udot4(b.w, b.w, nb, false);
            dot = __builtin_amdgcn_udot4(b.x, w.x, dot, false);
            dot = __builtin_amdgcn_udot4(b.y, w.y, dot, false);
            dot = __builtin_amdgcn_udot4(b.z, w.z, dot, false);
            dot = __builtin_amdgcn_udot4(b.w, w.w, dot, false);
        }
        return nb + qnorm - 2u * dot;
    }
    if ((dim & 3u) == 0) {
        const uint32_t* r1 = reinterpret_cast<const uint32_t*>(row);
        for (uint32_t i = 0; i < dim / 4; ++i) {
            const uint32_t b = r1[i];
            nb = __builtin_amdgcn_udot4(b, b, nb, false);
            dot = __builtin_amdgcn_udot4(b, q[i], dot, false);
        }
        return nb + qnorm - 2u * dot;
    }
    const uint8_t* qb = reinterpret_cast<const uint8_t*>(q);
    uint32_t acc = 0;
    for (uint32_t d = 0; d < dim; ++d) {
        const int diff = static_cast<int>(row[d]) - static_cast<int>(qb[d]);
        acc += static_cast<uint32_t>(diff * diff);
    }
    return acc;
}

__device__ __forceinline__ bool better(float ld, uint32_t lid, float rd, uint32_t rid)
{
    return ld < rd || (ld == rd && lid < rid);
}

// insert_best_result on LDS arrays (lane 0).
__device__ __forceinline__ bool best_insert(float d, uint32_t id, uint32_t K, float* bd,
                                            uint32_t* bi, uint32_t& size)
{
    bool changed = false;
    for (uint32_t i = 0; i < size; ++i) {
        if (bi[i] != id) continue;
        if (d >= bd[i]) return false;
        for (uint32_t j = i; j + 1 < size; ++j) {
            bd[j] = bd[j + 1];
            bi[j] = bi[j + 1];
        }
        --size;
        changed = true;
        break;
    }
    if (size == K && !better(d, id, bd[K - 1], bi[K - 1])) return changed;
    uint32_t pos = size;
    if (size < K)
        ++size;
    else
        pos = K - 1;
    while (pos > 0 && better(d, id, bd[pos - 1], bi[pos - 1])) {
        bd[pos] = bd[pos - 1];
        bi[pos] = bi[pos - 1];
        --pos;
    }
    bd[pos] = d;
    bi[pos] = id;
    return true;
}

// Lane j: adjacency entry j of the node `e` and, when the graph carries
// them, its sample id.
__device__ __forceinline__ void load_adjacency(const gofann_graph_view& g, uint32_t off,
                                               uint32_t degree, const Entry& e, int lane,
                                               uint32_t& adj, uint32_t& nsamp)
{
    const size_t row = static_cast<size_t>(off + (e.second & ~kPoolUsed)) * g.degree;
    const bool in_row = static_cast<uint32_t>(lane) < degree;
    adj = in_row ? g.graph[row + lane] : UINT32_MAX;
    nsamp = (in_row && g.neighbor_samples) ? g.neighbor_samples[row + lane] : 0u;
}

template <int kVisited>
__global__ __launch_bounds__(64) void exact_route_kernel(ExactArgs a)
{
    extern __shared__ __align__(16) unsigned char lds[];
    __shared__ uint32_t s_row[kMaxDegree];
    __shared__ uint32_t s_samp[kMaxDegree];
    __shared__ float s_dist[kMaxDegree];
    __shared__ float s_bd[kExactMaxTopk];
    __shared__ uint32_t s_bi[kExactMaxTopk];
    __shared__ uint64_t s_adm;

    const int lane = static_cast<int>(threadIdx.x);
    const uint32_t slot = xcd_slot(blockIdx.x, gridDim.x);
    if (slot >= a.routes.count) return;
    const uint32_t route = a.routes.launch_order ? a.routes.launch_order[slot] : slot;
    const int Q = a.params.queue_limit;
    const uint32_t K = static_cast<uint32_t>(a.params.topk);
    const int mode = a.params.early_stop_mode;

    uint32_t* qw = reinterpret_cast<uint32_t*>(lds);
    Entry* frontier = reinterpret_cast<Entry*>(lds + a.off_frontier);
    VisitedSet<kVisited> visited;

    const uint32_t group = a.routes.route_group[route];
    const uint32_t seed = a.routes.route_start[route];
    const uint32_t gsize = a.label_size ? a.label_size[group] : UINT32_MAX;
    const uint32_t off = a.graph.label_offset[group];
    const uint64_t qfbit = a.routes.query_filter_bits ? a.routes.query_filter_bits[route] : ~0ULL;
    const uint32_t active = count_active_ranges(a.routes.range_modes, route, a.routes.range_count);
    const bool enabled = pred_enabled(a.pred, route);
    const uint32_t degree = a.graph.degree < static_cast<uint32_t>(kMaxDegree)
                                ? a.graph.degree
                                : static_cast<uint32_t>(kMaxDegree);

    // Query row into LDS (zero-padded to 16 bytes) and |q|^2.
    const uint8_t* qrow = a.queries + static_cast<size_t>(a.routes.route_query[route]) * a.dim;
    const uint32_t qwords = (a.dim + 15u) / 16u * 4u;
    uint32_t qn = 0;
    for (uint32_t w = lane; w < qwords; w += kWave) {
        uint32_t v = 0;
        for (uint32_t b = 0; b < 4; ++b) {
            const uint32_t d = w * 4 + b;
            if (d < a.dim) v |= static_cast<uint32_t>(qrow[d]) << (8 * b);
        }
        qw[w] = v;
        qn = __builtin_amdgcn_udot4(v, v, qn, false);
    }
    for (int o = 32; o > 0; o >>= 1) qn += static_cast<uint32_t>(__shfl_xor(static_cast<int>(qn), o, kWave));
    visited.init(reinterpret_cast<uint32_t*>(lds + a.off_hash),
                 a.hash_global ? a.hash_global + static_cast<size_t>(slot) * kHashCapacity : nullptr,
                 lane);
    if (lane < kExactMaxTopk) {
        s_bd[lane] = FLT_MAX;
        s_bi[lane] = UINT32_MAX;
    }
    __threadfence_block();
    __syncthreads();

    gofann_route_stats st{0, 0, 0, 0, 0, 0, 0, 0};
    PredCounters pc{0, 0};
    uint32_t bsize = 0;
    int heap_size = 1;
    bool done = false;
    const Entry sentinel = {FLT_MAX, UINT32_MAX, FLT_MAX, UINT32_MAX};
    Entry now = sentinel, next = sentinel;

    // Seed (:1793-1850).
    if (gsize == 0 || seed == UINT32_MAX || seed >= gsize) {
        done = true;
    } else {
        const uint32_t s0 = a.graph.row_to_sample[off + seed];
        if (s0 < a.samples) {
            if (lane == 0) {
                const float d0 = static_cast<float>(
                    l2_u8_row(a.base + static_cast<size_t>(s0) * a.dim, qw, a.dim, qn));
                const Entry kp = {d0, seed, d0, s0};
                smmh_insert(frontier, heap_size, kp);
                (void)visited.add_serial(seed, 0);
            }
            visited.count = 1;
            st.scored = 1;
            heap_size = bcast0(heap_size);
        } else {
            done = true;
        }
    }
    __threadfence_block();
    __syncthreads();
    if (!done && !pickup(frontier, heap_size, now, lane)) done = true;
    if (done) st.exhausted = 1;

    // Adjacency of the node about to be expanded, loaded at pickup time.
    uint32_t adj = UINT32_MAX, nsamp = 0;
    if (!done) load_adjacency(a.graph, off, degree, now, lane, adj, nsamp);

    uint32_t steps = 0, finished = 0;
    bool first_step = true;
    while (!done) {
        if (a.params.max_steps != 0 && steps >= static_cast<uint32_t>(a.params.max_steps)) break;

        // Neighbour tests first (loads only), then the expanded node's filter.
        const bool fresh = adj != UINT32_MAX && adj < gsize && !visited.test(adj);
        uint32_t samp = 0;
        if (fresh) samp = a.graph.neighbor_samples ? nsamp : a.graph.row_to_sample[off + adj];
        const bool keep = fresh && samp < a.samples;

        int improved = 0;
        if (lane == 0) {
            const uint32_t grow = off + (now.second & ~kPoolUsed);
            const uint32_t sample = now.sample;
            const uint64_t rmask =
                a.routes.row_filter_mask ? a.routes.row_filter_mask[grow] : ~0ULL;
            bool pass = (rmask & qfbit) != 0;
            if (pass && active != 0) pass = count_matching_ranges(a.routes, route, sample) == active;
            if (pass && enabled) pass = pred_matches(a.pred, route, sample, pc);
            ++st.expanded;
            if (pass) {
                ++st.passed;
                improved = best_insert(now.first, sample, K, s_bd, s_bi, bsize) ? 1 : 0;
            }
        }
        ++steps;

        const float dist = keep ? static_cast<float>(l2_u8_row(
                                      a.base + static_cast<size_t>(samp) * a.dim, qw, a.dim, qn))
                                : FLT_MAX;
        st.scored += __popcll(ballot(keep));

        // Drop what cannot enter a full frontier (its maximum only falls
        // during the step), compact the rest in adjacency order.
        const bool full = heap_size > 2 && heap_size >= Q + 1;
        const float thr = full ? frontier[2].first : 0.0f;
        const bool cand = keep && !(full && thr < dist);
        const uint64_t cand_mask = ballot(cand);
        const int n_cand = __popcll(cand_mask);
        const uint32_t pos = lanes_below(cand_mask);
        if (cand) {
            s_row[pos] = adj;
            s_samp[pos] = samp;
            s_dist[pos] = dist;
        }
        __syncthreads();
        if (lane == 0) {
            uint64_t adm = 0;
            for (int i = 0; i < n_cand; ++i) {
                const Entry kp = {s_dist[i], s_row[i], s_dist[i], s_samp[i]};
                if (heap_size > 2 && heap_size >= Q + 1 && frontier[2].first < kp.first) continue;
                smmh_insert(frontier, heap_size, kp);
                adm |= 1ull << i;
                ++st.admitted;
                if (heap_size >= Q + 2) smmh_pop_max(frontier, heap_size);
            }
            s_adm = adm;
        }
        heap_size = bcast0(heap_size);
        __syncthreads();
        const uint64_t adm = s_adm;
        const uint32_t n_adm = static_cast<uint32_t>(__popcll(adm));
        visited.reserve(n_adm, lane);
        if (visited.count + n_adm <= kHashCapacity) {
            const bool mine = cand && ((adm >> pos) & 1ull);
            const int ins = mine ? visited.add_parallel(adj) : 0;
            visited.count += static_cast<uint32_t>(__popcll(ballot(ins != 0)));
        } else {
            uint32_t added = 0;
            if (lane == 0) {
                for (int i = 0; i < n_cand; ++i)
                    if ((adm >> i) & 1ull)
                        added += static_cast<uint32_t>(visited.add_serial(s_row[i], added));
            }
            visited.count += bcast0u(added);
        }
        __threadfence_block();
        __syncthreads();

        // Pickup and early stop (:1985-2030).
        if (!pickup(frontier, heap_size, next, lane)) {
            st.exhausted = 1;
            break;
        }
        load_adjacency(a.graph, off, degree, next, lane, adj, nsamp);
        int stop = 0;
        if (lane == 0 && !first_step) {
            if (mode == GOFANN_EARLY_STOP_ADAPTIVE && improved) {
                finished = 0;
            } else if (bsize == K && !better(next.first, next.sample, s_bd[K - 1], s_bi[K - 1])) {
                ++finished;
                stop = early_stop_reached(mode, static_cast<int>(finished), a.params.finish_limit,
                                          Q, st.expanded, st.passed, static_cast<int>(K))
                           ? 1
                           : 0;
            } else {
                finished = 0;
            }
        }
        if (bcast0(stop)) break;
        now = next;
        first_step = false;
    }

    __syncthreads();
    uint32_t* oid = a.out_ids + static_cast<size_t>(route) * K;
    float* od = a.out_dists + static_cast<size_t>(route) * K;
    const uint32_t nb = bcast0u(bsize);
    if (static_cast<uint32_t>(lane) < K) {
        oid[lane] = static_cast<uint32_t>(lane) < nb ? s_bi[lane] : UINT32_MAX;
        od[lane] = static_cast<uint32_t>(lane) < nb ? s_bd[lane] : FLT_MAX;
    }
    const int pred_rows = wave_sum(static_cast<int>(pc.rows));
    const int pred_labels = wave_sum(static_cast<int>(pc.labels));
    if (lane == 0 && a.stats) {
        st.steps = static_cast<int32_t>(steps);
        st.pred_rows = pred_rows;
        st.pred_labels = pred_labels;
        a.stats[route] = st;
    }
}

namespace {

inline uint32_t align16u(uint32_t x) { return (x + 15u) & ~15u; }

template <int kVisited>
int resident(Context* ctx, uint32_t lds)
{
    if (lds > static_cast<uint32_t>(ctx->lds_per_block)) return 0;
    const void* k = reinterpret_cast<const void*>(exact_route_kernel<kVisited>);
    if (hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(lds)) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    int blocks = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, k, kWave, lds) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return blocks;
}

}  // namespace

int exact_search(Context* ctx, const void* base, int base_elem, uint32_t dim, uint32_t samples,
                 const void* queries, const gofann_graph_view* g, const uint32_t* label_size,
                 const gofann_predicate_view* pred, const gofann_routes* r,
                 const gofann_exact_params* p, uint32_t* out_ids, float* out_dists,
                 gofann_route_stats* stats)
{
    if (!g || !r || !p) return ctx->fail(GOFANN_ERR_INVALID, "null view");
    if (base_elem != GOFANN_ELEM_U8)
        return ctx->fail(GOFANN_ERR_UNSUPPORTED, "the exact route takes u8 vectors");
    if (!base || !queries || dim == 0)
        return ctx->fail(GOFANN_ERR_INVALID, "exact route vectors missing");
    if (dim > 65536) return ctx->fail(GOFANN_ERR_INVALID, "dim must be <= 65536 (u32 distances)");
    if (p->queue_limit < 2 || p->queue_limit > 1024)
        return ctx->fail(GOFANN_ERR_INVALID, "queue_limit must be in [2, 1024]");
    if (p->topk < 1 || p->topk > kExactMaxTopk)
        return ctx->fail(GOFANN_ERR_INVALID, "topk must be in [1, 10]");
    if (p->early_stop_mode < 0 || p->early_stop_mode > 2)
        return ctx->fail(GOFANN_ERR_INVALID, "unknown early stop mode");
    if (p->hash_mode < GOFANN_PLACE_AUTO || p->hash_mode > GOFANN_PLACE_SPILL)
        return ctx->fail(GOFANN_ERR_INVALID, "hash_mode in [0, 3]");
    if (!g->graph || !g->row_to_sample || !g->label_offset || g->degree == 0)
        return ctx->fail(GOFANN_ERR_INVALID, "graph view incomplete");
    if (r->count == 0) return GOFANN_OK;
    if (!r->route_query || !r->route_group || !r->route_start || !out_ids || !out_dists)
        return ctx->fail(GOFANN_ERR_INVALID, "route arrays or outputs missing");
    if ((reinterpret_cast<uintptr_t>(base) & 15u) != 0)
        return ctx->fail(GOFANN_ERR_INVALID, "base must be 16-byte aligned");

    ExactArgs a;
    a.graph = *g;
    a.label_size = label_size;
    a.pred = pred ? *pred : gofann_predicate_view{};
    a.routes = *r;
    a.base = static_cast<const uint8_t*>(base);
    a.queries = static_cast<const uint8_t*>(queries);
    a.dim = dim;
    a.samples = samples;
    a.params = *p;
    a.out_ids = out_ids;
    a.out_dists = out_dists;
    a.stats = stats;
    a.off_frontier = align16u((dim + 15u) / 16u * 16u);
    a.off_hash = align16u(a.off_frontier + static_cast<uint32_t>(p->queue_limit + 2) * sizeof(Entry));
    const uint32_t lds_full = a.off_hash + kHashCapacity * 4u;
    const uint32_t lds_spill = a.off_hash + kSpillSlots * 4u;
    const uint32_t lds_glob = a.off_hash;
    const int rf = resident<kVisitedLds>(ctx, lds_full);
    const int rs = resident<kVisitedSpill>(ctx, lds_spill);
    const int rg = resident<kVisitedGlobal>(ctx, lds_glob);
    int mode = kVisitedLds;
    int res = rf;
    if (p->hash_mode == GOFANN_PLACE_GLOBAL) {
        mode = kVisitedGlobal;
        res = rg;
    } else if (p->hash_mode == GOFANN_PLACE_SPILL) {
        mode = kVisitedSpill;
        res = rs;
    } else if (p->hash_mode == GOFANN_PLACE_AUTO) {
        if (rs > res) {
            mode = kVisitedSpill;
            res = rs;
        }
        if (rg > res) {
            mode = kVisitedGlobal;
            res = rg;
        }
    }
    if (res <= 0)
        return ctx->fail(GOFANN_ERR_UNSUPPORTED, "per-route LDS state exceeds the workgroup limit");
    a.hash_global = nullptr;
    if (mode != kVisitedLds) {
        const size_t need = static_cast<size_t>(r->count) * kHashCapacity * sizeof(uint32_t);
        a.hash_global = static_cast<uint32_t*>(ctx->scratch(Context::kScratchHash, need));
        if (!a.hash_global) return ctx->fail(GOFANN_ERR_NOMEM, "visited set scratch");
    }
    const uint32_t lds = mode == kVisitedLds ? lds_full : (mode == kVisitedSpill ? lds_spill : lds_glob);
    const dim3 grid(r->count), block(kWave);
    if (mode == kVisitedLds)
        hipLaunchKernelGGL(exact_route_kernel<kVisitedLds>, grid, block, lds, ctx->stream, a);
    else if (mode == kVisitedSpill)
        hipLaunchKernelGGL(exact_route_kernel<kVisitedSpill>, grid, block, lds, ctx->stream, a);
    else
        hipLaunchKernelGGL(exact_route_kernel<kVisitedGlobal>, grid, block, lds, ctx->stream, a);
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("exact route launch");
    ctx->last_table_in_lds = 0;
    ctx->last_hash_in_lds = mode == kVisitedGlobal ? 0 : (mode == kVisitedLds ? 1 : 2);
    ctx->last_lds_bytes = static_cast<int>(lds);
    ctx->last_resident = res;
    return GOFANN_OK;
}

}  // namespace gofann
