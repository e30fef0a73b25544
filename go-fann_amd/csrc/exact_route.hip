// exact_route.hip -- the full-GPU exact-distance route on gfx950.
//
// Reference: run_full_gpu_highfreq_route (src/search/full_gpu/
// backend_full_gpu.cu:1682-2042) launched by full_gpu_highfreq_kernel
// (:2045-2122).  A beam search whose frontier is keyed by the exact squared
// L2 distance (u8 vectors: l2_distance_device :1199-1244, an integer, here
// |b|^2 + |q|^2 - 2 b.q in u32 through v_dot4_u32_u8, converted to float;
// f32 and f16 vectors: :1107-1160, in that function's warp order, with the
// query in LDS as f32), with the route filter applied to every expanded
// node and a sorted best-k with sample dedup (insert_best_result
// :1342-1375).
//
// Per step (one wave64 per route):
//  * lane 0: filter of the expanded node (row mask & route bits, every active
//    legacy range, the route predicate when enabled) and its best-k insert;
//  * lane j: adjacency entry j of the node (prefetched at pickup), its
//    visited test, group bound and sample id, then (u8) the exact distance
//    of its own base row -- every lane streams a different row, 16 bytes a
//    load; float rows are scored in the reference's warp order, 16 at a
//    time (one per quad of lanes) or, past 4 KB a row, 2 at a time (one per
//    32-lane half) (exact_dist.hpp);
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
#include <mutex>
#include <string>

#include "device_common.hpp"
#include "exact_dist.hpp"
#include "gofann_internal.hpp"

// Visited-set slabs of gofann_exact_search_noalloc: a fixed device array in
// place of context scratch, for callers that cannot allocate.  Each GPU the
// library runs on holds its own copy until the process ends.  Host code never
// passes this name to a kernel (on the host it is only a stand-in for the
// symbol); it uses the per-device address that hipGetSymbolAddress returned.
static __device__ __align__(256) uint32_t scratch[GOFANN_EXACT_NOALLOC_MAX_ROUTES * 4096u];

namespace gofann {

namespace {
constexpr int kNoAllocMaxDevices = 64;
std::mutex g_noalloc_mutex;
uint32_t* g_noalloc_slab[kNoAllocMaxDevices] = {};
std::string g_noalloc_error[kNoAllocMaxDevices];
}  // namespace

// Looks up this device's copy of `scratch` once (gofann_create calls it with
// the context's device current).  A failure is kept and reported by the
// no-alloc entry point; the other entry points do not need the array.
void noalloc_setup(int device)
{
    if (device < 0 || device >= kNoAllocMaxDevices) return;
    std::lock_guard<std::mutex> lock(g_noalloc_mutex);
    if (g_noalloc_slab[device] != nullptr) return;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
        (void)hipGetLastError();
        g_noalloc_error[device] = std::string("hipGetSymbolAddress(scratch): ") +
                                  hipGetErrorString(e);
        return;
    }
    g_noalloc_slab[device] = static_cast<uint32_t*>(p);
    g_noalloc_error[device].clear();
}

constexpr int kExactMaxTopk = 10;  // defaults::max_topk

// 1: rows of 128, 192 or 256 bytes use kernels with the row length fixed
// at compile time (all of a row's loads in flight at once, at the price of
// about 40 more VGPRs and so fewer resident routes); 0 keeps the loop.
#ifndef GOFANN_EXACT_FIXED_ROWS
#define GOFANN_EXACT_FIXED_ROWS 0
#endif

// Minimum waves per SIMD the u8 kernels are compiled for (register budget).
// 6 holds them to 80 VGPRs, 24 routes per CU, without spills (the lane id is
// opaque per step).  At C2, Q = 80: 46.1 ms, against 49.0 at 5 waves and
// 54.1 at 7 (the visited table leaves LDS).  The f32 / f16 kernels (eight
// partial sums and two 16-byte loads per lane) take 5: at 6 they spill.
#ifndef GOFANN_EXACT_MIN_WAVES
#define GOFANN_EXACT_MIN_WAVES 6
#endif

// 16-byte row chunks loaded per memory round trip in the any-dim row loop.
// At 6 waves, C2, Q = 80: three take 49.0 ms, four 46.1, six 48.9, the whole
// row (twelve) 47.5.
#ifndef GOFANN_EXACT_ROW_UNROLL
#define GOFANN_EXACT_ROW_UNROLL 4
#endif

// Waves per SIMD the f32 / f16 kernels are compiled for, and the 128-byte
// blocks per quad whose loads are issued before any is summed.  The quad
// kernels are bound by the loads in flight; their LDS holds them near 4
// waves per SIMD anyway (C4, 1 KB f16 rows, Q = 448: 17 routes per CU), so
// they take the registers for deeper batches: exact route 141.6 ms with two
// blocks left to the compiler's unrolling at 5 waves, 119.0 with explicit
// batches of two, 110.1 with batches of four at 4 waves (no spills; eight
// spill 8-14 VGPRs).
#ifndef GOFANN_EXACT_FLOAT_MIN_WAVES
#define GOFANN_EXACT_FLOAT_MIN_WAVES 4
#endif
#ifndef GOFANN_EXACT_QUAD_UNROLL
#define GOFANN_EXACT_QUAD_UNROLL 4
#endif
constexpr int kExactQuadUnroll = GOFANN_EXACT_QUAD_UNROLL;

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

// Squared L2 of a u8 row against the query held in LDS (q, |q|^2); kU
// 16-byte chunks per memory round trip when dim is a multiple of 16.
template <int kU>
__device__ __forceinline__ uint32_t l2_u8_row(const uint8_t* row, const uint32_t* q,
                                              uint32_t dim, uint32_t qnorm)
{
    uint32_t nb = 0, dot = 0;
    if ((dim & 15u) == 0) {
        const uint4* r4 = reinterpret_cast<const uint4*>(row);
        const uint4* q4 = reinterpret_cast<const uint4*>(q);
#pragma unroll kU
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

// Rows of kC 16-byte chunks (dim = 16 kC): every chunk's load is issued
// before the first dot product, so a row costs one memory round trip.
template <int kC>
__device__ __forceinline__ void row_load(const uint8_t* row, bool keep, uint4 (&b)[kC])
{
    const uint4* r4 = reinterpret_cast<const uint4*>(row);
#pragma unroll
    for (int i = 0; i < kC; ++i) b[i] = keep ? r4[i] : make_uint4(0, 0, 0, 0);
}

template <int kC>
__device__ __forceinline__ uint32_t row_dist(const uint4 (&b)[kC], const uint32_t* q,
                                             uint32_t qnorm)
{
    const uint4* q4 = reinterpret_cast<const uint4*>(q);
    uint32_t nb = 0, dot = 0;
#pragma unroll
    for (int i = 0; i < kC; ++i) {
        const uint4 w = q4[i];
        nb = __builtin_amdgcn_udot4(b[i].x, b[i].x, nb, false);
        nb = __builtin_amdgcn_udot4(b[i].y, b[i].y, nb, false);
        nb = __builtin_amdgcn_udot4(b[i].z, b[i].z, nb, false);
        nb = __builtin_amdgcn_udot4(b[i].w, b[i].w, nb, false);
        dot = __builtin_amdgcn_udot4(b[i].x, w.x, dot, false);
        dot = __builtin_amdgcn_udot4(b[i].y, w.y, dot, false);
        dot = __builtin_amdgcn_udot4(b[i].z, w.z, dot, false);
        dot = __builtin_amdgcn_udot4(b[i].w, w.w, dot, false);
    }
    return nb + qnorm - 2u * dot;
}

__device__ __forceinline__ bool better(float ld, uint32_t lid, float rd, uint32_t rid)
{
    return ld < rd || (ld == rd && lid < rid);
}

// insert_best_result (backend_full_gpu.cu:1342-1375) on a register array:
// lane i < K holds entry i, ascending by (distance, id), ids unique.  Every
// lane calls it with the same (d, id); size is wave-uniform.  The entries
// live in the first 16-lane row (K <= 10), so shifts are row DPP moves.
struct BestK {
    float d;
    uint32_t id;
};

__device__ __forceinline__ uint32_t dpp_u32(uint32_t v, int ctrl)
{
    switch (ctrl) {
    case 0x101: return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0x101, 0xF, 0xF, false));
    default: return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0x111, 0xF, 0xF, false));
    }
}

__device__ __forceinline__ bool best_insert(BestK& b, float d, uint32_t id, uint32_t K,
                                            uint32_t& size, int lane)
{
    const bool in = static_cast<uint32_t>(lane) < size;
    const uint64_t dup = ballot(in && b.id == id);
    if (dup) {
        const int i = __builtin_ctzll(dup);
        if (d >= __int_as_float(__builtin_amdgcn_readlane(__float_as_int(b.d), i))) return false;
        // drop entry i: lanes i.. take their right neighbour (row_shl:1)
        const uint32_t nd = dpp_u32(__float_as_uint(b.d), 0x101);
        const uint32_t ni = dpp_u32(b.id, 0x101);
        if (lane >= i) {
            b.d = __uint_as_float(nd);
            b.id = ni;
        }
        --size;
    }
    if (size == K) {
        const float ld = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(b.d), static_cast<int>(K) - 1));
        const uint32_t li = static_cast<uint32_t>(
            __builtin_amdgcn_readlane(static_cast<int>(b.id), static_cast<int>(K) - 1));
        if (!better(d, id, ld, li)) return false;
    }
    // entries before (d, id) stay; the rest move right (row_shr:1)
    const int pos = __popcll(ballot(static_cast<uint32_t>(lane) < size && better(b.d, b.id, d, id)));
    const uint32_t sd = dpp_u32(__float_as_uint(b.d), 0x111);
    const uint32_t si = dpp_u32(b.id, 0x111);
    if (lane > pos) {
        b.d = __uint_as_float(sd);
        b.id = si;
    } else if (lane == pos) {
        b.d = d;
        b.id = id;
    }
    if (size < K) ++size;
    return true;
}

// Loads a picked node needs when it is expanded, issued at pickup: lane j's
// adjacency entry j (and its sample id when the graph carries them), and the
// node's label slab or CSR bounds (.x/.y) for the filter.
struct ExactNode {
    uint32_t adj;
    uint32_t nsamp;
    uint4 row;
};

__device__ __forceinline__ void load_node(const gofann_graph_view& g,
                                          const gofann_predicate_view& pv, bool verdict_rows,
                                          uint32_t off, uint32_t degree, const Entry& e, int lane,
                                          ExactNode& n)
{
    const size_t row = static_cast<size_t>(off + (e.second & ~kPoolUsed)) * g.degree;
    const bool in_row = static_cast<uint32_t>(lane) < degree;
    n.adj = in_row ? g.graph[row + lane] : UINT32_MAX;
    n.nsamp = (in_row && g.neighbor_samples) ? g.neighbor_samples[row + lane] : 0u;
    n.row = make_uint4(0, 0, 0, 0);
    if (verdict_rows && e.sample < pv.rows && pv.csr_offsets != nullptr) {
        if (slab_usable(pv, e.sample)) {
            n.row = slab_load(pv, e.sample);
        } else {
            n.row.x = pv.csr_offsets[e.sample];
            n.row.y = pv.csr_offsets[e.sample + 1];
        }
    }
}

// Float rows (f32 / f16): the neighbours' exact distances in the warp
// order; lane j of the wave returns the distance of its own candidate
// (FLT_MAX where keep is false).  Rows up to kQuadMaxRowBytes: 16 rows at a
// time, one per quad of lanes (l2_w32_quad), candidates compacted through
// LDS in lane order (s_samp and s_dist, kMaxDegree entries, are free at
// this point of the step).  Longer rows (kLong, its own kernel): two at a
// time, one per 32-lane half (l2_w32_partial + w32_tree), which keeps every
// lane busy, with kExactLongBatch row words per lane in flight: at C3's
// 16 KB rows 181 ms a step for the graph routes, against 269 with 8 words
// and 348 for the quads; at C4's 1 KB rows the quads (then two blocks a
// lane in flight) took 140 against 329 for the halves.  Either form gives
// the same bits for any row length.
constexpr size_t kQuadMaxRowBytes = 4096;

#ifndef GOFANN_EXACT_LONG_BATCH
#define GOFANN_EXACT_LONG_BATCH 32
#endif
constexpr int kExactLongBatch = GOFANN_EXACT_LONG_BATCH;

template <int kElem, bool kLong>
__device__ __forceinline__ float wave_float_dists(const uint8_t* base, uint32_t dim,
                                                  const float* qf, bool keep, uint32_t samp,
                                                  int lane, uint32_t* s_samp, float* s_dist)
{
    const size_t row_bytes = static_cast<size_t>(dim) * elem_bytes(kElem);
    uint64_t m = ballot(keep);
    if constexpr (kLong) {
        float out = FLT_MAX;
        while (m) {
            const int ja = __builtin_ctzll(m);
            m &= m - 1;
            int jb = -1;
            if (m) {
                jb = __builtin_ctzll(m);
                m &= m - 1;
            }
            const uint32_t sa = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(samp), ja));
            const uint32_t sb =
                jb >= 0 ? static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(samp), jb))
                        : sa;
            const uint32_t s = lane < 32 ? sa : sb;
            const float t = w32_tree<kElem>(l2_w32_partial<kElem, kExactLongBatch>(
                base + static_cast<size_t>(s) * row_bytes, qf, dim, static_cast<uint32_t>(lane) & 31u));
            const float da = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t), 0));
            const float db = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t), 32));
            if (lane == ja) out = da;
            if (lane == jb) out = db;
        }
        return out;
    }
    const int n = __popcll(m);
    const uint32_t rank = lanes_below(m);
    if (keep) s_samp[rank] = samp;
    __threadfence_block();
    const int quad = lane >> 2;
    const uint32_t g = static_cast<uint32_t>(lane) & 3u;
    for (int c = quad; c - quad < n; c += 16) {
        if (c < n) {
            const uint32_t s = s_samp[c];
            const float d = l2_w32_quad<kElem, kExactQuadUnroll>(
                base + static_cast<size_t>(s) * row_bytes, qf, dim, g);
            if (g == 0) s_dist[c] = d;
        }
    }
    __threadfence_block();
    return keep ? s_dist[rank] : FLT_MAX;
}

// kC > 0 (u8): dim == 16 kC (rows loaded whole); kC == 0: any dim; kC < 0
// (f32 / f16): rows longer than kQuadMaxRowBytes.  The frontier lives in
// LDS.  kElem: the element type of base and queries
// (GOFANN_ELEM_*); u8 rows are scored per lane (integer, exact in any
// order), f32 / f16 rows by wave_float_dists.
template <int kVisited, int kC, int kElem>
__global__ __launch_bounds__(64, (kElem == GOFANN_ELEM_U8 ? GOFANN_EXACT_MIN_WAVES : GOFANN_EXACT_FLOAT_MIN_WAVES)) void exact_route_kernel(ExactArgs a)
{
    constexpr int kRowUnroll = GOFANN_EXACT_ROW_UNROLL;
    extern __shared__ __align__(16) unsigned char lds[];
    __shared__ uint32_t s_row[kMaxDegree];
    __shared__ uint32_t s_samp[kMaxDegree];
    __shared__ float s_dist[kMaxDegree];
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

    // Query row into LDS: u8 as words (zero-padded to 16 bytes) with |q|^2,
    // f32 / f16 as f32.
    const float* qf = reinterpret_cast<const float*>(lds);
    uint32_t qn = 0;
    if constexpr (kElem == GOFANN_ELEM_U8) {
        const uint8_t* qrow = a.queries + static_cast<size_t>(a.routes.route_query[route]) * a.dim;
        const uint32_t qwords = (a.dim + 15u) / 16u * 4u;
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
    } else {
        const uint8_t* qrow = a.queries + static_cast<size_t>(a.routes.route_query[route]) * a.dim *
                                              elem_bytes(kElem);
        float* qs = reinterpret_cast<float*>(lds);
        for (uint32_t d = lane; d < a.dim; d += kWave) qs[d] = elem_to_float<kElem>(qrow, d);
    }
    visited.init(reinterpret_cast<uint32_t*>(lds + a.off_hash),
                 a.hash_global ? a.hash_global + static_cast<size_t>(slot) * kHashCapacity : nullptr,
                 lane);
    __threadfence_block();
    __syncthreads();

    gofann_route_stats st{0, 0, 0, 0, 0, 0, 0, 0};
    PredCounters pc{0, 0};
    uint32_t bsize = 0;  // wave-uniform
    BestK bk{FLT_MAX, UINT32_MAX};
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
            float d0;
            if constexpr (kElem == GOFANN_ELEM_U8) {
                d0 = bcast0f(lane == 0 ? static_cast<float>(l2_u8_row<kRowUnroll>(
                                             a.base + static_cast<size_t>(s0) * a.dim, qw, a.dim, qn))
                                       : 0.0f);
            } else {
                // every quad scores the seed row; lane 0's sum is it
                d0 = bcast0f(l2_w32_quad<kElem>(
                    a.base + static_cast<size_t>(s0) * a.dim * elem_bytes(kElem), qf, a.dim,
                    static_cast<uint32_t>(lane) & 3u));
            }
            const Entry kp = {d0, seed, d0, s0};
            if (lane == 0) smmh_insert(frontier, heap_size, kp);
            heap_size = bcast0(heap_size);
            if (lane == 0) (void)visited.add_serial(seed, 0);
            visited.count = 1;
            st.scored = 1;
        } else {
            done = true;
        }
    }
    __threadfence_block();
    __syncthreads();
    if (!done) {
        if (!pickup(frontier, heap_size, now, lane)) done = true;
    }
    if (done) st.exhausted = 1;

    ExactNode cur{UINT32_MAX, 0, make_uint4(0, 0, 0, 0)};
    if (!done) load_node(a.graph, a.pred, enabled, off, degree, now, lane, cur);

    uint32_t steps = 0, finished = 0;
    bool first_step = true;
    const int wave_lane = lane;
    while (!done) {
        // per step: lane-derived values are not held across steps (no spills
        // at 6 waves; with the lane hoisted out of the loop, 10 VGPRs spilled)
        const int lane = opaque_lane(wave_lane);
        if (a.params.max_steps != 0 && steps >= static_cast<uint32_t>(a.params.max_steps)) break;

        // One memory round for the neighbours (visited tests, sample ids) and
        // the expanded node's label row, then one for the neighbours' rows.
        const uint32_t adj = cur.adj;
        const bool fresh = adj != UINT32_MAX && adj < gsize && !visited.test(adj);
        uint32_t samp = 0;
        if (fresh) samp = a.graph.neighbor_samples ? cur.nsamp : a.graph.row_to_sample[off + adj];
        const bool keep = fresh && samp < a.samples;
        const uint32_t sample = now.sample;
        WaveRow vrow{0, 0, UINT32_MAX, false};
        if (enabled) {
            if (!slab_usable(a.pred, sample)) {
                vrow = wave_row_load(a.pred, sample, cur.row.x, cur.row.y, lane);
            } else if (slab_count(cur.row) != kSlabOverflow) {
                vrow = wave_row_from_slab(cur.row, lane);
            } else {
                vrow = wave_row_load(a.pred, sample, a.pred.csr_offsets[sample],
                                     a.pred.csr_offsets[sample + 1], lane);
            }
        }
        uint32_t d32 = 0;
        float fdist = FLT_MAX;
        if constexpr (kElem == GOFANN_ELEM_U8) {
            const uint8_t* brow = a.base + static_cast<size_t>(samp) * a.dim;
            if constexpr (kC > 0) {
                uint4 rb[kC];
                row_load<kC>(brow, keep, rb);
                d32 = row_dist<kC>(rb, qw, qn);
            } else {
                d32 = keep ? l2_u8_row<kRowUnroll>(brow, qw, a.dim, qn) : 0u;
            }
            // The distance is complete here: the rows and query words are
            // dead before the filter below.
            asm volatile("" : "+v"(d32)::"memory");
        } else {
            fdist = wave_float_dists<kElem, (kC < 0)>(a.base, a.dim, qf, keep, samp, lane, s_samp,
                                                       s_dist);
            asm volatile("" : "+v"(fdist)::"memory");
        }

        // The expanded node's filter (wave-uniform) and best-k (lane 0).
        const uint32_t grow = off + (now.second & ~kPoolUsed);
        const uint64_t rmask = a.routes.row_filter_mask ? a.routes.row_filter_mask[grow] : ~0ULL;
        bool ok = (rmask & qfbit) != 0;
        if (ok && active != 0) ok = count_matching_ranges(a.routes, route, sample) == active;
        PredCounters c{0, 0};
        if (ok && enabled) ok = wave_pred_matches(a.pred, route, sample, vrow, lane, c);
        int improved = 0;
        if (lane == 0) {
            pc.rows += c.rows;
            pc.labels += c.labels;
        }
        if (ok) improved = best_insert(bk, now.first, sample, K, bsize, lane) ? 1 : 0;
        ++st.expanded;
        st.passed += ok ? 1 : 0;
        ++steps;

        const float dist = kElem == GOFANN_ELEM_U8 ? (keep ? static_cast<float>(d32) : FLT_MAX)
                                                   : fdist;
        st.scored += __popcll(ballot(keep));

        // Drop what cannot enter a full frontier (its maximum only falls
        // during the step), then admit the rest in adjacency order.
        const bool full = heap_size > 2 && heap_size >= Q + 1;
        const float thr = full ? frontier[2].first : 0.0f;
        const bool cand = keep && !(full && thr < dist);
        const uint64_t cand_mask = ballot(cand);
        uint64_t adm = 0;  // admitted lanes
        if (Q + 2 <= kWaveHeapSlots) {
            // the whole wave runs each heap operation (same array as the
            // lane-0 sifts below); hmax: the largest `first` in the heap
            float hmax = heap_size >= 3   ? frontier[2].first
                         : heap_size == 2 ? frontier[1].first
                                          : -__builtin_inff();
            for (uint64_t m = cand_mask; m; m &= m - 1) {
                const int j = __builtin_ctzll(m);
                Entry kp;
                kp.first = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dist), j));
                kp.second = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(adj), j));
                kp.sample = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(samp), j));
                kp.base = kp.first;
                if (heap_size > 2 && heap_size >= Q + 1 && hmax < kp.first) continue;
                wave_smmh_insert(frontier, heap_size, kp, lane);
                hmax = fmaxf(hmax, kp.first);
                adm |= 1ull << j;
                if (heap_size >= Q + 2) hmax = wave_smmh_pop_max(frontier, heap_size, lane);
            }
        } else {
            const int n_cand = __popcll(cand_mask);
            const uint32_t pos = lanes_below(cand_mask);
            if (cand) {
                s_row[pos] = adj;
                s_samp[pos] = samp;
                s_dist[pos] = dist;
            }
            __syncthreads();
            if (lane == 0) {
                uint64_t ap = 0;
                for (int i = 0; i < n_cand; ++i) {
                    const Entry kp = {s_dist[i], s_row[i], s_dist[i], s_samp[i]};
                    if (heap_size > 2 && heap_size >= Q + 1 && frontier[2].first < kp.first)
                        continue;
                    smmh_insert(frontier, heap_size, kp);
                    ap |= 1ull << i;
                    if (heap_size >= Q + 2) smmh_pop_max(frontier, heap_size);
                }
                s_adm = ap;
            }
            heap_size = bcast0(heap_size);
            __syncthreads();
            const uint64_t ap = s_adm;  // by compacted position
            adm = ballot(cand && ((ap >> pos) & 1ull));
        }
        const uint32_t n_adm = static_cast<uint32_t>(__popcll(adm));
        st.admitted += static_cast<int32_t>(n_adm);
        visited.reserve(n_adm, lane);
        if (visited.count + n_adm <= kHashCapacity) {
            const int ins = ((adm >> lane) & 1ull) ? visited.add_parallel(adj) : 0;
            visited.count += static_cast<uint32_t>(__popcll(ballot(ins != 0)));
        } else {
            // The set may fill: serial adds in admission (lane) order
            // reproduce which values the reference drops.
            uint32_t added = 0;
            for (uint64_t m = adm; m; m &= m - 1) {
                const int j = __builtin_ctzll(m);
                const uint32_t v = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(adj), j));
                if (lane == 0) added += static_cast<uint32_t>(visited.add_serial(v, added));
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
        load_node(a.graph, a.pred, enabled, off, degree, next, lane, cur);
        int stop = 0;
        const float kd = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bk.d), static_cast<int>(K) - 1));
        const uint32_t ki = static_cast<uint32_t>(
            __builtin_amdgcn_readlane(static_cast<int>(bk.id), static_cast<int>(K) - 1));
        if (lane == 0 && !first_step) {
            if (mode == GOFANN_EARLY_STOP_ADAPTIVE && improved) {
                finished = 0;
            } else if (bsize == K && !better(next.first, next.sample, kd, ki)) {
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
    const uint32_t nb = bsize;
    if (static_cast<uint32_t>(lane) < K) {
        oid[lane] = static_cast<uint32_t>(lane) < nb ? bk.id : UINT32_MAX;
        od[lane] = static_cast<uint32_t>(lane) < nb ? bk.d : FLT_MAX;
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

template <int kVisited, int kC, int kElem>
int resident(Context* ctx, uint32_t lds)
{
    if (lds > static_cast<uint32_t>(ctx->lds_per_block)) return 0;
    const void* k = reinterpret_cast<const void*>(exact_route_kernel<kVisited, kC, kElem>);
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

// Visited-set placement with the most resident routes per CU (ties: the
// full LDS table, then the spilling table, then the global slab), then the
// launch.
// fixed_slab: visited slabs for a placement outside LDS, holding at most
// fixed_routes routes (the no-alloc entry point); nullptr: context scratch.
template <int kC, int kElem>
int launch_exact(Context* ctx, ExactArgs& a, int hash_mode, uint32_t lds_full,
                 uint32_t lds_spill, uint32_t lds_glob, uint32_t count, uint32_t* fixed_slab,
                 uint32_t fixed_routes)
{
    const int rf = resident<kVisitedLds, kC, kElem>(ctx, lds_full);
    const int rs = resident<kVisitedSpill, kC, kElem>(ctx, lds_spill);
    const int rg = resident<kVisitedGlobal, kC, kElem>(ctx, lds_glob);
    int mode = kVisitedLds;
    int res = rf;
    if (hash_mode == GOFANN_PLACE_GLOBAL) {
        mode = kVisitedGlobal;
        res = rg;
    } else if (hash_mode == GOFANN_PLACE_SPILL) {
        mode = kVisitedSpill;
        res = rs;
    } else if (hash_mode == GOFANN_PLACE_AUTO) {
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
    if (mode != kVisitedLds && fixed_slab != nullptr) {
        if (count > fixed_routes)
            return ctx->fail(GOFANN_ERR_INVALID,
                             "no-alloc exact search: " + std::to_string(count) +
                                 " routes need visited slabs beyond the fixed scratch (at most " +
                                 std::to_string(fixed_routes) +
                                 " routes per call with a visited set outside LDS)");
        a.hash_global = fixed_slab;
    } else if (mode != kVisitedLds) {
        const size_t need = static_cast<size_t>(count) * kHashCapacity * sizeof(uint32_t);
        a.hash_global = static_cast<uint32_t*>(ctx->scratch(Context::kScratchHash, need));
        if (!a.hash_global) return ctx->fail(GOFANN_ERR_NOMEM, "visited set scratch");
    }
    const uint32_t lds = mode == kVisitedLds ? lds_full : (mode == kVisitedSpill ? lds_spill : lds_glob);
    const dim3 grid(count), block(kWave);
    if (mode == kVisitedLds)
        hipLaunchKernelGGL((exact_route_kernel<kVisitedLds, kC, kElem>), grid, block, lds,
                           ctx->stream, a);
    else if (mode == kVisitedSpill)
        hipLaunchKernelGGL((exact_route_kernel<kVisitedSpill, kC, kElem>), grid, block, lds,
                           ctx->stream, a);
    else
        hipLaunchKernelGGL((exact_route_kernel<kVisitedGlobal, kC, kElem>), grid, block, lds,
                           ctx->stream, a);
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("exact route launch");
    ctx->last_table_in_lds = 0;
    ctx->last_hash_in_lds = mode == kVisitedGlobal ? 0 : (mode == kVisitedLds ? 1 : 2);
    ctx->last_lds_bytes = static_cast<int>(lds);
    ctx->last_resident = res;
    return GOFANN_OK;
}


struct LaunchShape {
    Context* ctx;
    ExactArgs* a;
    int hash_mode;
    uint32_t lds_full, lds_spill, lds_glob, count;
    uint32_t* fixed_slab;
    uint32_t fixed_routes;
};

// Row length fixed at compile time only in builds that ask for it (u8).
template <int kElem>
int launch_rows(const LaunchShape& s, int chunks)
{
    if constexpr (kElem != GOFANN_ELEM_U8) {
        if (chunks < 0)
            return launch_exact<-1, kElem>(s.ctx, *s.a, s.hash_mode, s.lds_full, s.lds_spill,
                                           s.lds_glob, s.count, s.fixed_slab, s.fixed_routes);
    }
#if GOFANN_EXACT_FIXED_ROWS
    if constexpr (kElem == GOFANN_ELEM_U8) {
        switch (chunks) {
        case 8:
            return launch_exact<8, kElem>(s.ctx, *s.a, s.hash_mode, s.lds_full, s.lds_spill,
                                          s.lds_glob, s.count, s.fixed_slab, s.fixed_routes);
        case 12:
            return launch_exact<12, kElem>(s.ctx, *s.a, s.hash_mode, s.lds_full, s.lds_spill,
                                           s.lds_glob, s.count, s.fixed_slab, s.fixed_routes);
        case 16:
            return launch_exact<16, kElem>(s.ctx, *s.a, s.hash_mode, s.lds_full, s.lds_spill,
                                           s.lds_glob, s.count, s.fixed_slab, s.fixed_routes);
        default:
            break;
        }
    }
#else
    (void)chunks;
#endif
    return launch_exact<0, kElem>(s.ctx, *s.a, s.hash_mode, s.lds_full, s.lds_spill, s.lds_glob,
                                  s.count, s.fixed_slab, s.fixed_routes);
}

static int exact_search_impl(Context* ctx, const void* base, int base_elem, uint32_t dim,
                             uint32_t samples, const void* queries, const gofann_graph_view* g,
                             const uint32_t* label_size, const gofann_predicate_view* pred,
                             const gofann_routes* r, const gofann_exact_params* p,
                             uint32_t* out_ids, float* out_dists, gofann_route_stats* stats,
                             uint32_t* fixed_slab, uint32_t fixed_routes)
{
    if (!g || !r || !p) return ctx->fail(GOFANN_ERR_INVALID, "null view");
    if (base_elem != GOFANN_ELEM_U8 && base_elem != GOFANN_ELEM_F32 && base_elem != GOFANN_ELEM_F16)
        return ctx->fail(GOFANN_ERR_INVALID, "base_elem must be u8, f32 or f16");
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
    if (g->degree > static_cast<uint32_t>(kMaxDegree))
        return ctx->fail(GOFANN_ERR_UNSUPPORTED, "graph degree must be in [1, 64]");
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
    // LDS: the query row, then Q + 2 frontier entries, then the visited
    // table of the chosen placement.  (A frontier held in registers, lane i
    // holding entry i, was slower at every beam measured: C2 43.4 against
    // 41.0 ms a step at Q = 56 / 88, 26.6 against 25.8 at 32 / 88 -- the
    // wave-parallel LDS heap operations below issue fewer instructions
    // than its serial register sifts.)
    a.off_frontier = base_elem == GOFANN_ELEM_U8 ? align16u((dim + 15u) / 16u * 16u)
                                                 : align16u(dim * 4u);
    a.off_hash = align16u(a.off_frontier + static_cast<uint32_t>(p->queue_limit + 2) *
                                               sizeof(Entry));
    const uint32_t lds_full = a.off_hash + kHashCapacity * 4u;
    const uint32_t lds_spill = a.off_hash + kSpillSlots * 4u;
    const uint32_t lds_glob = a.off_hash;
    const int chunks = (GOFANN_EXACT_FIXED_ROWS && (dim == 128 || dim == 192 || dim == 256))
                           ? static_cast<int>(dim / 16)
                           : 0;
    const LaunchShape sh{ctx, &a, p->hash_mode, lds_full, lds_spill, lds_glob, r->count,
                         fixed_slab, fixed_routes};
    // float rows over kQuadMaxRowBytes take the long-row kernel
    const int fchunks = static_cast<size_t>(dim) * elem_bytes(base_elem) > kQuadMaxRowBytes ? -1 : 0;
    switch (base_elem) {
    case GOFANN_ELEM_F32: return launch_rows<GOFANN_ELEM_F32>(sh, fchunks);
    case GOFANN_ELEM_F16: return launch_rows<GOFANN_ELEM_F16>(sh, fchunks);
    default: return launch_rows<GOFANN_ELEM_U8>(sh, chunks);
    }
}

int exact_search(Context* ctx, const void* base, int base_elem, uint32_t dim, uint32_t samples,
                 const void* queries, const gofann_graph_view* g, const uint32_t* label_size,
                 const gofann_predicate_view* pred, const gofann_routes* r,
                 const gofann_exact_params* p, uint32_t* out_ids, float* out_dists,
                 gofann_route_stats* stats)
{
    return exact_search_impl(ctx, base, base_elem, dim, samples, queries, g, label_size, pred, r,
                             p, out_ids, out_dists, stats, nullptr, 0);
}

int exact_search_noalloc(Context* ctx, const void* base, int base_elem, uint32_t dim,
                         uint32_t samples, const void* queries, const gofann_graph_view* g,
                         const uint32_t* label_size, const gofann_predicate_view* pred,
                         const gofann_routes* r, const gofann_exact_params* p,
                         uint32_t* out_ids, float* out_dists, gofann_route_stats* stats)
{
    uint32_t* slab = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_noalloc_mutex);
        if (ctx->device >= 0 && ctx->device < kNoAllocMaxDevices)
            slab = g_noalloc_slab[ctx->device];
        if (slab == nullptr)
            return ctx->fail(GOFANN_ERR_HIP,
                             "no-alloc scratch unavailable on this device" +
                                 (ctx->device >= 0 && ctx->device < kNoAllocMaxDevices &&
                                          !g_noalloc_error[ctx->device].empty()
                                      ? ": " + g_noalloc_error[ctx->device]
                                      : std::string()));
    }
    return exact_search_impl(ctx, base, base_elem, dim, samples, queries, g, label_size, pred, r,
                             p, out_ids, out_dists, stats, slab, GOFANN_EXACT_NOALLOC_MAX_ROUTES);
}

}  // namespace gofann
