// rabitq_pair.hip -- the RaBitQ graph traversal with two routes per wave64,
// for graphs of degree <= 32 (one neighbour per lane of a half-wave).
//
// Same observable semantics as traversal_kernel<RabitqScorer> with an LDS
// frontier (run_rabitq_search_one_block, src/search/rabitq/backend_rabitq.cu:
// 3487-4291): pickup-before-expand, verdict chain, result and stop heaps,
// adaptive early stop, bias priority, admission, visited set and output, bit
// for bit.  Lanes 0..31 run the route of slot 2b, lanes 32..63 the route of
// slot 2b+1; every wave-level step of the one-route kernel (ballots,
// reductions, broadcasts, the cooperative label-row reads) becomes its
// half-wave counterpart, and the serial parts (frontier sifts, result and
// stop heaps) run on lanes 0 and 32 side by side.  With degree 32 the
// one-route kernel leaves half of every lane-parallel phase idle; here both
// halves work, and the serial work of two routes shares each instruction.
//
// Opt-in (environment variable GOFANN_RABITQ_PAIR=1) for per-lane RaBitQ
// scoring (padded_dim / 128 < 16), beams with Q + 2 > 64 (the LDS frontier)
// and the visited set in LDS or in the global slab.  It is not the default:
// the LDS a route needs (frontier, result and stop heaps, query planes), not
// its registers, bounds the routes resident per CU, so pairing routes in a
// wave keeps the same routes in flight and adds the divergence of two
// routes in one instruction stream (C4: 197.7 ms against 185.2 ms).
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>
#include <cstdlib>

#include "traversal.hpp"

// Waves per SIMD the pair kernel is compiled for: 3 (165 VGPRs, no spills)
// is six routes per SIMD; 4 would spill the per-half state.
#ifndef GOFANN_RABITQ_PAIR_MIN_WAVES
#define GOFANN_RABITQ_PAIR_MIN_WAVES 3
#endif

namespace gofann {

namespace {

constexpr int kHalf = 32;

// ---- half-wave primitives (h = lane >> 5, hl = lane & 31, hb = lane & 32)
__device__ __forceinline__ uint32_t hmask(bool p, int hb)
{
    return static_cast<uint32_t>(ballot(p) >> hb);
}

__device__ __forceinline__ int hb0(int v, int hb)
{
    const int a = __builtin_amdgcn_readlane(v, 0);
    const int b = __builtin_amdgcn_readlane(v, kHalf);
    return hb ? b : a;
}

__device__ __forceinline__ uint32_t hb0u(uint32_t v, int hb)
{
    return static_cast<uint32_t>(hb0(static_cast<int>(v), hb));
}

__device__ __forceinline__ float hb0f(float v, int hb)
{
    return __int_as_float(hb0(__float_as_int(v), hb));
}

__device__ __forceinline__ float hmin(float v)
{
    for (int off = 16; off > 0; off >>= 1) v = fminf(v, __shfl_xor(v, off, kWave));
    return v;
}

__device__ __forceinline__ int hsum(int v)
{
    for (int off = 16; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// pickup over this half's frontier (pickup_next_unused_from_native_frontier,
// backend_pq.cu:844-892): unused entry of least `first`, lowest index on
// ties; the half's lane 0 marks it used.
__device__ __forceinline__ bool pickup_h(Entry* f, int size, Entry& out, int hl, int hb)
{
    int best = -1;
    float bv = 0.0f;
    for (int i = hl + 1; i < size; i += kHalf) {
        const Entry e = f[i];
        if (e.second & kPoolUsed) continue;
        if (best < 0 || e.first < bv) {
            best = i;
            bv = e.first;
        }
    }
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) {
        const int ob = __shfl_xor(best, off, kWave);
        const float ov = __shfl_xor(bv, off, kWave);
        if (ob >= 0 && (best < 0 || ov < bv || (!(bv < ov) && ob < best))) {
            best = ob;
            bv = ov;
        }
    }
    best = hb0(best, hb);
    if (best < 0) return false;
    out = f[best];
    __threadfence_block();
    if (hl == 0) f[best].second |= kPoolUsed;
    __threadfence_block();
    return true;
}

__device__ __forceinline__ float min_pending_base_h(const Entry* f, int size, const Entry& now,
                                                    const Entry& next, int hl)
{
    float m = FLT_MAX;
    for (int i = hl + 1; i < size; i += kHalf) {
        const Entry e = f[i];
        if (!(e.second & kPoolUsed)) m = fminf(m, e.base);
    }
    m = hmin(m);
    m = fminf(m, now.base);
    m = fminf(m, next.base);
    return m;
}

// The expanded node's label row held across the half: lane hl holds label
// begin + hl of the first 32.
__device__ __forceinline__ WaveRow row_load_h(const gofann_predicate_view& v, uint32_t sample,
                                              uint32_t begin, uint32_t end, int hl)
{
    WaveRow r;
    r.valid = sample < v.rows && v.csr_offsets != nullptr;
    r.begin = begin;
    r.end = r.valid ? end : begin;
    const uint32_t len = r.end - r.begin;
    r.lab = static_cast<uint32_t>(hl) < len ? v.csr_labels[r.begin + hl] : UINT32_MAX;
    return r;
}

__device__ __forceinline__ WaveRow row_from_slab_h(const uint4& slab, int hl)
{
    WaveRow r;
    r.valid = true;
    r.begin = 0;
    r.end = slab_count(slab);
    const uint32_t l = static_cast<uint32_t>(hl);
    r.lab = l < r.end && l < kSlabCapacity ? slab_label(slab, l) : UINT32_MAX;
    return r;
}

// csr_contains_sorted over the half-held row (the first label >= handle
// decides; the labels a serial scan would read are counted exactly).
__device__ __forceinline__ bool row_contains_h(const gofann_predicate_view& v, const WaveRow& r,
                                               uint32_t handle, int hl, int hb, PredCounters& c)
{
    if (!r.valid) return false;
    ++c.rows;
    const uint32_t len = r.end - r.begin;
    for (uint32_t base = 0; base < len; base += kHalf) {
        const uint32_t k = base + static_cast<uint32_t>(hl);
        const uint32_t lab =
            base == 0 ? r.lab : (k < len ? v.csr_labels[r.begin + k] : UINT32_MAX);
        const uint32_t ge = hmask(k < len && lab >= handle, hb);
        if (ge) {
            const int f = __builtin_ctz(ge);
            c.labels += base + static_cast<uint32_t>(f) + 1u;
            return static_cast<uint32_t>(__shfl(static_cast<int>(lab), hb + f, kWave)) == handle;
        }
    }
    c.labels += len;
    return false;
}

__device__ __forceinline__ bool pred_matches_h(const gofann_predicate_view& v, uint32_t route,
                                               uint32_t sample, const WaveRow& row, int hl,
                                               int hb, PredCounters& c)
{
    if (sample >= v.rows) return false;
    if (v.clauses) {
        for (uint32_t i = v.route_offsets[route]; i < v.route_offsets[route + 1]; ++i) {
            const gofann_clause cl = v.clauses[i];
            bool pass = true;
            for (uint32_t j = cl.label_begin; pass && j < cl.label_end; ++j)
                pass = row_contains_h(v, row, v.route_handles[j], hl, hb, c);
            for (uint32_t j = cl.range_begin; pass && j < cl.range_end; ++j) {
                const gofann_range_atom at = v.ranges[j];
                pass = v.base_ranges != nullptr && at.dimension < range_columns(v) &&
                       range_matches(at.mode, at.lower, at.upper,
                                     v.base_ranges[static_cast<uint64_t>(sample) * v.range_stride +
                                                   at.dimension]);
            }
            if (pass) return true;
        }
        return false;
    }
    for (uint32_t i = v.route_offsets[route]; i < v.route_offsets[route + 1]; ++i)
        if (!row_contains_h(v, row, v.route_handles[i], hl, hb, c)) return false;
    return true;
}

// RabitqScorer::setup for this half's query: the eight bit planes into the
// half's LDS region, written by its 32 lanes.
__device__ __forceinline__ void setup_h(RabitqScorer& sc, uint32_t q, int hl, unsigned char* region)
{
    sc.planes = reinterpret_cast<uint32_t*>(region);
    const uint32_t words = sc.padded_dim / 32;
    const int8_t* qrow = sc.q8 + static_cast<size_t>(q) * sc.padded_dim;
    for (uint32_t w = hl; w < words; w += kHalf) {
        uint32_t pl[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (uint32_t b = 0; b < 32; ++b) {
            const uint32_t v = static_cast<uint8_t>(qrow[w * 32 + b]);
#pragma unroll
            for (int j = 0; j < 8; ++j) pl[j] |= ((v >> j) & 1u) << (31u - b);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) sc.planes[j * words + w] = pl[j];
    }
    sc.scale = sc.q_scale[q];
    sc.k1 = sc.q_k1[q];
    sc.g_row = sc.centroid_dists + static_cast<size_t>(q) * sc.num_anchors;
}

struct PairArgs {
    TraversalArgs t;
    uint32_t region;  // LDS bytes per route
};

}  // namespace

template <int kVisited>
__global__ __launch_bounds__(64, GOFANN_RABITQ_PAIR_MIN_WAVES) void rabitq_pair_kernel(
    PairArgs pa, RabitqScorer sc)
{
    extern __shared__ __align__(16) unsigned char lds[];
    __shared__ uint32_t s_row[kMaxDegree];
    __shared__ uint32_t s_samp[kMaxDegree];
    __shared__ float s_first[kMaxDegree];
    __shared__ float s_base[kMaxDegree];
    __shared__ uint64_t s_adm[2];

    const TraversalArgs& a = pa.t;
    const int lane = static_cast<int>(threadIdx.x);
    const int hl = lane & (kHalf - 1);
    const int hb = lane & kHalf;
    const int half = lane >> 5;
    const uint32_t npairs = (a.routes.count + 1) / 2;
    const uint32_t pslot = xcd_slot(blockIdx.x, gridDim.x);
    if (pslot >= npairs) return;
    const uint32_t slot = 2 * pslot + static_cast<uint32_t>(half);
    const bool has_route = slot < a.routes.count;
    const uint32_t route =
        has_route ? (a.routes.launch_order ? a.routes.launch_order[slot] : slot) : 0u;

    unsigned char* region = lds + static_cast<size_t>(half) * pa.region;
    Entry* frontier = reinterpret_cast<Entry*>(region + a.off_frontier);
    ResultEntry* topk = reinterpret_cast<ResultEntry*>(region + a.off_topk);
    StopEntry* stop = reinterpret_cast<StopEntry*>(region + a.off_stop);
    VisitedSet<kVisited> visited;
    visited.shared = {reinterpret_cast<uint32_t*>(region + a.off_hash), kHashCapacity};
    visited.global = {a.hash_global ? a.hash_global + static_cast<size_t>(slot) * kHashCapacity
                                    : nullptr,
                      kHashCapacity};
    visited.count = 0;
    visited.spilled = false;

    const int Q = a.params.queue_limit;
    const int W = a.params.result_width;
    const int SW = a.params.stop_width;
    const int mode = a.params.early_stop_mode;
    const bool bias = a.params.predicate_bias != 0;
    const bool bonuses = a.params.bit_filter_bonus != 1.0f || a.params.range_filter_bonus != 1.0f;
    const uint32_t degree = a.graph.degree < static_cast<uint32_t>(kHalf)
                                ? a.graph.degree
                                : static_cast<uint32_t>(kHalf);

    uint32_t group = 0, label_offset = 0, query = 0, begin_id = 0, active_ranges = 0;
    uint64_t qfbit = ~0ULL;
    bool enabled = false, compiled = false;
    if (has_route) {
        group = a.routes.route_group[route];
        label_offset = a.graph.label_offset[group];
        query = a.routes.route_query[route];
        begin_id = a.routes.route_start[route];
        qfbit = a.routes.query_filter_bits ? a.routes.query_filter_bits[route] : ~0ULL;
        active_ranges = count_active_ranges(a.routes.range_modes, route, a.routes.range_count);
        enabled = pred_enabled(a.pred, route);
        compiled = a.pred.route_compiled != nullptr && a.pred.route_compiled[route] != 0;
    }
    const bool fallback = !compiled;  // the RaBitQ verdict chain

    // visited table clear (this half's table) and the query's planes
    if (has_route) {
        if constexpr (kVisited == kVisitedGlobal) {
            uint4* p = reinterpret_cast<uint4*>(visited.global.slots);
            for (uint32_t i = hl; i < kHashCapacity / 4; i += kHalf)
                p[i] = make_uint4(UINT32_MAX, UINT32_MAX, UINT32_MAX, UINT32_MAX);
        } else {
            uint4* p = reinterpret_cast<uint4*>(visited.shared.slots);
            for (uint32_t i = hl; i < kHashCapacity / 4; i += kHalf)
                p[i] = make_uint4(UINT32_MAX, UINT32_MAX, UINT32_MAX, UINT32_MAX);
        }
        setup_h(sc, query, hl, region);
    }
    __threadfence_block();
    __syncthreads();

    PredCounters pc{0, 0};
    int scored = 1;
    int admitted = 0;
    float start = 0.0f;
    uint32_t begin_sample = 0;
    if (has_route) begin_sample = a.graph.row_to_sample[label_offset + begin_id];
    // seed (backend_pq.cu:4164-4187): every lane calls score, the half's
    // lane 0 scores
    start = hb0f(sc.score(begin_sample, has_route && hl == 0), hb);
    const float penalty = bias ? bias_penalty(a.pred.alpha, start) : 0.0f;

    int heap_size = 1;
    int stop_size = 0;
    int topk_size = 0;
    int finished = 0;
    int exhausted = 0;
    int expanded = 0;
    int passed = 0;
    float stop_worst = -FLT_MAX;
    const Entry sentinel = {FLT_MAX, UINT32_MAX, FLT_MAX, UINT32_MAX};
    if (has_route && hl == 0) {
        const Entry kp = {start, begin_id, start, begin_sample};
        smmh_insert(frontier, heap_size, kp);
        (void)visited.add_serial(begin_id, 0);
    }
    heap_size = hb0(heap_size, hb);
    visited.count = 1;
    __threadfence_block();
    __syncthreads();

    Entry now = sentinel;
    Entry next = sentinel;
    NodeLoads cur, nxt;
    cur.adj = nxt.adj = UINT32_MAX;
    cur.nsamp = nxt.nsamp = 0;
    cur.row = nxt.row = make_uint4(0, 0, 0, 0);
    bool active = has_route;
    if (active) {
        if (!pickup_h(frontier, heap_size, now, hl, hb)) {
            exhausted = 1;
            now = sentinel;
        } else {
            const uint32_t local = now.second & ~kPoolUsed;
            const size_t row = static_cast<size_t>(label_offset + local) * a.graph.degree;
            const bool in_row = static_cast<uint32_t>(hl) < degree;
            cur.adj = in_row ? a.graph.graph[row + hl] : UINT32_MAX;
            cur.nsamp = (in_row && a.graph.neighbor_samples) ? a.graph.neighbor_samples[row + hl] : 0u;
            cur.row = make_uint4(0, 0, 0, 0);
            if (enabled && now.sample < a.pred.rows && a.pred.csr_offsets != nullptr) {
                if (slab_usable(a.pred, now.sample)) {
                    cur.row = slab_load(a.pred, now.sample);
                } else {
                    cur.row.x = a.pred.csr_offsets[now.sample];
                    cur.row.y = a.pred.csr_offsets[now.sample + 1];
                }
            }
        }
    }

    // loads a picked node needs when it is expanded (load_node, one half)
    auto load_node_h = [&](const Entry& e, NodeLoads& n) {
        const uint32_t local = e.second & ~kPoolUsed;
        const size_t row = static_cast<size_t>(label_offset + local) * a.graph.degree;
        const bool in_row = static_cast<uint32_t>(hl) < degree;
        n.adj = in_row ? a.graph.graph[row + hl] : UINT32_MAX;
        n.nsamp = (in_row && a.graph.neighbor_samples) ? a.graph.neighbor_samples[row + hl] : 0u;
        n.row = make_uint4(0, 0, 0, 0);
        if (enabled && e.sample < a.pred.rows && a.pred.csr_offsets != nullptr) {
            if (slab_usable(a.pred, e.sample)) {
                n.row = slab_load(a.pred, e.sample);
            } else {
                n.row.x = a.pred.csr_offsets[e.sample];
                n.row.y = a.pred.csr_offsets[e.sample + 1];
            }
        }
    };

    int step = 0;
    for (;;) {
        const bool go = active && (step == 0 || heap_size > 1);
        if (ballot(go) == 0) break;
        if (!go) {
            active = false;
            continue;
        }
        do {
            const uint32_t now_local = now.second & ~kPoolUsed;
            ++step;

            if (step != 1) {
                if (!pickup_h(frontier, heap_size, next, hl, hb)) {
                    exhausted = 1;
                    next = sentinel;
                } else {
                    load_node_h(next, nxt);
                    if (stop_size == SW) {
                        float pending = next.first;
                        if (a.pred.pending_base_stop && enabled)
                            pending = min_pending_base_h(frontier, heap_size, now, next, hl);
                        if (mode != GOFANN_EARLY_STOP_OFF && stop_worst <= pending) ++finished;
                    }
                }
            }

            // First memory round: the expanded node's label row and every
            // unvisited neighbour's sample (lane hl takes neighbour hl).
            WaveRow vrow{0, 0, UINT32_MAX, false};
            if (!exhausted && enabled) {
                const uint32_t s0 = now.sample;
                if (!slab_usable(a.pred, s0)) {
                    vrow = row_load_h(a.pred, s0, cur.row.x, cur.row.y, hl);
                } else if (slab_count(cur.row) != kSlabOverflow) {
                    vrow = row_from_slab_h(cur.row, hl);
                } else {
                    vrow = row_load_h(a.pred, s0, a.pred.csr_offsets[s0],
                                      a.pred.csr_offsets[s0 + 1], hl);
                }
            }
            const uint32_t idx = cur.adj;
            const bool keep = idx != UINT32_MAX && !visited.test(idx);
            const int list_len = __popc(hmask(keep, hb));
            uint32_t my_sample = 0;
            if (keep)
                my_sample = a.graph.neighbor_samples ? cur.nsamp
                                                     : a.graph.row_to_sample[label_offset + idx];
            const bool need_pass = keep && bias && enabled;
            LaneRow lrow;
            uint4 lslab;
            lane_row_bounds(a.pred, my_sample, need_pass, lrow, lslab);

            // Verdict of the expanded node (backend_pq.cu:4393-4441).
            int filt = 1;
            const float rank = now.base;
            if (!exhausted) {
                const uint32_t sample = now.sample;
                PredCounters c{0, 0};
                if (enabled) filt = pred_matches_h(a.pred, route, sample, vrow, hl, hb, c) ? 1 : 2;
                if (fallback) {
                    const uint32_t global_row = label_offset + now_local;
                    const uint64_t rmask =
                        a.routes.row_filter_mask ? a.routes.row_filter_mask[global_row] : ~0ULL;
                    const bool bit_match = (rmask & qfbit) != 0;
                    const uint32_t matched = count_matching_ranges(a.routes, route, sample);
                    const bool exact_range = active_ranges == 0 || matched == active_ranges;
                    filt = (filt == 1 && bit_match && exact_range) ? 1 : 2;
                }
                if (hl == 0) {
                    pc.rows += c.rows;
                    pc.labels += c.labels;
                }
            }
            const float current = now.base;

            if (exhausted ||
                early_stop_reached(mode, finished, a.params.finish_limit, Q, expanded, passed, SW) ||
                (a.params.max_steps > 0 && step >= a.params.max_steps)) {
                active = false;
                break;
            }

            // Result and stop heaps (backend_pq.cu:4558-4631).
            ++expanded;
            if (filt == 1) {
                ++passed;
                int improved = 0;
                if (hl == 0) {
                    const ResultEntry te = {rank, now_local};
                    StopEntry se;
                    se.first = rank;
                    se.pad = 0;
                    se.second = (static_cast<uint64_t>(fbits(current)) << 32) | now_local;
                    if (stop_size < SW) {
                        stop[stop_size++] = se;
                        bin_push(stop, stop_size);
                        improved = 1;
                        if (stop_size == 1 || current > stop_worst) stop_worst = current;
                    } else if (se.first < stop[0].first) {
                        stop[stop_size++] = se;
                        bin_push(stop, stop_size);
                        const StopEntry removed = bin_pop(stop, stop_size);
                        --stop_size;
                        improved = 1;
                        const uint32_t removed_bits = static_cast<uint32_t>(removed.second >> 32);
                        if (current > stop_worst) {
                            stop_worst = current;
                        } else if (removed_bits == fbits(stop_worst)) {
                            stop_worst = -FLT_MAX;
                            for (int ii = 0; ii < stop_size; ++ii) {
                                const float d = bitsf(static_cast<uint32_t>(stop[ii].second >> 32));
                                if (d > stop_worst) stop_worst = d;
                            }
                        }
                    }
                    if (topk_size < W) {
                        topk[topk_size++] = te;
                        bin_push(topk, topk_size);
                    } else if (te.first < topk[0].first) {
                        topk[topk_size++] = te;
                        bin_push(topk, topk_size);
                        (void)bin_pop(topk, topk_size);
                        --topk_size;
                    }
                }
                stop_size = hb0(stop_size, hb);
                topk_size = hb0(topk_size, hb);
                stop_worst = hb0f(stop_worst, hb);
                improved = hb0(improved, hb);
                if (mode == GOFANN_EARLY_STOP_ADAPTIVE && improved) finished = 0;
            }

            if (early_stop_reached(mode, finished, a.params.finish_limit, Q, expanded, passed, SW) ||
                (a.params.max_steps > 0 && step >= a.params.max_steps)) {
                active = false;
                break;
            }

            // Second round: candidate label rows, code rows; pass bits and
            // priorities (backend_pq.cu:4704-4747, 4826-4864).
            if (need_pass) lane_row_fill(a.pred, lrow, my_sample, lslab);
            const float dist = sc.score(my_sample, keep);
            scored += list_len;
            float first = dist;
            if (keep && bonuses) {
                const uint32_t global_row = label_offset + idx;
                const uint64_t rmask =
                    a.routes.row_filter_mask ? a.routes.row_filter_mask[global_row] : ~0ULL;
                const uint32_t matched = count_matching_ranges(a.routes, route, my_sample);
                first = apply_filter_bonuses(dist, (rmask & qfbit) != 0, matched,
                                             a.params.bit_filter_bonus, a.params.range_filter_bonus);
            }
            const float base = first;
            if (need_pass) {
                const bool pass = lane_pred_eval(a.pred, route, my_sample, lrow, pc);
                first = priority(base, penalty, pass);
            }

            // Threshold pre-filter (a full frontier's maximum never rises
            // within a step), then ordered admission by the half's lane 0
            // (backend_pq.cu:4889-4907).
            const bool full = heap_size >= Q + 1;
            const float thr = full ? frontier[2].first : 0.0f;
            const bool cand = keep && !(full && thr < first);
            const uint64_t cand64 = ballot(cand) & (hb ? 0xFFFFFFFF00000000ull : 0xFFFFFFFFull);
            const int n_cand = __popcll(cand64);
            const uint32_t pos = lanes_below(cand64);
            if (cand) {
                s_row[hb + pos] = idx;
                s_samp[hb + pos] = my_sample;
                s_first[hb + pos] = first;
                s_base[hb + pos] = base;
            }
            __threadfence_block();
            if (hl == 0) {
                uint64_t adm = 0;
                for (int i = 0; i < n_cand; ++i) {
                    const Entry kp = {s_first[hb + i], s_row[hb + i], s_base[hb + i],
                                      s_samp[hb + i]};
                    if (heap_size >= Q + 1 && frontier[2].first < kp.first) continue;
                    smmh_insert(frontier, heap_size, kp);
                    adm |= 1ull << i;
                    ++admitted;
                    if (heap_size >= Q + 2) smmh_pop_max(frontier, heap_size);
                }
                s_adm[half] = adm;
            }
            heap_size = hb0(heap_size, hb);
            admitted = hb0(admitted, hb);
            __threadfence_block();
            const uint64_t adm = s_adm[half];  // by compacted position
            const bool mine = cand && ((adm >> pos) & 1ull);
            const uint32_t adm_lanes = hmask(mine, hb);
            const uint32_t n_adm = static_cast<uint32_t>(__popc(adm_lanes));
            if (visited.count + n_adm <= kHashCapacity) {
                const int ins = mine ? visited.add_parallel(idx) : 0;
                visited.count += static_cast<uint32_t>(__popc(hmask(ins != 0, hb)));
            } else {
                // the set may fill: serial adds in admission order
                uint32_t added = 0;
                for (uint32_t m = adm_lanes; m; m &= m - 1) {
                    const int j = __builtin_ctz(m);
                    const uint32_t v =
                        static_cast<uint32_t>(__shfl(static_cast<int>(idx), hb + j, kWave));
                    if (hl == 0) added += static_cast<uint32_t>(visited.add_serial(v, added));
                }
                visited.count += hb0u(added, hb);
            }
            __threadfence_block();

            if (step == 1) {
                if (!pickup_h(frontier, heap_size, next, hl, hb)) {
                    exhausted = 1;
                    next = sentinel;
                } else {
                    load_node_h(next, nxt);
                }
            }
            now = next;
            cur = nxt;
        } while (false);
    }

    if (!has_route) return;
    // Sorted output (backend_pq.cu:4961-4982).
    uint32_t* oid = a.out_ids + static_cast<size_t>(route) * W;
    float* od = a.out_dists + static_cast<size_t>(route) * W;
    for (int i = hl; i < W; i += kHalf) {
        oid[i] = UINT32_MAX;
        od[i] = FLT_MAX;
    }
    __threadfence_block();
    if (hl == 0) {
        const int valid = topk_size < W ? topk_size : W;
        for (int i = 0; i < valid; ++i) {
            const ResultEntry res = bin_pop(topk, topk_size - i);
            const int out_slot = valid - 1 - i;
            if (res.second == UINT32_MAX) continue;
            oid[out_slot] = a.graph.row_to_sample[label_offset + res.second];
            od[out_slot] = res.first;
        }
    }
    const int pred_rows = hsum(static_cast<int>(pc.rows));
    const int pred_labels = hsum(static_cast<int>(pc.labels));
    if (hl == 0 && a.stats) {
        gofann_route_stats st;
        st.steps = step;
        st.expanded = expanded;
        st.passed = passed;
        st.scored = scored;
        st.pred_rows = pred_rows;
        st.pred_labels = pred_labels;
        st.admitted = admitted;
        st.exhausted = exhausted;
        a.stats[route] = st;
    }
}

// True when the two-routes-per-wave kernel serves this launch: degree <= 32,
// per-lane scoring, an LDS frontier, a visited placement it has, and the
// environment variable GOFANN_RABITQ_PAIR=1 asks for it.
bool rabitq_pair_eligible(const gofann_rabitq_view* rq, const gofann_graph_view* g,
                          const gofann_search_params* p)
{
    const char* env = std::getenv("GOFANN_RABITQ_PAIR");
    if (!env || env[0] != '1') return false;
    return g->degree <= static_cast<uint32_t>(kHalf) && rq->padded_dim / 128 < 16 &&
           p->queue_limit + 2 > kWave && p->hash_mode != GOFANN_PLACE_SPILL;
}

int rabitq_pair_search(Context* ctx, const RabitqScorer& sc, const gofann_graph_view* g,
                       const gofann_predicate_view* pred, const gofann_routes* r,
                       const gofann_search_params* p, uint32_t* out_ids, float* out_dists,
                       gofann_route_stats* stats)
{
    const Layout l = make_layout(sc.padded_dim, p->queue_limit, p->result_width);
    const uint32_t reg_lds = align16(l.bytes(kVisitedLds));
    const uint32_t reg_glob = align16(l.bytes(kVisitedGlobal));
    const int res_lds = p->hash_mode == GOFANN_PLACE_GLOBAL
                            ? 0
                            : resident_per_cu(ctx, rabitq_pair_kernel<kVisitedLds>, 2 * reg_lds);
    const int res_glob = p->hash_mode == GOFANN_PLACE_LDS
                             ? 0
                             : resident_per_cu(ctx, rabitq_pair_kernel<kVisitedGlobal>, 2 * reg_glob);
    const bool in_lds = res_lds > 0 && res_lds >= res_glob;
    if (!in_lds && res_glob <= 0)
        return ctx->fail(GOFANN_ERR_UNSUPPORTED, "per-route LDS state exceeds the workgroup limit");
    PairArgs pa;
    TraversalArgs& a = pa.t;
    a.graph = *g;
    a.pred = pred ? *pred : gofann_predicate_view{};
    a.routes = *r;
    a.params = *p;
    a.out_ids = out_ids;
    a.out_dists = out_dists;
    a.stats = stats;
    a.off_frontier = l.off_frontier;
    a.off_topk = l.off_topk;
    a.off_stop = l.off_stop;
    a.off_hash = l.off_hash;
    a.rabitq_verdict = 1;
    a.hash_global = nullptr;
    pa.region = in_lds ? reg_lds : reg_glob;
    if (!in_lds) {
        // one table per route slot, as the one-route kernel's global slab
        const size_t need = static_cast<size_t>(r->count + 1) * kHashCapacity * sizeof(uint32_t);
        a.hash_global = static_cast<uint32_t*>(ctx->scratch(Context::kScratchHash, need));
        if (!a.hash_global) return ctx->fail(GOFANN_ERR_NOMEM, "visited set scratch");
    }
    const uint32_t pairs = (r->count + 1) / 2;
    const dim3 grid(pairs), block(kWave);
    const uint32_t lds = 2 * pa.region;
    if (in_lds)
        hipLaunchKernelGGL(rabitq_pair_kernel<kVisitedLds>, grid, block, lds, ctx->stream, pa, sc);
    else
        hipLaunchKernelGGL(rabitq_pair_kernel<kVisitedGlobal>, grid, block, lds, ctx->stream, pa,
                           sc);
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("pair traversal launch");
    ctx->last_hash_in_lds = in_lds ? 1 : 0;
    ctx->last_lds_bytes = static_cast<int>(pa.region);
    ctx->last_resident = 2 * (in_lds ? res_lds : res_glob);
    return GOFANN_OK;
}

}  // namespace gofann
