// search_kernels.hip -- gfx950 label-partitioned filtered beam search.
//
// One wave64 workgroup owns one route (a query restricted to one label
// group's graph).  The per-route state lives in LDS: the distance table of
// the scorer (PQ: M x 256 fp32 ADC table; RaBitQ: the query's eight bit
// planes), the symmetric min-max frontier, the result and stop heaps and,
// when the budget allows, the 4096-slot visited hash.  Per step every lane
// takes one neighbour of the expanded node: adjacency load, visited test,
// row -> sample gather, code gather and distance, predicate pass bit and
// priority are all lane-parallel.  Only the ordered frontier admission
// (smmh2 insert / pop_max, include/smmh2.h) and the result/stop heap
// updates run on lane 0, after a parallel threshold pre-filter that removes
// candidates the reference's serial loop would reject anyway (once the
// frontier is full its maximum never increases within a step).
//
// Observable semantics follow run_pq_search_one_block
// (src/search/pq/backend_pq.cu:3980-5013) in its device-resident transport
// and run_rabitq_search_one_block (src/search/rabitq/backend_rabitq.cu:
// 3487-4291): same pickup-before-expand pipeline, verdict chain, stop heap,
// adaptive early stop, bias priority, admission test and output order.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>

#include "device_common.hpp"
#include "gofann_internal.hpp"

namespace gofann {

// ---------------------------------------------------------------------------
// Scorers: one candidate per lane.
// ---------------------------------------------------------------------------

// PQ asymmetric distance.  Table: computePQTable (backend_pq.cu:1999-2022),
// LUT[m][k] = sum_t fma(diff, diff, acc).  Distance: the reference's 32-lane
// order -- partial j sums subspaces j, j+32, ... ascending, then the xor
// butterfly 16..1 folds partials pairwise (backend_pq.cu:4711-4722).  Each
// lane evaluates that fixed tree for its own candidate in registers.
template <int kM>
struct PqScorer {
    static constexpr bool kHasExact = true;
    const uint8_t* codes;
    const float* centroids;
    const void* queries;
    int query_f32;
    uint32_t dim;
    uint32_t pq_dim;
    float* lut;
    const void* exact_base;  // resident vectors for the inline exact distance
    uint32_t query;

    __device__ int m() const { return kM > 0 ? kM : static_cast<int>(pq_dim); }

    // Exact distance of the expanded node in the reference's 32-lane order
    // (backend_pq.cu:4507-4540): lane j < 32 sums the 4-element words j,
    // j+32, ... (elements in order), then the xor butterfly 16..1.  u8 uses
    // integer squares added as float; f32 uses fma.  Wave-uniform result.
    __device__ float exact(uint32_t sample, int lane) const
    {
        float acc = 0.0f;
        const uint32_t words = dim / 4;
        if (lane < 32) {
            if (query_f32) {
                const float* b = static_cast<const float*>(exact_base) + static_cast<size_t>(sample) * dim;
                const float* q = static_cast<const float*>(queries) + static_cast<size_t>(query) * dim;
                for (uint32_t w = lane; w < words; w += 32) {
                    const float4 bv = reinterpret_cast<const float4*>(b)[w];
                    const float4 qv = reinterpret_cast<const float4*>(q)[w];
                    float d = bv.x - qv.x;
                    acc = fmaf(d, d, acc);
                    d = bv.y - qv.y;
                    acc = fmaf(d, d, acc);
                    d = bv.z - qv.z;
                    acc = fmaf(d, d, acc);
                    d = bv.w - qv.w;
                    acc = fmaf(d, d, acc);
                }
            } else {
                const uint32_t* b = reinterpret_cast<const uint32_t*>(
                    static_cast<const uint8_t*>(exact_base) + static_cast<size_t>(sample) * dim);
                const uint32_t* q = reinterpret_cast<const uint32_t*>(
                    static_cast<const uint8_t*>(queries) + static_cast<size_t>(query) * dim);
                for (uint32_t w = lane; w < words; w += 32) {
                    const uint32_t bw = b[w], qw = q[w];
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const int diff = static_cast<int>((bw >> (8 * t)) & 0xffu) -
                                         static_cast<int>((qw >> (8 * t)) & 0xffu);
                        acc += static_cast<float>(diff * diff);
                    }
                }
            }
        }
#pragma unroll
        for (int off = 16; off > 0; off >>= 1) acc = acc + __shfl_xor(acc, off, 32);
        return bcast0f(acc);
    }

    __device__ void setup(uint32_t q, int lane, unsigned char* lds)
    {
        lut = reinterpret_cast<float*>(lds);
        query = q;
        const int M = m();
        const int sub = static_cast<int>(dim) / M;
        const float* qf = static_cast<const float*>(queries) + static_cast<size_t>(q) * dim;
        const uint8_t* qu = static_cast<const uint8_t*>(queries) + static_cast<size_t>(q) * dim;
        for (int k = lane; k < 256; k += kWave) {
            const float* crow = centroids + static_cast<size_t>(k) * dim;
            for (int mm = 0; mm < M; ++mm) {
                float acc = 0.0f;
                for (int t = 0; t < sub; ++t) {
                    const int d = mm * sub + t;
                    const float qv = query_f32 ? qf[d] : static_cast<float>(qu[d]);
                    const float diff = qv - crow[d];
                    acc = fmaf(diff, diff, acc);
                }
                lut[mm * 256 + k] = acc;
            }
        }
    }

    __device__ float score(uint32_t sample, bool active) const
    {
        float s[32];
#pragma unroll
        for (int j = 0; j < 32; ++j) s[j] = 0.0f;
        if (active) {
            const uint8_t* row = codes + static_cast<size_t>(sample) * m();
            if constexpr (kM > 0 && kM % 16 == 0) {
                uint4 w[kM / 16];
#pragma unroll
                for (int i = 0; i < kM / 16; ++i) w[i] = reinterpret_cast<const uint4*>(row)[i];
#pragma unroll
                for (int mm = 0; mm < kM; ++mm) {
                    const uint32_t word = reinterpret_cast<const uint32_t*>(w)[mm >> 2];
                    const uint32_t c = (word >> (8 * (mm & 3))) & 0xffu;
                    s[mm & 31] += lut[mm * 256 + c];
                }
            } else {
                const int M = m();
                for (int mm = 0; mm < M; ++mm) {
                    const float v = lut[mm * 256 + row[mm]];
                    // Runtime index into the partials: select chain keeps
                    // the partials in registers.
#pragma unroll
                    for (int j = 0; j < 32; ++j)
                        if ((mm & 31) == j) s[j] += v;
                }
            }
        }
#pragma unroll
        for (int off = 16; off > 0; off >>= 1) {
#pragma unroll
            for (int j = 0; j < off; ++j) s[j] = s[j] + s[j + off];
        }
        return s[0];
    }
};

// RaBitQ one-bit estimate (score_rabitq_code_device, backend_rabitq.cu:
// 3100-3200, int8 query path).  ip_int = sum_d q8[d] * bit[d] is computed as
// sum_j w_j * popcount(plane_j & code) over the query's two's-complement bit
// planes (w_j = 2^j, w_7 = -128), which equals the reference's dp4a dot over
// nibble masks exactly.  Planes are stored MSB-first like the codes: word w,
// bit 31-b <-> dimension 32w+b.  Estimate: fma(f_rescale, ip*scale + k1,
// f_add + g[anchor]).
struct RabitqScorer {
    static constexpr bool kHasExact = false;
    const uint8_t* codes;
    const float* factors;
    const uint32_t* anchor_ids;
    const int8_t* q8;
    const float* q_scale;
    const float* q_k1;
    const float* centroid_dists;
    uint32_t num_anchors;
    uint32_t padded_dim;
    uint32_t* planes;  // LDS [padded_dim/32][8]
    float scale;
    float k1;
    const float* g_row;

    __device__ void setup(uint32_t q, int lane, unsigned char* lds)
    {
        planes = reinterpret_cast<uint32_t*>(lds);
        const uint32_t words = padded_dim / 32;
        const int8_t* qrow = q8 + static_cast<size_t>(q) * padded_dim;
        for (uint32_t w = lane; w < words; w += kWave) {
            uint32_t pl[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (uint32_t b = 0; b < 32; ++b) {
                const uint32_t v = static_cast<uint8_t>(qrow[w * 32 + b]);
#pragma unroll
                for (int j = 0; j < 8; ++j) pl[j] |= ((v >> j) & 1u) << (31u - b);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) planes[w * 8 + j] = pl[j];
        }
        scale = q_scale[q];
        k1 = q_k1[q];
        g_row = centroid_dists + static_cast<size_t>(q) * num_anchors;
    }

    __device__ float score(uint32_t sample, bool active) const
    {
        if (!active) return 0.0f;
        const uint32_t words = padded_dim / 32;
        const uint4* row = reinterpret_cast<const uint4*>(codes + static_cast<size_t>(sample) * (padded_dim / 8));
        uint32_t cnt[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (uint32_t w4 = 0; w4 < words / 4; ++w4) {
            const uint4 c = row[w4];
            const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint4 p0 = reinterpret_cast<const uint4*>(planes)[(w4 * 4 + t) * 2];
                const uint4 p1 = reinterpret_cast<const uint4*>(planes)[(w4 * 4 + t) * 2 + 1];
                cnt[0] += __popc(p0.x & cw[t]);
                cnt[1] += __popc(p0.y & cw[t]);
                cnt[2] += __popc(p0.z & cw[t]);
                cnt[3] += __popc(p0.w & cw[t]);
                cnt[4] += __popc(p1.x & cw[t]);
                cnt[5] += __popc(p1.y & cw[t]);
                cnt[6] += __popc(p1.z & cw[t]);
                cnt[7] += __popc(p1.w & cw[t]);
            }
        }
        int32_t ip = 0;
#pragma unroll
        for (int j = 0; j < 7; ++j) ip += static_cast<int32_t>(cnt[j]) << j;
        ip -= 128 * static_cast<int32_t>(cnt[7]);
        const uint32_t anchor = anchor_ids[sample];
        const float f_add = factors[static_cast<size_t>(sample) * 3];
        const float f_rescale = factors[static_cast<size_t>(sample) * 3 + 1];
        const float short_ip = static_cast<float>(ip) * scale;
        const float t = short_ip + k1;
        return fmaf(f_rescale, t, f_add + g_row[anchor]);
    }

    __device__ int32_t ip_int(uint32_t sample) const
    {
        const uint32_t words = padded_dim / 32;
        const uint32_t* row = reinterpret_cast<const uint32_t*>(codes + static_cast<size_t>(sample) * (padded_dim / 8));
        int32_t ip = 0;
        for (uint32_t w = 0; w < words; ++w) {
            const uint32_t cw = row[w];
            for (int j = 0; j < 8; ++j) {
                const int32_t c = __popc(planes[w * 8 + j] & cw);
                ip += (j == 7) ? -128 * c : (c << j);
            }
        }
        return ip;
    }
};

// ---------------------------------------------------------------------------
// Frontier helpers (wave-cooperative).
// ---------------------------------------------------------------------------

// pickup_next_unused_from_native_frontier (backend_pq.cu:844-892): unused
// entry of least `first`, lowest index on ties; lane 0 marks it used.
__device__ bool pickup(Entry* f, int size, Entry& out, int lane)
{
    int best = -1;
    float bv = 0.0f;
    for (int i = lane + 1; i < size; i += kWave) {
        const Entry e = f[i];
        if (e.second & kPoolUsed) continue;
        if (best < 0 || e.first < bv) {
            best = i;
            bv = e.first;
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const int ob = __shfl_xor(best, off, kWave);
        const float ov = __shfl_xor(bv, off, kWave);
        if (ob >= 0 && (best < 0 || ov < bv || (!(bv < ov) && ob < best))) {
            best = ob;
            bv = ov;
        }
    }
    best = bcast0(best);
    if (best < 0) return false;
    out = f[best];
    __syncthreads();
    if (lane == 0) f[best].second |= kPoolUsed;
    __syncthreads();
    return true;
}

// minimum_pending_base (gpu_predicate_index.cuh:147-160) over the reserved
// current/next entries and every unused frontier entry.
__device__ float min_pending_base(const Entry* f, int size, const Entry& now, const Entry& next,
                                  int lane)
{
    float m = FLT_MAX;
    for (int i = lane + 1; i < size; i += kWave) {
        const Entry e = f[i];
        if (!(e.second & kPoolUsed)) m = fminf(m, e.base);
    }
    m = wave_min(m);
    m = fminf(m, now.base);
    m = fminf(m, next.base);
    return m;
}

struct TraversalArgs {
    gofann_graph_view graph;
    gofann_predicate_view pred;
    gofann_routes routes;
    gofann_search_params params;
    uint32_t* out_ids;
    float* out_dists;
    gofann_route_stats* stats;
    uint32_t* hash_global;  // [routes][4096] when the hash is not in LDS
    uint32_t off_frontier;
    uint32_t off_topk;
    uint32_t off_stop;
    uint32_t off_hash;
    int rabitq_verdict;
};

template <class Scorer, bool kHashLds>
__global__ __launch_bounds__(64) void traversal_kernel(TraversalArgs a, Scorer sc)
{
    extern __shared__ __align__(16) unsigned char lds[];
    __shared__ uint32_t s_list[kMaxDegree];
    __shared__ uint32_t s_cand[kMaxDegree];
    __shared__ float s_first[kMaxDegree];
    __shared__ float s_base[kMaxDegree];

    const int lane = static_cast<int>(threadIdx.x);
    const uint32_t slot = xcd_slot(blockIdx.x, gridDim.x);
    if (slot >= a.routes.count) return;
    const uint32_t route = a.routes.launch_order ? a.routes.launch_order[slot] : slot;

    Entry* frontier = reinterpret_cast<Entry*>(lds + a.off_frontier);
    ResultEntry* topk = reinterpret_cast<ResultEntry*>(lds + a.off_topk);
    StopEntry* stop = reinterpret_cast<StopEntry*>(lds + a.off_stop);
    // The global slab holds one table per launch slot (slot < routes.count).
    VisitedHash<kHashLds> hash{kHashLds ? reinterpret_cast<uint32_t*>(lds + a.off_hash)
                                        : a.hash_global + static_cast<size_t>(slot) * kHashCapacity};

    const int Q = a.params.queue_limit;
    const int W = a.params.result_width;
    const int SW = a.params.stop_width;
    const int mode = a.params.early_stop_mode;
    const bool bias = a.params.predicate_bias != 0;
    const bool bonuses = a.params.bit_filter_bonus != 1.0f || a.params.range_filter_bonus != 1.0f;

    const uint32_t group = a.routes.route_group[route];
    const uint32_t label_offset = a.graph.label_offset[group];
    const uint32_t query = a.routes.route_query[route];
    const uint32_t begin_id = a.routes.route_start[route];
    const uint64_t qfbit = a.routes.query_filter_bits ? a.routes.query_filter_bits[route] : ~0ULL;
    const uint32_t active_ranges =
        count_active_ranges(a.routes.range_modes, route, a.routes.range_count);
    const bool enabled = pred_enabled(a.pred, route);
    const bool compiled = a.pred.route_compiled != nullptr && a.pred.route_compiled[route] != 0;
    const uint32_t degree = a.graph.degree < static_cast<uint32_t>(kMaxDegree)
                                ? a.graph.degree
                                : static_cast<uint32_t>(kMaxDegree);

    hash.clear(lane);
    sc.setup(query, lane, lds);
    __threadfence_block();
    __syncthreads();

    PredCounters pc{0, 0};
    int scored = 1;
    int admitted = 0;

    // Seed (backend_pq.cu:4164-4187).
    const uint32_t begin_sample = a.graph.row_to_sample[label_offset + begin_id];
    const float start = bcast0f(sc.score(begin_sample, lane == 0));
    const float penalty = bias ? bias_penalty(a.pred.alpha, start) : 0.0f;

    int heap_size = 1;
    int stop_size = 0;
    int topk_size = 0;
    int finished = 0;
    int exhausted = 0;
    int expanded = 0;
    int passed = 0;
    float stop_worst = -FLT_MAX;
    const Entry sentinel = {FLT_MAX, UINT32_MAX, FLT_MAX};
    if (lane == 0) {
        const Entry kp = {start, begin_id, start};
        smmh_insert(frontier, heap_size, kp);
        hash.add(begin_id);
    }
    heap_size = bcast0(heap_size);
    __threadfence_block();
    __syncthreads();

    Entry now = sentinel;
    Entry next = sentinel;
    if (!pickup(frontier, heap_size, now, lane)) {
        exhausted = 1;
        now = sentinel;
    }

    int step = 0;
    while (step == 0 || heap_size > 1) {
        const uint32_t now_local = now.second & ~kPoolUsed;
        ++step;

        if (step != 1) {
            const bool found = pickup(frontier, heap_size, next, lane);
            if (!found) {
                exhausted = 1;
                next = sentinel;
            } else if (stop_size == SW) {
                float pending = next.first;
                if (a.pred.pending_base_stop && enabled)
                    pending = min_pending_base(frontier, heap_size, now, next, lane);
                if (mode != GOFANN_EARLY_STOP_OFF && stop_worst <= pending) ++finished;
            }
        }

        // Verdict of the expanded node (backend_pq.cu:4393-4441).  Skipped
        // when the pool ran dry: the loop leaves below before reading it.
        int filt = 1;
        float rank = now.base;
        if (!exhausted) {
            const uint32_t global_row = label_offset + now_local;
            const uint32_t sample = a.graph.row_to_sample[global_row];
            PredCounters c{0, 0};
            if (enabled) filt = pred_matches(a.pred, route, sample, c) ? 1 : 2;
            const bool fallback = a.rabitq_verdict ? !compiled : (!enabled && !compiled);
            if (fallback) {
                const uint64_t rmask =
                    a.routes.row_filter_mask ? a.routes.row_filter_mask[global_row] : ~0ULL;
                const bool bit_match = (rmask & qfbit) != 0;
                const uint32_t matched = count_matching_ranges(a.routes, route, sample);
                const bool exact_range = active_ranges == 0 || matched == active_ranges;
                filt = (filt == 1 && bit_match && exact_range) ? 1 : 2;
            }
            if (lane == 0) {
                pc.rows += c.rows;
                pc.labels += c.labels;
            }
            // Inline exact distance of a passing node ranks the heaps
            // (backend_pq.cu:4507-4546, 4566-4572).
            if constexpr (Scorer::kHasExact) {
                if (filt == 1 && a.params.inline_exact_rerank) rank = sc.exact(sample, lane);
            }
        }
        const float current = now.base;

        if (exhausted ||
            early_stop_reached(mode, finished, a.params.finish_limit, Q, expanded, passed, SW) ||
            (a.params.max_steps > 0 && step >= a.params.max_steps))
            break;

        // Result and stop heaps (backend_pq.cu:4558-4631).
        ++expanded;
        if (filt == 1) {
            ++passed;
            int improved = 0;
            if (lane == 0) {
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
            stop_size = bcast0(stop_size);
            topk_size = bcast0(topk_size);
            stop_worst = bcast0f(stop_worst);
            improved = bcast0(improved);
            if (mode == GOFANN_EARLY_STOP_ADAPTIVE && improved) finished = 0;
        }

        // Unvisited neighbours in adjacency order (backend_pq.cu:4636-4684):
        // lane i tests neighbour i; a ballot compacts the survivors in order.
        uint32_t idx = UINT32_MAX;
        bool keep = false;
        if (static_cast<uint32_t>(lane) < degree) {
            idx = a.graph.graph[static_cast<size_t>(label_offset + now_local) * a.graph.degree + lane];
            keep = idx != UINT32_MAX && !hash.test(idx);
        }
        const uint64_t keep_mask = ballot(keep);
        const int list_len = __popcll(keep_mask);
        if (keep) s_list[lanes_below(keep_mask)] = idx;
        __syncthreads();

        if (early_stop_reached(mode, finished, a.params.finish_limit, Q, expanded, passed, SW) ||
            (a.params.max_steps > 0 && step >= a.params.max_steps))
            break;

        // Lane-parallel scoring, predicate pass bits and priorities
        // (backend_pq.cu:4704-4747, 4826-4864).
        const bool active = lane < list_len;
        const uint32_t my_row = active ? s_list[lane] : 0u;
        const uint32_t my_sample = active ? a.graph.row_to_sample[label_offset + my_row] : 0u;
        const float dist = sc.score(my_sample, active);
        scored += list_len;
        float first = dist;
        if (active && bonuses) {
            const uint32_t global_row = label_offset + my_row;
            const uint64_t rmask =
                a.routes.row_filter_mask ? a.routes.row_filter_mask[global_row] : ~0ULL;
            const uint32_t matched = count_matching_ranges(a.routes, route, my_sample);
            first = apply_filter_bonuses(dist, (rmask & qfbit) != 0, matched,
                                         a.params.bit_filter_bonus, a.params.range_filter_bonus);
        }
        const float base = first;
        if (active && bias && enabled) {
            const bool pass = pred_matches(a.pred, route, my_sample, pc);
            first = priority(base, penalty, pass);
        }

        // Threshold pre-filter: with a full frontier (size >= Q+1) the serial
        // loop skips any candidate above frontier[2]; that maximum can only
        // fall during the step, so such candidates are dropped here.
        const bool full = heap_size >= Q + 1;
        const float thr = full ? frontier[2].first : 0.0f;
        const bool cand = active && !(full && thr < first);
        const uint64_t cand_mask = ballot(cand);
        const int n_cand = __popcll(cand_mask);
        if (cand) {
            const uint32_t p = lanes_below(cand_mask);
            s_cand[p] = my_row;
            s_first[p] = first;
            s_base[p] = base;
        }
        __syncthreads();

        // Ordered admission (backend_pq.cu:4889-4907).
        if (lane == 0) {
            for (int i = 0; i < n_cand; ++i) {
                const Entry kp = {s_first[i], s_cand[i], s_base[i]};
                if (heap_size >= Q + 1 && frontier[2].first < kp.first) continue;
                smmh_insert(frontier, heap_size, kp);
                hash.add(kp.second);
                ++admitted;
                if (heap_size >= Q + 2) smmh_pop_max(frontier, heap_size);
            }
        }
        heap_size = bcast0(heap_size);
        __threadfence_block();
        __syncthreads();

        if (step == 1) {
            if (!pickup(frontier, heap_size, next, lane)) {
                exhausted = 1;
                next = sentinel;
            }
        }
        now = next;
    }

    // Sorted output (backend_pq.cu:4961-4982).
    uint32_t* oid = a.out_ids + static_cast<size_t>(route) * W;
    float* od = a.out_dists + static_cast<size_t>(route) * W;
    for (int i = lane; i < W; i += kWave) {
        oid[i] = UINT32_MAX;
        od[i] = FLT_MAX;
    }
    __syncthreads();
    if (lane == 0) {
        const int valid = topk_size < W ? topk_size : W;
        for (int i = 0; i < valid; ++i) {
            const ResultEntry res = bin_pop(topk, topk_size - i);
            const int out_slot = valid - 1 - i;
            if (res.second == UINT32_MAX) continue;
            oid[out_slot] = a.graph.row_to_sample[label_offset + res.second];
            od[out_slot] = res.first;
        }
    }
    const int pred_rows = wave_sum(static_cast<int>(pc.rows));
    const int pred_labels = wave_sum(static_cast<int>(pc.labels));
    if (lane == 0 && a.stats) {
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

// Batched scoring of explicit (query, sample) pairs: one pair per lane.
template <int kM>
__global__ __launch_bounds__(64) void pq_score_kernel(PqScorer<kM> sc, const uint32_t* q_idx,
                                                     const uint32_t* s_idx, uint32_t n, float* out)
{
    extern __shared__ __align__(16) unsigned char lds[];
    // One workgroup per pair-chunk of 64 sharing one query is not assumed:
    // rebuild the table per distinct query of the chunk.
    const int lane = static_cast<int>(threadIdx.x);
    const uint32_t i = blockIdx.x * kWave + lane;
    const uint32_t first = blockIdx.x * kWave;
    const uint32_t last = first + kWave < n ? first + kWave : n;
    for (uint32_t j = first; j < last; ++j) {
        const uint32_t qj = q_idx[j];
        if (j > first && q_idx[j - 1] == qj) continue;
        __syncthreads();
        sc.setup(qj, lane, lds);
        __syncthreads();
        const bool mine = i < n && q_idx[i] == qj;
        const float d = sc.score(mine ? s_idx[i] : 0u, mine);
        if (mine) out[i] = d;
    }
}

__global__ __launch_bounds__(64) void rabitq_score_kernel(RabitqScorer sc, const uint32_t* q_idx,
                                                         const uint32_t* s_idx, uint32_t n,
                                                         float* out, int32_t* ip_out)
{
    extern __shared__ __align__(16) unsigned char lds[];
    const int lane = static_cast<int>(threadIdx.x);
    const uint32_t i = blockIdx.x * kWave + lane;
    const uint32_t first = blockIdx.x * kWave;
    const uint32_t last = first + kWave < n ? first + kWave : n;
    for (uint32_t j = first; j < last; ++j) {
        const uint32_t qj = q_idx[j];
        if (j > first && q_idx[j - 1] == qj) continue;
        __syncthreads();
        sc.setup(qj, lane, lds);
        __syncthreads();
        const bool mine = i < n && q_idx[i] == qj;
        if (mine) {
            out[i] = sc.score(s_idx[i], true);
            if (ip_out) ip_out[i] = sc.ip_int(s_idx[i]);
        }
    }
}

// ---------------------------------------------------------------------------
// Host launchers.
// ---------------------------------------------------------------------------
namespace {

uint32_t align16(uint32_t x) { return (x + 15u) & ~15u; }

struct Layout {
    uint32_t off_frontier, off_topk, off_stop, off_hash, total_no_hash, total_with_hash;
};

Layout make_layout(uint32_t scorer_bytes, int Q, int W)
{
    Layout l;
    l.off_frontier = align16(scorer_bytes);
    l.off_topk = align16(l.off_frontier + static_cast<uint32_t>(Q + 2) * sizeof(Entry));
    l.off_stop = align16(l.off_topk + static_cast<uint32_t>(W + 1) * sizeof(ResultEntry));
    l.off_hash = align16(l.off_stop + static_cast<uint32_t>(kMaxStopWidth + 1) * sizeof(StopEntry));
    l.total_no_hash = l.off_hash;
    l.total_with_hash = l.off_hash + kHashCapacity * sizeof(uint32_t);
    return l;
}

// Static LDS of traversal_kernel (s_list, s_cand, s_first, s_base).
constexpr uint32_t kStaticLds = 4 * kMaxDegree * 4;

int check_params(Context* ctx, const gofann_graph_view* g, const gofann_routes* r,
                 const gofann_search_params* p)
{
    if (!g || !r || !p) return ctx->fail(GOFANN_ERR_INVALID, "null view");
    if (p->queue_limit < 2 || p->queue_limit > 1024)
        return ctx->fail(GOFANN_ERR_INVALID, "queue_limit must be in [2, 1024]");
    if (p->result_width < 1 || p->result_width > 512)
        return ctx->fail(GOFANN_ERR_INVALID, "result_width must be in [1, 512]");
    if (p->stop_width < 0 || p->stop_width > kMaxStopWidth)
        return ctx->fail(GOFANN_ERR_INVALID, "stop_width must be in [0, 10]");
    if (p->early_stop_mode < 0 || p->early_stop_mode > 2)
        return ctx->fail(GOFANN_ERR_INVALID, "unknown early stop mode");
    if (!g->graph || !g->row_to_sample || !g->label_offset || g->degree == 0)
        return ctx->fail(GOFANN_ERR_INVALID, "graph view incomplete");
    if (r->count > 0 && (!r->route_query || !r->route_group || !r->route_start))
        return ctx->fail(GOFANN_ERR_INVALID, "route arrays missing");
    return GOFANN_OK;
}

template <class Scorer>
int launch_traversal(Context* ctx, const Scorer& sc, uint32_t scorer_bytes,
                     const gofann_graph_view* g, const gofann_predicate_view* pred,
                     const gofann_routes* r, const gofann_search_params* p, uint32_t* out_ids,
                     float* out_dists, gofann_route_stats* stats, int rabitq_verdict)
{
    if (r->count == 0) return GOFANN_OK;
    const Layout l = make_layout(scorer_bytes, p->queue_limit, p->result_width);
    TraversalArgs a;
    a.graph = *g;
    if (pred) {
        a.pred = *pred;
    } else {
        a.pred = gofann_predicate_view{};
    }
    a.routes = *r;
    a.params = *p;
    a.out_ids = out_ids;
    a.out_dists = out_dists;
    a.stats = stats;
    a.off_frontier = l.off_frontier;
    a.off_topk = l.off_topk;
    a.off_stop = l.off_stop;
    a.off_hash = l.off_hash;
    a.rabitq_verdict = rabitq_verdict;
    a.hash_global = nullptr;

    // The hash goes to LDS when that does not lower the number of routes a
    // CU holds (LDS is the occupancy limit of this kernel).
    const uint32_t budget = static_cast<uint32_t>(ctx->lds_per_cu);
    const uint32_t per_no = l.total_no_hash + kStaticLds;
    const uint32_t per_with = l.total_with_hash + kStaticLds;
    if (per_no > static_cast<uint32_t>(ctx->lds_per_block))
        return ctx->fail(GOFANN_ERR_UNSUPPORTED, "per-route LDS state exceeds the workgroup limit");
    const bool hash_lds = per_with <= static_cast<uint32_t>(ctx->lds_per_block) &&
                          (budget / per_with) >= (budget / per_no);
    const dim3 grid(r->count), block(kWave);
    if (hash_lds) {
        auto kern = traversal_kernel<Scorer, true>;
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                hipFuncAttributeMaxDynamicSharedMemorySize,
                                static_cast<int>(l.total_with_hash)) != hipSuccess)
            return ctx->fail_hip("hipFuncSetAttribute traversal");
        hipLaunchKernelGGL(kern, grid, block, l.total_with_hash, ctx->stream, a, sc);
    } else {
        const size_t need = static_cast<size_t>(r->count) * kHashCapacity * sizeof(uint32_t);
        a.hash_global = static_cast<uint32_t*>(ctx->scratch(Context::kScratchHash, need));
        if (!a.hash_global) return ctx->fail(GOFANN_ERR_NOMEM, "visited hash scratch");
        auto kern = traversal_kernel<Scorer, false>;
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                hipFuncAttributeMaxDynamicSharedMemorySize,
                                static_cast<int>(l.total_no_hash)) != hipSuccess)
            return ctx->fail_hip("hipFuncSetAttribute traversal");
        hipLaunchKernelGGL(kern, grid, block, l.total_no_hash, ctx->stream, a, sc);
    }
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("traversal launch");
    ctx->last_hash_in_lds = hash_lds ? 1 : 0;
    ctx->last_lds_bytes = static_cast<int>(hash_lds ? l.total_with_hash : l.total_no_hash) +
                          static_cast<int>(kStaticLds);
    return GOFANN_OK;
}

template <int kM>
PqScorer<kM> make_pq_scorer(const gofann_pq_view* pq, const void* queries, int query_elem)
{
    PqScorer<kM> sc;
    sc.codes = pq->codes;
    sc.centroids = pq->centroids;
    sc.queries = queries;
    sc.query_f32 = query_elem == GOFANN_ELEM_F32 ? 1 : 0;
    sc.dim = pq->dim;
    sc.pq_dim = pq->pq_dim;
    sc.lut = nullptr;
    sc.exact_base = pq->exact_base;
    sc.query = 0;
    return sc;
}

int check_pq(Context* ctx, const gofann_pq_view* pq, const void* queries, int query_elem)
{
    if (!pq || !pq->codes || !pq->centroids || !queries)
        return ctx->fail(GOFANN_ERR_INVALID, "PQ view incomplete");
    if (pq->pq_dim == 0 || pq->pq_dim > 256 || pq->dim % pq->pq_dim != 0)
        return ctx->fail(GOFANN_ERR_INVALID, "pq_dim must divide dim and be in [1, 256]");
    if (query_elem != GOFANN_ELEM_U8 && query_elem != GOFANN_ELEM_F32)
        return ctx->fail(GOFANN_ERR_INVALID, "PQ queries must be u8 or f32");
    if (pq->exact_base != nullptr && pq->dim % 4 != 0)
        return ctx->fail(GOFANN_ERR_INVALID, "inline exact distances need dim % 4 == 0");
    return GOFANN_OK;
}

RabitqScorer make_rabitq_scorer(const gofann_rabitq_view* rq, const gofann_rabitq_queries* pre)
{
    RabitqScorer sc;
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
    sc.scale = 0.0f;
    sc.k1 = 0.0f;
    sc.g_row = nullptr;
    return sc;
}

int check_rabitq(Context* ctx, const gofann_rabitq_view* rq, const gofann_rabitq_queries* pre)
{
    if (!rq || !pre || !rq->codes || !rq->factors || !rq->anchor_ids || !pre->q8 || !pre->scale ||
        !pre->k1 || !pre->centroid_dists)
        return ctx->fail(GOFANN_ERR_INVALID, "RaBitQ view incomplete");
    if (rq->padded_dim == 0 || rq->padded_dim % 128 != 0)
        return ctx->fail(GOFANN_ERR_INVALID, "padded_dim must be a positive multiple of 128");
    return GOFANN_OK;
}

}  // namespace

int pq_search(Context* ctx, const gofann_pq_view* pq, const void* queries, int query_elem,
              const gofann_graph_view* g, const gofann_predicate_view* pred,
              const gofann_routes* r, const gofann_search_params* p, uint32_t* out_ids,
              float* out_dists, gofann_route_stats* stats)
{
    int rc = check_pq(ctx, pq, queries, query_elem);
    if (rc) return rc;
    rc = check_params(ctx, g, r, p);
    if (rc) return rc;
    if (p->inline_exact_rerank && pq->exact_base == nullptr)
        return ctx->fail(GOFANN_ERR_INVALID, "inline exact rerank needs gofann_pq_view.exact_base");
    const uint32_t lut_bytes = pq->pq_dim * 256u * 4u;
    switch (pq->pq_dim) {
    case 16:
        return launch_traversal(ctx, make_pq_scorer<16>(pq, queries, query_elem), lut_bytes, g,
                                pred, r, p, out_ids, out_dists, stats, 0);
    case 32:
        return launch_traversal(ctx, make_pq_scorer<32>(pq, queries, query_elem), lut_bytes, g,
                                pred, r, p, out_ids, out_dists, stats, 0);
    case 48:
        return launch_traversal(ctx, make_pq_scorer<48>(pq, queries, query_elem), lut_bytes, g,
                                pred, r, p, out_ids, out_dists, stats, 0);
    case 64:
        return launch_traversal(ctx, make_pq_scorer<64>(pq, queries, query_elem), lut_bytes, g,
                                pred, r, p, out_ids, out_dists, stats, 0);
    default:
        return launch_traversal(ctx, make_pq_scorer<0>(pq, queries, query_elem), lut_bytes, g,
                                pred, r, p, out_ids, out_dists, stats, 0);
    }
}

int rabitq_search(Context* ctx, const gofann_rabitq_view* rq, const gofann_rabitq_queries* pre,
                  const gofann_graph_view* g, const gofann_predicate_view* pred,
                  const gofann_routes* r, const gofann_search_params* p, uint32_t* out_ids,
                  float* out_dists, gofann_route_stats* stats)
{
    int rc = check_rabitq(ctx, rq, pre);
    if (rc) return rc;
    rc = check_params(ctx, g, r, p);
    if (rc) return rc;
    if (p->inline_exact_rerank)
        return ctx->fail(GOFANN_ERR_UNSUPPORTED, "RaBitQ traversal has no inline exact rerank");
    const uint32_t plane_bytes = rq->padded_dim;  // 8 planes x padded_dim bits
    return launch_traversal(ctx, make_rabitq_scorer(rq, pre), plane_bytes, g, pred, r, p, out_ids,
                            out_dists, stats, 1);
}

int pq_score(Context* ctx, const gofann_pq_view* pq, const void* queries, int query_elem,
             const uint32_t* q_idx, const uint32_t* s_idx, uint32_t n, float* out)
{
    int rc = check_pq(ctx, pq, queries, query_elem);
    if (rc) return rc;
    if (n == 0) return GOFANN_OK;
    const uint32_t lut_bytes = pq->pq_dim * 256u * 4u;
    const dim3 grid((n + kWave - 1) / kWave), block(kWave);
    switch (pq->pq_dim) {
    case 32:
        hipLaunchKernelGGL(pq_score_kernel<32>, grid, block, lut_bytes, ctx->stream,
                           make_pq_scorer<32>(pq, queries, query_elem), q_idx, s_idx, n, out);
        break;
    case 48:
        hipLaunchKernelGGL(pq_score_kernel<48>, grid, block, lut_bytes, ctx->stream,
                           make_pq_scorer<48>(pq, queries, query_elem), q_idx, s_idx, n, out);
        break;
    default:
        hipLaunchKernelGGL(pq_score_kernel<0>, grid, block, lut_bytes, ctx->stream,
                           make_pq_scorer<0>(pq, queries, query_elem), q_idx, s_idx, n, out);
        break;
    }
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("pq_score launch");
    return GOFANN_OK;
}

int rabitq_score(Context* ctx, const gofann_rabitq_view* rq, const gofann_rabitq_queries* pre,
                 const uint32_t* q_idx, const uint32_t* s_idx, uint32_t n, float* out,
                 int32_t* ip_int)
{
    int rc = check_rabitq(ctx, rq, pre);
    if (rc) return rc;
    if (n == 0) return GOFANN_OK;
    const dim3 grid((n + kWave - 1) / kWave), block(kWave);
    hipLaunchKernelGGL(rabitq_score_kernel, grid, block, rq->padded_dim, ctx->stream,
                       make_rabitq_scorer(rq, pre), q_idx, s_idx, n, out, ip_int);
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("rabitq_score launch");
    return GOFANN_OK;
}

}  // namespace gofann
