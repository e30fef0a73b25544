// traversal.hpp -- gfx950 label-partitioned filtered beam search: scorers,
// the traversal kernel template and its host launch templates.  The PQ and
// RaBitQ entry points instantiate it in separate translation units
// (pq_search*.hip, rabitq_search.hip) so the build compiles them in parallel.
//
// One wave64 workgroup owns one route (a query restricted to one label
// group's graph).  Per-route state lives in LDS: the scorer's query-side
// table (PQ: the M x 256 fp32 ADC table, or just the fp32 query when table
// entries are computed on demand from the L2-resident centroid table;
// RaBitQ: the query's eight bit planes), the symmetric min-max frontier, the
// result and stop heaps and, when it does not lower residency, the 4096-slot
// visited hash.
//
// A step is a short chain of dependent memory rounds, so throughput comes
// from the number of routes resident per CU and from keeping each chain
// short:
//   * the node picked for the next step has its adjacency row, neighbour
//     sample ids, CSR bounds and exact-distance operand words loaded while
//     the current step runs (frontier entries carry the sample id);
//   * every lane takes one neighbour: visited test, sample, code gather,
//     distance, predicate pass bit and priority are lane-parallel, and the
//     expanded node's label row is read once across the wave;
//   * only the ordered frontier admission (smmh2 insert / pop_max) and the
//     result/stop heap updates run on lane 0, after a threshold pre-filter
//     that drops candidates the serial loop would reject anyway (a full
//     frontier's maximum never rises within a step); visited-set inserts of
//     the admitted candidates are lane-parallel compare-and-swaps.
//
// Observable semantics follow run_pq_search_one_block
// (src/search/pq/backend_pq.cu:3980-5013) in its device-resident transport
// and run_rabitq_search_one_block (src/search/rabitq/backend_rabitq.cu:
// 3487-4291): same pickup-before-expand pipeline, verdict chain, stop heap,
// adaptive early stop, bias priority, admission test, visited set and output
// order, bit for bit.
#pragma once

#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>

#include "device_common.hpp"
#include "gofann_internal.hpp"

// Minimum waves per SIMD the traversal kernel is compiled for (register
// budget: 4 waves -> at most 128 VGPRs; 5 spills the scorer state and is
// slower: C4 193.5 against 149.2 ms; C2 PQ route 181.1 against 180.3 ms,
// where the visited table also leaves LDS).
#ifndef GOFANN_TRAVERSAL_MIN_WAVES
#define GOFANN_TRAVERSAL_MIN_WAVES 4
#endif

namespace gofann {

// Operand words of the inline exact distance of u8 vectors held by lanes
// 0..31: words lane and lane+32 (four elements each).  f32 vectors are read
// when the distance is computed.
struct ExactWords {
    uint32_t w0;
    uint32_t w1;
};

// ---------------------------------------------------------------------------
// Scorers: one candidate per lane.
// ---------------------------------------------------------------------------

// PQ asymmetric distance.  Table entries: computePQTable
// (backend_pq.cu:1999-2022), LUT[m][k] = sum_t fma(diff, diff, acc) over the
// subspace's dims in order, diff = q - C[k].  kSub selects where entries come
// from: 0 = an M x 256 table built in LDS; > 0 = computed when needed from the
// L2-resident centroid table with kSub dims per subspace (< 0: runtime
// width) -- the same fma chain, hence the same bits, with 4 B of LDS per
// dimension instead of 1 KiB per subspace.  Distance: the reference's
// 32-lane order -- partial j sums subspaces j, j+32, ... ascending, then the
// xor butterfly 16..1 folds partials pairwise (backend_pq.cu:4711-4722).
// Each lane evaluates that fixed tree for its own candidate in registers,
// building the 16 first-level sums t_j = P_j + P_(j+16) one at a time.
template <int kM, int kSub>
struct PqScorer {
    static constexpr bool kHasExact = true;
    static constexpr bool kDirect = kSub != 0;
    const uint8_t* codes;
    const float* centroids;
    const void* queries;
    int query_f32;
    uint32_t dim;
    uint32_t pq_dim;
    uint32_t sub;            // dim / pq_dim
    uint32_t stride;         // bytes between code rows
    float* table;            // LDS: ADC table [M][256], or the fp32 query [dim]
    const void* exact_base;  // resident vectors for the inline exact distance
    uint32_t query;
    ExactWords qw;           // the query's exact-distance words (lanes < 32)

    static uint32_t lds_bytes(uint32_t dim_, uint32_t pq_dim_)
    {
        return kDirect ? dim_ * 4u : pq_dim_ * 256u * 4u;
    }

    __device__ int m() const { return kM > 0 ? kM : static_cast<int>(pq_dim); }
    __device__ uint32_t width() const { return kSub > 0 ? static_cast<uint32_t>(kSub) : sub; }

    __device__ void setup(uint32_t q, int lane, unsigned char* lds)
    {
        table = reinterpret_cast<float*>(lds);
        query = q;
        const float* qf = static_cast<const float*>(queries) + static_cast<size_t>(q) * dim;
        const uint8_t* qu = static_cast<const uint8_t*>(queries) + static_cast<size_t>(q) * dim;
        if constexpr (kDirect) {
            for (uint32_t d = lane; d < dim; d += kWave)
                table[d] = query_f32 ? qf[d] : static_cast<float>(qu[d]);
        } else {
            const int M = m();
            const int s = static_cast<int>(sub);
            for (int k = lane; k < 256; k += kWave) {
                const float* crow = centroids + static_cast<size_t>(k) * dim;
                for (int mm = 0; mm < M; ++mm) {
                    float acc = 0.0f;
                    for (int t = 0; t < s; ++t) {
                        const int d = mm * s + t;
                        const float qv = query_f32 ? qf[d] : static_cast<float>(qu[d]);
                        const float diff = qv - crow[d];
                        acc = fmaf(diff, diff, acc);
                    }
                    table[mm * 256 + k] = acc;
                }
            }
        }
        qw.w0 = qw.w1 = 0;
        if (exact_base != nullptr && lane < 32 && !query_f32) {
            const uint32_t words = dim / 4;
            const uint32_t* w = reinterpret_cast<const uint32_t*>(qu);
            if (static_cast<uint32_t>(lane) < words) qw.w0 = w[lane];
            if (static_cast<uint32_t>(lane) + 32 < words) qw.w1 = w[lane + 32];
        }
    }

    // LUT[mm][c].
    __device__ __forceinline__ float entry(int mm, uint32_t c) const
    {
        if constexpr (!kDirect) {
            return table[mm * 256 + c];
        } else {
            const uint32_t w = width();
            const float* crow = centroids + static_cast<size_t>(c) * dim + static_cast<uint32_t>(mm) * w;
            const float* qv = table + static_cast<uint32_t>(mm) * w;
            float acc = 0.0f;
            if (w == 4) {
                const float4 cv = *reinterpret_cast<const float4*>(crow);
                const float4 q4 = *reinterpret_cast<const float4*>(qv);
                float d = q4.x - cv.x;
                acc = fmaf(d, d, acc);
                d = q4.y - cv.y;
                acc = fmaf(d, d, acc);
                d = q4.z - cv.z;
                acc = fmaf(d, d, acc);
                d = q4.w - cv.w;
                acc = fmaf(d, d, acc);
            } else {
                for (uint32_t t = 0; t < w; ++t) {
                    const float d = qv[t] - crow[t];
                    acc = fmaf(d, d, acc);
                }
            }
            return acc;
        }
    }

    __device__ float score(uint32_t sample, bool active) const
    {
        if (!active) return 0.0f;
        const uint8_t* row = codes + static_cast<size_t>(sample) * stride;
        if constexpr (kM > 0 && kM % 16 == 0) {
            uint4 w[kM / 16];
#pragma unroll
            for (int i = 0; i < kM / 16; ++i) w[i] = reinterpret_cast<const uint4*>(row)[i];
            const uint32_t* words = reinterpret_cast<const uint32_t*>(w);
            float t[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                float lo = 0.0f;  // partial j:      subspaces j, j+32, ...
                float hi = 0.0f;  // partial j + 16: subspaces j+16, j+48, ...
#pragma unroll
                for (int mm = j; mm < kM; mm += 32)
                    lo += entry(mm, (words[mm >> 2] >> (8 * (mm & 3))) & 0xffu);
#pragma unroll
                for (int mm = j + 16; mm < kM; mm += 32)
                    hi += entry(mm, (words[mm >> 2] >> (8 * (mm & 3))) & 0xffu);
                t[j] = lo + hi;
                // Bound the table reads in flight (registers) to four
                // first-level sums at a time.
                if ((j & 3) == 3) __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int off = 8; off > 0; off >>= 1) {
#pragma unroll
                for (int j = 0; j < off; ++j) t[j] = t[j] + t[j + off];
            }
            return t[0];
        } else {
            float s[32];
#pragma unroll
            for (int j = 0; j < 32; ++j) s[j] = 0.0f;
            const int M = m();
            for (int mm = 0; mm < M; ++mm) {
                const float v = entry(mm, row[mm]);
                // Runtime index into the partials: the select chain keeps
                // them in registers.
#pragma unroll
                for (int j = 0; j < 32; ++j)
                    if ((mm & 31) == j) s[j] += v;
            }
#pragma unroll
            for (int off = 16; off > 0; off >>= 1) {
#pragma unroll
                for (int j = 0; j < off; ++j) s[j] = s[j] + s[j + off];
            }
            return s[0];
        }
    }

    // Start the loads of `sample`'s exact-distance words (u8, lanes < 32).
    __device__ void exact_load(uint32_t sample, int lane, ExactWords& ex) const
    {
        ex.w0 = ex.w1 = 0;
        if (lane >= 32 || query_f32) return;
        const uint32_t words = dim / 4;
        const uint32_t* b = reinterpret_cast<const uint32_t*>(
            static_cast<const uint8_t*>(exact_base) + static_cast<size_t>(sample) * dim);
        if (static_cast<uint32_t>(lane) < words) ex.w0 = b[lane];
        if (static_cast<uint32_t>(lane) + 32 < words) ex.w1 = b[lane + 32];
    }

    __device__ static __forceinline__ float acc_f32(float acc, float4 bv, float4 qv)
    {
        float d = bv.x - qv.x;
        acc = fmaf(d, d, acc);
        d = bv.y - qv.y;
        acc = fmaf(d, d, acc);
        d = bv.z - qv.z;
        acc = fmaf(d, d, acc);
        d = bv.w - qv.w;
        acc = fmaf(d, d, acc);
        return acc;
    }

    __device__ static __forceinline__ float acc_u8(float acc, uint32_t bw, uint32_t qw_)
    {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int diff = static_cast<int>((bw >> (8 * t)) & 0xffu) -
                             static_cast<int>((qw_ >> (8 * t)) & 0xffu);
            acc += static_cast<float>(diff * diff);
        }
        return acc;
    }

    // Exact distance of the expanded node in the reference's 32-lane order
    // (backend_pq.cu:4507-4540): lane j < 32 sums the 4-element words j,
    // j+32, ... (elements in order), then the xor butterfly 16..1.  u8 adds
    // integer squares as float; f32 uses fma.  Wave-uniform result.
    __device__ float exact_from(uint32_t sample, int lane, const ExactWords& ex) const
    {
        float acc = 0.0f;
        const uint32_t words = dim / 4;
        if (lane < 32) {
            const uint32_t l = static_cast<uint32_t>(lane);
            if (query_f32) {
                const float4* b = reinterpret_cast<const float4*>(
                    static_cast<const float*>(exact_base) + static_cast<size_t>(sample) * dim);
                const float4* q = reinterpret_cast<const float4*>(
                    static_cast<const float*>(queries) + static_cast<size_t>(query) * dim);
                for (uint32_t w = l; w < words; w += 32) acc = acc_f32(acc, b[w], q[w]);
            } else {
                if (l < words) acc = acc_u8(acc, ex.w0, qw.w0);
                if (l + 32 < words) acc = acc_u8(acc, ex.w1, qw.w1);
                const uint32_t* b = reinterpret_cast<const uint32_t*>(
                    static_cast<const uint8_t*>(exact_base) + static_cast<size_t>(sample) * dim);
                const uint32_t* q = reinterpret_cast<const uint32_t*>(
                    static_cast<const uint8_t*>(queries) + static_cast<size_t>(query) * dim);
                for (uint32_t w = l + 64; w < words; w += 32) acc = acc_u8(acc, b[w], q[w]);
            }
        }
#pragma unroll
        for (int off = 16; off > 0; off >>= 1) acc = acc + __shfl_xor(acc, off, 32);
        return bcast0f(acc);
    }
};

// RaBitQ one-bit estimate (score_rabitq_code_device, backend_rabitq.cu:
// 3100-3200, int8 query path).  ip_int = sum_d q8[d] * bit[d] is computed as
// sum_j w_j * popcount(plane_j & code) over the query's two's-complement bit
// planes (w_j = 2^j, w_7 = -128), which equals the reference's dp4a dot over
// nibble masks exactly.  Planes are stored MSB-first like the codes (word w,
// bit 31-b <-> dimension 32w+b) and plane-major in LDS: planes[j][word].
// Estimate: fma(f_rescale, ip*scale + k1, f_add + g[anchor]).
//
// Rows of 2048 or 4096 bits are scored by the whole wave: the candidates are
// packed into LDS and each 16-lane group scores one row per pass (lane l
// owns the row's 16-byte vectors l and l + 16), so every lane works and the
// code loads are coalesced; the group's integer partials are summed by DPP.
// Shorter or longer rows are scored one candidate per lane; in a traversal
// of a graph of degree <= 32 (lanes 32..63 never hold a candidate) lane l
// and lane l + 32 split lane l's row instead (`halves`), the low lane
// counting the first ceil(vectors / 2) 16-byte vectors, and the two
// integer partials add up to the same ip.
constexpr uint32_t kRabitqCoopBytes = 512;  // LDS after the planes: [64] ids, [64] ip

// x of lane l ^ 32 (v_permlane32_swap of x with itself: the first result
// holds the low half in both halves, the second the high half).
__device__ __forceinline__ uint32_t swap_wave_halves(uint32_t x, int lane)
{
    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return lane < 32 ? r[1] : r[0];
}

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
    uint32_t* planes;  // LDS [8][padded_dim/32], then kRabitqCoopBytes
    float scale;
    float k1;
    const float* g_row;
    const uint8_t* records;  // per-sample records (code, f_add, f_rescale, anchor) or null
    uint32_t record_stride;
    int halves;  // lanes 32..63 never score: they take half of lane l - 32's row

    __device__ __forceinline__ const uint8_t* code_row(uint32_t sample) const
    {
        return records ? records + static_cast<size_t>(sample) * record_stride
                       : codes + static_cast<size_t>(sample) * (padded_dim / 8);
    }

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
            for (int j = 0; j < 8; ++j) planes[j * words + w] = pl[j];
        }
        scale = q_scale[q];
        k1 = q_k1[q];
        g_row = centroid_dists + static_cast<size_t>(q) * num_anchors;
    }

    // sum_j w_j popc(plane_j & code) over one 16-byte code vector.
    __device__ __forceinline__ static void count_vec(const uint4* planes4, uint32_t vecs,
                                                     uint32_t v, const uint4& c, uint32_t (&cnt)[8])
    {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint4 p = planes4[j * vecs + v];
            cnt[j] = bcnt_acc(p.x & c.x, cnt[j]);
            cnt[j] = bcnt_acc(p.y & c.y, cnt[j]);
            cnt[j] = bcnt_acc(p.z & c.z, cnt[j]);
            cnt[j] = bcnt_acc(p.w & c.w, cnt[j]);
        }
    }

    __device__ __forceinline__ static int32_t combine(const uint32_t (&cnt)[8])
    {
        int32_t ip = 0;
#pragma unroll
        for (int j = 0; j < 7; ++j) ip += static_cast<int32_t>(cnt[j]) << j;
        return ip - 128 * static_cast<int32_t>(cnt[7]);
    }

    // Whole-wave ip of every active lane's candidate, rows of 16 * VPL
    // vectors.  All 64 lanes call it.
    template <int VPL>
    __device__ int32_t ip_coop(uint32_t sample, bool active, int lane) const
    {
        uint32_t* s_cand = planes + padded_dim / 4;        // after the 8 planes
        int32_t* s_ip = reinterpret_cast<int32_t*>(s_cand + kWave);
        constexpr uint32_t vecs = 16 * VPL;
        const uint4* planes4 = reinterpret_cast<const uint4*>(planes);
        const uint64_t m = ballot(active);
        const int n = __popcll(m);
        const int rank = __popcll(m & ((1ull << lane) - 1ull));
        if (active) s_cand[rank] = sample;
        __syncthreads();
        const int lg = lane & 15, grp = lane >> 4;
        for (int b0 = 0; b0 < n; b0 += 16) {
            // four rows per group in flight, then their counts
            uint4 cb[4][VPL];
#pragma unroll
            for (int it = 0; it < 4; ++it) {
                const int r = b0 + it * 4 + grp;
                const uint32_t sj = r < n ? s_cand[r] : 0u;
                const uint4* row = reinterpret_cast<const uint4*>(code_row(sj));
#pragma unroll
                for (int w = 0; w < VPL; ++w)
                    cb[it][w] = r < n ? row[lg + 16 * w] : make_uint4(0, 0, 0, 0);
            }
#pragma unroll
            for (int it = 0; it < 4; ++it) {
                const int r = b0 + it * 4 + grp;
                uint32_t cnt[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
                for (int w = 0; w < VPL; ++w) count_vec(planes4, vecs, lg + 16 * w, cb[it][w], cnt);
                const int32_t part = group_sum<16>(combine(cnt));
                if (lg == 0 && r < n) s_ip[r] = part;
            }
        }
        __syncthreads();
        return active ? s_ip[rank] : 0;
    }

    // Every lane of the wave calls score (the whole-wave path needs them all).
    __device__ float score(uint32_t sample, bool active) const
    {
        const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
        const uint32_t vecs = padded_dim / 128;
        uint32_t anchor = 0;
        float f_add = 0.0f, f_rescale = 0.0f;
        if (active && records) {
            const uint8_t* rec = records + static_cast<size_t>(sample) * record_stride + padded_dim / 8;
            const uint32_t* w = reinterpret_cast<const uint32_t*>(rec);
            f_add = __uint_as_float(w[0]);
            f_rescale = __uint_as_float(w[1]);
            anchor = w[2];
        } else if (active) {
            anchor = anchor_ids[sample];
            f_add = factors[static_cast<size_t>(sample) * 3];
            f_rescale = factors[static_cast<size_t>(sample) * 3 + 1];
        }
        int32_t ip;
        if (vecs == 32) {
            ip = ip_coop<2>(sample, active, lane);
        } else if (vecs == 16) {
            ip = ip_coop<1>(sample, active, lane);
        } else if (halves) {
            const bool hi = lane >= 32;
            const uint32_t s = swap_wave_halves(sample, lane);
            const uint64_t am = ballot(active);  // every lane votes (not inside the select)
            const bool act = ((am >> (lane & 31)) & 1ull) != 0;
            const uint32_t lo = (vecs + 1) / 2;
            int32_t part = 0;
            if (act) {
                const uint32_t v_end = hi ? vecs : lo;
                const uint4* row = reinterpret_cast<const uint4*>(code_row(hi ? s : sample));
                const uint4* planes4 = reinterpret_cast<const uint4*>(planes);
                uint32_t cnt[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                for (uint32_t v0 = hi ? lo : 0; v0 < v_end; v0 += kCodeBatch) {
                    uint4 cb[kCodeBatch];
#pragma unroll
                    for (int b = 0; b < kCodeBatch; ++b)
                        cb[b] = v0 + b < v_end ? row[v0 + b] : make_uint4(0, 0, 0, 0);
#pragma unroll
                    for (int b = 0; b < kCodeBatch; ++b) {
                        if (v0 + b >= v_end) break;
                        count_vec(planes4, vecs, v0 + b, cb[b], cnt);
                    }
                }
                part = combine(cnt);
            }
            ip = part + static_cast<int32_t>(swap_wave_halves(static_cast<uint32_t>(part), lane));
        } else {
            if (!active) return 0.0f;
            const uint4* row = reinterpret_cast<const uint4*>(code_row(sample));
            const uint4* planes4 = reinterpret_cast<const uint4*>(planes);
            uint32_t cnt[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            // Code loads go out kCodeBatch at a time before any is consumed, so
            // a row costs ceil(vectors / kCodeBatch) memory round trips, not one
            // per 16 bytes.
            for (uint32_t v0 = 0; v0 < vecs; v0 += kCodeBatch) {
                uint4 cb[kCodeBatch];
#pragma unroll
                for (int b = 0; b < kCodeBatch; ++b)
                    cb[b] = v0 + b < vecs ? row[v0 + b] : make_uint4(0, 0, 0, 0);
#pragma unroll
                for (int b = 0; b < kCodeBatch; ++b) {
                    if (v0 + b >= vecs) break;
                    count_vec(planes4, vecs, v0 + b, cb[b], cnt);
                }
            }
            ip = combine(cnt);
        }
        if (!active) return 0.0f;
        const float short_ip = static_cast<float>(ip) * scale;
        const float t = short_ip + k1;
        return fmaf(f_rescale, t, f_add + g_row[anchor]);
    }

    __device__ int32_t ip_int(uint32_t sample) const
    {
        const uint32_t words = padded_dim / 32;
        const uint32_t* row = reinterpret_cast<const uint32_t*>(code_row(sample));
        int32_t ip = 0;
        for (uint32_t w = 0; w < words; ++w) {
            const uint32_t cw = row[w];
            for (int j = 0; j < 8; ++j) {
                const int32_t c = __popc(planes[j * words + w] & cw);
                ip += (j == 7) ? -128 * c : (c << j);
            }
        }
        return ip;
    }

    __device__ void exact_load(uint32_t, int, ExactWords&) const {}
    __device__ float exact_from(uint32_t, int, const ExactWords&) const { return 0.0f; }
};

struct TraversalArgs {
    gofann_graph_view graph;
    gofann_predicate_view pred;
    gofann_routes routes;
    gofann_search_params params;
    uint32_t* out_ids;
    float* out_dists;
    gofann_route_stats* stats;
    uint32_t* hash_global;  // [launch slots][4096] when the hash is not in LDS
    uint32_t off_frontier;
    uint32_t off_topk;
    uint32_t off_stop;
    uint32_t off_hash;
    int rabitq_verdict;
};

// Loads a picked node needs when it is expanded, issued one step early.
struct NodeLoads {
    uint32_t adj;        // lane j: adjacency entry j (UINT32_MAX past the degree)
    uint32_t nsamp;      // lane j: its sample id (graph.neighbor_samples)
    uint4 row;           // the node's label slab, or its CSR bounds in .x/.y
    ExactWords ex;       // exact-distance words (inline exact)
};

template <class Scorer>
__device__ __forceinline__ void load_node(const TraversalArgs& a, const Scorer& sc,
                                          uint32_t label_offset, uint32_t degree, const Entry& e,
                                          bool verdict_rows, bool exact, int lane, NodeLoads& n)
{
    const uint32_t local = e.second & ~kPoolUsed;
    const size_t row = static_cast<size_t>(label_offset + local) * a.graph.degree;
    const bool in_row = static_cast<uint32_t>(lane) < degree;
    n.adj = in_row ? a.graph.graph[row + lane] : UINT32_MAX;
    n.nsamp = (in_row && a.graph.neighbor_samples) ? a.graph.neighbor_samples[row + lane] : 0u;
    n.row = make_uint4(0, 0, 0, 0);
    if (verdict_rows && e.sample < a.pred.rows && a.pred.csr_offsets != nullptr) {
        if (slab_usable(a.pred, e.sample)) {
            n.row = slab_load(a.pred, e.sample);
        } else {
            n.row.x = a.pred.csr_offsets[e.sample];
            n.row.y = a.pred.csr_offsets[e.sample + 1];
        }
    }
    if constexpr (Scorer::kHasExact) {
        if (exact) sc.exact_load(e.sample, lane, n.ex);
    }
}

template <class Scorer, int kVisited>
__global__ __launch_bounds__(64, GOFANN_TRAVERSAL_MIN_WAVES) void traversal_kernel(TraversalArgs a, Scorer sc)
{
    extern __shared__ __align__(16) unsigned char lds[];
    __shared__ uint32_t s_row[kMaxDegree];
    __shared__ uint32_t s_samp[kMaxDegree];
    __shared__ float s_first[kMaxDegree];
    __shared__ float s_base[kMaxDegree];
    __shared__ uint64_t s_adm;

    const int lane = static_cast<int>(threadIdx.x);
    const uint32_t slot = xcd_slot(blockIdx.x, gridDim.x);
    if (slot >= a.routes.count) return;
    const uint32_t route = a.routes.launch_order ? a.routes.launch_order[slot] : slot;

    Entry* frontier = reinterpret_cast<Entry*>(lds + a.off_frontier);
    ResultEntry* topk = reinterpret_cast<ResultEntry*>(lds + a.off_topk);
    StopEntry* stop = reinterpret_cast<StopEntry*>(lds + a.off_stop);
    VisitedSet<kVisited> visited;

    const int Q = a.params.queue_limit;
    const int W = a.params.result_width;
    const int SW = a.params.stop_width;
    const int mode = a.params.early_stop_mode;
    const bool bias = a.params.predicate_bias != 0;
    const bool bonuses = a.params.bit_filter_bonus != 1.0f || a.params.range_filter_bonus != 1.0f;
    const bool exact = Scorer::kHasExact && a.params.inline_exact_rerank != 0;

    const uint32_t group = a.routes.route_group[route];
    const uint32_t label_offset = a.graph.label_offset[group];
    const uint32_t query = a.routes.route_query[route];
    const uint32_t begin_id = a.routes.route_start[route];
    const uint64_t qfbit = a.routes.query_filter_bits ? a.routes.query_filter_bits[route] : ~0ULL;
    const uint32_t active_ranges =
        count_active_ranges(a.routes.range_modes, route, a.routes.range_count);
    const bool enabled = pred_enabled(a.pred, route);
    const bool compiled = a.pred.route_compiled != nullptr && a.pred.route_compiled[route] != 0;
    const bool fallback = a.rabitq_verdict ? !compiled : (!enabled && !compiled);
    const uint32_t degree = a.graph.degree < static_cast<uint32_t>(kMaxDegree)
                                ? a.graph.degree
                                : static_cast<uint32_t>(kMaxDegree);

    // The global slab holds one table per launch slot (slot < routes.count).
    visited.init(reinterpret_cast<uint32_t*>(lds + a.off_hash),
                 a.hash_global ? a.hash_global + static_cast<size_t>(slot) * kHashCapacity : nullptr,
                 lane);
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
    const Entry sentinel = {FLT_MAX, UINT32_MAX, FLT_MAX, UINT32_MAX};
    if (lane == 0) {
        const Entry kp = {start, begin_id, start, begin_sample};
        smmh_insert(frontier, heap_size, kp);
        (void)visited.add_serial(begin_id, 0);
    }
    heap_size = bcast0(heap_size);
    visited.count = 1;
    __threadfence_block();
    __syncthreads();

    Entry now = sentinel;
    Entry next = sentinel;
    NodeLoads cur, nxt;
    if (!pickup(frontier, heap_size, now, lane)) {
        exhausted = 1;
        now = sentinel;
    } else {
        load_node(a, sc, label_offset, degree, now, enabled, exact, lane, cur);
    }

    int step = 0;
    const int wave_lane = lane;
    while (step == 0 || heap_size > 1) {
        // per step: lane-derived values are not held across steps (PqScorer<48>
        // 111 VGPRs, RaBitQ 118-120, no spills; with the lane hoisted out of
        // the loop both reach the 128-VGPR budget and spill)
        const int lane = opaque_lane(wave_lane);
        const uint32_t now_local = now.second & ~kPoolUsed;
        ++step;

        if (step != 1) {
            bool found;
            // the pending-base stop needs minimum_pending_base
            // (gpu_predicate_index.cuh:147-160): the least base over the
            // current/next entries and every unused frontier entry; the LDS
            // pickup finds it in the same pass
            const bool want_base = stop_size == SW && a.pred.pending_base_stop && enabled;
            float unused_base = FLT_MAX;
            found = pickup(frontier, heap_size, next, lane, want_base, unused_base);
            if (!found) {
                exhausted = 1;
                next = sentinel;
            } else {
                load_node(a, sc, label_offset, degree, next, enabled, exact, lane, nxt);
                if (stop_size == SW) {
                    float pending = next.first;
                    if (want_base) pending = fminf(unused_base, now.base);
                    if (mode != GOFANN_EARLY_STOP_OFF && stop_worst <= pending) ++finished;
                }
            }
        }

        // First memory round of the step: the expanded node's label row and,
        // for every unvisited neighbour (adjacency order, lane i takes
        // neighbour i of the prefetched row, backend_pq.cu:4636-4684), its
        // CSR bounds.  Loads without side effects; the serial order of the
        // decisions below is the reference's.
        WaveRow vrow{0, 0, UINT32_MAX, false};
        if (!exhausted && enabled) {
            const uint32_t s0 = now.sample;
            if (!slab_usable(a.pred, s0)) {
                vrow = wave_row_load(a.pred, s0, cur.row.x, cur.row.y, lane);
            } else if (slab_count(cur.row) != kSlabOverflow) {
                vrow = wave_row_from_slab(cur.row, lane);
            } else {
                vrow = wave_row_load(a.pred, s0, a.pred.csr_offsets[s0], a.pred.csr_offsets[s0 + 1],
                                     lane);
            }
        }
        const uint32_t idx = cur.adj;
        const bool keep = idx != UINT32_MAX && !visited.test(idx);
        const uint64_t keep_mask = ballot(keep);
        const int list_len = __popcll(keep_mask);
        uint32_t my_sample = 0;
        if (keep)
            my_sample = a.graph.neighbor_samples ? cur.nsamp
                                                 : a.graph.row_to_sample[label_offset + idx];
        const bool need_pass = keep && bias && enabled;
        LaneRow lrow;
        uint4 lslab;
        lane_row_bounds(a.pred, my_sample, need_pass, lrow, lslab);

        // Verdict of the expanded node (backend_pq.cu:4393-4441).  Skipped
        // when the pool ran dry: the loop leaves below before reading it.
        int filt = 1;
        float rank = now.base;
        if (!exhausted) {
            const uint32_t sample = now.sample;
            PredCounters c{0, 0};
            if (enabled) filt = wave_pred_matches(a.pred, route, sample, vrow, lane, c) ? 1 : 2;
            if (fallback) {
                const uint32_t global_row = label_offset + now_local;
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
                if (filt == 1 && exact) rank = sc.exact_from(sample, lane, cur.ex);
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

        if (early_stop_reached(mode, finished, a.params.finish_limit, Q, expanded, passed, SW) ||
            (a.params.max_steps > 0 && step >= a.params.max_steps))
            break;

        // Second round: candidate label rows, then code rows and table
        // entries; predicate pass bits and priorities
        // (backend_pq.cu:4704-4747, 4826-4864).
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

        // Threshold pre-filter: with a full frontier (size >= Q+1) the serial
        // loop skips any candidate above frontier[2]; that maximum can only
        // fall during the step, so such candidates are dropped here.
        const bool full = heap_size >= Q + 1;
        const float thr = full ? frontier[2].first : 0.0f;
        const bool cand = keep && !(full && thr < first);
        const uint64_t cand_mask = ballot(cand);
        // Ordered admission (backend_pq.cu:4889-4907); the visited-set adds
        // of the admitted candidates follow lane-parallel.  `mine`: this
        // lane's candidate was admitted.
        bool mine;
        uint64_t adm_lanes;  // admitted lanes, in adjacency order
        if (Q + 2 <= kWaveHeapSlots) {
            // the whole wave runs each insert / pop_max on the LDS frontier;
            // hmax: the largest `first` in it (frontier[2] once full)
            adm_lanes = 0;
            float hmax = heap_size >= 3   ? frontier[2].first
                         : heap_size == 2 ? frontier[1].first
                                          : -__builtin_inff();
            for (uint64_t m = cand_mask; m; m &= m - 1) {
                const int j = __builtin_ctzll(m);
                Entry kp;
                kp.first = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(first), j));
                kp.second = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(idx), j));
                kp.base = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(base), j));
                kp.sample = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(my_sample), j));
                if (heap_size >= Q + 1 && hmax < kp.first) continue;
                wave_smmh_insert(frontier, heap_size, kp, lane);
                hmax = fmaxf(hmax, kp.first);
                adm_lanes |= 1ull << j;
                ++admitted;
                if (heap_size >= Q + 2) hmax = wave_smmh_pop_max(frontier, heap_size, lane);
            }
            mine = (adm_lanes >> lane) & 1ull;
        } else {
            const int n_cand = __popcll(cand_mask);
            const uint32_t pos = lanes_below(cand_mask);
            if (cand) {
                s_row[pos] = idx;
                s_samp[pos] = my_sample;
                s_first[pos] = first;
                s_base[pos] = base;
            }
            __syncthreads();
            if (lane == 0) {
                uint64_t adm = 0;
                for (int i = 0; i < n_cand; ++i) {
                    const Entry kp = {s_first[i], s_row[i], s_base[i], s_samp[i]};
                    if (heap_size >= Q + 1 && frontier[2].first < kp.first) continue;
                    smmh_insert(frontier, heap_size, kp);
                    adm |= 1ull << i;
                    ++admitted;
                    if (heap_size >= Q + 2) smmh_pop_max(frontier, heap_size);
                }
                s_adm = adm;
            }
            heap_size = bcast0(heap_size);
            __syncthreads();
            const uint64_t adm = s_adm;  // by compacted position
            mine = cand && ((adm >> pos) & 1ull);
            adm_lanes = ballot(mine);
        }
        const uint32_t n_adm = static_cast<uint32_t>(__popcll(adm_lanes));
        visited.reserve(n_adm, lane);
        if (visited.count + n_adm <= kHashCapacity) {
            const int ins = mine ? visited.add_parallel(idx) : 0;
            visited.count += static_cast<uint32_t>(__popcll(ballot(ins != 0)));
        } else {
            // The set may fill: serial adds in admission (adjacency) order
            // reproduce which values the reference drops.
            uint32_t added = 0;
            for (uint64_t m = adm_lanes; m; m &= m - 1) {
                const int j = __builtin_ctzll(m);
                const uint32_t v = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(idx), j));
                if (lane == 0) added += static_cast<uint32_t>(visited.add_serial(v, added));
            }
            visited.count += bcast0u(added);
        }
        __threadfence_block();
        __syncthreads();

        if (step == 1) {
            if (!pickup(frontier, heap_size, next, lane)) {
                exhausted = 1;
                next = sentinel;
            } else {
                load_node(a, sc, label_offset, degree, next, enabled, exact, lane, nxt);
            }
        }
        now = next;
        cur = nxt;
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

// ---------------------------------------------------------------------------
// Host launch templates.
// ---------------------------------------------------------------------------
inline uint32_t align16(uint32_t x) { return (x + 15u) & ~15u; }

struct Layout {
    uint32_t off_frontier, off_topk, off_stop, off_hash, base_bytes;
    uint32_t bytes(int visited) const
    {
        if (visited == kVisitedLds) return off_hash + kHashCapacity * 4u;
        if (visited == kVisitedSpill) return off_hash + kSpillSlots * 4u;
        return base_bytes;
    }
};

inline Layout make_layout(uint32_t scorer_bytes, int Q, int W)
{
    Layout l;
    l.off_frontier = align16(scorer_bytes);
    l.off_topk = align16(l.off_frontier + static_cast<uint32_t>(Q + 2) * sizeof(Entry));
    l.off_stop = align16(l.off_topk + static_cast<uint32_t>(W + 1) * sizeof(ResultEntry));
    l.off_hash = align16(l.off_stop + static_cast<uint32_t>(kMaxStopWidth + 1) * sizeof(StopEntry));
    l.base_bytes = l.off_hash;
    return l;
}

inline int check_params(Context* ctx, const gofann_graph_view* g, const gofann_routes* r,
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
    if (p->table_mode < GOFANN_PLACE_AUTO || p->table_mode > GOFANN_PLACE_GLOBAL ||
        p->hash_mode < GOFANN_PLACE_AUTO || p->hash_mode > GOFANN_PLACE_SPILL)
        return ctx->fail(GOFANN_ERR_INVALID, "table_mode in [0, 2], hash_mode in [0, 3]");
    if (!g->graph || !g->row_to_sample || !g->label_offset || g->degree == 0)
        return ctx->fail(GOFANN_ERR_INVALID, "graph view incomplete");
    // validate_pq_search_options rejects degree > FIXED_DEGREE
    // (backend_pq.cu:11486-11488); reading only a row prefix would change
    // results silently.
    if (g->degree > static_cast<uint32_t>(kMaxDegree))
        return ctx->fail(GOFANN_ERR_UNSUPPORTED, "graph degree must be in [1, 64]");
    if (r->count > 0 && (!r->route_query || !r->route_group || !r->route_start))
        return ctx->fail(GOFANN_ERR_INVALID, "route arrays missing");
    return GOFANN_OK;
}

// Resident workgroups per CU of a one-wave traversal launch with `lds`
// bytes of dynamic LDS (registers, LDS and wave slots all counted).
template <class Kernel>
int resident_per_cu(Context* ctx, Kernel kern, uint32_t lds)
{
    if (lds > static_cast<uint32_t>(ctx->lds_per_block)) return 0;
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                            hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(lds)) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    int blocks = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, reinterpret_cast<const void*>(kern),
                                                     kWave, lds) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return blocks;
}

struct Placement {
    int visited;  // kVisitedGlobal / kVisitedLds / kVisitedSpill
    uint32_t lds;
    int resident;
};

// Visited-set placement for one scorer configuration.  hash_mode picks it; auto takes the most resident routes per
// CU, preferring LDS storage on ties (full table, then the spilling table,
// then the global slab).
template <class Scorer>
Placement choose_visited(Context* ctx, const Layout& l, int hash_mode)
{
    const Placement full{kVisitedLds, l.bytes(kVisitedLds),
                         resident_per_cu(ctx, traversal_kernel<Scorer, kVisitedLds>,
                                         l.bytes(kVisitedLds))};
    const Placement spill{kVisitedSpill, l.bytes(kVisitedSpill),
                          resident_per_cu(ctx, traversal_kernel<Scorer, kVisitedSpill>,
                                          l.bytes(kVisitedSpill))};
    const Placement glob{kVisitedGlobal, l.bytes(kVisitedGlobal),
                         resident_per_cu(ctx, traversal_kernel<Scorer, kVisitedGlobal>,
                                         l.bytes(kVisitedGlobal))};
    if (hash_mode == GOFANN_PLACE_LDS) return full;
    if (hash_mode == GOFANN_PLACE_GLOBAL) return glob;
    if (hash_mode == GOFANN_PLACE_SPILL) return spill;
    Placement best = full;
    if (spill.resident > best.resident) best = spill;
    if (glob.resident > best.resident) best = glob;
    return best;
}

template <class Scorer>
int launch_traversal(Context* ctx, const Scorer& sc, const Layout& l, const Placement& pl,
                     const gofann_graph_view* g, const gofann_predicate_view* pred,
                     const gofann_routes* r, const gofann_search_params* p, uint32_t* out_ids,
                     float* out_dists, gofann_route_stats* stats, int rabitq_verdict)
{
    if (pl.resident <= 0)
        return ctx->fail(GOFANN_ERR_UNSUPPORTED, "per-route LDS state exceeds the workgroup limit");
    TraversalArgs a;
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
    a.rabitq_verdict = rabitq_verdict;
    a.hash_global = nullptr;
    if (pl.visited != kVisitedLds) {
        const size_t need = static_cast<size_t>(r->count) * kHashCapacity * sizeof(uint32_t);
        a.hash_global = static_cast<uint32_t*>(ctx->scratch(Context::kScratchHash, need));
        if (!a.hash_global) return ctx->fail(GOFANN_ERR_NOMEM, "visited set scratch");
    }
    const dim3 grid(r->count), block(kWave);
    if (pl.visited == kVisitedLds) {
        hipLaunchKernelGGL((traversal_kernel<Scorer, kVisitedLds>), grid, block, pl.lds,
                           ctx->stream, a, sc);
    } else if (pl.visited == kVisitedSpill) {
        hipLaunchKernelGGL((traversal_kernel<Scorer, kVisitedSpill>), grid, block, pl.lds,
                           ctx->stream, a, sc);
    } else {
        hipLaunchKernelGGL((traversal_kernel<Scorer, kVisitedGlobal>), grid, block, pl.lds,
                           ctx->stream, a, sc);
    }
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("traversal launch");
    ctx->last_hash_in_lds = pl.visited == kVisitedGlobal ? 0 : (pl.visited == kVisitedLds ? 1 : 2);
    ctx->last_lds_bytes = static_cast<int>(pl.lds);
    ctx->last_resident = pl.resident;
    return GOFANN_OK;
}

template <int kM, int kSub>
PqScorer<kM, kSub> make_pq_scorer(const gofann_pq_view* pq, const void* queries, int query_elem)
{
    PqScorer<kM, kSub> sc;
    sc.codes = pq->codes;
    sc.centroids = pq->centroids;
    sc.queries = queries;
    sc.query_f32 = query_elem == GOFANN_ELEM_F32 ? 1 : 0;
    sc.dim = pq->dim;
    sc.pq_dim = pq->pq_dim;
    sc.sub = pq->dim / pq->pq_dim;
    sc.stride = pq->code_stride ? pq->code_stride : pq->pq_dim;
    sc.table = nullptr;
    sc.exact_base = pq->exact_base;
    sc.query = 0;
    sc.qw.w0 = sc.qw.w1 = 0;
    return sc;
}

// PQ: choose the table placement (LDS table vs on-demand entries) and the
// visited-set placement by resident routes per CU, then launch.
template <int kM, int kMD, int kSub>
int pq_search_ms(Context* ctx, const gofann_pq_view* pq, const void* queries, int query_elem,
                 const gofann_graph_view* g, const gofann_predicate_view* pred,
                 const gofann_routes* r, const gofann_search_params* p, uint32_t* out_ids,
                 float* out_dists, gofann_route_stats* stats)
{
    using TableScorer = PqScorer<kM, 0>;
    using DirectScorer = PqScorer<kMD, kSub>;
    const Layout lt = make_layout(TableScorer::lds_bytes(pq->dim, pq->pq_dim), p->queue_limit,
                                  p->result_width);
    const Layout ld = make_layout(DirectScorer::lds_bytes(pq->dim, pq->pq_dim), p->queue_limit,
                                  p->result_width);
    Placement pt{kVisitedGlobal, 0, 0}, pd{kVisitedGlobal, 0, 0};
    if (p->table_mode != GOFANN_PLACE_GLOBAL) pt = choose_visited<TableScorer>(ctx, lt, p->hash_mode);
    if (p->table_mode != GOFANN_PLACE_LDS) pd = choose_visited<DirectScorer>(ctx, ld, p->hash_mode);
    const bool direct = p->table_mode == GOFANN_PLACE_GLOBAL ||
                        (p->table_mode == GOFANN_PLACE_AUTO && pd.resident > pt.resident);
    ctx->last_table_in_lds = direct ? 0 : 1;
    if (direct)
        return launch_traversal(ctx, make_pq_scorer<kMD, kSub>(pq, queries, query_elem), ld, pd, g,
                                pred, r, p, out_ids, out_dists, stats, 0);
    return launch_traversal(ctx, make_pq_scorer<kM, 0>(pq, queries, query_elem), lt, pt, g, pred,
                            r, p, out_ids, out_dists, stats, 0);
}

// One PQ width: four dims per subspace (C1 128/32, C2 192/48) get a
// compile-time width; other shapes use the runtime-width scorer.
template <int kM>
int pq_search_m(Context* ctx, const gofann_pq_view* pq, const void* queries, int query_elem,
                const gofann_graph_view* g, const gofann_predicate_view* pred,
                const gofann_routes* r, const gofann_search_params* p, uint32_t* out_ids,
                float* out_dists, gofann_route_stats* stats)
{
    if (pq->dim == 4u * pq->pq_dim)
        return pq_search_ms<kM, kM, 4>(ctx, pq, queries, query_elem, g, pred, r, p, out_ids,
                                       out_dists, stats);
    return pq_search_ms<kM, 0, -1>(ctx, pq, queries, query_elem, g, pred, r, p, out_ids,
                                   out_dists, stats);
}

#define GOFANN_PQ_SEARCH_M_ARGS                                                              \
    Context*, const gofann_pq_view*, const void*, int, const gofann_graph_view*,             \
        const gofann_predicate_view*, const gofann_routes*, const gofann_search_params*,     \
        uint32_t*, float*, gofann_route_stats*
extern template int pq_search_m<16>(GOFANN_PQ_SEARCH_M_ARGS);
extern template int pq_search_m<32>(GOFANN_PQ_SEARCH_M_ARGS);
extern template int pq_search_m<48>(GOFANN_PQ_SEARCH_M_ARGS);
extern template int pq_search_m<64>(GOFANN_PQ_SEARCH_M_ARGS);
extern template int pq_search_m<0>(GOFANN_PQ_SEARCH_M_ARGS);

}  // namespace gofann
