// build_kernels.hip -- index construction on gfx950: the per-label graphs,
// the coarse k-means that buckets them, and the PQ / RaBitQ encoders.  The
// reference builds these offline with cuVS: a CAGRA graph per label
// (build_cagra_graph_chunk, src/index/graph_builder.cu:1279-1315), PQ
// codebooks (tools/quantization/pq_builder.cu:49-153) and the IVF-RaBitQ
// encoder (third_party/cuvs_rabitq/src/neighbors/ivf_rabitq/gpu_index/
// quantizer_gpu_fast.cu:39-101, 180-265).
//
// Every result here has a fixed arithmetic order, so the CPU oracle
// (oracle/build_oracle.c) reproduces it bit for bit, and every kernel is
// deterministic: no floating-point atomics, and the sorts are stable radix
// sorts.  The orders:
//   * row-to-centre score  s(x, c) = |c|^2 - 2 <x, c>: <x, c> and |c|^2
//     accumulate in fp32, fmaf over d ascending; argmin over centres (the
//     row's own norm is the same for every centre);
//   * row-to-row distance  d(x, y) = sum_d (x_d - y_d)^2, fmaf over d
//     ascending (an exact integer for u8 rows of up to 258 dims);
//   * every ranking orders (value, index) pairs, so ties go to the lower
//     index.
//
// Distances are GEMM-shaped, but they run on the VALU: an MFMA's internal
// summation order is not specified, and the ids these kernels emit must be
// identical to the oracle's.  The tile kernel is a register-blocked
// product: 256 threads own a 64 x 64 tile, 4 x 4 per thread, with 32-dim
// chunks of both operands staged in LDS as fp32.
#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>

#include <cfloat>
#include <cstdint>
#include <vector>

#include "gofann_internal.hpp"

namespace gofann {

rocblas_handle blas_handle(Context* ctx);

namespace {

constexpr int kTile = 64;     // rows per tile side
constexpr int kTileD = 32;    // dims per staged chunk
constexpr int kThreads = 256;
constexpr int kWave = 64;
constexpr uint32_t kNone = 0xFFFFFFFFu;
constexpr int kMaxKnn = 128;  // list width of the kNN kernel

__device__ __forceinline__ float to_f(uint8_t v) { return static_cast<float>(v); }
__device__ __forceinline__ float to_f(float v) { return v; }
__device__ __forceinline__ float to_f(_Float16 v) { return static_cast<float>(v); }

__device__ __forceinline__ bool pair_lt(float ad, uint32_t ai, float bd, uint32_t bi)
{
    return ad < bd || (ad == bd && ai < bi);
}

// Rows [0, n) x dims [d0, d0 + kTileD) of `rows` (row r at rows + r * stride)
// into lds[dd * kTile + r] as fp32; zero outside the rows and dims.  Thread
// t takes row t % 64 and eight consecutive dims, so the LDS writes of a
// wave fall on consecutive banks.
template <class T>
__device__ __forceinline__ void stage_rows(const T* rows, size_t stride, int n, uint32_t d0,
                                           uint32_t dim, float* lds, int tid)
{
    const int r = tid & (kTile - 1);
    const int g = tid >> 6;  // 0..3
    const uint32_t db = d0 + static_cast<uint32_t>(g) * 8u;
    float v[8];
    if (r < n) {
        const T* p = rows + static_cast<size_t>(r) * stride;
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = db + i < dim ? to_f(p[db + i]) : 0.0f;
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = 0.0f;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) lds[(g * 8 + i) * kTile + r] = v[i];
}

// acc[i][j] += the chunk's terms for rows ty*4+i of sa and tx*4+j of sb
// (dims of the chunk ascending; zero-padded dims add exact zeros).
template <bool kDiff>
__device__ __forceinline__ void tile_chunk(const float* sa, const float* sb, int ty, int tx,
                                           float acc[4][4])
{
#pragma unroll 8
    for (int dd = 0; dd < kTileD; ++dd) {
        const float4 a = *reinterpret_cast<const float4*>(sa + dd * kTile + ty * 4);
        const float4 b = *reinterpret_cast<const float4*>(sb + dd * kTile + tx * 4);
        const float av[4] = {a.x, a.y, a.z, a.w};
        const float bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (kDiff) {
                    const float t = av[i] - bv[j];
                    acc[i][j] = fmaf(t, t, acc[i][j]);
                } else {
                    acc[i][j] = fmaf(av[i], bv[j], acc[i][j]);
                }
            }
    }
}

// |c|^2 per row of a float matrix, fmaf over d ascending.
__global__ void row_sqnorm_kernel(const float* m, uint32_t rows, uint32_t dim, float* out)
{
    const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    const float* p = m + static_cast<size_t>(r) * dim;
    float s = 0.0f;
    for (uint32_t d = 0; d < dim; ++d) s = fmaf(p[d], p[d], s);
    out[r] = s;
}

// Nearest centre of each row: argmin over k of (cnorm[k] - 2 <x, c_k>),
// ties to the lower k.  One workgroup per 64 rows; all centres in 64-row
// tiles.
template <class T>
__global__ __launch_bounds__(kThreads) void assign_kernel(const T* rows, size_t stride,
                                                          uint32_t dim, uint64_t n,
                                                          const float* centres,
                                                          const float* cnorm, uint32_t k,
                                                          uint32_t* out_idx, float* out_score)
{
    __shared__ __align__(16) float sa[kTileD * kTile];
    __shared__ __align__(16) float sb[kTileD * kTile];
    const int tid = static_cast<int>(threadIdx.x);
    const int ty = tid >> 4, tx = tid & 15;
    const uint64_t r0 = static_cast<uint64_t>(blockIdx.x) * kTile;
    if (r0 >= n) return;
    const int nq = static_cast<int>(n - r0 < kTile ? n - r0 : kTile);
    const T* qrows = rows + r0 * stride;
    float best[4];
    uint32_t bidx[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        best[i] = FLT_MAX;
        bidx[i] = kNone;
    }
    for (uint32_t c0 = 0; c0 < k; c0 += kTile) {
        const int nc = static_cast<int>(k - c0 < kTile ? k - c0 : kTile);
        float acc[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;
        for (uint32_t d0 = 0; d0 < dim; d0 += kTileD) {
            __syncthreads();
            stage_rows(qrows, stride, nq, d0, dim, sa, tid);
            stage_rows(centres + static_cast<size_t>(c0) * dim, static_cast<size_t>(dim), nc, d0,
                       dim, sb, tid);
            __syncthreads();
            tile_chunk<false>(sa, sb, ty, tx, acc);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int c = tx * 4 + j;
            if (c >= nc) break;
            const float cn = cnorm[c0 + c];
            const uint32_t ci = c0 + static_cast<uint32_t>(c);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float s = cn - 2.0f * acc[i][j];
                if (pair_lt(s, ci, best[i], bidx[i])) {
                    best[i] = s;
                    bidx[i] = ci;
                }
            }
        }
    }
    // the 16 lanes of a row group hold disjoint centres: reduce them
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int off = 8; off > 0; off >>= 1) {
            const float os = __shfl_xor(best[i], off, 16);
            const uint32_t oi = static_cast<uint32_t>(__shfl_xor(static_cast<int>(bidx[i]), off, 16));
            if (pair_lt(os, oi, best[i], bidx[i])) {
                best[i] = os;
                bidx[i] = oi;
            }
        }
    }
    if (tx == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int q = ty * 4 + i;
            if (q < nq) {
                out_idx[r0 + q] = bidx[i];
                if (out_score) out_score[r0 + q] = best[i];
            }
        }
    }
}

// kNN inside buckets: the rows are sorted by bucket (bucket b holds rows
// [bucket_off[b], bucket_off[b+1])); query tile t holds rows
// [tile_row0[t], +64) of bucket tile_bucket[t] and scans the rows of every
// bucket on its probe list (its own bucket when there is no list).  Each
// query row keeps its k least (distance, row) pairs, itself excluded, in
// LDS; the lists merge each candidate tile by rank.
template <class T>
__global__ __launch_bounds__(kThreads) void knn_kernel(const T* rows, uint32_t dim,
                                                       const uint32_t* bucket_off,
                                                       const uint32_t* probe_off,
                                                       const uint32_t* probe,
                                                       const uint32_t* tile_bucket,
                                                       const uint32_t* tile_row0, uint32_t tiles,
                                                       int k, uint32_t* out_ids, float* out_d)
{
    extern __shared__ __align__(16) unsigned char lds[];
    float* sa = reinterpret_cast<float*>(lds);
    float* sb = sa + kTileD * kTile;
    float* sd = sb + kTileD * kTile;                 // [64][65]
    float* ld_all = sd + kTile * (kTile + 1);        // [64][k]
    uint32_t* lid_all = reinterpret_cast<uint32_t*>(ld_all + kTile * k);
    const int tid = static_cast<int>(threadIdx.x);
    const int ty = tid >> 4, tx = tid & 15;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const uint32_t t = blockIdx.x;
    if (t >= tiles) return;
    const uint32_t b = tile_bucket[t];
    const uint32_t q0 = tile_row0[t];
    const uint32_t qe = bucket_off[b + 1];
    const int nq = static_cast<int>(qe - q0 < kTile ? qe - q0 : kTile);
    for (int e = tid; e < kTile * k; e += kThreads) {
        ld_all[e] = FLT_MAX;
        lid_all[e] = kNone;
    }
    const uint32_t p_begin = probe_off ? probe_off[b] : 0u;
    const uint32_t p_end = probe_off ? probe_off[b + 1] : 1u;
    const T* qrows = rows + static_cast<size_t>(q0) * dim;
    for (uint32_t p = p_begin; p < p_end; ++p) {
        const uint32_t pb = probe_off ? probe[p] : b;
        const uint32_t c_begin = bucket_off[pb], c_end = bucket_off[pb + 1];
        for (uint32_t c0 = c_begin; c0 < c_end; c0 += kTile) {
            const int nc = static_cast<int>(c_end - c0 < kTile ? c_end - c0 : kTile);
            float acc[4][4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;
            for (uint32_t d0 = 0; d0 < dim; d0 += kTileD) {
                __syncthreads();
                stage_rows(qrows, static_cast<size_t>(dim), nq, d0, dim, sa, tid);
                stage_rows(rows + static_cast<size_t>(c0) * dim, static_cast<size_t>(dim), nc, d0,
                           dim, sb, tid);
                __syncthreads();
                tile_chunk<true>(sa, sb, ty, tx, acc);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) sd[(ty * 4 + i) * (kTile + 1) + tx * 4 + j] = acc[i][j];
            __syncthreads();
            // wave w merges the tile into the lists of rows w*16 .. w*16+15
            for (int ii = 0; ii < kTile / 4; ++ii) {
                const int qi = wave * (kTile / 4) + ii;
                if (qi >= nq) break;
                const uint32_t self = q0 + static_cast<uint32_t>(qi);
                float* ld = ld_all + qi * k;
                uint32_t* lid = lid_all + qi * k;
                const uint32_t cid = c0 + static_cast<uint32_t>(lane);
                const float v = sd[qi * (kTile + 1) + lane];
                const bool valid = lane < nc && cid != self;
                const bool in = valid && pair_lt(v, cid, ld[k - 1], lid[k - 1]);
                const uint64_t sm = __ballot(in);
                if (!sm) continue;
                int c_self = 0;
                if (in) {
                    int lo = 0, hi = k;
                    while (lo < hi) {
                        const int mid = (lo + hi) >> 1;
                        if (pair_lt(ld[mid], lid[mid], v, cid))
                            lo = mid + 1;
                        else
                            hi = mid;
                    }
                    c_self = lo;
                }
                const int e0 = lane, e1 = lane + kWave;
                const float d0v = e0 < k ? ld[e0] : FLT_MAX;
                const uint32_t i0 = e0 < k ? lid[e0] : kNone;
                const float d1v = e1 < k ? ld[e1] : FLT_MAX;
                const uint32_t i1 = e1 < k ? lid[e1] : kNone;
                int c0n = 0, c1n = 0;
                for (uint64_t m = sm; m; m &= m - 1) {
                    const int src = __builtin_ctzll(m);
                    const float sv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), src));
                    const uint32_t si = static_cast<uint32_t>(
                        __builtin_amdgcn_readlane(static_cast<int>(cid), src));
                    c0n += pair_lt(sv, si, d0v, i0) ? 1 : 0;
                    c1n += pair_lt(sv, si, d1v, i1) ? 1 : 0;
                    c_self += pair_lt(sv, si, v, cid) ? 1 : 0;
                }
                // all reads of the old list precede these writes (one wave)
                if (e0 < k && e0 + c0n < k) {
                    ld[e0 + c0n] = d0v;
                    lid[e0 + c0n] = i0;
                }
                if (e1 < k && e1 + c1n < k) {
                    ld[e1 + c1n] = d1v;
                    lid[e1 + c1n] = i1;
                }
                if (in && c_self < k) {
                    ld[c_self] = v;
                    lid[c_self] = cid;
                }
            }
        }
    }
    __syncthreads();
    for (int e = tid; e < nq * k; e += kThreads) {
        const size_t o = static_cast<size_t>(q0) * k + static_cast<size_t>(e);
        out_ids[o] = lid_all[e];
        if (out_d) out_d[o] = ld_all[e];
    }
}

__global__ void knn_tile_count_kernel(const uint32_t* bucket_off, uint32_t buckets,
                                      uint32_t* counts)
{
    const uint32_t b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= buckets) return;
    const uint32_t n = bucket_off[b + 1] - bucket_off[b];
    counts[b] = (n + kTile - 1) / kTile;
}

__global__ void knn_tile_fill_kernel(const uint32_t* bucket_off, uint32_t buckets,
                                     const uint32_t* tile_off, uint32_t* tile_bucket,
                                     uint32_t* tile_row0)
{
    const uint32_t b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= buckets) return;
    const uint32_t s = bucket_off[b], e = bucket_off[b + 1];
    uint32_t t = tile_off[b];
    for (uint32_t r = s; r < e; r += kTile, ++t) {
        tile_bucket[t] = b;
        tile_row0[t] = r;
    }
}

// --- counter-based random numbers (SplitMix64's finaliser) ---------------
__host__ __device__ __forceinline__ uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Draw `index` of stream `stream` under `seed`.
__host__ __device__ __forceinline__ uint64_t draw64(uint64_t seed, uint64_t stream, uint64_t index)
{
    return mix64(mix64(seed ^ (stream * 0xD1B54A32D192ED03ull)) + index * 0x9E3779B97F4A7C15ull);
}

__host__ __device__ __forceinline__ double draw_unit(uint64_t seed, uint64_t stream, uint64_t index)
{
    return static_cast<double>(draw64(seed, stream, index) >> 11) * (1.0 / 9007199254740992.0);
}

// k-means++ distance update: best[i] = min(best[i], d(x_i, c)) for the
// centre picked last (row *pick of the rows), or best[i] = d(x_i, c) when
// `first`.  One wave per row: lane j sums dims j, j+64, ... (fmaf), then an
// xor butterfly over offsets 32..1.
template <class T>
__global__ __launch_bounds__(kThreads) void kpp_min_kernel(const T* rows, uint32_t dim, uint64_t n,
                                                           const uint32_t* pick, int first,
                                                           float* best)
{
    const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    const uint64_t r = static_cast<uint64_t>(blockIdx.x) * (kThreads / kWave) + threadIdx.x / kWave;
    if (r >= n) return;
    const T* x = rows + r * dim;
    const T* c = rows + static_cast<size_t>(*pick) * dim;
    float s = 0.0f;
    for (uint32_t d = static_cast<uint32_t>(lane); d < dim; d += kWave) {
        const float t = to_f(x[d]) - to_f(c[d]);
        s = fmaf(t, t, s);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, kWave);
    if (lane == 0) best[r] = first ? s : fminf(best[r], s);
}

// k-means++ pick: one 1024-thread workgroup.  Thread t sums best over rows
// [t*chunk, (t+1)*chunk) in fp64 (ascending); thread 0 adds the partial
// sums in order, sets target = u * total and walks the chunks, then the
// rows of the chunk, to the first row where the running sum reaches the
// target (the last row when rounding leaves it short; row floor(u * n) when
// every distance is zero).  Writes the pick and copies its row to centre j.
template <class T>
__global__ __launch_bounds__(1024) void kpp_pick_kernel(const T* rows, uint32_t dim, uint64_t n,
                                                        const float* best, double u,
                                                        uint32_t* pick, float* centre)
{
    __shared__ double part[1024];
    __shared__ uint32_t s_pick;
    const uint32_t t = threadIdx.x;
    const uint64_t chunk = (n + 1023) / 1024;
    const uint64_t b0 = static_cast<uint64_t>(t) * chunk;
    double s = 0.0;
    for (uint64_t i = b0; i < b0 + chunk && i < n; ++i) s += static_cast<double>(best[i]);
    part[t] = s;
    __syncthreads();
    if (t == 0) {
        double total = 0.0;
        for (int i = 0; i < 1024; ++i) total += part[i];
        uint64_t pk;
        if (!(total > 0.0)) {
            pk = static_cast<uint64_t>(u * static_cast<double>(n));
            if (pk >= n) pk = n - 1;
        } else {
            const double target = u * total;
            double run = 0.0;
            int c = 0;
            for (; c < 1023; ++c) {
                if (run + part[c] >= target) break;
                run += part[c];
            }
            pk = n - 1;
            const uint64_t e = static_cast<uint64_t>(c + 1) * chunk;
            for (uint64_t i = static_cast<uint64_t>(c) * chunk; i < e && i < n; ++i) {
                run += static_cast<double>(best[i]);
                if (run >= target) {
                    pk = i;
                    break;
                }
            }
        }
        s_pick = static_cast<uint32_t>(pk);
        *pick = s_pick;
    }
    __syncthreads();
    const T* x = rows + static_cast<size_t>(s_pick) * dim;
    for (uint32_t d = t; d < dim; d += 1024) centre[d] = to_f(x[d]);
}

__global__ void first_pick_kernel(uint32_t v, uint32_t* pick) { *pick = v; }

template <class T>
__global__ void copy_row_kernel(const T* rows, uint32_t dim, const uint32_t* pick, float* centre)
{
    const T* x = rows + static_cast<size_t>(*pick) * dim;
    for (uint32_t d = threadIdx.x; d < dim; d += blockDim.x) centre[d] = to_f(x[d]);
}

// Exclusive prefix sums of counts[0 .. m) into out[0 .. m] (out[m] = the
// total), one 1024-thread workgroup: thread t adds a contiguous chunk in
// order, thread 0 scans the 1024 chunk sums, then each thread writes its
// chunk's prefixes.
__global__ __launch_bounds__(1024) void exclusive_scan_kernel(const uint32_t* counts, uint64_t m,
                                                              uint32_t* out)
{
    __shared__ uint32_t part[1024];
    const uint32_t t = threadIdx.x;
    const uint64_t chunk = (m + 1023) / 1024;
    const uint64_t b0 = static_cast<uint64_t>(t) * chunk;
    const uint64_t b1 = b0 + chunk < m ? b0 + chunk : m;
    uint32_t s = 0;
    for (uint64_t i = b0; i < b1; ++i) s += counts[i];
    part[t] = s;
    __syncthreads();
    if (t == 0) {
        uint32_t run = 0;
        for (int i = 0; i < 1024; ++i) {
            const uint32_t v = part[i];
            part[i] = run;
            run += v;
        }
        out[m] = run;
    }
    __syncthreads();
    uint32_t run = part[t];
    for (uint64_t i = b0; i < b1; ++i) {
        out[i] = run;
        run += counts[i];
    }
}

// counts[c] = number of i with keys[i] == c (keys >= K are skipped).
__global__ void key_count_kernel(const uint32_t* keys, uint64_t n, uint32_t K, uint32_t* counts)
{
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint32_t k = keys[i];
    if (k < K) atomicAdd(&counts[k], 1u);
}

// The rows of each key in ascending order: one wave per key scans the keys
// in row order and compacts its matches with a ballot into
// order[start[c] ..).
__global__ __launch_bounds__(kThreads) void key_lists_kernel(const uint32_t* keys, uint64_t n,
                                                             uint32_t K, const uint32_t* start,
                                                             uint32_t* order)
{
    const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    const uint32_t c = blockIdx.x * (kThreads / kWave) + threadIdx.x / kWave;
    if (c >= K) return;
    uint32_t pos = start[c];
    const uint64_t below = (1ull << lane) - 1;
    for (uint64_t i0 = 0; i0 < n; i0 += kWave) {
        const uint64_t i = i0 + static_cast<uint64_t>(lane);
        const bool hit = i < n && keys[i] == c;
        const uint64_t m = __ballot(hit);
        if (hit) order[pos + static_cast<uint32_t>(__popcll(m & below))] = static_cast<uint32_t>(i);
        pos += static_cast<uint32_t>(__popcll(m));
    }
}

// Centre update: centre c = mean of its rows (fp64 sums over the rows in
// ascending order, then the quotient rounded to fp32); a centre with no row
// keeps its value.  One workgroup per centre, threads over dims.
template <class T>
__global__ __launch_bounds__(kThreads) void centre_mean_kernel(const T* rows, uint32_t dim, uint64_t n,
                                                               const uint32_t* order,
                                                               const uint32_t* start,
                                                               float* centres)
{
    const uint32_t c = blockIdx.x;
    const uint32_t s = start[c], e = start[c + 1];
    if (s >= e || e > n) return;
    for (uint32_t d = threadIdx.x; d < dim; d += kThreads) {
        double sum = 0.0;
        for (uint32_t i = s; i < e; ++i) {
            const uint32_t r = order[i];
            if (r < n) sum += static_cast<double>(to_f(rows[static_cast<size_t>(r) * dim + d]));
        }
        centres[static_cast<size_t>(c) * dim + d] = static_cast<float>(sum / static_cast<double>(e - s));
    }
}

// PQ: code of (row, subspace m) = argmin over the 256 centres of
// sum_t (x - c)^2 over the subspace's dims (fmaf, ascending; ties to the
// lower centre).  Block (x: 256 rows, y: subspace) with the subspace's
// centres in LDS.
template <class T, int S>
__global__ __launch_bounds__(kThreads) void pq_assign_kernel(const T* rows, uint32_t dim,
                                                             uint64_t n, uint32_t pq_dim,
                                                             const float* centroids,
                                                             uint8_t* codes, uint32_t code_stride)
{
    extern __shared__ __align__(16) unsigned char lds[];
    float* sc = reinterpret_cast<float*>(lds);  // [256][sub]
    const uint32_t sub = dim / pq_dim;
    const uint32_t m = blockIdx.y;
    for (uint32_t e = threadIdx.x; e < 256u * sub; e += kThreads)
        sc[e] = centroids[static_cast<size_t>(e / sub) * dim + m * sub + e % sub];
    __syncthreads();
    const uint64_t r = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (r >= n) return;
    const T* x = rows + r * dim + m * sub;
    float best = FLT_MAX;
    uint32_t bk = 0;
    if (S > 0) {  // the subspace in registers
        float xv[S > 0 ? S : 1];
#pragma unroll
        for (int t = 0; t < S; ++t) xv[t] = to_f(x[t]);
        for (uint32_t k = 0; k < 256; ++k) {
            float acc = 0.0f;
#pragma unroll
            for (int t = 0; t < S; ++t) {
                const float d = xv[t] - sc[k * S + t];
                acc = fmaf(d, d, acc);
            }
            if (acc < best) {
                best = acc;
                bk = k;
            }
        }
    } else {
        for (uint32_t k = 0; k < 256; ++k) {
            float acc = 0.0f;
            for (uint32_t t = 0; t < sub; ++t) {
                const float d = to_f(x[t]) - sc[k * sub + t];
                acc = fmaf(d, d, acc);
            }
            if (acc < best) {
                best = acc;
                bk = k;
            }
        }
    }
    codes[r * code_stride + m] = static_cast<uint8_t>(bk);
}

// PQ codebook update grouping: key m * 256 + code of each (row, subspace).
__global__ void pq_key_count_kernel(const uint8_t* codes, uint64_t n, uint32_t pq_dim,
                                    uint32_t* counts)
{
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n * pq_dim) return;
    const uint32_t m = static_cast<uint32_t>(i % pq_dim);
    atomicAdd(&counts[m * 256u + codes[i]], 1u);
}

// The rows of each PQ key in ascending order (one wave per key, as
// key_lists_kernel, reading the key's subspace column of the codes).
__global__ __launch_bounds__(kThreads) void pq_key_lists_kernel(const uint8_t* codes, uint64_t n,
                                                                uint32_t pq_dim,
                                                                const uint32_t* start,
                                                                uint32_t* order)
{
    const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    const uint32_t c = blockIdx.x * (kThreads / kWave) + threadIdx.x / kWave;
    if (c >= pq_dim * 256u) return;
    const uint32_t m = c / 256u, code = c % 256u;
    uint32_t pos = start[c];
    const uint64_t below = (1ull << lane) - 1;
    for (uint64_t r0 = 0; r0 < n; r0 += kWave) {
        const uint64_t r = r0 + static_cast<uint64_t>(lane);
        const bool hit = r < n && codes[r * pq_dim + m] == code;
        const uint64_t mk = __ballot(hit);
        if (hit) order[pos + static_cast<uint32_t>(__popcll(mk & below))] = static_cast<uint32_t>(r);
        pos += static_cast<uint32_t>(__popcll(mk));
    }
}

// PQ codebook update: entry (m, k) = mean over its rows of the subspace's
// dims (fp64 sums over rows ascending, rounded to fp32); empty keeps.
template <class T>
__global__ void pq_mean_kernel(const T* rows, uint32_t dim, uint64_t n, uint32_t pq_dim,
                               const uint32_t* order, const uint32_t* start, float* centroids)
{
    const uint32_t key = blockIdx.x;
    const uint32_t m = key / 256u, k = key % 256u;
    const uint32_t sub = dim / pq_dim;
    const uint32_t s = start[key], e = start[key + 1];
    if (s >= e || e > n * pq_dim) return;
    for (uint32_t t = threadIdx.x; t < sub; t += blockDim.x) {
        double sum = 0.0;
        for (uint32_t i = s; i < e; ++i) {
            const uint32_t r = order[i];
            if (r < n) sum += static_cast<double>(to_f(rows[static_cast<size_t>(r) * dim + m * sub + t]));
        }
        centroids[static_cast<size_t>(k) * dim + m * sub + t] =
            static_cast<float>(sum / static_cast<double>(e - s));
    }
}

template <class T>
__global__ void to_f32_kernel(const T* in, uint64_t count, float* out)
{
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < count) out[i] = to_f(in[i]);
}

// RaBitQ one-bit encoding of rotated rows against their anchors (the
// reference's pack_and_compute_factors_kernel, quantizer_gpu_fast.cu:
// 180-265).  One wave per row; lane j takes dims j, j+64, ...:
//   r = xr - c, bit = r > 0, xu = bit - 0.5, packed MSB-first in u32 words
//   (dim d is bit 31 - d%32 of word d/32: a word is the bit-reversed ballot
//   half of 32 lanes);
//   l2 = sum r^2, ip_r = sum r xu, ip_c = sum c xu (fmaf per lane, then an
//   xor butterfly 32..1); xu_sq = P / 4;
//   ip_r == 0 -> inf; f_add = l2 + 2 l2 (ip_c / ip_r); f_rescale = -2 l2 / ip_r;
//   ratio = l2 xu_sq / ip_r^2; inner = max((ratio - 1) / max(P - 1, 1), 0);
//   f_err = 2 (sqrt(max(l2, 0)) * 1.9 * sqrt(inner)).
__global__ __launch_bounds__(kThreads) void rabitq_encode_kernel(const float* xr, uint64_t n,
                                                                 uint32_t P, const float* anchors,
                                                                 uint32_t num_anchors,
                                                                 const uint32_t* aid,
                                                                 uint32_t* code_words,
                                                                 float* factors)
{
    const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    const uint64_t r = static_cast<uint64_t>(blockIdx.x) * (kThreads / kWave) + threadIdx.x / kWave;
    if (r >= n) return;
    const float* x = xr + r * P;
    uint32_t* w = code_words + r * (P / 32);
    if (aid[r] >= num_anchors) {  // no anchor (a row of NaN scores): zero code and factors
        for (uint32_t q = static_cast<uint32_t>(lane); q < P / 32; q += kWave) w[q] = 0u;
        if (lane < 3) factors[r * 3 + lane] = 0.0f;
        return;
    }
    const float* c = anchors + static_cast<size_t>(aid[r]) * P;
    float l2 = 0.0f, ipr = 0.0f, ipc = 0.0f;
    for (uint32_t t = 0; t < P / kWave; ++t) {
        const uint32_t d = t * kWave + static_cast<uint32_t>(lane);
        const float cv = c[d];
        const float rv = x[d] - cv;
        const bool bit = rv > 0.0f;
        const float xu = bit ? 0.5f : -0.5f;
        l2 = fmaf(rv, rv, l2);
        ipr = fmaf(rv, xu, ipr);
        ipc = fmaf(cv, xu, ipc);
        const uint64_t m = __ballot(bit);
        if (lane == 0) {
            w[2 * t] = __builtin_bitreverse32(static_cast<uint32_t>(m));
            w[2 * t + 1] = __builtin_bitreverse32(static_cast<uint32_t>(m >> 32));
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        l2 += __shfl_xor(l2, off, kWave);
        ipr += __shfl_xor(ipr, off, kWave);
        ipc += __shfl_xor(ipc, off, kWave);
    }
    if (lane == 0) {
        const float xu_sq = 0.25f * static_cast<float>(P);
        const float denom = ipr == 0.0f ? INFINITY : ipr;
        const float f_add = l2 + 2.0f * l2 * (ipc / denom);
        const float f_rescale = -2.0f * l2 / denom;
        const float ratio = (l2 * xu_sq) / (denom * denom);
        const float inner = fmaxf((ratio - 1.0f) / fmaxf(static_cast<float>(P) - 1.0f, 1.0f), 0.0f);
        const float l2n = sqrtf(fmaxf(l2, 0.0f));
        const float f_err = 2.0f * (l2n * 1.9f * sqrtf(inner));
        factors[r * 3 + 0] = f_add;
        factors[r * 3 + 1] = f_rescale;
        factors[r * 3 + 2] = f_err;
    }
}

// Column sums in fp64 over blocks of kColBlock rows (rows ascending within
// a block); the blocks' partial sums are then added in block order.
constexpr uint32_t kColBlock = 4096;

template <class T>
__global__ __launch_bounds__(kThreads) void col_partial_kernel(const T* rows, uint32_t dim,
                                                               uint64_t n, double* partial)
{
    const uint64_t b = blockIdx.x;
    const uint64_t s = b * kColBlock;
    const uint64_t e = s + kColBlock < n ? s + kColBlock : n;
    for (uint32_t d = threadIdx.x; d < dim; d += kThreads) {
        double sum = 0.0;
        for (uint64_t i = s; i < e; ++i) sum += static_cast<double>(to_f(rows[i * dim + d]));
        partial[b * dim + d] = sum;
    }
}

__global__ void col_mean_kernel(const double* partial, uint32_t dim, uint64_t blocks, uint64_t n,
                                double* mean)
{
    const uint32_t d = blockIdx.x * blockDim.x + threadIdx.x;
    if (d >= dim) return;
    double sum = 0.0;
    for (uint64_t b = 0; b < blocks; ++b) sum += partial[b * dim + d];
    mean[d] = sum / static_cast<double>(n);
}

// fp64 distance of each row to the mean: sum_d (x_d - mu_d)^2, fma over d
// ascending (one thread per row).
template <class T>
__global__ void mean_dist_kernel(const T* rows, uint32_t dim, uint64_t n, const double* mean,
                                 double* dist)
{
    const uint64_t r = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (r >= n) return;
    const T* x = rows + r * dim;
    double s = 0.0;
    for (uint32_t d = 0; d < dim; ++d) {
        const double t = static_cast<double>(to_f(x[d])) - mean[d];
        s = fma(t, t, s);
    }
    dist[r] = s;
}

// argmin of (dist, row): each block reduces its rows, then one block
// reduces the block results.
__global__ __launch_bounds__(kThreads) void argmin_block_kernel(const double* dist, uint64_t n,
                                                                double* bd, uint64_t* bi)
{
    __shared__ double sv[kThreads];
    __shared__ uint64_t si[kThreads];
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    sv[threadIdx.x] = i < n ? dist[i] : DBL_MAX;
    si[threadIdx.x] = i < n ? i : ~0ull;
    __syncthreads();
    for (int s = kThreads / 2; s > 0; s >>= 1) {
        if (static_cast<int>(threadIdx.x) < s) {
            const double ov = sv[threadIdx.x + s];
            const uint64_t oi = si[threadIdx.x + s];
            if (ov < sv[threadIdx.x] || (ov == sv[threadIdx.x] && oi < si[threadIdx.x])) {
                sv[threadIdx.x] = ov;
                si[threadIdx.x] = oi;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        bd[blockIdx.x] = sv[0];
        bi[blockIdx.x] = si[0];
    }
}

__global__ __launch_bounds__(kThreads) void argmin_final_kernel(const double* bd, const uint64_t* bi,
                                                                uint64_t blocks, uint32_t* out)
{
    __shared__ double sv[kThreads];
    __shared__ uint64_t si[kThreads];
    double v = DBL_MAX;
    uint64_t ix = ~0ull;
    for (uint64_t b = threadIdx.x; b < blocks; b += kThreads)
        if (bd[b] < v || (bd[b] == v && bi[b] < ix)) {
            v = bd[b];
            ix = bi[b];
        }
    sv[threadIdx.x] = v;
    si[threadIdx.x] = ix;
    __syncthreads();
    for (int s = kThreads / 2; s > 0; s >>= 1) {
        if (static_cast<int>(threadIdx.x) < s) {
            const double ov = sv[threadIdx.x + s];
            const uint64_t oi = si[threadIdx.x + s];
            if (ov < sv[threadIdx.x] || (ov == sv[threadIdx.x] && oi < si[threadIdx.x])) {
                sv[threadIdx.x] = ov;
                si[threadIdx.x] = oi;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) *out = static_cast<uint32_t>(si[0]);
}

// Bucket representative: the row of bucket b nearest the bucket's mean.
// The mean is fp64 sums over the bucket's rows (ascending) rounded to fp32;
// a row's distance is sum_d (x_d - mean_d)^2 in fp32 (fmaf, ascending); ties
// to the lower row.  One workgroup per bucket; `means` [buckets][dim] is
// written too.
template <class T>
__global__ __launch_bounds__(kThreads) void bucket_rep_kernel(const T* rows, uint32_t dim,
                                                              const uint32_t* bucket_off,
                                                              float* means, uint32_t* rep)
{
    __shared__ float sv[kThreads];
    __shared__ uint32_t si[kThreads];
    const uint32_t b = blockIdx.x;
    const uint32_t s = bucket_off[b], e = bucket_off[b + 1];
    float* mu = means + static_cast<size_t>(b) * dim;
    if (s == e) {
        if (threadIdx.x == 0) rep[b] = kNone;
        return;
    }
    for (uint32_t d = threadIdx.x; d < dim; d += kThreads) {
        double sum = 0.0;
        for (uint32_t i = s; i < e; ++i) sum += static_cast<double>(to_f(rows[static_cast<size_t>(i) * dim + d]));
        mu[d] = static_cast<float>(sum / static_cast<double>(e - s));
    }
    __syncthreads();
    float bv = FLT_MAX;
    uint32_t bi = kNone;
    for (uint32_t i = s + threadIdx.x; i < e; i += kThreads) {
        const T* x = rows + static_cast<size_t>(i) * dim;
        float acc = 0.0f;
        for (uint32_t d = 0; d < dim; ++d) {
            const float t = to_f(x[d]) - mu[d];
            acc = fmaf(t, t, acc);
        }
        if (pair_lt(acc, i, bv, bi)) {
            bv = acc;
            bi = i;
        }
    }
    sv[threadIdx.x] = bv;
    si[threadIdx.x] = bi;
    __syncthreads();
    for (int st = kThreads / 2; st > 0; st >>= 1) {
        if (static_cast<int>(threadIdx.x) < st &&
            pair_lt(sv[threadIdx.x + st], si[threadIdx.x + st], sv[threadIdx.x], si[threadIdx.x])) {
            sv[threadIdx.x] = sv[threadIdx.x + st];
            si[threadIdx.x] = si[threadIdx.x + st];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) rep[b] = si[0];
}

// Link rules of this repo's graph (one wave per row of the bucket-sorted
// space).  The candidate sequence of row i in bucket b:
//   an ordinary row: knn[i][0 .. local), rep[b] (not i), rep[near[b][0 ..
//     near)], then draws (seed, stream 1, i * 256 + j) mod n for j < R;
//   a bucket representative: knn[i][0 .. rep_local), rep[near[b][0 ..
//     rep_near)], then draws (seed, stream 2, i * 256 + j) mod n, j < R;
//   the entry row: draws (seed, stream 3, i * 256 + j) mod n, j < 4 R.
// The row keeps the first R distinct candidates that are valid and not
// itself, in sequence order, padded with UINT32_MAX.  The output is in the
// caller's row order: row order[i] gets order[candidate].
struct LinkArgs {
    uint32_t n;
    const uint32_t* knn;
    uint32_t knn_width;
    const uint32_t* bucket_of;
    const uint32_t* rep;
    const uint32_t* near;
    uint32_t near_width;
    uint32_t buckets;
    const uint32_t* order;
    uint32_t degree, local, near_links, rep_local, rep_near;
    uint32_t entry;  // sorted-space row of the entry (kNone: none)
    uint64_t seed;
    uint32_t* out;
};

constexpr int kLinkCand = 512;

__global__ __launch_bounds__(kThreads) void links_kernel(LinkArgs a)
{
    __shared__ uint32_t cand_all[(kThreads / kWave) * kLinkCand];
    const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    const uint32_t i = blockIdx.x * (kThreads / kWave) + static_cast<uint32_t>(wave);
    if (i >= a.n) return;
    uint32_t* cand = cand_all + wave * kLinkCand;
    const uint32_t dst = a.order[i];
    if (dst >= a.n) return;
    const uint32_t b = a.bucket_of[i];
    const bool bvalid = b < a.buckets;
    const uint32_t rep_b = bvalid ? a.rep[b] : kNone;
    const bool is_rep = rep_b == i;
    const bool is_entry = i == a.entry;
    const uint32_t R = a.degree;
    int nc = 0;
    if (is_entry) {
        for (uint32_t j = static_cast<uint32_t>(lane); j < 4 * R; j += kWave)
            cand[j] = static_cast<uint32_t>(draw64(a.seed, 3, static_cast<uint64_t>(i) * 256 + j) % a.n);
        nc = static_cast<int>(4 * R);
    } else {
        const uint32_t nk = is_rep ? a.rep_local : a.local;
        const uint32_t nn = is_rep ? a.rep_near : a.near_links;
        for (uint32_t j = static_cast<uint32_t>(lane); j < nk; j += kWave)
            cand[j] = j < a.knn_width ? a.knn[static_cast<size_t>(i) * a.knn_width + j] : kNone;
        nc = static_cast<int>(nk);
        if (!is_rep) {
            if (lane == 0) cand[nc] = rep_b;
            nc += 1;
        }
        for (uint32_t j = static_cast<uint32_t>(lane); j < nn; j += kWave) {
            const uint32_t nb = bvalid && j < a.near_width
                                    ? a.near[static_cast<size_t>(b) * a.near_width + j]
                                    : kNone;
            cand[nc + static_cast<int>(j)] = nb < a.buckets ? a.rep[nb] : kNone;
        }
        nc += static_cast<int>(nn);
        const uint64_t stream = is_rep ? 2 : 1;
        for (uint32_t j = static_cast<uint32_t>(lane); j < R; j += kWave)
            cand[nc + static_cast<int>(j)] =
                static_cast<uint32_t>(draw64(a.seed, stream, static_cast<uint64_t>(i) * 256 + j) % a.n);
        nc += static_cast<int>(R);
    }
    __threadfence_block();  // the wave's candidate writes before other lanes read them
    // a candidate is kept if valid, not the row, and not equal to an
    // earlier candidate; the first R kept, in order
    uint32_t kept = 0;
    uint32_t* out = a.out + static_cast<size_t>(dst) * R;
    for (int c0 = 0; c0 < nc && kept < R; c0 += kWave) {
        const int c = c0 + lane;
        bool keep = false;
        uint32_t v = kNone;
        if (c < nc) {
            v = cand[c];
            keep = v != kNone && v != i && v < a.n;
            for (int j = 0; keep && j < c; ++j) keep = cand[j] != v;
        }
        const uint64_t m = __ballot(keep);
        if (keep) {
            const uint32_t pos = kept + static_cast<uint32_t>(__popcll(m & ((1ull << lane) - 1)));
            if (pos < R) out[pos] = a.order[v] < a.n ? a.order[v] : kNone;
        }
        kept += static_cast<uint32_t>(__popcll(m));
    }
    for (uint32_t j = kept + static_cast<uint32_t>(lane); j < R; j += kWave) out[j] = kNone;
}

// CAGRA's rank-based reordering (Ootomo et al., "CAGRA: Highly Parallel
// Graph Construction and Approximate Nearest Neighbor Search for GPUs",
// ICDE 2024, sec. IV-B): the edge to the entry at rank j of row i's kNN
// list K_i counts a detour for every entry u at rank m of K_i whose own
// list holds K_i[j] at a rank r with max(m, r) < j.  The row keeps the
// `degree` valid entries of least (detours, j).  One wave per row; K_i's
// entries are looked up in an LDS hash of 256 slots (kin <= 128).
constexpr int kPruneSlots = 256;

__global__ __launch_bounds__(kThreads) void cagra_prune_kernel(const uint32_t* knn, uint32_t n,
                                                               uint32_t kin, uint32_t degree,
                                                               uint32_t* out)
{
    __shared__ uint32_t hkey_all[(kThreads / kWave) * kPruneSlots];
    __shared__ uint32_t hpos_all[(kThreads / kWave) * kPruneSlots];
    __shared__ uint32_t det_all[(kThreads / kWave) * kMaxKnn];
    __shared__ uint32_t lst_all[(kThreads / kWave) * kMaxKnn];
    const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    const uint32_t i = blockIdx.x * (kThreads / kWave) + static_cast<uint32_t>(wave);
    if (i >= n) return;
    uint32_t* hkey = hkey_all + wave * kPruneSlots;
    uint32_t* hpos = hpos_all + wave * kPruneSlots;
    uint32_t* det = det_all + wave * kMaxKnn;
    uint32_t* lst = lst_all + wave * kMaxKnn;
    for (int s = lane; s < kPruneSlots; s += kWave) hkey[s] = kNone;
    const uint32_t* ki = knn + static_cast<size_t>(i) * kin;
    for (uint32_t j = static_cast<uint32_t>(lane); j < kin; j += kWave) {
        lst[j] = ki[j];
        det[j] = 0;
    }
    __threadfence_block();  // the wave's LDS writes before other lanes read them
    if (lane == 0) {
        for (uint32_t j = 0; j < kin; ++j) {
            const uint32_t v = lst[j];
            if (v == kNone) continue;
            uint32_t s = (v * 2654435761u) & (kPruneSlots - 1);
            while (hkey[s] != kNone && hkey[s] != v) s = (s + 1) & (kPruneSlots - 1);
            if (hkey[s] == kNone) {
                hkey[s] = v;
                hpos[s] = j;
            }
        }
    }
    __threadfence_block();
    for (uint32_t m = 0; m < kin; ++m) {
        const uint32_t u = lst[m];
        if (u == kNone || u >= n) continue;
        const uint32_t* ku = knn + static_cast<size_t>(u) * kin;
        for (uint32_t r = static_cast<uint32_t>(lane); r < kin; r += kWave) {
            const uint32_t v = ku[r];
            if (v == kNone) continue;
            uint32_t s = (v * 2654435761u) & (kPruneSlots - 1);
            while (hkey[s] != kNone && hkey[s] != v) s = (s + 1) & (kPruneSlots - 1);
            if (hkey[s] == v) {
                const uint32_t j = hpos[s];
                if (j > m && j > r) atomicAdd(&det[j], 1u);
            }
        }
    }
    __threadfence_block();
    // rank of entry j among the valid entries by (detours, j)
    uint32_t* o = out + static_cast<size_t>(i) * degree;
    for (uint32_t j = static_cast<uint32_t>(lane); j < degree; j += kWave) o[j] = kNone;
    for (uint32_t j = static_cast<uint32_t>(lane); j < kin; j += kWave) {
        if (lst[j] == kNone) continue;
        const uint32_t dj = det[j];
        uint32_t rank = 0;
        for (uint32_t q = 0; q < kin; ++q)
            if (lst[q] != kNone && (det[q] < dj || (det[q] == dj && q < j))) ++rank;
        if (rank < degree) o[rank] = lst[j];
    }
}

// Reverse edges: counts per target row, then each edge u -> v at position
// k stored as the key (k << 27) | u in v's segment (n < 2^27, degree <=
// 128); a segment's order is arbitrary, its set is fixed.
__global__ void reverse_count_kernel(const uint32_t* g, uint32_t n, uint32_t degree, uint32_t* counts)
{
    const uint64_t e = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= static_cast<uint64_t>(n) * degree) return;
    const uint32_t v = g[e];
    if (v < n) atomicAdd(&counts[v], 1u);
}

__global__ void reverse_fill_kernel(const uint32_t* g, uint32_t n, uint32_t degree,
                                    const uint32_t* rstart, uint32_t* fill, uint64_t* rkeys)
{
    const uint64_t e = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= static_cast<uint64_t>(n) * degree) return;
    const uint32_t v = g[e];
    if (v >= n) return;
    const uint32_t u = static_cast<uint32_t>(e / degree);
    const uint32_t k = static_cast<uint32_t>(e % degree);
    const uint32_t slot = rstart[v] + atomicAdd(&fill[v], 1u);
    rkeys[slot] = (static_cast<uint64_t>(k) << 27) | u;
}

// CAGRA's reverse-edge merge (same paper, sec. IV-B): row i keeps the first
// degree/2 valid edges of its reordered list, then its reverse edges in
// order of (position in the source's list, source row), then the rest of
// its reordered list, skipping repeats; at most 2 * degree reverse edges
// are considered.  One thread per row.
__global__ void reverse_merge_kernel(const uint32_t* pruned, const uint64_t* rkeys,
                                     const uint32_t* rstart, uint32_t n, uint32_t degree,
                                     uint32_t* out)
{
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint32_t* f = pruned + static_cast<size_t>(i) * degree;
    uint32_t* o = out + static_cast<size_t>(i) * degree;
    uint32_t k = 0, kf = 0;
    auto has = [&](uint32_t v) {
        for (uint32_t q = 0; q < k; ++q)
            if (o[q] == v) return true;
        return false;
    };
    const uint32_t protect = degree / 2;
    for (; kf < degree && k < protect; ++kf) {
        const uint32_t v = f[kf];
        if (v == kNone || v == i || has(v)) continue;
        o[k++] = v;
    }
    // the reverse edges in (position, source) order: the segment's keys
    // taken by successive minima, the first 2 degree of them
    const uint32_t rs = rstart[i], re = rstart[i + 1];
    uint64_t prev = 0;
    bool have_prev = false;
    for (uint32_t t = 0; t < 2 * degree && k < degree; ++t) {
        uint64_t best = ~0ull;
        for (uint32_t r = rs; r < re; ++r) {
            const uint64_t key = rkeys[r];
            if ((!have_prev || key > prev) && key < best) best = key;
        }
        if (best == ~0ull) break;
        prev = best;
        have_prev = true;
        const uint32_t v = static_cast<uint32_t>(best & ((1ull << 27) - 1));
        if (v == i || has(v)) continue;
        o[k++] = v;
    }
    for (; kf < degree && k < degree; ++kf) {
        const uint32_t v = f[kf];
        if (v == kNone || v == i || has(v)) continue;
        o[k++] = v;
    }
    for (; k < degree; ++k) o[k] = kNone;
}

// One level of a breadth-first walk: marks the unreached targets of the
// frontier's edges and appends them to the next frontier (the reached set
// after the walk does not depend on the append order).
__global__ void bfs_level_kernel(const uint32_t* g, uint32_t n, uint32_t degree,
                                 const uint32_t* frontier, uint32_t count, uint32_t* reached,
                                 uint32_t* next, uint32_t* next_count)
{
    const uint64_t e = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= static_cast<uint64_t>(count) * degree) return;
    const uint32_t u = frontier[e / degree];
    const uint32_t v = g[static_cast<size_t>(u) * degree + e % degree];
    if (v >= n) return;
    if (atomicExch(&reached[v], 1u) == 0u) next[atomicAdd(next_count, 1u)] = v;
}

__global__ void bfs_seed_kernel(uint32_t entry, uint32_t* reached, uint32_t* frontier)
{
    reached[entry] = 1u;
    frontier[0] = entry;
}

template <class T>
int assign_t(Context* ctx, const void* rows, uint32_t dim, uint64_t n, const float* centres,
             uint32_t k, const float* cnorm, uint32_t* out_idx, float* out_score)
{
    const uint64_t blocks = (n + kTile - 1) / kTile;
    hipLaunchKernelGGL(assign_kernel<T>, dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0,
                       ctx->stream, static_cast<const T*>(rows), static_cast<size_t>(dim), dim, n,
                       centres, cnorm, k, out_idx, out_score);
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("assign launch");
    return GOFANN_OK;
}

int check_elem(Context* ctx, int elem)
{
    if (elem != GOFANN_ELEM_U8 && elem != GOFANN_ELEM_F32 && elem != GOFANN_ELEM_F16)
        return ctx->fail(GOFANN_ERR_INVALID, "element type must be u8, f32 or f16");
    return GOFANN_OK;
}

// Device scratch of the build entry points: one grow-only buffer, carved.
struct Carve {
    unsigned char* p;
    size_t used;
    template <class U>
    U* take(size_t count)
    {
        used = (used + 255) & ~static_cast<size_t>(255);
        U* r = reinterpret_cast<U*>(p + used);
        used += count * sizeof(U);
        return r;
    }
};

size_t carve_size(std::initializer_list<size_t> bytes)
{
    size_t s = 0;
    for (size_t b : bytes) s += ((b + 255) & ~static_cast<size_t>(255)) + 256;
    return s;
}

}  // namespace

int build_assign(Context* ctx, const void* rows, int elem, uint32_t dim, uint64_t n,
                 const float* centres, uint32_t k, uint32_t* out_idx, float* out_score)
{
    if (int rc = check_elem(ctx, elem)) return rc;
    if (!rows || !centres || !out_idx || dim == 0 || k == 0)
        return ctx->fail(GOFANN_ERR_INVALID, "assign: arrays missing or empty dims");
    if (n == 0) return GOFANN_OK;
    if ((n + kTile - 1) / kTile > 0x7FFFFFFFull) return ctx->fail(GOFANN_ERR_INVALID, "assign: too many rows");
    float* cnorm = static_cast<float*>(ctx->scratch(Context::kScratchBuild, static_cast<size_t>(k) * 4));
    if (!cnorm) return ctx->fail(GOFANN_ERR_NOMEM, "assign scratch allocation failed");
    hipLaunchKernelGGL(row_sqnorm_kernel, dim3((k + 255) / 256), dim3(256), 0, ctx->stream, centres, k,
                       dim, cnorm);
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("centre norm launch");
    switch (elem) {
        case GOFANN_ELEM_U8: return assign_t<uint8_t>(ctx, rows, dim, n, centres, k, cnorm, out_idx, out_score);
        case GOFANN_ELEM_F16: return assign_t<_Float16>(ctx, rows, dim, n, centres, k, cnorm, out_idx, out_score);
        default: return assign_t<float>(ctx, rows, dim, n, centres, k, cnorm, out_idx, out_score);
    }
}

namespace {

template <class T>
int kmeanspp_t(Context* ctx, const T* rows, uint32_t dim, uint64_t n, uint32_t k, uint64_t seed,
               float* centres)
{
    unsigned char* buf = static_cast<unsigned char*>(
        ctx->scratch(Context::kScratchBuild, carve_size({n * 4, 64})));
    if (!buf) return ctx->fail(GOFANN_ERR_NOMEM, "k-means++ scratch allocation failed");
    Carve cv{buf, 0};
    float* best = cv.take<float>(n);
    uint32_t* pick = cv.take<uint32_t>(1);
    uint64_t first = static_cast<uint64_t>(draw_unit(seed, 0, 0) * static_cast<double>(n));
    if (first >= n) first = n - 1;
    hipLaunchKernelGGL(first_pick_kernel, dim3(1), dim3(1), 0, ctx->stream,
                       static_cast<uint32_t>(first), pick);
    hipLaunchKernelGGL(copy_row_kernel<T>, dim3(1), dim3(256), 0, ctx->stream, rows, dim, pick, centres);
    const uint32_t blocks = static_cast<uint32_t>((n + 3) / 4);
    for (uint32_t j = 1; j < k; ++j) {
        hipLaunchKernelGGL(kpp_min_kernel<T>, dim3(blocks), dim3(kThreads), 0, ctx->stream, rows, dim,
                           n, pick, j == 1 ? 1 : 0, best);
        hipLaunchKernelGGL(kpp_pick_kernel<T>, dim3(1), dim3(1024), 0, ctx->stream, rows, dim, n, best,
                           draw_unit(seed, 0, j), pick, centres + static_cast<size_t>(j) * dim);
    }
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("k-means++ launch");
    return GOFANN_OK;
}

template <class T>
int kmeans_t(Context* ctx, const T* rows, uint32_t dim, uint64_t n, uint32_t k, uint32_t iters,
             float* centres)
{
    unsigned char* buf = static_cast<unsigned char*>(ctx->scratch(
        Context::kScratchBuild,
        carve_size({n * 4, n * 4, (static_cast<size_t>(k) + 1) * 4, (static_cast<size_t>(k) + 1) * 4,
                    k * 4ull})));
    if (!buf) return ctx->fail(GOFANN_ERR_NOMEM, "k-means scratch allocation failed");
    Carve cv{buf, 0};
    uint32_t* idx = cv.take<uint32_t>(n);
    uint32_t* order = cv.take<uint32_t>(n);
    uint32_t* counts = cv.take<uint32_t>(static_cast<size_t>(k) + 1);
    uint32_t* start = cv.take<uint32_t>(static_cast<size_t>(k) + 1);
    float* cnorm = cv.take<float>(k);
    for (uint32_t it = 0; it < iters; ++it) {
        hipLaunchKernelGGL(row_sqnorm_kernel, dim3((k + 255) / 256), dim3(256), 0, ctx->stream, centres,
                           k, dim, cnorm);
        hipLaunchKernelGGL(assign_kernel<T>, dim3(static_cast<uint32_t>((n + kTile - 1) / kTile)),
                           dim3(kThreads), 0, ctx->stream, rows, static_cast<size_t>(dim), dim, n,
                           centres, cnorm, k, idx, static_cast<float*>(nullptr));
        // the rows of each centre in ascending order
        if (hipMemsetAsync(counts, 0, (static_cast<size_t>(k) + 1) * 4, ctx->stream) != hipSuccess)
            return ctx->fail_hip("k-means counts clear");
        hipLaunchKernelGGL(key_count_kernel, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0,
                           ctx->stream, idx, n, k, counts);
        hipLaunchKernelGGL(exclusive_scan_kernel, dim3(1), dim3(1024), 0, ctx->stream, counts,
                           static_cast<uint64_t>(k), start);
        hipLaunchKernelGGL(key_lists_kernel, dim3((k + 3) / 4), dim3(kThreads), 0, ctx->stream, idx, n,
                           k, start, order);
        hipLaunchKernelGGL(centre_mean_kernel<T>, dim3(k), dim3(kThreads), 0, ctx->stream, rows, dim,
                           n, order, start, centres);
    }
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("k-means launch");
    return GOFANN_OK;
}

template <class T>
int knn_t(Context* ctx, const T* rows, uint32_t dim, const gofann_build_buckets* b, uint32_t k,
          uint32_t* out_ids, float* out_d)
{
    const uint32_t nb = b->buckets;
    // The bucket and probe arrays index the rows: check them on the host
    // (they are small) before any kernel reads through them.
    {
        std::vector<uint32_t> off(nb + 1ull);
        if (hipMemcpyAsync(off.data(), b->bucket_offsets, off.size() * 4, hipMemcpyDeviceToHost,
                           ctx->stream) != hipSuccess ||
            hipStreamSynchronize(ctx->stream) != hipSuccess)
            return ctx->fail_hip("kNN bucket offsets copy");
        for (uint32_t i = 0; i < nb; ++i)
            if (off[i] > off[i + 1]) return ctx->fail(GOFANN_ERR_INVALID, "kNN: bucket offsets decrease");
        if (off[nb] != b->rows) return ctx->fail(GOFANN_ERR_INVALID, "kNN: bucket offsets do not end at rows");
        if (b->probe_offsets) {
            std::vector<uint32_t> po(nb + 1ull);
            if (hipMemcpyAsync(po.data(), b->probe_offsets, po.size() * 4, hipMemcpyDeviceToHost,
                               ctx->stream) != hipSuccess ||
                hipStreamSynchronize(ctx->stream) != hipSuccess)
                return ctx->fail_hip("kNN probe offsets copy");
            for (uint32_t i = 0; i < nb; ++i)
                if (po[i] > po[i + 1]) return ctx->fail(GOFANN_ERR_INVALID, "kNN: probe offsets decrease");
            std::vector<uint32_t> pb(po[nb]);
            if (!pb.empty() &&
                (hipMemcpyAsync(pb.data(), b->probe_buckets, pb.size() * 4, hipMemcpyDeviceToHost,
                                ctx->stream) != hipSuccess ||
                 hipStreamSynchronize(ctx->stream) != hipSuccess))
                return ctx->fail_hip("kNN probe buckets copy");
            for (uint32_t i = 0; i < nb; ++i)
                for (uint32_t q = po[i]; q < po[i + 1]; ++q) {
                    if (pb[q] >= nb) return ctx->fail(GOFANN_ERR_INVALID, "kNN: probe bucket out of range");
                    for (uint32_t q2 = po[i]; q2 < q; ++q2)
                        if (pb[q2] == pb[q]) return ctx->fail(GOFANN_ERR_INVALID, "kNN: a probe list repeats a bucket");
                }
        }
    }
    // query tiles per bucket: counts, exclusive sum, fill
    // (tiles <= rows / 64 + buckets)
    const size_t max_tiles = static_cast<size_t>(b->rows) / kTile + nb + 1;
    unsigned char* buf = static_cast<unsigned char*>(ctx->scratch(
        Context::kScratchBuild,
        carve_size({(nb + 1ull) * 4, (nb + 1ull) * 4, max_tiles * 4, max_tiles * 4})));
    if (!buf) return ctx->fail(GOFANN_ERR_NOMEM, "kNN scratch allocation failed");
    Carve cv{buf, 0};
    uint32_t* counts = cv.take<uint32_t>(nb + 1ull);
    uint32_t* tile_off = cv.take<uint32_t>(nb + 1ull);
    uint32_t* tile_bucket = cv.take<uint32_t>(max_tiles);
    uint32_t* tile_row0 = cv.take<uint32_t>(max_tiles);
    hipLaunchKernelGGL(knn_tile_count_kernel, dim3((nb + 255) / 256), dim3(256), 0, ctx->stream,
                       b->bucket_offsets, nb, counts);
    hipLaunchKernelGGL(exclusive_scan_kernel, dim3(1), dim3(1024), 0, ctx->stream, counts,
                       static_cast<uint64_t>(nb), tile_off);
    uint32_t tiles = 0;
    if (hipMemcpyAsync(&tiles, tile_off + nb, 4, hipMemcpyDeviceToHost, ctx->stream) != hipSuccess ||
        hipStreamSynchronize(ctx->stream) != hipSuccess)
        return ctx->fail_hip("kNN tile count");
    if (tiles > max_tiles) return ctx->fail(GOFANN_ERR_INVALID, "kNN: bucket offsets exceed the rows");
    if (tiles == 0) return GOFANN_OK;
    hipLaunchKernelGGL(knn_tile_fill_kernel, dim3((nb + 255) / 256), dim3(256), 0, ctx->stream,
                       b->bucket_offsets, nb, tile_off, tile_bucket, tile_row0);
    const size_t lds = (2 * kTileD * kTile + kTile * (kTile + 1)) * 4 + static_cast<size_t>(kTile) * k * 8;
    if (lds > static_cast<size_t>(ctx->lds_per_block))
        return ctx->fail(GOFANN_ERR_UNSUPPORTED, "kNN list exceeds the workgroup LDS");
    const void* kern = reinterpret_cast<const void*>(knn_kernel<T>);
    if (hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)) !=
        hipSuccess)
        return ctx->fail_hip("hipFuncSetAttribute kNN");
    hipLaunchKernelGGL(knn_kernel<T>, dim3(tiles), dim3(kThreads), lds, ctx->stream, rows, dim,
                       b->bucket_offsets, b->probe_offsets, b->probe_buckets, tile_bucket, tile_row0,
                       tiles, static_cast<int>(k), out_ids, out_d);
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("kNN launch");
    // the scratch is reused by the next call: finish here
    if (hipStreamSynchronize(ctx->stream) != hipSuccess) return ctx->fail_hip("kNN synchronize");
    return GOFANN_OK;
}

}  // namespace

int build_kmeanspp(Context* ctx, const void* rows, int elem, uint32_t dim, uint64_t n, uint32_t k,
                   uint64_t seed, float* centres)
{
    if (int rc = check_elem(ctx, elem)) return rc;
    if (!rows || !centres || dim == 0 || n == 0 || k == 0)
        return ctx->fail(GOFANN_ERR_INVALID, "k-means++: arrays missing or empty");
    if (n > 0xFFFFFFFFull) return ctx->fail(GOFANN_ERR_INVALID, "k-means++: at most 2^32 - 1 rows");
    switch (elem) {
        case GOFANN_ELEM_U8: return kmeanspp_t(ctx, static_cast<const uint8_t*>(rows), dim, n, k, seed, centres);
        case GOFANN_ELEM_F16: return kmeanspp_t(ctx, static_cast<const _Float16*>(rows), dim, n, k, seed, centres);
        default: return kmeanspp_t(ctx, static_cast<const float*>(rows), dim, n, k, seed, centres);
    }
}

int build_kmeans(Context* ctx, const void* rows, int elem, uint32_t dim, uint64_t n, uint32_t k,
                 uint32_t iters, float* centres)
{
    if (int rc = check_elem(ctx, elem)) return rc;
    if (!rows || !centres || dim == 0 || n == 0 || k == 0)
        return ctx->fail(GOFANN_ERR_INVALID, "k-means: arrays missing or empty");
    if (n > 0x7FFFFFFFull) return ctx->fail(GOFANN_ERR_INVALID, "k-means: at most 2^31 - 1 rows");
    switch (elem) {
        case GOFANN_ELEM_U8: return kmeans_t(ctx, static_cast<const uint8_t*>(rows), dim, n, k, iters, centres);
        case GOFANN_ELEM_F16: return kmeans_t(ctx, static_cast<const _Float16*>(rows), dim, n, k, iters, centres);
        default: return kmeans_t(ctx, static_cast<const float*>(rows), dim, n, k, iters, centres);
    }
}

int build_knn(Context* ctx, const void* rows, int elem, uint32_t dim,
              const gofann_build_buckets* b, uint32_t k, uint32_t* out_ids, float* out_dists)
{
    if (int rc = check_elem(ctx, elem)) return rc;
    if (!b || !b->bucket_offsets || !rows || !out_ids || dim == 0)
        return ctx->fail(GOFANN_ERR_INVALID, "kNN: arrays missing");
    if (k == 0 || k > kMaxKnn) return ctx->fail(GOFANN_ERR_UNSUPPORTED, "kNN: k must be 1..128");
    if ((b->probe_offsets == nullptr) != (b->probe_buckets == nullptr))
        return ctx->fail(GOFANN_ERR_INVALID, "kNN: probe offsets and buckets go together");
    if (b->buckets == 0 || b->rows == 0) return GOFANN_OK;
    switch (elem) {
        case GOFANN_ELEM_U8: return knn_t(ctx, static_cast<const uint8_t*>(rows), dim, b, k, out_ids, out_dists);
        case GOFANN_ELEM_F16: return knn_t(ctx, static_cast<const _Float16*>(rows), dim, b, k, out_ids, out_dists);
        default: return knn_t(ctx, static_cast<const float*>(rows), dim, b, k, out_ids, out_dists);
    }
}

namespace {
template <class T, int S>
int pq_encode_launch(Context* ctx, const T* rows, uint32_t dim, uint64_t n, uint32_t pq_dim,
                     const float* centroids, uint8_t* codes, uint32_t code_stride)
{
    const size_t lds = 256ull * (dim / pq_dim) * 4;
    const dim3 grid(static_cast<uint32_t>((n + kThreads - 1) / kThreads), pq_dim);
    const void* kern = reinterpret_cast<const void*>(pq_assign_kernel<T, S>);
    if (hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)) !=
        hipSuccess)
        return ctx->fail_hip("hipFuncSetAttribute PQ assign");
    hipLaunchKernelGGL((pq_assign_kernel<T, S>), grid, dim3(kThreads), lds, ctx->stream, rows, dim, n,
                       pq_dim, centroids, codes, code_stride);
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("PQ encode launch");
    return GOFANN_OK;
}

template <class T>
int pq_encode_t(Context* ctx, const T* rows, uint32_t dim, uint64_t n, uint32_t pq_dim,
                const float* centroids, uint8_t* codes, uint32_t code_stride)
{
    switch (dim / pq_dim) {
        case 2: return pq_encode_launch<T, 2>(ctx, rows, dim, n, pq_dim, centroids, codes, code_stride);
        case 4: return pq_encode_launch<T, 4>(ctx, rows, dim, n, pq_dim, centroids, codes, code_stride);
        case 8: return pq_encode_launch<T, 8>(ctx, rows, dim, n, pq_dim, centroids, codes, code_stride);
        case 16: return pq_encode_launch<T, 16>(ctx, rows, dim, n, pq_dim, centroids, codes, code_stride);
        default: return pq_encode_launch<T, 0>(ctx, rows, dim, n, pq_dim, centroids, codes, code_stride);
    }
}
}  // namespace

int build_pq_encode(Context* ctx, const void* rows, int elem, uint32_t dim, uint64_t n,
                    uint32_t pq_dim, const float* centroids, uint8_t* codes, uint32_t code_stride)
{
    if (int rc = check_elem(ctx, elem)) return rc;
    if (!rows || !centroids || !codes || pq_dim == 0 || dim % pq_dim != 0 || code_stride < pq_dim)
        return ctx->fail(GOFANN_ERR_INVALID, "PQ encode: invalid arrays or dims");
    if (dim / pq_dim > 256) return ctx->fail(GOFANN_ERR_UNSUPPORTED, "PQ encode: at most 256 dims per subspace");
    if (n == 0) return GOFANN_OK;
    if (n / kThreads >= 0x7FFFFFFFull || pq_dim > 65535)
        return ctx->fail(GOFANN_ERR_INVALID, "PQ encode: too many rows or subspaces");
    switch (elem) {
        case GOFANN_ELEM_U8:
            return pq_encode_t(ctx, static_cast<const uint8_t*>(rows), dim, n, pq_dim, centroids, codes, code_stride);
        case GOFANN_ELEM_F16:
            return pq_encode_t(ctx, static_cast<const _Float16*>(rows), dim, n, pq_dim, centroids, codes, code_stride);
        default:
            return pq_encode_t(ctx, static_cast<const float*>(rows), dim, n, pq_dim, centroids, codes, code_stride);
    }
}

namespace {
template <class T>
int pq_train_t(Context* ctx, const T* rows, uint32_t dim, uint64_t n, uint32_t pq_dim, uint32_t iters,
               float* centroids, int elem)
{
    const uint64_t pairs = n * pq_dim;
    const uint32_t nkeys = pq_dim * 256u;
    unsigned char* buf = static_cast<unsigned char*>(ctx->scratch(
        Context::kScratchBuild,
        carve_size({pairs, pairs * 4, (nkeys + 1ull) * 4, (nkeys + 1ull) * 4})));
    if (!buf) return ctx->fail(GOFANN_ERR_NOMEM, "PQ training scratch allocation failed");
    Carve cv{buf, 0};
    uint8_t* codes = cv.take<uint8_t>(pairs);
    uint32_t* order = cv.take<uint32_t>(pairs);
    uint32_t* counts = cv.take<uint32_t>(nkeys + 1ull);
    uint32_t* start = cv.take<uint32_t>(nkeys + 1ull);
    for (uint32_t it = 0; it < iters; ++it) {
        if (int rc = build_pq_encode(ctx, rows, elem, dim, n, pq_dim, centroids, codes, pq_dim)) return rc;
        // the rows of each (subspace, centre) in ascending order
        if (hipMemsetAsync(counts, 0, (nkeys + 1ull) * 4, ctx->stream) != hipSuccess)
            return ctx->fail_hip("PQ counts clear");
        hipLaunchKernelGGL(pq_key_count_kernel, dim3(static_cast<uint32_t>((pairs + 255) / 256)), dim3(256),
                           0, ctx->stream, codes, n, pq_dim, counts);
        hipLaunchKernelGGL(exclusive_scan_kernel, dim3(1), dim3(1024), 0, ctx->stream, counts,
                           static_cast<uint64_t>(nkeys), start);
        hipLaunchKernelGGL(pq_key_lists_kernel, dim3((nkeys + 3) / 4), dim3(kThreads), 0, ctx->stream,
                           codes, n, pq_dim, start, order);
        hipLaunchKernelGGL(pq_mean_kernel<T>, dim3(nkeys), dim3(64), 0, ctx->stream, rows, dim, n,
                           pq_dim, order, start, centroids);
    }
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("PQ training launch");
    return GOFANN_OK;
}
}  // namespace

int build_pq_train(Context* ctx, const void* rows, int elem, uint32_t dim, uint64_t n,
                   uint32_t pq_dim, uint32_t iters, float* centroids)
{
    if (int rc = check_elem(ctx, elem)) return rc;
    if (!rows || !centroids || pq_dim == 0 || dim % pq_dim != 0)
        return ctx->fail(GOFANN_ERR_INVALID, "PQ training: invalid arrays or dims");
    if (n == 0 || iters == 0) return GOFANN_OK;
    if (n * pq_dim > 0x7FFFFFFFull) return ctx->fail(GOFANN_ERR_INVALID, "PQ training: too many rows");
    switch (elem) {
        case GOFANN_ELEM_U8: return pq_train_t(ctx, static_cast<const uint8_t*>(rows), dim, n, pq_dim, iters, centroids, elem);
        case GOFANN_ELEM_F16: return pq_train_t(ctx, static_cast<const _Float16*>(rows), dim, n, pq_dim, iters, centroids, elem);
        default: return pq_train_t(ctx, static_cast<const float*>(rows), dim, n, pq_dim, iters, centroids, elem);
    }
}

int build_rotate(Context* ctx, const void* rows, int elem, uint32_t dim, uint32_t n,
                 const float* rotation, uint32_t padded_dim, float* out)
{
    if (int rc = check_elem(ctx, elem)) return rc;
    if (!rows || !rotation || !out || dim == 0 || padded_dim < dim)
        return ctx->fail(GOFANN_ERR_INVALID, "rotate: invalid arrays or dims");
    if (n == 0) return GOFANN_OK;
    const float* x = static_cast<const float*>(rows);
    if (elem != GOFANN_ELEM_F32) {
        const uint64_t count = static_cast<uint64_t>(n) * dim;
        float* f = static_cast<float*>(ctx->scratch(Context::kScratchBuild, count * 4));
        if (!f) return ctx->fail(GOFANN_ERR_NOMEM, "rotate scratch allocation failed");
        const dim3 g(static_cast<uint32_t>((count + 255) / 256));
        if (elem == GOFANN_ELEM_U8)
            hipLaunchKernelGGL(to_f32_kernel<uint8_t>, g, dim3(256), 0, ctx->stream,
                               static_cast<const uint8_t*>(rows), count, f);
        else
            hipLaunchKernelGGL(to_f32_kernel<_Float16>, g, dim3(256), 0, ctx->stream,
                               static_cast<const _Float16*>(rows), count, f);
        if (hipGetLastError() != hipSuccess) return ctx->fail_hip("rotate convert launch");
        x = f;
    }
    rocblas_handle h = blas_handle(ctx);
    if (!h) return ctx->fail(GOFANN_ERR_HIP, "rocBLAS handle");
    const float one = 1.0f, zero = 0.0f;
    // out[n][P] = x[n][D] R[D][P]; column-major: out^T = R^T x^T
    if (rocblas_sgemm(h, rocblas_operation_none, rocblas_operation_none, static_cast<int>(padded_dim),
                      static_cast<int>(n), static_cast<int>(dim), &one, rotation,
                      static_cast<int>(padded_dim), x, static_cast<int>(dim), &zero, out,
                      static_cast<int>(padded_dim)) != rocblas_status_success)
        return ctx->fail(GOFANN_ERR_HIP, "rocblas_sgemm (base rotation)");
    // the conversion scratch is reused by the next call: finish here
    if (elem != GOFANN_ELEM_F32 && hipStreamSynchronize(ctx->stream) != hipSuccess)
        return ctx->fail_hip("rotate synchronize");
    return GOFANN_OK;
}

int build_rabitq_encode(Context* ctx, const float* rotated, uint32_t n, uint32_t padded_dim,
                        const float* anchors, uint32_t num_anchors, uint32_t* anchor_ids,
                        uint8_t* codes, float* factors)
{
    if (!rotated || !anchors || !anchor_ids || !codes || !factors || num_anchors == 0)
        return ctx->fail(GOFANN_ERR_INVALID, "RaBitQ encode: arrays missing");
    if (padded_dim == 0 || padded_dim % 64 != 0)
        return ctx->fail(GOFANN_ERR_INVALID, "RaBitQ encode: padded_dim must be a multiple of 64");
    if (reinterpret_cast<uintptr_t>(codes) & 3u)
        return ctx->fail(GOFANN_ERR_INVALID, "RaBitQ encode: codes must be 4-byte aligned");
    if (n == 0) return GOFANN_OK;
    if (int rc = build_assign(ctx, rotated, GOFANN_ELEM_F32, padded_dim, n, anchors, num_anchors,
                              anchor_ids, nullptr))
        return rc;
    hipLaunchKernelGGL(rabitq_encode_kernel, dim3((n + 3) / 4), dim3(kThreads), 0, ctx->stream, rotated,
                       static_cast<uint64_t>(n), padded_dim, anchors, num_anchors, anchor_ids,
                       reinterpret_cast<uint32_t*>(codes), factors);
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("RaBitQ encode launch");
    return GOFANN_OK;
}

int build_medoid(Context* ctx, const void* rows, int elem, uint32_t dim, uint64_t n, uint32_t* out)
{
    if (int rc = check_elem(ctx, elem)) return rc;
    if (!rows || !out || dim == 0 || n == 0)
        return ctx->fail(GOFANN_ERR_INVALID, "medoid: arrays missing or empty");
    const uint64_t cblocks = (n + kColBlock - 1) / kColBlock;
    const uint64_t ablocks = (n + kThreads - 1) / kThreads;
    unsigned char* buf = static_cast<unsigned char*>(ctx->scratch(
        Context::kScratchBuild,
        carve_size({cblocks * dim * 8, dim * 8ull, n * 8, ablocks * 8, ablocks * 8, 16})));
    if (!buf) return ctx->fail(GOFANN_ERR_NOMEM, "medoid scratch allocation failed");
    Carve cv{buf, 0};
    double* partial = cv.take<double>(cblocks * dim);
    double* mean = cv.take<double>(dim);
    double* dist = cv.take<double>(n);
    double* bd = cv.take<double>(ablocks);
    uint64_t* bi = cv.take<uint64_t>(ablocks);
    uint32_t* res = cv.take<uint32_t>(4);
    const dim3 cg(static_cast<uint32_t>(cblocks));
    const dim3 rg(static_cast<uint32_t>((n + 255) / 256));
    switch (elem) {
        case GOFANN_ELEM_U8:
            hipLaunchKernelGGL(col_partial_kernel<uint8_t>, cg, dim3(kThreads), 0, ctx->stream,
                               static_cast<const uint8_t*>(rows), dim, n, partial);
            break;
        case GOFANN_ELEM_F16:
            hipLaunchKernelGGL(col_partial_kernel<_Float16>, cg, dim3(kThreads), 0, ctx->stream,
                               static_cast<const _Float16*>(rows), dim, n, partial);
            break;
        default:
            hipLaunchKernelGGL(col_partial_kernel<float>, cg, dim3(kThreads), 0, ctx->stream,
                               static_cast<const float*>(rows), dim, n, partial);
    }
    hipLaunchKernelGGL(col_mean_kernel, dim3((dim + 255) / 256), dim3(256), 0, ctx->stream, partial, dim,
                       cblocks, n, mean);
    switch (elem) {
        case GOFANN_ELEM_U8:
            hipLaunchKernelGGL(mean_dist_kernel<uint8_t>, rg, dim3(256), 0, ctx->stream,
                               static_cast<const uint8_t*>(rows), dim, n, mean, dist);
            break;
        case GOFANN_ELEM_F16:
            hipLaunchKernelGGL(mean_dist_kernel<_Float16>, rg, dim3(256), 0, ctx->stream,
                               static_cast<const _Float16*>(rows), dim, n, mean, dist);
            break;
        default:
            hipLaunchKernelGGL(mean_dist_kernel<float>, rg, dim3(256), 0, ctx->stream,
                               static_cast<const float*>(rows), dim, n, mean, dist);
    }
    hipLaunchKernelGGL(argmin_block_kernel, dim3(static_cast<uint32_t>(ablocks)), dim3(kThreads), 0,
                       ctx->stream, dist, n, bd, bi);
    hipLaunchKernelGGL(argmin_final_kernel, dim3(1), dim3(kThreads), 0, ctx->stream, bd, bi, ablocks, res);
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("medoid launch");
    if (hipMemcpyAsync(out, res, 4, hipMemcpyDeviceToHost, ctx->stream) != hipSuccess ||
        hipStreamSynchronize(ctx->stream) != hipSuccess)
        return ctx->fail_hip("medoid result copy");
    return GOFANN_OK;
}

int build_bucket_reps(Context* ctx, const void* rows, int elem, uint32_t dim,
                      const uint32_t* bucket_offsets, uint32_t buckets, float* means, uint32_t* reps)
{
    if (int rc = check_elem(ctx, elem)) return rc;
    if (!rows || !bucket_offsets || !means || !reps || dim == 0)
        return ctx->fail(GOFANN_ERR_INVALID, "bucket representatives: arrays missing");
    if (buckets == 0) return GOFANN_OK;
    {
        std::vector<uint32_t> off(buckets + 1ull);
        if (hipMemcpyAsync(off.data(), bucket_offsets, off.size() * 4, hipMemcpyDeviceToHost,
                           ctx->stream) != hipSuccess ||
            hipStreamSynchronize(ctx->stream) != hipSuccess)
            return ctx->fail_hip("bucket offsets copy");
        for (uint32_t i = 0; i < buckets; ++i)
            if (off[i] > off[i + 1])
                return ctx->fail(GOFANN_ERR_INVALID, "bucket representatives: offsets decrease");
    }
    switch (elem) {
        case GOFANN_ELEM_U8:
            hipLaunchKernelGGL(bucket_rep_kernel<uint8_t>, dim3(buckets), dim3(kThreads), 0, ctx->stream,
                               static_cast<const uint8_t*>(rows), dim, bucket_offsets, means, reps);
            break;
        case GOFANN_ELEM_F16:
            hipLaunchKernelGGL(bucket_rep_kernel<_Float16>, dim3(buckets), dim3(kThreads), 0, ctx->stream,
                               static_cast<const _Float16*>(rows), dim, bucket_offsets, means, reps);
            break;
        default:
            hipLaunchKernelGGL(bucket_rep_kernel<float>, dim3(buckets), dim3(kThreads), 0, ctx->stream,
                               static_cast<const float*>(rows), dim, bucket_offsets, means, reps);
    }
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("bucket representative launch");
    return GOFANN_OK;
}

int build_links(Context* ctx, const gofann_build_link_inputs* in, const gofann_build_link_params* p,
                uint32_t* out_graph)
{
    if (!in || !p || !out_graph || !in->bucket_of || !in->reps || !in->order)
        return ctx->fail(GOFANN_ERR_INVALID, "links: arrays missing");
    if (p->degree == 0 || p->degree > 256) return ctx->fail(GOFANN_ERR_UNSUPPORTED, "links: degree must be 1..256");
    const uint32_t nk = p->local > p->rep_local ? p->local : p->rep_local;
    const uint32_t nn = p->near_links > p->rep_near ? p->near_links : p->rep_near;
    if ((nk > 0 && !in->knn) || nk > in->knn_width)
        return ctx->fail(GOFANN_ERR_INVALID, "links: local links exceed the kNN width");
    if ((nn > 0 && !in->near_buckets) || nn > in->near_width)
        return ctx->fail(GOFANN_ERR_INVALID, "links: near links exceed the near-bucket width");
    if (nk + 1 + nn + p->degree > static_cast<uint32_t>(kLinkCand) || 4 * p->degree > static_cast<uint32_t>(kLinkCand))
        return ctx->fail(GOFANN_ERR_UNSUPPORTED, "links: more than 512 candidates per row");
    if (in->rows == 0) return GOFANN_OK;
    LinkArgs a{};
    a.n = in->rows;
    a.knn = in->knn;
    a.knn_width = in->knn_width;
    a.bucket_of = in->bucket_of;
    a.rep = in->reps;
    a.near = in->near_buckets;
    a.near_width = in->near_width;
    a.buckets = in->buckets;
    a.order = in->order;
    a.degree = p->degree;
    a.local = p->local;
    a.near_links = p->near_links;
    a.rep_local = p->rep_local;
    a.rep_near = p->rep_near;
    a.entry = p->entry_row;
    a.seed = p->seed;
    a.out = out_graph;
    hipLaunchKernelGGL(links_kernel, dim3((in->rows + 3) / 4), dim3(kThreads), 0, ctx->stream, a);
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("links launch");
    return GOFANN_OK;
}

int build_cagra_optimize(Context* ctx, const uint32_t* knn, uint32_t n, uint32_t kin, uint32_t degree,
                         uint32_t* pruned, uint32_t* out_graph)
{
    if (!knn || !pruned || !out_graph) return ctx->fail(GOFANN_ERR_INVALID, "CAGRA optimise: arrays missing");
    if (kin == 0 || kin > static_cast<uint32_t>(kMaxKnn) || degree == 0 || degree > kin || degree > 127)
        return ctx->fail(GOFANN_ERR_UNSUPPORTED, "CAGRA optimise: needs 0 < degree <= kin <= 128, degree < 128");
    if (n >= (1u << 27)) return ctx->fail(GOFANN_ERR_UNSUPPORTED, "CAGRA optimise: at most 2^27 - 1 rows");
    if (n == 0) return GOFANN_OK;
    hipLaunchKernelGGL(cagra_prune_kernel, dim3((n + 3) / 4), dim3(kThreads), 0, ctx->stream, knn, n, kin,
                       degree, pruned);
    const uint64_t edges = static_cast<uint64_t>(n) * degree;
    unsigned char* buf = static_cast<unsigned char*>(ctx->scratch(
        Context::kScratchBuild, carve_size({edges * 8, (n + 1ull) * 4, (n + 1ull) * 4, (n + 1ull) * 4})));
    if (!buf) return ctx->fail(GOFANN_ERR_NOMEM, "CAGRA optimise scratch allocation failed");
    Carve cv{buf, 0};
    uint64_t* rkeys = cv.take<uint64_t>(edges);
    uint32_t* counts = cv.take<uint32_t>(n + 1ull);
    uint32_t* rstart = cv.take<uint32_t>(n + 1ull);
    uint32_t* fill = cv.take<uint32_t>(n + 1ull);
    if (hipMemsetAsync(counts, 0, (n + 1ull) * 4, ctx->stream) != hipSuccess ||
        hipMemsetAsync(fill, 0, (n + 1ull) * 4, ctx->stream) != hipSuccess)
        return ctx->fail_hip("reverse counts clear");
    const dim3 eg(static_cast<uint32_t>((edges + 255) / 256));
    hipLaunchKernelGGL(reverse_count_kernel, eg, dim3(256), 0, ctx->stream, pruned, n, degree, counts);
    hipLaunchKernelGGL(exclusive_scan_kernel, dim3(1), dim3(1024), 0, ctx->stream, counts,
                       static_cast<uint64_t>(n), rstart);
    hipLaunchKernelGGL(reverse_fill_kernel, eg, dim3(256), 0, ctx->stream, pruned, n, degree, rstart, fill,
                       rkeys);
    hipLaunchKernelGGL(reverse_merge_kernel, dim3((n + 255) / 256), dim3(256), 0, ctx->stream, pruned, rkeys,
                       rstart, n, degree, out_graph);
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("CAGRA optimise launch");
    if (hipStreamSynchronize(ctx->stream) != hipSuccess) return ctx->fail_hip("CAGRA optimise synchronize");
    return GOFANN_OK;
}

int build_reach(Context* ctx, const uint32_t* graph, uint32_t n, uint32_t degree, uint32_t entry,
                uint32_t* reached, uint32_t* out_count)
{
    if (!graph || !reached || !out_count) return ctx->fail(GOFANN_ERR_INVALID, "reach: arrays missing");
    if (entry >= n) return ctx->fail(GOFANN_ERR_INVALID, "reach: entry row out of range");
    unsigned char* buf = static_cast<unsigned char*>(
        ctx->scratch(Context::kScratchBuild, carve_size({n * 4ull, n * 4ull, 16})));
    if (!buf) return ctx->fail(GOFANN_ERR_NOMEM, "reach scratch allocation failed");
    Carve cv{buf, 0};
    uint32_t* fa = cv.take<uint32_t>(n);
    uint32_t* fb = cv.take<uint32_t>(n);
    uint32_t* cnt = cv.take<uint32_t>(4);
    if (hipMemsetAsync(reached, 0, n * 4ull, ctx->stream) != hipSuccess) return ctx->fail_hip("reach clear");
    hipLaunchKernelGGL(bfs_seed_kernel, dim3(1), dim3(1), 0, ctx->stream, entry, reached, fa);
    uint32_t count = 1, total = 1;
    while (count > 0) {
        if (hipMemsetAsync(cnt, 0, 4, ctx->stream) != hipSuccess) return ctx->fail_hip("reach count clear");
        const uint64_t work = static_cast<uint64_t>(count) * degree;
        hipLaunchKernelGGL(bfs_level_kernel, dim3(static_cast<uint32_t>((work + 255) / 256)), dim3(256), 0,
                           ctx->stream, graph, n, degree, fa, count, reached, fb, cnt);
        if (hipGetLastError() != hipSuccess) return ctx->fail_hip("reach launch");
        if (hipMemcpyAsync(&count, cnt, 4, hipMemcpyDeviceToHost, ctx->stream) != hipSuccess ||
            hipStreamSynchronize(ctx->stream) != hipSuccess)
            return ctx->fail_hip("reach count");
        total += count;
        uint32_t* t = fa;
        fa = fb;
        fb = t;
    }
    *out_count = total;
    return GOFANN_OK;
}

}  // namespace gofann
