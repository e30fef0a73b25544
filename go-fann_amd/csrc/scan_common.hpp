// scan_common.hpp -- pieces shared by the posting-scan kernels: the
// (distance, id) order of posting_shortlist_heap (src/search/common/
// posting_shortlist_heap.cuh:14-21), an LDS bitonic sort on that order, and
// the per-thread PQ / RaBitQ candidate scorers.
#pragma once

#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>

#include "device_common.hpp"

namespace gofann {

constexpr int kScanThreads = 256;
constexpr int kScanSlots = 2048;       // LDS pairs: running top-k + chunk
constexpr int kMaxShortlist = 512;

__device__ __forceinline__ bool admissible(float d, uint32_t id)
{
    return id != UINT32_MAX && d <= FLT_MAX;
}

// (distance, id) ascending; (FLT_MAX, UINT32_MAX) pads sort last.
__device__ __forceinline__ bool pair_less(float ad, uint32_t aid, float bd, uint32_t bid)
{
    return ad < bd || (ad == bd && aid < bid);
}

__device__ inline void bitonic_sort(float* d, uint32_t* id, int n, int tid, int nthreads)
{
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = tid; i < n / 2; i += nthreads) {
                const int lo = 2 * i - (i & (stride - 1));
                const int hi = lo + stride;
                const bool ascending = (lo & size) == 0;
                const bool swap = ascending ? pair_less(d[hi], id[hi], d[lo], id[lo])
                                            : pair_less(d[lo], id[lo], d[hi], id[hi]);
                if (swap) {
                    const float td = d[lo];
                    d[lo] = d[hi];
                    d[hi] = td;
                    const uint32_t ti = id[lo];
                    id[lo] = id[hi];
                    id[hi] = ti;
                }
            }
            __syncthreads();
        }
    }
}

// Serial-order ADC of the posting scan (backend_pq.cu:2102-2106).
__device__ __forceinline__ float adc_serial(const float* lut, const uint8_t* row, int M)
{
    float dist = 0.0f;
    if (M % 16 == 0) {
        for (int m0 = 0; m0 < M; m0 += 16) {
            const uint4 w = *reinterpret_cast<const uint4*>(row + m0);
            const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int t = 0; t < 16; ++t)
                dist += lut[(m0 + t) * 256 + ((ws[t >> 2] >> (8 * (t & 3))) & 0xffu)];
        }
    } else {
        for (int m = 0; m < M; ++m) dist += lut[m * 256 + row[m]];
    }
    return dist;
}

struct PqScanScorer {
    const uint8_t* codes;
    const float* centroids;
    const void* queries;
    int query_f32;
    uint32_t dim;
    uint32_t pq_dim;
    uint32_t stride;  // bytes between code rows
    float* lut;

    __device__ void setup(uint32_t q, int tid, unsigned char* lds)
    {
        lut = reinterpret_cast<float*>(lds);
        const int M = static_cast<int>(pq_dim);
        const int sub = static_cast<int>(dim) / M;
        const float* qf = static_cast<const float*>(queries) + static_cast<size_t>(q) * dim;
        const uint8_t* qu = static_cast<const uint8_t*>(queries) + static_cast<size_t>(q) * dim;
        for (int e = tid; e < M * 256; e += kScanThreads) {
            const int mm = e >> 8, k = e & 255;
            const float* crow = centroids + static_cast<size_t>(k) * dim;
            float acc = 0.0f;
            for (int t = 0; t < sub; ++t) {
                const int d = mm * sub + t;
                const float qv = query_f32 ? qf[d] : static_cast<float>(qu[d]);
                const float diff = qv - crow[d];
                acc = fmaf(diff, diff, acc);
            }
            lut[e] = acc;
        }
    }
    __device__ float score(uint32_t sample) const
    {
        return adc_serial(lut, codes + static_cast<size_t>(sample) * stride, static_cast<int>(pq_dim));
    }
};

struct RabitqScanScorer {
    const uint8_t* codes;
    const float* factors;
    const uint32_t* anchor_ids;
    const int8_t* q8;
    const float* q_scale;
    const float* q_k1;
    const float* centroid_dists;
    uint32_t num_anchors;
    uint32_t padded_dim;
    uint32_t* planes;
    float scale, k1;
    const float* g_row;

    __device__ void setup(uint32_t q, int tid, unsigned char* lds)
    {
        planes = reinterpret_cast<uint32_t*>(lds);
        const uint32_t words = padded_dim / 32;
        const int8_t* qrow = q8 + static_cast<size_t>(q) * padded_dim;
        for (uint32_t w = tid; w < words; w += kScanThreads) {
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
    __device__ float score(uint32_t sample) const
    {
        const uint32_t words = padded_dim / 32;
        const uint4* row =
            reinterpret_cast<const uint4*>(codes + static_cast<size_t>(sample) * (padded_dim / 8));
        uint32_t cnt[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        // Code loads go out kCodeBatch at a time before any is consumed, so
        // a row costs ceil(vectors / kCodeBatch) memory round trips, not one
        // per 16 bytes.
        const uint32_t vecs = words / 4;
        for (uint32_t v0 = 0; v0 < vecs; v0 += kCodeBatch) {
            uint4 cb[kCodeBatch];
#pragma unroll
            for (int b = 0; b < kCodeBatch; ++b)
                cb[b] = v0 + b < vecs ? row[v0 + b] : make_uint4(0, 0, 0, 0);
#pragma unroll
            for (int b = 0; b < kCodeBatch; ++b) {
                if (v0 + b >= vecs) break;
                const uint32_t w4 = v0 + b;
                const uint32_t cw[4] = {cb[b].x, cb[b].y, cb[b].z, cb[b].w};
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const uint4 p0 = reinterpret_cast<const uint4*>(planes)[(w4 * 4 + t) * 2];
                    const uint4 p1 = reinterpret_cast<const uint4*>(planes)[(w4 * 4 + t) * 2 + 1];
                    cnt[0] = bcnt_acc(p0.x & cw[t], cnt[0]);
                    cnt[1] = bcnt_acc(p0.y & cw[t], cnt[1]);
                    cnt[2] = bcnt_acc(p0.z & cw[t], cnt[2]);
                    cnt[3] = bcnt_acc(p0.w & cw[t], cnt[3]);
                    cnt[4] = bcnt_acc(p1.x & cw[t], cnt[4]);
                    cnt[5] = bcnt_acc(p1.y & cw[t], cnt[5]);
                    cnt[6] = bcnt_acc(p1.z & cw[t], cnt[6]);
                    cnt[7] = bcnt_acc(p1.w & cw[t], cnt[7]);
                }
            }
        }
        int32_t ip = 0;
#pragma unroll
        for (int j = 0; j < 7; ++j) ip += static_cast<int32_t>(cnt[j]) << j;
        ip -= 128 * static_cast<int32_t>(cnt[7]);
        const uint32_t anchor = anchor_ids[sample];
        const float short_ip = static_cast<float>(ip) * scale;
        const float t = short_ip + k1;
        return fmaf(factors[static_cast<size_t>(sample) * 3 + 1], t,
                    factors[static_cast<size_t>(sample) * 3] + g_row[anchor]);
    }
};

}  // namespace gofann
