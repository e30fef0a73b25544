// exact_dist.hpp -- exact squared L2 of u8 / f32 / f16 rows against a query
// held in LDS as f32, in the two summation orders of the reference's
// full-GPU backend:
//
//  * warp order (l2_distance_device, src/search/full_gpu/
//    backend_full_gpu.cu:1107-1160; the graph route and the low-frequency
//    group scan :2124-2262): 32 partial sums, partial j a fused
//    multiply-add chain over the elements j, j + 32, ... (f16 rows of even
//    dim: over the element pairs j, j + 32, ..., each pair adding
//    fma(dx, dx, dy * dy)), then the shfl_down halving tree (j, j + 16),
//    (j, j + 8), ... whose result is partial 0.  Here one 32-lane half of a
//    wave computes one row: lane j of the half owns partial j, and an xor
//    butterfly over 16, 8, 4, 2, 1 leaves in the half's first lane the same
//    sums the reference's shfl_down tree leaves in lane 0 (each level adds
//    the same two operands; addition commutes exactly).
//  * serial order (full_gpu_range_posting_kernel :1443-1469): one chain
//    over d ascending (f16 even dim: dist + fma(dx, dx, dy * dy) per pair);
//    one thread computes one row.
//
// diff = base - query.  u8 rows in the warp order are the integer sum (the
// dp4a form :1199-1244), exact in any order; in the serial order they are
// converted to float first (T = uint8_t there).  The grouping of
// dx * dx + dy * dy is left to nvcc's contraction by the reference; the one
// fixed here is the expression's own (the products' pair fused, the running
// sum added after).  Every kernel including this header is compiled with
// -ffp-contract=off, so no other operation fuses.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstdint>

#include "device_common.hpp"

namespace gofann {

template <int kElem>
__device__ __forceinline__ float elem_to_float(const void* v, uint32_t i)
{
    if constexpr (kElem == GOFANN_ELEM_F32)
        return static_cast<const float*>(v)[i];
    else if constexpr (kElem == GOFANN_ELEM_F16)
        return __half2float(static_cast<const __half*>(v)[i]);
    else
        return static_cast<float>(static_cast<const uint8_t*>(v)[i]);
}

constexpr uint32_t elem_bytes(int elem)
{
    return elem == GOFANN_ELEM_F32 ? 4u : (elem == GOFANN_ELEM_F16 ? 2u : 1u);
}

// Warp order, lane j (0..31) of the half computing `row`: partial j.
// kBatch row words per lane are loaded before the first is consumed, so a
// row costs about dim / (32 kBatch) memory round trips; the chain of sums
// keeps its order whatever kBatch is.
template <int kElem, int kBatch = 8>
__device__ __forceinline__ float l2_w32_partial(const void* row, const float* q, uint32_t dim,
                                                uint32_t j)
{
    float p = 0.0f;
    if constexpr (kElem == GOFANN_ELEM_F32) {
        const float* b = static_cast<const float*>(row);
        uint32_t d = j;
        for (; d + 32u * (kBatch - 1) < dim; d += 32u * kBatch) {
            float v[kBatch];
#pragma unroll
            for (int t = 0; t < kBatch; ++t) v[t] = b[d + 32u * t];
#pragma unroll
            for (int t = 0; t < kBatch; ++t) {
                const float diff = v[t] - q[d + 32u * t];
                p = fmaf(diff, diff, p);
            }
        }
        for (; d < dim; d += 32) {
            const float diff = b[d] - q[d];
            p = fmaf(diff, diff, p);
        }
    } else if constexpr (kElem == GOFANN_ELEM_F16) {
        if ((dim & 1u) == 0) {
            const __half2* b2 = static_cast<const __half2*>(row);
            const float2* q2 = reinterpret_cast<const float2*>(q);
            const uint32_t dim2 = dim >> 1;
            uint32_t d2 = j;
            for (; d2 + 32u * (kBatch - 1) < dim2; d2 += 32u * kBatch) {
                __half2 v[kBatch];
#pragma unroll
                for (int t = 0; t < kBatch; ++t) v[t] = b2[d2 + 32u * t];
#pragma unroll
                for (int t = 0; t < kBatch; ++t) {
                    const float2 bf = __half22float2(v[t]);
                    const float2 qf = q2[d2 + 32u * t];
                    const float dx = bf.x - qf.x;
                    const float dy = bf.y - qf.y;
                    p = p + fmaf(dx, dx, dy * dy);
                }
            }
            for (; d2 < dim2; d2 += 32) {
                const float2 bf = __half22float2(b2[d2]);
                const float2 qf = q2[d2];
                const float dx = bf.x - qf.x;
                const float dy = bf.y - qf.y;
                p = p + fmaf(dx, dx, dy * dy);
            }
        } else {
            const __half* b = static_cast<const __half*>(row);
#pragma unroll 8
            for (uint32_t d = j; d < dim; d += 32) {
                const float diff = __half2float(b[d]) - q[d];
                p = fmaf(diff, diff, p);
            }
        }
    } else {
        // integer: the u32 partial travels in the float's bits and
        // w32_tree sums the partials as u32 (exact for dim <= 65536).
        const uint8_t* b = static_cast<const uint8_t*>(row);
        uint32_t acc = 0;
        for (uint32_t d = j; d < dim; d += 32) {
            const int diff = static_cast<int>(b[d]) - static_cast<int>(q[d]);
            acc += static_cast<uint32_t>(diff * diff);
        }
        p = __uint_as_float(acc);  // bits carried, summed as u32 below
    }
    return p;
}

// The halving tree over the 32 lanes of each half; the half's first lane
// holds the reference's result.  u8: partials carried as u32 bits.
template <int kElem>
__device__ __forceinline__ float w32_tree(float p)
{
    if constexpr (kElem == GOFANN_ELEM_U8) {
        uint32_t v = __float_as_uint(p);
#pragma unroll
        for (int off = 16; off > 0; off >>= 1)
            v += static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), off, 32));
        return static_cast<float>(v);
    } else {
#pragma unroll
        for (int off = 16; off > 0; off >>= 1) p = p + __shfl_xor(p, off, 32);
        return p;
    }
}

// ---- warp order, four lanes per row --------------------------------------
// The same 32 partials and the same tree, laid out for a quad of lanes
// (g = lane & 3) so that a wave scores 16 rows at once and each quad reads
// whole 128-byte lines: counting units (f32: elements; f16 rows of even dim:
// element pairs; u8: bytes), lane g owns partials 8g .. 8g + 7, i.e. units
// 8g + i of every 32-unit block.  The tree's first two levels pair lanes
// (j + 16: lane g ^ 2; j + 8: lane g ^ 1, by DPP quad permutes), the last
// three run inside lane 0 (i + 4, i + 2, i + 1).  Lane 0 of the quad ends
// with the reference's sum.  u8 partials are integers (any order).
__device__ __forceinline__ float quad_xor1(float v)
{
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));
}
__device__ __forceinline__ float quad_xor2(float v)
{
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true));
}
__device__ __forceinline__ uint32_t quad_xor1u(uint32_t v)
{
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0xB1, 0xF, 0xF, true));
}
__device__ __forceinline__ uint32_t quad_xor2u(uint32_t v)
{
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0x4E, 0xF, 0xF, true));
}

__device__ __forceinline__ float2 half2_bits_to_float2(uint32_t w)
{
    __half2 h;
    __builtin_memcpy(&h, &w, 4);
    return __half22float2(h);
}

// One quad, one row: the squared L2 in the warp order, valid in lane g == 0
// of the quad.  Every lane of the quad must be active.  kU: 128-byte blocks
// whose loads are issued together.
template <int kElem, int kU = 2>
__device__ __forceinline__ float l2_w32_quad(const uint8_t* row, const float* q, uint32_t dim,
                                             uint32_t g)
{
    if constexpr (kElem == GOFANN_ELEM_U8) {
        uint32_t acc = 0;
        const uint32_t nb = dim / 32;
        if ((dim & 7u) == 0) {
            for (uint32_t t = 0; t < nb; ++t) {
                const uint2 w = *reinterpret_cast<const uint2*>(row + 32u * t + 8u * g);
                const uint32_t d0 = 32u * t + 8u * g;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const uint32_t b = ((i < 4 ? w.x : w.y) >> (8 * (i & 3))) & 0xffu;
                    const int diff = static_cast<int>(b) - static_cast<int>(q[d0 + i]);
                    acc += static_cast<uint32_t>(diff * diff);
                }
            }
        } else {
            for (uint32_t t = 0; t < nb; ++t)
                for (uint32_t i = 0; i < 8; ++i) {
                    const uint32_t d = 32u * t + 8u * g + i;
                    const int diff = static_cast<int>(row[d]) - static_cast<int>(q[d]);
                    acc += static_cast<uint32_t>(diff * diff);
                }
        }
        for (uint32_t i = 0; i < 8; ++i) {
            const uint32_t d = 32u * nb + 8u * g + i;
            if (d < dim) {
                const int diff = static_cast<int>(row[d]) - static_cast<int>(q[d]);
                acc += static_cast<uint32_t>(diff * diff);
            }
        }
        acc += quad_xor2u(acc);
        acc += quad_xor1u(acc);
        return static_cast<float>(acc);
    } else {
        float p[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) p[i] = 0.0f;
        const bool pairs = kElem == GOFANN_ELEM_F16 && (dim & 1u) == 0;
        const uint32_t units = pairs ? dim / 2 : dim;
        const uint32_t nb = units / 32;
        // whole blocks by two 16-byte loads where the row allows it
        const bool vec = kElem == GOFANN_ELEM_F32 ? (dim & 3u) == 0 : (dim & 7u) == 0;
        if (vec) {
            // one 128-byte block: this lane's two 16-byte loads, summed in order
            const auto block = [&](uint32_t t, const uint4& a, const uint4& b) {
                const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
                const uint32_t k0 = 32u * t + 8u * g;
                if constexpr (kElem == GOFANN_ELEM_F32) {
                    const float4 q0 = *reinterpret_cast<const float4*>(q + k0);
                    const float4 q1 = *reinterpret_cast<const float4*>(q + k0 + 4);
                    const float qv[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const float diff = __uint_as_float(w[i]) - qv[i];
                        p[i] = fmaf(diff, diff, p[i]);
                    }
                } else {
                    const float4* q4 = reinterpret_cast<const float4*>(q + 2u * k0);
#pragma unroll
                    for (int i = 0; i < 8; i += 2) {
                        const float4 qq = q4[i / 2];
                        const float2 b0 = half2_bits_to_float2(w[i]);
                        const float2 b1 = half2_bits_to_float2(w[i + 1]);
                        float dx = b0.x - qq.x, dy = b0.y - qq.y;
                        p[i] = p[i] + fmaf(dx, dx, dy * dy);
                        dx = b1.x - qq.z;
                        dy = b1.y - qq.w;
                        p[i + 1] = p[i + 1] + fmaf(dx, dx, dy * dy);
                    }
                }
            };
            // kU blocks' loads are issued before the first of them is summed
            uint32_t t = 0;
            for (; t + kU <= nb; t += kU) {
                uint4 a[kU], b[kU];
#pragma unroll
                for (int u = 0; u < kU; ++u) {
                    const uint4* src = reinterpret_cast<const uint4*>(row + 128u * (t + u) + 32u * g);
                    a[u] = src[0];
                    b[u] = src[1];
                }
#pragma unroll
                for (int u = 0; u < kU; ++u) block(t + u, a[u], b[u]);
            }
            for (; t < nb; ++t) {
                const uint4* src = reinterpret_cast<const uint4*>(row + 128u * t + 32u * g);
                block(t, src[0], src[1]);
            }
        }
        // blocks not read above (the unaligned case), then the partial block
        for (uint32_t t = vec ? nb : 0; t <= nb; ++t) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t k = 32u * t + 8u * g + static_cast<uint32_t>(i);
                if (k >= units) continue;
                if (pairs) {
                    const float2 bf = half2_bits_to_float2(
                        *reinterpret_cast<const uint32_t*>(row + 4u * k));
                    const float dx = bf.x - q[2u * k];
                    const float dy = bf.y - q[2u * k + 1u];
                    p[i] = p[i] + fmaf(dx, dx, dy * dy);
                } else {
                    const float diff = elem_to_float<kElem>(row, k) - q[k];
                    p[i] = fmaf(diff, diff, p[i]);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) p[i] = p[i] + quad_xor2(p[i]);  // j + 16
#pragma unroll
        for (int i = 0; i < 8; ++i) p[i] = p[i] + quad_xor1(p[i]);  // j + 8
#pragma unroll
        for (int i = 0; i < 4; ++i) p[i] = p[i] + p[i + 4];
        p[0] = p[0] + p[2];
        p[1] = p[1] + p[3];
        return p[0] + p[1];
    }
}

// ---- serial order through an LDS tile ------------------------------------
// A wave scores 64 rows, one per lane, each lane's chain in d order, while
// the rows are read whole lines at a time: tile t of every row (kTileWords
// 4-byte words) is loaded by kTileWords / 4 lanes per row (16 bytes each)
// into a [64][kTileWords + 1] LDS tile (the odd stride keeps the per-row
// reads conflict-free), the next tile's loads are issued, and each lane
// then runs its row's words from LDS.  Needs row_bytes % 16 == 0 (so f16
// rows are of even dim and every word is one element pair).  ids: the
// rows' sample ids; rows <= 64; returns lane's sum (lanes >= rows: 0).
template <int kElem, int kTileWords>
__device__ __forceinline__ float l2_serial_tiled(const uint8_t* base, size_t row_bytes,
                                                 const float* q, const uint32_t* ids, int rows,
                                                 uint32_t* tile, int lane)
{
    constexpr int kLanesPerRow = kTileWords / 4;
    constexpr int kRowsPerLoad = 64 / kLanesPerRow;
    constexpr int kLoads = 64 / kRowsPerLoad;
    constexpr int kStride = kTileWords + 1;
    const uint32_t words = static_cast<uint32_t>(row_bytes / 4);
    const uint32_t ntiles = (words + kTileWords - 1) / kTileWords;
    const int col = (lane % kLanesPerRow) * 4;
    const uint8_t* src[kLoads];
#pragma unroll
    for (int k = 0; k < kLoads; ++k) {
        const int r = k * kRowsPerLoad + lane / kLanesPerRow;
        const uint32_t id = ids[r < rows ? r : rows - 1];  // rows >= 1
        src[k] = r < rows ? base + static_cast<size_t>(id) * row_bytes : nullptr;
    }
    uint4 buf[kLoads];
    auto load = [&](uint32_t t) {
        const uint32_t w0 = t * kTileWords + static_cast<uint32_t>(col);
#pragma unroll
        for (int k = 0; k < kLoads; ++k)
            buf[k] = (src[k] != nullptr && w0 < words)
                         ? *reinterpret_cast<const uint4*>(src[k] + 4u * w0)
                         : make_uint4(0, 0, 0, 0);
    };
    load(0);
    float acc = 0.0f;
    const uint32_t* mine = tile + lane * kStride;
    for (uint32_t t = 0; t < ntiles; ++t) {
#pragma unroll
        for (int k = 0; k < kLoads; ++k) {
            uint32_t* dst = tile + (k * kRowsPerLoad + lane / kLanesPerRow) * kStride + col;
            dst[0] = buf[k].x;
            dst[1] = buf[k].y;
            dst[2] = buf[k].z;
            dst[3] = buf[k].w;
        }
        __threadfence_block();
        if (t + 1 < ntiles) load(t + 1);
        const uint32_t w0 = t * kTileWords;
        const uint32_t nw = words - w0 < static_cast<uint32_t>(kTileWords) ? words - w0
                                                                            : kTileWords;
        if (lane < rows) {
            for (uint32_t w = 0; w < nw; ++w) {
                const uint32_t v = mine[w];
                const uint32_t k = w0 + w;  // word index in the row
                if constexpr (kElem == GOFANN_ELEM_F32) {
                    const float diff = __uint_as_float(v) - q[k];
                    acc = fmaf(diff, diff, acc);
                } else if constexpr (kElem == GOFANN_ELEM_F16) {
                    const float2 bf = half2_bits_to_float2(v);
                    const float dx = bf.x - q[2u * k];
                    const float dy = bf.y - q[2u * k + 1u];
                    acc = acc + fmaf(dx, dx, dy * dy);
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float diff = static_cast<float>((v >> (8 * i)) & 0xffu) - q[4u * k + i];
                        acc = fmaf(diff, diff, acc);
                    }
                }
            }
        }
        __threadfence_block();
    }
    return acc;
}

// Serial order: one thread, one row.  Rows whose byte length is a multiple
// of 16 (and so 16-byte aligned when the base is) are read 16 bytes at a
// time; the sum stays in d order either way.
template <int kElem>
__device__ __forceinline__ float l2_serial(const void* row, const float* q, uint32_t dim)
{
    float acc = 0.0f;
    const bool vec = ((dim * elem_bytes(kElem)) & 15u) == 0;
    if constexpr (kElem == GOFANN_ELEM_F32) {
        if (vec) {
            const float4* b4 = static_cast<const float4*>(row);
            const float4* q4 = reinterpret_cast<const float4*>(q);
            for (uint32_t i = 0; i < dim / 4; ++i) {
                const float4 b = b4[i];
                const float4 qq = q4[i];
                float t = b.x - qq.x;
                acc = fmaf(t, t, acc);
                t = b.y - qq.y;
                acc = fmaf(t, t, acc);
                t = b.z - qq.z;
                acc = fmaf(t, t, acc);
                t = b.w - qq.w;
                acc = fmaf(t, t, acc);
            }
            return acc;
        }
        const float* b = static_cast<const float*>(row);
        for (uint32_t d = 0; d < dim; ++d) {
            const float t = b[d] - q[d];
            acc = fmaf(t, t, acc);
        }
        return acc;
    } else if constexpr (kElem == GOFANN_ELEM_F16) {
        if ((dim & 1u) == 0) {
            if (vec) {
                const uint4* b16 = static_cast<const uint4*>(row);
                for (uint32_t i = 0; i < dim / 8; ++i) {
                    const uint4 w = b16[i];
                    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        __half2 h;
                        __builtin_memcpy(&h, &ws[k], 4);
                        const float2 bf = __half22float2(h);
                        const uint32_t d = 8 * i + 2 * k;
                        const float dx = bf.x - q[d];
                        const float dy = bf.y - q[d + 1];
                        acc = acc + fmaf(dx, dx, dy * dy);
                    }
                }
                return acc;
            }
            const __half2* b2 = static_cast<const __half2*>(row);
            for (uint32_t d2 = 0; d2 < dim / 2; ++d2) {
                const float2 bf = __half22float2(b2[d2]);
                const float dx = bf.x - q[2 * d2];
                const float dy = bf.y - q[2 * d2 + 1];
                acc = acc + fmaf(dx, dx, dy * dy);
            }
            return acc;
        }
        const __half* b = static_cast<const __half*>(row);
        for (uint32_t d = 0; d < dim; ++d) {
            const float t = __half2float(b[d]) - q[d];
            acc = fmaf(t, t, acc);
        }
        return acc;
    } else {
        const uint8_t* b = static_cast<const uint8_t*>(row);
        if (vec) {
            const uint4* b16 = static_cast<const uint4*>(row);
            for (uint32_t i = 0; i < dim / 16; ++i) {
                const uint4 w = b16[i];
                const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                for (int k = 0; k < 16; ++k) {
                    const float t = static_cast<float>((ws[k >> 2] >> (8 * (k & 3))) & 0xffu) -
                                    q[16 * i + k];
                    acc = fmaf(t, t, acc);
                }
            }
            return acc;
        }
        for (uint32_t d = 0; d < dim; ++d) {
            const float t = static_cast<float>(b[d]) - q[d];
            acc = fmaf(t, t, acc);
        }
        return acc;
    }
}

}  // namespace gofann
