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
template <int kElem>
__device__ __forceinline__ float l2_w32_partial(const void* row, const float* q, uint32_t dim,
                                                uint32_t j)
{
    float p = 0.0f;
    if constexpr (kElem == GOFANN_ELEM_F32) {
        const float* b = static_cast<const float*>(row);
#pragma unroll 8
        for (uint32_t d = j; d < dim; d += 32) {
            const float diff = b[d] - q[d];
            p = fmaf(diff, diff, p);
        }
    } else if constexpr (kElem == GOFANN_ELEM_F16) {
        if ((dim & 1u) == 0) {
            const __half2* b2 = static_cast<const __half2*>(row);
            const float2* q2 = reinterpret_cast<const float2*>(q);
            const uint32_t dim2 = dim >> 1;
#pragma unroll 8
            for (uint32_t d2 = j; d2 < dim2; d2 += 32) {
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
