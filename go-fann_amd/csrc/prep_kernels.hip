// prep_kernels.hip -- RaBitQ query preparation on gfx950
// (init_prepared_query_state, src/search/rabitq/backend_rabitq.cu:7800-8084):
//   rotated = Q R                 (FP32 SGEMM on MFMA through rocBLAS -- a
//                                  plain library GEMM; RabitqQueryRotation::
//                                  apply, rabitq_query_rotation.cuh:71-87)
//   k1 = -0.5 * sum(rotated)      (compute_rabitq_query_factors_kernel,
//                                  backend_rabitq.cu:2898-2929)
//   q8, scale                     (quantize_rabitq_queries_int8_kernel,
//                                  backend_rabitq.cu:2931-2964)
//   g[q][a] = |q - c_a|^2         (centroid_distances, rabitq_query_rotation.
//                                  cuh:12-39, 89-113; computed directly, not
//                                  through the cancelling norm expansion)
// The reductions that feed the integer path (scale, k1) use the reference's
// 256-thread order exactly: strided partial sums, then a shared tree.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>

#include "device_common.hpp"
#include "gofann_internal.hpp"

#include <rocblas/rocblas.h>

namespace gofann {

// One 256-thread block per query row: scale, q8 and k1.
__global__ __launch_bounds__(256) void quantize_queries_kernel(const float* rotated, uint32_t P,
                                                               uint32_t count, int8_t* q8,
                                                               float* scale, float* k1)
{
    __shared__ float part[256];
    const uint32_t q = blockIdx.x;
    const uint32_t t = threadIdx.x;
    if (q >= count) return;
    const float* row = rotated + static_cast<size_t>(q) * P;
    float sum = 0.0f;
    float mx = 0.0f;
    for (uint32_t d = t; d < P; d += 256) {
        sum += row[d];
        mx = fmaxf(mx, fabsf(row[d]));
    }
    part[t] = sum;
    __syncthreads();
    for (uint32_t s = 128; s > 0; s >>= 1) {
        if (t < s) part[t] += part[t + s];
        __syncthreads();
    }
    const float total = part[0];
    __syncthreads();
    part[t] = mx;
    __syncthreads();
    for (uint32_t s = 128; s > 0; s >>= 1) {
        if (t < s) part[t] = fmaxf(part[t], part[t + s]);
        __syncthreads();
    }
    const float sc = part[0] > 0.0f ? part[0] / 127.0f : 1.0f;
    if (t == 0) {
        scale[q] = sc;
        k1[q] = total * -0.5f;
    }
    for (uint32_t d = t; d < P; d += 256) {
        int v = __float2int_rn(row[d] / sc);
        v = v < -127 ? -127 : (v > 127 ? 127 : v);
        q8[static_cast<size_t>(q) * P + d] = static_cast<int8_t>(v);
    }
}

// g[q][a] = sum_p (y[q][p] - c[a][p])^2, accumulated directly (fma, p
// ascending) rather than as |y|^2 + |c|^2 - 2<y,c>: the expansion cancels
// catastrophically when a query sits on an anchor.  A 256-thread block owns
// a 32 x 32 (query, anchor) tile; both operand tiles stream through LDS in
// 64-wide slices of the padded dimension.
constexpr int kCdTile = 32;
constexpr int kCdSlice = 64;

__global__ __launch_bounds__(256) void centroid_dist_kernel(const float* y, const float* c,
                                                            uint32_t queries, uint32_t anchors,
                                                            uint32_t P, float* out)
{
    __shared__ float ys[kCdTile][kCdSlice + 1];
    __shared__ float cs[kCdTile][kCdSlice + 1];
    const int t = static_cast<int>(threadIdx.x);
    const uint32_t q0 = blockIdx.y * kCdTile;
    const uint32_t a0 = blockIdx.x * kCdTile;
    // thread t owns pairs (qi, ai) with qi = t / 8, ai = (t % 8) * 4 + j
    const int qi = t >> 3;
    const int ai = (t & 7) * 4;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t p0 = 0; p0 < P; p0 += kCdSlice) {
        for (int e = t; e < kCdTile * kCdSlice; e += 256) {
            const int r = e / kCdSlice, k = e % kCdSlice;
            const uint32_t pk = p0 + k;
            ys[r][k] = (q0 + r < queries && pk < P) ? y[static_cast<size_t>(q0 + r) * P + pk] : 0.0f;
            cs[r][k] = (a0 + r < anchors && pk < P) ? c[static_cast<size_t>(a0 + r) * P + pk] : 0.0f;
        }
        __syncthreads();
        const int kmax = (P - p0) < static_cast<uint32_t>(kCdSlice) ? static_cast<int>(P - p0) : kCdSlice;
        for (int k = 0; k < kmax; ++k) {
            const float yv = ys[qi][k];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float d = yv - cs[ai + j][k];
                acc[j] = fmaf(d, d, acc[j]);
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t qq = q0 + qi, aa = a0 + ai + j;
        if (qq < queries && aa < anchors) out[static_cast<size_t>(qq) * anchors + aa] = acc[j];
    }
}

// The context's rocBLAS handle, created on first use and bound to the
// context's current stream before every call.
rocblas_handle blas_handle(Context* ctx)
{
    if (!ctx->blas) {
        rocblas_handle h = nullptr;
        if (rocblas_create_handle(&h) != rocblas_status_success) return nullptr;
        ctx->blas = h;
    }
    rocblas_handle h = static_cast<rocblas_handle>(ctx->blas);
    if (rocblas_set_stream(h, ctx->stream) != rocblas_status_success) return nullptr;
    return h;
}

void destroy_blas(Context* ctx)
{
    if (ctx->blas) (void)rocblas_destroy_handle(static_cast<rocblas_handle>(ctx->blas));
    ctx->blas = nullptr;
}

int rabitq_prepare(Context* ctx, const gofann_rabitq_view* rq, const float* queries,
                   uint32_t count, const float* rotation, gofann_rabitq_queries* out)
{
    if (!rq || !queries || !rotation || !out || !out->rotated || !out->q8 || !out->scale ||
        !out->k1 || !out->centroid_dists)
        return ctx->fail(GOFANN_ERR_INVALID, "RaBitQ preparation inputs incomplete");
    if (rq->dim == 0 || rq->padded_dim < rq->dim || rq->padded_dim % 64 != 0)
        return ctx->fail(GOFANN_ERR_INVALID, "invalid RaBitQ dimensions");
    if (count == 0) return GOFANN_OK;
    const uint32_t D = rq->dim, P = rq->padded_dim, A = rq->num_anchors;
    // rotated[N][P] = Q[N][D] R[D][P]: FP32 SGEMM on the MFMA units through
    // rocBLAS; column-major, that is rotated^T = R^T Q^T.
    rocblas_handle h = blas_handle(ctx);
    if (!h) return ctx->fail(GOFANN_ERR_HIP, "rocBLAS handle");
    const float one = 1.0f, zero = 0.0f;
    if (rocblas_sgemm(h, rocblas_operation_none, rocblas_operation_none, static_cast<int>(P),
                      static_cast<int>(count), static_cast<int>(D), &one, rotation,
                      static_cast<int>(P), queries, static_cast<int>(D), &zero, out->rotated,
                      static_cast<int>(P)) != rocblas_status_success)
        return ctx->fail(GOFANN_ERR_HIP, "rocblas_sgemm (query rotation)");
    hipLaunchKernelGGL(quantize_queries_kernel, dim3(count), dim3(256), 0, ctx->stream, out->rotated,
                       P, count, out->q8, out->scale, out->k1);
    if (A > 0 && rq->anchors) {
        const dim3 grid((A + kCdTile - 1) / kCdTile, (count + kCdTile - 1) / kCdTile);
        hipLaunchKernelGGL(centroid_dist_kernel, grid, dim3(256), 0, ctx->stream, out->rotated,
                           rq->anchors, count, A, P, out->centroid_dists);
    }
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("RaBitQ preparation launch");
    return GOFANN_OK;
}

}  // namespace gofann
