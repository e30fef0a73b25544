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

// Centroid distances as the reference computes them
// (RabitqQueryRotation::centroid_distances, src/search/rabitq/
// rabitq_query_rotation.cuh:88-113): row norms, an SGEMM for -2 <y, c>,
// then g = max(0, -2 <y, c> + |y|^2 + |c|^2) (the clamp absorbs the
// cancellation when a query sits on an anchor).
__global__ __launch_bounds__(256) void row_norms_kernel(const float* m, uint32_t rows, uint32_t dim,
                                                        float* norms)
{
    __shared__ float part[256];
    const uint32_t r = blockIdx.x;
    if (r >= rows) return;
    const int t = static_cast<int>(threadIdx.x);
    float sum = 0.0f;
    for (uint32_t d = t; d < dim; d += 256) {
        const float v = m[static_cast<size_t>(r) * dim + d];
        sum = fmaf(v, v, sum);
    }
    part[t] = sum;
    __syncthreads();
    for (int stride = 128; stride > 0; stride >>= 1) {
        if (t < stride) part[t] += part[t + stride];
        __syncthreads();
    }
    if (t == 0) norms[r] = part[0];
}

__global__ __launch_bounds__(256) void finish_centroid_dist_kernel(float* g, const float* qn,
                                                                   const float* an,
                                                                   uint32_t queries,
                                                                   uint32_t anchors)
{
    const size_t pair = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
    if (pair >= static_cast<size_t>(queries) * anchors) return;
    g[pair] = fmaxf(0.0f, g[pair] + qn[pair / anchors] + an[pair % anchors]);
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
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("RaBitQ preparation launch");
    if (A > 0 && rq->anchors) {
        float* norms = static_cast<float*>(
            ctx->scratch(Context::kScratchMisc, (static_cast<size_t>(count) + A) * sizeof(float)));
        if (!norms) return ctx->fail(GOFANN_ERR_NOMEM, "centroid norm scratch allocation failed");
        float* qn = norms;
        float* an = norms + count;
        hipLaunchKernelGGL(row_norms_kernel, dim3(count), dim3(256), 0, ctx->stream, out->rotated,
                           count, P, qn);
        hipLaunchKernelGGL(row_norms_kernel, dim3(A), dim3(256), 0, ctx->stream, rq->anchors, A, P,
                           an);
        // column-major g[A][N] = -2 anchors^T[A][P] rotated[P][N]
        const float minus2 = -2.0f;
        if (rocblas_sgemm(h, rocblas_operation_transpose, rocblas_operation_none,
                          static_cast<int>(A), static_cast<int>(count), static_cast<int>(P),
                          &minus2, rq->anchors, static_cast<int>(P), out->rotated,
                          static_cast<int>(P), &zero, out->centroid_dists,
                          static_cast<int>(A)) != rocblas_status_success)
            return ctx->fail(GOFANN_ERR_HIP, "rocblas_sgemm (centroid distances)");
        const size_t pairs = static_cast<size_t>(count) * A;
        hipLaunchKernelGGL(finish_centroid_dist_kernel, dim3(static_cast<uint32_t>((pairs + 255) / 256)),
                           dim3(256), 0, ctx->stream, out->centroid_dists, qn, an, count, A);
        if (hipGetLastError() != hipSuccess) return ctx->fail_hip("centroid distance launch");
    }
    return GOFANN_OK;
}

}  // namespace gofann
