// prep_kernels.hip -- RaBitQ query preparation on gfx950
// (init_prepared_query_state, src/search/rabitq/backend_rabitq.cu:7800-8084):
//   rotated = Q R                 (FP32 GEMM on MFMA; RabitqQueryRotation::
//                                  apply, rabitq_query_rotation.cuh:71-87)
//   k1 = -0.5 * sum(rotated)      (compute_rabitq_query_factors_kernel,
//                                  backend_rabitq.cu:2898-2929)
//   q8, scale                     (quantize_rabitq_queries_int8_kernel,
//                                  backend_rabitq.cu:2931-2964)
//   g[q][a] = max(0, -2<q,c_a> + |q|^2 + |c_a|^2)
//                                 (centroid_distances, rabitq_query_rotation.
//                                  cuh:12-39, 89-113)
// The reductions that feed the integer path (scale, k1) use the reference's
// 256-thread order exactly: strided partial sums, then a shared tree.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>

#include "device_common.hpp"
#include "gofann_internal.hpp"

namespace gofann {

// C[m][n] = alpha * sum_k A(m,k) B(k,n) in FP32 on the 32x32x2 MFMA.  One
// wave computes one 32x32 tile; a 256-thread workgroup covers 64x64.
// A(m,k) = A[m*a_m + k*a_k], B(k,n) = B[k*b_k + n*b_n], C row-major ldc.
struct GemmArgs {
    const float* A;
    const float* B;
    float* C;
    uint32_t M, N, K;
    size_t a_m, a_k, b_k, b_n, ldc;
    float alpha;
};

__global__ __launch_bounds__(256) void gemm_f32_mfma_kernel(GemmArgs g)
{
    const int lane = static_cast<int>(threadIdx.x) & 63;
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    const uint32_t m0 = blockIdx.y * 64 + (wave >> 1) * 32;
    const uint32_t n0 = blockIdx.x * 64 + (wave & 1) * 32;
    const uint32_t row = m0 + (lane & 31);   // A operand row of this lane
    const uint32_t col = n0 + (lane & 31);   // B operand column of this lane
    const uint32_t kk = static_cast<uint32_t>(lane >> 5);
    typedef float float16v __attribute__((ext_vector_type(16)));
    float16v acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
    for (uint32_t k = 0; k < g.K; k += 2) {
        const uint32_t kx = k + kk;
        const float a = (row < g.M && kx < g.K) ? g.A[row * g.a_m + kx * g.a_k] : 0.0f;
        const float b = (col < g.N && kx < g.K) ? g.B[kx * g.b_k + col * g.b_n] : 0.0f;
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc, 0, 0, 0);
    }
    // Output layout of the 32x32 MFMA: lane l, register i holds
    // D[8*(i/4) + 4*(l/32) + i%4][l%32].
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t r = m0 + 8 * (i / 4) + 4 * (lane >> 5) + (i % 4);
        const uint32_t c = n0 + (lane & 31);
        if (r < g.M && c < g.N) g.C[r * g.ldc + c] = g.alpha * acc[i];
    }
}

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

// rabitq_row_norms_kernel order: 256 strided fma partials, shared tree.
__global__ __launch_bounds__(256) void row_norms_kernel(const float* m, uint32_t rows, uint32_t dim,
                                                        float* norms)
{
    __shared__ float part[256];
    const uint32_t r = blockIdx.x;
    const uint32_t t = threadIdx.x;
    if (r >= rows) return;
    float sum = 0.0f;
    for (uint32_t d = t; d < dim; d += 256) {
        const float v = m[static_cast<size_t>(r) * dim + d];
        sum = fmaf(v, v, sum);
    }
    part[t] = sum;
    __syncthreads();
    for (uint32_t s = 128; s > 0; s >>= 1) {
        if (t < s) part[t] += part[t + s];
        __syncthreads();
    }
    if (t == 0) norms[r] = part[0];
}

__global__ void finish_centroid_kernel(float* dists, const float* qn, const float* an,
                                       uint32_t queries, uint32_t anchors)
{
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<size_t>(queries) * anchors) return;
    dists[i] = fmaxf(0.0f, dists[i] + qn[i / anchors] + an[i % anchors]);
}

namespace {
void launch_gemm(Context* ctx, const GemmArgs& g)
{
    const dim3 grid((g.N + 63) / 64, (g.M + 63) / 64), block(256);
    hipLaunchKernelGGL(gemm_f32_mfma_kernel, grid, block, 0, ctx->stream, g);
}
}  // namespace

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
    // rotated[N][P] = Q[N][D] R[D][P]
    GemmArgs g{queries, rotation, out->rotated, count, P, D, D, 1, P, 1, P, 1.0f};
    launch_gemm(ctx, g);
    hipLaunchKernelGGL(quantize_queries_kernel, dim3(count), dim3(256), 0, ctx->stream, out->rotated,
                       P, count, out->q8, out->scale, out->k1);
    if (A > 0 && rq->anchors) {
        const size_t need = (static_cast<size_t>(count) + A) * sizeof(float);
        float* norms = static_cast<float*>(ctx->scratch(Context::kScratchMisc, need));
        if (!norms) return ctx->fail(GOFANN_ERR_NOMEM, "norm scratch");
        hipLaunchKernelGGL(row_norms_kernel, dim3(count), dim3(256), 0, ctx->stream, out->rotated,
                           count, P, norms);
        hipLaunchKernelGGL(row_norms_kernel, dim3(A), dim3(256), 0, ctx->stream, rq->anchors, A, P,
                           norms + count);
        // dots[N][A] = -2 * rotated[N][P] anchors[A][P]^T
        GemmArgs h{out->rotated, rq->anchors, out->centroid_dists, count, A, P, P, 1, 1, P, A, -2.0f};
        launch_gemm(ctx, h);
        const size_t pairs = static_cast<size_t>(count) * A;
        hipLaunchKernelGGL(finish_centroid_kernel, dim3(static_cast<uint32_t>((pairs + 255) / 256)),
                           dim3(256), 0, ctx->stream, out->centroid_dists, norms, norms + count,
                           count, A);
    }
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("RaBitQ preparation launch");
    return GOFANN_OK;
}

}  // namespace gofann
