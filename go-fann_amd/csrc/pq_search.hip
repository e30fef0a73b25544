// pq_search.hip -- PQ graph search entry (pq_dim dispatch) and batched PQ
// scoring of explicit (query, sample) pairs.
#include "traversal.hpp"

namespace gofann {
template int pq_search_m<0>(GOFANN_PQ_SEARCH_M_ARGS);

// Batched scoring of explicit (query, sample) pairs: one pair per lane.
template <int kM>
__global__ __launch_bounds__(64) void pq_score_kernel(PqScorer<kM, 0> sc, const uint32_t* q_idx,
                                                     const uint32_t* s_idx, uint32_t n, float* out)
{
    extern __shared__ __align__(16) unsigned char lds[];
    // Pairs of one workgroup need not share a query: the table is rebuilt
    // for every distinct query of the chunk.
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


namespace {

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
    if (pq->code_stride != 0 &&
        (pq->code_stride < pq->pq_dim || (pq->pq_dim % 16 == 0 && pq->code_stride % 16 != 0)))
        return ctx->fail(GOFANN_ERR_INVALID,
                         "code_stride must be >= pq_dim (and a multiple of 16 when pq_dim is)");
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
    if (r->count == 0) return GOFANN_OK;
    switch (pq->pq_dim) {
    case 16: return pq_search_m<16>(ctx, pq, queries, query_elem, g, pred, r, p, out_ids, out_dists, stats);
    case 32: return pq_search_m<32>(ctx, pq, queries, query_elem, g, pred, r, p, out_ids, out_dists, stats);
    case 48: return pq_search_m<48>(ctx, pq, queries, query_elem, g, pred, r, p, out_ids, out_dists, stats);
    case 64: return pq_search_m<64>(ctx, pq, queries, query_elem, g, pred, r, p, out_ids, out_dists, stats);
    default: return pq_search_m<0>(ctx, pq, queries, query_elem, g, pred, r, p, out_ids, out_dists, stats);
    }
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
                           (make_pq_scorer<32, 0>(pq, queries, query_elem)), q_idx, s_idx, n, out);
        break;
    case 48:
        hipLaunchKernelGGL(pq_score_kernel<48>, grid, block, lut_bytes, ctx->stream,
                           (make_pq_scorer<48, 0>(pq, queries, query_elem)), q_idx, s_idx, n, out);
        break;
    default:
        hipLaunchKernelGGL(pq_score_kernel<0>, grid, block, lut_bytes, ctx->stream,
                           (make_pq_scorer<0, 0>(pq, queries, query_elem)), q_idx, s_idx, n, out);
        break;
    }
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("pq_score launch");
    return GOFANN_OK;
}

}  // namespace gofann
