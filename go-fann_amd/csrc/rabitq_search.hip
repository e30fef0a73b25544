// rabitq_search.hip -- RaBitQ graph search entry and batched RaBitQ scoring.
#include "traversal.hpp"

namespace gofann {
// rabitq_pair.hip: the two-routes-per-wave traversal for degree <= 32.
bool rabitq_pair_eligible(const gofann_rabitq_view* rq, const gofann_graph_view* g,
                          const gofann_search_params* p);
int rabitq_pair_search(Context* ctx, const RabitqScorer& sc, const gofann_graph_view* g,
                       const gofann_predicate_view* pred, const gofann_routes* r,
                       const gofann_search_params* p, uint32_t* out_ids, float* out_dists,
                       gofann_route_stats* stats);

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
        const float v = sc.score(mine ? s_idx[i] : 0u, mine);  // every lane calls score
        if (mine) {
            out[i] = v;
            if (ip_out) ip_out[i] = sc.ip_int(s_idx[i]);
        }
    }
}


namespace {

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
    sc.records = rq->records;
    sc.record_stride = rq->record_stride;
    sc.halves = 0;
    return sc;
}

int check_rabitq(Context* ctx, const gofann_rabitq_view* rq, const gofann_rabitq_queries* pre)
{
    if (!rq || !pre || !rq->codes || !rq->factors || !rq->anchor_ids || !pre->q8 || !pre->scale ||
        !pre->k1 || !pre->centroid_dists)
        return ctx->fail(GOFANN_ERR_INVALID, "RaBitQ view incomplete");
    if (rq->padded_dim == 0 || rq->padded_dim % 128 != 0)
        return ctx->fail(GOFANN_ERR_INVALID, "padded_dim must be a positive multiple of 128");
    if (rq->records != nullptr &&
        (rq->record_stride % 16 != 0 || rq->record_stride < rq->padded_dim / 8 + 12 ||
         (reinterpret_cast<uintptr_t>(rq->records) & 15u) != 0))
        return ctx->fail(GOFANN_ERR_INVALID,
                         "RaBitQ records: stride a multiple of 16 of at least padded_dim/8 + 12, "
                         "16-byte aligned");
    return GOFANN_OK;
}

}  // namespace

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
    if (r->count == 0) return GOFANN_OK;
    // 8 planes x padded_dim bits, then the whole-wave scorer's candidates
    const uint32_t plane_bytes = rq->padded_dim + kRabitqCoopBytes;
    const Layout l = make_layout(plane_bytes, p->queue_limit, p->result_width);
    ctx->last_table_in_lds = 1;
    // Every beam keeps its frontier in LDS.  (A frontier held in registers
    // for Q + 2 <= 64, lane i holding entry i, was slower than the
    // wave-parallel LDS heap operations: C3 traversal 47.8 against 46.9 ms,
    // C5 at Q = 16 1.42 against 1.36 ms.)
    // Degree <= 32: two routes per wave (rabitq_pair.hip), same results.
    if (rabitq_pair_eligible(rq, g, p))
        return rabitq_pair_search(ctx, make_rabitq_scorer(rq, pre), g, pred, r, p, out_ids,
                                  out_dists, stats);
    const Placement pl = choose_visited<RabitqScorer>(ctx, l, p->hash_mode);
    RabitqScorer sc = make_rabitq_scorer(rq, pre);
    // no neighbour past lane 31: rows scored a candidate per lane take two
    // lanes each (the whole-wave rows of 2048 / 4096 bits are unaffected)
    sc.halves = g->degree <= 32 ? 1 : 0;
    return launch_traversal<RabitqScorer>(ctx, sc, l, pl, g, pred, r, p, out_ids, out_dists, stats, 1);
}

int rabitq_score(Context* ctx, const gofann_rabitq_view* rq, const gofann_rabitq_queries* pre,
                 const uint32_t* q_idx, const uint32_t* s_idx, uint32_t n, float* out,
                 int32_t* ip_int)
{
    int rc = check_rabitq(ctx, rq, pre);
    if (rc) return rc;
    if (n == 0) return GOFANN_OK;
    const dim3 grid((n + kWave - 1) / kWave), block(kWave);
    hipLaunchKernelGGL(rabitq_score_kernel, grid, block, rq->padded_dim + kRabitqCoopBytes, ctx->stream,
                       make_rabitq_scorer(rq, pre), q_idx, s_idx, n, out, ip_int);
    if (hipGetLastError() != hipSuccess) return ctx->fail_hip("rabitq_score launch");
    return GOFANN_OK;
}

}  // namespace gofann
