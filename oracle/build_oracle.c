/*
 * build_oracle.c -- CPU restatement of the index construction path (the
 * per-label graphs, the coarse k-means, the PQ and RaBitQ encoders).  TEST
 * INFRASTRUCTURE ONLY: the checker the HIP build kernels
 * (go-fann_amd/csrc/build_kernels.hip) are compared against; only tests/
 * load it, and the product never links it.
 *
 * The reference builds these with cuVS (CAGRA graphs,
 * src/index/graph_builder.cu:1279-1315; PQ, tools/quantization/
 * pq_builder.cu:49-153; the IVF-RaBitQ encoder, third_party/cuvs_rabitq/
 * src/neighbors/ivf_rabitq/gpu_index/quantizer_gpu_fast.cu:39-101, 180-265).
 * cuVS is not in this tree's build, so graph and codebook *quality* is
 * parity unpinned; what is restated here is each step's definition with
 * its arithmetic order, so that the GPU build is checked bit for bit:
 *   score(x, c) = |c|^2 - 2 <x, c>, fp32 sums with fmaf over d ascending;
 *   dist(x, y) = sum_d (x_d - y_d)^2, fmaf over d ascending;
 *   rankings order (value, index) pairs.
 * Compiled with -ffp-contract=off, so every fused multiply-add is an
 * explicit fmaf / fma.
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "gofann_oracle.h"

#define NONE 0xFFFFFFFFu

static float elem_f(const void* rows, int elem, size_t idx)
{
    if (elem == 0) return (float)((const uint8_t*)rows)[idx];
    if (elem == 2) return orc_half_to_float(((const uint16_t*)rows)[idx]);
    return ((const float*)rows)[idx];
}

static int pair_lt(float ad, uint32_t ai, float bd, uint32_t bi)
{
    return ad < bd || (ad == bd && ai < bi);
}

/* SplitMix64's finaliser and the counter-based draws of the build. */
static uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t orc_build_draw64(uint64_t seed, uint64_t stream, uint64_t index)
{
    return mix64(mix64(seed ^ (stream * 0xD1B54A32D192ED03ull)) + index * 0x9E3779B97F4A7C15ull);
}

double orc_build_draw_unit(uint64_t seed, uint64_t stream, uint64_t index)
{
    return (double)(orc_build_draw64(seed, stream, index) >> 11) * (1.0 / 9007199254740992.0);
}

/* The rows as fp32 (exact for u8, f16 and f32). */
static float* rows_f32(const void* rows, int elem, uint32_t dim, uint64_t n)
{
    float* f = (float*)malloc(sizeof(float) * (n * dim > 0 ? n * dim : 1));
    for (uint64_t i = 0; i < n * dim; ++i) f[i] = elem_f(rows, elem, i);
    return f;
}

static void centre_norms(const float* c, uint32_t k, uint32_t dim, float* out)
{
    for (uint32_t r = 0; r < k; ++r) {
        float s = 0.0f;
        for (uint32_t d = 0; d < dim; ++d) s = fmaf(c[(size_t)r * dim + d], c[(size_t)r * dim + d], s);
        out[r] = s;
    }
}

/* Nearest centre: least (|c|^2 - 2 <x, c>, k). */
void orc_build_assign(const void* rows, int elem, uint32_t dim, uint64_t n, const float* centres,
                      uint32_t k, uint32_t* out_idx, float* out_score)
{
    float* cn = (float*)malloc(sizeof(float) * k);
    centre_norms(centres, k, dim, cn);
    float* f = rows_f32(rows, elem, dim, n);
    for (uint64_t i = 0; i < n; ++i) {
        float best = FLT_MAX;
        uint32_t bi = NONE;
        const float* x = f + i * dim;
        for (uint32_t c = 0; c < k; ++c) {
            float acc = 0.0f;
            const float* cc = centres + (size_t)c * dim;
            for (uint32_t d = 0; d < dim; ++d) acc = fmaf(x[d], cc[d], acc);
            const float s = cn[c] - 2.0f * acc;
            if (pair_lt(s, c, best, bi)) {
                best = s;
                bi = c;
            }
        }
        out_idx[i] = bi;
        if (out_score) out_score[i] = best;
    }
    free(f);
    free(cn);
}

/* Distance of two rows as the wave sums it: lane j adds dims j, j + 64, ...
 * with fmaf, then an xor butterfly over offsets 32 .. 1 (lane 0's value). */
static float lane_dist(const void* rows, int elem, uint32_t dim, uint64_t a, uint64_t b)
{
    float s[64];
    for (int l = 0; l < 64; ++l) {
        float acc = 0.0f;
        for (uint32_t d = (uint32_t)l; d < dim; d += 64) {
            const float t = elem_f(rows, elem, a * dim + d) - elem_f(rows, elem, b * dim + d);
            acc = fmaf(t, t, acc);
        }
        s[l] = acc;
    }
    for (int off = 32; off > 0; off >>= 1) {
        float t[64];
        for (int l = 0; l < 64; ++l) t[l] = s[l] + s[l ^ off];
        memcpy(s, t, sizeof(s));
    }
    return s[0];
}

static void copy_row(const void* rows, int elem, uint32_t dim, uint64_t r, float* out)
{
    for (uint32_t d = 0; d < dim; ++d) out[d] = elem_f(rows, elem, r * dim + d);
}

/* k-means++ seeding with the build's draws and its chunked fp64 sums
 * (gofann_build_kmeanspp). */
void orc_build_kmeanspp(const void* rows, int elem, uint32_t dim, uint64_t n, uint32_t k,
                        uint64_t seed, float* centres)
{
    float* best = (float*)malloc(sizeof(float) * n);
    uint64_t pick = (uint64_t)(orc_build_draw_unit(seed, 0, 0) * (double)n);
    if (pick >= n) pick = n - 1;
    copy_row(rows, elem, dim, pick, centres);
    const uint64_t chunk = (n + 1023) / 1024;
    double part[1024];
    for (uint32_t j = 1; j < k; ++j) {
        for (uint64_t i = 0; i < n; ++i) {
            const float d = lane_dist(rows, elem, dim, i, pick);
            best[i] = j == 1 ? d : fminf(best[i], d);
        }
        for (uint64_t t = 0; t < 1024; ++t) {
            double s = 0.0;
            for (uint64_t i = t * chunk; i < (t + 1) * chunk && i < n; ++i) s += (double)best[i];
            part[t] = s;
        }
        double total = 0.0;
        for (int t = 0; t < 1024; ++t) total += part[t];
        const double u = orc_build_draw_unit(seed, 0, j);
        if (!(total > 0.0)) {
            pick = (uint64_t)(u * (double)n);
            if (pick >= n) pick = n - 1;
        } else {
            const double target = u * total;
            double run = 0.0;
            int c = 0;
            for (; c < 1023; ++c) {
                if (run + part[c] >= target) break;
                run += part[c];
            }
            pick = n - 1;
            for (uint64_t i = (uint64_t)c * chunk; i < (uint64_t)(c + 1) * chunk && i < n; ++i) {
                run += (double)best[i];
                if (run >= target) {
                    pick = i;
                    break;
                }
            }
        }
        copy_row(rows, elem, dim, pick, centres + (size_t)j * dim);
    }
    free(best);
}

/* Lloyd iterations: assign, then each centre = mean of its rows (fp64 sums
 * over its rows ascending, rounded to fp32); an empty centre keeps. */
void orc_build_kmeans(const void* rows, int elem, uint32_t dim, uint64_t n, uint32_t k,
                      uint32_t iters, float* centres)
{
    uint32_t* idx = (uint32_t*)malloc(sizeof(uint32_t) * n);
    double* sum = (double*)malloc(sizeof(double) * dim);
    for (uint32_t it = 0; it < iters; ++it) {
        orc_build_assign(rows, elem, dim, n, centres, k, idx, NULL);
        for (uint32_t c = 0; c < k; ++c) {
            uint64_t cnt = 0;
            memset(sum, 0, sizeof(double) * dim);
            for (uint64_t i = 0; i < n; ++i) {
                if (idx[i] != c) continue;
                ++cnt;
                for (uint32_t d = 0; d < dim; ++d) sum[d] += (double)elem_f(rows, elem, i * dim + d);
            }
            if (cnt == 0) continue;
            for (uint32_t d = 0; d < dim; ++d) centres[(size_t)c * dim + d] = (float)(sum[d] / (double)cnt);
        }
    }
    free(sum);
    free(idx);
}

static float row_dist(const float* rows, uint32_t dim, uint64_t a, uint64_t b)
{
    const float* x = rows + a * dim;
    const float* y = rows + b * dim;
    float acc = 0.0f;
    for (uint32_t d = 0; d < dim; ++d) {
        const float t = x[d] - y[d];
        acc = fmaf(t, t, acc);
    }
    return acc;
}


typedef struct {
    float d;
    uint32_t id;
} dpair;

static int dpair_cmp(const void* a, const void* b)
{
    const dpair* x = (const dpair*)a;
    const dpair* y = (const dpair*)b;
    if (x->d < y->d) return -1;
    if (x->d > y->d) return 1;
    return x->id < y->id ? -1 : (x->id > y->id ? 1 : 0);
}

/* kNN inside buckets by brute force: every candidate of the row's probe
 * buckets (its own bucket without a probe list), itself excluded, sorted by
 * (distance, row); the first k. */
void orc_build_knn(const void* rows, int elem, uint32_t dim, const uint32_t* bucket_off,
                   uint32_t buckets, const uint32_t* probe_off, const uint32_t* probe, uint32_t k,
                   uint32_t* out_ids, float* out_d)
{
    const uint32_t n = bucket_off[buckets];
    float* f = rows_f32(rows, elem, dim, n);
    dpair* cand = (dpair*)malloc(sizeof(dpair) * (n > 0 ? n : 1));
    for (uint32_t b = 0; b < buckets; ++b) {
        for (uint32_t i = bucket_off[b]; i < bucket_off[b + 1]; ++i) {
            uint32_t nc = 0;
            const uint32_t pb0 = probe_off ? probe_off[b] : 0, pb1 = probe_off ? probe_off[b + 1] : 1;
            for (uint32_t p = pb0; p < pb1; ++p) {
                const uint32_t q = probe_off ? probe[p] : b;
                for (uint32_t j = bucket_off[q]; j < bucket_off[q + 1]; ++j) {
                    if (j == i) continue;
                    cand[nc].d = row_dist(f, dim, i, j);
                    cand[nc].id = j;
                    ++nc;
                }
            }
            qsort(cand, nc, sizeof(dpair), dpair_cmp);
            for (uint32_t e = 0; e < k; ++e) {
                out_ids[(size_t)i * k + e] = e < nc ? cand[e].id : NONE;
                if (out_d) out_d[(size_t)i * k + e] = e < nc ? cand[e].d : FLT_MAX;
            }
        }
    }
    free(cand);
    free(f);
}

/* PQ code: least (sum_t (x - c)^2 over the subspace, k), fmaf ascending. */
void orc_build_pq_encode(const void* rows, int elem, uint32_t dim, uint64_t n, uint32_t pq_dim,
                         const float* centroids, uint8_t* codes, uint32_t code_stride)
{
    const uint32_t sub = dim / pq_dim;
    for (uint64_t i = 0; i < n; ++i)
        for (uint32_t m = 0; m < pq_dim; ++m) {
            float best = FLT_MAX;
            uint32_t bk = 0;
            for (uint32_t c = 0; c < 256; ++c) {
                float acc = 0.0f;
                for (uint32_t t = 0; t < sub; ++t) {
                    const float d = elem_f(rows, elem, i * dim + m * sub + t) -
                                    centroids[(size_t)c * dim + m * sub + t];
                    acc = fmaf(d, d, acc);
                }
                if (acc < best) {
                    best = acc;
                    bk = c;
                }
            }
            codes[i * code_stride + m] = (uint8_t)bk;
        }
}

/* PQ codebook training: per iteration, encode, then each (subspace, centre)
 * becomes the mean of its rows' subvectors (fp64, rows ascending). */
void orc_build_pq_train(const void* rows, int elem, uint32_t dim, uint64_t n, uint32_t pq_dim,
                        uint32_t iters, float* centroids)
{
    const uint32_t sub = dim / pq_dim;
    uint8_t* codes = (uint8_t*)malloc(n * pq_dim);
    double* sum = (double*)malloc(sizeof(double) * sub);
    for (uint32_t it = 0; it < iters; ++it) {
        orc_build_pq_encode(rows, elem, dim, n, pq_dim, centroids, codes, pq_dim);
        for (uint32_t m = 0; m < pq_dim; ++m)
            for (uint32_t c = 0; c < 256; ++c) {
                uint64_t cnt = 0;
                memset(sum, 0, sizeof(double) * sub);
                for (uint64_t i = 0; i < n; ++i) {
                    if (codes[i * pq_dim + m] != c) continue;
                    ++cnt;
                    for (uint32_t t = 0; t < sub; ++t) sum[t] += (double)elem_f(rows, elem, i * dim + m * sub + t);
                }
                if (cnt == 0) continue;
                for (uint32_t t = 0; t < sub; ++t)
                    centroids[(size_t)c * dim + m * sub + t] = (float)(sum[t] / (double)cnt);
            }
    }
    free(sum);
    free(codes);
}

/* RaBitQ one-bit encoding of rotated rows (quantizer_gpu_fast.cu:180-265,
 * the sums over lanes d % 64 with fmaf, then an xor butterfly). */
void orc_build_rabitq_encode(const float* xr, uint32_t n, uint32_t P, const float* anchors,
                             uint32_t A, uint32_t* aid, uint8_t* codes, float* factors)
{
    orc_build_assign(xr, 1, P, n, anchors, A, aid, NULL);
    for (uint32_t i = 0; i < n; ++i) {
        const float* x = xr + (size_t)i * P;
        const float* c = anchors + (size_t)aid[i] * P;
        uint32_t* w = (uint32_t*)(codes + (size_t)i * (P / 8));
        for (uint32_t q = 0; q < P / 32; ++q) w[q] = 0;
        float l2[64], ipr[64], ipc[64];
        for (int l = 0; l < 64; ++l) l2[l] = ipr[l] = ipc[l] = 0.0f;
        for (uint32_t t = 0; t < P / 64; ++t)
            for (int l = 0; l < 64; ++l) {
                const uint32_t d = t * 64 + (uint32_t)l;
                const float rv = x[d] - c[d];
                const int bit = rv > 0.0f;
                const float xu = bit ? 0.5f : -0.5f;
                l2[l] = fmaf(rv, rv, l2[l]);
                ipr[l] = fmaf(rv, xu, ipr[l]);
                ipc[l] = fmaf(c[d], xu, ipc[l]);
                if (bit) w[d / 32] |= 1u << (31 - d % 32);
            }
        for (int off = 32; off > 0; off >>= 1) {
            float a[64], b[64], e[64];
            for (int l = 0; l < 64; ++l) {
                a[l] = l2[l] + l2[l ^ off];
                b[l] = ipr[l] + ipr[l ^ off];
                e[l] = ipc[l] + ipc[l ^ off];
            }
            memcpy(l2, a, sizeof(a));
            memcpy(ipr, b, sizeof(b));
            memcpy(ipc, e, sizeof(e));
        }
        const float L2 = l2[0], IPR = ipr[0], IPC = ipc[0];
        const float xu_sq = 0.25f * (float)P;
        const float denom = IPR == 0.0f ? INFINITY : IPR;
        const float f_add = L2 + 2.0f * L2 * (IPC / denom);
        const float f_rescale = -2.0f * L2 / denom;
        const float ratio = (L2 * xu_sq) / (denom * denom);
        const float inner = fmaxf((ratio - 1.0f) / fmaxf((float)P - 1.0f, 1.0f), 0.0f);
        const float l2n = sqrtf(fmaxf(L2, 0.0f));
        factors[(size_t)i * 3 + 0] = f_add;
        factors[(size_t)i * 3 + 1] = f_rescale;
        factors[(size_t)i * 3 + 2] = 2.0f * (l2n * 1.9f * sqrtf(inner));
    }
}

/* Row nearest the mean (build_seed_local_ids_typed, dataloader.cpp:
 * 7361-7406, with the build's two-level fp64 mean). */
uint32_t orc_build_medoid(const void* rows, int elem, uint32_t dim, uint64_t n)
{
    const uint64_t blk = 4096, blocks = (n + blk - 1) / blk;
    double* part = (double*)calloc(blocks * dim, sizeof(double));
    double* mean = (double*)calloc(dim, sizeof(double));
    for (uint64_t b = 0; b < blocks; ++b)
        for (uint32_t d = 0; d < dim; ++d) {
            double s = 0.0;
            for (uint64_t i = b * blk; i < (b + 1) * blk && i < n; ++i) s += (double)elem_f(rows, elem, i * dim + d);
            part[b * dim + d] = s;
        }
    for (uint32_t d = 0; d < dim; ++d) {
        double s = 0.0;
        for (uint64_t b = 0; b < blocks; ++b) s += part[b * dim + d];
        mean[d] = s / (double)n;
    }
    double best = DBL_MAX;
    uint64_t bi = 0;
    for (uint64_t i = 0; i < n; ++i) {
        double s = 0.0;
        for (uint32_t d = 0; d < dim; ++d) {
            const double t = (double)elem_f(rows, elem, i * dim + d) - mean[d];
            s = fma(t, t, s);
        }
        if (s < best) {
            best = s;
            bi = i;
        }
    }
    free(part);
    free(mean);
    return (uint32_t)bi;
}

/* Bucket means (fp64 sums, rounded to fp32) and the row nearest each mean
 * (fp32 distance, least (distance, row)). */
void orc_build_bucket_reps(const void* rows, int elem, uint32_t dim, const uint32_t* bucket_off,
                           uint32_t buckets, float* means, uint32_t* reps)
{
    for (uint32_t b = 0; b < buckets; ++b) {
        const uint32_t s = bucket_off[b], e = bucket_off[b + 1];
        float* mu = means + (size_t)b * dim;
        if (s == e) {
            reps[b] = NONE;
            continue;
        }
        for (uint32_t d = 0; d < dim; ++d) {
            double sum = 0.0;
            for (uint32_t i = s; i < e; ++i) sum += (double)elem_f(rows, elem, (size_t)i * dim + d);
            mu[d] = (float)(sum / (double)(e - s));
        }
        float bv = FLT_MAX;
        uint32_t bi = NONE;
        for (uint32_t i = s; i < e; ++i) {
            float acc = 0.0f;
            for (uint32_t d = 0; d < dim; ++d) {
                const float t = elem_f(rows, elem, (size_t)i * dim + d) - mu[d];
                acc = fmaf(t, t, acc);
            }
            if (pair_lt(acc, i, bv, bi)) {
                bv = acc;
                bi = i;
            }
        }
        reps[b] = bi;
    }
}

/* The link rules of gofann_build_links. */
void orc_build_links(uint32_t n, const uint32_t* knn, uint32_t knn_width, const uint32_t* bucket_of,
                     const uint32_t* reps, const uint32_t* near, uint32_t near_width, uint32_t buckets,
                     const uint32_t* order, uint32_t degree, uint32_t local, uint32_t near_links,
                     uint32_t rep_local, uint32_t rep_near, uint32_t entry, uint64_t seed,
                     uint32_t* out)
{
    uint32_t* cand = (uint32_t*)malloc(sizeof(uint32_t) * 1024);
    for (uint32_t i = 0; i < n; ++i) {
        const uint32_t dst = order[i];
        if (dst >= n) continue;
        const uint32_t b = bucket_of[i];
        const int bvalid = b < buckets;
        const uint32_t rep_b = bvalid ? reps[b] : NONE;
        const int is_rep = rep_b == i;
        uint32_t nc = 0;
        if (i == entry) {
            for (uint32_t j = 0; j < 4 * degree; ++j)
                cand[nc++] = (uint32_t)(orc_build_draw64(seed, 3, (uint64_t)i * 256 + j) % n);
        } else {
            const uint32_t nk = is_rep ? rep_local : local;
            const uint32_t nn = is_rep ? rep_near : near_links;
            for (uint32_t j = 0; j < nk; ++j) cand[nc++] = j < knn_width ? knn[(size_t)i * knn_width + j] : NONE;
            if (!is_rep) cand[nc++] = rep_b;
            for (uint32_t j = 0; j < nn; ++j) {
                const uint32_t nb = bvalid && j < near_width ? near[(size_t)b * near_width + j] : NONE;
                cand[nc++] = nb < buckets ? reps[nb] : NONE;
            }
            const uint64_t stream = is_rep ? 2 : 1;
            for (uint32_t j = 0; j < degree; ++j)
                cand[nc++] = (uint32_t)(orc_build_draw64(seed, stream, (uint64_t)i * 256 + j) % n);
        }
        uint32_t* o = out + (size_t)dst * degree;
        uint32_t kept = 0;
        for (uint32_t c = 0; c < nc && kept < degree; ++c) {
            const uint32_t v = cand[c];
            int keep = v != NONE && v != i && v < n;
            for (uint32_t j = 0; keep && j < c; ++j) keep = cand[j] != v;
            if (keep) o[kept++] = order[v] < n ? order[v] : NONE;
        }
        for (; kept < degree; ++kept) o[kept] = NONE;
    }
    free(cand);
}

static int u64_cmp(const void* a, const void* b)
{
    const uint64_t x = *(const uint64_t*)a, y = *(const uint64_t*)b;
    return x < y ? -1 : (x > y ? 1 : 0);
}

static int has_entry(const uint32_t* o, uint32_t k, uint32_t v)
{
    for (uint32_t q = 0; q < k; ++q)
        if (o[q] == v) return 1;
    return 0;
}

/* CAGRA's rank-based reordering and reverse-edge merge
 * (gofann_build_cagra_optimize). */
void orc_build_cagra_optimize(const uint32_t* knn, uint32_t n, uint32_t kin, uint32_t degree,
                              uint32_t* pruned, uint32_t* out)
{
    uint32_t* det = (uint32_t*)malloc(sizeof(uint32_t) * kin);
    /* first[v] = first position of row v in the current row's list */
    uint32_t* first = (uint32_t*)malloc(sizeof(uint32_t) * (n > 0 ? n : 1));
    for (uint32_t v = 0; v < n; ++v) first[v] = NONE;
    for (uint32_t i = 0; i < n; ++i) {
        const uint32_t* ki = knn + (size_t)i * kin;
        memset(det, 0, sizeof(uint32_t) * kin);
        for (uint32_t j = kin; j-- > 0;)
            if (ki[j] < n) first[ki[j]] = j;
        for (uint32_t m = 0; m < kin; ++m) {
            const uint32_t u = ki[m];
            if (u == NONE || u >= n) continue;
            const uint32_t* ku = knn + (size_t)u * kin;
            for (uint32_t r = 0; r < kin; ++r) {
                const uint32_t v = ku[r];
                if (v >= n) continue;
                const uint32_t j = first[v];
                if (j != NONE && j > m && j > r) ++det[j];
            }
        }
        for (uint32_t j = 0; j < kin; ++j)
            if (ki[j] < n) first[ki[j]] = NONE;
        uint32_t* o = pruned + (size_t)i * degree;
        for (uint32_t j = 0; j < degree; ++j) o[j] = NONE;
        for (uint32_t j = 0; j < kin; ++j) {
            if (ki[j] == NONE) continue;
            uint32_t rank = 0;
            for (uint32_t q = 0; q < kin; ++q)
                if (ki[q] != NONE && (det[q] < det[j] || (det[q] == det[j] && q < j))) ++rank;
            if (rank < degree) o[rank] = ki[j];
        }
    }
    free(first);
    free(det);
    /* reverse edges of v in order of (position k in the source's list, source u) */
    uint64_t* rk = (uint64_t*)malloc(sizeof(uint64_t) * ((size_t)n * degree + 1));
    uint64_t cnt = 0;
    for (uint32_t u = 0; u < n; ++u)
        for (uint32_t k = 0; k < degree; ++k) {
            const uint32_t v = pruned[(size_t)u * degree + k];
            if (v < n) rk[cnt++] = ((uint64_t)v << 34) | ((uint64_t)k << 27) | u;
        }
    qsort(rk, cnt, sizeof(uint64_t), u64_cmp);
    uint64_t pos = 0;
    for (uint32_t i = 0; i < n; ++i) {
        const uint32_t* f = pruned + (size_t)i * degree;
        uint32_t* o = out + (size_t)i * degree;
        uint32_t k = 0, kf = 0;
        const uint32_t protect = degree / 2;
        for (; kf < degree && k < protect; ++kf) {
            const uint32_t v = f[kf];
            if (v == NONE || v == i || has_entry(o, k, v)) continue;
            o[k++] = v;
        }
        while (pos < cnt && (uint32_t)(rk[pos] >> 34) < i) ++pos;
        uint64_t re = pos;
        while (re < cnt && (uint32_t)(rk[re] >> 34) == i) ++re;
        const uint64_t rcap = pos + 2ull * degree < re ? pos + 2ull * degree : re;
        for (uint64_t r = pos; r < rcap && k < degree; ++r) {
            const uint32_t v = (uint32_t)(rk[r] & ((1ull << 27) - 1));
            if (v == i || has_entry(o, k, v)) continue;
            o[k++] = v;
        }
        for (; kf < degree && k < degree; ++kf) {
            const uint32_t v = f[kf];
            if (v == NONE || v == i || has_entry(o, k, v)) continue;
            o[k++] = v;
        }
        for (; k < degree; ++k) o[k] = NONE;
    }
    free(rk);
}

/* Rows reachable from `entry` (breadth-first); returns their number. */
uint32_t orc_build_reach(const uint32_t* graph, uint32_t n, uint32_t degree, uint32_t entry,
                         uint32_t* reached)
{
    uint32_t* queue = (uint32_t*)malloc(sizeof(uint32_t) * (n > 0 ? n : 1));
    memset(reached, 0, sizeof(uint32_t) * n);
    uint32_t head = 0, tail = 0;
    reached[entry] = 1;
    queue[tail++] = entry;
    while (head < tail) {
        const uint32_t u = queue[head++];
        for (uint32_t j = 0; j < degree; ++j) {
            const uint32_t v = graph[(size_t)u * degree + j];
            if (v < n && !reached[v]) {
                reached[v] = 1;
                queue[tail++] = v;
            }
        }
    }
    free(queue);
    return tail;
}
