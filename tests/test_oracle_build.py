"""Pins of the oracle's index-construction restatement (oracle/build_oracle.c)
against independent statements: numpy brute force on integer-valued data
(where every fp32 sum is exact, so a wrong index, term or tie rule shows as
a different id), the published SplitMix64 vector, fp64 closed forms of the
RaBitQ encoder (quantizer_gpu_fast.cu:200-245), the CAGRA paper's detour
definition enumerated over two-hop paths, and scipy's breadth-first order.
CPU only."""
from __future__ import annotations

import numpy as np
import pytest

import pyoracle as po
from gofann_amd import index as gi

U32MAX = 0xFFFFFFFF


def test_splitmix64_published_vector_and_host_draw():
    # SplitMix64 (Steele, Lea, Flood 2014; Vigna's splitmix64.c): the first
    # output from state 0 is mix(0x9E3779B97F4A7C15) = 0xE220A8397B1DCDAF.
    # orc_build_draw64(seed, stream, index) = mix(mix(seed ^ stream * C) +
    # index * golden): with seed = mix^-1 unknown, check through stream 0,
    # seed 0: mix(mix(0) + 1 * golden) = mix(golden) since mix(0) = 0.
    assert po.build_draw64(0, 0, 1) == 0xE220A8397B1DCDAF
    for seed, stream, idx in [(0, 0, 0), (7, 1, 5), (123456789, 3, 2**40 + 3), (2**63, 4, 99)]:
        u = po.build_draw_unit(seed, stream, idx)
        assert u == gi._draw_unit(seed, stream, idx)
        assert 0.0 <= u < 1.0
        assert u == (po.build_draw64(seed, stream, idx) >> 11) / 2.0**53


def _ints(rng, shape, hi=6):
    return rng.integers(0, hi, size=shape).astype(np.float32)


@pytest.mark.parametrize("dtype", [np.uint8, np.float16, np.float32])
def test_assign_equals_integer_brute_force(dtype):
    """Nearest centre = least (|c|^2 - 2 <x, c>, index): on small integers
    the fp32 values are exact, so the ids equal numpy's int64 argmin with
    the lowest index on ties (the data has many)."""
    rng = np.random.default_rng(3)
    x = _ints(rng, (400, 7)).astype(dtype)
    c = _ints(rng, (23, 7), hi=4)
    c[5] = c[2]  # duplicate centres: ties resolve to the lower index
    idx, score = po.build_assign(x, c)
    xi, ci = x.astype(np.int64), c.astype(np.int64)
    s = (ci * ci).sum(1)[None, :] - 2 * xi @ ci.T
    want = s.argmin(1)  # numpy returns the first minimum
    assert np.array_equal(idx, want)
    assert np.array_equal(score, s[np.arange(len(x)), want].astype(np.float32))
    assert not np.any(idx == 5)


def _brute_knn(x, off, k, probe_off=None, probe=None):
    xi = x.astype(np.int64)
    n = len(xi)
    ids = np.full((n, k), U32MAX, np.uint32)
    nb = len(off) - 1
    for b in range(nb):
        buckets = [b] if probe_off is None else probe[probe_off[b]:probe_off[b + 1]]
        cand = np.concatenate([np.zeros(0, np.int64)] +
                              [np.arange(off[q], off[q + 1], dtype=np.int64) for q in buckets])
        for i in range(off[b], off[b + 1]):
            c = cand[cand != i]
            d = ((xi[c] - xi[i]) ** 2).sum(1)
            o = np.lexsort((c, d))[:k]
            ids[i, :len(o)] = c[o]
    return ids


@pytest.mark.parametrize("dtype", [np.uint8, np.float16, np.float32])
def test_knn_equals_integer_brute_force(dtype):
    rng = np.random.default_rng(5)
    off = np.array([0, 1, 40, 40, 150, 151, 260], np.uint32)  # a 1-row, an empty bucket
    x = _ints(rng, (260, 5), hi=4).astype(dtype)
    for k in (1, 6, 60):
        ids, d = po.build_knn(x, off, k)
        assert np.array_equal(ids, _brute_knn(x, off, k))
        valid = ids != U32MAX
        xi = x.astype(np.int64)
        rows = np.nonzero(valid)[0]
        assert np.array_equal(d[valid], ((xi[ids[valid]] - xi[rows]) ** 2).sum(1).astype(np.float32))
    # probe lists: own bucket plus others
    po_ = np.array([0, 2, 3, 3, 5, 6, 8], np.uint32)
    pb = np.array([0, 3, 1, 3, 0, 4, 5, 1], np.uint32)
    ids, _ = po.build_knn(x, off, 9, po_, pb)
    assert np.array_equal(ids, _brute_knn(x, off, 9, po_, pb))


@pytest.mark.parametrize("dtype", [np.uint8, np.float32])
def test_pq_encode_and_training_step_equal_brute_force(dtype):
    rng = np.random.default_rng(7)
    x = _ints(rng, (300, 12), hi=5).astype(dtype)
    c = _ints(rng, (256, 12), hi=5)
    codes = po.build_pq_encode(x, c, 3)
    xi, ci = x.astype(np.int64), c.astype(np.int64)
    for m in range(3):
        sl = slice(4 * m, 4 * m + 4)
        d = ((xi[:, None, sl] - ci[None, :, sl]) ** 2).sum(2)
        assert np.array_equal(codes[:, m], d.argmin(1))
    # one training step: every (subspace, centre) = the fp64 mean of its
    # rows' subvectors (exact sums of integers); empty ones keep
    c1 = po.build_pq_train(x, c, 3, 1)
    want = c.copy()
    for m in range(3):
        sl = slice(4 * m, 4 * m + 4)
        for k in range(256):
            rows = codes[:, m] == k
            if rows.any():
                want[k, sl] = (xi[rows][:, sl].sum(0) / rows.sum()).astype(np.float32)
    assert np.array_equal(c1, want)


def test_kmeans_step_and_kmeanspp_equal_restatement_on_integers():
    rng = np.random.default_rng(9)
    x = _ints(rng, (500, 6), hi=8)
    c = x[:9].copy()
    c1 = po.build_kmeans(x, c, 1)
    idx, _ = po.build_assign(x, c)
    want = c.copy()
    for k in range(9):
        rows = idx == k
        if rows.any():
            want[k] = (x[rows].astype(np.float64).sum(0) / rows.sum()).astype(np.float32)
    assert np.array_equal(c1, want)
    # k-means++: D^2 sampling with the build's draws.  Integer distances and
    # their fp64 sums are exact, so numpy's cumulative sum restates the
    # chunked walk: the pick is the first row whose running sum reaches
    # u * total.
    seed, k = 17, 12
    cen = po.build_kmeanspp(x, k, seed)
    n = len(x)
    xi = x.astype(np.int64)
    pick = min(int(po.build_draw_unit(seed, 0, 0) * n), n - 1)
    picks = [pick]
    best = None
    for j in range(1, k):
        d = ((xi - xi[pick]) ** 2).sum(1).astype(np.float64)
        best = d if best is None else np.minimum(best, d)
        cs = np.cumsum(best)
        u = po.build_draw_unit(seed, 0, j)
        pick = int(np.searchsorted(cs, u * cs[-1], side="left"))
        picks.append(pick)
    assert np.array_equal(cen, x[picks])
    assert len(set(picks)) == k  # D^2 sampling never repeats a chosen row


def test_rabitq_encode_closed_form():
    """Codes: bit d of row i = (xr - c) > 0, MSB-first in u32 words; anchor =
    nearest by |c|^2 - 2 <xr, c>; factors within 1e-5 of the fp64 closed
    form of quantizer_gpu_fast.cu:200-245."""
    rng = np.random.default_rng(11)
    P, A, n = 128, 9, 200
    xr = rng.standard_normal((n, P)).astype(np.float32)
    an = rng.standard_normal((A, P)).astype(np.float32)
    aid, codes, fac = po.build_rabitq_encode(xr, an)
    s = (an.astype(np.float64) ** 2).sum(1)[None, :] - 2 * xr.astype(np.float64) @ an.T.astype(np.float64)
    assert np.mean(aid == s.argmin(1)) > 0.99  # fp32 vs fp64 near-ties only
    c = an[aid].astype(np.float64)
    r = xr.astype(np.float64) - c
    bits = (xr - an[aid]) > 0
    words = codes.view("<u4")
    for i in range(n):
        for d in range(P):
            assert ((words[i, d // 32] >> (31 - d % 32)) & 1) == bits[i, d]
    xu = bits - 0.5
    l2 = (r * r).sum(1)
    ipr = (r * xu).sum(1)
    ipc = (c * xu).sum(1)
    f_add = l2 + 2 * l2 * ipc / ipr
    f_res = -2 * l2 / ipr
    ratio = l2 * (P / 4) / ipr ** 2
    f_err = 2 * np.sqrt(l2) * 1.9 * np.sqrt(np.maximum((ratio - 1) / (P - 1), 0))
    # f_add = l2 + 2 l2 ip_c / ip_r can cancel: the fp32 error is relative
    # to the magnitude of its two terms, not of their sum
    scale = np.abs(l2) + np.abs(2 * l2 * ipc / ipr)
    assert np.all(np.abs(fac[:, 0] - f_add) <= 1e-5 * scale)
    np.testing.assert_allclose(fac[:, 1], f_res, rtol=1e-5)
    np.testing.assert_allclose(fac[:, 2], f_err, rtol=1e-4, atol=1e-6)


def test_medoid_and_bucket_reps_equal_brute_force():
    rng = np.random.default_rng(13)
    x = rng.standard_normal((9000, 5)).astype(np.float32) * 3
    mu = x.astype(np.float64).mean(0)
    d = ((x.astype(np.float64) - mu) ** 2).sum(1)
    assert po.build_medoid(x) == int(d.argmin())
    assert po.build_medoid(x.astype(np.float16)) == int(
        ((x.astype(np.float16).astype(np.float64) - x.astype(np.float16).astype(np.float64).mean(0))
         ** 2).sum(1).argmin())
    off = np.array([0, 1, 700, 2000, 9000], np.uint32)
    means, reps = po.build_bucket_reps(x, off)
    for b in range(4):
        rows = x[off[b]:off[b + 1]].astype(np.float64)
        m = (rows.sum(0) / len(rows)).astype(np.float32)
        assert np.array_equal(means[b], m)
        dd = ((rows - m.astype(np.float64)) ** 2).sum(1)
        assert reps[b] == off[b] + int(dd.argmin())


def test_links_follow_the_rule():
    """The candidate sequence of gofann_build_links, checked piece by piece
    on a small case: knn prefix, own representative, near representatives,
    then the draws (SplitMix64, pinned above), first R distinct non-self."""
    rng = np.random.default_rng(15)
    n, R, nb = 60, 12, 4
    bucket_of = np.repeat(np.arange(nb, dtype=np.uint32), 15)
    order = rng.permutation(n).astype(np.uint32)
    knn = np.stack([rng.choice(np.flatnonzero(bucket_of == bucket_of[i]), 6, replace=False)
                    for i in range(n)]).astype(np.uint32)
    knn[3, 1] = knn[3, 0]  # a repeated candidate
    knn[4, 2] = 4          # the row itself
    knn[5, 3] = U32MAX
    reps = np.array([2, 20, 31, 59], np.uint32)
    near = np.array([[1, 2], [0, 3], [3, 0], [2, 1]], np.uint32)
    seed, entry = 99, 40
    g = po.build_links(knn, bucket_of, reps, near, order, R, 4, 2, 2, 1, entry, seed)
    for i in range(n):
        b = bucket_of[i]
        if i == entry:
            seq = [po.build_draw64(seed, 3, i * 256 + j) % n for j in range(4 * R)]
        elif reps[b] == i:
            seq = list(knn[i, :2]) + [reps[near[b, 0]]] + \
                [po.build_draw64(seed, 2, i * 256 + j) % n for j in range(R)]
        else:
            seq = list(knn[i, :4]) + [reps[b]] + [reps[near[b, j]] for j in range(2)] + \
                [po.build_draw64(seed, 1, i * 256 + j) % n for j in range(R)]
        kept = []
        for v in seq:
            if v != U32MAX and v != i and v < n and v not in kept:
                kept.append(v)
        want = [order[v] for v in kept[:R]] + [U32MAX] * (R - min(R, len(kept)))
        assert g[order[i]].tolist() == want, i


def _detours_by_paths(knn):
    """CAGRA's detour count (Ootomo et al., sec. IV-B) by enumerating every
    two-hop path X -> Z -> Y over the kNN lists: the edge X -> Y at rank j
    gains one detour per Z at rank m of X's list whose list has Y at rank r,
    with max(m, r) < j."""
    n, kin = knn.shape
    det = np.zeros((n, kin), np.int64)
    for x in range(n):
        rank_x = {int(v): j for j, v in reversed(list(enumerate(knn[x]))) if v != U32MAX}
        for m, z in enumerate(knn[x]):
            if z == U32MAX:
                continue
            for r, y in enumerate(knn[z]):
                if y == U32MAX or int(y) not in rank_x:
                    continue
                j = rank_x[int(y)]
                if max(m, r) < j:
                    det[x, j] += 1
    return det


def test_cagra_optimize_equals_paper_definition():
    rng = np.random.default_rng(17)
    n, kin, R = 80, 12, 6
    x = rng.standard_normal((n, 4)).astype(np.float32)
    ids, _ = po.build_knn(x, np.array([0, n], np.uint32), kin)
    ids[7, 5:] = U32MAX  # a short list
    pruned, g = po.build_cagra_optimize(ids, R)
    det = _detours_by_paths(ids)
    for i in range(n):
        valid = [j for j in range(kin) if ids[i, j] != U32MAX]
        keep = sorted(valid, key=lambda j: (det[i, j], j))[:R]
        want = [int(ids[i, j]) for j in keep] + [U32MAX] * (R - len(keep))
        assert pruned[i].tolist() == want, i
    # reverse merge: R/2 protected, then reverse edges by (rank, source),
    # then the rest of the pruned list; no repeats or self
    rev = {v: [] for v in range(n)}
    for u in range(n):
        for k in range(R):
            v = int(pruned[u, k])
            if v != U32MAX:
                rev[v].append((k, u))
    for i in range(n):
        out = []
        f = [int(v) for v in pruned[i]]
        kf = 0
        while kf < R and len(out) < R // 2:
            v = f[kf]
            kf += 1
            if v != U32MAX and v != i and v not in out:
                out.append(v)
        for _, u in sorted(rev[i])[:2 * R]:
            if len(out) < R and u != i and u not in out:
                out.append(u)
        while kf < R and len(out) < R:
            v = f[kf]
            kf += 1
            if v != U32MAX and v != i and v not in out:
                out.append(v)
        assert g[i].tolist() == out + [U32MAX] * (R - len(out)), i


def test_reach_equals_scipy_bfs():
    from scipy.sparse import csr_matrix
    from scipy.sparse.csgraph import breadth_first_order
    rng = np.random.default_rng(19)
    n, R = 300, 3
    g = rng.integers(0, n, size=(n, R)).astype(np.uint32)
    g[rng.random((n, R)) < 0.4] = U32MAX
    reached, cnt = po.build_reach(g, 5)
    rows, cols = np.nonzero(g != U32MAX)
    m = csr_matrix((np.ones(len(rows)), (rows, g[rows, cols].astype(np.int64))), shape=(n, n))
    want = breadth_first_order(m, 5, directed=True, return_predecessors=False)
    assert cnt == len(want)
    assert np.array_equal(np.flatnonzero(reached), np.sort(want))
