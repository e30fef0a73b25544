"""Pins of the oracle's posting scans, RaBitQ query factors and score, and the
RaBitQ encoder, each by brute force or a closed form that a plausible mistake
(a dropped term, a wrong sign, a reordered reduction, LSB-first packing)
would fail."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest
import torch

import pyoracle as po
from gofann_amd import index as gi
from gofann_amd import plan as gp

# the index is built by the oracle's restatement of the GPU build (no GPU here)
CPU_BUILD = po.OracleBuild()

U32MAX = 0xFFFFFFFF


def _world(seed, n=2500, labels=6, routes=24):
    rng = np.random.default_rng(seed)
    counts = rng.integers(0, 4, n)
    rows = [np.sort(rng.choice(labels, c, replace=False)) for c in counts]
    csr_off = np.zeros(n + 1, np.uint32)
    np.cumsum([len(r) for r in rows], out=csr_off[1:])
    csr_lab = np.concatenate(rows).astype(np.uint32) if csr_off[-1] else np.zeros(1, np.uint32)
    residual = [sorted(rng.choice(labels, int(rng.integers(0, 3)), replace=False).tolist())
                for _ in range(routes)]
    comp = gp.compile_residuals(residual, [[] for _ in range(routes)])
    enabled = (rng.random(routes) < 0.85).astype(np.uint8)
    pred = po.PredicateArrays(comp.route_offsets, comp.handles, comp.clauses, comp.ranges,
                              enabled, comp.compiled, csr_off, csr_lab, n)
    sizes = rng.integers(0, 400, routes).astype(np.uint32)
    sizes[0] = 0
    offs = np.zeros(routes, np.uint32)
    offs[1:] = np.cumsum(sizes)[:-1]
    cand = []
    for r in range(routes):
        c = rng.choice(n, int(sizes[r]), replace=False).astype(np.uint32)
        if len(c) > 3:
            c[rng.integers(0, len(c), 2)] = U32MAX  # empty posting slots
        cand.append(c)
    cand = np.concatenate(cand) if sizes.sum() else np.zeros(1, np.uint32)
    return rng, pred, rows, residual, enabled, cand, offs, sizes


def _passes(rows, residual, enabled, r, s):
    """Route r's residual is a conjunction of labels (one clause)."""
    if not enabled[r]:
        return True
    return all(l in rows[s] for l in residual[r])


def _expect(scores_of, rows, residual, enabled, cand, offs, sizes, k, r):
    c = cand[offs[r]:offs[r] + sizes[r]]
    c = c[c != U32MAX]
    ok = np.array([_passes(rows, residual, enabled, r, int(s)) for s in c], bool)
    keep = c[ok]
    d = scores_of(keep)
    order = np.lexsort((keep, d))[:k]
    ids = np.full(k, U32MAX, np.uint32)
    dd = np.full(k, np.finfo(np.float32).max, np.float32)
    ids[:len(order)] = keep[order]
    dd[:len(order)] = d[order]
    return ids, dd, int(ok.sum()) if enabled[r] else 0


@pytest.mark.parametrize("score_first", [False, True])
@pytest.mark.parametrize("k", [1, 10, 37])
def test_pq_posting_scan_brute_force(score_first, k):
    """lowfreq_pq_scan_kernel (backend_pq.cu:2046-2133): the shortlist is the
    k least (ADC distance, id) pairs among the route's valid candidates that
    pass its predicate, whichever order (filter-first or score-first) the
    predicate is consulted in.  ADC here: the serial table (per-subspace sum
    in ascending subspace order, float32)."""
    rng, pred, rows, residual, enabled, cand, offs, sizes = _world(31 + k)
    n, dim, M = len(rows), 32, 8
    codes = rng.integers(0, 256, (n, M), dtype=np.uint8)
    table = rng.normal(0, 3, (256, dim)).astype(np.float32)
    queries = rng.integers(0, 256, (5, dim), dtype=np.uint8)
    rq = rng.integers(0, 5, len(sizes)).astype(np.uint32)
    ids, dists, passes = po.posting_scan_pq(pred, codes, table, queries, rq, cand, offs, sizes,
                                            k, score_first=score_first)
    for r in range(len(sizes)):
        lut = po.pq_lut(table, queries[rq[r]], M).reshape(M, 256)

        def adc(keep):
            if len(keep) == 0:
                return np.zeros(0, np.float32)
            terms = lut[np.arange(M)[None, :], codes[keep].astype(np.int64)]
            return np.cumsum(terms, axis=1, dtype=np.float32)[:, -1]

        ei, ed, ep = _expect(adc, rows, residual, enabled, cand, offs, sizes, k, r)
        assert np.array_equal(ids[r], ei), r
        assert np.array_equal(dists[r].view(np.uint32), ed.view(np.uint32)), r
        assert passes[r] == (0 if score_first else ep), r


@pytest.mark.parametrize("k", [1, 10, 64])
def test_rabitq_posting_scan_brute_force(k):
    """lowfreq_rabitq_resident_posting_kernel (backend_rabitq.cu:5494-5682),
    filter-first: the k least (score, id) pairs among passing candidates,
    pass count = passing candidates of an enabled route."""
    rng, pred, rows, residual, enabled, cand, offs, sizes = _world(71 + k)
    n, P, A, nq = len(rows), 128, 7, 5
    codes = rng.integers(0, 256, (n, P // 8), dtype=np.uint8)
    factors = rng.normal(0, 2, (n, 3)).astype(np.float32)
    aid = rng.integers(0, A, n).astype(np.uint32)
    q8 = rng.integers(-127, 128, (nq, P)).astype(np.int8)
    scale = rng.uniform(0.001, 0.05, nq).astype(np.float32)
    k1 = rng.normal(0, 1, nq).astype(np.float32)
    cdist = rng.uniform(0, 4, (nq, A)).astype(np.float32)
    rq = rng.integers(0, nq, len(sizes)).astype(np.uint32)
    ids, dists, passes = po.posting_scan_rabitq(pred, codes, factors, aid, q8, scale, k1, cdist,
                                                rq, cand, offs, sizes, k)
    L = po.lib()
    for r in range(len(sizes)):
        q = int(rq[r])

        def score(keep):
            out = np.empty(len(keep), np.float32)
            for i, s in enumerate(keep):
                ip = po.rabitq_ip(q8[q], codes[s], "popcount")
                out[i] = L.orc_rabitq_score_b1(ip, float(scale[q]), float(k1[q]),
                                               float(factors[s, 0]), float(factors[s, 1]),
                                               float(cdist[q, aid[s]]))
            return out

        ei, ed, ep = _expect(score, rows, residual, enabled, cand, offs, sizes, k, r)
        assert np.array_equal(ids[r], ei), r
        assert np.array_equal(dists[r].view(np.uint32), ed.view(np.uint32)), r
        assert passes[r] == ep, r


def _block256_sum_f32(row):
    """compute_rabitq_query_factors_kernel's reduction (backend_rabitq.cu:
    2908-2922), stated independently: thread t accumulates row[t::256] in
    order in float32, then a shared-memory tree halves 256 partials."""
    part = np.zeros(256, np.float32)
    for t in range(256):
        acc = np.float32(0)
        for v in row[t::256]:
            acc = np.float32(acc + v)
        part[t] = acc
    stride = 128
    while stride:
        part[:stride] = (part[:stride] + part[stride:2 * stride]).astype(np.float32)
        stride //= 2
    return part[0]


@pytest.mark.parametrize("P", [64, 256, 320, 1024, 4096])
def test_rabitq_query_factors_block_reduce(P):
    L = po.lib()
    rng = np.random.default_rng(P)
    for trial in range(4):
        row = (rng.normal(0, 1, P) * (10.0 ** rng.integers(-3, 3))).astype(np.float32)
        k1, kb = C.c_float(), C.c_float()
        L.orc_rabitq_query_factors(po.p(row), C.c_uint32(P), C.byref(k1), C.byref(kb))
        want = np.float32(_block256_sum_f32(row) * np.float32(-0.5))
        assert np.float32(k1.value).view(np.uint32) == want.view(np.uint32)
        # one bit per dimension: (2^(ex_bits + 1) - 1) / 2 = 1/2, so kb == k1
        assert np.float32(kb.value).view(np.uint32) == want.view(np.uint32)
        exact = -0.5 * float(np.sum(row.astype(np.float64)))
        assert abs(k1.value - exact) <= 1e-5 * np.abs(row).astype(np.float64).sum() + 1e-30


def test_rabitq_score_b1_closed_form():
    """score_rabitq_code_device with ex_bits = 0 (backend_rabitq.cu:3186-3190):
    f_add + g + f_rescale * (ip_int * scale + k1), the product-sum fused."""
    L = po.lib()
    rng = np.random.default_rng(3)
    fused_miss = unfused_miss = 0
    trials = 4000
    for _ in range(trials):
        ip = int(rng.integers(-200000, 200000))
        sc, k1, fa, fr, g = [float(np.float32(v)) for v in rng.normal(0, 3, 5)]
        got = np.float32(L.orc_rabitq_score_b1(ip, sc, k1, fa, fr, g))
        short = np.float32(np.float32(ip) * np.float32(sc))
        t = np.float32(short + np.float32(k1))
        base = np.float32(np.float32(fa) + np.float32(g))
        # fma: one rounding of the exact product-sum (float64 holds the
        # 48-bit product exactly; the sum rounds twice only in rare cases)
        fused = np.float32(np.float64(fr) * np.float64(t) + np.float64(base))
        unfused = np.float32(np.float32(np.float32(fr) * t) + base)
        fused_miss += int(got.view(np.uint32) != fused.view(np.uint32))
        unfused_miss += int(got.view(np.uint32) != unfused.view(np.uint32))
        exact = fa + g + fr * (ip * sc + k1)
        assert abs(float(got) - exact) <= 1e-4 * (abs(fa) + abs(g) + abs(fr * (ip * sc + k1))) + 1e-6
    assert fused_miss <= trials // 1000
    assert unfused_miss > trials // 100  # the test can tell the two apart


@pytest.mark.parametrize("dim,P", [(64, 64), (100, 128), (192, 192), (256, 512)])
def test_rabitq_encode_closed_form(dim, P):
    """index.rabitq_encode against quantizer_gpu_fast.cu:207-262 in float64:
    anchor = nearest rotated centre, residual r = x R - c, bit d = r[d] > 0
    packed MSB-first (bit 31 - d % 32 of little-endian word d / 32),
    f_add = |r|^2 + 2 |r|^2 <c, xu> / <r, xu>, f_rescale = -2 |r|^2 / <r, xu>,
    f_err = 2 * 1.9 |r| sqrt(max(0, (|r|^2 |xu|^2 / <r, xu>^2 - 1) / (P - 1)))."""
    rng = np.random.default_rng(dim)
    n, A = 600, 9
    cen = rng.normal(0, 1, (A, dim)).astype(np.float32)
    x = (cen[rng.integers(0, A, n)] + 0.4 * rng.normal(0, 1, (n, dim))).astype(np.float32)
    rot = gi.random_rotation(dim, P, 11 + dim, "cpu")
    codes, fac, aid, anchors = gi.rabitq_encode(torch.from_numpy(x), rot, torch.from_numpy(cen),
                                                 backend=CPU_BUILD)
    codes, fac, aid, anchors = codes.numpy(), fac.numpy(), aid.numpy(), anchors.numpy()
    R = rot.numpy().astype(np.float64)
    xr = x.astype(np.float64) @ R
    an = cen.astype(np.float64) @ R
    assert np.allclose(anchors, an, rtol=1e-5, atol=1e-5)
    d2 = ((xr[:, None, :] - an[None, :, :]) ** 2).sum(-1)
    want_a = d2.argmin(1)
    srt = np.sort(d2, 1)
    clear = srt[:, 1] - srt[:, 0] > 1e-3 * srt[:, 1]
    assert np.array_equal(aid[clear], want_a[clear])
    c = an[aid]
    r = xr - c
    bits = (r > 0)
    words = codes.reshape(n, P // 32, 4).astype(np.uint32)
    words = words[..., 0] | (words[..., 1] << 8) | (words[..., 2] << 16) | (words[..., 3] << 24)
    got_bits = ((words[:, :, None] >> (31 - np.arange(32))[None, None, :]) & 1).reshape(n, P)
    sure = np.abs(r) > 1e-4 * np.abs(r).max(1, keepdims=True)
    assert np.array_equal(got_bits.astype(bool)[sure], bits[sure])
    xu = got_bits.astype(np.float64) - 0.5
    l2 = (r * r).sum(1)
    ip_r = (r * xu).sum(1)
    ip_c = (c * xu).sum(1)
    f_add = l2 + 2 * l2 * ip_c / ip_r
    f_rescale = -2 * l2 / ip_r
    ratio = l2 * (xu * xu).sum(1) / ip_r ** 2
    f_err = 2 * np.sqrt(l2) * 1.9 * np.sqrt(np.maximum((ratio - 1) / max(P - 1, 1), 0))
    scale = np.abs(l2) + np.abs(2 * l2 * ip_c / ip_r)
    assert np.all(np.abs(fac[:, 0] - f_add) <= 2e-4 * scale + 1e-5)
    assert np.allclose(fac[:, 1], f_rescale, rtol=2e-4, atol=1e-6)
    assert np.allclose(fac[:, 2], f_err, rtol=2e-3, atol=1e-5)
