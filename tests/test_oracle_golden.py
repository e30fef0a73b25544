"""Pins the oracle against the golden vectors of GO-FANN's own tests
(tests/golden/*.json, transcribed by tests/golden/make_fixtures.py) and,
where oracle/_ref was built from the reference's host-compilable headers,
against those headers on the same inputs."""
from __future__ import annotations

import ctypes as C
import math

import numpy as np
import pytest

import pyoracle as po
from conftest import load_golden

FLT_MAX = np.finfo(np.float32).max
U32MAX = 0xFFFFFFFF


def _f(x):
    return {"inf": math.inf, "-inf": -math.inf, "nan": math.nan}.get(x, x) if isinstance(x, str) else x


def _pred(fx, route_enabled="route_enabled"):
    clauses = None
    ranges = None
    if "clauses" in fx:
        from gofann_amd.plan import CLAUSE_DTYPE, RANGE_DTYPE
        clauses = np.array([tuple(c) for c in fx["clauses"]], dtype=CLAUSE_DTYPE)
        ranges = np.array([tuple(r) for r in fx.get("ranges", [[0, 0, 0, 0]])], dtype=RANGE_DTYPE)
    base = fx.get("base_ranges")
    return po.PredicateArrays(fx.get("route_offsets", [0]), fx.get("handles", [0]), clauses,
                              ranges, fx.get(route_enabled), None, fx["csr_offsets"],
                              fx["csr_labels"], fx["rows"],
                              None if base is None else np.array(base, np.float32))


def _ref_matches(ref, pa: po.PredicateArrays, route, sample):
    a = pa.arrs
    s = pa.struct
    return ref.ref_pred_matches(s.route_offsets, s.route_handles, s.clauses, s.ranges,
                                s.route_enabled, s.base_ranges, s.range_stride, s.csr_offsets,
                                s.csr_labels, s.rows, route, sample)


def test_residual_dnf_fixture():
    fx = load_golden("predicate.json")["residual_dnf"]
    pa = _pred(fx)
    L = po.lib()
    for route, row in enumerate(fx["expected"]):
        for sample, want in enumerate(row):
            assert L.orc_pred_matches(C.byref(pa.struct), route, sample, None) == want
    for route, want in enumerate(fx["enabled"]):
        assert L.orc_pred_enabled(C.byref(pa.struct), route) == want
    for route, sample, want in fx["out_of_range"]:
        assert L.orc_pred_matches(C.byref(pa.struct), route, sample, None) == want
    ref = po.ref()
    if ref is not None:
        for route in range(4):
            for sample in range(4):
                assert _ref_matches(ref, pa, route, sample) == \
                    L.orc_pred_matches(C.byref(pa.struct), route, sample, None)


def _pairs(rows):
    arr = (po.Pair * len(rows))()
    for i, (f, s, b) in enumerate(rows):
        arr[i] = po.Pair(f, s, b)
    return arr


def test_minimum_pending_base_fixture():
    fx = load_golden("predicate.json")["pending_base"]
    L = po.lib()
    for case in fx["cases"]:
        pool = [list(e) for e in fx["pool"]]
        for i in case["mark_used"]:
            pool[i][1] |= 0x80000000
        arr = _pairs(pool)
        got = L.orc_minimum_pending_base(arr, len(pool), po.Pair(*fx["current"]),
                                         po.Pair(*fx["next"]), case["current_valid"],
                                         case["next_valid"])
        assert got == case["expected"]
        ref = po.ref()
        if ref is not None:
            cur = po.Pair(*fx["current"])
            nxt = po.Pair(*fx["next"])
            r = ref.ref_minimum_pending_base(arr, len(pool), C.byref(cur), C.byref(nxt),
                                             case["current_valid"], case["next_valid"])
            assert r == got
    arr = _pairs(fx["compact_pool"])
    rv = po.Pair(*fx["compact_reserved"])
    assert L.orc_minimum_pending_base(arr, 3, rv, rv, 1, 1) == fx["compact_expected"]


def test_csr_original_id_fixture():
    fx = load_golden("predicate.json")["csr_original_ids"]
    off = np.array(fx["csr_offsets"], np.uint32)
    lab = np.array(fx["csr_labels"], np.uint32)
    pa = po.PredicateArrays([0, 1], [0], None, None, None, None, off, lab, fx["rows"])
    L = po.lib()
    assert L.orc_pred_enabled(C.byref(pa.struct), 0) == fx["enabled_route0"]
    for handle, sample, want in fx["probes"]:
        # contains(handle, sample): route with the single handle
        one = po.PredicateArrays([0, 1], [handle], None, None, None, None, off, lab, fx["rows"])
        assert L.orc_pred_matches(C.byref(one.struct), 0, sample, None) == want
        ref = po.ref()
        if ref is not None:
            assert ref.ref_csr_contains(po.p(off), po.p(lab), fx["rows"], handle, sample) == want


def test_membership_fixture():
    fx = load_golden("predicate.json")["membership"]
    pa = _pred(fx, route_enabled="none")
    L = po.lib()
    t0, t1 = set(fx["route0_true"]), set(fx["route1_true"])
    probe = sorted(t0 | t1 | {1, 2, 65534, fx["rows"], fx["rows"] - 1, 40000})
    for s in probe:
        assert L.orc_pred_matches(C.byref(pa.struct), 0, s, None) == (s in t0)
        assert L.orc_pred_matches(C.byref(pa.struct), 1, s, None) == (s in t1)


def test_csr_lookup_cases():
    fx = load_golden("csr_lookup.json")
    off = np.array(fx["csr_offsets"], np.uint32)
    lab = np.array(fx["csr_labels"], np.uint32)
    L = po.lib()
    ref = po.ref()
    for row, key, want in fx["probes"]:
        one = po.PredicateArrays([0, 1], [key], None, None, None, None, off, lab, fx["rows"])
        assert L.orc_pred_matches(C.byref(one.struct), 0, row, None) == want, (row, key)
        if ref is not None:
            assert ref.ref_csr_contains(po.p(off), po.p(lab), fx["rows"], key, row) == want


def test_parallel_fixture_against_reference_headers():
    fx = load_golden("predicate_parallel.json")
    pa = _pred(fx)
    L = po.lib()
    ref = po.ref()
    if ref is None:
        pytest.skip("oracle/_ref not built (reference sources absent)")
    for route in range(len(fx["route_enabled"])):
        for sample in range(fx["rows"] + 1):
            assert L.orc_pred_matches(C.byref(pa.struct), route, sample, None) == \
                _ref_matches(ref, pa, route, sample)
        assert L.orc_pred_enabled(C.byref(pa.struct), route) == fx["route_enabled"][route]


def test_parallel_fixture_closed_form():
    # route 1 = labels {0} with range atom (dim0 > 3) OR labels {1}: checked
    # against the fixture's generating rules directly.
    fx = load_golden("predicate_parallel.json")
    pa = _pred(fx)
    L = po.lib()
    for s in range(fx["rows"] + 1):
        lab0 = s < 67 and s % 2 == 0
        lab1 = s < 67 and s % 3 == 0
        v0 = float(s % 9)
        want1 = (lab0 and v0 > 3) or lab1
        assert L.orc_pred_matches(C.byref(pa.struct), 1, s, None) == int(want1)
        assert L.orc_pred_matches(C.byref(pa.struct), 0, s, None) == int(s < 67)


def _heap_insert_all(cands, k, fn_insert, fn_sort):
    d = np.full(k, FLT_MAX, np.float32)
    ids = np.full(k, U32MAX, np.uint32)
    for dist, i in cands:
        fn_insert(C.c_float(_f(dist)), C.c_uint32(i), po.p(d), po.p(ids), k)
    fn_sort(po.p(d), po.p(ids), k)
    return d, ids


def test_shortlist_heap_fixtures():
    fx = load_golden("shortlist_heap.json")
    L = po.lib()
    L.orc_shortlist_insert.argtypes = [C.c_float, C.c_uint32, C.c_void_p, C.c_void_p, C.c_int]
    L.orc_shortlist_can_enter.argtypes = [C.c_float, C.c_uint32, C.c_void_p, C.c_void_p, C.c_int]
    for case in fx["top_m"]:
        d, ids = _heap_insert_all(case["candidates"], case["k"], L.orc_shortlist_insert,
                                  L.orc_shortlist_sort)
        exp = case["expected"]
        for i, (ed, ei) in enumerate(exp):
            assert d[i] == np.float32(ed) and ids[i] == ei
        assert np.all(d[len(exp):] == FLT_MAX) and np.all(ids[len(exp):] == U32MAX)
    # can_enter table
    d = np.full(2, FLT_MAX, np.float32)
    ids = np.full(2, U32MAX, np.uint32)
    ce = lambda dist, i: L.orc_shortlist_can_enter(C.c_float(_f(dist)), C.c_uint32(i),
                                                   po.p(d), po.p(ids), 2)
    for dist, i, want in fx["can_enter_initial"]:
        assert ce(dist, i) == want
    L.orc_shortlist_insert(C.c_float(2.0), C.c_uint32(9), po.p(d), po.p(ids), 2)
    for dist, i, want in fx["can_enter_after_one"]:
        assert ce(dist, i) == want
    L.orc_shortlist_insert(C.c_float(2.0), C.c_uint32(7), po.p(d), po.p(ids), 2)
    for dist, i, want in fx["can_enter_after_two"]:
        assert ce(dist, i) == want
    ref = po.ref()
    if ref is not None:
        rng = np.random.default_rng(3)
        for k in (1, 2, 5, 64, 400):
            cands = [(float(rng.integers(0, 50)), int(rng.integers(0, 300))) for _ in range(900)]
            a = _heap_insert_all(cands, k, L.orc_shortlist_insert, L.orc_shortlist_sort)
            b = _heap_insert_all(cands, k, ref.ref_shortlist_insert, ref.ref_shortlist_sort)
            assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def test_resident_posting_fixture():
    fx = load_golden("resident_posting.json")
    L = po.lib()
    L.orc_resident_candidate.restype = C.c_uint32
    arr = lambda v, t: np.array([_f(x) for x in v], dtype=t)
    offs, sizes = arr(fx["offsets"], np.uint32), arr(fx["sizes"], np.uint32)
    ids, masks = arr(fx["ids"], np.uint32), arr(fx["masks"], np.uint64)
    groups, qm = arr(fx["groups"], np.uint32), arr(fx["query_masks"], np.uint64)
    modes = arr(fx["modes"], np.uint8)
    lo, hi, vals = arr(fx["lower"], np.float32), arr(fx["upper"], np.float32), arr(fx["values"], np.float32)
    out = []
    for route in fx["probe_routes"]:
        b, c = C.c_uint32(), C.c_uint32()
        L.orc_resident_bounds(po.p(offs), po.p(sizes), po.p(groups), fx["n_groups"], fx["rows"],
                              fx["routes"], route, C.byref(b), C.byref(c))
        for i in range(3):
            if i < c.value:
                out.append(L.orc_resident_candidate(po.p(ids), po.p(masks), po.p(qm), po.p(modes),
                                                    po.p(lo), po.p(hi), po.p(vals), fx["rows"],
                                                    fx["samples"], fx["routes"],
                                                    fx["range_count"], route, b.value + i))
            else:
                out.append(U32MAX)
    assert out == fx["expected"]


def test_route_merge_fixtures():
    fx = load_golden("route_merge.json")
    ref = po.ref()
    for case in fx["cases"]:
        ids = np.array(case["ids"], np.uint32)
        d = np.array(case["dists"], np.float32)
        oi, od = po.merge(np.array(case["route_to_query"], np.uint32), ids, d, case["queries"],
                          case["topk"])
        assert oi.tolist() == case["expected"]
        if "expected_dists" in case:
            assert np.array_equal(od, np.array(case["expected_dists"], np.float32))
        if ref is not None:
            ri = np.empty_like(oi)
            rd = np.empty_like(od)
            r2q = np.array(case["route_to_query"], np.uint32)
            ref.ref_merge_routes(po.p(r2q), len(r2q), case["queries"], po.p(ids), po.p(d),
                                 ids.shape[1], case["topk"], po.p(ri), po.p(rd))
            assert np.array_equal(ri, oi) and np.array_equal(rd, od)


def test_route_merge_random_vs_reference_headers():
    ref = po.ref()
    if ref is None:
        pytest.skip("oracle/_ref not built (reference sources absent)")
    rng = np.random.default_rng(11)
    for trial in range(20):
        routes, width, queries, topk = int(rng.integers(1, 30)), int(rng.integers(1, 12)), \
            int(rng.integers(1, 6)), int(rng.integers(1, 10))
        r2q = rng.integers(0, queries, size=routes).astype(np.uint32)
        ids = rng.integers(0, 40, size=(routes, width)).astype(np.uint32)
        ids[rng.random((routes, width)) < 0.2] = U32MAX
        d = rng.integers(0, 30, size=(routes, width)).astype(np.float32) / 4
        oi, od = po.merge(r2q, ids, d, queries, topk)
        ri, rd = np.empty_like(oi), np.empty_like(od)
        ref.ref_merge_routes(po.p(r2q), routes, queries, po.p(ids), po.p(d), width, topk,
                             po.p(ri), po.p(rd))
        assert np.array_equal(oi, ri) and np.array_equal(od, rd), trial


def test_fp16_fixture():
    fx = load_golden("fp16_l2.json")
    L = po.lib()
    L.orc_l2_f16.argtypes = [C.c_void_p, C.c_void_p, C.c_uint32]
    for case in fx["cases"]:
        q = np.array(case["query"], np.float32)
        for row in case["rows"]:
            b = np.array(row, np.uint16)
            got = L.orc_l2_f16(po.p(q), po.p(b), case["cols"])
            ref64 = float(((q.astype(np.float64) - b.view(np.float16).astype(np.float64)) ** 2).sum())
            assert math.isfinite(got)
            assert abs(got - ref64) <= fx["tolerance"] * max(1.0, ref64)
    q = np.zeros(8, np.float32)
    for value, kind in fx["specials"]:
        b = np.zeros(8, np.uint16)
        b[0] = value
        got = L.orc_l2_f16(po.p(q), po.p(b), 8)
        assert {"inf": math.isinf, "nan": math.isnan, "finite": math.isfinite}[kind](got)
    # every binary16 decodes identically to numpy and to the reference header
    allh = np.arange(65536, dtype=np.uint16)
    mine = np.array([L.orc_half_to_float(int(h)) for h in allh[::97]], np.float32)
    want = allh[::97].view(np.float16).astype(np.float32)
    assert np.array_equal(np.isnan(mine), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(mine[ok].view(np.uint32), want[ok].view(np.uint32))
    ref = po.ref()
    if ref is not None:
        for h in allh[::97]:
            a, b = L.orc_half_to_float(int(h)), ref.ref_fp16_decode(int(h))
            assert (math.isnan(a) and math.isnan(b)) or a == b


def test_priority_and_bonuses_vs_reference_headers():
    L = po.lib()
    ref = po.ref()
    cases = [(1.0, 5.0, 0), (1.0, 5.0, 1), (-3.0, 2.0, 0), (FLT_MAX, 1.0, 0), (float("inf"), 1.0, 0),
             (3.0e38, 1.0e38, 0), (0.5, 0.0, 0), (float("nan"), 1.0, 0)]
    for base, pen, ok in cases:
        s1 = C.c_int(0)
        got = L.orc_priority(base, pen, ok, C.byref(s1))
        if base == 3.0e38:
            assert got == FLT_MAX and s1.value == 1
        if ref is not None:
            s2 = C.c_int(0)
            r = ref.ref_priority(base, pen, ok, C.byref(s2))
            assert (math.isnan(got) and math.isnan(r)) or got == r
            assert s1.value == s2.value
    for args in [(2.0, 1, 2, 0.95, 0.9), (2.0, 0, 0, 0.95, 0.9), (-1.5, 1, 1, 0.5, 2.0)]:
        got = L.orc_apply_filter_bonuses(*args)
        want = np.float32(args[0])
        if args[1]:
            want = np.float32(want * np.float32(args[3]))
        for _ in range(args[2]):
            want = np.float32(want * np.float32(args[4]))
        assert got == want
        if ref is not None:
            assert ref.ref_apply_filter_bonuses(*args) == got
