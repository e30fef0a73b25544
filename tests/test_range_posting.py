"""Range postings on the CPU: the segment plan (library, oracle and the
reference's own make_plan), the FARPIDX1 format and smallest-slice choice
(against the reference test's fixture and, where oracle/_ref is built, the
reference loader itself), and the oracle's range-posting scan and segment
merge against brute force and size-independent invariants."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import pyoracle as po
from conftest import load_golden
from gofann_amd import plan as gp
from gofann_amd import range_posting as rp

U32MAX = 0xFFFFFFFF
FLT_MAX = np.float32(3.4028234663852886e38)


# ---------------------------------------------------------------- segment plan
def _plan_inputs(rng, n):
    sizes = rng.integers(0, 40, n).astype(np.uint64)
    sizes[rng.random(n) < 0.2] = 0
    offsets = rng.integers(0, 10_000, n).astype(np.uint64)
    routes = rng.integers(0, 50, n).astype(np.uint32)
    return routes, offsets, sizes


@pytest.mark.parametrize("target", [1, 3, 7, 16, 64])
def test_segment_plan_library_oracle_reference(hip_lib_path, target):
    rng = np.random.default_rng(target)
    routes, offsets, sizes = _plan_inputs(rng, 60)
    lib = rp.segment_plan(routes, offsets, sizes, target)
    orc = po.segment_plan(routes, offsets, sizes, target)
    got = (lib.route_ids, lib.positions, lib.offsets, lib.sizes, lib.query_indptr)
    for a, b in zip(got, orc):
        assert np.array_equal(a, b)
    ref = po.ref_segment_plan(routes, offsets, sizes, target)
    if ref is not None:
        for a, b in zip(got, ref):
            assert np.array_equal(a, b)
    # Invariants fixed by the plan's definition: each posting is tiled in
    # order by max(1, ceil(size / target)) parts whose sizes differ by <= 1.
    for q in range(routes.size):
        s0, s1 = int(lib.query_indptr[q]), int(lib.query_indptr[q + 1])
        parts = s1 - s0
        assert parts == max(1, -(-int(sizes[q]) // target))
        assert np.all(lib.positions[s0:s1] == q) and np.all(lib.route_ids[s0:s1] == routes[q])
        sz = lib.sizes[s0:s1].astype(np.int64)
        assert sz.sum() == sizes[q] and sz.max() - sz.min() <= 1 and np.all(np.diff(sz) <= 0)
        assert np.all(sz <= target)
        ends = lib.offsets[s0:s1] + lib.sizes[s0:s1]
        assert lib.offsets[s0] == offsets[q] and np.array_equal(lib.offsets[s0 + 1:s1], ends[:-1])


def test_segment_plan_errors(hip_lib_path):
    from gofann_amd import _lib
    L = _lib.load()
    r = np.zeros(1, np.uint32)
    o = np.array([2**64 - 5], np.uint64)
    s = np.array([10], np.uint64)
    cnt = C.c_uint32(0)
    assert L.gofann_posting_segment_plan(r.ctypes.data, o.ctypes.data, s.ctypes.data, 1, 0, 0,
                                         None, None, None, None, None, C.byref(cnt)) == _lib.ERR_INVALID
    assert L.gofann_posting_segment_plan(r.ctypes.data, o.ctypes.data, s.ctypes.data, 1, 4, 0,
                                         None, None, None, None, None, C.byref(cnt)) == _lib.ERR_UNSUPPORTED
    assert po.segment_plan(r, o, s, 4) == -2
    if po.ref_segment_plan(r, np.zeros(1, np.uint64), s, 4) is not None:
        assert po.ref_segment_plan(r, o, s, 4) == -1
    with pytest.raises(rp.RangeIndexError):
        rp.segment_plan(r, np.zeros(1, np.uint64), s, 0)
    # an empty posting list still yields one empty segment per route
    e = rp.segment_plan(np.array([4, 9], np.uint32), np.array([7, 8], np.uint64),
                        np.zeros(2, np.uint64), 16)
    assert e.count == 2 and list(e.sizes) == [0, 0] and list(e.query_indptr) == [0, 1, 2]


# ------------------------------------------------------- FARPIDX1 and slices
def _fixture_index():
    fx = load_golden("range_posting.json")
    dims = [rp.RangeDimension(np.array(d["values"], np.float32), np.array(d["offsets"], np.uint64),
                              np.array(d["ids"], np.uint32)) for d in fx["dimensions"]]
    return fx, rp.RangePostingIndex(len(fx["dimensions"][0]["ids"]), dims)


def _query_table(queries, range_count):
    n = len(queries)
    modes = np.zeros((n, range_count), np.uint8)
    lower = np.zeros((n, range_count), np.float32)
    upper = np.zeros((n, range_count), np.float32)
    for q, atoms in enumerate(queries):
        for (r, m, lo, hi) in atoms:
            modes[q, r], lower[q, r], upper[q, r] = m, lo, hi
    return modes, lower, upper


def test_range_slices_golden(hip_lib_path, tmp_path):
    fx, index = _fixture_index()
    path = tmp_path / "valid.bin"
    index.write(path)
    loaded = rp.RangePostingIndex.load(path)
    assert loaded.row_count == 6 and loaded.range_count == 2
    for a, b in zip(index.dimensions, loaded.dimensions):
        assert np.array_equal(a.unique_values, b.unique_values)
        assert np.array_equal(a.offsets, b.offsets) and np.array_equal(a.sample_ids, b.sample_ids)
    modes, lower, upper = _query_table(fx["queries"], 2)
    got = rp.choose_slices(loaded, modes, lower, upper)
    assert got.tolist() == fx["expected"]
    for threshold, eligible in fx["eligible"]:   # eligible_for_scan (range_posting_index.h:104)
        assert (bool(got[0, 0]) and int(got[0, 4]) <= threshold) == eligible
    ref = po.ref_range_slices(path, modes, lower, upper)
    if ref is not None:
        out, rows = ref
        assert rows == 6 and out.tolist() == fx["expected"]


def _patched(src, dst, mutate):
    data = bytearray(src.read_bytes())
    mutate(data)
    dst.write_bytes(bytes(data))
    return dst


def test_range_index_rejections(hip_lib_path, tmp_path):
    fx, index = _fixture_index()
    valid = tmp_path / "valid.bin"
    index.write(valid)
    hdr = rp.HEADER.size
    desc0 = rp.DESCRIPTOR.unpack_from(valid.read_bytes(), hdr)
    ids_off = desc0[6]

    def bad_magic(d):
        d[0] = ord("X")

    def bad_unique(d):
        C.c_uint64.from_buffer(d, hdr + 8).value = desc0[3] + 1

    def bad_id(d):
        C.c_uint32.from_buffer(d, ids_off + 5 * 4).value = 6

    def dup_id(d):
        C.c_uint32.from_buffer(d, ids_off + 5 * 4).value = C.c_uint32.from_buffer(d, ids_off).value

    def truncated(d):
        del d[-1]

    muts = dict(bad_magic=bad_magic, bad_unique_count=bad_unique, bad_id=bad_id,
                duplicate_id=dup_id, truncated=truncated)
    modes, lower, upper = _query_table([[]], 2)
    for name, needle in fx["rejections"]:
        path = _patched(valid, tmp_path / f"{name}.bin", muts[name])
        with pytest.raises(rp.RangeIndexError, match=needle):
            rp.RangePostingIndex.load(path)
        ref = po.ref_range_slices(path, modes, lower, upper)
        if ref is not None:
            assert ref[0] is None and needle in ref[1]


def test_range_slices_random_vs_brute_force(hip_lib_path, tmp_path):
    rng = np.random.default_rng(5)
    rows, rc, n = 500, 3, 200
    base = rng.integers(0, 40, (rows, rc)).astype(np.float32)
    index = rp.RangePostingIndex.build(base)
    path = tmp_path / "rand.bin"
    index.write(path)
    modes = rng.integers(0, 4, (n, rc)).astype(np.uint8)
    lower = rng.integers(-2, 42, (n, rc)).astype(np.float32)
    upper = lower + rng.integers(-3, 20, (n, rc)).astype(np.float32)
    got = rp.choose_slices(index, modes, lower, upper)
    ref = po.ref_range_slices(path, modes, lower, upper)
    if ref is not None:
        assert np.array_equal(got, ref[0])
    for q in range(n):
        act = [r for r in range(rc) if modes[q, r]]
        assert got[q, 0] == (1 if act else 0) and got[q, 1] == len(act)
        if not act:
            continue
        sizes = {}
        for r in act:
            v = base[:, r]
            m = {1: v > lower[q, r], 2: v < upper[q, r],
                 3: (v >= lower[q, r]) & (v < upper[q, r])}[int(modes[q, r])]
            sizes[r] = (m, int(m.sum()))
        best = min(act, key=lambda r: (sizes[r][1], r))
        assert got[q, 2] == best and got[q, 4] == sizes[best][1]
        b, c = int(got[q, 3]), int(got[q, 4])
        chosen = index.dimensions[best].sample_ids[b:b + c]
        assert set(chosen.tolist()) == set(np.nonzero(sizes[best][0])[0].tolist())


# ---------------------------------------------------------- oracle range scan
def _rq_world(rng, n=400, P=128, A=6, nq=5):
    codes = rng.integers(0, 256, (n, P // 8)).astype(np.uint8)
    fac = rng.standard_normal((n, 3)).astype(np.float32)
    fac[rng.random(n) < 0.03, 0] = np.nan          # inadmissible distances
    aid = rng.integers(0, A, n).astype(np.uint32)
    q8 = rng.integers(-128, 128, (nq, P)).astype(np.int8)
    scale = rng.uniform(0.01, 0.1, nq).astype(np.float32)
    k1 = rng.standard_normal(nq).astype(np.float32)
    cd = rng.uniform(0, 10, (nq, A)).astype(np.float32)
    return codes, fac, aid, q8, scale, k1, cd


def _scores(world, q, samples):
    codes, fac, aid, q8, scale, k1, cd = world
    L = po.lib()
    out = np.empty(len(samples), np.float32)
    for i, s in enumerate(samples):
        ip = po.rabitq_ip(q8[q], codes[s], "int")
        out[i] = L.orc_rabitq_score_b1(ip, scale[q], k1[q], fac[s, 0].item(), fac[s, 1].item(),
                                       cd[q, aid[s]])
    return out


def _range_mask(base, modes, lower, upper, route):
    m = np.ones(base.shape[0], bool)
    for r in range(base.shape[1]):
        mode = int(modes[route, r])
        v = base[:, r]
        if mode == 1:
            m &= v > lower[route, r]
        elif mode == 2:
            m &= v < upper[route, r]
        elif mode == 3:
            m &= (v >= lower[route, r]) & (v < upper[route, r])
    return m


def _scan_case(seed=3, n=400, routes=6, rc=2, with_pred=False):
    rng = np.random.default_rng(seed)
    world = _rq_world(rng, n=n)
    base = rng.integers(0, 20, (n, rc)).astype(np.float32)
    modes = rng.integers(0, 4, (routes, rc)).astype(np.uint8)
    modes[0] = 0                       # a route with no active range
    modes[1] = [3, 3]                  # two active ranges
    for r in range(2, routes):         # the scanned dimension is active elsewhere
        modes[r, r % rc] = max(int(modes[r, r % rc]), 1 + r % 3)
    lower = rng.integers(0, 10, (routes, rc)).astype(np.float32)
    upper = lower + rng.integers(3, 12, (routes, rc)).astype(np.float32)
    index = rp.RangePostingIndex.build(base)
    posting = np.concatenate([d.sample_ids for d in index.dimensions])
    route_query = rng.integers(0, 5, routes).astype(np.uint32)
    # each route scans a slice of dimension r % rc that satisfies its range
    offs, sizes = [], []
    for r in range(routes):
        d = r % rc
        col = base[index.dimensions[d].sample_ids, d]
        if modes[r, d] == 0:
            lo, hi = 0, n
        else:
            sel = _range_mask(base[:, [d]], modes[[r]][:, [d]], lower[[r]][:, [d]],
                              upper[[r]][:, [d]], 0)[index.dimensions[d].sample_ids]
            idx = np.nonzero(sel)[0]
            lo, hi = (int(idx[0]), int(idx[-1]) + 1) if idx.size else (0, 0)
            assert np.all(sel[lo:hi]) and col.size == n
        offs.append(d * n + lo)
        sizes.append(hi - lo)
    pred = None
    if with_pred:
        ranges_per_route = [[(r2, int(modes[r, r2]), float(lower[r, r2]), float(upper[r, r2]))
                             for r2 in range(rc) if modes[r, r2]] for r in range(routes)]
        cp = gp.compile_residuals([[] for _ in range(routes)], ranges_per_route)
        csr_off = np.zeros(n + 1, np.uint32)
        pred = po.PredicateArrays(cp.route_offsets, cp.handles, cp.clauses, cp.ranges, cp.enabled,
                                  cp.compiled, csr_off, np.zeros(1, np.uint32), n, base_ranges=base)
    return dict(world=world, base=base, modes=modes, lower=lower, upper=upper,
                posting=posting, route_query=route_query, offsets=np.array(offs, np.uint64),
                sizes=np.array(sizes, np.uint64), pred=pred, n=n, routes=routes)


def _run_scan(cs, seg_routes, seg_off, seg_size, k, score_first=False, resident=None,
              base_rows=None):
    w = cs["world"]
    return po.rabitq_range_scan(cs["pred"], cs["modes"], cs["lower"], cs["upper"], cs["base"],
                                w[0], w[1], w[2], w[3], w[4], w[5], w[6], cs["route_query"],
                                cs["posting"], cs["posting"].size if resident is None else resident,
                                cs["n"] if base_rows is None else base_rows, seg_routes, seg_off,
                                seg_size, k, score_first)


@pytest.mark.parametrize("with_pred", [False, True])
@pytest.mark.parametrize("k", [1, 7, 40])
def test_oracle_range_scan_brute_force(with_pred, k):
    cs = _scan_case(with_pred=with_pred)
    routes = np.arange(cs["routes"], dtype=np.uint32)
    ids, dists, passes = _run_scan(cs, routes, cs["offsets"], cs["sizes"], k)
    for r in range(cs["routes"]):
        rows = cs["posting"][int(cs["offsets"][r]):int(cs["offsets"][r] + cs["sizes"][r])]
        active = int((cs["modes"][r] != 0).sum())
        if active == 0:
            keep = np.zeros(rows.size, bool)
        elif with_pred or active > 1:
            keep = _range_mask(cs["base"], cs["modes"], cs["lower"], cs["upper"], r)[rows]
        else:
            keep = np.ones(rows.size, bool)   # the slice satisfies the single range
        cand = rows[keep]
        assert passes[r] == cand.size
        d = _scores(cs["world"], int(cs["route_query"][r]), cand)
        ok = ~np.isnan(d) & (d <= FLT_MAX)
        order = np.lexsort((cand[ok], d[ok]))[:k]
        want_ids = np.full(k, U32MAX, np.uint32)
        want_d = np.full(k, FLT_MAX, np.float32)
        want_ids[:order.size] = cand[ok][order]
        want_d[:order.size] = d[ok][order]
        assert np.array_equal(ids[r], want_ids)
        assert np.array_equal(dists[r].view(np.uint32), want_d.view(np.uint32))


def _prefix_entries(cs, r, k):
    """Rows of route r that enter a k-slot heap at their scan position: an
    admitted row enters iff fewer than k earlier admitted rows are <= it."""
    rows = cs["posting"][int(cs["offsets"][r]):int(cs["offsets"][r] + cs["sizes"][r])]
    if not (cs["modes"][r] != 0).any():
        return 0
    keep = _range_mask(cs["base"], cs["modes"], cs["lower"], cs["upper"], r)[rows]
    d = _scores(cs["world"], int(cs["route_query"][r]), rows)
    adm = keep & ~np.isnan(d) & (d <= FLT_MAX)
    seen = []
    entered = 0
    for i in np.nonzero(adm)[0]:
        key = (float(d[i]), int(rows[i]))
        if sum(1 for e in seen if e <= key) < k:
            entered += 1
        seen.append(key)
    return entered


@pytest.mark.parametrize("k", [1, 5, 30])
def test_oracle_range_scan_score_first(k):
    cs = _scan_case(seed=9, with_pred=True)
    routes = np.arange(cs["routes"], dtype=np.uint32)
    fi, fd, fp = _run_scan(cs, routes, cs["offsets"], cs["sizes"], k, score_first=False)
    si, sd, sp = _run_scan(cs, routes, cs["offsets"], cs["sizes"], k, score_first=True)
    assert np.array_equal(fi, si) and np.array_equal(fd.view(np.uint32), sd.view(np.uint32))
    for r in range(cs["routes"]):
        assert sp[r] == _prefix_entries(cs, r, k)
        assert sp[r] <= fp[r]


@pytest.mark.parametrize("target", [1, 9, 64, 1000])
@pytest.mark.parametrize("score_first", [False, True])
def test_oracle_segments_merge_to_the_unsegmented_scan(target, score_first):
    cs = _scan_case(seed=21, with_pred=True)
    k = 12
    routes = np.arange(cs["routes"], dtype=np.uint32)
    ui, ud, up = _run_scan(cs, routes, cs["offsets"], cs["sizes"], k, score_first)
    plan = po.segment_plan(routes, cs["offsets"], cs["sizes"], target)
    si, sd, sp = _run_scan(cs, plan[0], plan[2], plan[3], k, score_first)
    mi, md, mp = po.merge_segments(plan[4], si, sd, sp, k)
    assert np.array_equal(mi, ui) and np.array_equal(md.view(np.uint32), ud.view(np.uint32))
    if not score_first:
        assert np.array_equal(mp, up)
    else:  # each segment starts with an empty heap: at least as many entries
        assert np.all(mp >= up)


def test_oracle_range_scan_clipping():
    cs = _scan_case(seed=4)
    k = 10
    routes = np.arange(cs["routes"], dtype=np.uint32)
    full_i, _, full_p = _run_scan(cs, routes, cs["offsets"], cs["sizes"], k)
    # rows past resident_rows are never read
    cut = int(cs["offsets"][2] + cs["sizes"][2] // 2)
    ci, _, cp = _run_scan(cs, routes, cs["offsets"], cs["sizes"], k, resident=cut)
    off = cs["offsets"].copy()
    sz = np.minimum(cs["sizes"], np.maximum(0, cut - off.astype(np.int64)).astype(np.uint64))
    wi, _, wp = _run_scan(cs, routes, off, sz, k)
    assert np.array_equal(ci, wi) and np.array_equal(cp, wp)
    # samples >= base_rows are skipped
    lim = cs["n"] // 2
    bi, _, _ = _run_scan(cs, routes, cs["offsets"], cs["sizes"], k, base_rows=lim)
    assert np.all((bi == U32MAX) | (bi < lim))
    assert full_p[0] == 0 and np.all(full_i[0] == U32MAX)   # no active range


def test_share_plan_groups_segments_that_scan_the_same_rows():
    """share_plan: every plan segment lands in exactly one item; an item's
    segments scan the same rows (equal offset and size); at most 16 per
    item; heavier items (rows x segments) first."""
    from gofann_amd import range_posting as rp
    rng = np.random.default_rng(5)
    # 40 routes over 7 labels of different posting sizes, cut at 300 rows
    lab_off = np.array([0, 50, 1250, 1260, 4000, 4001, 9000, 9500], np.uint64)
    labels = rng.choice([0, 2, 3, 4, 5, 6], 40)
    labels[:20] = 1  # one label (1200 rows, 4 segments) scanned by 20 routes
    off = lab_off[labels]
    size = lab_off[labels + 1] - lab_off[labels]
    plan = rp.segment_plan(np.arange(40), off, size, 300)
    sp = rp.share_plan(plan)
    assert sp.begin[0] == 0 and sp.begin[-1] == plan.count
    assert np.array_equal(np.sort(sp.slots), np.arange(plan.count))
    counts = np.diff(sp.begin.astype(np.int64))
    assert counts.min() >= 1 and counts.max() <= rp.SHARE_ROUTES
    for i in range(sp.items):
        sl = sp.slots[sp.begin[i]:sp.begin[i + 1]]
        assert np.all(plan.offsets[sl] == sp.offsets[i]) and np.all(plan.sizes[sl] == sp.sizes[i])
    w = sp.sizes.astype(np.float64) * counts
    assert np.all(np.diff(w) <= 0)
    # per segment of the shared label, its 20 routes split into items of 16 and 4
    big = [i for i in range(sp.items) if lab_off[1] <= sp.offsets[i] < lab_off[2]]
    assert sorted(counts[big].tolist()) == [4] * 4 + [16] * 4
    assert sorted(set(sp.offsets[big].tolist())) == [50, 350, 650, 950]


def test_share_plan_rejects_route_counts_outside_the_kernel_slots():
    """share_plan holds items to 1..SHARE_ROUTES routes (the shared scan's
    route slots per pass over an item's rows)."""
    from gofann_amd import range_posting as rp
    plan = rp.segment_plan(np.arange(4), np.zeros(4, np.uint64), np.full(4, 100, np.uint64), 64)
    for bad in (0, rp.SHARE_ROUTES + 1, 17, -3):
        with pytest.raises(ValueError):
            rp.share_plan(plan, bad)
    for ok in (1, 5, rp.SHARE_ROUTES):
        sp = rp.share_plan(plan, ok)
        assert np.diff(sp.begin.astype(np.int64)).max() <= ok

