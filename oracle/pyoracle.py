"""ctypes front-end of the CPU oracle (oracle/libgofann_oracle.so) and of the
reference-header checker (oracle/_ref/libgofann_ref.so).

TEST INFRASTRUCTURE ONLY.  Importable from tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg; the product path never imports it.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "libgofann_oracle.so"
REF_LIB = HERE / "_ref" / "libgofann_ref.so"

P = C.c_void_p
U32 = C.c_uint32


class Pair(C.Structure):
    _fields_ = [("first", C.c_float), ("second", C.c_uint32), ("base", C.c_float)]


class Predicate(C.Structure):
    _fields_ = [("route_offsets", P), ("route_handles", P), ("clauses", P), ("ranges", P),
                ("route_enabled", P), ("route_compiled", P), ("base_ranges", P),
                ("csr_offsets", P), ("csr_labels", P), ("rows", U32), ("range_stride", U32),
                ("alpha", C.c_float), ("pending_base_stop", C.c_int)]


class PredCounters(C.Structure):
    _fields_ = [("rows_checked", C.c_uint64), ("label_words", C.c_uint64),
                ("range_values", C.c_uint64)]


class Graph(C.Structure):
    _fields_ = [("graph", P), ("degree", U32), ("row_to_sample", P), ("label_offset", P),
                ("route_group", P), ("route_start", P), ("row_filter_mask", P),
                ("query_filter_bits", P), ("range_modes", P), ("range_lower", P),
                ("range_upper", P), ("base_range_values", P), ("range_count", U32)]


class Params(C.Structure):
    _fields_ = [("queue_limit", C.c_int), ("finish_limit", C.c_int),
                ("early_stop_mode", C.c_int), ("max_steps", C.c_int), ("stop_width", C.c_int),
                ("result_width", C.c_int), ("bit_filter_bonus", C.c_float),
                ("range_filter_bonus", C.c_float), ("bias", C.c_int),
                ("rabitq_verdict", C.c_int), ("inline_exact", C.c_int)]


class Stats(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("steps", "expanded", "passed", "scored", "pred_rows",
                                          "pred_labels", "admitted", "exhausted")]


_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            raise RuntimeError(f"{LIB} missing: run make -C oracle")
        _lib = C.CDLL(str(LIB))
        _lib.orc_hash_code.restype = U32
        _lib.orc_hash_test.restype = C.c_int
        _lib.orc_smmh2_pop_max.restype = Pair
        _lib.orc_smmh2_pop_min.restype = Pair
        _lib.orc_smmh2_insert.argtypes = [P, C.POINTER(C.c_int), Pair]
        _lib.orc_smmh2_pop_max.argtypes = [P, C.POINTER(C.c_int)]
        _lib.orc_smmh2_pop_min.argtypes = [P, C.POINTER(C.c_int)]
        for name in ("orc_pq_adc", "orc_priority", "orc_bias_penalty", "orc_rabitq_score_b1",
                     "orc_l2_u8", "orc_l2_f32", "orc_l2_f16", "orc_half_to_float",
                     "orc_minimum_pending_base", "orc_apply_filter_bonuses", "orc_l2_w32",
                     "orc_l2_serial"):
            getattr(_lib, name).restype = C.c_float
        _lib.orc_l2_w32.argtypes = [P, P, C.c_int, U32]
        _lib.orc_l2_serial.argtypes = [P, P, C.c_int, U32]
        _lib.orc_priority.argtypes = [C.c_float, C.c_float, C.c_int, P]
        _lib.orc_bias_penalty.argtypes = [C.c_float, C.c_float]
        _lib.orc_rabitq_score_b1.argtypes = [C.c_int32, C.c_float, C.c_float, C.c_float,
                                             C.c_float, C.c_float]
        _lib.orc_half_to_float.argtypes = [C.c_uint16]
        _lib.orc_minimum_pending_base.argtypes = [P, C.c_int, Pair, Pair, C.c_int, C.c_int]
        _lib.orc_apply_filter_bonuses.argtypes = [C.c_float, C.c_int, U32, C.c_float, C.c_float]
        _lib.orc_rabitq_ip_int.restype = C.c_int32
        _lib.orc_rabitq_ip_popcount.restype = C.c_int32
        _lib.orc_rabitq_ip_dp4a.restype = C.c_int32
        _lib.orc_range_matches.argtypes = [U32, C.c_float, C.c_float, C.c_float]
        _lib.orc_csr_contains.argtypes = [P, U32, U32, U32, P]
        _lib.orc_pred_matches.argtypes = [C.POINTER(Predicate), U32, U32, P]
        _lib.orc_pred_enabled.argtypes = [C.POINTER(Predicate), U32]
    return _lib


BASELINE_LIB = HERE / "libgofann_cpu_baseline.so"
_baseline = None


def baseline_lib():
    """The oracle's batch drivers over all host cores (cpu_baseline.c)."""
    global _baseline
    if _baseline is None:
        if not BASELINE_LIB.exists():
            raise RuntimeError(f"{BASELINE_LIB} missing: run make -C oracle")
        _baseline = C.CDLL(str(BASELINE_LIB))
    return _baseline


def _drive(name, *args, threads=None):
    """orc_<name>(*args) on one core, or cbl_<name>(*args, threads) on
    `threads` host cores (0 = OpenMP's default); the results are the same."""
    if threads is None:
        return getattr(lib(), "orc_" + name)(*args)
    return getattr(baseline_lib(), "cbl_" + name)(*args, C.c_int(int(threads)))


def ref():
    """Reference-header checker, or None when oracle/_ref was not built."""
    global _ref
    if _ref is None:
        if not REF_LIB.exists():
            return None
        _ref = C.CDLL(str(REF_LIB))
        _ref.ref_priority.restype = C.c_float
        _ref.ref_priority.argtypes = [C.c_float, C.c_float, C.c_int, P]
        _ref.ref_minimum_pending_base.restype = C.c_float
        _ref.ref_apply_filter_bonuses.restype = C.c_float
        _ref.ref_apply_filter_bonuses.argtypes = [C.c_float, C.c_int, U32, C.c_float, C.c_float]
        _ref.ref_fp16_decode.restype = C.c_float
        _ref.ref_fp16_decode.argtypes = [C.c_uint16]
        _ref.ref_fp16_l2_scalar.restype = C.c_float
        _ref.ref_pred_matches.argtypes = [P, P, P, P, P, P, U32, P, P, U32, U32, U32]
        _ref.ref_pred_enabled.argtypes = [P, P, P, U32]
        _ref.ref_csr_contains.argtypes = [P, P, U32, U32, U32]
        _ref.ref_minimum_pending_base.argtypes = [P, C.c_int, P, P, C.c_int, C.c_int]
        _ref.ref_merge_routes.argtypes = [P, U32, U32, P, P, U32, U32, P, P]
        _ref.ref_fp16_l2_scalar.argtypes = [P, P, U32]
        _ref.ref_shortlist_sort.argtypes = [P, P, C.c_int]
        _ref.ref_shortlist_insert.argtypes = [C.c_float, U32, P, P, C.c_int]
        _ref.ref_shortlist_can_enter.argtypes = [C.c_float, U32, P, P, C.c_int]
    return _ref


def p(a):
    """Address of a numpy array (None passes through)."""
    if a is None:
        return None
    return a.ctypes.data_as(C.c_void_p)


def c_arr(a, dtype):
    if a is None:
        return None
    return np.ascontiguousarray(a, dtype=dtype)


class PredicateArrays:
    """Keeps numpy buffers alive behind a Predicate struct."""

    def __init__(self, route_offsets, handles, clauses, ranges, enabled, compiled,
                 csr_offsets, csr_labels, rows, base_ranges=None, alpha=0.0,
                 pending_base_stop=False):
        self.arrs = dict(
            route_offsets=c_arr(route_offsets, np.uint32), handles=c_arr(handles, np.uint32),
            clauses=None if clauses is None else np.ascontiguousarray(clauses),
            ranges=None if ranges is None else np.ascontiguousarray(ranges),
            enabled=c_arr(enabled, np.uint8), compiled=c_arr(compiled, np.uint8),
            csr_offsets=c_arr(csr_offsets, np.uint32), csr_labels=c_arr(csr_labels, np.uint32),
            base_ranges=c_arr(base_ranges, np.float32))
        a = self.arrs
        stride = 0 if base_ranges is None else int(np.asarray(base_ranges).shape[1])
        self.struct = Predicate(p(a["route_offsets"]), p(a["handles"]), p(a["clauses"]),
                                p(a["ranges"]), p(a["enabled"]), p(a["compiled"]),
                                p(a["base_ranges"]), p(a["csr_offsets"]), p(a["csr_labels"]),
                                rows, stride, alpha, 1 if pending_base_stop else 0)

    @classmethod
    def from_plan(cls, compiled, index, base_ranges=None, alpha=0.0, pending_base_stop=False):
        return cls(compiled.route_offsets, compiled.handles, compiled.clauses, compiled.ranges,
                   compiled.enabled, compiled.compiled, index.csr_offsets, index.csr_labels,
                   int(index.csr_offsets.shape[0] - 1), base_ranges, alpha, pending_base_stop)


def params(queue_limit=64, result_width=100, early_stop_mode=2, finish_limit=1, max_steps=0,
           stop_width=10, bias=True, bit_bonus=1.0, range_bonus=1.0, rabitq_verdict=0,
           inline_exact=False) -> Params:
    return Params(queue_limit, finish_limit, early_stop_mode, max_steps, stop_width,
                  result_width, bit_bonus, range_bonus, 1 if bias else 0, rabitq_verdict,
                  1 if inline_exact else 0)


def graph_struct(index, route_group, route_start):
    keep = dict(graph=c_arr(index.graph.reshape(-1), np.uint32),
                r2s=c_arr(index.row_to_sample, np.uint32),
                lo=c_arr(index.label_offset, np.uint32),
                rg=c_arr(route_group, np.uint32), rs=c_arr(route_start, np.uint32))
    g = Graph(p(keep["graph"]), index.degree, p(keep["r2s"]), p(keep["lo"]), p(keep["rg"]),
              p(keep["rs"]), None, None, None, None, None, None, 0)
    return g, keep


def pq_search(index, routes, pred: PredicateArrays, prm: Params, codes, table, queries,
              base=None, threads=None):
    """Oracle beam search of every route.  Returns ids [R][W] u32,
    dists [R][W] f32, stats structured array."""
    L = lib()
    g, keep = graph_struct(index, routes.route_group, routes.route_start)
    n = routes.count
    W = prm.result_width
    ids = np.empty((n, W), np.uint32)
    dists = np.empty((n, W), np.float32)
    stats = (Stats * max(n, 1))()
    codes = c_arr(codes, np.uint8)
    table = c_arr(table, np.float32)
    qf = queries.dtype == np.float32
    q = np.ascontiguousarray(queries)
    rq = c_arr(routes.route_query, np.uint32)
    b = None if base is None else np.ascontiguousarray(base)
    rc = _drive("pq_search_batch", C.byref(g), C.byref(pred.struct), C.byref(prm), p(codes),
                               p(table), p(q), 1 if qf else 0, p(b), p(rq), int(table.shape[1]),
                               int(codes.shape[1]), n, p(ids), p(dists), stats, threads=threads)
    assert rc == 0
    return ids, dists, stats_array(stats, n)


def rabitq_search(index, routes, pred: PredicateArrays, prm: Params, codes, factors,
                  anchor_ids, q8, scale, k1, cdist, num_anchors, padded_dim, threads=None):
    L = lib()
    g, keep = graph_struct(index, routes.route_group, routes.route_start)
    n = routes.count
    W = prm.result_width
    ids = np.empty((n, W), np.uint32)
    dists = np.empty((n, W), np.float32)
    stats = (Stats * max(n, 1))()
    arrs = [c_arr(codes, np.uint8), c_arr(factors, np.float32), c_arr(anchor_ids, np.uint32),
            c_arr(q8, np.int8), c_arr(scale, np.float32), c_arr(k1, np.float32),
            c_arr(cdist, np.float32), c_arr(routes.route_query, np.uint32)]
    rc = _drive("rabitq_search_batch", C.byref(g), C.byref(pred.struct), C.byref(prm), p(arrs[0]),
                                   U32(padded_dim // 8), p(arrs[1]), p(arrs[2]), p(arrs[3]),
                                   p(arrs[4]), p(arrs[5]), p(arrs[6]), U32(num_anchors),
                                   U32(padded_dim), p(arrs[7]), U32(n), p(ids), p(dists), stats, threads=threads)
    assert rc == 0
    return ids, dists, stats_array(stats, n)


STATS_FIELDS = [f[0] for f in Stats._fields_]


def stats_array(stats, n):
    out = np.zeros((n, len(STATS_FIELDS)), np.int32)
    for i in range(n):
        out[i] = [getattr(stats[i], f) for f in STATS_FIELDS]
    return out


def pq_lut(table, query, pq_dim):
    L = lib()
    table = c_arr(table, np.float32)
    lut = np.empty(pq_dim * 256, np.float32)
    if query.dtype == np.uint8:
        L.orc_pq_lut_u8(p(table), p(np.ascontiguousarray(query)), int(table.shape[1]), pq_dim,
                        p(lut))
    else:
        L.orc_pq_lut_f32(p(table), p(c_arr(query, np.float32)), int(table.shape[1]), pq_dim,
                         p(lut))
    return lut


def pq_adc(lut, code):
    code = c_arr(code, np.uint8)
    return lib().orc_pq_adc(p(lut), p(code), int(code.shape[0]))


def rabitq_quantize(rotated_row):
    r = c_arr(rotated_row, np.float32)
    q8 = np.empty(r.shape[0], np.int8)
    s = C.c_float()
    lib().orc_rabitq_quantize(p(r), U32(r.shape[0]), p(q8), C.byref(s))
    k1 = C.c_float()
    lib().orc_rabitq_query_factors(p(r), U32(r.shape[0]), C.byref(k1), None)
    return q8, s.value, k1.value


def rabitq_ip(q8, code, which="int"):
    q8 = c_arr(q8, np.int8)
    code = c_arr(code, np.uint8)
    fn = {"int": lib().orc_rabitq_ip_int, "popcount": lib().orc_rabitq_ip_popcount,
          "dp4a": lib().orc_rabitq_ip_dp4a}[which]
    return fn(p(q8), p(code), U32(q8.shape[0]))


def posting_scan_pq(pred, codes, table, queries, route_query, cand_ids, cand_offsets,
                    cand_sizes, k, score_first=False, threads=None):
    L = lib()
    n = len(route_query)
    ids = np.empty((max(n, 1), k), np.uint32)
    dists = np.empty((max(n, 1), k), np.float32)
    passes = np.empty(max(n, 1), np.uint32)
    arrs = [c_arr(codes, np.uint8), c_arr(table, np.float32), np.ascontiguousarray(queries),
            c_arr(route_query, np.uint32), c_arr(cand_ids, np.uint32),
            c_arr(cand_offsets, np.uint32), c_arr(cand_sizes, np.uint32)]
    rc = _drive("pq_posting_scan", C.byref(pred.struct) if pred else None, p(arrs[0]), p(arrs[1]),
                               p(arrs[2]), 1 if queries.dtype == np.float32 else 0, p(arrs[3]),
                               p(arrs[4]), p(arrs[5]), p(arrs[6]), U32(n),
                               int(arrs[1].shape[1]), int(arrs[0].shape[1]), k,
                               1 if score_first else 0, p(ids), p(dists), p(passes), threads=threads)
    assert rc == 0
    return ids[:n], dists[:n], passes[:n]


def posting_scan_rabitq(pred, codes, factors, anchor_ids, q8, q_scale, q_k1, centroid_dists,
                        route_query, cand_ids, cand_offsets, cand_sizes, k, threads=None):
    """orc_rabitq_posting_scan (filter-first label postings): ids, dists,
    pass counts per route."""
    L = lib()
    n = len(route_query)
    codes = c_arr(codes, np.uint8)
    q8 = c_arr(q8, np.int8)
    cd = c_arr(centroid_dists, np.float32)
    ids = np.empty((max(n, 1), k), np.uint32)
    dists = np.empty((max(n, 1), k), np.float32)
    passes = np.empty(max(n, 1), np.uint32)
    arrs = [codes, c_arr(factors, np.float32), c_arr(anchor_ids, np.uint32), q8,
            c_arr(q_scale, np.float32), c_arr(q_k1, np.float32), cd,
            c_arr(route_query, np.uint32), c_arr(cand_ids, np.uint32),
            c_arr(cand_offsets, np.uint32), c_arr(cand_sizes, np.uint32)]
    rc = _drive("rabitq_posting_scan", C.byref(pred.struct) if pred else None, p(arrs[0]),
                                   U32(codes.shape[1]), *[p(a) for a in arrs[1:7]],
                                   U32(cd.shape[1]), U32(q8.shape[1]),
                                   *[p(a) for a in arrs[7:]], U32(n), k, p(ids), p(dists),
                                   p(passes), threads=threads)
    assert rc == 0
    return ids[:n], dists[:n], passes[:n]


def rerank(base, queries, route_query, shortlist, topk, threads=None):
    L = lib()
    elem = {np.dtype(np.uint8): 0, np.dtype(np.float32): 1, np.dtype(np.float16): 2}[base.dtype]
    base_c = np.ascontiguousarray(base)
    if elem == 2:
        base_c = base_c.view(np.uint16)
    q = np.ascontiguousarray(queries)
    sl = c_arr(shortlist, np.uint32)
    n, width = sl.shape
    ids = np.empty((n, topk), np.uint32)
    dists = np.empty((n, topk), np.float32)
    rq = c_arr(route_query, np.uint32)
    rc = _drive("rerank", p(base_c), elem, U32(base.shape[1]), U32(base.shape[0]), p(q), p(rq),
                      p(sl), U32(width), U32(n), U32(topk), p(ids), p(dists), threads=threads)
    assert rc == 0
    return ids, dists


def merge(route_to_query, ids, dists, queries, topk):
    L = lib()
    ids = c_arr(ids, np.uint32)
    dists = c_arr(dists, np.float32)
    r2q = c_arr(route_to_query, np.uint32)
    n, width = ids.shape
    oi = np.empty((queries, topk), np.uint32)
    od = np.empty((queries, topk), np.float32)
    assert L.orc_merge_routes(p(r2q), U32(n), U32(queries), p(ids), p(dists), U32(width),
                              U32(topk), p(oi), p(od)) == 0
    return oi, od


class RangeTable(C.Structure):
    _fields_ = [("modes", P), ("lower", P), ("upper", P), ("base_values", P), ("count", U32)]


def segment_plan(route_ids, offsets, sizes, target_rows):
    """orc_segment_plan -> (routes, positions, offsets, sizes, indptr)."""
    L = lib()
    r = c_arr(route_ids, np.uint32)
    o = c_arr(offsets, np.uint64)
    s = c_arr(sizes, np.uint64)
    n = r.size
    cnt = U32(0)
    rc = L.orc_segment_plan(p(r), p(o), p(s), U32(n), U32(target_rows), U32(0), None, None,
                            None, None, None, C.byref(cnt))
    if rc < 0:
        return rc
    m = cnt.value
    out = (np.empty(m, np.uint32), np.empty(m, np.uint32), np.empty(m, np.uint64),
           np.empty(m, np.uint64), np.empty(n + 1, np.uint32))
    assert L.orc_segment_plan(p(r), p(o), p(s), U32(n), U32(target_rows), U32(m),
                              *[p(a) for a in out], C.byref(cnt)) == 0
    return out


def ref_segment_plan(route_ids, offsets, sizes, target_rows):
    """posting_segments::make_plan through oracle/_ref, or None."""
    R = ref()
    if R is None or not hasattr(R, "ref_segment_plan"):
        return None
    r = c_arr(route_ids, np.uint32)
    o = c_arr(offsets, np.uint64)
    s = c_arr(sizes, np.uint64)
    n = r.size
    cap = int(sum(max(1, -(-int(x) // target_rows)) for x in s)) + 1
    out = (np.empty(cap, np.uint32), np.empty(cap, np.uint32), np.empty(cap, np.uint64),
           np.empty(cap, np.uint64), np.empty(n + 1, np.uint32))
    m = R.ref_segment_plan(p(r), p(o), p(s), U32(n), U32(target_rows), U32(cap),
                           *[p(a) for a in out])
    if m < 0:
        return m
    return tuple(a[:m] for a in out[:4]) + (out[4],)


def ref_range_slices(path, modes, lower, upper):
    """choose_smallest_slice over a FARPIDX1 file loaded by the reference
    loader: ([n][5] uint64, row_count) or (None, message)."""
    R = ref()
    if R is None or not hasattr(R, "ref_range_slices"):
        return None
    modes = c_arr(modes, np.uint8)
    n, rc = modes.shape
    out = np.zeros((max(n, 1), 5), np.uint64)
    rows = C.c_uint64(0)
    err = C.create_string_buffer(512)
    code = R.ref_range_slices(str(path).encode(), p(modes), p(c_arr(lower, np.float32)),
                              p(c_arr(upper, np.float32)), U32(n), U32(rc), p(out),
                              C.byref(rows), err, U32(512))
    if code != 0:
        return None, err.value.decode()
    return out[:n], rows.value


def _ref_graph_fn(name, argtypes):
    R = ref()
    if R is None or not hasattr(R, name):
        return None
    fn = getattr(R, name)
    fn.argtypes = argtypes
    return fn


def ref_graph_file_header(path):
    """read_graph_file_header -> 40 header bytes, or (None, message)."""
    fn = _ref_graph_fn("ref_graph_file_header", [C.c_char_p, P, C.c_char_p, U32])
    if fn is None:
        return None
    out = np.zeros(40, np.uint8)
    err = C.create_string_buffer(512)
    if fn(str(path).encode(), p(out), err, U32(512)) != 0:
        return None, err.value.decode()
    return out.tobytes()


def ref_graph_file_load(path, capacity_words):
    """load_graph_file_as_contiguous_matrix -> [rows][cols] u32, or (None, message)."""
    fn = _ref_graph_fn("ref_graph_file_load",
                       [C.c_char_p, P, C.c_uint64, P, P, C.c_char_p, U32])
    if fn is None:
        return None
    out = np.zeros(max(capacity_words, 1), np.uint32)
    rows, cols = C.c_uint64(0), C.c_uint64(0)
    err = C.create_string_buffer(512)
    code = fn(str(path).encode(), p(out), C.c_uint64(capacity_words), C.byref(rows),
              C.byref(cols), err, U32(512))
    if code != 0:
        return None, err.value.decode() if code == -1 else "capacity"
    return out[: rows.value * cols.value].reshape(rows.value, cols.value)


def ref_graph_file_write(path, rows, chunk=7):
    """GraphFileSequentialWriter, rows appended `chunk` at a time -> True or message."""
    fn = _ref_graph_fn("ref_graph_file_write",
                       [C.c_char_p, P, C.c_uint64, U32, C.c_uint64, C.c_char_p, U32])
    if fn is None:
        return None
    rows = np.ascontiguousarray(rows, np.uint32)
    err = C.create_string_buffer(512)
    code = fn(str(path).encode(), p(rows), C.c_uint64(rows.shape[0]), U32(rows.shape[1]),
              C.c_uint64(chunk), err, U32(512))
    return True if code == 0 else err.value.decode()


def ref_graph_file_convert_legacy(legacy_path, path):
    fn = _ref_graph_fn("ref_graph_file_convert_legacy", [C.c_char_p, C.c_char_p, C.c_char_p, U32])
    if fn is None:
        return None
    err = C.create_string_buffer(512)
    code = fn(str(legacy_path).encode(), str(path).encode(), err, U32(512))
    return True if code == 0 else err.value.decode()


def rabitq_range_scan(pred, modes, lower, upper, base_values, codes, factors, anchor_ids, q8,
                      q_scale, q_k1, centroid_dists, route_query, posting, resident_rows,
                      base_rows, seg_routes, seg_offsets, seg_sizes, k, score_first=False, threads=None):
    """orc_rabitq_range_scan -> per-segment (ids, dists, passes)."""
    L = lib()
    modes = c_arr(modes, np.uint8)
    lower, upper = c_arr(lower, np.float32), c_arr(upper, np.float32)
    bv = c_arr(base_values, np.float32)
    rt = RangeTable(p(modes), p(lower), p(upper), p(bv),
                    U32(modes.shape[1] if modes is not None and modes.ndim == 2 else 0))
    codes = c_arr(codes, np.uint8)
    arrs = [c_arr(factors, np.float32), c_arr(anchor_ids, np.uint32), c_arr(q8, np.int8),
            c_arr(q_scale, np.float32), c_arr(q_k1, np.float32),
            c_arr(centroid_dists, np.float32)]
    cd = arrs[5]
    padded = int(np.asarray(q8).shape[1])
    rq = c_arr(route_query, np.uint32)
    post = c_arr(posting, np.uint32)
    sr, so, ss = c_arr(seg_routes, np.uint32), c_arr(seg_offsets, np.uint64), c_arr(seg_sizes, np.uint64)
    n = sr.size
    ids = np.empty((max(n, 1), k), np.uint32)
    dists = np.empty((max(n, 1), k), np.float32)
    passes = np.empty(max(n, 1), np.uint32)
    rc = _drive("rabitq_range_scan", C.byref(pred.struct) if pred else None, C.byref(rt), p(codes),
                                 U32(codes.shape[1]), *[p(a) for a in arrs], U32(cd.shape[1]),
                                 U32(padded), p(rq), p(post), C.c_uint64(resident_rows), U32(base_rows),
                                 p(sr), p(so), p(ss), U32(n), k, 1 if score_first else 0,
                                 p(ids), p(dists), p(passes), threads=threads)
    assert rc == 0
    return ids[:n], dists[:n], passes[:n]


def merge_segments(indptr, seg_ids, seg_dists, seg_pass, k):
    """orc_merge_segments -> per-position (ids, dists, passes)."""
    L = lib()
    ip = c_arr(indptr, np.uint32)
    n = ip.size - 1
    ids = np.empty((max(n, 1), k), np.uint32)
    dists = np.empty((max(n, 1), k), np.float32)
    passes = np.empty(max(n, 1), np.uint32)
    assert L.orc_merge_segments(p(ip), U32(n), p(c_arr(seg_ids, np.uint32)),
                                p(c_arr(seg_dists, np.float32)), p(c_arr(seg_pass, np.uint32)),
                                k, p(ids), p(dists), p(passes)) == 0
    return ids[:n], dists[:n], passes[:n]


class ExactParams(C.Structure):
    _fields_ = [("queue_limit", C.c_int), ("finish_limit", C.c_int),
                ("early_stop_mode", C.c_int), ("max_steps", C.c_int), ("topk", C.c_int)]


def exact_search(index, routes, pred, base, queries, queue_limit=64, topk=10,
                 early_stop_mode=2, finish_limit=1, max_steps=0, label_size=None,
                 row_filter_mask=None, query_filter_bits=None, range_modes=None,
                 range_lower=None, range_upper=None, base_range_values=None, threads=None):
    """orc_exact_search over every route: ids [R][topk] u32, dists f32, stats.
    base and queries: u8, f32 or f16 rows of one element type."""
    L = lib()
    g, keep = graph_struct(index, routes.route_group, routes.route_start)
    extra = dict(rm=c_arr(row_filter_mask, np.uint64), qb=c_arr(query_filter_bits, np.uint64),
                 modes=c_arr(range_modes, np.uint8), lo=c_arr(range_lower, np.float32),
                 hi=c_arr(range_upper, np.float32), brv=c_arr(base_range_values, np.float32),
                 ls=c_arr(label_size, np.uint32))
    g.row_filter_mask, g.query_filter_bits = p(extra["rm"]), p(extra["qb"])
    g.range_modes, g.range_lower, g.range_upper = p(extra["modes"]), p(extra["lo"]), p(extra["hi"])
    g.base_range_values = p(extra["brv"])
    g.range_count = 0 if range_modes is None else int(np.asarray(range_modes).shape[1])
    n = routes.count
    ids = np.empty((max(n, 1), topk), np.uint32)
    dists = np.empty((max(n, 1), topk), np.float32)
    stats = (Stats * max(n, 1))()
    b, elem = _rows(base)
    q, qelem = _rows(queries)
    assert qelem == elem, "queries have the element type of the base rows"
    rq = c_arr(routes.route_query, np.uint32)
    prm = ExactParams(queue_limit, finish_limit, early_stop_mode, max_steps, topk)
    rc = _drive("exact_search", C.byref(g), p(extra["ls"]), C.byref(pred.struct) if pred else None,
                            C.byref(prm), p(b), C.c_int(elem), U32(b.shape[1]), U32(b.shape[0]),
                            p(q), p(rq), U32(n), p(ids), p(dists), stats, threads=threads)
    assert rc == 0
    return ids[:n], dists[:n], stats_array(stats, n)


EXACT_ORDER_SERIAL, EXACT_ORDER_W32 = 0, 1


def l2_w32(row, q) -> float:
    """orc_l2_w32: the warp-order exact distance of one row and one query."""
    r, e = _rows(np.asarray(row)[None])
    qq, _ = _rows(np.asarray(q)[None])
    return float(lib().orc_l2_w32(p(r), p(qq), e, r.shape[1]))


def l2_serial(row, q) -> float:
    """orc_l2_serial: the serial-order exact distance of one row and one query."""
    r, e = _rows(np.asarray(row)[None])
    qq, _ = _rows(np.asarray(q)[None])
    return float(lib().orc_l2_serial(p(r), p(qq), e, r.shape[1]))


def exact_posting_scan(pred, base, queries, route_query, cand_ids, cand_offsets, cand_sizes,
                       topk, order=EXACT_ORDER_SERIAL):
    """orc_exact_posting_scan: per route the topk distinct listed samples by
    exact (distance, id); (ids [R][topk], dists, pass counts)."""
    b, elem = _rows(base)
    q, qelem = _rows(queries)
    assert qelem == elem
    rq = c_arr(route_query, np.uint32)
    ci = c_arr(cand_ids, np.uint32)
    co = c_arr(cand_offsets, np.uint32)
    cs = c_arr(cand_sizes, np.uint32)
    n = len(rq)
    ids = np.empty((max(n, 1), topk), np.uint32)
    dists = np.empty((max(n, 1), topk), np.float32)
    passes = np.empty(max(n, 1), np.uint32)
    rc = lib().orc_exact_posting_scan(C.byref(pred.struct) if pred else None, p(b), elem,
                                      U32(b.shape[1]), U32(b.shape[0]), p(q), p(rq), p(ci),
                                      p(co), p(cs), U32(n), topk, order, p(ids), p(dists),
                                      p(passes))
    assert rc == 0
    return ids[:n], dists[:n], passes[:n]


# ---- index construction (build_oracle.c) --------------------------------
U64 = C.c_uint64
_BUILD_SIGS = {
    "orc_build_draw64": (U64, [U64, U64, U64]),
    "orc_build_draw_unit": (C.c_double, [U64, U64, U64]),
    "orc_build_assign": (None, [P, C.c_int, U32, U64, P, U32, P, P]),
    "orc_build_kmeanspp": (None, [P, C.c_int, U32, U64, U32, U64, P]),
    "orc_build_kmeans": (None, [P, C.c_int, U32, U64, U32, U32, P]),
    "orc_build_knn": (None, [P, C.c_int, U32, P, U32, P, P, U32, P, P]),
    "orc_build_pq_encode": (None, [P, C.c_int, U32, U64, U32, P, P, U32]),
    "orc_build_pq_train": (None, [P, C.c_int, U32, U64, U32, U32, P]),
    "orc_build_rabitq_encode": (None, [P, U32, U32, P, U32, P, P, P]),
    "orc_build_medoid": (U32, [P, C.c_int, U32, U64]),
    "orc_build_bucket_reps": (None, [P, C.c_int, U32, P, U32, P, P]),
    "orc_build_links": (None, [U32, P, U32, P, P, P, U32, U32, P, U32, U32, U32, U32, U32, U32,
                               U64, P]),
    "orc_build_cagra_optimize": (None, [P, U32, U32, U32, P, P]),
    "orc_build_reach": (U32, [P, U32, U32, U32, P]),
}


def _blib():
    L = lib()
    if not getattr(L, "_build_ready", False):
        for name, (res, args) in _BUILD_SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        L._build_ready = True
    return L


def _rows(rows):
    """(contiguous array, elem code) of a row matrix: u8 0, f32 1, f16 2."""
    a = np.ascontiguousarray(rows)
    elem = {np.dtype(np.uint8): 0, np.dtype(np.float32): 1, np.dtype(np.float16): 2}[a.dtype]
    return a, elem


def build_draw64(seed, stream, index):
    return int(_blib().orc_build_draw64(seed, stream, index))


def build_draw_unit(seed, stream, index):
    return float(_blib().orc_build_draw_unit(seed, stream, index))


def build_assign(rows, centres):
    a, elem = _rows(rows)
    c = np.ascontiguousarray(centres, np.float32)
    idx = np.empty(a.shape[0], np.uint32)
    score = np.empty(a.shape[0], np.float32)
    _blib().orc_build_assign(p(a), elem, a.shape[1], a.shape[0], p(c), c.shape[0], p(idx), p(score))
    return idx, score


def build_kmeanspp(rows, k, seed):
    a, elem = _rows(rows)
    out = np.empty((k, a.shape[1]), np.float32)
    _blib().orc_build_kmeanspp(p(a), elem, a.shape[1], a.shape[0], k, seed, p(out))
    return out


def build_kmeans(rows, centres, iters):
    a, elem = _rows(rows)
    c = np.array(centres, np.float32, copy=True)
    _blib().orc_build_kmeans(p(a), elem, a.shape[1], a.shape[0], c.shape[0], iters, p(c))
    return c


def build_knn(rows, bucket_off, k, probe_off=None, probe=None):
    a, elem = _rows(rows)
    bo = np.ascontiguousarray(bucket_off, np.uint32)
    po = c_arr(probe_off, np.uint32)
    pb = c_arr(probe, np.uint32)
    n = int(bo[-1])
    ids = np.empty((n, k), np.uint32)
    d = np.empty((n, k), np.float32)
    _blib().orc_build_knn(p(a), elem, a.shape[1], p(bo), len(bo) - 1, p(po), p(pb), k, p(ids), p(d))
    return ids, d


def build_pq_encode(rows, centroids, pq_dim):
    a, elem = _rows(rows)
    c = np.ascontiguousarray(centroids, np.float32)
    codes = np.empty((a.shape[0], pq_dim), np.uint8)
    _blib().orc_build_pq_encode(p(a), elem, a.shape[1], a.shape[0], pq_dim, p(c), p(codes), pq_dim)
    return codes


def build_pq_train(rows, centroids, pq_dim, iters):
    a, elem = _rows(rows)
    c = np.array(centroids, np.float32, copy=True)
    _blib().orc_build_pq_train(p(a), elem, a.shape[1], a.shape[0], pq_dim, iters, p(c))
    return c


def build_rabitq_encode(rotated, anchors):
    x = np.ascontiguousarray(rotated, np.float32)
    an = np.ascontiguousarray(anchors, np.float32)
    n, P_ = x.shape
    aid = np.empty(n, np.uint32)
    codes = np.empty((n, P_ // 8), np.uint8)
    fac = np.empty((n, 3), np.float32)
    _blib().orc_build_rabitq_encode(p(x), n, P_, p(an), an.shape[0], p(aid), p(codes), p(fac))
    return aid, codes, fac


def build_medoid(rows):
    a, elem = _rows(rows)
    return int(_blib().orc_build_medoid(p(a), elem, a.shape[1], a.shape[0]))


def build_bucket_reps(rows, bucket_off):
    a, elem = _rows(rows)
    bo = np.ascontiguousarray(bucket_off, np.uint32)
    nb = len(bo) - 1
    means = np.empty((nb, a.shape[1]), np.float32)
    reps = np.empty(nb, np.uint32)
    _blib().orc_build_bucket_reps(p(a), elem, a.shape[1], p(bo), nb, p(means), p(reps))
    return means, reps


def build_links(knn, bucket_of, reps, near, order, degree, local, near_links, rep_local,
                rep_near, entry, seed):
    knn = np.ascontiguousarray(knn, np.uint32)
    n = int(bucket_of.shape[0])
    bo = np.ascontiguousarray(bucket_of, np.uint32)
    rp = np.ascontiguousarray(reps, np.uint32)
    nr = np.ascontiguousarray(near, np.uint32)
    od = np.ascontiguousarray(order, np.uint32)
    out = np.empty((n, degree), np.uint32)
    _blib().orc_build_links(n, p(knn), knn.shape[1] if knn.ndim == 2 else 0, p(bo), p(rp), p(nr),
                            nr.shape[1] if nr.ndim == 2 else 0, rp.shape[0], p(od), degree, local,
                            near_links, rep_local, rep_near,
                            0xFFFFFFFF if entry is None else int(entry), seed, p(out))
    return out


def build_cagra_optimize(knn, degree):
    knn = np.ascontiguousarray(knn, np.uint32)
    n, kin = knn.shape
    pruned = np.empty((n, degree), np.uint32)
    out = np.empty((n, degree), np.uint32)
    _blib().orc_build_cagra_optimize(p(knn), n, kin, degree, p(pruned), p(out))
    return pruned, out


def build_reach(graph, entry):
    g = np.ascontiguousarray(graph, np.uint32)
    n, deg = g.shape
    reached = np.empty(n, np.uint32)
    cnt = _blib().orc_build_reach(p(g), n, deg, entry, p(reached))
    return reached.astype(bool), int(cnt)


class OracleBuild:
    """The index-construction primitives of gofann_amd.builder.HipBuild,
    restated on the CPU (build_oracle.c), over numpy arrays.  Tests pass it
    to gofann_amd.index's builders to build fixtures on the CPU, and to
    check the GPU build step for step; the product never selects it."""

    def rows(self, x):
        if hasattr(x, "detach"):
            x = x.detach().cpu().numpy()
        x = np.asarray(x)
        if x.dtype not in (np.uint8, np.float32, np.float16):
            x = x.astype(np.float32)
        return np.ascontiguousarray(x)

    def take(self, rows, idx):
        return np.ascontiguousarray(rows[np.asarray(idx, np.int64)])

    def host(self, a):
        if hasattr(a, "detach"):
            a = a.detach().cpu().numpy()
        return np.asarray(a)

    def dev(self, a, dtype=None):
        a = self.host(a)
        return a if dtype is None else a.astype(dtype)

    def assign(self, rows, centres):
        return build_assign(rows, self.host(centres))[0]

    def kmeanspp(self, rows, k, seed):
        return build_kmeanspp(rows, k, seed)

    def kmeans(self, rows, centres, iters):
        return build_kmeans(rows, self.host(centres), iters)

    def knn(self, rows, bucket_off, k, probe_off=None, probe=None):
        return build_knn(rows, bucket_off, k, probe_off, probe)[0]

    def bucket_reps(self, rows, bucket_off):
        return build_bucket_reps(rows, bucket_off)

    def medoid(self, rows):
        return build_medoid(rows)

    def links(self, knn, bucket_of, reps, near, order, degree, local, near_links, rep_local,
              rep_near, entry, seed):
        knn = np.zeros((len(bucket_of), 0), np.uint32) if knn is None else self.host(knn)
        return build_links(knn.view(np.uint32) if knn.dtype == np.int32 else knn, bucket_of,
                           self.host(reps), self.host(near), order, degree, local, near_links,
                           rep_local, rep_near, 0xFFFFFFFF if entry is None else int(entry), seed)

    def cagra_optimize(self, knn, degree):
        return build_cagra_optimize(self.host(knn), degree)

    def reach(self, graph, entry):
        return build_reach(self.host(graph), int(entry))

    def pq_train(self, rows, centroids, pq_dim, iters):
        return build_pq_train(rows, self.host(centroids), pq_dim, iters)

    def pq_encode(self, rows, centroids, pq_dim):
        return build_pq_encode(rows, self.host(centroids), pq_dim)

    def rotate(self, rows, rotation):
        # fp64 product rounded to fp32 (the GPU's rocBLAS SGEMM is checked
        # against the same fp64 product within a tolerance)
        return (rows.astype(np.float64) @ self.host(rotation).astype(np.float64)).astype(np.float32)

    def rabitq_encode(self, rotated, anchors):
        return build_rabitq_encode(rotated, self.host(anchors))
