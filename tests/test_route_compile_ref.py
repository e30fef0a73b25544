"""Route residual compile (plan.py: dnf_route_rows + compile_residuals)
against the reference's own route_predicate::compile
(src/planning/route_predicate_plan.h:175-315, compiled into oracle/_ref from
the reference tree): random DNF queries over labels with and without graphs,
range atoms on two dimensions, graph routes (dual AND routes included) and
label-posting routes (clause scans included).  For every route the residual
clauses -- labels in order, range atoms, the entailed form -- are equal."""
from __future__ import annotations

import ctypes as C
import struct

import numpy as np
import pytest

import pyoracle as po
from gofann_amd import plan as gp

ref = po.ref()
pytestmark = pytest.mark.skipif(ref is None, reason="oracle/_ref not built (no reference tree)")

L = 40        # labels; 0..14 without graph (posting only), 15..39 with graph
DIMS = 2      # range dimensions


class Ix:
    def __init__(self, rng):
        self.cat_freq = np.concatenate([rng.integers(5, 400, 15),
                                        rng.integers(2000, 90000, 25)]).astype(np.int64)
        self.label_size = np.where(np.arange(L) >= 15, self.cat_freq, 0)
        self.seed_local = np.zeros(L, np.uint32)

    def has_graph(self, l):
        return self.label_size[l] > 0


def _queries(rng, n):
    out, ranges = [], []
    for _ in range(n):
        clauses = []
        for _ in range(int(rng.integers(1, 4))):
            m = int(rng.integers(1, 4))
            labels = [int(x) for x in rng.integers(0, L, m)]  # duplicates possible
            clauses.append((labels, bool(rng.integers(0, 2))))
        out.append(clauses)
        atoms = []
        for d in range(DIMS):
            mode = int(rng.integers(0, 4))
            if mode:
                lo = float(rng.integers(0, 500))
                atoms.append((d, mode, lo, lo + float(rng.integers(1, 300))))
        ranges.append(atoms)
    return out, ranges


def _table(queries, ranges):
    q_indptr = [0]
    label_indptr = [0]
    labels, uses = [], []
    for clauses in queries:
        for lab, ur in clauses:
            labels.extend(lab)
            label_indptr.append(len(labels))
            uses.append(1 if ur else 0)
        q_indptr.append(len(uses))
    nq = len(queries)
    modes = np.zeros((nq, DIMS), np.uint8)
    lo = np.zeros((nq, DIMS), np.float32)
    hi = np.zeros((nq, DIMS), np.float32)
    for q, atoms in enumerate(ranges):
        for d, m, a, b in atoms:
            modes[q, d], lo[q, d], hi[q, d] = m, a, b
    return (np.array(q_indptr, np.uint64), np.array(label_indptr, np.uint64),
            np.array(labels if labels else [0], np.uint32), np.array(uses, np.uint8),
            modes, lo, hi)


def _ref_routes(producer, ix, table, rows):
    q_indptr, label_indptr, labels, uses, modes, lo, hi = table
    n = len(rows)
    rq = np.array([r[0] for r in rows], np.uint32)
    anchor = np.array([r[1] for r in rows], np.uint32)
    cids = np.array([int(q_indptr[r[0]]) + r[4] for r in rows], np.uint32)
    cptr = np.arange(n + 1, dtype=np.uint64)
    label_rows = ix.cat_freq.astype(np.uint32)
    cap = 64 * n + 64
    out = np.zeros(cap, np.uint32)
    words = C.c_uint64(0)
    err = C.create_string_buffer(512)
    p = po.p
    rc = ref.ref_route_compile(C.c_int(producer), C.c_uint32(len(q_indptr) - 1), p(q_indptr),
                               p(label_indptr), p(labels), p(uses), C.c_uint32(DIMS), p(modes),
                               p(lo), p(hi), C.c_uint32(L), C.c_uint32(100000), p(label_rows),
                               C.c_uint32(n), p(rq), p(anchor), p(cptr), p(cids), p(out),
                               C.c_uint64(cap), C.byref(words), err, C.c_uint32(512))
    assert rc == 0, err.value
    w = out[: words.value].tolist()
    res, i = [], 0
    for _ in range(n):
        avail, ent, nc = w[i:i + 3]
        i += 3
        cl = []
        for _ in range(nc):
            nl = w[i]
            labs = w[i + 1:i + 1 + nl]
            i += 1 + nl
            nr = w[i]
            i += 1
            atoms = []
            for _ in range(nr):
                d, m, a, b = w[i:i + 4]
                i += 4
                atoms.append((d, m, struct.unpack("<f", struct.pack("<I", a))[0],
                              struct.unpack("<f", struct.pack("<I", b))[0]))
            cl.append((labs, atoms))
        res.append((avail, ent, cl))
    return res


def _our_routes(ix, rows):
    pr = gp._routeset([r[:4] for r in rows], ix).predicate
    out = []
    for r in range(len(rows)):
        cl = []
        for c in pr.clauses[pr.route_offsets[r]:pr.route_offsets[r + 1]]:
            labs = pr.handles[c["label_begin"]:c["label_end"]].tolist()
            atoms = [(int(a["dimension"]), int(a["mode"]), float(a["lower"]), float(a["upper"]))
                     for a in pr.ranges[c["range_begin"]:c["range_end"]]]
            cl.append((labs, atoms))
        out.append(cl)
    return out


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_residual_compile_matches_reference(seed):
    rng = np.random.default_rng(700 + seed)
    ix = Ix(rng)
    queries, ranges = _queries(rng, 300)
    table = _table(queries, ranges)
    g_rows, p_rows = gp.dnf_route_rows(ix, queries, ranges, clause_scans=True, with_clause=True)
    assert len(g_rows) > 200 and len(p_rows) > 100
    for producer, rows in ((0, g_rows), (1, p_rows)):
        theirs = _ref_routes(producer, ix, table, rows)
        ours = _our_routes(ix, rows)
        entailed = 0
        for r, ((avail, ent, cl), mine) in enumerate(zip(theirs, ours)):
            assert avail == 1, (producer, r)
            assert cl == mine, (producer, r, rows[r], cl, mine)
            entailed += ent
            # the entailed form: one empty clause
            assert (ent == 1) == (mine == [([], [])])
        assert entailed > 0


def test_reference_rejects_foreign_clause():
    """A route that names a clause of another query is an error in the
    reference; the planner never emits one (each row owns a clause of its
    own query)."""
    rng = np.random.default_rng(9)
    ix = Ix(rng)
    queries, ranges = _queries(rng, 20)
    table = _table(queries, ranges)
    g_rows, _ = gp.dnf_route_rows(ix, queries, ranges, with_clause=True)
    bad = [list(g_rows[0])]
    other = next(i for i, r in enumerate(g_rows) if r[0] != g_rows[0][0])
    q0 = g_rows[0][0]
    # clause ordinal that lands in the next query's clause range
    bad[0][4] = int(table[0][q0 + 1] - table[0][q0])
    with pytest.raises(AssertionError, match="another original query"):
        _ref_routes(0, ix, table, [tuple(bad[0])])
    assert other > 0
