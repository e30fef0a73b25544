"""Route planning and device-predicate compilation (host side).

A filtered query (AND of labels, optional range atoms) becomes one or more
routes:
  * every label has a graph (frequency above the threshold): one graph route
    per label (dual AND routing -- and_dual_route_posting_ratio_threshold
    defaults to 1e30, src/app/runtime_defaults.h:31, so two graph labels
    always give two routes; src/data/dataloader.cpp:9064-9080, 9804-9810);
  * some label is rare: one posting route over the rarest rare label
    (dataloader.cpp:9793-9808).
Each route's residual predicate is the query's labels minus the route's
anchor plus its range atoms, compiled to one DNF clause
(route_predicate::compile / finish, src/planning/route_predicate_plan.h:
88-101, 134-144; device packing backend_pq.cu:5815-5832).  An empty residual
is entailed: one empty clause.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

CLAUSE_DTYPE = np.dtype([("label_begin", "<u4"), ("label_end", "<u4"),
                         ("range_begin", "<u4"), ("range_end", "<u4")])
RANGE_DTYPE = np.dtype([("dimension", "<u4"), ("mode", "<u4"),
                        ("lower", "<f4"), ("upper", "<f4")])


@dataclass
class CompiledPredicate:
    route_offsets: np.ndarray   # u32 [routes+1] -> clauses
    handles: np.ndarray         # u32
    clauses: np.ndarray         # CLAUSE_DTYPE
    ranges: np.ndarray          # RANGE_DTYPE
    enabled: np.ndarray         # u8 [routes]
    compiled: np.ndarray        # u8 [routes]


@dataclass
class RouteSet:
    route_query: np.ndarray     # u32 query vector row
    route_group: np.ndarray     # u32 label (graph routes) / anchor label (posting)
    route_start: np.ndarray     # u32 label-local seed row (graph routes)
    route_to_query: np.ndarray  # u32 original query
    predicate: CompiledPredicate

    @property
    def count(self) -> int:
        return int(self.route_query.shape[0])


@dataclass
class Plan:
    graph: RouteSet
    posting: RouteSet
    cand_offsets: np.ndarray    # u32 [posting routes] into posting_ids
    cand_sizes: np.ndarray      # u32 [posting routes]
    queries: int


def compile_residuals(residual_labels: list, residual_ranges: list) -> CompiledPredicate:
    offsets = [0]
    handles: list[int] = []
    clauses = []
    ranges = []
    for labels, rng in zip(residual_labels, residual_ranges):
        lb = len(handles)
        handles.extend(int(l) for l in labels)
        rb = len(ranges)
        ranges.extend(rng)
        clauses.append((lb, len(handles), rb, len(ranges)))
        offsets.append(len(clauses))
    n = len(residual_labels)
    cl = np.array(clauses if clauses else [(0, 0, 0, 0)], dtype=CLAUSE_DTYPE)
    rg = np.array([tuple(r) for r in ranges] if ranges else [(0, 0, 0.0, 0.0)], dtype=RANGE_DTYPE)
    return CompiledPredicate(np.array(offsets, dtype=np.uint32),
                             np.array(handles if handles else [0], dtype=np.uint32),
                             cl, rg, np.ones(n, dtype=np.uint8), np.ones(n, dtype=np.uint8))


def _routeset(rows: list, index) -> RouteSet:
    rq = np.array([r[0] for r in rows], dtype=np.uint32)
    rg = np.array([r[1] for r in rows], dtype=np.uint32)
    rs = np.array([index.seed_local[r[1]] if index.has_graph(r[1]) else 0 for r in rows],
                  dtype=np.uint32)
    pred = compile_residuals([r[2] for r in rows], [r[3] for r in rows])
    return RouteSet(rq, rg, rs, rq.copy(), pred)


def nearest_bucket_seeds(index, rs: RouteSet, queries) -> np.ndarray:
    """Per-route seed: the representative row of the route label's bucket
    whose mixture centre is nearest the query (an IVF-style entry point).
    The reference seeds every route of a label at the label's medoid
    (dataloader.cpp:7361-7406); this mode only changes `route_start`."""
    import torch
    q = torch.as_tensor(queries).float()
    cen = torch.as_tensor(index.centres, device=q.device)
    out = rs.route_start.copy()
    groups = rs.route_group
    for g in np.unique(groups):
        lo, hi = int(index.rep_offset[g]), int(index.rep_offset[g + 1])
        if hi == lo:
            continue
        sel = np.nonzero(groups == g)[0]
        c = cen[torch.as_tensor(index.rep_cluster[lo:hi].astype(np.int64), device=q.device)]
        qq = q[torch.as_tensor(rs.route_query[sel].astype(np.int64), device=q.device)]
        d = (c * c).sum(1)[None, :] - 2 * qq @ c.t()
        best = d.argmin(1).cpu().numpy()
        out[sel] = index.rep_row[lo + best]
    return out


def plan_queries(index, query_labels: list, query_ranges: list | None = None,
                 sort_by_group: bool = True, seeds: str = "medoid", queries=None) -> Plan:
    """Routes for every query (see module docstring).  seeds="medoid" keeps
    the reference's one seed per label; "nearest_bucket" needs `queries`."""
    graph_rows, post_rows = [], []
    for q, labels in enumerate(query_labels):
        rng = [tuple(a) for a in (query_ranges[q] if query_ranges is not None else [])]
        labels = sorted(set(int(l) for l in labels))
        if not labels:
            raise ValueError("queries without a label route are not planned here")
        rare = [l for l in labels if not index.has_graph(l)]
        if rare:
            anchor = min(rare, key=lambda l: (int(index.cat_freq[l]), l))
            post_rows.append((q, anchor, [l for l in labels if l != anchor], rng))
        else:
            for anchor in labels:
                graph_rows.append((q, anchor, [l for l in labels if l != anchor], rng))
    if sort_by_group:
        graph_rows.sort(key=lambda r: (r[1], r[0]))
    g = _routeset(graph_rows, index)
    if seeds == "nearest_bucket" and g.count:
        g.route_start = nearest_bucket_seeds(index, g, queries)
    elif seeds != "medoid":
        raise ValueError(f"unknown seed mode {seeds}")
    p = _routeset(post_rows, index)
    off = np.array([index.posting_offset[r[1]] for r in post_rows], dtype=np.uint64)
    size = np.array([index.posting_offset[r[1] + 1] - index.posting_offset[r[1]]
                     for r in post_rows], dtype=np.uint64)
    return Plan(g, p, off.astype(np.uint32), size.astype(np.uint32), len(query_labels))


def filter_mask(index, labels: list, ranges: list, base_ranges) -> np.ndarray:
    """Exact per-sample predicate of one query (for ground truth)."""
    n = index.csr_offsets.shape[0] - 1
    mask = np.ones(n, dtype=bool)
    for l in labels:
        m = np.zeros(n, dtype=bool)
        s0, s1 = int(index.posting_offset[l]), int(index.posting_offset[l + 1])
        m[index.posting_ids[s0:s1]] = True
        mask &= m
    for (dim, mode, lo, hi) in ranges:
        v = base_ranges[:, dim]
        if mode == 1:
            mask &= v > lo
        elif mode == 2:
            mask &= v < hi
        elif mode == 3:
            mask &= (v >= lo) & (v < hi)
    return mask
