"""Route planning and device-predicate compilation (host side).

A filtered query is an OR of conjunctions (clauses); a clause is an AND of
labels, optionally with the query's range atoms.  Each clause becomes routes
(clause_anchors; prepare_query_route_chunk and plan_hybrid_clause_routes,
src/data/dataloader.cpp:9741-9853, 10860-10960):
  * some label of the clause has no graph: one posting route over the
    rarest such label;
  * two graph labels: a graph route per label (dual AND routing:
    and_dual_route_posting_ratio_threshold defaults to 1e30,
    src/app/runtime_defaults.h:31, dataloader.cpp:9066-9077);
  * otherwise: a graph route over the label with the smallest posting list.
Each route's residual predicate is its clause minus the route's anchor plus
the clause's range atoms, compiled to one DNF clause (route_predicate::
compile / finish, src/planning/route_predicate_plan.h:175-315; device
packing backend_pq.cu:5815-5832).  An empty residual is entailed: one empty
clause.  Routes of one query merge per query.
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


def clause_anchors(index, labels: list, dual_ratio: float = 1e30,
                   routing_mode: str = "greedy_min_posting") -> tuple:
    """Anchor labels of one conjunction (the route choice of
    prepare_query_route_chunk, dataloader.cpp:10860-10960, and of
    plan_hybrid_clause_routes, :9741-9853): ("posting", [l]) for the rarest
    label without a graph when there is one; ("graph", [a, b]) for two graph
    labels whose posting sizes are within dual_ratio of each other
    (should_dual_route_and_labels, :9066-9077; the default threshold 1e30,
    runtime_defaults.h:31, routes both), the smaller first; otherwise
    ("graph", [l]) for the label of least posting size (greedy_min_posting;
    greedy_max_posting takes the largest), the first of equals.  Labels with
    neither a graph nor a posting list are not routable; ("none", [])
    when no label is."""
    cand = [l for l in labels if int(index.cat_freq[l]) > 0]
    rare = [l for l in cand if not index.has_graph(l)]
    if rare:
        best = rare[0]
        for l in rare[1:]:
            if int(index.cat_freq[l]) < int(index.cat_freq[best]):
                best = l
        return "posting", [best]
    if not cand:
        return "none", []
    if routing_mode == "per_label_multi_route":
        return "graph", list(cand)
    if len(cand) == 2:
        a, b = (int(index.cat_freq[cand[0]]), int(index.cat_freq[cand[1]]))
        if max(a, b) / min(a, b) < dual_ratio:
            return "graph", [cand[1], cand[0]] if b < a else [cand[0], cand[1]]
    best = cand[0]
    for l in cand[1:]:
        f, fb = int(index.cat_freq[l]), int(index.cat_freq[best])
        if (f < fb) if routing_mode == "greedy_min_posting" else (f > fb):
            best = l
    return "graph", [best]


def plan_queries(index, query_labels: list, query_ranges: list | None = None,
                 sort_by_group: bool = True, seeds: str = "medoid", queries=None,
                 dual_ratio: float = 1e30) -> Plan:
    """Routes for every query: an AND of labels plus optional range atoms
    (one conjunction per query, see clause_anchors).  seeds="medoid" keeps
    the reference's one seed per label; "nearest_bucket" needs `queries`."""
    clauses = [[(sorted(set(int(l) for l in labels)), True)] for labels in query_labels]
    for q, cl in enumerate(clauses):
        if not cl[0][0]:
            raise ValueError("queries without a label route are not planned here")
    return plan_dnf(index, clauses, query_ranges, sort_by_group=sort_by_group, seeds=seeds,
                    queries=queries, dual_ratio=dual_ratio)


def interval_route_rows(index, query_labels: list, query_ranges: list, categories: int,
                        intervals: int, attr_max: int):
    """Route rows of a query set in which every query is either one
    categorical equality or one range [lo, hi) (mode 3) over an integer
    attribute in [0, attr_max), where each row also carries the interval
    label categories + floor(attr * intervals / attr_max) (interval virtual
    labels: scripts/laion/range_index.py:1-12):
      * equality on label L: a graph route over L when L has a graph, else a
        posting route;
      * range: one graph route per interval label it overlaps -- the
        finest-level pure-range cover (plan_pure_range_cover_labels,
        dataloader.cpp:9204-9345, over a one-level layout) -- whose residual
        is the range, except on an interval that lies inside [lo, hi), where
        the range is entailed and the residual is empty.
    Interval i holds the integers [ceil(i attr_max / intervals),
    ceil((i + 1) attr_max / intervals)).  Rows are (query, label, residual
    labels, residual ranges) in query order.  Returns (graph_rows, post_rows,
    interior), interior = routes whose residual is empty because entailed."""
    starts = [-(-(i * attr_max) // intervals) for i in range(intervals + 1)]
    graph_rows, post_rows, interior = [], [], 0
    for q, labels in enumerate(query_labels):
        if labels:
            lab = labels[0]
            (graph_rows if index.has_graph(lab) else post_rows).append((q, lab, [], []))
            continue
        (dim, mode, lo, hi), = query_ranges[q]
        if dim != 0 or mode != 3:
            raise ValueError("interval routes take one [lo, hi) range on dimension 0")
        i0 = int(lo) * intervals // attr_max
        i1 = (int(hi) - 1) * intervals // attr_max
        for i in range(i0, i1 + 1):
            inside = starts[i] >= lo and starts[i + 1] <= hi
            interior += int(inside)
            graph_rows.append((q, categories + i, [], [] if inside else [(0, 3, lo, hi)]))
    return graph_rows, post_rows, interior


def dnf_route_rows(index, query_clauses: list, query_ranges: list | None = None,
                   dual_ratio: float = 1e30, clause_scans: bool = False,
                   with_clause: bool = False) -> tuple:
    """(graph rows, posting rows) of plan_dnf, unsorted: one tuple
    (query, anchor label, residual labels, residual range atoms) per route,
    with the ordinal of the clause the route owns (its position in the
    query's clause list) appended when `with_clause`.

    clause_scans: a clause that carries range atoms and labels also gets the
    route that enumerates its candidates exhaustively -- the reference's
    range route of a hybrid clause (plan.append_range_route,
    dataloader.cpp:9755-9757, appended at :9874-9885), whose candidates are
    the rows of the range slice that satisfy the clause's labels.  Here it
    is a filter-first posting scan over the clause's label of least posting
    size, with the rest of the clause (labels and ranges) as its residual:
    the same candidate set, from a smaller list.  It is not added when the
    clause's own route already is that scan."""
    graph_rows, post_rows = [], []
    for q, clauses in enumerate(query_clauses):
        rng = [tuple(a) for a in (query_ranges[q] if query_ranges is not None else [])]
        for k, (labels, uses_range) in enumerate(clauses):
            labels = [int(l) for l in labels]
            cr = rng if uses_range else []
            if not labels:
                raise ValueError(f"query {q}: a range-only clause needs a range-posting route")
            kind, anchors = clause_anchors(index, labels, dual_ratio)
            if kind == "none":
                continue
            tag = (k,) if with_clause else ()
            for anchor in anchors:
                row = (q, anchor, [l for l in labels if l != anchor], cr) + tag
                (post_rows if kind == "posting" else graph_rows).append(row)
            if clause_scans and cr:
                cand = [l for l in labels if int(index.cat_freq[l]) > 0]
                src = min(cand, key=lambda l: (int(index.cat_freq[l]), l))
                if not (kind == "posting" and anchors == [src]):
                    post_rows.append((q, src, [l for l in labels if l != src], cr) + tag)
    return graph_rows, post_rows


def plan_dnf(index, query_clauses: list, query_ranges: list | None = None,
             sort_by_group: bool = True, seeds: str = "medoid", queries=None,
             dual_ratio: float = 1e30) -> Plan:
    """Routes of queries given in disjunctive normal form: query q is the OR
    of its clauses, clause = (labels, uses_range), where uses_range puts the
    query's range atoms into the clause.  Each clause gets its own routes
    (plan_hybrid_clause_routes, dataloader.cpp:9741-9853, via
    clause_anchors), and each route owns the clause it was planned for: its
    residual predicate is that clause without the anchor label (a singleton
    label group or posting list proves its label, route_predicate_plan.h:
    226-234, 260-276) plus the range atoms when the clause uses them
    (RouteResidualMode::RemainingConjunction, :9513-9609).  Routes of one
    query merge their results (rabitq_lowfreq_merge.h:709-815).  A clause
    with ranges but no label needs a range-posting route, which this
    planner does not produce (ValueError)."""
    graph_rows, post_rows = dnf_route_rows(index, query_clauses, query_ranges, dual_ratio)
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
    return Plan(g, p, off.astype(np.uint32), size.astype(np.uint32), len(query_clauses))


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


# ---------------------------------------------------------------------------
# Pure-range cover over interval labels (range label manifest)
# ---------------------------------------------------------------------------
@dataclass
class RangeLabelIntervals:
    """Per-label interval metadata of a range label manifest
    (RangeLabelIntervals, src/data/dataloader.h:555-563)."""
    range_count: int
    has_interval: np.ndarray   # [labels] u8
    lower: np.ndarray          # [labels] f32
    upper: np.ndarray          # [labels] f32
    level: np.ndarray          # [labels] u32 (UINT32_MAX: none)
    bin: np.ndarray            # [labels] u32
    range_index: np.ndarray    # [labels] u32


def load_range_label_manifest(path, label_count: int) -> RangeLabelIntervals:
    """load_range_label_manifest (dataloader.cpp:6883-7001): JSON with either
    "ranges": [{range_index, levels: [{level_index, partitions: [{label_id,
    interval: [lo, hi], bin_index}]}]}] or a flat "levels" array whose
    partitions carry range_index (default 0)."""
    import json
    U = 0xFFFFFFFF
    iv = RangeLabelIntervals(1, np.zeros(label_count, np.uint8), np.zeros(label_count, np.float32),
                             np.zeros(label_count, np.float32), np.full(label_count, U, np.uint32),
                             np.full(label_count, U, np.uint32), np.full(label_count, U, np.uint32))
    if not path:
        return iv
    with open(path) as f:
        root = json.load(f)
    if not isinstance(root, dict):
        raise ValueError("range label manifest root must be an object")

    def note(r):
        if r != U:
            iv.range_count = max(iv.range_count, r + 1)

    def partitions(levels, range_index):
        for level in levels:
            if not isinstance(level, dict) or not isinstance(level.get("partitions"), list):
                continue
            li = level.get("level_index", U)
            for part in level["partitions"]:
                if not isinstance(part, dict):
                    continue
                lab = part.get("label_id", U)
                if lab >= label_count:
                    raise ValueError("range label manifest label_id out of range")
                pair = part.get("interval")
                if not isinstance(pair, list) or len(pair) != 2:
                    raise ValueError("range label manifest partition missing interval pair")
                r = range_index if range_index is not None else part.get("range_index", 0)
                if range_index is None:
                    note(r)
                iv.has_interval[lab] = 1
                iv.lower[lab], iv.upper[lab] = pair
                iv.level[lab], iv.bin[lab] = li, part.get("bin_index", U)
                iv.range_index[lab] = r

    if "ranges" in root:
        if not isinstance(root["ranges"], list):
            raise ValueError("range label manifest ranges field must be an array")
        for pos, entry in enumerate(root["ranges"]):
            if not isinstance(entry, dict):
                continue
            r = entry.get("range_index", pos)
            note(r)
            if isinstance(entry.get("levels"), list):
                partitions(entry["levels"], r)
        return iv
    if not isinstance(root.get("levels"), list):
        raise ValueError("range label manifest missing levels/ranges array")
    partitions(root["levels"], None)
    return iv


def coarsen_range_cover_bins(child_active: np.ndarray, parent_active: np.ndarray,
                             parent_labels: np.ndarray) -> None:
    """In place: a parent bin whose children are all active (and that has a
    label) becomes active and its children inactive (coarsen_range_cover_bins,
    dataloader.cpp:9104-9130).  Child counts are an integer multiple of the
    parent count."""
    if (len(parent_active) == 0 or len(parent_active) != len(parent_labels)
            or len(child_active) % len(parent_active)):
        raise ValueError("range hierarchy levels must have dense integer-multiple bin counts")
    per = len(child_active) // len(parent_active)
    for p in range(len(parent_active)):
        kids = child_active[p * per:(p + 1) * per]
        if kids.all() and parent_labels[p] != 0xFFFFFFFF:
            kids[:] = 0
            parent_active[p] = 1


@dataclass
class RangeCoverLayout:
    """Labels, lower and upper bounds of every (level, bin) of one range
    dimension (build_range_cover_layout, dataloader.cpp:9141-9202)."""
    domain_low: float
    domain_high: float
    labels: list      # [level] -> u32 array by bin (UINT32_MAX: missing)
    lowers: list
    uppers: list


def build_range_cover_layout(iv: RangeLabelIntervals, range_index: int,
                             usable: np.ndarray | None = None) -> RangeCoverLayout:
    """`usable[label]`: the label has a graph or a posting list
    (range_route_label_usable, dataloader.cpp:7872-7898); default all."""
    U = 0xFFFFFFFF
    mine = (iv.has_interval != 0) & (iv.range_index == range_index)
    if not mine.any():
        raise ValueError("pure-range query requires range_label_manifest_path with valid intervals")
    lo = float(np.min(iv.lower[mine]))
    hi = float(np.max(iv.upper[mine]))
    if not (np.isfinite(lo) and np.isfinite(hi) and lo < hi):
        raise ValueError("pure-range query requires range_label_manifest_path with valid intervals")
    use = mine & (iv.level != U) & (iv.bin != U)
    if usable is not None:
        use &= np.asarray(usable, bool)
    if not use.any():
        raise ValueError("pure-range query requires usable range labels in manifest")
    top = int(iv.level[use].max())
    labels = [np.zeros(0, np.uint32) for _ in range(top + 1)]
    lowers = [np.zeros(0, np.float32) for _ in range(top + 1)]
    uppers = [np.zeros(0, np.float32) for _ in range(top + 1)]
    for lab in np.flatnonzero(use):
        lv, b = int(iv.level[lab]), int(iv.bin[lab])
        if len(labels[lv]) <= b:
            grow = b + 1 - len(labels[lv])
            labels[lv] = np.concatenate([labels[lv], np.full(grow, U, np.uint32)])
            lowers[lv] = np.concatenate([lowers[lv], np.zeros(grow, np.float32)])
            uppers[lv] = np.concatenate([uppers[lv], np.zeros(grow, np.float32)])
        labels[lv][b] = lab
        lowers[lv][b] = iv.lower[lab]
        uppers[lv][b] = iv.upper[lab]
    return RangeCoverLayout(lo, hi, labels, lowers, uppers)


def _overlap(a_lo, a_hi, b_lo, b_hi) -> bool:
    # intervals_overlap (dataloader.cpp:7866-7870), in float32 as the reference
    eps = np.float32(1e-6)
    return bool(np.float32(a_hi) > np.float32(b_lo) + eps and np.float32(a_lo) < np.float32(b_hi) - eps)


def plan_pure_range_cover(layout: RangeCoverLayout, mode: int, lower: float, upper: float,
                          finest_only: bool = False) -> list:
    """Interval labels whose routes cover a query range (plan_pure_range_cover_labels,
    dataloader.cpp:9204-9345): the finest bins overlapping the target, bins
    coarsened into parents whose children are all selected (unless
    finest_only), then a gap-checked walk in (lower, upper, level, bin)
    order.  mode 0 = inactive (no labels); 1 lower bound, 2 upper, 3 both."""
    if mode == 0:
        return []
    f32 = np.float32
    lo, hi = f32(layout.domain_low), f32(layout.domain_high)
    if mode in (1, 3):
        lo = max(lo, f32(lower))
    if mode in (2, 3):
        hi = min(hi, f32(upper))
    if not lo < hi:
        return []
    top = len(layout.labels) - 1
    if len(layout.labels[top]) == 0:
        raise ValueError("pure-range query has no usable finest-level range labels")
    active = [np.zeros(len(l), np.uint8) for l in layout.labels]
    for b, lab in enumerate(layout.labels[top]):
        if lab != 0xFFFFFFFF and _overlap(layout.lowers[top][b], layout.uppers[top][b], lo, hi):
            active[top][b] = 1
    if not active[top].any():
        raise ValueError("unable to construct pure-range cover")
    if not finest_only:
        for lv in range(top, 0, -1):
            if len(active[lv]) and len(layout.labels[lv - 1]):
                coarsen_range_cover_bins(active[lv], active[lv - 1], layout.labels[lv - 1])
    nodes = []
    for lv in range(top + 1):
        for b in np.flatnonzero(active[lv]):
            lab = layout.labels[lv][b]
            if lab == 0xFFFFFFFF:
                raise ValueError("pure-range planner selected missing label")
            nodes.append((f32(layout.lowers[lv][b]), f32(layout.uppers[lv][b]), lv, int(b), int(lab)))
    eps = f32(1e-6)

    def key_cmp(x, y):
        if abs(x[0] - y[0]) > eps:
            return -1 if x[0] < y[0] else 1
        if abs(x[1] - y[1]) > eps:
            return -1 if x[1] < y[1] else 1
        return -1 if (x[2], x[3]) < (y[2], y[3]) else (1 if (x[2], x[3]) > (y[2], y[3]) else 0)

    import functools
    nodes.sort(key=functools.cmp_to_key(key_cmp))
    out, covered = [], lo
    for nlo, nhi, _, _, lab in nodes:
        if nhi <= covered + eps:
            continue
        if nlo > covered + eps:
            raise ValueError("canonical pure-range cover leaves a gap")
        covered = max(covered, nhi)
        out.append(lab)
    if covered < hi - eps:
        raise ValueError("canonical pure-range cover did not reach target interval")
    return out
