"""Host driver of the GPU stage (mirrors backend_pq / backend_rabitq's
init_benchmark_contexts -> execute_single_iteration shape,
src/search/pq/backend_pq.cu:11088-11439): device-resident index arrays,
route batches through the C ABI, rerank, route merge.

All compute runs in libgofann_hip.so kernels; torch supplies device memory
and the stream.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from ._lib import (ELEM_F16, ELEM_F32, ELEM_U8, GraphView, PqView, PredicateView,
                   RabitqQueries, RabitqView, Routes, SearchParams)

DEV = "cuda"


def to_dev(a, dtype=None):
    if a is None:
        return None
    if isinstance(a, torch.Tensor):
        return a.to(DEV).contiguous()
    arr = np.ascontiguousarray(a)
    if arr.dtype.fields is not None:  # structured -> raw bytes
        arr = arr.view(np.uint8).reshape(-1)
    t = torch.from_numpy(arr.copy())
    if dtype is not None:
        t = t.to(dtype)
    return t.to(DEV)


def u32(a):
    """uint32 numpy -> int32 torch bit pattern on the device."""
    return to_dev(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32))


def u64(a):
    return to_dev(np.ascontiguousarray(a, dtype=np.uint64).view(np.int64))


@dataclass
class DeviceGraph:
    graph: torch.Tensor
    row_to_sample: torch.Tensor
    label_offset: torch.Tensor
    csr_offsets: torch.Tensor
    csr_labels: torch.Tensor
    posting_ids: torch.Tensor
    rows: int
    degree: int
    groups: int
    samples: int
    # [rows][degree] sample id of every adjacency entry (optional)
    neighbor_samples: torch.Tensor | None = None

    @classmethod
    def upload(cls, index, neighbor_samples: bool = False) -> "DeviceGraph":
        g = index.graph if index.rows > 0 else np.full((1, index.degree), 0xFFFFFFFF, np.uint32)
        r2s = index.row_to_sample if index.rows > 0 else np.zeros(1, np.uint32)
        dg = cls(u32(g.reshape(-1)), u32(r2s), u32(index.label_offset), u32(index.csr_offsets),
                 u32(index.csr_labels), u32(index.posting_ids), index.rows, index.degree,
                 index.num_labels, int(index.csr_offsets.shape[0] - 1))
        if neighbor_samples:
            dg.neighbor_samples = neighbor_sample_table(dg, index)
        return dg

    def view(self) -> GraphView:
        return GraphView(_lib.ptr(self.graph), _lib.ptr(self.row_to_sample),
                         _lib.ptr(self.label_offset), self.rows, self.degree, self.groups,
                         self.samples, _lib.ptr(self.neighbor_samples))


def neighbor_sample_table(dg: "DeviceGraph", index) -> torch.Tensor:
    """row_to_sample[label_offset[g] + graph[r][j]] for every row r of group
    g (0 where the slot is empty; the kernel never reads those), built on the
    device one group at a time."""
    out = torch.zeros_like(dg.graph)
    if index.rows == 0:
        return out
    deg = index.degree
    g2 = dg.graph.view(-1, deg)
    o2 = out.view(-1, deg)
    r2s = dg.row_to_sample.long() & 0xFFFFFFFF
    for grp in np.nonzero(index.label_size)[0]:
        lo = int(index.label_offset[grp])
        hi = lo + int(index.label_size[grp])
        step = 1 << 20
        for a in range(lo, hi, step):
            b = min(hi, a + step)
            adj = g2[a:b].long() & 0xFFFFFFFF
            valid = adj != 0xFFFFFFFF
            idx = torch.where(valid, adj + lo, torch.zeros_like(adj))
            o2[a:b] = torch.where(valid, r2s[idx], torch.zeros_like(adj)).to(torch.int32)
    return out


SLAB_BYTES = 16
SLAB_CAPACITY = 7
SLAB_OVERFLOW = 0xFFFF


@dataclass
class SampleRecords:
    """Per-sample fixed-width device records: the PQ code row, then a
    16-byte label slab (u16 count, up to 7 u16 labels ascending: the sample's
    CSR row inline).  One cache line per scored candidate serves the code
    gather and its predicate test.  Rows with more than 7 labels (or labels
    >= 0xFFFF) get count 0xFFFF and are read from the CSR."""
    data: torch.Tensor   # u8 [samples][stride]
    pq_dim: int
    stride: int
    slab_offset: int

    @classmethod
    def build(cls, codes: torch.Tensor, csr_offsets: np.ndarray, csr_labels: np.ndarray,
              overflow_every: int = 0) -> "SampleRecords":
        n, M = int(codes.shape[0]), int(codes.shape[1])
        slab_off = (M + 15) // 16 * 16
        stride = slab_off + SLAB_BYTES
        rec = torch.zeros(n, stride, dtype=torch.uint8, device=DEV)
        rec[:, :M] = codes.to(DEV)
        off = torch.from_numpy(csr_offsets.astype(np.int64)).to(DEV)
        lab = torch.from_numpy(csr_labels.astype(np.int64)).to(DEV)
        rec[:, slab_off:] = label_slabs(off, lab, 0, n, overflow_every)
        return cls(rec, M, stride, slab_off)

    def slab(self):
        return self.data.data_ptr() + self.slab_offset, self.stride


def label_slabs(off: torch.Tensor, lab: torch.Tensor, s: int, e: int,
                overflow_every: int = 0) -> torch.Tensor:
    """The 16-byte label slabs (u8 [e - s][16]) of rows s..e of a
    sample-major CSR (device int64 offsets [n + 1] and labels): u16 count,
    then up to 7 u16 labels ascending; count 0xFFFF (labels zeroed) where the
    row has more than 7 labels or a label >= 0xFFFF."""
    o = off[s:e + 1]
    cnt = o[1:] - o[:-1]
    slab = torch.zeros(e - s, 8, dtype=torch.int64, device=off.device)
    ok = cnt <= SLAB_CAPACITY
    for k in range(SLAB_CAPACITY):
        has = cnt > k
        idx = torch.where(has, o[:-1] + k, torch.zeros_like(cnt))
        v = torch.where(has, lab[idx] if lab.numel() else torch.zeros_like(cnt),
                        torch.zeros_like(cnt))
        ok &= v < SLAB_OVERFLOW
        slab[:, k + 1] = v
    if overflow_every > 0:  # test hook: force the CSR path on some rows
        ok &= (torch.arange(s, e, device=off.device) % overflow_every) != 0
    slab[:, 0] = torch.where(ok, cnt, torch.full_like(cnt, SLAB_OVERFLOW))
    slab = torch.where(ok[:, None] | (torch.arange(8, device=off.device) == 0)[None, :], slab,
                       torch.zeros_like(slab))
    return _u16_bytes(slab)


@dataclass
class RabitqRecords:
    """Per-sample RaBitQ records for the graph traversal
    (gofann_rabitq_view.records): the code row, f_add and f_rescale, the
    anchor id, then (optional) the sample's attribute values and its
    16-byte label slab, padded to whole 128-byte lines -- one line per
    scored candidate for 64-byte codes, where the separate arrays cost one
    line each.  The predicate view reads the slab and the attribute values
    in place (DeviceRoutes.predicate_view(records=...))."""
    data: torch.Tensor   # u8 [samples][stride]
    stride: int
    range_offset: int    # -1: no attribute values
    range_stride: int
    slab_offset: int     # -1: no label slab

    @classmethod
    def build(cls, codes: torch.Tensor, factors: torch.Tensor, anchor_ids: torch.Tensor,
              base_ranges=None, csr_offsets=None, csr_labels=None,
              chunk: int = 1 << 22, overflow_every: int = 0) -> "RabitqRecords":
        n, cb = int(codes.shape[0]), int(codes.shape[1])
        if cb % 16:
            raise ValueError("code rows must be a multiple of 16 bytes")
        pos = cb + 12
        r_off, rs = -1, 0
        if base_ranges is not None:
            rs = int(base_ranges.shape[1])
            r_off, pos = pos, pos + 4 * rs
        s_off = -1
        if csr_offsets is not None:
            s_off = (pos + 15) // 16 * 16
            pos = s_off + SLAB_BYTES
        stride = (pos + 127) // 128 * 128
        rec = torch.zeros(n, stride, dtype=torch.uint8, device=DEV)
        br = None
        if base_ranges is not None:
            br = base_ranges if isinstance(base_ranges, torch.Tensor) else \
                torch.from_numpy(np.ascontiguousarray(base_ranges, dtype=np.float32))
        off = lab = None
        if csr_offsets is not None:
            off = torch.from_numpy(np.asarray(csr_offsets).astype(np.int64)).to(DEV)
            lab = torch.from_numpy(np.asarray(csr_labels).astype(np.int64)).to(DEV)
        for s in range(0, n, chunk):
            e = min(n, s + chunk)
            rec[s:e, :cb] = codes[s:e].to(DEV)
            f = factors[s:e, :2].to(DEV, torch.float32).reshape(-1).contiguous()
            rec[s:e, cb:cb + 8] = f.view(torch.uint8).view(e - s, 8)
            a = anchor_ids[s:e].to(DEV, torch.int32).contiguous()
            rec[s:e, cb + 8:cb + 12] = a.view(torch.uint8).view(e - s, 4)
            if br is not None:
                v = br[s:e].to(DEV, torch.float32).reshape(-1).contiguous()
                rec[s:e, r_off:r_off + 4 * rs] = v.view(torch.uint8).view(e - s, 4 * rs)
            if off is not None:
                rec[s:e, s_off:s_off + SLAB_BYTES] = label_slabs(off, lab, s, e, overflow_every)
        return cls(rec, stride, r_off, rs, s_off)

    def view_fields(self):
        """(records pointer, stride) for gofann_rabitq_view."""
        return self.data.data_ptr(), self.stride

    def slab(self):
        if self.slab_offset < 0:
            return None, 0
        return self.data.data_ptr() + self.slab_offset, self.stride

    def ranges(self):
        """(pointer, stride in floats) of the attribute values, or None."""
        if self.range_offset < 0:
            return None
        return self.data.data_ptr() + self.range_offset, self.stride // 4


def _u16_bytes(x: torch.Tensor) -> torch.Tensor:
    """int64 [n][8] values < 2^16 -> little-endian u8 [n][16]."""
    lo = (x & 0xFF).to(torch.uint8)
    hi = ((x >> 8) & 0xFF).to(torch.uint8)
    return torch.stack([lo, hi], dim=-1).reshape(x.shape[0], 16)


@dataclass
class DeviceRoutes:
    route_query: torch.Tensor
    route_group: torch.Tensor
    route_start: torch.Tensor
    launch_order: torch.Tensor
    pred_offsets: torch.Tensor
    pred_handles: torch.Tensor
    pred_clauses: torch.Tensor
    pred_ranges: torch.Tensor
    pred_enabled: torch.Tensor
    pred_compiled: torch.Tensor
    base_ranges: torch.Tensor | None
    range_stride: int
    count: int

    @classmethod
    def upload(cls, rs, base_ranges=None) -> "DeviceRoutes":
        p = rs.predicate
        br = None
        stride = 0
        if base_ranges is not None:
            br = to_dev(np.ascontiguousarray(base_ranges, dtype=np.float32))
            stride = int(base_ranges.shape[1])
        n = max(rs.count, 1)
        return cls(u32(rs.route_query if rs.count else np.zeros(1, np.uint32)),
                   u32(rs.route_group if rs.count else np.zeros(1, np.uint32)),
                   u32(rs.route_start if rs.count else np.zeros(1, np.uint32)),
                   u32(np.arange(n, dtype=np.uint32)),
                   u32(p.route_offsets), u32(p.handles), to_dev(p.clauses), to_dev(p.ranges),
                   to_dev(p.enabled if rs.count else np.zeros(1, np.uint8)),
                   to_dev(p.compiled if rs.count else np.zeros(1, np.uint8)),
                   br, stride, rs.count)

    def routes_view(self, begin: int = 0, end: int | None = None,
                    start: torch.Tensor | None = None) -> Routes:
        """`start`: per-route entry rows to use instead of route_start
        (e.g. CoarseEntry.seeds)."""
        end = self.count if end is None else end
        order = self.launch_order[begin:end]
        st = self.route_start if start is None else start
        return Routes(_lib.ptr(self.route_query), _lib.ptr(self.route_group),
                      _lib.ptr(st), None, None, None, None, None, None, 0,
                      end - begin, _lib.ptr(order))

    def predicate_view(self, dg: DeviceGraph, alpha: float, pending_base_stop: bool,
                       enabled: bool = True,
                       records: "SampleRecords | RabitqRecords | None" = None
                       ) -> PredicateView:
        """`records`: per-sample records whose label slab (and, for
        RabitqRecords holding them, attribute values) the predicate reads in
        place of the separate arrays; the values are the same."""
        slab, slab_stride = records.slab() if records is not None else (None, 0)
        base_ranges, range_stride = _lib.ptr(self.base_ranges), self.range_stride
        columns = 0
        rr = records.ranges() if isinstance(records, RabitqRecords) else None
        if rr is not None and self.base_ranges is not None:
            if records.range_stride != self.range_stride:
                raise ValueError("records hold a different number of attribute columns")
            base_ranges, range_stride = rr
            columns = self.range_stride
        return PredicateView(_lib.ptr(self.pred_offsets), _lib.ptr(self.pred_handles),
                             _lib.ptr(self.pred_clauses), _lib.ptr(self.pred_ranges),
                             _lib.ptr(self.pred_enabled) if enabled else None,
                             _lib.ptr(self.pred_compiled), base_ranges,
                             _lib.ptr(dg.csr_offsets), _lib.ptr(dg.csr_labels),
                             dg.samples, range_stride, float(alpha),
                             1 if pending_base_stop else 0, slab, slab_stride, columns)


class CoarseEntry:
    """Per-route entry rows picked on the GPU from trained coarse centres (an
    IVF-style entry; no counterpart in the reference, which starts every
    route of a label at the label's medoid, dataloader.cpp:7361-7406).

    For route (query q, label group g): the centre c nearest q, then the
    representative row of bucket (g, c) -- the row of g nearest that bucket's
    mean, kept by the graph builder -- or g's medoid when g has no row in
    that bucket.  Everything runs on the device (one GEMM of queries against
    centres, an argmin, a gather), so a step that uses it pays for it."""

    def __init__(self, index, centres: torch.Tensor):
        K = int(centres.shape[0])
        L = int(index.num_labels)
        table = np.repeat(index.seed_local.astype(np.uint32)[:, None], K, axis=1)
        for g in range(L):
            lo, hi = int(index.rep_offset[g]), int(index.rep_offset[g + 1])
            if hi > lo:
                table[g, index.rep_cluster[lo:hi].astype(np.int64)] = index.rep_row[lo:hi]
        self.table = torch.from_numpy(table.reshape(-1).view(np.int32)).to(DEV)
        self.K = K
        self.centres = centres.to(DEV).float().contiguous()
        self.cnorm = (self.centres * self.centres).sum(1)

    def nearest(self, queries: torch.Tensor, chunk: int = 1 << 15) -> torch.Tensor:
        """Nearest centre of every query row (int64 [n])."""
        out = torch.empty(queries.shape[0], dtype=torch.int64, device=DEV)
        for s in range(0, queries.shape[0], chunk):
            q = queries[s:s + chunk].float()
            out[s:s + chunk] = torch.addmm(self.cnorm[None, :], q, self.centres.t(),
                                           alpha=-2.0).argmin(1)
        return out

    def seeds(self, nearest: torch.Tensor, route_query: torch.Tensor, route_group: torch.Tensor,
              out: torch.Tensor | None = None) -> torch.Tensor:
        """int32 [routes] entry rows for routes (route_query, route_group)."""
        c = nearest[route_query.long()]
        idx = route_group.long() * self.K + c
        if out is None:
            return self.table[idx]
        torch.index_select(self.table, 0, idx, out=out)
        return out


def search_params(queue_limit=64, result_width=100, early_stop_mode=_lib.EARLY_STOP_ADAPTIVE,
                  finish_limit=1, max_steps=0, stop_width=10, bias=True,
                  bit_bonus=1.0, range_bonus=1.0, inline_exact=False,
                  table_mode=_lib.PLACE_AUTO, hash_mode=_lib.PLACE_AUTO) -> SearchParams:
    return SearchParams(queue_limit, finish_limit, early_stop_mode, max_steps, stop_width,
                        result_width, bit_bonus, range_bonus, 1 if bias else 0,
                        1 if inline_exact else 0, table_mode, hash_mode)


def pq_view(codes, table: torch.Tensor, exact_base: torch.Tensor | None = None) -> PqView:
    """codes: u8 [samples][M] tensor, or SampleRecords (codes inside records)."""
    if isinstance(codes, SampleRecords):
        return PqView(codes.data.data_ptr(), _lib.ptr(table), int(table.shape[1]), codes.pq_dim,
                      int(codes.data.shape[0]), _lib.ptr(exact_base), codes.stride)
    return PqView(_lib.ptr(codes), _lib.ptr(table), int(table.shape[1]), int(codes.shape[1]),
                  int(codes.shape[0]), _lib.ptr(exact_base), 0)


def query_elem(q: torch.Tensor) -> int:
    if q.dtype == torch.uint8:
        return ELEM_U8
    if q.dtype == torch.float32:
        return ELEM_F32
    raise ValueError("queries must be uint8 or float32")


def run_pq_routes(ctx: _lib.Context, pqv: PqView, queries: torch.Tensor, dg: DeviceGraph,
                  dr: DeviceRoutes, params: SearchParams, alpha: float = 0.15,
                  pending_base_stop: bool = True, begin: int = 0, end: int | None = None,
                  out=None, records: SampleRecords | None = None):
    end = dr.count if end is None else end
    n = dr.count
    W = params.result_width
    if out is None:
        ids = torch.empty(n * W, dtype=torch.int32, device=DEV)
        dists = torch.empty(n * W, dtype=torch.float32, device=DEV)
        stats = torch.zeros(n * 8, dtype=torch.int32, device=DEV)
    else:
        ids, dists, stats = out
    gv = dg.view()
    pv = dr.predicate_view(dg, alpha, pending_base_stop, records=records)
    rv = dr.routes_view(begin, end)
    ctx.check(ctx.lib.gofann_pq_search(ctx.handle, pqv, _lib.ptr(queries), query_elem(queries),
                                       gv, pv, rv, params, _lib.ptr(ids), _lib.ptr(dists),
                                       _lib.ptr(stats)))
    return ids, dists, stats


def run_pq_posting(ctx, pqv: PqView, queries: torch.Tensor, dg: DeviceGraph, dr: DeviceRoutes,
                   cand_offsets, cand_sizes, shortlist_k: int):
    n = dr.count
    ids = torch.empty(max(n, 1) * shortlist_k, dtype=torch.int32, device=DEV)
    dists = torch.empty(max(n, 1) * shortlist_k, dtype=torch.float32, device=DEV)
    passes = torch.empty(max(n, 1), dtype=torch.int32, device=DEV)
    if n == 0:
        return ids[:0], dists[:0], passes[:0]
    co = u32(cand_offsets)
    cs = u32(cand_sizes)
    pv = dr.predicate_view(dg, 0.0, False)
    ctx.check(ctx.lib.gofann_pq_posting_scan(ctx.handle, pqv, _lib.ptr(queries),
                                             query_elem(queries), pv, _lib.ptr(dr.route_query),
                                             _lib.ptr(dg.posting_ids), _lib.ptr(co),
                                             _lib.ptr(cs), n, shortlist_k, _lib.ptr(ids),
                                             _lib.ptr(dists), _lib.ptr(passes)))
    return ids, dists, passes


def exact_rerank(ctx, base: torch.Tensor, queries: torch.Tensor, route_query: torch.Tensor,
                 shortlist: torch.Tensor, width: int, routes: int, topk: int):
    elem = {torch.uint8: ELEM_U8, torch.float32: ELEM_F32, torch.float16: ELEM_F16}[base.dtype]
    ids = torch.empty(max(routes, 1) * topk, dtype=torch.int32, device=DEV)
    dists = torch.empty(max(routes, 1) * topk, dtype=torch.float32, device=DEV)
    if routes == 0:
        return ids[:0], dists[:0]
    ctx.check(ctx.lib.gofann_exact_rerank(ctx.handle, _lib.ptr(base), elem, int(base.shape[1]),
                                          int(base.shape[0]), _lib.ptr(queries),
                                          _lib.ptr(route_query), _lib.ptr(shortlist), width,
                                          routes, topk, _lib.ptr(ids), _lib.ptr(dists)))
    return ids, dists


def exact_posting(ctx, base: torch.Tensor, queries: torch.Tensor, route_query, cand_ids,
                  cand_offsets, cand_sizes, topk: int, order: int = _lib.EXACT_ORDER_SERIAL,
                  predicate: PredicateView | None = None):
    """Exact posting scan (gofann_exact_posting_scan; the full-GPU backend's
    posting routes, backend_full_gpu.cu:1383-1493 and 2124-2262): per route
    the topk distinct listed samples by exact (distance, id), in the serial
    or the warp summation order.  base and queries: device rows of one
    element type.  Returns (ids, dists, pass counts) device tensors."""
    if queries.dtype != base.dtype:
        raise ValueError("queries must have the element type of the base rows")
    elem = {torch.uint8: ELEM_U8, torch.float32: ELEM_F32, torch.float16: ELEM_F16}[base.dtype]
    def dev(a):
        return a.to(DEV, torch.int32).contiguous() if isinstance(a, torch.Tensor) else u32(a)

    rq = dev(route_query)
    n = int(rq.shape[0])
    ids = torch.empty(max(n, 1) * topk, dtype=torch.int32, device=DEV)
    dists = torch.empty(max(n, 1) * topk, dtype=torch.float32, device=DEV)
    passes = torch.empty(max(n, 1), dtype=torch.int32, device=DEV)
    if n == 0:
        return ids[:0], dists[:0], passes[:0]
    ci, co, cs = dev(cand_ids), dev(cand_offsets), dev(cand_sizes)
    pv = predicate if predicate is not None else PredicateView()
    ctx.check(ctx.lib.gofann_exact_posting_scan(ctx.handle, _lib.ptr(base), elem,
                                                int(base.shape[1]), int(base.shape[0]),
                                                _lib.ptr(queries), pv, _lib.ptr(rq),
                                                _lib.ptr(ci), _lib.ptr(co), _lib.ptr(cs), n, topk,
                                                order, _lib.ptr(ids), _lib.ptr(dists),
                                                _lib.ptr(passes)))
    return ids, dists, passes


def merge_routes(route_to_query: np.ndarray, ids: np.ndarray, dists: np.ndarray, queries: int,
                 topk: int):
    """Route -> original query merge (rabitq_lowfreq_merge.h:709-815):
    minimum distance per sample, (distance, id) order, top-k."""
    width = ids.shape[1] if ids.ndim == 2 else topk
    ids = ids.reshape(-1, width)
    dists = dists.reshape(-1, width)
    out_i = np.full((queries, topk), 0xFFFFFFFF, dtype=np.uint32)
    out_d = np.full((queries, topk), np.finfo(np.float32).max, dtype=np.float32)
    q_of = np.repeat(route_to_query.astype(np.int64), width)
    fi = ids.reshape(-1).astype(np.uint32)
    fd = dists.reshape(-1)
    ok = fi != 0xFFFFFFFF
    q_of, fi, fd = q_of[ok], fi[ok], fd[ok]
    order = np.lexsort((fd, fi, q_of))  # per query, per sample, min distance first
    q_of, fi, fd = q_of[order], fi[order], fd[order]
    first = np.ones(len(fi), dtype=bool)
    first[1:] = (q_of[1:] != q_of[:-1]) | (fi[1:] != fi[:-1])
    q_of, fi, fd = q_of[first], fi[first], fd[first]
    order = np.lexsort((fi, fd, q_of))
    q_of, fi, fd = q_of[order], fi[order], fd[order]
    start = np.searchsorted(q_of, np.arange(queries))
    rank = np.arange(len(q_of)) - start[q_of]
    keep = rank < topk
    out_i[q_of[keep], rank[keep]] = fi[keep]
    out_d[q_of[keep], rank[keep]] = fd[keep]
    return out_i, out_d


def query_route_csr(route_to_query: np.ndarray, queries: int):
    """CSR of routes per original query (route ids grouped by query)."""
    r2q = np.asarray(route_to_query, dtype=np.int64)
    order = np.argsort(r2q, kind="stable").astype(np.uint32)
    counts = np.bincount(r2q, minlength=queries)
    offsets = np.zeros(queries + 1, dtype=np.uint32)
    np.cumsum(counts, out=offsets[1:])
    return offsets, order


def merge_routes_gpu(ctx, q_offsets: torch.Tensor, q_routes: torch.Tensor, ids: torch.Tensor,
                     dists: torch.Tensor, width: int, queries: int, topk: int):
    out_i = torch.empty(max(queries, 1) * topk, dtype=torch.int32, device=DEV)
    out_d = torch.empty(max(queries, 1) * topk, dtype=torch.float32, device=DEV)
    if queries == 0:
        return out_i[:0], out_d[:0]
    ctx.check(ctx.lib.gofann_merge_routes(ctx.handle, _lib.ptr(q_offsets), _lib.ptr(q_routes),
                                          _lib.ptr(ids), _lib.ptr(dists), width, queries, topk,
                                          _lib.ptr(out_i), _lib.ptr(out_d)))
    return out_i, out_d


# ---------------------------------------------------------------------------
# Host side: streamed CPU exact rerank (libgofann_hip.so host pool).
# ---------------------------------------------------------------------------
def _np_ptr(a: np.ndarray) -> int:
    return a.ctypes.data


class HostRerank:
    """CPU exact rerank over host copies of the base vectors and queries
    (gofann_host_rerank_*): a worker pool that reranks GPU shortlists, alone
    or streamed behind the GPU search in route chunks."""

    def __init__(self, base: np.ndarray, queries: np.ndarray, threads: int = 16):
        import ctypes as C
        self.lib = _lib.load()
        elem = {np.dtype(np.uint8): ELEM_U8, np.dtype(np.float32): ELEM_F32,
                np.dtype(np.float16): ELEM_F16}[base.dtype]
        self.base = np.ascontiguousarray(base)
        self.queries = np.ascontiguousarray(queries, dtype=np.uint8 if elem == ELEM_U8
                                            else np.float32)
        h = C.c_void_p()
        rc = self.lib.gofann_host_rerank_create(_np_ptr(self.base), elem, self.base.shape[1],
                                                self.base.shape[0], _np_ptr(self.queries),
                                                threads, C.byref(h))
        if rc != 0:
            raise _lib.GofannError(f"gofann_host_rerank_create failed ({rc})")
        self.handle = h

    @property
    def fp16_kernel(self) -> str:
        """The fp16 L2 kernel chosen at create ("scalar", "avx2", "avx512")."""
        return self.lib.gofann_host_rerank_fp16_kernel(self.handle).decode()

    def _check(self, rc):
        if rc != 0:
            msg = self.lib.gofann_host_rerank_last_error(self.handle)
            raise _lib.GofannError(f"host rerank failed ({rc}): {msg.decode() if msg else ''}")

    def rerank(self, shortlist: np.ndarray, route_query: np.ndarray, topk: int):
        sl = np.ascontiguousarray(shortlist, dtype=np.uint32)
        rq = np.ascontiguousarray(route_query, dtype=np.uint32)
        n, width = sl.shape
        ids = np.empty((n, topk), np.uint32)
        dists = np.empty((n, topk), np.float32)
        self._check(self.lib.gofann_host_rerank_routes(self.handle, _np_ptr(sl), width,
                                                       _np_ptr(rq), n, topk, _np_ptr(ids),
                                                       _np_ptr(dists)))
        return ids, dists

    def search(self, ctx, pqv: PqView, queries: torch.Tensor, dg: DeviceGraph,
               dr: "DeviceRoutes", params: SearchParams, route_query: np.ndarray,
               chunk_routes: int, topk: int, alpha: float = 0.15,
               pending_base_stop: bool = True, records: "SampleRecords | None" = None,
               stats: torch.Tensor | None = None, out=None):
        """GPU traversal in chunks with the shortlist handed to the host pool
        chunk by chunk (gofann_pq_search_host_rerank); host outputs."""
        n = dr.count
        rq = np.ascontiguousarray(route_query, dtype=np.uint32)
        if out is None:
            out = (np.empty((n, topk), np.uint32), np.empty((n, topk), np.float32))
        ids, dists = out
        gv = dg.view()
        pv = dr.predicate_view(dg, alpha, pending_base_stop, records=records)
        rv = Routes(_lib.ptr(dr.route_query), _lib.ptr(dr.route_group), _lib.ptr(dr.route_start),
                    None, None, None, None, None, None, 0, n, None)
        ctx.check(self.lib.gofann_pq_search_host_rerank(
            ctx.handle, self.handle, pqv, _lib.ptr(queries), query_elem(queries), gv, pv, rv,
            params, _np_ptr(rq), chunk_routes, topk, _np_ptr(ids), _np_ptr(dists),
            _lib.ptr(stats)))
        return ids, dists

    def close(self):
        if getattr(self, "handle", None):
            self.lib.gofann_host_rerank_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class StreamedRerank:
    """Host exact rerank streamed behind GPU work in route chunks, for any
    producer of device shortlists (the schedule of the reference's
    run_highfreq_streaming_rerank, backend_pq.cu:9646-9738, which overlaps
    the host rerank of finished routes with the search of the next ones).

    run() takes tasks (r0, r1, launch): launch() enqueues, on the current
    stream, the GPU work that writes the shortlist rows [r0, r1) of `d_ids`
    (width ids each).  After each task an event is recorded; a copy stream
    waits for it and copies the task's rows into pinned host memory; a host
    thread waits for each copy and reranks those routes with the HostRerank
    pool while the GPU runs later tasks.  Timing of the last run:
    gpu_ms = GPU time from the first launch to the end of the last (events
    on the compute stream), wall_ms = the whole call, exposed_ms =
    wall_ms - gpu_ms (rerank time not hidden behind the GPU)."""

    def __init__(self, hr: HostRerank, rows: int, width: int):
        self.hr, self.width = hr, int(width)
        self.pinned = torch.empty(max(int(rows), 1) * self.width, dtype=torch.int32,
                                  pin_memory=True)
        self.copy_stream = torch.cuda.Stream()
        self.timing = {}

    def run(self, tasks, d_ids: torch.Tensor, route_query: np.ndarray, topk: int,
            out_ids: np.ndarray, out_dists: np.ndarray):
        import queue
        import threading
        import time
        W = self.width
        rq = np.ascontiguousarray(route_query, dtype=np.uint32)
        base = self.pinned.data_ptr()
        lib, handle = self.hr.lib, self.hr.handle
        work: queue.Queue = queue.Queue()
        errors = []

        def worker():
            while True:
                item = work.get()
                if item is None:
                    return
                r0, r1, done = item
                done.synchronize()
                if errors:
                    continue
                rc = lib.gofann_host_rerank_routes(
                    handle, base + r0 * W * 4, W, _np_ptr(rq) + r0 * 4, r1 - r0, topk,
                    _np_ptr(out_ids) + r0 * topk * 4, _np_ptr(out_dists) + r0 * topk * 4)
                if rc != 0:
                    errors.append(rc)

        cur = torch.cuda.current_stream()
        t0 = time.perf_counter()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        th = threading.Thread(target=worker, daemon=True)
        th.start()
        try:
            e0.record(cur)
            for r0, r1, launch in tasks:
                launch()
                ready = torch.cuda.Event()
                ready.record(cur)
                self.copy_stream.wait_event(ready)
                with torch.cuda.stream(self.copy_stream):
                    self.pinned[r0 * W:r1 * W].copy_(d_ids[r0 * W:r1 * W], non_blocking=True)
                    done = torch.cuda.Event()
                    done.record(self.copy_stream)
                work.put((r0, r1, done))
            e1.record(cur)
        finally:
            work.put(None)
            th.join()
        wall = (time.perf_counter() - t0) * 1000.0
        e1.synchronize()
        gpu = e0.elapsed_time(e1)
        if errors:
            self.hr._check(errors[0])
        self.timing = {"gpu_ms": gpu, "wall_ms": wall, "exposed_ms": max(0.0, wall - gpu)}
        return out_ids, out_dists


def host_merge_routes(route_to_query: np.ndarray, ids: np.ndarray, dists: np.ndarray,
                      queries: int, topk: int):
    """Route -> query merge on the host (gofann_host_merge_routes)."""
    lib = _lib.load()
    off, order = query_route_csr(route_to_query, queries)
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    dists = np.ascontiguousarray(dists, dtype=np.float32)
    width = ids.shape[1] if ids.ndim == 2 else topk
    out_i = np.empty((queries, topk), np.uint32)
    out_d = np.empty((queries, topk), np.float32)
    rc = lib.gofann_host_merge_routes(_np_ptr(off), _np_ptr(order), _np_ptr(ids), _np_ptr(dists),
                                      width, queries, topk, _np_ptr(out_i), _np_ptr(out_d))
    if rc != 0:
        raise _lib.GofannError(f"gofann_host_merge_routes failed ({rc})")
    return out_i, out_d
