"""Ordered range postings and the RaBitQ range-posting scan.

Index layout (range_posting::Index, src/index/range_posting_index.h:12-92):
for every range dimension the sample ids ordered by the sample's value in
that dimension, the dimension's strictly increasing unique values and the
row offsets of each value's run.  On disk this is the reference's FARPIDX1
file (FileHeader 40 bytes, one 72-byte DimensionDescriptor per dimension,
64-byte aligned arrays); on the device the dimensions' sample-id arrays are
concatenated, dimension r at rows [r * row_count, (r + 1) * row_count).

A route with active ranges scans the smallest slice one of its ranges
selects (choose_smallest_slice, range_posting_index.cpp:277-312) -- split
into segments of about `segment_rows` rows (posting_segment_plan.h:20-51)
so long slices spread over many workgroups -- and the segments' shortlists
merge per route (posting_segment_merge.cuh:12-46).  Planning runs in the C
library (gofann_posting_segment_plan, gofann_range_slices); scoring in the
HIP kernels behind gofann_rabitq_range_scan.
"""
from __future__ import annotations

import ctypes as C
import os
import struct
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch

from . import _lib

MAGIC = b"FARPIDX1"
VERSION = 1
HEADER = struct.Struct("<8sIIQQII")          # FileHeader, 40 bytes
DESCRIPTOR = struct.Struct("<IIQQQQQQQQ")    # DimensionDescriptor, 72 bytes
ALIGNMENT = 64
DEFAULT_SEGMENT_ROWS = 4096                  # rabitq_range_posting_segment_rows


def _align(x: int) -> int:
    return (x + ALIGNMENT - 1) // ALIGNMENT * ALIGNMENT


class RangeIndexError(RuntimeError):
    pass


@dataclass
class RangeDimension:
    unique_values: np.ndarray  # float32 [unique], strictly increasing, finite
    offsets: np.ndarray        # uint64 [unique + 1], 0 .. row_count
    sample_ids: np.ndarray     # uint32 [row_count], a permutation of [0, row_count)


class RangePostingIndex:
    """Ordered range postings of every range dimension of the base."""

    def __init__(self, row_count: int, dimensions: list[RangeDimension]):
        self.row_count = int(row_count)
        self.dimensions = dimensions

    @property
    def range_count(self) -> int:
        return len(self.dimensions)

    @classmethod
    def build(cls, base_range_values: np.ndarray) -> "RangePostingIndex":
        """From base values [rows][range_count]: ids ordered by (value, id)."""
        v = np.asarray(base_range_values, dtype=np.float32)
        if v.ndim != 2 or v.shape[0] == 0 or v.shape[1] == 0:
            raise RangeIndexError("base range values must be a nonempty [rows][ranges] matrix")
        if not np.all(np.isfinite(v)):
            raise RangeIndexError("base range values must be finite")
        rows = v.shape[0]
        dims = []
        for r in range(v.shape[1]):
            col = v[:, r]
            order = np.argsort(col, kind="stable").astype(np.uint32)
            uniq, counts = np.unique(col, return_counts=True)
            offsets = np.zeros(uniq.size + 1, np.uint64)
            np.cumsum(counts, out=offsets[1:])
            dims.append(RangeDimension(uniq.astype(np.float32), offsets, order))
        return cls(rows, dims)

    # -- FARPIDX1 -----------------------------------------------------------
    def write(self, path: str | os.PathLike) -> None:
        header_bytes = HEADER.size + DESCRIPTOR.size * self.range_count
        cursor = _align(header_bytes)
        descs = []
        for r, d in enumerate(self.dimensions):
            vb = d.unique_values.size * 4
            ob = d.offsets.size * 8
            sb = d.sample_ids.size * 4
            vo = cursor
            oo = _align(vo + vb)
            so = _align(oo + ob)
            cursor = _align(so + sb)
            descs.append((r, 0, d.unique_values.size, d.sample_ids.size, vo, oo, so, vb, ob, sb))
        with open(path, "wb") as f:
            f.write(HEADER.pack(MAGIC, VERSION, header_bytes, cursor, self.row_count,
                                self.range_count, 0))
            for t in descs:
                f.write(DESCRIPTOR.pack(*t))
            for t, d in zip(descs, self.dimensions):
                for off, arr, dt in ((t[4], d.unique_values, "<f4"), (t[5], d.offsets, "<u8"),
                                     (t[6], d.sample_ids, "<u4")):
                    f.write(b"\0" * (off - f.tell()))
                    f.write(np.ascontiguousarray(arr, dtype=dt).tobytes())
            f.write(b"\0" * (cursor - f.tell()))

    @classmethod
    def load(cls, path: str | os.PathLike) -> "RangePostingIndex":
        """Memory-maps a FARPIDX1 file and applies the loader's checks
        (range_posting_index.cpp:150-260)."""
        size = Path(path).stat().st_size
        if size < HEADER.size:
            raise RangeIndexError("file is too small")
        mm = np.memmap(path, dtype=np.uint8, mode="r")
        magic, version, header_bytes, file_bytes, rows, ranges, _ = HEADER.unpack_from(mm, 0)
        if magic != MAGIC:
            raise RangeIndexError("magic mismatch")
        if version != VERSION:
            raise RangeIndexError(f"unsupported version {version}")
        if file_bytes != size:
            raise RangeIndexError("header file size does not match the actual file")
        if rows == 0 or rows > 0xFFFFFFFF:
            raise RangeIndexError("row count must fit nonzero uint32 sample ids")
        if ranges == 0:
            raise RangeIndexError("range count must be nonzero")
        if header_bytes != HEADER.size + DESCRIPTOR.size * ranges or header_bytes > size:
            raise RangeIndexError("descriptor table size is invalid")

        def region(off, nbytes, count, item, name):
            if nbytes != count * item:
                raise RangeIndexError(f"{name} byte count does not match element count")
            if off % item or off > size or nbytes > size - off:
                raise RangeIndexError(f"{name} region is unaligned or outside the file")
            return off

        dims = []
        for r in range(ranges):
            (ri, res, uc, rc, vo, oo, so, vb, ob, sb) = DESCRIPTOR.unpack_from(
                mm, HEADER.size + r * DESCRIPTOR.size)
            if ri != r or res != 0:
                raise RangeIndexError("dimension descriptors must be dense, ordered, and reserved-zero")
            if rc != rows or uc == 0 or uc > rc:
                raise RangeIndexError("dimension row count mismatch or invalid value-domain size")
            vals = np.frombuffer(mm, "<f4", uc, region(vo, vb, uc, 4, "unique values"))
            offs = np.frombuffer(mm, "<u8", uc + 1, region(oo, ob, uc + 1, 8, "value offsets"))
            ids = np.frombuffer(mm, "<u4", rc, region(so, sb, rc, 4, "sample ids"))
            if not np.all(np.isfinite(vals)) or not np.all(vals[1:] > vals[:-1]):
                raise RangeIndexError("unique values must be finite and strictly increasing")
            if offs[0] != 0 or offs[-1] != rc:
                raise RangeIndexError("value offsets must begin at zero and end at row_count")
            if not np.all(offs[1:] >= offs[:-1]):
                raise RangeIndexError("value offsets must be monotonic and in range")
            if ids.size and int(ids.max()) >= rc:
                raise RangeIndexError("sample id is outside the base row range")
            if np.unique(ids).size != rc:
                raise RangeIndexError("sample ids must form a permutation without duplicates")
            dims.append(RangeDimension(vals, offs, ids))
        return cls(rows, dims)

    # -- device -------------------------------------------------------------
    def device_postings(self, device="cuda") -> torch.Tensor:
        """[range_count * row_count] sample ids, dimension r at r * row_count."""
        flat = np.concatenate([d.sample_ids for d in self.dimensions]).astype(np.uint32)
        return torch.from_numpy(flat.view(np.int32)).to(device)

    @property
    def resident_rows(self) -> int:
        return self.row_count * self.range_count


def choose_slices(index: RangePostingIndex, modes: np.ndarray, lower: np.ndarray,
                  upper: np.ndarray) -> np.ndarray:
    """[n][5] uint64: has_active_range, active_dimension_count, range_index,
    begin (dimension-local), count -- through gofann_range_slices."""
    lib = _lib.load()
    modes = np.ascontiguousarray(modes, np.uint8)
    lower = np.ascontiguousarray(lower, np.float32)
    upper = np.ascontiguousarray(upper, np.float32)
    n, rc = modes.shape
    if rc != index.range_count:
        raise RangeIndexError("query and posting range counts do not match")
    vals = [np.ascontiguousarray(d.unique_values, np.float32) for d in index.dimensions]
    offs = [np.ascontiguousarray(d.offsets, np.uint64) for d in index.dimensions]
    vptr = (C.c_void_p * rc)(*[v.ctypes.data for v in vals])
    optr = (C.c_void_p * rc)(*[o.ctypes.data for o in offs])
    uc = np.array([v.size for v in vals], np.uint64)
    out = np.zeros((max(n, 1), 5), np.uint64)
    rcode = lib.gofann_range_slices(C.cast(vptr, C.c_void_p), C.cast(optr, C.c_void_p),
                                    uc.ctypes.data, rc, modes.ctypes.data, lower.ctypes.data,
                                    upper.ctypes.data, n, out.ctypes.data)
    if rcode != _lib.OK:
        raise RangeIndexError(f"gofann_range_slices failed ({rcode})")
    return out[:n]


@dataclass
class SegmentPlan:
    route_ids: np.ndarray     # uint32 [count]
    positions: np.ndarray     # uint32 [count] output row of each segment
    offsets: np.ndarray       # uint64 [count]
    sizes: np.ndarray         # uint64 [count]
    query_indptr: np.ndarray  # uint32 [n + 1]

    @property
    def count(self) -> int:
        return int(self.route_ids.size)


def segment_plan(route_ids, offsets, sizes, target_rows: int = DEFAULT_SEGMENT_ROWS) -> SegmentPlan:
    """posting_segments::make_plan through gofann_posting_segment_plan."""
    lib = _lib.load()
    r = np.ascontiguousarray(route_ids, np.uint32)
    o = np.ascontiguousarray(offsets, np.uint64)
    s = np.ascontiguousarray(sizes, np.uint64)
    n = r.size
    if target_rows <= 0:
        raise RangeIndexError("target_rows must be positive")
    cnt = C.c_uint32(0)
    # First call sizes the plan (capacity 0 leaves the outputs untouched).
    rc = lib.gofann_posting_segment_plan(r.ctypes.data, o.ctypes.data, s.ctypes.data, n,
                                         target_rows, 0, None, None, None, None, None,
                                         C.byref(cnt))
    if rc == _lib.ERR_UNSUPPORTED:
        raise RangeIndexError("segment plan overflows")
    m = cnt.value
    plan = SegmentPlan(np.empty(m, np.uint32), np.empty(m, np.uint32), np.empty(m, np.uint64),
                       np.empty(m, np.uint64), np.empty(n + 1, np.uint32))
    rc = lib.gofann_posting_segment_plan(r.ctypes.data, o.ctypes.data, s.ctypes.data, n,
                                         target_rows, m, plan.route_ids.ctypes.data,
                                         plan.positions.ctypes.data, plan.offsets.ctypes.data,
                                         plan.sizes.ctypes.data, plan.query_indptr.ctypes.data,
                                         C.byref(cnt))
    if rc != _lib.OK:
        raise RangeIndexError(f"segment plan failed ({rc})")
    return plan


class DeviceSegments:
    """A SegmentPlan on the device and its gofann_posting_segments view."""

    def __init__(self, plan: SegmentPlan, merged: bool = True, device="cuda"):
        self.plan = plan
        self.route_ids = torch.from_numpy(plan.route_ids.view(np.int32)).to(device)
        self.offsets = torch.from_numpy(plan.offsets.view(np.int64)).to(device)
        self.sizes = torch.from_numpy(plan.sizes.view(np.int64)).to(device)
        self.indptr = (torch.from_numpy(plan.query_indptr.view(np.int32)).to(device)
                       if merged else None)
        self.positions = plan.query_indptr.size - 1 if merged else plan.count

    def view(self) -> _lib.PostingSegments:
        return _lib.PostingSegments(_lib.ptr(self.route_ids), _lib.ptr(self.offsets),
                                    _lib.ptr(self.sizes), self.plan.count,
                                    _lib.ptr(self.indptr), self.positions if self.indptr is not None else 0)


SHARE_ROUTES = 16  # segments per share item (kShareRoutes)


@dataclass
class SharePlan:
    """Segments of a SegmentPlan that scan the same posting rows, grouped:
    item i covers rows [offsets[i], + sizes[i]) for plan segments
    slots[begin[i] .. begin[i + 1])."""
    offsets: np.ndarray
    sizes: np.ndarray
    begin: np.ndarray
    slots: np.ndarray

    @property
    def items(self) -> int:
        return int(self.offsets.size)


def share_plan(plan: SegmentPlan, routes_per_item: int = SHARE_ROUTES) -> SharePlan:
    """Groups the plan's segments by (offset, size) -- the routes of one
    label cut the same way -- into items of at most `routes_per_item`,
    the heaviest items (rows x routes) first.  `routes_per_item` is 1 to
    SHARE_ROUTES: the kernel holds that many route slots per pass over an
    item's rows, so a larger item would re-read its rows."""
    if not 1 <= int(routes_per_item) <= SHARE_ROUTES:
        raise ValueError(f"routes_per_item must be 1..{SHARE_ROUTES}, got {routes_per_item}")
    m = plan.count
    if m == 0:
        z = np.zeros(0, np.uint64)
        return SharePlan(z, z, np.zeros(1, np.uint32), np.zeros(0, np.uint32))
    order = np.lexsort((np.arange(m), plan.sizes, plan.offsets))
    o, sz = plan.offsets[order], plan.sizes[order]
    new = np.ones(m, bool)
    new[1:] = (o[1:] != o[:-1]) | (sz[1:] != sz[:-1])
    gid = np.cumsum(new) - 1
    gstart = np.flatnonzero(new)
    # position inside the group, then items of routes_per_item
    pos = np.arange(m) - gstart[gid]
    item_key = gid * (m + 1) + pos // routes_per_item
    istart = np.flatnonzero(np.r_[True, item_key[1:] != item_key[:-1]])
    counts = np.diff(np.r_[istart, m])
    weight = sz[istart].astype(np.float64) * counts
    iorder = np.argsort(-weight, kind="stable")
    slots, offs, sizes, begin = [], [], [], [0]
    for i in iorder:
        a = istart[i]
        slots.append(order[a:a + counts[i]])
        offs.append(o[a])
        sizes.append(sz[a])
        begin.append(begin[-1] + int(counts[i]))
    return SharePlan(np.array(offs, np.uint64), np.array(sizes, np.uint64),
                     np.array(begin, np.uint32), np.concatenate(slots).astype(np.uint32))


class DeviceShare:
    """A SharePlan on the device and its gofann_posting_share view."""

    def __init__(self, sp: SharePlan, device="cuda"):
        self.sp = sp
        self.offsets = torch.from_numpy(sp.offsets.view(np.int64)).to(device)
        self.sizes = torch.from_numpy(sp.sizes.view(np.int64)).to(device)
        self.begin = torch.from_numpy(sp.begin.view(np.int32)).to(device)
        self.slots = torch.from_numpy(sp.slots.view(np.int32)).to(device)

    def view(self) -> _lib.PostingShare:
        return _lib.PostingShare(_lib.ptr(self.offsets), _lib.ptr(self.sizes),
                                 _lib.ptr(self.begin), _lib.ptr(self.slots), self.sp.items)


def route_postings(index: RangePostingIndex, slices: np.ndarray):
    """Flat device offsets and sizes of each route's chosen slice."""
    rng = slices[:, 2].astype(np.int64)
    rng[slices[:, 0] == 0] = 0
    offsets = (rng.astype(np.uint64) * np.uint64(index.row_count) + slices[:, 3]).astype(np.uint64)
    sizes = np.where(slices[:, 0] != 0, slices[:, 4], 0).astype(np.uint64)
    return offsets, sizes


class PostingRows:
    """Posting-order copies of the RaBitQ rows (gofann_rabitq_posting_rows):
    codes [rows][padded_dim/8] and aux [rows][4] u32, so the range scan
    streams them instead of gathering by sample id."""

    def __init__(self, ctx: _lib.Context, rv: _lib.RabitqView, postings: torch.Tensor,
                 rows: int):
        self.rows = int(rows)
        dev = postings.device
        self.codes = torch.empty(max(self.rows, 1), rv.padded_dim // 8, dtype=torch.uint8,
                                 device=dev)
        self.aux = torch.empty(max(self.rows, 1), 4, dtype=torch.int32, device=dev)
        ctx.check(ctx.lib.gofann_rabitq_posting_rows(ctx.handle, rv, _lib.ptr(postings),
                                                      self.rows, _lib.ptr(self.codes),
                                                      _lib.ptr(self.aux)))


class PostingPredicateColumns:
    """Posting-order predicate columns (gofann_posting_predicate_rows): each
    posting row's 16-byte label slab [rows][4] u32 and base range row
    [rows][range_stride] f32, so a label-posting scan streams its filter's
    inputs instead of gathering them by sample id.  The range row holds the
    view's attribute columns (range_columns, else range_stride)."""

    def __init__(self, ctx: _lib.Context, pred: _lib.PredicateView, postings: torch.Tensor,
                 rows: int):
        self.rows = int(rows)
        dev = postings.device
        stride = int(pred.range_columns or pred.range_stride)
        self.slab = torch.empty(max(self.rows, 1), 4, dtype=torch.int32, device=dev)
        self.ranges = (torch.empty(max(self.rows * stride, 1), dtype=torch.float32, device=dev)
                       if stride else None)
        ctx.check(ctx.lib.gofann_posting_predicate_rows(
            ctx.handle, pred, _lib.ptr(postings), self.rows, _lib.ptr(self.slab),
            _lib.ptr(self.ranges) if self.ranges is not None else None))


def rabitq_posting_scan_segments(ctx: _lib.Context, rv: _lib.RabitqView,
                                 rq: _lib.RabitqQueries, pred: _lib.PredicateView,
                                 route_query: torch.Tensor, postings: torch.Tensor,
                                 posting_rows: int, segs: DeviceSegments, shortlist_k: int,
                                 rows: PostingRows | None = None,
                                 cols: PostingPredicateColumns | None = None, out=None,
                                 share: DeviceShare | None = None):
    """Runs gofann_rabitq_posting_scan_segments (with `share`, and the rows
    and columns, gofann_rabitq_posting_scan_shared: the same outputs);
    returns (ids int32, dists, passes) on the device, [positions][shortlist_k]
    (into `out` = (ids, dists, passes) flat tensors when given)."""
    n = segs.positions
    dev = postings.device
    if out is None:
        out = (torch.empty(max(n, 1) * shortlist_k, dtype=torch.int32, device=dev),
               torch.empty(max(n, 1) * shortlist_k, dtype=torch.float32, device=dev),
               torch.empty(max(n, 1), dtype=torch.int32, device=dev))
    ids, dists, passes = out
    if share is not None:
        if rows is None or cols is None:
            raise RangeIndexError("the shared scan reads the posting-order rows and columns")
        ctx.check(ctx.lib.gofann_rabitq_posting_scan_shared(
            ctx.handle, rv, rq, pred, _lib.ptr(route_query), _lib.ptr(postings),
            int(posting_rows), segs.view(), share.view(), shortlist_k, _lib.ptr(rows.codes),
            _lib.ptr(rows.aux), _lib.ptr(cols.slab),
            _lib.ptr(cols.ranges) if cols.ranges is not None else None,
            _lib.ptr(ids), _lib.ptr(dists), _lib.ptr(passes)))
        return (ids[: n * shortlist_k].view(n, shortlist_k),
                dists[: n * shortlist_k].view(n, shortlist_k), passes[:n])
    ctx.check(ctx.lib.gofann_rabitq_posting_scan_segments(
        ctx.handle, rv, rq, pred, _lib.ptr(route_query), _lib.ptr(postings), int(posting_rows),
        segs.view(), shortlist_k,
        _lib.ptr(rows.codes) if rows is not None else None,
        _lib.ptr(rows.aux) if rows is not None else None,
        _lib.ptr(cols.slab) if cols is not None else None,
        _lib.ptr(cols.ranges) if cols is not None and cols.ranges is not None else None,
        _lib.ptr(ids), _lib.ptr(dists), _lib.ptr(passes)))
    return (ids[: n * shortlist_k].view(n, shortlist_k),
            dists[: n * shortlist_k].view(n, shortlist_k), passes[:n])


def rabitq_range_scan(ctx: _lib.Context, rv: _lib.RabitqView, rq: _lib.RabitqQueries,
                      pred: _lib.PredicateView, routes: _lib.Routes, postings: torch.Tensor,
                      resident_rows: int, segs: DeviceSegments, shortlist_k: int,
                      score_first: bool = False, rows: PostingRows | None = None):
    """Runs gofann_rabitq_range_scan (or, given posting-order `rows`,
    gofann_rabitq_range_scan_resident); returns (ids int32, dists, passes)
    on the device, [rows][shortlist_k]."""
    n = segs.positions
    ids = torch.empty(max(n, 1) * shortlist_k, dtype=torch.int32, device=postings.device)
    dists = torch.empty(max(n, 1) * shortlist_k, dtype=torch.float32, device=postings.device)
    passes = torch.empty(max(n, 1), dtype=torch.int32, device=postings.device)
    if rows is None:
        ctx.check(ctx.lib.gofann_rabitq_range_scan(
            ctx.handle, rv, rq, pred, routes, _lib.ptr(postings), resident_rows, segs.view(),
            shortlist_k, 1 if score_first else 0, _lib.ptr(ids), _lib.ptr(dists),
            _lib.ptr(passes)))
    else:
        ctx.check(ctx.lib.gofann_rabitq_range_scan_resident(
            ctx.handle, rv, rq, pred, routes, _lib.ptr(postings), resident_rows,
            _lib.ptr(rows.codes), _lib.ptr(rows.aux), segs.view(), shortlist_k,
            1 if score_first else 0, _lib.ptr(ids), _lib.ptr(dists), _lib.ptr(passes)))
    rows = n
    return (ids[: rows * shortlist_k].view(rows, shortlist_k),
            dists[: rows * shortlist_k].view(rows, shortlist_k), passes[:rows])
