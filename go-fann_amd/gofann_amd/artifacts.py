"""Reference artifacts on disk, through the library's host readers/writers
(gofann_graph_file_*, gofann_graph_metadata_*, gofann_graph_seeds_*,
gofann_spmat_*, gofann_query_range_*, gofann_rabitq_file_*, gofann_pq_*).

An index the reference built -- graph.bin (FDRG, src/index/
graph_file_format.h:16-25), its metadata and seed sidecars (src/data/
dataloader.h:609-644), the .spmat label matrix (dataloader.cpp:6663-6760),
query_range.bin (:6780-6880), rabitq.b1.bin v2 (backend_rabitq.cu:2748-2845)
or the DiskANN-style PQ pivots/codes (tools/quantization/pq_builder.cu:
110-122) -- loads into the arrays this package searches, and a LabelIndex
built here saves to files the reference loads.  Arrays come back as numpy
host arrays; callers move them to the device.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

from . import _lib
from .index import LabelIndex, postings_from_csr

U32MAX = 0xFFFFFFFF


class ArtifactError(RuntimeError):
    """A reader or writer refused a file (the reference's loader would throw)."""


def _call(name: str, *args):
    lib = _lib.load()
    rc = getattr(lib, name)(*args)
    if rc < 0:
        raise ArtifactError(f"{name}: {lib.gofann_io_last_error().decode()} (status {rc})")
    return rc


def _b(path) -> bytes | None:
    return None if path is None else os.fsencode(path)


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


# ------------------------------------------------------------------- graph
def graph_file_header(path) -> dict:
    h = _lib.GraphFileHeader()
    _call("gofann_graph_file_read_header", _b(path), C.byref(h))
    return {f: getattr(h, f) for f, _ in h._fields_}


def is_graph_file(path) -> bool:
    return _call("gofann_graph_file_has_magic", _b(path)) == 1


def read_graph(path, row_begin: int = 0, row_count: int | None = None,
               out: np.ndarray | None = None) -> np.ndarray:
    """Rows [row_begin, row_begin + row_count) as [rows][degree] u32."""
    h = graph_file_header(path)
    if row_count is None:
        row_count = h["rows"] - row_begin
    if out is None:
        out = np.empty((row_count, h["degree"]), dtype=np.uint32)
    elif out.dtype != np.uint32 or out.size < row_count * h["degree"] or not out.flags.c_contiguous:
        raise ValueError("out must be C-contiguous u32 with room for the rows")
    _call("gofann_graph_file_read_rows", _b(path), row_begin, row_count, _p(out))
    return out


def write_graph(path, graph: np.ndarray) -> None:
    g = np.ascontiguousarray(graph, dtype=np.uint32)
    if g.ndim != 2:
        raise ValueError("graph must be [rows][degree]")
    _call("gofann_graph_file_write", _b(path), _p(g), g.shape[0], g.shape[1])


def convert_legacy_graph(legacy_path, path) -> None:
    _call("gofann_graph_file_convert_legacy", _b(legacy_path), _b(path))


# ---------------------------------------------------------------- sidecars
@dataclass
class GraphMetadata:
    header: dict
    cat_freq: np.ndarray
    group_posting_size: np.ndarray
    label_size: np.ndarray
    label_offset: np.ndarray
    row_to_sample: np.ndarray
    row_filter_mask: np.ndarray
    label_filter_bit: np.ndarray


def read_metadata(path) -> GraphMetadata:
    h = _lib.GraphMetadataHeader()
    _call("gofann_graph_metadata_read_header", _b(path), C.byref(h))
    L, R, O = h.label_count, h.total_rows, h.original_label_count
    a = [np.empty(L, np.uint32) for _ in range(4)]
    rts = np.empty(R, np.uint32)
    rfm = np.empty(R, np.uint64)
    lfb = np.empty(O, np.uint64)
    _call("gofann_graph_metadata_read", _b(path), *map(_p, a), _p(rts), _p(rfm), _p(lfb))
    return GraphMetadata({f: getattr(h, f) for f, _ in h._fields_}, *a, rts, rfm, lfb)


def group_layout_checksum(label_count: int, group_offsets=None, group_labels=None) -> int:
    """group_layout_checksum (dataloader.cpp:320-332); no groups given = one
    label per group."""
    groups = label_count if group_offsets is None else len(group_offsets) - 1
    go = None if group_offsets is None else np.ascontiguousarray(group_offsets, np.uint32)
    gl = None if group_labels is None else np.ascontiguousarray(group_labels, np.uint32)
    return int(_lib.load().gofann_group_layout_checksum(_p(go), _p(gl), groups, label_count))


def read_seeds(path, label_size: np.ndarray | None = None) -> tuple[dict, np.ndarray]:
    h = _lib.GraphSeedHeader()
    _call("gofann_graph_seeds_read_header", _b(path), C.byref(h))
    seeds = np.empty(h.label_count, np.uint32)
    ls = None if label_size is None else np.ascontiguousarray(label_size, np.uint32)
    _call("gofann_graph_seeds_read", _b(path), _p(ls), _p(seeds))
    return {f: getattr(h, f) for f, _ in h._fields_}, seeds


# ------------------------------------------------------------------ labels
def read_spmat(path, row_limit: int = 0) -> tuple[np.ndarray, np.ndarray, int]:
    """(indptr u64 [rows+1], indices u32, cols): each row sorted, unique."""
    rows, cols, nnz = C.c_uint64(), C.c_uint64(), C.c_uint64()
    _call("gofann_spmat_read_header", _b(path), C.byref(rows), C.byref(cols), C.byref(nnz))
    eff = rows.value if row_limit <= 0 or row_limit >= rows.value else row_limit
    indptr = np.empty(eff + 1, np.uint64)
    indices = np.empty(max(nnz.value, 1), np.uint32)
    out_nnz = C.c_uint64()
    _call("gofann_spmat_read", _b(path), row_limit, _p(indptr), _p(indices), nnz.value,
          C.byref(out_nnz))
    return indptr, indices[: out_nnz.value].copy(), int(cols.value)


def write_spmat(path, indptr: np.ndarray, indices: np.ndarray, cols: int) -> None:
    """u64 rows, cols, nnz, indptr, u32 indices -- the layout load_spmat_labels reads."""
    indptr = np.asarray(indptr, np.uint64)
    indices = np.asarray(indices, np.uint32)
    with open(path, "wb") as f:
        f.write(np.array([len(indptr) - 1, cols, len(indices)], np.uint64).tobytes())
        f.write(indptr.tobytes())
        f.write(indices.tobytes())


def read_query_ranges(path, queries: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """(modes u8, lower f32, upper f32), each [queries][range_count]."""
    rc, rec = C.c_uint32(), C.c_uint32()
    _call("gofann_query_range_read_header", _b(path), queries, C.byref(rc), C.byref(rec))
    shape = (queries, rc.value)
    modes = np.empty(shape, np.uint8)
    lower = np.empty(shape, np.float32)
    upper = np.empty(shape, np.float32)
    _call("gofann_query_range_read", _b(path), queries, _p(modes), _p(lower), _p(upper))
    return modes, lower, upper


# ----------------------------------------------------------- dense vectors
_VECS = {".bvecs": np.uint8, ".fvecs": np.float32, ".hvecs": np.float16}


def read_vectors(path, row_limit: int = 0) -> np.ndarray:
    """A dense vector file as a read-only [rows][dim] memory map
    (inspect_dense_vector_file and its loaders, dataloader.cpp:1321-1480):
    .u8bin/.ibin u32 rows, u32 cols, u8 rows; .fbin the same with f32 rows
    and an exact file size; .bvecs/.fvecs/.hvecs one u32 dim before every row
    (u8 / f32 / f16).  row_limit > 0 keeps the first rows."""
    path = os.fspath(path)
    ext = os.path.splitext(path)[1].lower()
    size = os.path.getsize(path)
    if ext in (".u8bin", ".ibin", ".fbin"):
        rows, cols = (int(v) for v in np.fromfile(path, np.uint32, 2))
        dt = np.float32 if ext == ".fbin" else np.uint8
        if cols == 0 or (ext == ".fbin" and rows == 0):
            raise ArtifactError(f"invalid vector header in {path}")
        if ext == ".fbin" and size != 8 + rows * cols * 4:
            raise ArtifactError(f"fbin file size does not match header in {path}")
        if size < 8 + rows * cols * np.dtype(dt).itemsize:
            raise ArtifactError(f"failed to read payload from {path}")
        keep = rows if row_limit <= 0 or row_limit >= rows else row_limit
        return np.memmap(path, dt, "r", offset=8, shape=(keep, cols))
    if ext in _VECS:
        dt = np.dtype(_VECS[ext])
        dim = int(np.fromfile(path, np.uint32, 1)[0]) if size >= 4 else 0
        if dim == 0:
            raise ArtifactError(f"invalid {ext} dimension in {path}")
        rec = 4 + dim * dt.itemsize
        if size % rec:
            raise ArtifactError(f"{ext} file size is not row-aligned for {path}")
        rows = size // rec
        keep = rows if row_limit <= 0 or row_limit >= rows else row_limit
        raw = np.memmap(path, np.uint8, "r", shape=(rows, rec))[:keep]
        dims = np.ascontiguousarray(raw[:, :4]).view(np.uint32).ravel()
        bad = np.flatnonzero(dims != dim)
        if bad.size:
            raise ArtifactError(f"inconsistent {ext} dimension at row {int(bad[0])} in {path}")
        return np.ascontiguousarray(raw[:, 4:]).view(dt)
    raise ArtifactError(f"unsupported dense vector extension for {path} "
                        "(supported: .bvecs, .ibin, .u8bin, .fbin, .fvecs, .hvecs)")


def write_vectors(path, x: np.ndarray) -> None:
    """The inverse of read_vectors for the extension of `path`."""
    path = os.fspath(path)
    ext = os.path.splitext(path)[1].lower()
    x = np.ascontiguousarray(x)
    n, d = x.shape
    with open(path, "wb") as f:
        if ext in (".u8bin", ".ibin", ".fbin"):
            dt = np.float32 if ext == ".fbin" else np.uint8
            f.write(np.array([n, d], np.uint32).tobytes())
            f.write(x.astype(dt).tobytes())
        elif ext in _VECS:
            rec = np.empty((n, 4 + d * np.dtype(_VECS[ext]).itemsize), np.uint8)
            rec[:, :4] = np.frombuffer(np.uint32(d).tobytes(), np.uint8)
            rec[:, 4:] = x.astype(_VECS[ext]).view(np.uint8).reshape(n, -1)
            f.write(rec.tobytes())
        else:
            raise ArtifactError(f"unsupported dense vector extension for {path}")


# ------------------------------------------------------------------ RaBitQ
RABITQ_ARRAYS = ("anchors", "rotation", "query_scaling_factors", "anchor_ids", "codes",
                 "long_codes", "factors", "ex_factors")


def rabitq_file_header(path) -> dict:
    h = _lib.RabitqFileHeader()
    _call("gofann_rabitq_file_read_header", _b(path), C.byref(h))
    return {f: getattr(h, f) for f, _ in h._fields_}


def read_rabitq(path) -> dict:
    """Header fields plus the eight arrays, shaped: anchors [A][P], rotation
    [P][P] (its first dim rows are the [dim][P] rotation the query
    preparation takes), codes [N][code_bytes], factors [N][3], ...."""
    h = rabitq_file_header(path)
    n, P = h["num_points"], h["padded_dim"]
    arr = {
        "anchors": np.empty((h["num_anchors"], P), np.float32),
        "rotation": np.empty((P, P), np.float32),
        "query_scaling_factors": np.empty(2, np.float32),
        "anchor_ids": np.empty(n, np.uint32),
        "codes": np.empty((n, h["code_bytes"]), np.uint8),
        "long_codes": np.empty((n, h["long_code_bytes"]), np.uint8),
        "factors": np.empty((n, h["short_factor_count"]), np.float32),
        "ex_factors": np.empty((n, h["ex_factor_count"]), np.float32),
    }
    _call("gofann_rabitq_file_read", _b(path), *(_p(arr[k]) for k in RABITQ_ARRAYS))
    return {**h, **arr}


def write_rabitq(path, dim: int, anchors: np.ndarray, anchor_ids: np.ndarray,
                 codes: np.ndarray, factors: np.ndarray, rotation: np.ndarray | None = None,
                 query_scaling_factors: np.ndarray | None = None,
                 ex_factors: np.ndarray | None = None) -> None:
    """A one-bit artifact (bits_per_dim 1, no long codes).  rotation may be
    [dim][P] (rows dim..P written as zeros: they multiply zero padding) or
    [P][P]."""
    anchors = np.ascontiguousarray(anchors, np.float32)
    A, P = anchors.shape
    codes = np.ascontiguousarray(codes, np.uint8)
    n = codes.shape[0]
    h = _lib.RabitqFileHeader(version=2, dim=dim, num_anchors=A, code_bytes=(P + 31) // 32 * 4,
                              num_points=n, padded_dim=P, bits_per_dim=1,
                              short_code_words=(P + 31) // 32, long_code_bytes=0,
                              layout_flags=7, short_factor_count=3, ex_factor_count=2)
    rot = None
    if rotation is not None:
        rot = np.zeros((P, P), np.float32)
        rot[: rotation.shape[0]] = rotation
    arrays = [anchors, rot,
              None if query_scaling_factors is None else np.ascontiguousarray(query_scaling_factors, np.float32),
              np.ascontiguousarray(anchor_ids, np.uint32), codes, None,
              np.ascontiguousarray(factors, np.float32),
              None if ex_factors is None else np.ascontiguousarray(ex_factors, np.float32)]
    _call("gofann_rabitq_file_write", _b(path), C.byref(h), *map(_p, arrays))


# ---------------------------------------------------------------------- PQ
def read_pq(pivots_path, codes_path, pq_dim: int = 0, row_begin: int = 0,
            row_count: int | None = None, code_stride: int = 0):
    """(centroids f32 [256][dim], codes u8 [rows][stride or pq_dim])."""
    dim, m = C.c_uint32(), C.c_uint32()
    _call("gofann_pq_pivots_read_header", _b(pivots_path), C.byref(dim), C.byref(m))
    cent = np.empty((256, dim.value), np.float32)
    _call("gofann_pq_pivots_read", _b(pivots_path), pq_dim, _p(cent))
    rows, cm = C.c_uint64(), C.c_uint32()
    _call("gofann_pq_codes_read_header", _b(codes_path), C.byref(rows), C.byref(cm))
    if row_count is None:
        row_count = rows.value - row_begin
    codes = np.zeros((row_count, code_stride or cm.value), np.uint8)
    _call("gofann_pq_codes_read", _b(codes_path), row_begin, row_count, _p(codes), code_stride)
    return cent, codes


def write_pq(pivots_path, codes_path, centroids: np.ndarray, codes: np.ndarray) -> None:
    cent = np.ascontiguousarray(centroids, np.float32)
    codes = np.ascontiguousarray(codes, np.uint8)
    _call("gofann_pq_files_write", _b(pivots_path), _b(codes_path), _p(cent), cent.shape[1],
          codes.shape[1], _p(codes), codes.shape[0])


# ------------------------------------------------------------ label index
def save_label_index(index: LabelIndex, graph_path, metadata_path, seeds_path,
                     spmat_path=None, num_points: int | None = None) -> None:
    """Writes graph.bin, the metadata and seed sidecars (one label per
    group) and, optionally, the .spmat label matrix of a LabelIndex."""
    L = index.num_labels
    n = int(num_points if num_points is not None else len(index.csr_offsets) - 1)
    write_graph(graph_path, index.graph)
    h = _lib.GraphMetadataHeader(
        version=1, label_count=L, group_count=L, original_label_count=L, num_points=n,
        row_limit=n, graph_rows=index.rows, total_rows=index.rows, graph_degree=index.degree,
        specificity_threshold=index.threshold, group_layout_checksum=group_layout_checksum(L))
    cf = np.ascontiguousarray(index.cat_freq, np.uint32)
    lfb = np.ones(L, np.uint64)  # label bit 0 of its own group
    _call("gofann_graph_metadata_write", _b(metadata_path), C.byref(h), _p(cf), _p(cf),
          _p(np.ascontiguousarray(index.label_size, np.uint32)),
          _p(np.ascontiguousarray(index.label_offset, np.uint32)),
          _p(np.ascontiguousarray(index.row_to_sample, np.uint32)), None, _p(lfb))
    sh = _lib.GraphSeedHeader(version=2, label_count=L, num_points=n, graph_rows=index.rows,
                              graph_degree=index.degree, specificity_threshold=index.threshold)
    _call("gofann_graph_seeds_write", _b(seeds_path), C.byref(sh),
          _p(np.ascontiguousarray(index.seed_local, np.uint32)))
    if spmat_path is not None:
        write_spmat(spmat_path, index.csr_offsets.astype(np.uint64), index.csr_labels, L)


def load_label_index(graph_path, metadata_path, seeds_path, spmat_path) -> LabelIndex:
    """A LabelIndex from the reference's graph artifacts (one label per
    group: every row_filter_mask all-ones)."""
    md = read_metadata(metadata_path)
    hdr = md.header
    if hdr["label_count"] != hdr["original_label_count"]:
        raise ArtifactError("grouped label layouts (several labels per group) are not supported")
    g = read_graph(graph_path)
    if g.shape[0] != hdr["total_rows"]:
        raise ArtifactError("graph rows do not match the metadata sidecar's total_rows")
    _, seeds = read_seeds(seeds_path, md.label_size)
    indptr, indices, cols = read_spmat(spmat_path, int(hdr["row_limit"]))
    if cols != hdr["original_label_count"] or len(indptr) - 1 != hdr["num_points"]:
        raise ArtifactError("spmat shape does not match the metadata sidecar")
    L = int(hdr["label_count"])
    csr_offsets = indptr.astype(np.uint32)
    _, posting_offset, posting_ids = postings_from_csr(csr_offsets, indices, L)
    return LabelIndex(num_labels=L, threshold=int(hdr["specificity_threshold"]),
                      cat_freq=md.cat_freq, label_offset=md.label_offset,
                      label_size=md.label_size, row_to_sample=md.row_to_sample, graph=g,
                      seed_local=seeds, posting_offset=posting_offset, posting_ids=posting_ids,
                      csr_offsets=csr_offsets, csr_labels=indices, degree=int(g.shape[1]))


# ------------------------------------------------------- streamed to HBM
def graph_to_device(path, device, chunk_rows: int = 1 << 20):
    """The whole graph file as a [rows][degree] int32 device tensor (u32 bit
    patterns), read in windows of chunk_rows rows into two pinned staging
    buffers that alternate, so a file larger than host memory never needs a
    host copy and the disk read of one window overlaps the copy of the last."""
    import torch
    h = graph_file_header(path)
    rows, degree = h["rows"], h["degree"]
    out = torch.empty((rows, degree), dtype=torch.int32, device=device)
    if rows == 0:
        return out
    chunk = max(1, min(chunk_rows, rows))
    stage = [torch.empty((chunk, degree), dtype=torch.int32, pin_memory=True) for _ in range(2)]
    done = [None, None]
    for i, r in enumerate(range(0, rows, chunk)):
        c = min(chunk, rows - r)
        s = stage[i % 2]
        if done[i % 2] is not None:
            done[i % 2].synchronize()       # the copy out of this buffer has finished
        view = s.numpy().view(np.uint32)
        _call("gofann_graph_file_read_rows", _b(path), r, c, _p(view))
        out[r:r + c].copy_(s[:c], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        done[i % 2] = ev
    torch.cuda.synchronize(device)
    return out


def pq_codes_to_device(path, device, code_stride: int = 0, chunk_rows: int = 1 << 22):
    """DiskANN code file as a [rows][stride or pq_dim] uint8 device tensor,
    streamed as graph_to_device."""
    import torch
    rows, m = C.c_uint64(), C.c_uint32()
    _call("gofann_pq_codes_read_header", _b(path), C.byref(rows), C.byref(m))
    n, width = rows.value, code_stride or m.value
    out = torch.zeros((n, width), dtype=torch.uint8, device=device)
    if n == 0:
        return out
    chunk = max(1, min(chunk_rows, n))
    stage = [torch.zeros((chunk, width), dtype=torch.uint8, pin_memory=True) for _ in range(2)]
    done = [None, None]
    for i, r in enumerate(range(0, n, chunk)):
        c = min(chunk, n - r)
        s = stage[i % 2]
        if done[i % 2] is not None:
            done[i % 2].synchronize()
        _call("gofann_pq_codes_read", _b(path), r, c, _p(s.numpy()), code_stride)
        out[r:r + c].copy_(s[:c], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        done[i % 2] = ev
    torch.cuda.synchronize(device)
    return out
