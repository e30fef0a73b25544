"""ctypes binding of libgofann_hip.so (C ABI declared in include/gofann_hip.h).

The structures mirror the header field by field.  Device arrays are passed as
raw pointers taken from torch tensors on the GPU; torch is used only for
device memory and streams.  The library must exist (built by
go-fann_amd/build.py): there is no fallback implementation.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

_HERE = Path(__file__).resolve().parent
# GOFANN_HIP_LIB may name an alternative build of the same library.
LIB_PATH = Path(os.environ.get("GOFANN_HIP_LIB", str(_HERE.parent / "libgofann_hip.so")))

GOFANN_OK = 0
OK, ERR_INVALID, ERR_HIP, ERR_UNSUPPORTED, ERR_NOMEM = 0, -1, -2, -3, -4
EARLY_STOP_FIXED, EARLY_STOP_OFF, EARLY_STOP_ADAPTIVE = 0, 1, 2
ELEM_U8, ELEM_F32, ELEM_F16 = 0, 1, 2
EXACT_ORDER_SERIAL, EXACT_ORDER_WARP = 0, 1
PLACE_AUTO, PLACE_LDS, PLACE_GLOBAL, PLACE_SPILL = 0, 1, 2, 3

P = C.c_void_p
U32 = C.c_uint32


class GraphView(C.Structure):
    _fields_ = [("graph", P), ("row_to_sample", P), ("label_offset", P),
                ("rows", U32), ("degree", U32), ("groups", U32), ("samples", U32),
                ("neighbor_samples", P)]


class Clause(C.Structure):
    _fields_ = [("label_begin", U32), ("label_end", U32), ("range_begin", U32),
                ("range_end", U32)]


class RangeAtom(C.Structure):
    _fields_ = [("dimension", U32), ("mode", U32), ("lower", C.c_float),
                ("upper", C.c_float)]


class PredicateView(C.Structure):
    _fields_ = [("route_offsets", P), ("route_handles", P), ("clauses", P),
                ("ranges", P), ("route_enabled", P), ("route_compiled", P),
                ("base_ranges", P), ("csr_offsets", P), ("csr_labels", P),
                ("rows", U32), ("range_stride", U32), ("alpha", C.c_float),
                ("pending_base_stop", C.c_int), ("label_slab", P), ("slab_stride", U32),
                ("range_columns", U32)]


class Routes(C.Structure):
    _fields_ = [("route_query", P), ("route_group", P), ("route_start", P),
                ("row_filter_mask", P), ("query_filter_bits", P), ("range_modes", P),
                ("range_lower", P), ("range_upper", P), ("base_range_values", P),
                ("range_count", U32), ("count", U32), ("launch_order", P)]


class SearchParams(C.Structure):
    _fields_ = [("queue_limit", C.c_int), ("finish_limit", C.c_int),
                ("early_stop_mode", C.c_int), ("max_steps", C.c_int),
                ("stop_width", C.c_int), ("result_width", C.c_int),
                ("bit_filter_bonus", C.c_float), ("range_filter_bonus", C.c_float),
                ("predicate_bias", C.c_int), ("inline_exact_rerank", C.c_int),
                ("table_mode", C.c_int), ("hash_mode", C.c_int)]


class RouteStats(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("steps", "expanded", "passed", "scored",
                                          "pred_rows", "pred_labels", "admitted",
                                          "exhausted")]


STATS_FIELDS = [f[0] for f in RouteStats._fields_]


class PqView(C.Structure):
    _fields_ = [("codes", P), ("centroids", P), ("dim", U32), ("pq_dim", U32),
                ("samples", U32), ("exact_base", P), ("code_stride", U32)]


class RabitqView(C.Structure):
    _fields_ = [("codes", P), ("factors", P), ("anchor_ids", P), ("anchors", P),
                ("dim", U32), ("padded_dim", U32), ("num_anchors", U32),
                ("samples", U32), ("records", P), ("record_stride", U32)]


class RabitqQueries(C.Structure):
    _fields_ = [("rotated", P), ("q8", P), ("scale", P), ("k1", P),
                ("centroid_dists", P), ("count", U32)]


class ExactParams(C.Structure):
    _fields_ = [("queue_limit", C.c_int), ("finish_limit", C.c_int),
                ("early_stop_mode", C.c_int), ("max_steps", C.c_int), ("topk", C.c_int),
                ("hash_mode", C.c_int)]


class PostingSegments(C.Structure):
    _fields_ = [("route_ids", P), ("offsets", P), ("sizes", P), ("count", U32),
                ("query_indptr", P), ("positions", U32)]


class PostingShare(C.Structure):
    _fields_ = [("item_offsets", P), ("item_sizes", P), ("item_begin", P), ("item_slots", P),
                ("items", U32)]


U64 = C.c_uint64
CS = C.c_char_p


class BuildBuckets(C.Structure):
    _fields_ = [("bucket_offsets", P), ("buckets", U32), ("rows", U32), ("probe_offsets", P),
                ("probe_buckets", P)]


class BuildLinkInputs(C.Structure):
    _fields_ = [("rows", U32), ("knn", P), ("knn_width", U32), ("bucket_of", P), ("reps", P),
                ("near_buckets", P), ("near_width", U32), ("buckets", U32), ("order", P)]


class BuildLinkParams(C.Structure):
    _fields_ = [("degree", U32), ("local", U32), ("near_links", U32), ("rep_local", U32),
                ("rep_near", U32), ("entry_row", U32), ("seed", U64)]


class GraphFileHeader(C.Structure):
    _fields_ = [("magic", U32), ("version", U32), ("block_size", U32), ("header_size", U32),
                ("rows", U64), ("degree", U32), ("row_size_bytes", U32),
                ("rows_per_block", U64)]


class GraphMetadataHeader(C.Structure):
    _fields_ = [("version", U32), ("reserved", U32)] + [
        (n, U64) for n in ("label_count", "group_count", "original_label_count", "num_points",
                           "row_limit", "graph_rows", "total_rows", "graph_degree",
                           "specificity_threshold", "group_layout_checksum")]


class GraphSeedHeader(C.Structure):
    _fields_ = [("version", U32), ("reserved", U32)] + [
        (n, U64) for n in ("label_count", "num_points", "graph_rows", "graph_degree",
                           "specificity_threshold")]


class RabitqFileHeader(C.Structure):
    _fields_ = [("version", U32), ("dim", U32), ("num_anchors", U32), ("code_bytes", U32),
                ("num_points", U64)] + [
        (n, U32) for n in ("padded_dim", "bits_per_dim", "short_code_words",
                           "long_code_bytes", "layout_flags", "short_factor_count",
                           "ex_factor_count")]


# Every symbol include/gofann_hip.h declares, with its ctypes signature.
SIGNATURES = {
    "gofann_create": (C.c_int, [C.c_int, C.POINTER(P)]),
    "gofann_destroy": (None, [P]),
    "gofann_last_error": (C.c_char_p, [P]),
    "gofann_set_stream": (C.c_int, [P, P]),
    "gofann_synchronize": (C.c_int, [P]),
    "gofann_device_info": (C.c_int, [P, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "gofann_last_placement": (C.c_int, [P, C.POINTER(C.c_int), C.POINTER(C.c_int),
                                        C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "gofann_pq_search": (C.c_int, [P, C.POINTER(PqView), P, C.c_int, C.POINTER(GraphView),
                                   C.POINTER(PredicateView), C.POINTER(Routes),
                                   C.POINTER(SearchParams), P, P, P]),
    "gofann_rabitq_prepare_queries": (C.c_int, [P, C.POINTER(RabitqView), P, U32, P,
                                                C.POINTER(RabitqQueries)]),
    "gofann_rabitq_search": (C.c_int, [P, C.POINTER(RabitqView), C.POINTER(RabitqQueries),
                                       C.POINTER(GraphView), C.POINTER(PredicateView),
                                       C.POINTER(Routes), C.POINTER(SearchParams), P, P, P]),
    "gofann_pq_posting_scan": (C.c_int, [P, C.POINTER(PqView), P, C.c_int,
                                         C.POINTER(PredicateView), P, P, P, P, U32, C.c_int,
                                         P, P, P]),
    "gofann_rabitq_posting_scan": (C.c_int, [P, C.POINTER(RabitqView),
                                             C.POINTER(RabitqQueries),
                                             C.POINTER(PredicateView), P, P, P, P, U32,
                                             C.c_int, P, P, P]),
    "gofann_exact_search": (C.c_int, [P, P, C.c_int, U32, U32, P, C.POINTER(GraphView), P,
                                      C.POINTER(PredicateView), C.POINTER(Routes),
                                      C.POINTER(ExactParams), P, P, P]),
    "gofann_exact_search_noalloc": (C.c_int, [P, P, C.c_int, U32, U32, P, C.POINTER(GraphView),
                                              P, C.POINTER(PredicateView), C.POINTER(Routes),
                                              C.POINTER(ExactParams), P, P, P]),
    "gofann_posting_segment_plan": (C.c_int, [P, P, P, U32, U32, U32, P, P, P, P, P,
                                              C.POINTER(U32)]),
    "gofann_range_slices": (C.c_int, [P, P, P, U32, P, P, P, U32, P]),
    "gofann_rabitq_range_scan": (C.c_int, [P, C.POINTER(RabitqView), C.POINTER(RabitqQueries),
                                           C.POINTER(PredicateView), C.POINTER(Routes), P,
                                           C.c_uint64, C.POINTER(PostingSegments), C.c_int,
                                           C.c_int, P, P, P]),
    "gofann_rabitq_posting_rows": (C.c_int, [P, C.POINTER(RabitqView), P, C.c_uint64, P, P]),
    "gofann_rabitq_range_scan_resident": (C.c_int, [P, C.POINTER(RabitqView),
                                                    C.POINTER(RabitqQueries),
                                                    C.POINTER(PredicateView), C.POINTER(Routes),
                                                    P, C.c_uint64, P, P,
                                                    C.POINTER(PostingSegments), C.c_int,
                                                    C.c_int, P, P, P]),
    "gofann_posting_predicate_rows": (C.c_int, [P, C.POINTER(PredicateView), P, C.c_uint64,
                                                P, P]),
    "gofann_rabitq_posting_scan_segments": (C.c_int, [P, C.POINTER(RabitqView),
                                                      C.POINTER(RabitqQueries),
                                                      C.POINTER(PredicateView), P, P, C.c_uint64,
                                                      C.POINTER(PostingSegments), C.c_int, P, P,
                                                      P, P, P, P, P]),
    "gofann_rabitq_posting_scan_shared": (C.c_int, [P, C.POINTER(RabitqView),
                                                    C.POINTER(RabitqQueries),
                                                    C.POINTER(PredicateView), P, P, C.c_uint64,
                                                    C.POINTER(PostingSegments),
                                                    C.POINTER(PostingShare), C.c_int, P, P,
                                                    P, P, P, P, P]),
    "gofann_exact_rerank": (C.c_int, [P, P, C.c_int, U32, U32, P, P, P, U32, U32, U32, P, P]),
    "gofann_exact_posting_scan": (C.c_int, [P, P, C.c_int, U32, U32, P, C.POINTER(PredicateView),
                                            P, P, P, P, U32, C.c_int, C.c_int, P, P, P]),
    "gofann_merge_routes": (C.c_int, [P, P, P, P, P, U32, U32, U32, P, P]),
    "gofann_predicate_masks": (C.c_int, [P, C.POINTER(PredicateView), P, P, U32, P]),
    "gofann_pq_score": (C.c_int, [P, C.POINTER(PqView), P, C.c_int, P, P, U32, P]),
    "gofann_rabitq_score": (C.c_int, [P, C.POINTER(RabitqView), C.POINTER(RabitqQueries),
                                      P, P, U32, P, P]),
    "gofann_host_rerank_create": (C.c_int, [P, C.c_int, U32, U32, P, U32, C.POINTER(P)]),
    "gofann_host_rerank_destroy": (None, [P]),
    "gofann_host_rerank_last_error": (C.c_char_p, [P]),
    "gofann_host_rerank_fp16_kernel": (C.c_char_p, [P]),
    "gofann_host_rerank_routes": (C.c_int, [P, P, U32, P, U32, U32, P, P]),
    "gofann_pq_search_host_rerank": (C.c_int, [P, P, C.POINTER(PqView), P, C.c_int,
                                               C.POINTER(GraphView), C.POINTER(PredicateView),
                                               C.POINTER(Routes), C.POINTER(SearchParams), P,
                                               U32, U32, P, P, P]),
    "gofann_host_merge_routes": (C.c_int, [P, P, P, P, U32, U32, U32, P, P]),
    "gofann_io_last_error": (C.c_char_p, []),
    "gofann_graph_file_has_magic": (C.c_int, [CS]),
    "gofann_graph_file_read_header": (C.c_int, [CS, C.POINTER(GraphFileHeader)]),
    "gofann_graph_file_read_rows": (C.c_int, [CS, U64, U64, P]),
    "gofann_graph_file_write": (C.c_int, [CS, P, U64, U32]),
    "gofann_graph_file_convert_legacy": (C.c_int, [CS, CS]),
    "gofann_graph_metadata_read_header": (C.c_int, [CS, C.POINTER(GraphMetadataHeader)]),
    "gofann_graph_metadata_read": (C.c_int, [CS, P, P, P, P, P, P, P]),
    "gofann_graph_metadata_write": (C.c_int, [CS, C.POINTER(GraphMetadataHeader), P, P, P, P,
                                              P, P, P]),
    "gofann_group_layout_checksum": (U64, [P, P, U32, U32]),
    "gofann_graph_seeds_read_header": (C.c_int, [CS, C.POINTER(GraphSeedHeader)]),
    "gofann_graph_seeds_read": (C.c_int, [CS, P, P]),
    "gofann_graph_seeds_write": (C.c_int, [CS, C.POINTER(GraphSeedHeader), P]),
    "gofann_spmat_read_header": (C.c_int, [CS, C.POINTER(U64), C.POINTER(U64), C.POINTER(U64)]),
    "gofann_spmat_read": (C.c_int, [CS, U32, P, P, U64, C.POINTER(U64)]),
    "gofann_query_range_read_header": (C.c_int, [CS, U32, C.POINTER(U32), C.POINTER(U32)]),
    "gofann_query_range_read": (C.c_int, [CS, U32, P, P, P]),
    "gofann_rabitq_file_read_header": (C.c_int, [CS, C.POINTER(RabitqFileHeader)]),
    "gofann_rabitq_file_read": (C.c_int, [CS, P, P, P, P, P, P, P, P]),
    "gofann_rabitq_file_write": (C.c_int, [CS, C.POINTER(RabitqFileHeader), P, P, P, P, P, P, P,
                                           P]),
    "gofann_pq_pivots_read_header": (C.c_int, [CS, C.POINTER(U32), C.POINTER(U32)]),
    "gofann_pq_pivots_read": (C.c_int, [CS, U32, P]),
    "gofann_pq_codes_read_header": (C.c_int, [CS, C.POINTER(U64), C.POINTER(U32)]),
    "gofann_pq_codes_read": (C.c_int, [CS, U64, U64, P, U32]),
    "gofann_pq_files_write": (C.c_int, [CS, CS, P, U32, U32, P, U64]),
    "gofann_build_assign": (C.c_int, [P, P, C.c_int, U32, U64, P, U32, P, P]),
    "gofann_build_kmeanspp": (C.c_int, [P, P, C.c_int, U32, U64, U32, U64, P]),
    "gofann_build_kmeans": (C.c_int, [P, P, C.c_int, U32, U64, U32, U32, P]),
    "gofann_build_knn": (C.c_int, [P, P, C.c_int, U32, C.POINTER(BuildBuckets), U32, P, P]),
    "gofann_build_pq_train": (C.c_int, [P, P, C.c_int, U32, U64, U32, U32, P]),
    "gofann_build_pq_encode": (C.c_int, [P, P, C.c_int, U32, U64, U32, P, P, U32]),
    "gofann_build_rotate": (C.c_int, [P, P, C.c_int, U32, U32, P, U32, P]),
    "gofann_build_rabitq_encode": (C.c_int, [P, P, U32, U32, P, U32, P, P, P]),
    "gofann_build_medoid": (C.c_int, [P, P, C.c_int, U32, U64, C.POINTER(U32)]),
    "gofann_build_bucket_reps": (C.c_int, [P, P, C.c_int, U32, P, U32, P, P]),
    "gofann_build_links": (C.c_int, [P, C.POINTER(BuildLinkInputs), C.POINTER(BuildLinkParams),
                                     P]),
    "gofann_build_cagra_optimize": (C.c_int, [P, P, U32, U32, U32, P, P]),
    "gofann_build_reach": (C.c_int, [P, P, U32, U32, U32, P, C.POINTER(U32)]),
}

_lib = None


def load() -> C.CDLL:
    """Load the HIP library; raises if it was not built (no fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is missing: run go-fann_amd/build.py "
                           "(the GPU path has no CPU fallback)")
    lib = C.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | os.RTLD_GLOBAL)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def ptr(t) -> int | None:
    """Device (or host) address of a torch tensor, None for None."""
    if t is None:
        return None
    return t.data_ptr()


class GofannError(RuntimeError):
    pass


class Context:
    """Owns one gofann_ctx bound to torch's current stream on `device`."""

    def __init__(self, device: int = 0):
        import torch
        self.lib = load()
        self.device = device
        h = P()
        rc = self.lib.gofann_create(device, C.byref(h))
        if rc != GOFANN_OK:
            raise GofannError(f"gofann_create failed ({rc})")
        self.handle = h
        self.bind_stream(torch.cuda.current_stream(device))

    def bind_stream(self, stream) -> None:
        self.check(self.lib.gofann_set_stream(self.handle, P(stream.cuda_stream)))

    def check(self, rc: int) -> None:
        if rc != GOFANN_OK:
            msg = self.lib.gofann_last_error(self.handle)
            raise GofannError(f"gofann call failed ({rc}): {msg.decode() if msg else ''}")

    def last_error(self) -> str:
        msg = self.lib.gofann_last_error(self.handle)
        return msg.decode() if msg else ""

    def synchronize(self) -> None:
        self.check(self.lib.gofann_synchronize(self.handle))

    def device_info(self) -> tuple[int, int]:
        cu, lds = C.c_int(), C.c_int()
        self.check(self.lib.gofann_device_info(self.handle, C.byref(cu), C.byref(lds)))
        return cu.value, lds.value

    def last_placement(self) -> dict:
        """Placement chosen by the last traversal launch."""
        v = [C.c_int() for _ in range(4)]
        self.check(self.lib.gofann_last_placement(self.handle, *[C.byref(x) for x in v]))
        return dict(table_in_lds=v[0].value, hash_in_lds=v[1].value, lds_bytes=v[2].value,
                    resident_per_cu=v[3].value)

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.lib.gofann_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
