"""Writes the golden fixtures under tests/golden/ (JSON data only).

Each fixture transcribes the inputs and the asserted expectations of one of
GO-FANN's own tests (cited per fixture).  Constructions the reference test
builds with a loop are re-expressed here as the resulting data.  Nothing is
imported or executed from the reference: its test files were read as text.

Run: python tests/golden/make_fixtures.py
"""
from __future__ import annotations

import json
from pathlib import Path

HERE = Path(__file__).resolve().parent
U32MAX = 0xFFFFFFFF
FLT_MAX = 3.4028234663852886e38
USED = 0x80000000


def predicate_fixtures():
    out = {}
    # tests/native/gpu_predicate_cuda_test.cu:47-93 (residual_and_stop_fixture), CSR storage.
    out["residual_dnf"] = dict(
        source="tests/native/gpu_predicate_cuda_test.cu:47-79",
        csr_offsets=[0, 1, 2, 4], csr_labels=[0, 1, 0, 1], rows=3,
        route_offsets=[0, 1, 3, 4, 4, 4], handles=[0, 1],
        clauses=[[0, 0, 0, 0], [0, 1, 0, 1], [1, 2, 0, 0], [0, 0, 1, 2]],
        ranges=[[0, 1, 10.0, 0.0], [1, 3, 2.0, 4.0]],
        base_ranges=[[10.0, 2.0], [11.0, 4.0], [11.0, 3.0]],
        route_enabled=[1, 1, 1, 1, 0],
        # expected[route][sample] for samples 0..2 (entailed / DNF strict
        # boundary / half-open range / empty disjunction)
        expected=[[1, 1, 1], [0, 1, 1], [1, 0, 1], [0, 0, 0]],
        enabled=[1, 1, 1, 1, 0],
        out_of_range=[[0, 3, 0]],  # matches(route 0, sample 3) is false
    )
    out["pending_base"] = dict(
        source="tests/native/gpu_predicate_cuda_test.cu:80-93",
        pool=[[0.0, 0, 0.0], [50.0, USED | 1, 1.0], [100.0, 2, -8.0], [0.0, USED | 3, -100.0],
              [2.0, 4, 2.0]],
        current=[70.0, USED | 5, -5.0], next=[80.0, USED | 6, -2.0],
        cases=[
            dict(mark_used=[], current_valid=1, next_valid=1, expected=-8.0),
            dict(mark_used=[2], current_valid=1, next_valid=1, expected=-5.0),
            dict(mark_used=[2], current_valid=0, next_valid=1, expected=-2.0),
            dict(mark_used=[2], current_valid=0, next_valid=0, expected=2.0),
        ],
        # compact pairs carry no base: base == first
        compact_pool=[[0.0, 0, 0.0], [3.0, 7, 3.0], [-20.0, USED | 8, -20.0]],
        compact_reserved=[1.0, USED | 9, 1.0], compact_expected=1.0,
    )
    # gpu_predicate_cuda_test.cu:94-101 (csr_original_id_fixture)
    out["csr_original_ids"] = dict(
        source="tests/native/gpu_predicate_cuda_test.cu:94-101",
        csr_offsets=[0, 3, 3, 4], csr_labels=[0, 65536, 7330000, 65535], rows=3,
        probes=[[65536, 0, 1], [7330000, 0, 1], [65535, 0, 0], [0, 1, 0], [65535, 2, 1],
                [0, 3, 0], [U32MAX, 0, 0]],
        enabled_route0=1,
    )
    # gpu_predicate_cuda_test.cu:10-16, 102-118 (membership_fixture): label 0
    # = samples {0, 65535, 65536, 65537}, label 1 = {65537} over 65538 rows
    # (Roaring chunks 0/1 re-expressed as the equivalent sample-major CSR).
    rows = 65538
    labels_of = {0: [0], 65535: [0], 65536: [0], 65537: [0, 1]}
    off = [0]
    lab = []
    for s in range(rows):
        lab.extend(labels_of.get(s, []))
        off.append(len(lab))
    out["membership"] = dict(
        source="tests/native/gpu_predicate_cuda_test.cu:10-16, 102-118",
        csr_offsets=off, csr_labels=lab, rows=rows,
        route_offsets=[0, 1, 3], handles=[0, 0, 1],
        route0_true=[0, 65535, 65536, 65537], route1_true=[65537],
    )
    # gpu_predicate_cuda_test.cu:17-45 (navigation_fixture, failed bridge)
    out["failed_bridge"] = dict(
        source="tests/native/gpu_predicate_cuda_test.cu:29-45",
        samples=[2, 65536, 65537], route=1, expected_visited=7, expected_passed=4,
        penalty=10.0,
    )
    out["whole_entry_heap"] = dict(
        source="tests/native/gpu_predicate_cuda_test.cu:19-28",
        count=20, penalty=5.0, pop_at=10,
    )
    return out


def csr_lookup_cases():
    """tests/native/gpu_predicate_csr_lookup_cases.h:12-37."""
    offsets = [0]
    labels = []
    probes = []

    def expected(row, key):
        if row >= len(offsets) - 1:
            return 0
        return 1 if key in set(labels[offsets[row]:offsets[row + 1]]) else 0

    def add(row, key):
        probes.append([row, key, expected(row, key)])

    for length in (0, 1, 2, 7, 8, 9, 15, 16, 17, 31, 32, 33, 63, 64, 65, 1025, 65537):
        row = len(offsets) - 1
        first = 0 if row % 3 == 0 else (65536 if row % 3 == 1 else
                                         U32MAX - ((length - 1) * 7 if length else 0))
        for i in range(length):
            labels.append(first + 7 * i)
        offsets.append(len(labels))
        for key in (0, 1, 65535, 65536, 65537, U32MAX - 1, U32MAX):
            add(row, key)
        samples = min(length, 65)
        for i in range(samples):
            position = 0 if samples == 1 else (i * (length - 1)) // (samples - 1)
            key = labels[offsets[row] + position]
            add(row, key)
            if key:
                add(row, key - 1)
            if key < U32MAX:
                add(row, key + 1)
    add(len(offsets) - 1, 65536)
    add(U32MAX, U32MAX)
    while len(probes) % 32 != 13:
        add(0, 7)
    return dict(source="tests/native/gpu_predicate_csr_lookup_cases.h:12-37",
                csr_offsets=offsets, csr_labels=labels, rows=len(offsets) - 1, probes=probes)


def parallel_fixture():
    """tests/native/gpu_predicate_parallel_test.cu:109-146 data; expectations
    are the scalar matches() of the same test (recorded by the checker)."""
    rows = 67
    off = [0]
    lab = []
    for s in range(rows):
        if s % 2 == 0:
            lab.append(0)
        if s % 3 == 0:
            lab.append(1)
        if s % 5 == 0:
            lab.append(65536)
        off.append(len(lab))
    values = [[float(s % 9), float(s % 7)] for s in range(rows)]
    mapping = [U32MAX] * (3 + 97)
    for i in range(97):
        mapping[3 + i] = U32MAX if i % 13 == 0 else (i * 19) % (rows + 1)
    return dict(
        source="tests/native/gpu_predicate_parallel_test.cu:109-146",
        csr_offsets=off, csr_labels=lab, rows=rows, base_ranges=values,
        route_offsets=[0, 1, 3, 4, 4, 5, 6, 7], handles=[0, 1],
        route_enabled=[1, 1, 1, 1, 0, 1, 1],
        clauses=[[0, 0, 0, 0], [0, 1, 0, 1], [1, 2, 0, 0], [0, 0, 1, 2], [0, 1, 0, 0],
                 [0, 2, 0, 0], [0, 0, 0, 4]],
        ranges=[[0, 1, 3.0, 0.0], [1, 3, 2.0, 4.0], [0, 2, 0.0, 7.0], [0, 0, 0.0, 0.0]],
        mapping=mapping, offset=3, counts=[0, 1, 17, 31, 32, 33, 63, 64, 65, 97],
    )


def shortlist_fixtures():
    """tests/native/posting_shortlist_heap_test.cpp:47-89."""
    large = [[float((i * 37) % 997), 10000 - i] for i in range(10000)]
    return dict(
        source="tests/native/posting_shortlist_heap_test.cpp:47-89",
        top_m=[
            dict(candidates=[[9.0, 9], [1.0, 7], [4.0, 4], [1.0, 3], [2.0, 8], [0.5, U32MAX],
                             [3.0, 2]], k=4,
                 expected=[[1.0, 3], [1.0, 7], [2.0, 8], [3.0, 2]]),
            dict(candidates=[[3.0, 4], [2.0, 5], [1.0, 6]], k=1, expected=[[1.0, 6]]),
            dict(candidates=large, k=4000, expected=sorted(large)[:4000]),
        ],
        # state after inserting (2, 9) then (2, 7) into a 2-slot heap
        can_enter_empty_k0=[0.0, 1, 0],
        can_enter_initial=[[FLT_MAX, 4, 1], [0.0, U32MAX, 0], ["inf", 1, 0], ["nan", 1, 0]],
        can_enter_after_one=[[100.0, 1, 1]],
        can_enter_after_two=[[2.0, 8, 1], [2.0, 9, 0], [2.0, 10, 0], ["-inf", 1, 1]],
    )


def resident_posting_fixture():
    """tests/native/pq_resident_posting_fixture.h:6-39."""
    return dict(
        source="tests/native/pq_resident_posting_fixture.h:6-39",
        offsets=[0, 3], sizes=[3, 3], ids=[4, 2, 0, 5, 1, 3], masks=[1, 2, 1, 1, 2, 3],
        groups=[1, 0, 1], query_masks=[2, 1, 1], modes=[1, 2, 3], lower=[2.0, 0.0, 2.0],
        upper=[0.0, 5.0, 4.0], values=[2.0, 1.0, 0.0, 4.0, "nan", 3.0],
        n_groups=2, rows=6, samples=6, routes=3, range_count=1, probe_routes=[2, 0, 1],
        expected=[5, U32MAX, U32MAX, U32MAX, U32MAX, 3, U32MAX, U32MAX, 0],
    )


def merge_fixtures():
    """tests/native/rabitq_lowfreq_merge_test.cpp:268-357, 359-415."""
    sorted_routes = []
    for route in range(64):
        q = route % 2
        qr = route // 2
        sorted_routes.append(dict(query=q, ids=[42 + q, 100 + q * 1000 + qr],
                                  dists=[0.01 + qr * 0.001, 1.0 + qr]))
    return dict(
        source="tests/native/rabitq_lowfreq_merge_test.cpp:268-415",
        cases=[
            dict(route_to_query=[0, 0, 0, 1], queries=2, topk=3,
                 ids=[[9, 7, 4], [7, 8, U32MAX], [7, 8, U32MAX], [U32MAX, U32MAX, U32MAX]],
                 dists=[[0.5, 2.0, 1.0], [0.4, 0.5, FLT_MAX], [0.4, 0.5, FLT_MAX],
                        [FLT_MAX, FLT_MAX, FLT_MAX]],
                 expected=[[7, 8, 9], [U32MAX, U32MAX, U32MAX]]),
            dict(route_to_query=[0, 1], queries=2, topk=2,
                 ids=[[5, 7, U32MAX], [U32MAX, U32MAX, U32MAX]],
                 dists=[[0.1, 0.2, FLT_MAX], [FLT_MAX, FLT_MAX, FLT_MAX]],
                 expected=[[5, 7], [U32MAX, U32MAX]],
                 expected_dists=[[0.1, 0.2], [FLT_MAX, FLT_MAX]]),
            dict(route_to_query=[r["query"] for r in sorted_routes], queries=2, topk=10,
                 ids=[r["ids"] for r in sorted_routes], dists=[r["dists"] for r in sorted_routes],
                 expected=[[42] + [99 + r for r in range(1, 10)],
                           [43] + [99 + r + 1000 for r in range(1, 10)]]),
        ],
    )


def fp16_fixture():
    """tests/native/fp16_l2_test.cpp:15-56: hashed fp16 rows vs an fp64
    reference, tolerance 2e-5 * max(1, ref); special values."""
    cases = []
    for cols in (1, 7, 8, 15, 16, 37, 512, 4096):
        query = [float(int(c % 23) - 11) / 7 for c in range(cols)]
        rows = []
        for row in range(3):
            rows.append([((row * 997 + c * 251 + 17) % 0x7C00) |
                         (((row * 997 + c * 251 + 17) & 1) << 15) for c in range(cols)])
        cases.append(dict(cols=cols, query=query, rows=rows))
    return dict(source="tests/native/fp16_l2_test.cpp:15-56", cases=cases, tolerance=2e-5,
                specials=[[1, "finite"], [0x8000, "finite"], [0x7C00, "inf"], [0x7E00, "nan"]])


def rotation_fixture():
    """tests/native/rabitq_query_rotation_test.cu:8-61: shapes and tolerances
    of the FP32 query rotation and centroid distances against FP64."""
    return dict(source="tests/native/rabitq_query_rotation_test.cu:8-61",
                shapes=[[1, 1, 1], [7, 17, 32], [33, 65, 96], [13, 512, 512], [3, 4096, 4096]],
                rotation_tol=[2e-5, 2e-5], centroid_tol=[1e-3, 2e-5])


def range_posting_fixture():
    """tests/native/range_posting_index_test.cpp:123-205: a two-dimension
    FARPIDX1 index, the smallest-slice choices for five query rows and the
    loader's rejections (mutation -> expected message fragment)."""
    return dict(
        source="tests/native/range_posting_index_test.cpp:123-205",
        dimensions=[
            dict(values=[1.0, 2.0, 4.0], offsets=[0, 2, 4, 6], ids=[0, 1, 2, 3, 4, 5]),
            dict(values=[10.0, 20.0, 30.0], offsets=[0, 1, 3, 6], ids=[5, 3, 4, 0, 1, 2]),
        ],
        # per query row: active ranges [range_index, mode, lower, upper]
        queries=[
            [[0, 1, 2.0, 0.0]],
            [[1, 2, 0.0, 20.0]],
            [[0, 3, 2.0, 4.0]],
            [[0, 3, 1.0, 4.0], [1, 3, 10.0, 20.0]],
            [],
        ],
        # expected [has_active_range, active_dimension_count, range_index, begin, count]
        expected=[[1, 1, 0, 4, 2], [1, 1, 1, 0, 1], [1, 1, 0, 2, 2], [1, 2, 1, 0, 1],
                  [0, 0, U32MAX, 0, 0]],
        # eligible_for_scan(slice of row 0, threshold) cases
        eligible=[[1, False], [2, True]],
        rejections=[["bad_magic", "magic mismatch"], ["bad_unique_count", "value-domain size"],
                    ["bad_id", "sample id"], ["duplicate_id", "permutation"],
                    ["truncated", "file size"]],
    )


def main():
    fixtures = {
        "predicate.json": predicate_fixtures(),
        "csr_lookup.json": csr_lookup_cases(),
        "predicate_parallel.json": parallel_fixture(),
        "shortlist_heap.json": shortlist_fixtures(),
        "resident_posting.json": resident_posting_fixture(),
        "route_merge.json": merge_fixtures(),
        "fp16_l2.json": fp16_fixture(),
        "rotation.json": rotation_fixture(),
        "range_posting.json": range_posting_fixture(),
    }
    for name, data in fixtures.items():
        (HERE / name).write_text(json.dumps(data, separators=(",", ":")))
        print("wrote", name)


if __name__ == "__main__":
    main()
