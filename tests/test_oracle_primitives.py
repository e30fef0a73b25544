"""Pins the oracle's search primitives against the reference's own headers
compiled into oracle/_ref (include/smmh2.h, include/bin_heap.h,
src/search/common/native_visited_hash.cuh), array for array, and the frontier
pickup rule (backend_pq.cu:824-892) by brute force.

Operation sequences are random with many ties on purpose: the layout of a
heap decides which of several equal entries a later pop or pickup returns,
so a different but valid heap would fail here."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import pyoracle as po

U32MAX = 0xFFFFFFFF


def _ref():
    R = po.ref()
    if R is None or not hasattr(R, "ref_smmh2_insert"):
        pytest.skip("oracle/_ref not built (reference sources absent)")
    R.ref_hash_code.restype = C.c_uint32
    R.ref_hash_code.argtypes = [C.c_uint32]
    R.ref_hash_add.argtypes = [C.c_void_p, C.c_uint32]
    R.ref_hash_test.argtypes = [C.c_void_p, C.c_uint32]
    R.ref_hash_clear.argtypes = [C.c_void_p]
    R.ref_smmh2_insert.argtypes = [C.c_void_p, C.POINTER(C.c_int), C.c_void_p]
    R.ref_smmh2_pop_max.argtypes = [C.c_void_p, C.POINTER(C.c_int), C.c_void_p]
    R.ref_smmh2_pop_min.argtypes = [C.c_void_p, C.POINTER(C.c_int), C.c_void_p]
    R.ref_bin_heap_push.argtypes = [C.c_void_p, C.c_int]
    R.ref_bin_heap_pop.argtypes = [C.c_void_p, C.c_int, C.c_void_p]
    return R


def _heap_bytes(h, size):
    return bytes(memoryview(h).cast("B")[: size * C.sizeof(po.Pair)])


# ---------------------------------------------------------------- smmh2
@pytest.mark.parametrize("seed", range(6))
def test_smmh2_layout_matches_reference_header(seed):
    """insert / pop_max / pop_min leave the same array (first, second, base)
    as smmh2.h over the reference's BiasedPair after every operation."""
    L, R = po.lib(), _ref()
    rng = np.random.default_rng(100 + seed)
    cap = 700
    ho, hr = (po.Pair * cap)(), (po.Pair * cap)()
    so, sr = C.c_int(1), C.c_int(1)
    # distance alphabets: few values (heavy ties), halves, and wide floats
    alphabet = [4, 17, 1000][seed % 3]
    for step in range(3000):
        op = rng.random()
        if (op < 0.55 or so.value < 3) and so.value < cap - 1:
            d = float(rng.integers(0, alphabet)) / 2.0
            e = po.Pair(d, int(rng.integers(0, 1 << 31)), float(rng.integers(0, 9)))
            L.orc_smmh2_insert(ho, C.byref(so), e)
            R.ref_smmh2_insert(hr, C.byref(sr), C.byref(e))
        elif op < 0.8:
            out = po.Pair()
            got = L.orc_smmh2_pop_max(ho, C.byref(so))
            R.ref_smmh2_pop_max(hr, C.byref(sr), C.byref(out))
            assert (got.first, got.second, got.base) == (out.first, out.second, out.base)
        else:
            out = po.Pair()
            got = L.orc_smmh2_pop_min(ho, C.byref(so))
            R.ref_smmh2_pop_min(hr, C.byref(sr), C.byref(out))
            assert (got.first, got.second, got.base) == (out.first, out.second, out.base)
        assert so.value == sr.value
        assert _heap_bytes(ho, so.value)[C.sizeof(po.Pair):] == \
            _heap_bytes(hr, sr.value)[C.sizeof(po.Pair):], f"step {step}"


def test_smmh2_bounded_beam_sequence_matches_reference_header():
    """The traversal's use: insert, then pop_max once the heap holds Q + 2
    slots (backend_pq.cu:4889-4907), over a long tie-heavy stream."""
    L, R = po.lib(), _ref()
    rng = np.random.default_rng(7)
    for Q in (2, 5, 16, 63):
        ho, hr = (po.Pair * (Q + 4))(), (po.Pair * (Q + 4))()
        so, sr = C.c_int(1), C.c_int(1)
        for i in range(2000):
            e = po.Pair(float(rng.integers(0, 12)), i, 0.0)
            L.orc_smmh2_insert(ho, C.byref(so), e)
            R.ref_smmh2_insert(hr, C.byref(sr), C.byref(e))
            if so.value >= Q + 2:
                out = po.Pair()
                L.orc_smmh2_pop_max(ho, C.byref(so))
                R.ref_smmh2_pop_max(hr, C.byref(sr), C.byref(out))
            assert so.value == sr.value
            assert _heap_bytes(ho, so.value)[C.sizeof(po.Pair):] == \
                _heap_bytes(hr, sr.value)[C.sizeof(po.Pair):], f"Q {Q} insert {i}"


# ---------------------------------------------------------------- bin heap
class _RP(C.Structure):
    _fields_ = [("first", C.c_float), ("second", C.c_uint32)]


@pytest.mark.parametrize("seed", range(4))
def test_bin_heap_matches_reference_header(seed):
    """orc_result_push / orc_result_pop (the result and stop heaps) leave the
    same array as bin_heap.h's push_heap / pop_heap after every operation."""
    L, R = po.lib(), _ref()
    L.orc_result_pop.restype = _RP
    L.orc_result_pop.argtypes = [C.c_void_p, C.c_int]
    L.orc_result_push.argtypes = [C.c_void_p, C.c_int]
    rng = np.random.default_rng(200 + seed)
    cap = 300
    ho, hr = (_RP * cap)(), (_RP * cap)()
    size = 0
    for step in range(4000):
        if (rng.random() < 0.6 or size == 0) and size < cap:
            e = _RP(float(rng.integers(0, [3, 20, 500, 9][seed])), step)
            ho[size], hr[size] = e, e
            size += 1
            L.orc_result_push(ho, size)
            R.ref_bin_heap_push(hr, size)
        else:
            out = _RP()
            got = L.orc_result_pop(ho, size)
            R.ref_bin_heap_pop(hr, size, C.byref(out))
            assert (got.first, got.second) == (out.first, out.second)
            size -= 1
        assert bytes(memoryview(ho).cast("B")[: 8 * size]) == \
            bytes(memoryview(hr).cast("B")[: 8 * size]), f"step {step}"


# ---------------------------------------------------------------- visited hash
def test_hash_code_matches_reference_header():
    L, R = po.lib(), _ref()
    rng = np.random.default_rng(11)
    vals = np.concatenate([rng.integers(0, 2**32, 20000, dtype=np.uint64),
                           np.arange(0, 70000, 7), [65535, 65536, 131071, U32MAX - 1, U32MAX]])
    for v in vals:
        assert L.orc_hash_code(C.c_uint32(int(v))) == R.ref_hash_code(int(v))


@pytest.mark.parametrize("spread", [1 << 12, 1 << 20, 1 << 32])
def test_hash_table_matches_reference_header_through_full(spread):
    """Random adds (duplicates included) until the 4096-slot table is full
    and beyond: the tables stay identical, and test() agrees on present,
    absent and full-table lookups."""
    L, R = po.lib(), _ref()
    rng = np.random.default_rng(spread % 97)
    to, tr = np.empty(4096, np.uint32), np.empty(4096, np.uint32)
    L.orc_hash_clear(po.p(to))
    R.ref_hash_clear(po.p(tr))
    assert np.array_equal(to, tr) and np.all(to == U32MAX)
    vals = rng.integers(0, spread - 1, 6000, dtype=np.uint64)
    for i, v in enumerate(vals):
        L.orc_hash_add(po.p(to), C.c_uint32(int(v)))
        R.ref_hash_add(po.p(tr), int(v))
        if i % 97 == 0 or i > 4000:
            assert np.array_equal(to, tr), f"add {i}"
    assert np.array_equal(to, tr)
    probe = np.concatenate([vals[:300], rng.integers(0, spread - 1, 300, dtype=np.uint64)])
    for v in probe:
        assert L.orc_hash_test(po.p(to), C.c_uint32(int(v))) == \
            R.ref_hash_test(po.p(tr), int(v))


# ---------------------------------------------------------------- pickup
def test_pickup_unused_tie_rule_brute_force():
    """pickup_next_unused_from_pool (backend_pq.cu:824-842) and its
    cooperative twin (:844-892): among entries 1..size-1 without the used bit,
    the least `first`, and the lowest index among equal ones, is returned and
    marked used.  Brute force: lexicographic minimum of (first, index)."""
    L = po.lib()
    L.orc_pickup_unused.argtypes = [C.c_void_p, C.c_int, C.POINTER(po.Pair)]
    rng = np.random.default_rng(5)
    USED = 0x80000000
    for trial in range(3000):
        size = int(rng.integers(1, 70))
        first = rng.integers(0, int(rng.integers(1, 6)), size).astype(np.float32)
        if trial % 5 == 0:
            first[rng.random(size) < 0.2] = -0.0
        used = rng.random(size) < rng.random()
        pool = (po.Pair * max(size, 1))()
        for i in range(size):
            pool[i] = po.Pair(float(first[i]), (i | USED) if used[i] else i, 0.0)
        cand = [i for i in range(1, size) if not used[i]]
        out = po.Pair()
        found = L.orc_pickup_unused(pool, size, C.byref(out))
        if not cand:
            assert found == 0
            continue
        idx = np.array(cand)
        order = np.lexsort((idx, first[idx]))  # by first, then index
        want = int(idx[order[0]])
        assert found == 1
        assert out.second == want
        assert pool[want].second == (want | USED)
        for i in range(size):
            if i != want:
                assert pool[i].second == ((i | USED) if used[i] else i)
