"""Pins oracle functions that no reference fixture covers, by closed forms,
invariants and brute force (each chosen so a dropped term, wrong sign,
index or transposed operand fails)."""
from __future__ import annotations

import ctypes as C
import math

import numpy as np
import pytest

import pyoracle as po

FLT_MAX = np.finfo(np.float32).max
U32MAX = 0xFFFFFFFF


# ---------------------------------------------------------------- visited hash
def test_hash_code_closed_form():
    L = po.lib()
    rng = np.random.default_rng(1)
    vals = np.concatenate([rng.integers(0, 2**32, 2000, dtype=np.uint64), [0, 1, 65535, 65536, U32MAX]])
    for v in vals:
        v = int(v)
        mixed = (v ^ (((v >> 16) * 0x4BCB391F924ED183) & 0xFFFFFFFFFFFFFFFF) ^ 0xA0AB69CCD854FC0A)
        assert L.orc_hash_code(C.c_uint32(v)) == mixed % 4096


def test_hash_set_semantics_until_full():
    L = po.lib()
    table = np.empty(4096, np.uint32)
    L.orc_hash_clear(po.p(table))
    assert np.all(table == U32MAX)
    rng = np.random.default_rng(2)
    added = set()
    for v in rng.integers(0, 1 << 22, 4000):
        L.orc_hash_add(po.p(table), C.c_uint32(int(v)))
        added.add(int(v))
    for v in list(added)[:500] + [int(x) for x in rng.integers(1 << 22, 1 << 23, 500)]:
        assert L.orc_hash_test(po.p(table), C.c_uint32(v)) == (v in added)
    # full table: add drops silently, test of a new value stays false
    for v in range(100000, 100000 + 200):
        L.orc_hash_add(po.p(table), C.c_uint32(v))
    assert int((table != U32MAX).sum()) == 4096
    assert L.orc_hash_test(po.p(table), C.c_uint32(999_999_999)) == 0


# ---------------------------------------------------------------- smmh2
def _smmh_state(h, size):
    return [(h[i].first, h[i].second) for i in range(1, size)]


def test_smmh2_min_max_invariants_random_ops():
    L = po.lib()
    rng = np.random.default_rng(4)
    for trial in range(30):
        h = (po.Pair * 600)()
        size = C.c_int(1)
        ref = []
        for step in range(400):
            op = rng.random()
            if op < 0.6 or size.value < 3:
                d = float(rng.integers(0, 50)) / 2.0  # many ties on purpose
                e = po.Pair(d, step, d)
                L.orc_smmh2_insert(h, C.byref(size), e)
                ref.append((d, step))
            elif op < 0.8:
                got = L.orc_smmh2_pop_max(h, C.byref(size))
                m = max(r[0] for r in ref)
                assert got.first == m
                ref.remove((got.first, got.second))
            else:
                got = L.orc_smmh2_pop_min(h, C.byref(size))
                m = min(r[0] for r in ref)
                assert got.first == m
                ref.remove((got.first, got.second))
            assert size.value == len(ref) + 1
            st = _smmh_state(h, size.value)
            assert sorted(st) == sorted(ref)            # multiset preserved
            if len(ref) >= 1:
                assert h[1].first == min(r[0] for r in ref)
            if len(ref) >= 2:
                assert h[2].first == max(r[0] for r in ref)
            for i in range(1, size.value):              # base travels with entry
                assert h[i].base == h[i].first


def test_whole_entry_heap_fixture():
    """gpu_predicate_cuda_test.cu:19-28: biased entries keep their raw base
    through swaps and pop_max (base == id - 10)."""
    L = po.lib()
    h = (po.Pair * 40)()
    size = C.c_int(1)
    for i in range(20):
        raw = float(i) - 10
        pri = L.orc_priority(raw, 5.0, int(i % 2 == 0), None)
        L.orc_smmh2_insert(h, C.byref(size), po.Pair(pri, i, raw))
        if size.value >= 10:
            L.orc_smmh2_pop_max(h, C.byref(size))
        for j in range(1, size.value):
            assert h[j].base == float(h[j].second) - 10


def test_failed_bridge_navigation_fixture():
    """gpu_predicate_cuda_test.cu:29-45: a failed predicate never suppresses
    adjacency: chain 0 -> 1 -> 2 over samples {2, 65536, 65537}, route 1
    requires labels {0, 1}; all three are visited, only the last passes."""
    L = po.lib()
    off = [0]
    lab = []
    for s in range(65538):
        lab.extend({0: [0], 65535: [0], 65536: [0], 65537: [0, 1]}.get(s, []))
        off.append(len(lab))
    pa = po.PredicateArrays([0, 1, 3], [0, 0, 1], None, None, None, None, off, lab, 65538)
    sample = [2, 65536, 65537]
    h = (po.Pair * 8)()
    size = C.c_int(1)
    L.orc_smmh2_insert(h, C.byref(size), po.Pair(0.0, 0, 0.0))
    visited = passed = 0
    while size.value > 1:
        best = 1
        for j in range(2, size.value):
            if h[j].first < h[best].first:
                best = j
        now = po.Pair(h[best].first, h[best].second, h[best].base)
        size.value -= 1
        h[best] = h[size.value]
        if visited & (1 << now.second):
            continue
        visited |= 1 << now.second
        if L.orc_pred_matches(C.byref(pa.struct), 1, sample[now.second], None):
            passed |= 1 << now.second
        if now.second < 2:
            nxt = now.second + 1
            ok = L.orc_pred_matches(C.byref(pa.struct), 1, sample[nxt], None)
            base = -float(nxt)
            L.orc_smmh2_insert(h, C.byref(size), po.Pair(L.orc_priority(base, 10.0, ok, None), nxt, base))
    assert visited == 7 and passed == 4


# ---------------------------------------------------------------- early stop
def test_adaptive_limit_closed_form():
    L = po.lib()
    for Q in (1, 2, 16, 64, 100, 512):
        for exp in (0, 1, 5, 40, 300):
            for ps in (0, 1, exp):
                for sw in (0, 10):
                    base = max((max(Q, 1) + 1) // 2, sw * 2 if sw > 0 else 1)
                    denom = max(exp + 16, 1)
                    pe = min(ps + 8, denom)
                    rej = max(denom - pe, 0)
                    extra = min(max(-(-(Q * rej) // (2 * denom)), 0), 32)
                    assert L.orc_adaptive_early_stop_limit(Q, exp, ps, sw) == base + extra
    # modes: off never stops, fixed compares with the fixed limit
    assert L.orc_early_stop_reached(1, 10**6, 1, 64, 0, 0, 10) == 0
    assert L.orc_early_stop_reached(0, 3, 3, 64, 0, 0, 10) == 1
    assert L.orc_early_stop_reached(0, 2, 3, 64, 0, 0, 10) == 0


# ---------------------------------------------------------------- PQ
def test_pq_lut_and_adc_against_float64():
    rng = np.random.default_rng(5)
    for dim, M in ((128, 32), (192, 48), (64, 16), (128, 64)):
        table = rng.normal(size=(256, dim)).astype(np.float32) * 20 + 128
        q = rng.integers(0, 256, dim).astype(np.uint8)
        lut = po.pq_lut(table, q, M).reshape(M, 256)
        sub = dim // M
        q64 = q.astype(np.float64)
        want = ((q64.reshape(M, 1, sub) - table.astype(np.float64).reshape(256, M, sub)
                 .transpose(1, 0, 2)) ** 2).sum(-1)
        assert np.allclose(lut, want, rtol=1e-6, atol=1e-3)
        # ADC of a code == squared distance to its reconstruction
        for _ in range(20):
            code = rng.integers(0, 256, M).astype(np.uint8)
            recon = np.concatenate([table[code[m], m * sub:(m + 1) * sub] for m in range(M)])
            exact = float(((q64 - recon.astype(np.float64)) ** 2).sum())
            got = po.pq_adc(lut.reshape(-1), code)
            assert abs(got - exact) <= 1e-5 * exact


def test_pq_adc_tree_order_is_pairwise_32():
    """The graph ADC's float order is the 32-lane xor-butterfly tree: with
    values chosen so a different association rounds differently, only the
    tree order reproduces the oracle's bits."""
    L = po.lib()
    M = 64
    lut = np.zeros((M, 256), np.float32)
    code = np.zeros(M, np.uint8)
    vals = np.float32(1.0) + np.arange(M, dtype=np.float32) * np.float32(1e-7) * 3
    vals[::7] = np.float32(2 ** 24)
    lut[np.arange(M), 0] = vals
    got = po.pq_adc(lut.reshape(-1), code)
    s = np.zeros(32, np.float32)
    for j in range(32):
        acc = np.float32(0)
        for m in range(j, M, 32):
            acc = np.float32(acc + vals[m])
        s[j] = acc
    off = 16
    while off:
        s[:off] = (s[:off] + s[off:2 * off]).astype(np.float32)
        off //= 2
    assert np.float32(got) == s[0]


def test_pq_lut_f32_queries():
    rng = np.random.default_rng(6)
    table = rng.normal(size=(256, 128)).astype(np.float32)
    q = rng.normal(size=128).astype(np.float32)
    lut = po.pq_lut(table, q, 32).reshape(32, 256)
    want = ((q.astype(np.float64).reshape(32, 1, 4) -
             table.astype(np.float64).reshape(256, 32, 4).transpose(1, 0, 2)) ** 2).sum(-1)
    assert np.allclose(lut, want, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------- RaBitQ
def _pack_msb(bits):
    P = bits.shape[0]
    words = np.zeros(P // 32, np.uint32)
    for d in range(P):
        if bits[d]:
            words[d // 32] |= np.uint32(1 << (31 - d % 32))
    return words.view(np.uint8)


def test_rabitq_ip_three_ways_and_brute_force():
    rng = np.random.default_rng(7)
    for P in (64, 128, 512, 4096):
        for _ in range(10):
            q8 = rng.integers(-127, 128, P).astype(np.int8)
            q8[:3] = [-127, 127, 0]
            bits = rng.random(P) < 0.5
            code = _pack_msb(bits)
            want = int(q8.astype(np.int64)[bits].sum())
            assert po.rabitq_ip(q8, code, "int") == want
            assert po.rabitq_ip(q8, code, "popcount") == want
            assert po.rabitq_ip(q8, code, "dp4a") == want


def test_rabitq_quantize_properties():
    rng = np.random.default_rng(8)
    for P in (64, 512, 4096):
        r = rng.normal(size=P).astype(np.float32)
        q8, scale, k1 = po.rabitq_quantize(r)
        assert scale == np.float32(np.abs(r).max() / np.float32(127))
        assert np.all(np.abs(q8) <= 127)
        # round half to even on the exact quotient
        quot = (r / np.float32(scale)).astype(np.float32)
        assert np.array_equal(q8, np.clip(np.rint(quot), -127, 127).astype(np.int8))
        assert abs(k1 + 0.5 * float(r.astype(np.float64).sum())) <= 1e-5 * (1 + abs(r).sum())
    q8, scale, k1 = po.rabitq_quantize(np.zeros(64, np.float32))
    assert scale == 1.0 and np.all(q8 == 0) and k1 == 0.0


def test_rabitq_k1_block256_order():
    """k1 follows the 256-thread strided-partial + tree order exactly."""
    rng = np.random.default_rng(9)
    r = (rng.normal(size=4096) * 1000).astype(np.float32)
    r[::5] *= 1e-4
    _, _, k1 = po.rabitq_quantize(r)
    part = np.zeros(256, np.float32)
    for t in range(256):
        acc = np.float32(0)
        for d in range(t, 4096, 256):
            acc = np.float32(acc + r[d])
        part[t] = acc
    s = 128
    while s:
        part[:s] = (part[:s] + part[s:2 * s]).astype(np.float32)
        s //= 2
    assert np.float32(k1) == np.float32(part[0] * np.float32(-0.5))


def test_rabitq_estimator_matches_reconstruction_identity():
    """f_add + g + f_rescale*<q_r, xu> equals the RaBitQ estimate
    |r|^2 + |q-c|^2 - 2|r|^2 <q-c, xu>/<r, xu> (float64 closed form)."""
    L = po.lib()
    rng = np.random.default_rng(10)
    P = 128
    for _ in range(20):
        r = rng.normal(size=P)
        c = rng.normal(size=P)
        qr = rng.normal(size=P).astype(np.float32)
        bits = r > 0
        xu = bits - 0.5
        l2 = (r * r).sum()
        ipr = (r * xu).sum()
        f_add = l2 + 2 * l2 * (c * xu).sum() / ipr
        f_res = -2 * l2 / ipr
        g = ((qr - c) ** 2).sum()
        q8, scale, k1 = po.rabitq_quantize(qr)
        ip = po.rabitq_ip(q8, _pack_msb(bits), "int")
        got = L.orc_rabitq_score_b1(ip, scale, k1, np.float32(f_add), np.float32(f_res), np.float32(g))
        want = l2 + g - 2 * l2 * ((qr - c) * xu).sum() / ipr
        # int8 quantization of q_r dominates the error
        assert abs(got - want) <= 0.05 * (abs(want) + l2)


# ---------------------------------------------------------------- rerank
def test_rerank_brute_force():
    rng = np.random.default_rng(12)
    for dtype in (np.uint8, np.float32, np.float16):
        n, d = 300, 48
        if dtype == np.uint8:
            base = rng.integers(0, 256, (n, d)).astype(np.uint8)
            q = rng.integers(0, 256, (5, d)).astype(np.uint8)
        else:
            base = rng.normal(size=(n, d)).astype(dtype)
            q = rng.normal(size=(5, d)).astype(np.float32)
        sl = rng.integers(0, n + 5, (5, 40)).astype(np.uint32)
        sl[:, ::9] = U32MAX
        sl[:, 1] = sl[:, 2]  # duplicate candidate
        ids, dists = po.rerank(base, q, np.arange(5, dtype=np.uint32), sl, 10)
        for r in range(5):
            cand = sorted({int(s) for s in sl[r] if s != U32MAX and s < n})
            d64 = [float(((base[s].astype(np.float64) - q[r].astype(np.float64)) ** 2).sum()) for s in cand]
            order = sorted(zip(d64, cand))[:10]
            if dtype == np.uint8:
                assert [i for _, i in order] == ids[r, :len(order)].tolist()
                assert np.array_equal(dists[r, :len(order)], np.array([x for x, _ in order], np.float32))
            else:
                assert np.allclose(dists[r, :len(order)], [x for x, _ in order], rtol=1e-5)
            assert np.all(ids[r, len(order):] == U32MAX)
