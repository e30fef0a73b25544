"""Lane-level model of the wave-parallel frontier operations
(`wave_smmh_insert`, `wave_smmh_pop_max` in go-fann_amd/csrc/device_common.hpp),
checked against the oracle's serial symmetric min-max heap (include/smmh2.h:76-147,
restated in oracle/gofann_oracle.c) on admission sequences with many ties.

Each function below follows its HIP counterpart step by step: what every one of
the 64 lanes reads, the ballots, the DPP row moves (row shift right by n: lane i
reads lane i - n within its row of 16, else keeps the old value; row shift left
by 1: lane i reads lane i + 1), the scalar walk, and the predicated writes, which
must hit distinct slots.  The array must equal the serial heap's after every
operation, tie for tie, and the maximum the kernels keep in a register (the
admission threshold) must equal slot 2.  The GPU parity tests then compare the
kernels themselves with the oracle.
"""
import ctypes as C
import random

import numpy as np
import pytest

import pyoracle as po

def ctz(x):
    x &= (1 << 64) - 1
    return (x & -x).bit_length() - 1 if x else 64

def msb(x):
    return x.bit_length() - 1

def wave_insert(h, size, e):
    y0 = size; size = y0 + 1
    pair = (y0 - 1) >> 1
    depth = (pair + 1).bit_length() - 1 if pair > 0 else 0
    al, ar = {}, {}
    for lane in range(64):
        act = 1 <= lane <= depth
        a1 = 2 * (((pair + 1) >> lane) - 1) + 1 if act else 1
        al[lane] = h[a1]; ar[lane] = h[a1 + 1]
    sib = h[y0 - 1]
    moved = (y0 & 1) == 0 and e[0] < sib[0]
    y = y0 - 1 if moved else y0
    side = -1
    if depth > 0:
        if al[1][0] > e[0]: side = 0
        elif ar[1][0] < e[0]: side = 1
    mask = 0
    for l in range(64):
        act = 1 <= l <= depth
        v = ar[l] if side == 1 else al[l]
        sg = -1.0 if side == 1 else 1.0
        if side >= 0 and act and sg * v[0] > sg * e[0]:
            mask |= 1 << l
    t = ctz(~(mask >> 1))
    sd = 1 if side == 1 else 0
    writes = []
    for l in range(64):
        act = 1 <= l <= depth
        lv = t if l == 0 else l - 1
        dst = y if lv == 0 else 2 * (((pair + 1) >> lv) - 1) + 1 + sd
        w = e if l == 0 else (ar[l] if side == 1 else al[l])
        wr = l == 0 or (act and l <= t)
        if l == 63:
            dst, w, wr = y0, sib, moved
        if wr:
            writes.append((dst, w))
    idx = [w[0] for w in writes]
    assert len(set(idx)) == len(idx)
    for i, val in writes:
        h[i] = val
    return size

def wave_pop_max(h, size):
    size -= 1
    v = h[size]
    b0 = b1 = 0
    for lane in range(64):
        cl = 4 * lane + 4; cr = cl + 2
        if cr < size and h[min(cr, size - 1)][0] > h[min(cl, size - 1)][0]:
            b0 |= 1 << lane
    if size > 260:
        for lane in range(64):
            cl = 4 * lane + 260; cr = cl + 2
            if cr < size and h[min(cr, size - 1)][0] > h[min(cl, size - 1)][0]:
                b1 |= 1 << lane
    p = d = 0
    while 4 * p + 4 < size:
        bits = b0 if p < 64 else b1
        p = 2 * p + 1 + ((bits >> (p & 63)) & 1)
        d += 1
    assert d <= 15
    slot, R, L = {}, {}, {}
    for lane in range(64):
        k = lane if lane <= d else 0
        slot[lane] = 2 * (((p + 1) >> (d - k)) - 1) + 2
        R[lane] = h[slot[lane]]; L[lane] = h[slot[lane] - 1]
    x = [L[l][0] for l in range(64)]
    for n in (1, 2, 4, 8):
        x = [max(x[l], x[l - n]) if (l % 16) >= n else x[l] for l in range(64)]
    vf = [max(v[0], x[l]) for l in range(64)]
    prev = [vf[l - 1] if (l % 16) >= 1 else v[0] for l in range(64)]
    swapped = 0
    for l in range(64):
        if l <= d and L[l][0] > prev[l]:
            swapped |= 1 << l
    rn = [R[l + 1] if (l % 16) < 15 else R[l] for l in range(64)]
    cm = 0
    for l in range(64):
        if l < d and rn[l][0] > vf[l]:
            cm |= 1 << l
    stop = ctz(~cm)
    upto = swapped & ((2 << stop) - 1)
    lfin = L[msb(upto)] if upto else L[0]
    writes = []
    for lane in range(64):
        above = swapped & ((1 << lane) - 1)
        lsrc = L[msb(above)] if above else L[0]
        if lane <= stop:
            last = lane == stop
            w = (lfin if upto else v) if last else rn[lane]
            writes.append((slot[lane], w))
            if (swapped >> lane) & 1:
                writes.append((slot[lane] - 1, lsrc if above else v))
    idx = [w[0] for w in writes]
    assert len(set(idx)) == len(idx), writes
    for i, val in writes:
        h[i] = val
    newmax = (lfin if upto else v)[0] if stop == 0 else R[1][0]
    assert size < 3 or newmax == h[2][0]
    return size, newmax

def _run(Q, n_ops, vals, seed):
    rng = random.Random(seed)
    N = 520
    ref = (po.Pair * N)()
    rs = C.c_int(1)
    h = [(0.0, 0)] * N
    size = 1
    hmax = -1e30
    for i in range(n_ops):
        e = (float(np.float32(rng.choice(vals))), i + 1)
        if size >= Q + 1 and hmax < e[0]:
            # the kernels skip it; the serial reference check agrees
            assert ref[2].first < e[0]
            continue
        po.lib().orc_smmh2_insert(ref, C.byref(rs), po.Pair(e[0], e[1], 0.0))
        size = wave_insert(h, size, e)
        hmax = max(hmax, e[0])
        if size >= Q + 2:
            po.lib().orc_smmh2_pop_max(ref, C.byref(rs))
            size, hmax = wave_pop_max(h, size)
        assert size == rs.value
        for s in range(1, size):
            assert (ref[s].first, ref[s].second) == h[s], (Q, i, s)
        if size >= 3:
            assert hmax == ref[2].first
    return True



@pytest.mark.parametrize("Q", [2, 3, 62, 126, 127, 258, 259, 260, 261, 300, 448, 510])
@pytest.mark.parametrize("vals", ["three", "ten", "fine"])
def test_wave_heap_model_matches_serial_heap(Q, vals):
    v = {"three": [0, 1, 2], "ten": list(range(10)), "fine": [x / 7 for x in range(1000)]}[vals]
    assert _run(Q, 3 * Q + 150, v, Q * 7 + len(v))
