"""Host-side (CPU) parts of the C-ABI library: the exact rerank worker pool
and the route -> query merge, against the oracle on seeded inputs.  These
entry points touch no GPU, so they run in the CPU suite."""
from __future__ import annotations

import numpy as np
import pytest

import pyoracle as po
from gofann_amd import search as gs

U32MAX = 0xFFFFFFFF


def _shortlists(rng, routes, width, samples, dup=True):
    sl = rng.integers(0, samples, size=(routes, width)).astype(np.uint32)
    sl[rng.random((routes, width)) < 0.1] = U32MAX           # empty slots
    sl[rng.random((routes, width)) < 0.05] = samples + 7     # ids past the base
    if dup:
        sl[:, -3:] = sl[:, :3]                               # duplicates
    return sl


@pytest.mark.parametrize("elem", ["u8", "f32", "f16"])
@pytest.mark.parametrize("threads", [1, 4])
def test_host_rerank_matches_oracle(elem, threads):
    rng = np.random.default_rng(11)
    n, dim, nq, routes, width, topk = 3000, 40, 30, 200, 60, 10
    if elem == "u8":
        base = rng.integers(0, 256, size=(n, dim)).astype(np.uint8)
        queries = rng.integers(0, 256, size=(nq, dim)).astype(np.uint8)
    else:
        base = rng.standard_normal((n, dim)).astype(np.float32 if elem == "f32" else np.float16)
        queries = rng.standard_normal((nq, dim)).astype(np.float32)
    rq = rng.integers(0, nq, size=routes).astype(np.uint32)
    sl = _shortlists(rng, routes, width, n)
    oi, od = po.rerank(base, queries, rq, sl, topk)
    hr = gs.HostRerank(base, queries, threads=threads)
    hi, hd = hr.rerank(sl, rq, topk)
    hr.close()
    if elem == "u8":
        # both sums of squared u8 differences are exact integers: same bits
        assert np.array_equal(hi, oi)
        assert np.array_equal(hd.view(np.uint32), od.view(np.uint32))
    else:
        # fp32 sequential order (host) vs the 64-lane order (oracle/GPU):
        # 1e-5 relative, the north star's rerank tolerance
        assert np.allclose(hd, od, rtol=1e-5, atol=0)
        assert (hi == oi).mean() > 0.99
    # ascending by (distance, id), padding last
    for r in range(routes):
        valid = hi[r] != U32MAX
        d = hd[r][valid]
        assert np.all(d[:-1] <= d[1:])
        assert np.all(hd[r][~valid] == np.finfo(np.float32).max)


def test_host_rerank_matches_brute_force_u8():
    rng = np.random.default_rng(5)
    base = rng.integers(0, 256, size=(500, 192)).astype(np.uint8)
    queries = rng.integers(0, 256, size=(4, 192)).astype(np.uint8)
    sl = np.tile(np.arange(500, dtype=np.uint32)[None, :], (4, 1))
    hr = gs.HostRerank(base, queries, threads=2)
    ids, dists = hr.rerank(sl, np.arange(4, dtype=np.uint32), 10)
    hr.close()
    for q in range(4):
        d = ((base.astype(np.int64) - queries[q].astype(np.int64)) ** 2).sum(1)
        order = np.lexsort((np.arange(500), d))[:10]
        assert np.array_equal(ids[q], order.astype(np.uint32))
        assert np.array_equal(dists[q], d[order].astype(np.float32))


def test_host_merge_matches_oracle():
    rng = np.random.default_rng(3)
    routes, width, queries, topk = 300, 10, 120, 10
    r2q = rng.integers(0, queries, size=routes).astype(np.uint32)
    ids = rng.integers(0, 400, size=(routes, width)).astype(np.uint32)
    ids[rng.random((routes, width)) < 0.1] = U32MAX
    d = rng.integers(0, 50, size=(routes, width)).astype(np.float32)  # ties on purpose
    oi, od = po.merge(r2q, ids, d, queries, topk)
    hi, hd = gs.host_merge_routes(r2q, ids, d, queries, topk)
    assert np.array_equal(hi, oi)
    assert np.array_equal(hd.view(np.uint32), od.view(np.uint32))


def _lane_order_l2(q, b, lanes):
    """Squared L2 in one fp16 kernel's summation order, float32 throughout:
    lane l sums the squared differences of dimensions d = l (mod lanes) of
    the whole blocks, the lane sums are added in lane order, then the tail
    in order (lanes = 1: the dimensions in order)."""
    q = q.astype(np.float32)
    b = b.astype(np.float32)  # fp16 -> fp32 is exact
    dim = q.shape[0]
    main = dim - dim % lanes if lanes > 1 else 0
    total = np.float32(0)
    if main:
        sq = (q[:main] - b[:main]) * (q[:main] - b[:main])
        acc = np.zeros(lanes, np.float32)
        for blk in range(main // lanes):
            acc = acc + sq[blk * lanes:(blk + 1) * lanes]
        for l in range(lanes):
            total = np.float32(total + acc[l])
    for d in range(main, dim):
        diff = np.float32(q[d] - b[d])
        total = np.float32(total + np.float32(diff * diff))
    return total


@pytest.mark.parametrize("kernel,lanes", [("scalar", 1), ("avx2", 8), ("avx512", 16)])
@pytest.mark.parametrize("dim", [40, 512, 77])
def test_host_rerank_fp16_kernels_follow_their_order(monkeypatch, kernel, lanes, dim):
    """Each fp16 kernel (fp16_l2.h's scalar / avx2 / avx512) computes every
    distance in its own summation order, bit for bit; "auto" picks the
    widest the CPU supports, as fp16_l2::select does."""
    lib = gs._lib.load()
    monkeypatch.setenv("GOFANN_FP16_RERANK_KERNEL", kernel)
    rng = np.random.default_rng(dim)
    n, nq, routes, width = 600, 8, 40, 30
    base = (rng.standard_normal((n, dim)) * 3).astype(np.float16)
    queries = (rng.standard_normal((nq, dim)) * 3).astype(np.float32)
    rq = rng.integers(0, nq, size=routes).astype(np.uint32)
    sl = _shortlists(rng, routes, width, n, dup=False)
    try:
        hr = gs.HostRerank(base, queries, threads=2)
    except gs._lib.GofannError:
        pytest.skip(f"this CPU lacks the {kernel} kernel's ISA")
    assert hr.fp16_kernel == kernel
    hi, hd = hr.rerank(sl, rq, 10)
    hr.close()
    for r in range(routes):
        for i, d in zip(hi[r], hd[r]):
            if i == U32MAX:
                continue
            want = _lane_order_l2(queries[rq[r]], base[i], lanes)
            assert np.float32(d).view(np.uint32) == want.view(np.uint32), (r, i)
    # auto = the reference's rule
    monkeypatch.setenv("GOFANN_FP16_RERANK_KERNEL", "auto")
    hr = gs.HostRerank(base, queries, threads=1)
    import ctypes as C
    avail = ["scalar"]
    if all(f in open("/proc/cpuinfo").read() for f in (" avx2", " f16c")):
        avail.append("avx2")
        if " avx512f" in open("/proc/cpuinfo").read():
            avail.append("avx512")
    assert hr.fp16_kernel == avail[-1]
    hr.close()
    monkeypatch.setenv("GOFANN_FP16_RERANK_KERNEL", "bogus")
    with pytest.raises(gs._lib.GofannError):
        gs.HostRerank(base, queries, threads=1)
    assert lib is not None and C is not None


def test_host_rerank_fp16_variable_read_for_fp16_rows_only(monkeypatch):
    """The fp16 kernel variable is read only for fp16 rows, as the
    reference reads GO_FANN_FP16_RERANK_KERNEL only for fp16 sources
    (dataloader.cpp:2132): an unknown name fails an fp16 create and leaves
    u8 and f32 creates alone; the reference's variable name is honoured when
    this library's is unset."""
    rng = np.random.default_rng(5)
    q = rng.standard_normal((4, 16)).astype(np.float32)
    monkeypatch.delenv("GOFANN_FP16_RERANK_KERNEL", raising=False)
    monkeypatch.setenv("GO_FANN_FP16_RERANK_KERNEL", "bogus")
    for base in (rng.integers(0, 255, (50, 16)).astype(np.uint8),
                 rng.standard_normal((50, 16)).astype(np.float32)):
        hr = gs.HostRerank(base, q if base.dtype != np.uint8 else q.astype(np.uint8), threads=1)
        assert hr.fp16_kernel == "scalar"
        hr.close()
    f16 = rng.standard_normal((50, 16)).astype(np.float16)
    with pytest.raises(gs._lib.GofannError):
        gs.HostRerank(f16, q, threads=1)
    monkeypatch.setenv("GO_FANN_FP16_RERANK_KERNEL", "scalar")
    hr = gs.HostRerank(f16, q, threads=1)
    assert hr.fp16_kernel == "scalar"
    hr.close()
    # this library's name wins when both are set
    monkeypatch.setenv("GOFANN_FP16_RERANK_KERNEL", "bogus")
    with pytest.raises(gs._lib.GofannError):
        gs.HostRerank(f16, q, threads=1)
