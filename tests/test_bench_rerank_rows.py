"""bench.rerank_rows hands gofann_exact_rerank the right slice of a pipeline.

The C3/C4/C5 pipelines rerank each route class on its own stream and the
posting routes behind the scan, each call covering shortlist rows lo..hi.
Routes are independent, so the split gives the single launch's results only
if every call starts its route_query, shortlist and output pointers at row
lo (shortlists W wide, outputs 10 wide) and passes hi - lo routes.  This
checks the arguments on the host with a recording stand-in for the library
(no GPU).
"""
from __future__ import annotations

import types

import torch

import bench
from gofann_amd import _lib


class _Lib:
    def __init__(self):
        self.calls = []

    def gofann_exact_rerank(self, *args):
        self.calls.append(args)
        return 0


class _Ctx:
    def __init__(self):
        self.lib = _Lib()
        self.handle = object()

    def check(self, rc):
        assert rc == 0


def _pipe(n, W, dim, dtype):
    return types.SimpleNamespace(
        L=_lib, W=W, torch=torch,
        wl=types.SimpleNamespace(base=torch.zeros(50, dim, dtype=dtype),
                                 queries=torch.zeros(7, dim, dtype=torch.float32)),
        route_query=torch.arange(n, dtype=torch.int32),
        sl_i=torch.zeros(n * W, dtype=torch.int32),
        fin_i=torch.zeros(n * 10, dtype=torch.int32),
        fin_d=torch.zeros(n * 10, dtype=torch.float32))


def test_rows_lo_hi_offsets_every_pointer():
    n, W, dim = 12, 6, 24
    p = _pipe(n, W, dim, torch.float16)
    ctx = _Ctx()
    bench.rerank_rows(p, ctx, 4, 9)
    (args,) = ctx.lib.calls
    (handle, base, elem, d, samples, queries, rq, sl, width, routes, topk, oi, od) = args
    assert handle is ctx.handle
    assert base == p.wl.base.data_ptr() and elem == _lib.ELEM_F16
    assert (d, samples, width, routes, topk) == (dim, 50, W, 5, 10)
    assert queries == p.wl.queries.data_ptr()
    assert rq == p.route_query.data_ptr() + 4 * 4
    assert sl == p.sl_i.data_ptr() + 4 * W * 4
    assert oi == p.fin_i.data_ptr() + 4 * 10 * 4
    assert od == p.fin_d.data_ptr() + 4 * 10 * 4


def test_empty_range_launches_nothing_and_splits_cover_every_row():
    n, W = 10, 4
    p = _pipe(n, W, 8, torch.float32)
    ctx = _Ctx()
    bench.rerank_rows(p, ctx, 6, 6)
    assert ctx.lib.calls == []
    # classes (0, 3) and (3, 7) on their streams, posting rows (7, 10) after the scan
    for lo, hi in ((0, 3), (3, 7), (7, 10)):
        bench.rerank_rows(p, ctx, lo, hi)
    starts = [(c[6] - p.route_query.data_ptr()) // 4 for c in ctx.lib.calls]
    counts = [c[9] for c in ctx.lib.calls]
    assert starts == [0, 3, 7] and counts == [3, 4, 3] and sum(counts) == n
    assert all(c[2] == _lib.ELEM_F32 for c in ctx.lib.calls)
