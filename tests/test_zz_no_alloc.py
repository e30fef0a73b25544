"""GPU check of gofann_exact_search_noalloc against gofann_exact_search.

The no-alloc entry point keeps visited slabs in a fixed per-GPU device array
instead of context scratch.  Through the C ABI, two calls in a row (the second
on a smaller batch, so it reuses the array the first call left behind) must
equal the allocating entry point bit for bit (ids, distance bits, the eight
per-route counters) in every visited-set placement; a batch beyond the
array's route limit is rejected before anything is launched, and an LDS
placement (no slab) takes any batch size."""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from gofann_amd import _lib
from gofann_amd import index as gi
from gofann_amd import plan as gp
from gofann_amd import search as gs
from gofann_amd import synth

pytestmark = pytest.mark.gpu
MAX_ROUTES = 4096


def say(*a):
    print("[gpu-test]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def world(gpu_ctx):
    wl = synth.small_labelled(n=6000, nq=96, dim=64, k=10, sigma=0.7, labels=5, seed=83,
                              tags=True, dtype="u8")
    li = gi.build_label_index(wl.base, wl.label_offsets, wl.label_values, wl.num_labels,
                              wl.centroids, degree=32, threshold=300)
    rs = gp.plan_queries(li, wl.query_labels).graph
    dev = dict(base=wl.base.cuda(), q=wl.queries.cuda(), ls=gs.u32(li.label_size))
    return wl, li, rs, dev


def _subset(rs, idx):
    idx = np.asarray(idx)
    pred = gp.compile_residuals(
        [list(rs.predicate.handles[rs.predicate.clauses[rs.predicate.route_offsets[i]]["label_begin"]:
                                   rs.predicate.clauses[rs.predicate.route_offsets[i]]["label_end"]])
         for i in idx], [[] for _ in idx])
    return gp.RouteSet(rs.route_query[idx], rs.route_group[idx], rs.route_start[idx],
                       rs.route_to_query[idx], pred)


def _call(ctx, fn, wl, dev, dg, dr, n, prm, topk):
    ids = torch.full((n * topk,), -7, dtype=torch.int32, device="cuda")
    dists = torch.full((n * topk,), -7.0, device="cuda")
    st = torch.full((n * 8,), -7, dtype=torch.int32, device="cuda")
    rc = fn(ctx.handle, _lib.ptr(dev["base"]), _lib.ELEM_U8, wl.dim, wl.n, _lib.ptr(dev["q"]),
            dg.view(), _lib.ptr(dev["ls"]), dr.predicate_view(dg, 0.0, False), dr.routes_view(),
            prm, _lib.ptr(ids), _lib.ptr(dists), _lib.ptr(st))
    torch.cuda.synchronize()
    return rc, ids.cpu().numpy().view(np.uint32).reshape(n, topk), \
        dists.cpu().numpy().reshape(n, topk).view(np.uint32), st.cpu().numpy().reshape(n, 8)


@pytest.mark.parametrize("hash_mode", [_lib.PLACE_AUTO, _lib.PLACE_GLOBAL, _lib.PLACE_SPILL,
                                       _lib.PLACE_LDS])
@pytest.mark.parametrize("Q", [32, 96])
def test_noalloc_matches_allocating_entry_point(gpu_ctx, world, hash_mode, Q):
    wl, li, rs, dev = world
    dg = gs.DeviceGraph.upload(li, neighbor_samples=True)
    prm = _lib.ExactParams(Q, 1, _lib.EARLY_STOP_ADAPTIVE, 0, 10, hash_mode)
    rng = np.random.default_rng(Q + hash_mode)
    first = np.arange(rs.count)
    second = np.sort(rng.choice(rs.count, size=rs.count // 3, replace=False))
    for label, idx in (("first", first), ("second (smaller)", second)):
        sub = _subset(rs, idx)
        dr = gs.DeviceRoutes.upload(sub)
        say("no-alloc exact search, hash_mode", hash_mode, "Q", Q, label, "batch", sub.count)
        ref = _call(gpu_ctx, gpu_ctx.lib.gofann_exact_search, wl, dev, dg, dr, sub.count, prm, 10)
        got = _call(gpu_ctx, gpu_ctx.lib.gofann_exact_search_noalloc, wl, dev, dg, dr, sub.count,
                    prm, 10)
        assert ref[0] == _lib.OK and got[0] == _lib.OK, gpu_ctx.last_error()
        assert np.array_equal(got[1], ref[1])
        assert np.array_equal(got[2], ref[2])
        assert np.array_equal(got[3], ref[3])
        assert (ref[1][:, 0] != 0xFFFFFFFF).sum() > sub.count // 2
        assert ref[3][:, 0].max() > 3


def test_noalloc_batch_limit(gpu_ctx, world):
    wl, li, rs, dev = world
    dg = gs.DeviceGraph.upload(li)
    reps = -(-(MAX_ROUTES + 1) // rs.count)
    big = _subset(rs, np.tile(np.arange(rs.count), reps)[:MAX_ROUTES + 4])
    dr = gs.DeviceRoutes.upload(big)
    say("no-alloc exact search, batch of", big.count, "routes with a global visited slab")
    rc, *_ = _call(gpu_ctx, gpu_ctx.lib.gofann_exact_search_noalloc, wl, dev, dg, dr, big.count,
                   _lib.ExactParams(32, 1, 2, 0, 10, _lib.PLACE_GLOBAL), 10)
    assert rc == _lib.ERR_INVALID
    assert "no-alloc" in gpu_ctx.last_error()
    say("no-alloc exact search, batch of", big.count, "routes with the visited set in LDS")
    prm = _lib.ExactParams(32, 1, 2, 0, 10, _lib.PLACE_LDS)
    ref = _call(gpu_ctx, gpu_ctx.lib.gofann_exact_search, wl, dev, dg, dr, big.count, prm, 10)
    got = _call(gpu_ctx, gpu_ctx.lib.gofann_exact_search_noalloc, wl, dev, dg, dr, big.count,
                prm, 10)
    assert ref[0] == _lib.OK and got[0] == _lib.OK
    for a, b in zip(got[1:], ref[1:]):
        assert np.array_equal(a, b)
