"""Reference-format artifacts searched on the GPU: a label index written as
graph.bin + metadata/seed sidecars + .spmat and u8bin base vectors, loaded
back (graph streamed into HBM through pinned windows) and searched by the
exact route, must give the oracle's results; the PQ code file streams into
strided per-sample records unchanged."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import pyoracle as po
from gofann_amd import _lib
from gofann_amd import artifacts as ga
from gofann_amd import plan as gp
from gofann_amd import search as gs
from test_gpu_exact import _world, say

pytestmark = pytest.mark.gpu


def test_graph_streams_into_hbm(gpu_ctx, tmp_path):
    g = np.random.default_rng(2).integers(0, 1 << 32, size=(5000, 24), dtype=np.uint32)
    path = tmp_path / "graph.bin"
    ga.write_graph(path, g)
    say("graph_to_device 5000x24 in windows of 333 rows")
    dev = ga.graph_to_device(path, "cuda", chunk_rows=333)
    assert np.array_equal(dev.cpu().numpy().view(np.uint32), g)


def test_pq_codes_stream_into_records(gpu_ctx, tmp_path):
    rng = np.random.default_rng(3)
    codes = rng.integers(0, 256, size=(4000, 16), dtype=np.uint8)
    cent = rng.normal(size=(256, 64)).astype(np.float32)
    ga.write_pq(tmp_path / "p.bin", tmp_path / "c.bin", cent, codes)
    say("pq_codes_to_device 4000x16 into 64-byte records")
    dev = ga.pq_codes_to_device(tmp_path / "c.bin", "cuda", code_stride=64, chunk_rows=999)
    host = dev.cpu().numpy()
    assert np.array_equal(host[:, :16], codes) and not host[:, 16:].any()


def test_exact_search_over_reference_format_index(gpu_ctx, tmp_path):
    wl, li, _ = _world(64, 53, n=4000, nq=24)
    paths = [tmp_path / f for f in ("graph.bin", "meta.bin", "seeds.bin", "labels.spmat")]
    ga.save_label_index(li, *paths)
    ga.write_vectors(tmp_path / "base.u8bin", wl.base.numpy())
    loaded = ga.load_label_index(*paths)
    base = np.asarray(ga.read_vectors(tmp_path / "base.u8bin"))
    rs = gp.plan_queries(loaded, wl.query_labels).graph
    say("exact search over loaded index, routes", rs.count)
    Q, topk = 32, 10
    oi, od, ost = po.exact_search(loaded, rs, None, base, wl.queries.numpy(), queue_limit=Q,
                                  topk=topk, early_stop_mode=2, finish_limit=2,
                                  label_size=loaded.label_size)
    dg = gs.DeviceGraph.upload(loaded)
    # the graph as streamed from graph.bin, not the host copy
    streamed = ga.graph_to_device(paths[0], "cuda", chunk_rows=1000)
    assert torch.equal(streamed.view(-1), dg.graph.view(-1))
    dr = gs.DeviceRoutes.upload(rs)
    dbase = torch.from_numpy(np.array(base)).cuda()
    q = wl.queries.cuda()
    ls = gs.u32(loaded.label_size)
    n = rs.count
    ids = torch.empty(n * topk, dtype=torch.int32, device="cuda")
    dists = torch.empty(n * topk, device="cuda")
    st = torch.zeros(n * 8, dtype=torch.int32, device="cuda")
    gv = dg.view()
    gv.graph = _lib.ptr(streamed)
    prm = _lib.ExactParams(Q, 2, 2, 0, topk, _lib.PLACE_AUTO)
    gpu_ctx.check(gpu_ctx.lib.gofann_exact_search(
        gpu_ctx.handle, _lib.ptr(dbase), _lib.ELEM_U8, base.shape[1], base.shape[0], _lib.ptr(q),
        gv, _lib.ptr(ls), _lib.PredicateView(), dr.routes_view(), prm, _lib.ptr(ids),
        _lib.ptr(dists), _lib.ptr(st)))
    torch.cuda.synchronize()
    assert np.array_equal(ids.cpu().numpy().view(np.uint32).reshape(n, topk), oi)
    assert np.array_equal(dists.cpu().numpy().reshape(n, topk).view(np.uint32), od.view(np.uint32))
    assert np.array_equal(st.cpu().numpy().reshape(n, 8), ost)
