"""GPU parity of the index construction (gofann_build_*, build_kernels.hip):
every primitive against the oracle's restatement (oracle/build_oracle.c) on
the same seeded inputs -- ids, codes and distances bit for bit -- and whole
builds (k-means, PQ codebooks, label graphs of both designs) through
gofann_amd.index with the GPU backend against the same orchestration over
the oracle backend."""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

import pyoracle as po
from gofann_amd import builder as gb
from gofann_amd import index as gi
from gofann_amd import synth

pytestmark = pytest.mark.gpu
U32MAX = 0xFFFFFFFF
ORC = po.OracleBuild()


def say(*a):
    print("[gpu-test]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def hip(gpu_ctx):
    return gb.HipBuild(gpu_ctx)


def _rows(rng, n, dim, dtype):
    if dtype == np.uint8:
        return rng.integers(0, 256, size=(n, dim)).astype(np.uint8)
    x = (rng.standard_normal((n, dim)) * 2).astype(np.float32)
    return x.astype(dtype)


def _u32(t):
    return t.cpu().numpy().view(np.uint32)


DT = [np.uint8, np.float16, np.float32]


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("n,dim,k", [(1000, 40, 37), (300, 192, 64), (130, 7, 1), (2049, 512, 130)])
def test_assign_matches_oracle(hip, dtype, n, dim, k):
    say("assign", dtype.__name__, n, dim, k)
    rng = np.random.default_rng(n + dim + k)
    x = _rows(rng, n, dim, dtype)
    c = (rng.standard_normal((k, dim)) * 2).astype(np.float32)
    if dtype == np.uint8:
        c = (c * 40 + 128).astype(np.float32)
    if k > 3:
        c[3] = c[1]  # a tie: the lower centre
    want, wscore = po.build_assign(x, c)
    got = hip.assign(hip.rows(torch.from_numpy(x)), torch.from_numpy(c))
    assert np.array_equal(_u32(got), want)


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("dim,k", [(24, 8), (192, 32), (100, 64), (512, 128)])
def test_knn_matches_oracle(hip, dtype, dim, k):
    say("knn", dtype.__name__, dim, k)
    rng = np.random.default_rng(dim * 7 + k)
    sizes = [1, 0, 63, 64, 65, 200, 3, 130]
    off = np.concatenate([[0], np.cumsum(sizes)]).astype(np.uint32)
    x = _rows(rng, int(off[-1]), dim, dtype)
    want, wd = po.build_knn(x, off, k)
    got = hip.knn(hip.rows(torch.from_numpy(x)), off, k)
    assert np.array_equal(_u32(got), want)
    # probe lists over several buckets (each list holds its own bucket)
    nb = len(sizes)
    pl = [[b] + [(b + j) % nb for j in (1, 3)] for b in range(nb)]
    po_ = np.concatenate([[0], np.cumsum([len(p) for p in pl])]).astype(np.uint32)
    pb = np.concatenate(pl).astype(np.uint32)
    want2, _ = po.build_knn(x, off, k, po_, pb)
    got2 = hip.knn(hip.rows(torch.from_numpy(x)), off, k, po_, pb)
    assert np.array_equal(_u32(got2), want2)


@pytest.mark.parametrize("dtype", [np.uint8, np.float32])
@pytest.mark.parametrize("dim,pq_dim", [(192, 48), (128, 32), (60, 6), (96, 3)])
def test_pq_encode_and_train_match_oracle(hip, dtype, dim, pq_dim):
    say("pq", dtype.__name__, dim, pq_dim)
    rng = np.random.default_rng(dim + pq_dim)
    x = _rows(rng, 3000, dim, dtype)
    c0 = x[rng.choice(3000, 256, replace=False)].astype(np.float32)
    want = po.build_pq_encode(x, c0, pq_dim)
    xd = hip.rows(torch.from_numpy(x))
    got = hip.pq_encode(xd, torch.from_numpy(c0), pq_dim)
    assert np.array_equal(got.cpu().numpy(), want)
    wc = po.build_pq_train(x, c0, pq_dim, 3)
    gc = hip.pq_train(xd, torch.from_numpy(c0), pq_dim, 3)
    assert np.array_equal(gc.cpu().numpy().view(np.uint32), wc.view(np.uint32))


@pytest.mark.parametrize("dtype", DT)
def test_kmeans_match_oracle(hip, dtype):
    say("kmeans", dtype.__name__)
    rng = np.random.default_rng(17)
    x = _rows(rng, 2500, 48, dtype)
    xd = hip.rows(torch.from_numpy(x))
    for seed in (3, 99):
        want = po.build_kmeanspp(x, 24, seed)
        got = hip.kmeanspp(xd, 24, seed)
        assert np.array_equal(got.cpu().numpy().view(np.uint32), want.view(np.uint32))
    w2 = po.build_kmeans(x, want, 4)
    g2 = hip.kmeans(xd, torch.from_numpy(want), 4)
    assert np.array_equal(g2.cpu().numpy().view(np.uint32), w2.view(np.uint32))


@pytest.mark.parametrize("P", [128, 512, 4096])
def test_rabitq_encode_matches_oracle_on_the_same_rotation(hip, P):
    """The encoder on the GPU's own rotated rows: anchor ids, codes and
    factors equal the oracle's bit for bit; the rotation SGEMM is within
    fp32 rounding of the fp64 product."""
    say("rabitq encode", P)
    rng = np.random.default_rng(P)
    dim = P - 40 if P > 128 else 100
    x = (rng.standard_normal((700, dim))).astype(np.float16)
    rot = gi.random_rotation(dim, P, 9, "cpu")
    cen = rng.standard_normal((33, dim)).astype(np.float32)
    xd = hip.rows(torch.from_numpy(x))
    xr = hip.rotate(xd, rot)
    want_r = x.astype(np.float64) @ rot.numpy().astype(np.float64)
    np.testing.assert_allclose(xr.cpu().numpy(), want_r, rtol=1e-4, atol=1e-4)
    an = hip.rotate(hip.rows(torch.from_numpy(cen)), rot)
    aid, codes, fac = hip.rabitq_encode(xr, an)
    wa, wc, wf = po.build_rabitq_encode(xr.cpu().numpy(), an.cpu().numpy())
    assert np.array_equal(_u32(aid), wa)
    assert np.array_equal(codes.cpu().numpy(), wc)
    assert np.array_equal(fac.cpu().numpy().view(np.uint32), wf.view(np.uint32))


@pytest.mark.parametrize("dtype", DT)
def test_medoid_reps_links_match_oracle(hip, dtype):
    say("medoid / reps / links", dtype.__name__)
    rng = np.random.default_rng(23)
    sizes = [1, 70, 300, 5, 64, 900]
    off = np.concatenate([[0], np.cumsum(sizes)]).astype(np.uint32)
    n = int(off[-1])
    x = _rows(rng, n, 36, dtype)
    xd = hip.rows(torch.from_numpy(x))
    assert hip.medoid(xd) == po.build_medoid(x)
    wm, wr = po.build_bucket_reps(x, off)
    gm, gr = hip.bucket_reps(xd, off)
    assert np.array_equal(_u32(gr), wr)
    assert np.array_equal(gm.cpu().numpy().view(np.uint32), wm.view(np.uint32))
    knn, _ = po.build_knn(x, off, 9)
    bucket_of = np.repeat(np.arange(len(sizes), dtype=np.uint32), sizes)
    near = np.array([[(b + 1) % 6, (b + 2) % 6, (b + 4) % 6] for b in range(6)], np.uint32)
    order = rng.permutation(n).astype(np.uint32)
    for R, local, entry in ((32, 9, 40), (16, 4, None), (64, 0, 3)):
        want = po.build_links(knn, bucket_of, wr, near, order, R, local, 2, min(local, 3), 1,
                              entry, 77)
        got = hip.links(torch.from_numpy(knn.view(np.int32)) if local else None, bucket_of,
                        gr, near, order, R, local, 2, min(local, 3), 1, entry, 77)
        assert np.array_equal(got, want)


@pytest.mark.parametrize("kin,degree", [(64, 32), (128, 64), (20, 9)])
def test_cagra_optimize_and_reach_match_oracle(hip, kin, degree):
    say("cagra optimise", kin, degree)
    rng = np.random.default_rng(kin)
    n = 3000
    x = rng.standard_normal((n, 16)).astype(np.float32)
    off = np.array([0, 1000, 1001, n], np.uint32)
    knn, _ = po.build_knn(x, off, kin)
    wp, wg = po.build_cagra_optimize(knn, degree)
    gp_, gg = hip.cagra_optimize(torch.from_numpy(knn.view(np.int32)), degree)
    assert np.array_equal(_u32(gp_), wp)
    assert np.array_equal(_u32(gg), wg)
    wr, wc = po.build_reach(wg, 5)
    gr, gc = hip.reach(torch.from_numpy(wg.view(np.int32)), 5)
    assert gc == wc and np.array_equal(gr, wr)


@pytest.mark.parametrize("design", ["navigable", "cagra"])
@pytest.mark.parametrize("dtype", ["u8", "f32"])
def test_label_index_build_matches_oracle(gpu_ctx, design, dtype):
    """The whole label-index build (k-means buckets, medoid seeds, graphs of
    either design, connectivity repair) through gofann_amd.index on the GPU
    equals the same orchestration over the oracle backend."""
    say("label index", design, dtype)
    wl = synth.small_labelled(n=5000, nq=4, dim=48, k=12, sigma=0.7, labels=4, seed=29,
                              dtype=dtype, tags=True)
    hip = gb.HipBuild(gpu_ctx)
    cg = gi.train_kmeans(wl.base, 20, iters=6, sample=4000, seed=5, backend=hip)
    co = gi.train_kmeans(wl.base, 20, iters=6, sample=4000, seed=5, backend=ORC)
    assert np.array_equal(cg.cpu().numpy().view(np.uint32), co.numpy().view(np.uint32))
    args = (wl.base, wl.label_offsets, wl.label_values, wl.num_labels)
    lg = gi.build_label_index(*args, cg, degree=32, threshold=300, design=design, backend=hip)
    lo = gi.build_label_index(*args, co, degree=32, threshold=300, design=design, backend=ORC)
    assert np.array_equal(lg.seed_local, lo.seed_local)
    assert np.array_equal(lg.graph, lo.graph)
    assert np.array_equal(lg.rep_row, lo.rep_row)
    tg = gi.train_pq(wl.base, 12, iters=4, sample=3000, backend=hip)
    to = gi.train_pq(wl.base, 12, iters=4, sample=3000, backend=ORC)
    assert np.array_equal(tg.cpu().numpy().view(np.uint32), to.numpy().view(np.uint32))
    assert np.array_equal(gi.pq_encode(wl.base, tg, 12, backend=hip).cpu().numpy(),
                          gi.pq_encode(wl.base, to, 12, backend=ORC).numpy())


def test_grouping_at_larger_sizes_matches_oracle(hip):
    """The build's grouping steps (counts, the one-workgroup scan and the
    per-key row lists) at sizes above a million keys: PQ training over 1.15M
    (row, subspace) pairs, k-means over 70k rows, and the reverse edges of a
    20k-row CAGRA graph; each equal to the oracle."""
    say("grouping at larger sizes")
    rng = np.random.default_rng(99)
    x = rng.integers(0, 256, size=(24000, 192)).astype(np.uint8)
    c0 = x[rng.choice(24000, 256, replace=False)].astype(np.float32)
    wc = po.build_pq_train(x, c0, 48, 2)
    gc = hip.pq_train(hip.rows(torch.from_numpy(x)), torch.from_numpy(c0), 48, 2)
    assert np.array_equal(gc.cpu().numpy().view(np.uint32), wc.view(np.uint32))
    y = (rng.standard_normal((70000, 24)) * 3).astype(np.float32)
    k0 = y[:64].copy()
    wk = po.build_kmeans(y, k0, 2)
    gk = hip.kmeans(hip.rows(torch.from_numpy(y)), torch.from_numpy(k0), 2)
    assert np.array_equal(gk.cpu().numpy().view(np.uint32), wk.view(np.uint32))
    z = rng.standard_normal((20000, 8)).astype(np.float32)
    off = np.array([0, 20000], np.uint32)
    knn = _u32(hip.knn(hip.rows(torch.from_numpy(z)), off, 64))
    wp, wg = po.build_cagra_optimize(knn, 32)
    gp_, gg = hip.cagra_optimize(torch.from_numpy(knn.view(np.int32)), 32)
    assert np.array_equal(_u32(gp_), wp) and np.array_equal(_u32(gg), wg)
