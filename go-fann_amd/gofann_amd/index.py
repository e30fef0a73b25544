"""Offline index construction for the synthetic workloads, on the GPU.

This is the build side the GPU search path consumes; the reference builds it
with cuVS (CAGRA graphs, PQ, IVF-RaBitQ).  Every computation here runs in
the HIP kernels behind gofann_build_* (gofann_amd.builder.HipBuild, the
default backend); this module holds the host orchestration: samples, row
orders, bucket offsets and the connectivity repair.  A backend object
(builder.HipBuild, or the oracle's restatement of the same primitives)
is passed as `backend=`.

Formats follow the reference's in-memory layouts:

  * PQ: centroid table C[256][D] (subspace m owns dims [m*D/M, (m+1)*D/M)),
    codes u8 [N][M] by sample id (backend_pq.cu:1760-1823,
    tools/quantization/pq_builder.cu:92-153).
  * RaBitQ one-bit: rotation R (x_rot = x R), anchors = rotated centroids,
    per-sample anchor id, codes packed MSB-first in u32 words, factors
    (f_add, f_rescale, f_err) (third_party/cuvs_rabitq/.../
    quantizer_gpu_fast.cu:39-101, 180-265).
  * Label-partitioned graphs: one graph per label whose frequency exceeds
    the specificity threshold; rows of group g are global rows
    [label_offset[g], label_offset[g] + label_size[g]) in ascending sample
    order; row_to_sample maps rows to samples; seed = row nearest the
    group mean (src/data/dataloader.cpp:7154-7251, 7361-7406).  Rare labels
    are served by posting lists.

Two graph designs:
  * "navigable" (default, this project's own): exact kNN inside (label,
    cluster) buckets plus links to bucket representatives and uniformly
    drawn links, so a single seed reaches every cluster;
  * "cagra": the reference's recipe (graph_builder.cu:1279-1315): exact kNN
    at 2R over each row's bucket and its nearest buckets, CAGRA's rank-based
    pruning to R and reverse-edge merge, then every row made reachable from
    the seed.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

UINT32_MAX = np.uint32(0xFFFFFFFF)


def _backend(backend):
    if backend is not None:
        return backend
    from .builder import default_backend
    return default_backend()


def _torch(be, a, like=None) -> torch.Tensor:
    """A backend array as a torch tensor on the device of `like` (the
    caller's input) when that is a torch tensor, else where it lies."""
    t = a if isinstance(a, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(be.host(a)))
    if isinstance(like, torch.Tensor) and t.device != like.device:
        t = t.to(like.device)
    return t


def _sample(n: int, m: int, seed: int) -> np.ndarray:
    """`m` distinct rows of `n`, drawn with numpy's PCG64 under `seed`,
    ascending (all rows when m >= n)."""
    if m >= n:
        return np.arange(n, dtype=np.int64)
    return np.sort(np.random.default_rng(seed).choice(n, size=m, replace=False)).astype(np.int64)


# ---------------------------------------------------------------------------
# PQ
# ---------------------------------------------------------------------------
def train_pq(x: torch.Tensor, pq_dim: int, iters: int = 25, sample: int = 65536,
             seed: int = 5, backend=None) -> torch.Tensor:
    """Per-subspace k-means (256 centres) on a row sample, from 256 distinct
    sample rows (gofann_build_pq_train).  Returns C [256][D] float32."""
    be = _backend(backend)
    n, d = x.shape
    assert d % pq_dim == 0
    xb = be.rows(x)
    idx = _sample(n, sample, seed)
    xs = be.take(xb, idx)
    s = len(idx)
    rng = np.random.default_rng(seed + 1)
    init = rng.choice(s, size=256, replace=False) if s >= 256 else np.arange(256) % s
    c0 = be.take(xs, init)
    c0 = c0.float() if isinstance(c0, torch.Tensor) else c0.astype(np.float32)
    return _torch(be, be.pq_train(xs, c0, pq_dim, iters), x)


def pq_encode(x: torch.Tensor, table: torch.Tensor, pq_dim: int, backend=None) -> torch.Tensor:
    """Nearest centre per subspace -> codes u8 [N][M] (gofann_build_pq_encode)."""
    be = _backend(backend)
    return _torch(be, be.pq_encode(be.rows(x), be.dev(table), pq_dim), x)


# ---------------------------------------------------------------------------
# Coarse k-means (graph buckets, RaBitQ anchors)
# ---------------------------------------------------------------------------
def train_kmeans(x: torch.Tensor, k: int, iters: int = 15, sample: int = 262144,
                 seed: int = 6, backend=None) -> torch.Tensor:
    """Seeded k-means over a uniform row sample of the base: k-means++
    seeding (D^2 sampling), then Lloyd iterations; an empty cluster keeps its
    previous centre (gofann_build_kmeanspp, gofann_build_kmeans).  Returns
    [k][D] float32.  The index is built from these trained centres only
    (never from how the data was generated): they bucket the graph builder's
    rows and become the RaBitQ anchors.  Deterministic for a given seed."""
    be = _backend(backend)
    xb = be.rows(x)
    n = x.shape[0]
    idx = _sample(n, max(sample, k), seed)
    xs = be.take(xb, idx)
    k = min(k, len(idx))
    c = be.kmeanspp(xs, k, seed)
    return _torch(be, be.kmeans(xs, c, iters), x)


# ---------------------------------------------------------------------------
# RaBitQ (one bit)
# ---------------------------------------------------------------------------
def random_rotation(dim: int, padded: int, seed: int, device) -> torch.Tensor:
    """Seeded orthogonal [padded][padded] matrix (QR of a Gaussian); the
    rows beyond `dim` multiply zero padding.  Returns R[:dim] as [dim][padded]
    row-major so that x_rot = x R."""
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    a = torch.randn(padded, padded, generator=g, dtype=torch.float64)
    q, r = torch.linalg.qr(a)
    q = q * torch.sign(torch.diagonal(r))[None, :]
    return q[:dim].to(torch.float32).to(device).contiguous()


def rabitq_encode(x: torch.Tensor, rotation: torch.Tensor, centroids: torch.Tensor,
                  chunk: int = 1 << 18, backend=None):
    """Returns (codes u8 [N][P/8], factors f32 [N][3], anchor_ids i32 [N],
    anchors f32 [A][P]).  Anchors = centroids R; each chunk of rows is
    rotated (gofann_build_rotate) and encoded against its nearest anchor
    (gofann_build_rabitq_encode): bit = (x R - c R) > 0, MSB-first in u32
    words, f_add / f_rescale / f_err as quantizer_gpu_fast.cu:200-245."""
    be = _backend(backend)
    xb = be.rows(x)
    n = x.shape[0]
    anchors = be.rotate(be.rows(centroids), rotation)
    parts = []
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        xc = xb[s:e]
        parts.append(be.rabitq_encode(be.rotate(xc, rotation), anchors))
    if isinstance(anchors, torch.Tensor):
        aid = torch.cat([p[0] for p in parts])
        codes = torch.cat([p[1] for p in parts])
        fac = torch.cat([p[2] for p in parts])
        return (_torch(be, codes, x), _torch(be, fac, x), _torch(be, aid, x),
                _torch(be, anchors.contiguous(), x))
    aid = np.concatenate([p[0] for p in parts]).view(np.int32)
    codes = np.concatenate([p[1] for p in parts])
    fac = np.concatenate([p[2] for p in parts])
    return (torch.from_numpy(codes), torch.from_numpy(fac), torch.from_numpy(aid),
            torch.from_numpy(np.ascontiguousarray(anchors)))


# ---------------------------------------------------------------------------
# Label-partitioned graph metadata + graphs
# ---------------------------------------------------------------------------
@dataclass
class LabelIndex:
    num_labels: int
    threshold: int
    cat_freq: np.ndarray        # [L] posting size per label
    label_offset: np.ndarray    # [L] u32 first global row (graph labels)
    label_size: np.ndarray      # [L] u32 rows (0 for posting-only labels)
    row_to_sample: np.ndarray   # [rows] u32
    graph: np.ndarray           # [rows][R] u32 label-local ids
    seed_local: np.ndarray      # [L] u32 (UINT32_MAX when no graph)
    posting_offset: np.ndarray  # [L+1] u64 into posting_ids
    posting_ids: np.ndarray     # u32 sample ids, ascending per label
    csr_offsets: np.ndarray     # [N+1] u32 sample-major labels
    csr_labels: np.ndarray      # u32
    degree: int
    # bucket representatives per graph label (entry points of the
    # nearest-bucket seed mode): CSR over labels of (cluster, local row)
    rep_offset: np.ndarray | None = None
    rep_cluster: np.ndarray | None = None
    rep_row: np.ndarray | None = None
    centres: np.ndarray | None = None

    @property
    def rows(self) -> int:
        return int(self.row_to_sample.shape[0])

    def has_graph(self, label: int) -> bool:
        return int(self.label_size[label]) > 0


def postings_from_csr(offsets: np.ndarray, values: np.ndarray, num_labels: int):
    n = offsets.shape[0] - 1
    counts = np.diff(offsets.astype(np.int64))
    samples = np.repeat(np.arange(n, dtype=np.uint32), counts)
    # by label, then sample: samples are nondecreasing in CSR order, so a
    # stable sort by label alone keeps them ascending within a label
    # (torch's multi-threaded sort; int64 keys hold any uint32 label)
    order = torch.sort(torch.from_numpy(values.astype(np.int64)), stable=True).indices.numpy()
    lab_sorted = values[order]
    post_ids = samples[order].astype(np.uint32)
    cat_freq = np.bincount(lab_sorted.astype(np.int64), minlength=num_labels)
    post_off = np.zeros(num_labels + 1, dtype=np.uint64)
    np.cumsum(cat_freq, out=post_off[1:])
    return cat_freq, post_off, post_ids


def _bucket_order(cl: np.ndarray):
    """Rows of one label group ordered by bucket (stable: ascending row within
    a bucket): the order, the distinct buckets, their row offsets in the
    sorted space and each sorted row's bucket index."""
    order = np.argsort(cl, kind="stable").astype(np.int64)
    uniq, counts = np.unique(cl[order], return_counts=True)
    off = np.zeros(len(uniq) + 1, np.uint32)
    np.cumsum(counts, out=off[1:])
    bucket_of = np.repeat(np.arange(len(uniq), dtype=np.uint32), counts)
    return order, uniq, off, bucket_of


def _u32h(be, a) -> np.ndarray:
    h = be.host(a)
    return h.view(np.uint32) if h.dtype == np.int32 else h.astype(np.uint32)


def _draw_unit(seed: int, stream: int, index: int) -> float:
    """The build's counter-based uniform draw (SplitMix64's finaliser; the
    same function as the device's draw64 in build_kernels.hip)."""
    M = (1 << 64) - 1

    def mix(z):
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
        return z ^ (z >> 31)
    r = mix((mix(seed ^ ((stream * 0xD1B54A32D192ED03) & M)) + index * 0x9E3779B97F4A7C15) & M)
    return (r >> 11) * (1.0 / 9007199254740992.0)


def repair_reach(be, graph: np.ndarray, entry: int, bucket_of: np.ndarray, seed: int,
                 max_rounds: int = 64) -> int:
    """Makes every row reachable from `entry` (the connectivity guarantee of
    the reference's CAGRA build, graph_builder.cu:1295).  Each round walks
    the graph from the entry (gofann_build_reach); in every bucket with
    unreached rows the lowest unreached row becomes a root, and root u gets
    an edge from reached row number floor(d_u * reached) (ascending rows;
    d_u the build's draw (seed, stream 4, round * 2^32 + u)), written into
    that row's last slot not yet used by the repair (at most half its
    slots; a full row passes the edge to the next reached row).  Rounds
    repeat until every row is reached.  Edits `graph` in place; returns the
    number of edges added."""
    n, R = graph.shape
    uses = {}
    added = 0
    for rnd in range(max_rounds):
        reached, cnt = be.reach(graph, entry)
        if cnt >= n:
            return added
        rows_un = np.flatnonzero(~reached)
        _, first = np.unique(bucket_of[rows_un], return_index=True)
        roots = rows_un[first]
        reached_rows = np.flatnonzero(reached)
        for u in roots.tolist():
            k = min(int(_draw_unit(seed, 4, (rnd << 32) + u) * cnt), cnt - 1)
            for _ in range(cnt):
                w = int(reached_rows[k])
                used = uses.get(w, 0)
                if used < R // 2:
                    graph[w, R - 1 - used] = u
                    uses[w] = used + 1
                    added += 1
                    break
                k = (k + 1) % cnt
    reached, cnt = be.reach(graph, entry)
    if cnt < n:
        raise RuntimeError(f"graph repair left {n - cnt} of {n} rows unreachable")
    return added


def build_group_graph(be, xs, order: np.ndarray, uniq: np.ndarray, off: np.ndarray,
                      bucket_of: np.ndarray, centres, degree: int, local: int | None = None,
                      near: int = 2, rep_local: int | None = None, rep_near: int | None = None,
                      seed: int = 0, entry: int | None = None, design: str = "navigable",
                      probe: int = 3):
    """Graph over the rows of one label group.  `xs` holds the group's rows
    sorted by bucket (`order[i]` is the caller row of sorted row i; `off`
    the bucket offsets, `uniq` the bucket ids, `bucket_of` each sorted row's
    bucket index); `entry` is the caller row every route starts from.
    Returns (graph u32 [n][degree] in the caller's row order and ids,
    bucket ids, bucket representatives as caller rows).

    "navigable": a row links to its `local` exact nearest rows inside its
    bucket, its bucket's representative (the row nearest the bucket mean),
    the representatives of the `near` nearest other buckets (by centre
    distance) and uniformly drawn rows up to the degree; a representative
    links to `rep_local` rows of its bucket, the representatives of the
    `rep_near` nearest buckets, and drawn rows; the entry row links to
    `degree` drawn rows.  The drawn links make the graph searchable from
    one entry row when bucket centres are spread without structure (a
    mixture with random centres): distances to the wrong buckets then carry
    no direction towards the right one, so a beam finds a query's bucket
    only by seeing one of its rows, and every expansion that reveals fresh
    buckets brings that closer.

    "cagra": the reference's recipe (build_cagra_graph_chunk,
    graph_builder.cu:1279-1315; graph_degree R, intermediate degree 2R,
    guarantee_connectivity): exact 2R nearest rows over the row's bucket and
    its `probe` - 1 nearest buckets (gofann_build_knn), CAGRA's rank-based
    pruning to R and reverse-edge merge (gofann_build_cagra_optimize), and
    every row made reachable from the entry (repair_reach)."""
    n = len(order)
    R = degree
    nb = len(uniq)
    cen = be.take(be.rows(centres), uniq)
    cen = cen.float() if isinstance(cen, torch.Tensor) else cen.astype(np.float32)
    inv = np.empty(n, np.int64)
    inv[order] = np.arange(n)
    entry_s = int(inv[entry]) if entry is not None else None
    _, reps = be.bucket_reps(xs, off)
    rep_row = order[_u32h(be, reps).astype(np.int64)].astype(np.uint32)
    if design == "cagra":
        kin = min(2 * R, 128)
        p = max(1, min(probe, nb))
        if p > 1:
            near_b = _u32h(be, be.knn(cen, np.array([0, nb], np.uint32), p - 1))
        else:
            near_b = np.zeros((nb, 0), np.uint32)
        plist = np.concatenate([np.arange(nb, dtype=np.uint32)[:, None], near_b], 1)
        probe_off = np.arange(nb + 1, dtype=np.uint32) * p
        knn = be.knn(xs, off, kin, probe_off, plist.reshape(-1))
        _, g = be.cagra_optimize(knn, R)
        g = _u32h(be, g).copy()
        if entry_s is not None:
            repair_reach(be, g, entry_s, bucket_of, seed)
        out = np.full((n, R), UINT32_MAX, np.uint32)
        valid = g < n
        out[order] = np.where(valid, order[np.minimum(g, n - 1)], UINT32_MAX).astype(np.uint32)
        return out, uniq.astype(np.int32), rep_row
    local = local if local is not None else R // 2
    rep_local = rep_local if rep_local is not None else max(R // 8, 1)
    rep_near = rep_near if rep_near is not None else max(R // 8, 1)
    kk = max(local, rep_local)
    knn = be.knn(xs, off, kk) if kk > 0 else None
    m_near = min(max(rep_near, near), max(nb - 1, 0))
    if m_near > 0:
        near_b = be.knn(cen, np.array([0, nb], np.uint32), m_near)
    else:
        near_b = np.zeros((nb, 0), np.uint32)
    graph = be.links(knn, bucket_of, reps, near_b, order.astype(np.uint32), R, local,
                     min(near, m_near), rep_local, min(rep_near, m_near), entry_s, seed)
    return graph, uniq.astype(np.int32), rep_row


def nearest_centre(x: torch.Tensor, centres: torch.Tensor, backend=None) -> np.ndarray:
    """Nearest trained centre of each row (gofann_build_assign), on the host."""
    be = _backend(backend)
    return _u32h(be, be.assign(be.rows(x), be.rows(centres))).astype(np.int64)


def build_label_index(base: torch.Tensor, label_offsets: np.ndarray, label_values: np.ndarray,
                      num_labels: int, centres: torch.Tensor, degree: int,
                      threshold: int = 2000, progress=None,
                      graph_seed: int = 6, local: int | None = None, design: str = "navigable",
                      probe: int = 3, backend=None, near: int = 2) -> LabelIndex:
    """Label-partitioned graphs for labels with more than `threshold` rows,
    built on the GPU (`design` "navigable" or "cagra", see
    build_group_graph).  Rows are bucketed by their nearest trained centre;
    each group's seed is its medoid (gofann_build_medoid).
    `progress(msg)` (optional) is called about every 30 s of building."""
    import time
    be = _backend(backend)
    cat_freq, post_off, post_ids = postings_from_csr(label_offsets, label_values, num_labels)
    graph_labels = np.nonzero(cat_freq > threshold)[0]
    label_size = np.zeros(num_labels, dtype=np.uint32)
    label_size[graph_labels] = cat_freq[graph_labels]
    label_offset = np.zeros(num_labels, dtype=np.uint32)
    total = 0
    for l in range(num_labels):
        label_offset[l] = total
        total += int(label_size[l])
    row_to_sample = np.zeros(total, dtype=np.uint32)
    graph = np.full((total, degree), UINT32_MAX, dtype=np.uint32)
    seed_local = np.full(num_labels, UINT32_MAX, dtype=np.uint32)
    xb = be.rows(base)
    cen = be.rows(centres)
    cluster = nearest_centre(xb, cen, backend=be)
    rep_cluster = [np.zeros(0, np.int32)] * num_labels
    rep_row = [np.zeros(0, np.uint32)] * num_labels
    t_last = time.time()
    for done, l in enumerate(graph_labels):
        if progress is not None and time.time() - t_last > 30.0:
            progress(f"label graphs: {done}/{len(graph_labels)} labels built")
            t_last = time.time()
        s0, s1 = int(post_off[l]), int(post_off[l + 1])
        samples = post_ids[s0:s1].astype(np.int64)
        o = int(label_offset[l])
        row_to_sample[o:o + len(samples)] = samples
        whole = len(samples) == int(base.shape[0])
        # seed: row nearest the group mean (fp64), dataloader.cpp:7361-7406,
        # on the group's rows in their local (ascending sample) order
        xg = xb if whole else be.take(xb, samples)
        seed_local[l] = be.medoid(xg)
        xg = None
        order, uniq, off, bucket_of = _bucket_order(cluster[samples])
        xs = be.take(xb, samples[order])
        graph[o:o + len(samples)], rep_cluster[l], rep_row[l] = build_group_graph(
            be, xs, order, uniq, off, bucket_of, cen, degree, local=local, near=near,
            seed=graph_seed + int(l), entry=int(seed_local[l]), design=design, probe=probe)
        xs = None
    rep_off = np.zeros(num_labels + 1, dtype=np.int64)
    np.cumsum([len(r) for r in rep_row], out=rep_off[1:])
    return LabelIndex(num_labels, threshold, cat_freq, label_offset, label_size, row_to_sample,
                      graph, seed_local, post_off, post_ids,
                      label_offsets.astype(np.uint32), label_values.astype(np.uint32), degree,
                      rep_off, np.concatenate(rep_cluster), np.concatenate(rep_row),
                      be.host(cen).astype(np.float32))
