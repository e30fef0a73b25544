"""Offline index construction for the synthetic workloads (torch, CPU or GPU).

This is the build side the GPU search path consumes; the reference builds it
with cuVS (CAGRA graphs, PQ, IVF-RaBitQ).  Formats follow the reference's
in-memory layouts:

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

The graph builder is this project's own (the reference's CAGRA build is out
of scope): exact kNN inside (label, cluster) buckets plus bridge edges
between bucket representatives, so a single seed reaches every cluster.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

UINT32_MAX = np.uint32(0xFFFFFFFF)


# ---------------------------------------------------------------------------
# PQ
# ---------------------------------------------------------------------------
def train_pq(x: torch.Tensor, pq_dim: int, iters: int = 25, sample: int = 65536,
             seed: int = 5) -> torch.Tensor:
    """Per-subspace k-means (256 centres).  Returns C [256][D] float32."""
    dev = x.device
    n, d = x.shape
    assert d % pq_dim == 0
    sub = d // pq_dim
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    idx = torch.randperm(n, generator=g)[: min(sample, n)].to(dev)
    xs = x[idx].float().reshape(-1, pq_dim, sub).permute(1, 0, 2).contiguous()  # [M, s, sub]
    s = xs.shape[1]
    init = torch.randperm(s, generator=g)[:256].to(dev)
    if s < 256:
        init = torch.arange(256, device=dev) % s
    cen = xs[:, init, :].clone()  # [M, 256, sub]
    for _ in range(iters):
        d2 = (xs * xs).sum(-1, keepdim=True) - 2 * torch.bmm(xs, cen.transpose(1, 2)) + \
            (cen * cen).sum(-1)[:, None, :]
        a = d2.argmin(-1)  # [M, s]
        sums = torch.zeros_like(cen)
        cnt = torch.zeros(pq_dim, 256, device=dev)
        sums.scatter_add_(1, a[..., None].expand(-1, -1, sub), xs)
        cnt.scatter_add_(1, a, torch.ones_like(a, dtype=torch.float32))
        upd = cnt > 0
        cen = torch.where(upd[..., None], sums / cnt.clamp(min=1)[..., None], cen)
    return cen.permute(1, 0, 2).reshape(256, d).contiguous()


def pq_encode(x: torch.Tensor, table: torch.Tensor, pq_dim: int, chunk: int = 1 << 18) -> torch.Tensor:
    """Nearest centre per subspace -> codes u8 [N][M]."""
    n, d = x.shape
    sub = d // pq_dim
    cen = table.reshape(256, pq_dim, sub).permute(1, 0, 2).contiguous()  # [M,256,sub]
    cn = (cen * cen).sum(-1)  # [M,256]
    out = torch.empty(n, pq_dim, dtype=torch.uint8, device=x.device)
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        xs = x[s:e].float().reshape(e - s, pq_dim, sub).permute(1, 0, 2)  # [M,c,sub]
        d2 = cn[:, None, :] - 2 * torch.bmm(xs, cen.transpose(1, 2))
        out[s:e] = d2.argmin(-1).t().to(torch.uint8)
    return out


# ---------------------------------------------------------------------------
# Coarse k-means (graph buckets, RaBitQ anchors)
# ---------------------------------------------------------------------------
def train_kmeans(x: torch.Tensor, k: int, iters: int = 15, sample: int = 262144,
                 seed: int = 6, chunk: int = 1 << 16) -> torch.Tensor:
    """Seeded k-means over a uniform row sample of the base: k-means++
    seeding (D^2 sampling), then Lloyd iterations; an empty cluster keeps its
    previous centre.  Returns [k][D] float32 on x's device.  The index is
    built from these trained centres only (never from how the data was
    generated): they bucket the graph builder's rows and become the RaBitQ
    anchors."""
    dev = x.device
    n, d = x.shape
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    m = min(n, max(sample, k))
    idx = torch.randperm(n, generator=g)[:m].to(dev) if m < n else torch.arange(n, device=dev)
    xs = x[idx].float()
    xn = (xs * xs).sum(1)
    k = min(k, m)
    cen = torch.empty(k, d, dtype=torch.float32, device=dev)
    first = int(torch.randint(m, (1,), generator=g))
    cen[0] = xs[first]
    best = (xn - 2 * xs @ cen[0] + xn[first]).clamp_(min=0)
    u = torch.rand(k, generator=g, dtype=torch.float64).to(dev)
    for j in range(1, k):
        cdf = torch.cumsum(best.double(), 0)
        pick = torch.searchsorted(cdf, (u[j] * cdf[-1]).reshape(1)).clamp_(max=m - 1)
        c = xs[pick[0]]
        cen[j] = c
        dj = (xn - 2 * xs @ c + (c * c).sum()).clamp_(min=0)
        torch.minimum(best, dj, out=best)
    for _ in range(iters):
        cn = (cen * cen).sum(1)
        assign = torch.empty(m, dtype=torch.int64, device=dev)
        for s in range(0, m, chunk):
            assign[s:s + chunk] = (cn[None, :] - 2 * xs[s:s + chunk] @ cen.t()).argmin(1)
        sums = torch.zeros_like(cen).index_add_(0, assign, xs)
        cnt = torch.bincount(assign, minlength=k).float()
        cen = torch.where(cnt[:, None] > 0, sums / cnt.clamp(min=1)[:, None], cen)
    return cen.contiguous()


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
                  chunk: int = 1 << 16):
    """Returns (codes u8 [N][P/8], factors f32 [N][3], anchor_ids u32 [N],
    anchors f32 [A][P]).  Residual r = x R - c R; bit = r > 0 (MSB-first in
    u32 words); f_add = |r|^2 + 2|r|^2 <c,xu>/<r,xu>, f_rescale =
    -2|r|^2/<r,xu> with xu = bit - 0.5 (quantizer_gpu_fast.cu:207-235)."""
    dev = x.device
    n, d = x.shape
    P = rotation.shape[1]
    anchors = centroids.float() @ rotation  # [A, P]
    an = (anchors * anchors).sum(1)
    codes = torch.empty(n, P // 8, dtype=torch.uint8, device=dev)
    factors = torch.empty(n, 3, dtype=torch.float32, device=dev)
    aid = torch.empty(n, dtype=torch.int64, device=dev)
    shifts = (31 - torch.arange(32, device=dev, dtype=torch.int64))
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        xr = x[s:e].float() @ rotation  # [c, P]
        a = ((xr * xr).sum(1, keepdim=True) - 2 * xr @ anchors.t() + an[None, :]).argmin(1)
        aid[s:e] = a
        c = anchors[a]
        r = xr - c
        bits = (r > 0)
        xu = bits.float() - 0.5
        l2 = (r * r).sum(1)
        ip_r = (r * xu).sum(1)
        ip_r = torch.where(ip_r == 0, torch.full_like(ip_r, float("inf")), ip_r)
        ip_c = (c * xu).sum(1)
        xu_sq = (xu * xu).sum(1)
        f_add = l2 + 2.0 * l2 * (ip_c / ip_r)
        f_rescale = -2.0 * l2 / ip_r
        ratio = (l2 * xu_sq) / (ip_r * ip_r)
        inner = torch.clamp((ratio - 1.0) / max(P - 1, 1), min=0.0)
        f_err = 2.0 * torch.sqrt(l2.clamp(min=0)) * 1.9 * torch.sqrt(inner)
        factors[s:e, 0] = f_add
        factors[s:e, 1] = f_rescale
        factors[s:e, 2] = f_err
        w = bits.reshape(e - s, P // 32, 32).to(torch.int64)
        words = (w << shifts).sum(-1)  # [c, P/32] values < 2^32
        le = torch.stack([(words >> (8 * k)) & 0xFF for k in range(4)], dim=-1)
        codes[s:e] = le.reshape(e - s, P // 8).to(torch.uint8)
    return codes, factors, aid.to(torch.int32), anchors.contiguous()


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


def _row_norms(x: torch.Tensor, chunk: int = 1 << 18) -> torch.Tensor:
    """Squared row norms of a large matrix, a chunk of rows at a time."""
    out = torch.empty(x.shape[0], dtype=torch.float32, device=x.device)
    for s0 in range(0, x.shape[0], chunk):
        xs = x[s0:s0 + chunk].float()
        out[s0:s0 + chunk] = (xs * xs).sum(1)
    return out


# Groups above this many bytes of fp32 rows are built without full copies
# (rows gathered per bucket batch, means and distances a chunk at a time).
LEAN_GROUP_BYTES = 8 << 30


def _bucket_knn(xg: torch.Tensor, bucket_of: torch.Tensor, k: int, max_batch_elems: int,
                order: torch.Tensor | None = None):
    """Exact k nearest rows inside each bucket (self excluded).  The rows
    xg[order[i]] (xg[i] without `order`) are sorted by bucket.  Returns int64
    [n, k] ids in that sorted row space, -1 where missing."""
    dev = xg.device
    n = xg.shape[0]
    out = torch.full((n, k), -1, dtype=torch.int64, device=dev)
    if n == 0 or k == 0:
        return out
    uniq, counts = torch.unique_consecutive(bucket_of, return_counts=True)
    starts = torch.zeros_like(counts)
    starts[1:] = torch.cumsum(counts, 0)[:-1]
    counts_h = counts.cpu().numpy()
    starts_h = starts.cpu().numpy()
    i = 0
    if order is None:
        xn = (xg * xg).sum(1)
    else:
        xn = _row_norms(xg)[order]
    border = order
    order = np.argsort(counts_h, kind="stable")
    while i < len(order):
        bm = int(counts_h[order[i]])
        j = i
        # batch buckets of similar size (padding to the batch maximum)
        while j < len(order) and counts_h[order[j]] <= max(bm, 1) * 1.25 + 8 and \
                (j - i + 1) * int(counts_h[order[j]]) ** 2 <= max_batch_elems:
            j += 1
        j = max(j, i + 1)
        sel = order[i:j]
        bmax = int(counts_h[sel].max())
        nb = len(sel)
        st = torch.as_tensor(starts_h[sel], device=dev)
        ct = torch.as_tensor(counts_h[sel], device=dev)
        ar = torch.arange(bmax, device=dev)
        rows = st[:, None] + ar[None, :]  # [nb, bmax]
        valid = ar[None, :] < ct[:, None]
        rows_c = torch.where(valid, rows, torch.zeros_like(rows))
        xb = xg[rows_c] if border is None else xg[border[rows_c]]  # [nb, bmax, D]
        d2 = xn[rows_c][:, :, None] + xn[rows_c][:, None, :] - 2 * torch.bmm(xb, xb.transpose(1, 2))
        big = torch.finfo(d2.dtype).max
        d2 = d2.masked_fill(~valid[:, None, :], big)
        d2 = d2.masked_fill(torch.eye(bmax, dtype=torch.bool, device=dev)[None], big)
        kk = min(k, bmax)
        val, idx = torch.topk(d2, kk, dim=2, largest=False)
        loc = torch.gather(rows_c, 1, idx.reshape(nb, -1)).reshape(nb, bmax, kk)
        loc = torch.where(val < big, loc, torch.full_like(loc, -1))
        dst = rows_c[valid]
        out[dst, :kk] = loc[valid]
        i = j
    return out


def _compact_unique(cand: torch.Tensor, width: int) -> torch.Tensor:
    """First `width` distinct non-negative entries of each row, in their
    original order, padded with -1."""
    n, w = cand.shape
    srt, idx = torch.sort(cand, dim=1, stable=True)
    dup_sorted = torch.zeros_like(srt, dtype=torch.bool)
    dup_sorted[:, 1:] = srt[:, 1:] == srt[:, :-1]
    dup = torch.zeros_like(dup_sorted).scatter_(1, idx, dup_sorted)
    bad = dup | (cand < 0)
    perm = torch.sort(bad.to(torch.int8), dim=1, stable=True).indices
    out = torch.gather(cand, 1, perm)[:, :width]
    out = torch.where(torch.gather(bad, 1, perm)[:, :width], torch.full_like(out, -1), out)
    if out.shape[1] < width:
        out = torch.cat([out, torch.full((n, width - out.shape[1]), -1, dtype=out.dtype,
                                         device=out.device)], 1)
    return out


def build_group_graph(xg: torch.Tensor, cluster_of: torch.Tensor, centres: torch.Tensor,
                      degree: int, local: int | None = None, near: int = 2,
                      rep_local: int | None = None, rep_near: int | None = None, seed: int = 0,
                      max_batch_elems: int = 1 << 27, return_reps: bool = False):
    """Graph over the rows of one label group (rows in the given order).

    Rows are bucketed by their nearest coarse centre; each bucket has a
    representative (the row nearest the bucket mean).  An ordinary row links
    to its `local` exact nearest rows inside its bucket, its bucket's
    representative, the representatives of the `near` nearest other buckets,
    and uniformly drawn rows of the group up to the degree.  A
    representative links to `rep_local` rows of its bucket, the
    representatives of the `rep_near` nearest buckets, and drawn rows.

    The drawn links are what make the graph searchable from one entry row
    when bucket centres are spread without structure (a mixture with random
    centres): distances to the wrong buckets then carry no direction towards
    the right one, so a beam finds a query's bucket only by seeing one of
    its rows, and every expansion that reveals fresh buckets brings that
    closer.  The in-bucket links then let the beam search the bucket, and
    the nearest-bucket links cover clusters that the coarse centres split."""
    dev = xg.device
    n = xg.shape[0]
    R = degree
    local = local if local is not None else R // 2
    rep_local = rep_local if rep_local is not None else max(R // 8, 1)
    rep_near = rep_near if rep_near is not None else max(R // 8, 1)
    lean = n * xg.shape[1] * 4 > LEAN_GROUP_BYTES
    xg = xg.float()
    order = torch.argsort(cluster_of, stable=True)
    bs = cluster_of[order]
    xs = None if lean else xg[order]
    if lean:
        knn = _bucket_knn(xg, bs, local, max_batch_elems, order=order)
    else:
        knn = _bucket_knn(xs, bs, local, max_batch_elems)  # in sorted row space
    uniq, counts = torch.unique_consecutive(bs, return_counts=True)
    nb = uniq.shape[0]
    bucket_idx = torch.repeat_interleave(torch.arange(nb, device=dev), counts)
    # representative: row nearest its bucket mean
    if lean:
        b_orig = torch.searchsorted(uniq, cluster_of)
        sums = torch.zeros(nb, xg.shape[1], device=dev)
        for s0 in range(0, n, 1 << 18):
            sums.index_add_(0, b_orig[s0:s0 + (1 << 18)], xg[s0:s0 + (1 << 18)])
        means = sums / counts[:, None].float()
        dm_o = torch.empty(n, dtype=torch.float32, device=dev)
        for s0 in range(0, n, 1 << 18):
            d = xg[s0:s0 + (1 << 18)] - means[b_orig[s0:s0 + (1 << 18)]]
            dm_o[s0:s0 + (1 << 18)] = (d * d).sum(1)
        dm = dm_o[order]
    else:
        sums = torch.zeros(nb, xs.shape[1], device=dev).index_add_(0, bucket_idx, xs)
        means = sums / counts[:, None].float()
        dm = ((xs - means[bucket_idx]) ** 2).sum(1)
    big = torch.finfo(dm.dtype).max
    for_min = torch.full((nb,), big, device=dev).scatter_reduce(0, bucket_idx, dm, "amin")
    is_min = dm <= for_min[bucket_idx]
    cand = torch.where(is_min, torch.arange(n, device=dev), torch.full_like(bucket_idx, n))
    rep = torch.full((nb,), n, dtype=torch.int64, device=dev).scatter_reduce(0, bucket_idx, cand, "amin")
    # nearest other buckets by coarse-centre distance
    c = centres[uniq].float()
    cd = ((c * c).sum(1)[:, None] + (c * c).sum(1)[None, :] - 2 * c @ c.t())
    cd.fill_diagonal_(float("inf"))
    m_near = min(max(rep_near, near), max(nb - 1, 0))
    nn_b = torch.argsort(cd, dim=1)[:, :m_near]  # [nb, m_near]
    ar = torch.arange(n, device=dev)
    g = torch.Generator(device="cpu")
    g.manual_seed(int(seed))
    out = torch.empty(n, R, dtype=torch.int64, device=dev)
    step = 1 << 20
    for s0 in range(0, n, step):
        s1 = min(n, s0 + step)
        rows = ar[s0:s1]
        b = bucket_idx[s0:s1]
        own = rep[b][:, None]
        own = torch.where(own == rows[:, None], torch.full_like(own, -1), own)
        drawn = torch.randint(0, n, (s1 - s0, R), generator=g).to(dev)
        drawn = torch.where(drawn == rows[:, None], torch.full_like(drawn, -1), drawn)
        cand = torch.cat([knn[s0:s1], own, rep[nn_b[b, :near]], drawn], dim=1)
        out[s0:s1] = _compact_unique(cand, R)
    # representatives: a few in-bucket rows, the nearest buckets' reps, drawn rows
    drawn = torch.randint(0, n, (nb, R), generator=g).to(dev)
    rep_cand = torch.cat([knn[rep, :rep_local], rep[nn_b[:, :rep_near]], drawn], dim=1)
    rep_cand = torch.where(rep_cand == rep[:, None], torch.full_like(rep_cand, -1), rep_cand)
    out[rep] = _compact_unique(rep_cand, R)
    # back to the caller's row order
    # sorted position i is the caller's row order[i]; so are its edge targets
    mapped = torch.where(out >= 0, order[out.clamp(min=0)], torch.full_like(out, -1))
    res = torch.empty_like(mapped)
    res[order] = mapped
    res_np = res.cpu().numpy()
    graph_np = np.where(res_np >= 0, res_np, 0xFFFFFFFF).astype(np.uint32)
    if return_reps:
        # (cluster id, representative row in the caller's order) per bucket
        return graph_np, uniq.cpu().numpy().astype(np.int32), \
            order[rep].cpu().numpy().astype(np.uint32)
    return graph_np


def entry_adjacency(seed_row: int, rows: int, degree: int, seed: int) -> np.ndarray:
    """Adjacency of a group's entry row (its medoid, where every route of the
    group starts): `degree` distinct rows drawn uniformly from the group, so
    that the first expansion already reveals as many buckets as it can."""
    rng = np.random.default_rng(seed)
    m = min(degree, rows - 1)
    pick = rng.choice(rows - 1, size=m, replace=False) if m > 0 else np.zeros(0, np.int64)
    pick = pick + (pick >= seed_row)  # skip the entry row itself
    out = np.full(degree, UINT32_MAX, dtype=np.uint32)
    out[:m] = pick.astype(np.uint32)
    return out


def nearest_centre(x: torch.Tensor, centres: torch.Tensor, chunk: int = 1 << 18) -> torch.Tensor:
    c = centres.float()
    cn = (c * c).sum(1)
    out = torch.empty(x.shape[0], dtype=torch.int64, device=x.device)
    for s in range(0, x.shape[0], chunk):
        e = min(x.shape[0], s + chunk)
        xs = x[s:e].float()
        out[s:e] = (cn[None, :] - 2 * xs @ c.t()).argmin(1)
    return out


def build_label_index(base: torch.Tensor, label_offsets: np.ndarray, label_values: np.ndarray,
                      num_labels: int, centres: torch.Tensor, degree: int,
                      threshold: int = 2000, progress=None,
                      graph_seed: int = 6, local: int | None = None) -> LabelIndex:
    """Label-partitioned graphs for labels with more than `threshold` rows.
    `progress(msg)` (optional) is called about every 30 s of building."""
    import time
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
    cluster = nearest_centre(base, centres)
    rep_cluster = [np.zeros(0, np.int32)] * num_labels
    rep_row = [np.zeros(0, np.uint32)] * num_labels
    t_last = time.time()
    for done, l in enumerate(graph_labels):
        if progress is not None and time.time() - t_last > 30.0:
            progress(f"label graphs: {done}/{len(graph_labels)} labels built")
            t_last = time.time()
        s0, s1 = int(post_off[l]), int(post_off[l + 1])
        samples = post_ids[s0:s1]
        o = int(label_offset[l])
        row_to_sample[o:o + len(samples)] = samples
        sidx = torch.as_tensor(samples.astype(np.int64), device=base.device)
        whole = len(samples) == base.shape[0] and base.dtype == torch.float32
        xg = base if whole else base[sidx].float()  # every row, in order: no copy
        graph[o:o + len(samples)], rep_cluster[l], rep_row[l] = build_group_graph(
            xg, cluster[sidx], centres, degree, local=local, seed=graph_seed + int(l),
            return_reps=True)
        # seed: row nearest the group mean (fp64), dataloader.cpp:7361-7406
        if xg.shape[0] * xg.shape[1] * 4 > LEAN_GROUP_BYTES:
            step = 1 << 16
            mu = torch.zeros(1, xg.shape[1], dtype=torch.float64, device=xg.device)
            for s0 in range(0, xg.shape[0], step):
                mu += xg[s0:s0 + step].double().sum(0, keepdim=True)
            mu /= xg.shape[0]
            dist = torch.empty(xg.shape[0], dtype=torch.float64, device=xg.device)
            for s0 in range(0, xg.shape[0], step):
                dist[s0:s0 + step] = ((xg[s0:s0 + step].double() - mu) ** 2).sum(1)
            seed_local[l] = int(dist.argmin())
        else:
            xd = xg.double()
            mu = xd.mean(0, keepdim=True)
            seed_local[l] = int(((xd - mu) ** 2).sum(1).argmin())
        # the entry row's adjacency fans out over the navigation layer
        sl = int(seed_local[l])
        graph[o + sl] = entry_adjacency(sl, len(samples), degree, graph_seed + 7919 * int(l))
    rep_off = np.zeros(num_labels + 1, dtype=np.int64)
    np.cumsum([len(r) for r in rep_row], out=rep_off[1:])
    return LabelIndex(num_labels, threshold, cat_freq, label_offset, label_size, row_to_sample,
                      graph, seed_local, post_off, post_ids,
                      label_offsets.astype(np.uint32), label_values.astype(np.uint32), degree,
                      rep_off, np.concatenate(rep_cluster), np.concatenate(rep_row),
                      centres.detach().float().cpu().numpy())
