"""Seeded synthetic workloads of the BASELINE configurations.

Seeds follow the convention seed = 1000 * cfg + role (1 centroids, 2 points,
3 attributes, 4 queries, 5 quantizer / rotation, 6 graph).  Generation runs
in torch on the requested device (the GPU for full-size configs, the CPU for
test-size ones); the returned arrays live on that device.

Attribute models:
  * labels:  one categorical label per vector (uniform or Zipf)
  * tags:    1..5 distinct tags per vector drawn Zipf(s) from a vocabulary
  * ranges:  numeric attribute(s) per vector
Query filters are conjunctions of labels/tags plus optional half-open ranges.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    return g


@dataclass
class Workload:
    name: str
    base: torch.Tensor            # [N, D] uint8 / float32 / float16
    queries: torch.Tensor         # [Q, D] same element type (f32 queries for f16 base)
    cluster_of: torch.Tensor      # [N] int64 generating mixture component
    centroids: torch.Tensor       # [K, D] float32 mixture centres
    label_offsets: np.ndarray     # CSR over samples, uint32 [N+1]
    label_values: np.ndarray      # uint32, strictly increasing per row
    num_labels: int
    query_labels: list            # per query: list of required labels (AND)
    base_ranges: np.ndarray | None = None      # [N, range_count] float32
    query_ranges: list | None = None           # per query: list of (dim, mode, lo, hi)
    meta: dict = field(default_factory=dict)

    @property
    def n(self) -> int:
        return int(self.base.shape[0])

    @property
    def dim(self) -> int:
        return int(self.base.shape[1])


def gaussian_mixture(n: int, dim: int, k: int, sigma: float, seed_base: int, device,
                     centre_scale: float = 1.0, centre_offset: float = 0.0,
                     chunk: int = 1 << 20):
    """Points = centre[c] + N(0, sigma^2), c uniform over k centres."""
    gc = _gen(seed_base + 1, device)
    centres = torch.randn(k, dim, generator=gc, device=device) * centre_scale + centre_offset
    gp = _gen(seed_base + 2, device)
    cluster = torch.randint(0, k, (n,), generator=gp, device=device)
    out = torch.empty(n, dim, dtype=torch.float32, device=device)
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        out[s:e] = centres[cluster[s:e]] + sigma * torch.randn(e - s, dim, generator=gp, device=device)
    return out, cluster, centres


def _zipf_probs(vocab: int, s: float) -> np.ndarray:
    w = 1.0 / np.arange(1, vocab + 1, dtype=np.float64) ** s
    return w / w.sum()


def zipf_tags(n: int, vocab: int, s: float, min_tags: int, max_tags: int, seed: int):
    """1..k distinct tags per row, Zipf-distributed; CSR (offsets, values)."""
    rng = np.random.default_rng(seed)
    probs = _zipf_probs(vocab, s)
    counts = rng.integers(min_tags, max_tags + 1, size=n)
    # draw extra candidates so rows keep `count` distinct tags in draw order
    extra = 2 * max_tags
    draws = rng.choice(vocab, size=(n, extra), p=probs)
    seen_before = np.zeros_like(draws, dtype=bool)
    for j in range(1, extra):
        seen_before[:, j] = (draws[:, :j] == draws[:, j:j + 1]).any(axis=1)
    fresh = ~seen_before
    rank = np.cumsum(fresh, axis=1)
    keep = fresh & (rank <= counts[:, None])
    rows = np.where(keep, draws, vocab)
    rows = np.sort(rows, axis=1)                           # CSR rows are sorted
    valid = rows < vocab
    nnz = valid.sum(axis=1)
    offsets = np.zeros(n + 1, dtype=np.uint64)
    np.cumsum(nnz, out=offsets[1:])
    values = rows[valid].astype(np.uint32)
    return offsets.astype(np.uint32), values


def categorical_labels(n: int, vocab: int, seed: int, zipf_s: float | None = None):
    rng = np.random.default_rng(seed)
    if zipf_s is None:
        lab = rng.integers(0, vocab, size=n)
    else:
        lab = rng.choice(vocab, size=n, p=_zipf_probs(vocab, zipf_s))
    offsets = np.arange(n + 1, dtype=np.uint32)
    return offsets, lab.astype(np.uint32)


def label_frequencies(offsets: np.ndarray, values: np.ndarray, vocab: int) -> np.ndarray:
    return np.bincount(values.astype(np.int64), minlength=vocab)


def config1(n=1_000_000, nq=10_000, device="cpu", dim=128, k=256, sigma=0.3, labels=10):
    """C1: fp32 mixture, one uniform label of 10, single-label equality queries."""
    cfg = 1000
    x, cl, cen = gaussian_mixture(n, dim, k, sigma, cfg, device)
    gq = _gen(cfg + 4, device)
    qc = torch.randint(0, k, (nq,), generator=gq, device=device)
    q = cen[qc] + sigma * torch.randn(nq, dim, generator=gq, device=device)
    lo, lv = categorical_labels(n, labels, cfg + 3)
    rng = np.random.default_rng(cfg + 4)
    ql = [[int(v)] for v in rng.integers(0, labels, size=nq)]
    return Workload("C1", x, q, cl, cen, lo, lv, labels, ql,
                    meta=dict(config=1, sigma=sigma, clusters=k))


def config2(n=10_000_000, nq=100_000, device="cpu", dim=192, k=1024, sigma=16.0,
            vocab=2000, zipf_s=1.1, sel_lo=0.001, sel_hi=0.20):
    """C2: uint8 mixture (clipped), 1-5 Zipf tags, AND of 1-2 tags per query
    with estimated selectivity in [sel_lo, sel_hi]."""
    cfg = 2000
    # centres uniform in [32, 224] per dimension, points clipped to 0..255
    gc = _gen(cfg + 1, device)
    cen = 32.0 + 192.0 * torch.rand(k, dim, generator=gc, device=device)
    gp = _gen(cfg + 2, device)
    cl = torch.randint(0, k, (n,), generator=gp, device=device)
    chunk = 1 << 20
    base = torch.empty(n, dim, dtype=torch.uint8, device=device)
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        v = cen[cl[s:e]] + sigma * torch.randn(e - s, dim, generator=gp, device=device)
        base[s:e] = v.round_().clamp_(0, 255).to(torch.uint8)
    gq = _gen(cfg + 4, device)
    qc = torch.randint(0, k, (nq,), generator=gq, device=device)
    q = (cen[qc] + sigma * torch.randn(nq, dim, generator=gq, device=device)).round_().clamp_(0, 255)
    q = q.to(torch.uint8)
    lo, lv = zipf_tags(n, vocab, zipf_s, 1, 5, cfg + 3)
    freq = label_frequencies(lo, lv, vocab) / float(n)
    rng = np.random.default_rng(cfg + 4)
    probs = _zipf_probs(vocab, zipf_s)
    ql = []
    while len(ql) < nq:
        m = int(rng.integers(1, 3))
        tags = rng.choice(vocab, size=m, p=probs)
        if m == 2 and tags[0] == tags[1]:
            continue
        sel = float(np.prod(freq[tags]))
        if sel_lo <= sel <= sel_hi:
            ql.append(sorted(int(t) for t in tags))
    return Workload("C2", base, q, cl, cen, lo, lv, vocab, ql,
                    meta=dict(config=2, sigma=sigma, clusters=k))


def small_labelled(n=4096, nq=64, dim=32, k=16, sigma=0.6, labels=6, seed=77, device="cpu",
                   dtype="f32", tags=False, ranges=False):
    """Test-size workload: overlapping mixture so per-label kNN graphs are
    navigable; optional tags (AND of 1-2) and one numeric range attribute."""
    cfg = seed * 1000
    x, cl, cen = gaussian_mixture(n, dim, k, sigma, cfg, device)
    gq = _gen(cfg + 4, device)
    qc = torch.randint(0, k, (nq,), generator=gq, device=device)
    q = cen[qc] + sigma * torch.randn(nq, dim, generator=gq, device=device)
    if dtype == "u8":
        lo_, hi_ = float(x.min()), float(x.max())
        sc = 255.0 / (hi_ - lo_)
        x = ((x - lo_) * sc).round().clamp(0, 255).to(torch.uint8)
        q = ((q - lo_) * sc).round().clamp(0, 255).to(torch.uint8)
        cen = (cen - lo_) * sc
    rng = np.random.default_rng(cfg + 3)
    if tags:
        lo, lv = zipf_tags(n, labels, 0.7, 1, 3, cfg + 3)
        ql = []
        for _ in range(nq):
            m = int(rng.integers(1, 3))
            ql.append(sorted(set(int(t) for t in rng.integers(0, labels, size=m))))
    else:
        lo, lv = categorical_labels(n, labels, cfg + 3)
        ql = [[int(v)] for v in rng.integers(0, labels, size=nq)]
    base_ranges = None
    query_ranges = None
    if ranges:
        base_ranges = rng.integers(0, 1000, size=(n, 1)).astype(np.float32)
        query_ranges = []
        for _ in range(nq):
            lo_v = float(rng.integers(0, 800))
            query_ranges.append([(0, 3, lo_v, lo_v + float(rng.integers(100, 400)))])
    return Workload("small", x, q, cl, cen, lo, lv, labels, ql, base_ranges, query_ranges,
                    meta=dict(sigma=sigma, clusters=k))


def config3(n=2_700_000, nq=10_000, device="cuda", dim=4096, k=512, rank=64, spread=0.7,
            noise=0.05, selectivities=(0.005, 0.05, 0.5), attr_range=10_000, seed=3,
            chunk=1 << 17):
    """C3: unit-normalised vectors from a k-centre mixture in `dim`
    dimensions and one int32 attribute uniform in [0, attr_range).  A point
    is centre + U z + e, normalised: U a shared random [rank][dim] basis
    (so the data has low intrinsic dimension and meaningful nearest
    neighbours), z ~ N(0, spread^2 |c|^2 / rank) per coordinate so that |U z|
    is about spread |c|, e ~ N(0, noise^2).  Queries come from the same
    mixture; query i carries the range [lo, lo + w) of the attribute with
    w = selectivities[i % len] * attr_range and lo uniform (mode 3)."""
    cfg = seed * 1000
    gc = _gen(cfg + 1, device)
    centres = torch.randn(k, dim, generator=gc, device=device)
    basis = torch.randn(rank, dim, generator=gc, device=device)
    zscale = spread / rank ** 0.5  # |U z| ~ spread * sqrt(dim) ~ spread * |c|

    def draw(m, g):
        cl = torch.randint(0, k, (m,), generator=g, device=device)
        out = torch.empty(m, dim, dtype=torch.float32, device=device)
        for s in range(0, m, chunk):
            e = min(m, s + chunk)
            z = torch.randn(e - s, rank, generator=g, device=device) * zscale
            x = centres[cl[s:e]] + z @ basis + noise * torch.randn(e - s, dim, generator=g,
                                                                   device=device)
            out[s:e] = x / x.norm(dim=1, keepdim=True)
        return out, cl

    base, cl = draw(n, _gen(cfg + 2, device))
    queries, _ = draw(nq, _gen(cfg + 4, device))
    rng = np.random.default_rng(cfg + 3)
    attr = rng.integers(0, attr_range, size=n).astype(np.float32)
    sel = np.array([selectivities[i % len(selectivities)] for i in range(nq)], dtype=np.float64)
    width = np.maximum(1, np.round(sel * attr_range)).astype(np.int64)
    lo = (rng.random(nq) * (attr_range - width + 1)).astype(np.int64)
    query_ranges = [[(0, 3, float(lo[i]), float(lo[i] + width[i]))] for i in range(nq)]
    cn = centres / centres.norm(dim=1, keepdim=True)
    wl = Workload("config3", base, queries, cl, cn,
                  np.arange(n + 1, dtype=np.uint32), np.zeros(n, dtype=np.uint32), 1,
                  [[0] for _ in range(nq)], attr[:, None].copy(), query_ranges,
                  meta=dict(selectivity=sel, spread=spread, rank=rank, noise=noise))
    return wl


def config4(n=100_000_000, nq=10_000, device="cuda", dim=512, k=4096, rank=64, spread=0.7,
            noise=0.05, labels=1000, zipf_s=1.1, attr_max=1 << 24, intervals=100,
            sel_lo=0.01, sel_hi=0.10, seed=4, chunk=1 << 17):
    """C4: fp16 vectors from a k-centre mixture (the config3 model: centre +
    shared rank-`rank` spread + noise, normalised), one categorical label
    Zipf(zipf_s) over `labels` values and one uint32 attribute uniform in
    [0, attr_max) (attr_max <= 2^24, so float32 holds it exactly).

    Every row also carries an interval label: labels + floor(attr *
    intervals / attr_max), the attribute's bucket among `intervals` equal
    ones, so that a range query can run as one graph route per interval it
    overlaps with the range as residual predicate (the hybrid label +
    interval graphs of the reference's RaBitQ benchmark).  Row labels are
    [category, labels + interval].

    Even queries are categorical equality (label drawn from the same Zipf);
    odd queries are ranges [lo, lo + w) with w = U(sel_lo, sel_hi) *
    attr_max (mode 3).  query_labels holds [label] for equality queries and
    [] for range queries."""
    if attr_max > 1 << 24:
        raise ValueError("attr_max above 2^24 is not exact in float32")
    cfg = seed * 1000
    gc = _gen(cfg + 1, device)
    centres = torch.randn(k, dim, generator=gc, device=device)
    basis = torch.randn(rank, dim, generator=gc, device=device)
    zscale = spread / rank ** 0.5

    def draw(m, g, dtype):
        cl = torch.randint(0, k, (m,), generator=g, device=device)
        out = torch.empty(m, dim, dtype=dtype, device=device)
        for s in range(0, m, chunk):
            e = min(m, s + chunk)
            z = torch.randn(e - s, rank, generator=g, device=device) * zscale
            x = centres[cl[s:e]] + z @ basis + noise * torch.randn(e - s, dim, generator=g,
                                                                   device=device)
            out[s:e] = (x / x.norm(dim=1, keepdim=True)).to(dtype)
        return out, cl

    base, cl = draw(n, _gen(cfg + 2, device), torch.float16)
    queries, _ = draw(nq, _gen(cfg + 4, device), torch.float32)
    rng = np.random.default_rng(cfg + 3)
    probs = _zipf_probs(labels, zipf_s)
    cat = rng.choice(labels, size=n, p=probs).astype(np.uint32)
    attr = rng.integers(0, attr_max, size=n, dtype=np.int64)
    interval = (attr * intervals // attr_max).astype(np.uint32)
    lv = np.empty(2 * n, dtype=np.uint32)
    lv[0::2] = cat
    lv[1::2] = labels + interval
    lo_off = np.arange(0, 2 * n + 1, 2, dtype=np.uint64)
    if lo_off[-1] < 1 << 32:
        lo_off = lo_off.astype(np.uint32)
    qrng = np.random.default_rng(cfg + 5)
    qcat = qrng.choice(labels, size=nq, p=probs)
    sel = qrng.uniform(sel_lo, sel_hi, size=nq)
    width = np.maximum(1, np.round(sel * attr_max)).astype(np.int64)
    qlo = (qrng.random(nq) * (attr_max - width + 1)).astype(np.int64)
    query_labels, query_ranges = [], []
    for i in range(nq):
        if i % 2 == 0:
            query_labels.append([int(qcat[i])])
            query_ranges.append([])
        else:
            query_labels.append([])
            query_ranges.append([(0, 3, float(qlo[i]), float(qlo[i] + width[i]))])
    cn = centres / centres.norm(dim=1, keepdim=True)
    return Workload("config4", base, queries, cl, cn, lo_off, lv, labels + intervals,
                    query_labels, attr.astype(np.float32)[:, None], query_ranges,
                    meta=dict(selectivity=np.where(np.arange(nq) % 2 == 1, width / attr_max, 0.0),
                              row_category=cat,
                              categories=labels, intervals=intervals, attr_max=attr_max,
                              zipf_s=zipf_s, spread=spread, rank=rank, noise=noise))


QUERY_TYPES_C5 = ("exact", "fuzzy", "hybrid_exact", "hybrid_fuzzy")


def config5(n=100_000_000, nq=10_000, device="cuda", vocab=50_000, zipf_strings=1.0,
            min_score=0.6, fuzzy_edits=1, seed=5, **c4_kw):
    """C5: the C4 set plus a string attribute per vector and string filters.

    Vectors, categories and the uint32 attribute are config4's.  The string
    attribute takes one of `vocab` distinct 8..32-character strings from a
    seeded order-2 character Markov chain (strings.markov_strings), reused
    Zipf(zipf_strings) over a random rank order.  Each distinct string is a
    token label: label categories + intervals + string id.  Row labels are
    [category, categories + interval, token].

    Query q has type QUERY_TYPES_C5[q % 4] and a filter in disjunctive
    normal form (meta["query_clauses"][q]: list of (labels, uses_range)):
      * exact: the token of a string drawn by row frequency;
      * fuzzy: a string drawn by row frequency with `fuzzy_edits` character
        substitutions, expanded by the 3-gram index to the tokens whose
        3-gram Jaccard score is >= min_score; one clause per token;
      * hybrid_exact: category AND range AND token, all taken from a random
        row (so the filter matches at least that row), the range [lo, lo+w)
        with w uniform in 1-10% of the attribute domain around the row's
        value;
      * hybrid_fuzzy: as hybrid_exact with the row's string fuzzed and
        expanded: one clause (category, token) with the range per token.
    A fuzzy pattern that expands to no token is drawn again."""
    from . import strings as st
    wl = config4(n=n, nq=nq, device=device, **c4_kw)
    cats, nint, amax = wl.meta["categories"], wl.meta["intervals"], wl.meta["attr_max"]
    base_label = cats + nint
    texts = st.markov_strings(vocab, 1000 * seed + 7)
    index = st.NgramIndex(texts)
    rng = np.random.default_rng(1000 * seed + 8)
    probs = _zipf_probs(vocab, zipf_strings)
    rank_to_sid = rng.permutation(vocab)
    sid = rank_to_sid[rng.choice(vocab, size=n, p=probs)].astype(np.uint32)
    lv = np.empty(3 * n, dtype=np.uint32)
    lv[0::3] = wl.label_values[0::2]
    lv[1::3] = wl.label_values[1::2]
    lv[2::3] = base_label + sid
    lo_off = np.arange(0, 3 * n + 1, 3, dtype=np.uint64)
    if lo_off[-1] < 1 << 32:
        lo_off = lo_off.astype(np.uint32)
    cat = wl.label_values[0::2]
    attr = wl.base_ranges[:, 0]
    qrng = np.random.default_rng(1000 * seed + 9)
    clauses, ranges, qtypes, patterns = [], [], [], []
    for i in range(nq):
        kind = QUERY_TYPES_C5[i % 4]
        qtypes.append(kind)
        if kind in ("exact", "fuzzy"):
            while True:
                s = int(rank_to_sid[qrng.choice(vocab, p=probs)])
                if kind == "exact":
                    toks, pat = [s], texts[s]
                else:
                    pat = st.mutate(texts[s], qrng, fuzzy_edits)
                    toks = index.expand(pat, min_score).tolist()
                if toks:
                    break
            clauses.append([([base_label + t], False) for t in toks])
            ranges.append([])
            patterns.append(pat)
            continue
        while True:
            r = int(qrng.integers(0, n))
            s = int(sid[r])
            if kind == "hybrid_exact":
                toks, pat = [s], texts[s]
            else:
                pat = st.mutate(texts[s], qrng, fuzzy_edits)
                toks = index.expand(pat, min_score).tolist()
            if toks:
                break
        w = int(max(1, round(qrng.uniform(0.01, 0.10) * amax)))
        a = int(attr[r])
        lo = int(qrng.integers(max(0, a - w + 1), min(a, amax - w) + 1))
        c = int(cat[r])
        clauses.append([(sorted([c, base_label + t]), True) for t in toks])
        ranges.append([(0, 3, float(lo), float(lo + w))])
        patterns.append(pat)
    meta = dict(wl.meta)
    meta.update(c4_query_labels=wl.query_labels, c4_query_ranges=wl.query_ranges,
                strings=texts, string_label_base=base_label, string_ids=sid,
                query_clauses=clauses, query_types=qtypes, patterns=patterns,
                min_score=min_score, ngram_index=index)
    return Workload("config5", wl.base, wl.queries, wl.cluster_of, wl.centroids, lo_off, lv,
                    base_label + vocab, [[] for _ in range(nq)], wl.base_ranges, ranges,
                    meta=meta)


def c4_view(wl5: Workload) -> Workload:
    """The C4 workload over a C5 world: the same vectors, categories and
    attribute (a superset of C4's labels), with C4's query filters."""
    meta = {k: v for k, v in wl5.meta.items()
            if k not in ("query_clauses", "query_types", "patterns")}
    return Workload("config4", wl5.base, wl5.queries, wl5.cluster_of, wl5.centroids,
                    wl5.label_offsets, wl5.label_values, wl5.num_labels,
                    wl5.meta["c4_query_labels"], wl5.base_ranges, wl5.meta["c4_query_ranges"],
                    meta=meta)
