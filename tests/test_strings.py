"""String predicates (C5): token normalisation and n-grams, the n-gram
expansion of fuzzy patterns against brute-force 3-gram Jaccard, the DNF
route planner on category AND range AND string filters, and a small C5 world
searched end to end through the oracle (every returned row satisfies its
query's filter; recall against exact filtered ground truth)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import pyoracle as po
from gofann_amd import index as gi
from gofann_amd import plan as gp
from gofann_amd import strings as st
from gofann_amd import synth

# the index is built by the oracle's restatement of the GPU build (no GPU here)
CPU_BUILD = po.OracleBuild()

U32MAX = 0xFFFFFFFF


def test_normalize_rules():
    # normalize_manifest_token_text (dataloader.cpp:2973-2991)
    assert st.normalize("Hello, World!!") == "hello world"
    assert st.normalize("  --Ab9__cD  ") == "ab9 cd"
    assert st.normalize("") == ""
    assert st.normalize("!!!") == ""
    assert st.normalize("a  b\tc") == "a b c"
    assert st.normalize("café") == "caf"  # non-ASCII bytes are separators


def test_ngram_rules():
    # token_ngrams (dataloader.cpp:2993-3011): sorted distinct; short text whole
    assert st.ngrams("abcd", 3) == ["abc", "bcd"]
    assert st.ngrams("abab", 2) == ["ab", "ba"]
    assert st.ngrams("ab", 3) == ["ab"]
    assert st.ngrams("abc", 3) == ["abc"]
    assert st.ngrams("", 3) == []
    assert st.ngrams("aaaa", 3) == ["aaa"]


def _jaccard_brute(pattern, tokens, n):
    p = set(st.ngrams(st.normalize(pattern), n))
    out = []
    for t, text in enumerate(tokens):
        g = set(st.ngrams(st.normalize(text), n))
        inter = len(p & g)
        if inter == 0:
            continue
        union = len(p | g)
        out.append((t, np.float32(inter) / np.float32(union)))
    return out


@pytest.mark.parametrize("n,min_score", [(3, 0.6), (3, 0.25), (2, 0.5)])
def test_expand_matches_brute_force_jaccard(n, min_score):
    rng = np.random.default_rng(n * 100 + int(min_score * 10))
    vocab = st.markov_strings(3000, 11)
    vocab += ["ab", "abc", "Mixed Case-Token", "x"]
    ix = st.NgramIndex(vocab, n)
    pats = [st.mutate(vocab[int(rng.integers(0, len(vocab)))], rng, int(rng.integers(0, 3)))
            for _ in range(150)] + ["ab", "ABC!", "mixed case token", "zz", ""]
    for pat in pats:
        got = ix.expand(pat, min_score, max_terms=1 << 30).tolist()
        want = sorted(t for t, sc in _jaccard_brute(pat, vocab, n) if sc >= np.float32(min_score))
        assert got == want, pat


def _capped_brute(pattern, tokens, n, min_score, mode, max_terms):
    """ManifestNgramIndex::expand's selection restated by brute force
    (dataloader.cpp:3700-3786): every token sharing a gram with the pattern,
    kept if a direct match (ranked as max(1, score)) or if score >=
    min_score; sorted direct first, score descending, token id ascending;
    the first max_terms, returned ascending."""
    norm = st.normalize(pattern)
    cands = []
    for t, sc in _jaccard_brute(pattern, tokens, n):
        text = st.normalize(tokens[t])
        direct = (mode == "prefix" and text.startswith(norm)) or \
                 (mode == "suffix" and text.endswith(norm)) or \
                 (mode in ("contains", "substring") and norm in text)
        if not direct and sc < np.float32(min_score):
            continue
        cands.append((t, max(np.float32(1), sc) if direct else sc, direct))
    cands.sort(key=lambda c: (not c[2], -float(c[1]), c[0]))
    return sorted(c[0] for c in cands[:max_terms])


@pytest.mark.parametrize("mode", ["", "contains", "prefix"])
def test_expand_caps_terms_by_reference_ranking(mode):
    """A pattern that matches more than max_terms tokens keeps the
    reference's top max_terms (query_manifest_max_fuzzy_terms, 64 by
    default): direct matches first, then the highest scores, ties by the
    lower token id.  The vocabulary holds many tokens of equal score, so a
    wrong tie order or a missing cap changes the returned set."""
    rng = np.random.default_rng(71)
    stem = "abcdefgh"
    vocab = [stem + "".join(rng.choice(list("xyz"), 3)) for _ in range(300)]
    vocab += ["".join(rng.choice(list("xyz"), 3)) + stem for _ in range(100)]
    vocab += [stem, stem[:6] + "qq", "zz" + stem[2:]]
    vocab += st.markov_strings(500, 5)
    ix = st.NgramIndex(vocab, 3)
    for pat, ms in ((stem, 0.25), (stem + "x", 0.3), ("bcdefg", 0.2)):
        full = ix.expand(pat, ms, mode, max_terms=1 << 30)
        assert len(full) > 64, (pat, len(full))
        for cap in (64, 7, 1):
            got = ix.expand(pat, ms, mode, max_terms=cap).tolist()
            assert got == _capped_brute(pat, vocab, 3, ms, mode, cap), (pat, mode, cap)
        assert ix.expand(pat, ms, mode).tolist() == _capped_brute(pat, vocab, 3, ms, mode, 64)
    with pytest.raises(ValueError):
        ix.expand(stem, 0.25, mode, max_terms=0)


def test_expand_direct_modes():
    vocab = ["prefixmatch", "matchsuffix", "xxmatchxx", "unrelated", "mat"]
    ix = st.NgramIndex(vocab, 3)
    assert 0 in ix.expand("prefix", 0.99, "prefix").tolist()
    assert 1 in ix.expand("suffix", 0.99, "suffix").tolist()
    got = ix.expand("match", 0.99, "contains").tolist()
    assert {0, 1, 2} <= set(got) and 3 not in got
    assert ix.expand("match", 0.99).tolist() == []


def test_markov_strings_shape():
    v = st.markov_strings(5000, 3)
    assert len(v) == len(set(v)) == 5000
    assert all(8 <= len(s) <= 32 and s.isalpha() and s.islower() for s in v)
    assert v == st.markov_strings(5000, 3)  # seeded


def test_clause_anchor_rules():
    """prepare_query_route_chunk / plan_hybrid_clause_routes route choice."""
    class Ix:
        cat_freq = np.array([0, 50, 5000, 8000, 20, 9000, 100000])
        label_size = np.array([0, 0, 5000, 8000, 0, 9000, 100000])

        def has_graph(self, l):
            return self.label_size[l] > 0
    ix = Ix()
    assert gp.clause_anchors(ix, [2]) == ("graph", [2])
    assert gp.clause_anchors(ix, [2, 1, 4]) == ("posting", [4])  # rarest posting label
    assert gp.clause_anchors(ix, [3, 2]) == ("graph", [2, 3])  # dual, smaller first
    assert gp.clause_anchors(ix, [3, 2], dual_ratio=1.2) == ("graph", [2])
    assert gp.clause_anchors(ix, [5, 3, 6]) == ("graph", [3])  # least posting
    assert gp.clause_anchors(ix, [0]) == ("none", [])
    assert gp.clause_anchors(ix, [0, 2]) == ("graph", [2])


def test_plan_dnf_residuals():
    class Ix:
        cat_freq = np.array([10, 5000, 6000, 30])
        label_size = np.array([0, 5000, 6000, 0])
        seed_local = np.array([U32MAX, 0, 0, U32MAX], np.uint32)
        posting_offset = np.array([0, 10, 5010, 11010, 11040], np.uint64)

        def has_graph(self, l):
            return self.label_size[l] > 0
    rng = [(0, 3, 5.0, 9.0)]
    clauses = [[([1, 3], True), ([1, 2], True)], [([2], False)]]
    pl = gp.plan_dnf(Ix(), clauses, [rng, []], sort_by_group=False)
    # query 0 clause 0: posting over label 3, residual {1} + range;
    # clause 1: dual graph routes on 1 and 2, residual the other + range;
    # query 1: graph route on 2, entailed
    assert pl.posting.route_group.tolist() == [3]
    assert pl.graph.route_group.tolist() == [1, 2, 2]
    assert pl.graph.route_query.tolist() == [0, 0, 1]
    pr = pl.posting.predicate
    c = pr.clauses[pr.route_offsets[0]]
    assert pr.handles[c["label_begin"]:c["label_end"]].tolist() == [1]
    assert c["range_end"] - c["range_begin"] == 1
    g = pl.graph.predicate
    res = [g.handles[g.clauses[g.route_offsets[r]]["label_begin"]:
                     g.clauses[g.route_offsets[r]]["label_end"]].tolist() for r in range(3)]
    assert res == [[2], [1], []]
    with pytest.raises(ValueError):
        gp.plan_dnf(Ix(), [[([], True)]], [rng])
    # clause scans: a ranged clause with graph anchors also gets the
    # exhaustive scan over its least-posting label (the reference's range
    # route); a clause already routed as that scan gets no second one
    g_rows, p_rows = gp.dnf_route_rows(Ix(), clauses, [rng, []], clause_scans=True)
    assert [(r[0], r[1], r[2]) for r in p_rows] == [(0, 3, [1]), (0, 1, [2])]
    assert all(r[3] == rng for r in p_rows)
    assert len(g_rows) == 3


@pytest.fixture(scope="module")
def c5_small():
    wl = synth.config5(n=60_000, nq=160, device="cpu", dim=64, k=32, labels=20, intervals=10,
                       vocab=600)
    cen = gi.train_kmeans(wl.base, 32, seed=4, backend=CPU_BUILD)
    li = gi.build_label_index(wl.base.float(), wl.label_offsets, wl.label_values, wl.num_labels,
                              cen, degree=32, threshold=800, local=12,
                              backend=CPU_BUILD)
    return wl, li, cen


def _passes(wl, q, s):
    cat = int(wl.label_values[3 * s])
    tok = int(wl.label_values[3 * s + 2])
    attr = float(wl.base_ranges[s, 0])
    for labels, uses_range in wl.meta["query_clauses"][q]:
        ok = all(l in (cat, tok) for l in labels)
        if ok and uses_range:
            (_, _, lo, hi), = wl.query_ranges[q]
            ok = lo <= attr < hi
        if ok:
            return True
    return False


def test_c5_routes_end_to_end_through_oracle(c5_small):
    """Plan every C5 query, search graph routes (RaBitQ) and posting routes
    with their residual predicates in the oracle, rerank exactly and merge:
    every returned sample satisfies its query's DNF filter, and recall@10
    against exact filtered ground truth is high."""
    wl, li, cen = c5_small
    types = wl.meta["query_types"]
    assert set(types) == set(synth.QUERY_TYPES_C5)
    g_rows, p_rows = gp.dnf_route_rows(li, wl.meta["query_clauses"], wl.query_ranges,
                                       clause_scans=True)
    assert g_rows and p_rows
    rs, ps = gp._routeset(g_rows, li), gp._routeset(p_rows, li)
    x = wl.base.float()
    P = 64
    rot = gi.random_rotation(wl.dim, P, 5, "cpu")
    codes, fac, aid, anchors = gi.rabitq_encode(x, rot, cen, backend=CPU_BUILD)
    qr = (wl.queries.float() @ rot).numpy()
    nq = qr.shape[0]
    q8 = np.empty((nq, P), np.int8)
    sc = np.empty(nq, np.float32)
    k1 = np.empty(nq, np.float32)
    for i in range(nq):
        q8[i], sc[i], k1[i] = po.rabitq_quantize(qr[i])
    an = anchors.numpy().astype(np.float64)
    cd = ((qr.astype(np.float64)[:, None, :] - an[None]) ** 2).sum(-1).astype(np.float32)
    W = 60
    pg = po.PredicateArrays.from_plan(rs.predicate, li, base_ranges=wl.base_ranges, alpha=0.15,
                                      pending_base_stop=True)
    gi_, _, _ = po.rabitq_search(li, rs, pg, po.params(queue_limit=160, result_width=W,
                                                       rabitq_verdict=1),
                                 codes.numpy(), fac.numpy(), aid.numpy().astype(np.uint32), q8,
                                 sc, k1, cd, anchors.shape[0], P, threads=4)
    pp = po.PredicateArrays.from_plan(ps.predicate, li, base_ranges=wl.base_ranges)
    off = np.array([li.posting_offset[r[1]] for r in p_rows], np.uint32)
    size = np.array([li.posting_offset[r[1] + 1] - li.posting_offset[r[1]] for r in p_rows],
                    np.uint32)
    pi_, _, _ = po.posting_scan_rabitq(pp, codes.numpy(), fac.numpy(),
                                       aid.numpy().astype(np.uint32), q8, sc, k1, cd,
                                       ps.route_query, li.posting_ids, off, size, W)
    base = wl.base.numpy()
    qs = wl.queries.numpy()
    sl = np.concatenate([gi_, pi_])
    rq = np.concatenate([rs.route_query, ps.route_query]).astype(np.uint32)
    ri, rd = po.rerank(base, qs, rq, sl, 10)
    mi, md = po.merge(rq, ri, rd, nq, 10)
    recalls = {t: [] for t in synth.QUERY_TYPES_C5}
    for q in range(nq):
        got = [int(s) for s in mi[q] if s != U32MAX]
        assert all(_passes(wl, q, s) for s in got), q
        ok = np.array([_passes(wl, q, s) for s in range(wl.n)])
        cand = np.flatnonzero(ok)
        if cand.size == 0:
            continue
        d = ((base[cand].astype(np.float64) - qs[q].astype(np.float64)) ** 2).sum(1)
        want = cand[np.lexsort((cand, d))[:10]]
        recalls[types[q]].append(len(set(got) & set(want.tolist())) / len(want))
    for t, r in recalls.items():
        assert r and np.mean(r) > 0.8, (t, np.mean(r) if r else None)
