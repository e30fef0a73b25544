"""String predicates: token labels and the n-gram index that expands a fuzzy
pattern into token labels (host side of the hybrid-predicate path).

A string attribute value is one token; each distinct token is a label in the
sample-major label CSR, so exact string match is an ordinary label route and
fuzzy match is an OR over the token labels the n-gram index returns
(expand_manifest_fuzzy_labels, src/data/dataloader.cpp:5046-5156).  The
device evaluates every resulting predicate as labels, like any other.

Semantics follow the reference:
  * normalize: alphanumeric bytes lower-cased, every other run of bytes one
    space (not leading), trailing spaces dropped
    (normalize_manifest_token_text, dataloader.cpp:2973-2991);
  * n-grams: the sorted distinct substrings of length n; a normalized text
    of at most n characters is its own single gram (token_ngrams,
    :2993-3011);
  * score of a token against a pattern: |G_p & G_t| / |G_p | G_t| in
    float32, kept when >= min_score; prefix / suffix / contains modes keep a
    direct match whatever its score, ranked as max(1, score)
    (ManifestNgramIndex::expand, :3647-3760);
  * at most max_terms tokens (query_manifest_max_fuzzy_terms, default 64,
    dataloader.h:1032): the kept tokens are ranked direct matches first,
    then by score descending, then by token id ascending, and the first
    max_terms are returned (:3748-3762).  Output: ascending distinct token
    ids.
"""
from __future__ import annotations

import numpy as np

# query_manifest_max_fuzzy_terms (dataloader.h:1032)
MAX_FUZZY_TERMS = 64


def normalize(text: str) -> str:
    out = []
    prev_space = False
    for ch in text.encode("utf-8", errors="ignore"):
        c = chr(ch)
        if c.isascii() and c.isalnum():
            out.append(c.lower())
            prev_space = False
        elif not prev_space and out:
            out.append(" ")
            prev_space = True
    while out and out[-1] == " ":
        out.pop()
    return "".join(out)


def ngrams(normalized: str, n: int = 3) -> list:
    if not normalized:
        return []
    n = max(1, int(n))
    if len(normalized) <= n:
        return [normalized]
    return sorted(set(normalized[i:i + n] for i in range(len(normalized) - n + 1)))


class NgramIndex:
    """Inverted n-gram index over token texts (token id = position)."""

    def __init__(self, tokens: list, n: int = 3):
        self.n = n
        self.texts = [normalize(t) for t in tokens]
        gram_id: dict = {}
        post_tok, post_gram = [], []
        counts = np.zeros(len(tokens), dtype=np.int64)
        for tid, text in enumerate(self.texts):
            grams = ngrams(text, n)
            counts[tid] = len(grams)
            for g in grams:
                gid = gram_id.setdefault(g, len(gram_id))
                post_gram.append(gid)
                post_tok.append(tid)
        self.gram_id = gram_id
        self.gram_counts = counts
        pg = np.asarray(post_gram, dtype=np.int64)
        pt = np.asarray(post_tok, dtype=np.int64)
        order = np.lexsort((pt, pg))  # by gram, tokens ascending
        self.post_tokens = pt[order]
        self.post_offsets = np.zeros(len(gram_id) + 1, dtype=np.int64)
        np.cumsum(np.bincount(pg, minlength=len(gram_id)), out=self.post_offsets[1:])

    def expand(self, pattern: str, min_score: float = 0.25, mode: str = "",
               max_terms: int = MAX_FUZZY_TERMS) -> np.ndarray:
        """Token ids matching `pattern`, at most `max_terms` of them by the
        reference's ranking, ascending."""
        if int(max_terms) <= 0:
            raise ValueError("max_terms (query_manifest_max_fuzzy_terms) must be positive")
        norm = normalize(pattern)
        if not norm:
            return np.zeros(0, dtype=np.int64)
        grams = ngrams(norm, self.n)
        ids = [self.gram_id[g] for g in grams if g in self.gram_id]
        if not ids:
            return np.zeros(0, dtype=np.int64)
        hits = np.concatenate([self.post_tokens[self.post_offsets[i]:self.post_offsets[i + 1]]
                               for i in ids])
        toks, overlap = np.unique(hits, return_counts=True)
        union = len(grams) + self.gram_counts[toks] - overlap
        score = np.where(union == 0, np.float32(0),
                         overlap.astype(np.float32) / union.astype(np.float32))
        direct = np.zeros(toks.shape[0], bool)
        mode = mode.lower()
        if mode in ("prefix", "suffix", "contains", "substring"):
            direct = np.array([self._direct(self.texts[t], norm, mode) for t in toks], bool)
        keep = direct | (score >= np.float32(min_score))
        toks, score, direct = toks[keep], score[keep], direct[keep]
        if toks.shape[0] > max_terms:
            rank = np.where(direct, np.maximum(np.float32(1), score), score).astype(np.float32)
            # direct first, then score descending, then token id ascending
            order = np.lexsort((toks, -rank.astype(np.float64), ~direct))
            toks = np.sort(toks[order[:int(max_terms)]])
        return toks

    @staticmethod
    def _direct(text: str, pattern: str, mode: str) -> bool:
        if mode == "prefix":
            return text.startswith(pattern)
        if mode == "suffix":
            return text.endswith(pattern)
        return pattern in text


def _chain(rng, A: int, branching: int):
    """Transition CDF [A][A][A] of an order-2 chain (each two-character
    context has `branching` likely next characters, a small floor on the
    others) and the CDF of the first two characters."""
    w = np.full((A, A, A), 0.02)
    for a in range(A):
        for b in range(A):
            nxt = rng.choice(A, size=branching, replace=False)
            w[a, b, nxt] += rng.gamma(1.0, 1.0, size=branching) * 4.0
    cdf = np.cumsum(w / w.sum(-1, keepdims=True), axis=-1)
    first = np.cumsum(rng.gamma(1.0, 1.0, size=(A, A)).ravel())
    return cdf, first / first[-1]


def _run_chain(rng, cdf, ctx: np.ndarray, steps: int) -> np.ndarray:
    """Continue each row's two-character context `steps` characters."""
    m, A = ctx.shape[0], cdf.shape[0]
    out = np.empty((m, steps + 2), dtype=np.int64)
    out[:, :2] = ctx
    u = rng.random((m, max(steps, 1)))
    for j in range(steps):
        c = cdf[out[:, j], out[:, j + 1]]
        out[:, j + 2] = np.minimum((c < u[:, j:j + 1]).sum(1), A - 1)
    return out[:, 2:]


def markov_strings(count: int, seed: int, min_len: int = 8, max_len: int = 32,
                   family: int = 4, max_suffix: int = 6,
                   alphabet: str = "abcdefghijklmnopqrstuvwxyz", branching: int = 5) -> list:
    """`count` distinct lowercase strings of min_len..max_len characters from
    a seeded order-2 character Markov chain.  Strings come in families, as
    words of a language do: a stem is drawn from the chain, then the chain
    continues from the stem's last two characters into `family` endings of
    0..max_suffix characters, so relatives share most of their 3-grams."""
    rng = np.random.default_rng(seed)
    letters = np.array(list(alphabet))
    A = len(alphabet)
    cdf, first = _chain(rng, A, branching)
    out, seen = [], set()
    while len(out) < count:
        m = max(256, (count - len(out)) // family + 1)
        stem_len = rng.integers(min_len, max_len - max_suffix + 1, size=m)
        start = np.searchsorted(first, rng.random(m))
        body = _run_chain(rng, cdf, np.stack([start // A, start % A], 1), int(stem_len.max()) - 2)
        stems = np.concatenate([np.stack([start // A, start % A], 1), body], 1)
        rep = np.repeat(np.arange(m), family)
        last = np.stack([stems[rep, stem_len[rep] - 2], stems[rep, stem_len[rep] - 1]], 1)
        suf_len = rng.integers(0, max_suffix + 1, size=rep.shape[0])
        tails = _run_chain(rng, cdf, last, max_suffix)
        for i in range(rep.shape[0]):
            st_ = stems[rep[i], :stem_len[rep[i]]]
            s = "".join(letters[np.concatenate([st_, tails[i, :suf_len[i]]])])
            if min_len <= len(s) <= max_len and s not in seen:
                seen.add(s)
                out.append(s)
                if len(out) == count:
                    break
    return out


def mutate(text: str, rng, edits: int = 1, alphabet: str = "abcdefghijklmnopqrstuvwxyz") -> str:
    """`edits` random single-character substitutions (a fuzzy pattern)."""
    chars = list(text)
    for _ in range(edits):
        i = int(rng.integers(0, len(chars)))
        chars[i] = alphabet[int(rng.integers(0, len(alphabet)))]
    return "".join(chars)
