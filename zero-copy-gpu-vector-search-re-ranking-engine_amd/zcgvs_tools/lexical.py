"""BM25 CSR index builder over documents given as term-id lists, and the synthetic corpus of the
hybrid configuration (Poisson(200) document lengths, Zipf(1.1) term draws over a 30,000-term
vocabulary, 8 distinct Zipf terms per query).

Weights follow python/zcgvs_tools/build_lexical.py:143-154 of the reference, in float64, cast to
float32 when stored: idf = ln(1 + (N - df + 0.5) / (df + 0.5)),
w = idf * tf * (k1 + 1) / (tf + k1 * (1 - b + b * len / avgdl)). Postings of a term are in
ascending document order.
"""

from __future__ import annotations

import numpy as np


def build_bm25(doc_terms: list[np.ndarray], vocab_size: int, k1: float = 1.2, b: float = 0.75) -> dict:
    """CSR arrays (offsets [V + 1] int64, posting_docs int32, posting_weights float32) and stats."""
    n = len(doc_terms)
    lengths = np.array([len(t) for t in doc_terms], dtype=np.float64)
    avgdl = float(lengths.mean()) if n else 0.0
    if avgdl <= 0.0:
        avgdl = 1.0
    doc_ids, term_ids, tfs = [], [], []
    for d, terms in enumerate(doc_terms):
        terms = np.asarray(terms, dtype=np.int64)
        terms = terms[(terms >= 0) & (terms < vocab_size)]
        uniq, counts = np.unique(terms, return_counts=True)
        doc_ids.append(np.full(uniq.size, d, dtype=np.int64))
        term_ids.append(uniq)
        tfs.append(counts)
    doc_ids = np.concatenate(doc_ids) if doc_ids else np.zeros(0, np.int64)
    term_ids = np.concatenate(term_ids) if term_ids else np.zeros(0, np.int64)
    tfs = np.concatenate(tfs).astype(np.float64) if tfs else np.zeros(0)
    df = np.bincount(term_ids, minlength=vocab_size).astype(np.float64)
    idf = np.log(1.0 + (n - df[term_ids] + 0.5) / (df[term_ids] + 0.5))
    norm = k1 * (1.0 - b + b * lengths[doc_ids] / avgdl)
    weights = idf * (tfs * (k1 + 1.0)) / (tfs + norm)
    order = np.lexsort((doc_ids, term_ids))  # by term, then document
    offsets = np.zeros(vocab_size + 1, dtype=np.int64)
    offsets[1:] = np.cumsum(np.bincount(term_ids, minlength=vocab_size))
    return {"offsets": offsets, "posting_docs": doc_ids[order].astype(np.int32),
            "posting_weights": weights[order].astype(np.float32), "doc_count": n, "vocab_size": vocab_size,
            "k1": k1, "b": b, "average_doc_length": avgdl}


def zipf_terms(rng: np.random.Generator, count: int, vocab_size: int, s: float = 1.1) -> np.ndarray:
    """`count` term ids with P(rank r) proportional to r^-s over ranks 1..vocab_size (id = rank - 1)."""
    ranks = np.arange(1, vocab_size + 1, dtype=np.float64)
    cdf = np.cumsum(ranks ** -s)
    cdf /= cdf[-1]
    return np.minimum(np.searchsorted(cdf, rng.random(count), side="right"), vocab_size - 1).astype(np.int64)


def synthetic_corpus(doc_count: int, vocab_size: int = 30_000, mean_length: float = 200.0, s: float = 1.1,
                     seed: int = 7) -> list[np.ndarray]:
    rng = np.random.default_rng(seed)
    lengths = rng.poisson(mean_length, size=doc_count)
    flat = zipf_terms(rng, int(lengths.sum()), vocab_size, s)
    return np.split(flat, np.cumsum(lengths)[:-1])


def zero_truncated_poisson(rng: np.random.Generator, lam: np.ndarray) -> np.ndarray:
    """One draw of Poisson(lam) conditioned on >= 1 per element, by inverting its CDF; each
    round continues only with the elements whose draw exceeds the current count."""
    lam = np.asarray(lam, dtype=np.float64)
    out = np.ones(lam.size, dtype=np.int64)
    u = rng.random(lam.size)
    denom = -np.expm1(-lam)
    term = lam * np.exp(-lam) / denom  # P(k = 1 | k >= 1)
    cum = term.copy()
    live = np.flatnonzero(u > cum)
    term, cum, lam_live, u_live = term[live], cum[live], lam[live], u[live]
    k = 1
    while live.size and k < 1000:
        k += 1
        term *= lam_live / k
        cum += term
        out[live] = k
        keep = u_live > cum
        live, term, cum, lam_live, u_live = live[keep], term[keep], cum[keep], lam_live[keep], u_live[keep]
    return out


def synthetic_index(doc_count: int, vocab_size: int = 30_000, mean_length: float = 200.0, s: float = 1.1,
                    seed: int = 7, k1: float = 1.2, b: float = 0.75) -> dict:
    """The BM25 index of synthetic_corpus's model, generated term by term without tokens.

    With document lengths ~ Poisson(mean_length) and tokens drawn i.i.d. from the Zipf law p_t,
    the term counts n_{d,t} are independent Poisson(mean_length * p_t) (Poisson splitting), and
    a document's length is the sum of its counts. So each term's postings are drawn directly: the
    documents holding a frequent term are a Bernoulli(1 - exp(-lambda_t)) subset; a rare term
    gets a binomial number of uniform documents (a document drawn twice for one term counts
    once, which at these rates changes almost nothing); counts are zero-truncated
    Poisson(lambda_t). The cost is linear in the postings (about 1.2e8 at 1M documents), not in
    the 2e8 tokens. Weights and layout are those of build_bm25."""
    rng = np.random.default_rng(seed)
    ranks = np.arange(1, vocab_size + 1, dtype=np.float64)
    p = ranks ** -s
    p /= p.sum()
    lam = mean_length * p
    present = -np.expm1(-lam)  # P(n_{d,t} >= 1)
    frequent = np.flatnonzero(present > 0.05)
    rare = np.flatnonzero(present <= 0.05)
    term_parts, doc_parts = [], []
    for t in frequent:
        docs = np.flatnonzero(rng.random(doc_count) < present[t])
        term_parts.append(np.full(docs.size, t, dtype=np.int64))
        doc_parts.append(docs.astype(np.int64))
    sizes = rng.binomial(doc_count, present[rare])
    rare_terms = np.repeat(rare.astype(np.int64), sizes)
    rare_keys = np.unique(rare_terms * doc_count + rng.integers(0, doc_count, size=rare_terms.size))
    term_parts.append(rare_keys // doc_count)
    doc_parts.append(rare_keys % doc_count)
    terms = np.concatenate(term_parts)
    docs = np.concatenate(doc_parts)
    order = np.argsort(terms, kind="stable")  # frequent terms come first; rare keys are sorted
    terms, docs = terms[order], docs[order].astype(np.int32)
    tfs = zero_truncated_poisson(rng, lam[terms]).astype(np.float64)
    counts = np.bincount(terms, minlength=vocab_size)
    lengths = np.bincount(docs, weights=tfs, minlength=doc_count)
    avgdl = float(lengths.mean()) if doc_count else 1.0
    avgdl = avgdl if avgdl > 0.0 else 1.0
    offsets = np.zeros(vocab_size + 1, dtype=np.int64)
    offsets[1:] = np.cumsum(counts)
    df = counts.astype(np.float64)
    idf = np.log(1.0 + (doc_count - df[terms] + 0.5) / (df[terms] + 0.5))
    norm = k1 * (1.0 - b + b * lengths[docs] / avgdl)
    weights = (idf * (tfs * (k1 + 1.0)) / (tfs + norm)).astype(np.float32)
    return {"offsets": offsets, "posting_docs": docs, "posting_weights": weights, "doc_count": doc_count,
            "vocab_size": vocab_size, "k1": k1, "b": b, "average_doc_length": avgdl}


def synthetic_queries(batch: int, terms: int = 8, vocab_size: int = 30_000, s: float = 1.1,
                      seed: int = 11) -> np.ndarray:
    """[batch, terms] int32 distinct Zipf term ids per query."""
    rng = np.random.default_rng(seed)
    out = np.empty((batch, terms), dtype=np.int32)
    for q in range(batch):
        chosen: list[int] = []
        while len(chosen) < terms:
            for t in zipf_terms(rng, terms, vocab_size, s):
                if int(t) not in chosen:
                    chosen.append(int(t))
                if len(chosen) == terms:
                    break
        out[q] = chosen
    return out
