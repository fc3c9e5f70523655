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
