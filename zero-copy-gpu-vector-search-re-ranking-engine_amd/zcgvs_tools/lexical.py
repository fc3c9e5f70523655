"""BM25 CSR index builder over documents given as term-id lists, and the synthetic index of the
hybrid configuration (Poisson(200) document lengths, i.i.d. Zipf(1.1) tokens over a 30,000-term
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
    return _ZipfSampler(vocab_size, s).draw(rng.random(count)).astype(np.int64)


class _ZipfSampler:
    """Inverse-CDF sampling, searchsorted(cdf, u, 'right') capped at vocab_size - 1, through a
    table of 2^20 equal-width buckets of u: a bucket holding no CDF point maps all of its u to
    one term (u * 2^20 is exact, so the bucket of u is exact); only the u in the few buckets that
    hold a CDF point are searched. Results equal the plain search for every u."""

    BITS = 20

    def __init__(self, vocab_size: int, s: float):
        ranks = np.arange(1, vocab_size + 1, dtype=np.float64)
        cdf = np.cumsum(ranks ** -s)
        cdf /= cdf[-1]
        self.cdf = cdf
        self.vocab_size = vocab_size
        edges = np.arange((1 << self.BITS) + 1, dtype=np.float64) / float(1 << self.BITS)
        below = np.searchsorted(cdf, edges[:-1], side="right")   # count(cdf <= bucket start)
        inside = np.searchsorted(cdf, edges[1:], side="left")    # count(cdf < bucket end)
        self.table = below.astype(np.int32)
        self.mixed = inside != below

    def draw(self, u: np.ndarray) -> np.ndarray:
        bucket = (u * float(1 << self.BITS)).astype(np.int64)
        out = self.table[bucket]
        hard = np.flatnonzero(self.mixed[bucket])
        out[hard] = np.searchsorted(self.cdf, u[hard], side="right")
        return np.minimum(out, self.vocab_size - 1)


def synthetic_corpus(doc_count: int, vocab_size: int = 30_000, mean_length: float = 200.0, s: float = 1.1,
                     seed: int = 7) -> list[np.ndarray]:
    rng = np.random.default_rng(seed)
    lengths = rng.poisson(mean_length, size=doc_count)
    flat = zipf_terms(rng, int(lengths.sum()), vocab_size, s)
    return np.split(flat, np.cumsum(lengths)[:-1])


def synthetic_index(doc_count: int, vocab_size: int = 30_000, mean_length: float = 200.0, s: float = 1.1,
                    seed: int = 7, k1: float = 1.2, b: float = 0.75, chunk_docs: int = 65_536,
                    with_counts: bool = False) -> dict:
    """The BM25 index of the synthetic token model, built exactly: document lengths ~
    Poisson(mean_length), every token an i.i.d. Zipf(s) term (zipf_terms), tf = the number of
    times a term occurs in a document, length = the document's token count (the reference's
    builder counts tokens the same way, python/zcgvs_tools/build_lexical.py:128-154).

    Documents are tokenized and counted in chunks of `chunk_docs` documents: one sort of
    (term, document) inside the chunk gives its postings term-major with documents ascending and
    their counts as run lengths; the chunks, taken in document order, are then placed term by term
    behind each other, so every term's documents ascend. Memory stays proportional to one chunk's
    tokens plus the postings. With `with_counts` the result also holds the per-posting term counts
    ("tf") and the document lengths ("lengths")."""
    rng = np.random.default_rng(seed)
    lengths = rng.poisson(mean_length, size=doc_count).astype(np.int64)
    sampler = _ZipfSampler(vocab_size, s)
    shift = max(1, int(chunk_docs - 1).bit_length())
    key_type = np.uint32 if (vocab_size << shift) <= (1 << 32) else np.uint64
    chunks = []
    df = np.zeros(vocab_size, dtype=np.int64)
    for d0 in range(0, doc_count, chunk_docs):
        d1 = min(doc_count, d0 + chunk_docs)
        counts = lengths[d0:d1]
        tokens = sampler.draw(rng.random(int(counts.sum()))).astype(key_type)
        keys = (tokens << key_type(shift)) | np.repeat(np.arange(d1 - d0, dtype=key_type), counts)
        del tokens
        keys.sort()
        if keys.size == 0:
            continue
        starts = np.flatnonzero(np.concatenate(([True], keys[1:] != keys[:-1])))
        uniq = keys[starts]
        tf = np.diff(np.append(starts, keys.size)).astype(np.int32)
        del keys, starts
        terms = (uniq >> key_type(shift)).astype(np.int32)
        docs = (d0 + (uniq & key_type((1 << shift) - 1)).astype(np.int64)).astype(np.int32)
        df += np.bincount(terms, minlength=vocab_size)
        chunks.append((terms, docs, tf))
    offsets = np.zeros(vocab_size + 1, dtype=np.int64)
    offsets[1:] = np.cumsum(df)
    nnz = int(offsets[-1])
    docs_out = np.empty(nnz, dtype=np.int32)
    tf_out = np.empty(nnz, dtype=np.int32)
    cursor = offsets[:-1].copy()
    for terms, docs, tf in chunks:
        # postings of the chunk are term-major: rank within the term's run + the term's cursor
        run = np.flatnonzero(np.concatenate(([True], terms[1:] != terms[:-1])))
        run_length = np.diff(np.append(run, terms.size))
        rank = np.arange(terms.size, dtype=np.int64) - np.repeat(run, run_length)
        position = cursor[terms] + rank
        docs_out[position] = docs
        tf_out[position] = tf
        cursor[terms[run]] += run_length
    chunks.clear()
    avgdl = float(lengths.mean()) if doc_count else 1.0
    avgdl = avgdl if avgdl > 0.0 else 1.0
    term_of = np.repeat(np.arange(vocab_size, dtype=np.int64), df)
    dfp = df[term_of].astype(np.float64)
    del term_of
    idf = np.log(1.0 + (doc_count - dfp + 0.5) / (dfp + 0.5))
    del dfp
    tf64 = tf_out.astype(np.float64)
    norm = k1 * (1.0 - b + b * lengths[docs_out].astype(np.float64) / avgdl)
    weights = (idf * (tf64 * (k1 + 1.0)) / (tf64 + norm)).astype(np.float32)
    index = {"offsets": offsets, "posting_docs": docs_out, "posting_weights": weights, "doc_count": doc_count,
             "vocab_size": vocab_size, "k1": k1, "b": b, "average_doc_length": avgdl}
    if with_counts:
        index["tf"] = tf_out
        index["lengths"] = lengths
    return index


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
