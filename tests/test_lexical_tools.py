"""The synthetic BM25 index of the hybrid configuration (CPU): the chunked generator equals the
list-based builder on the same tokens, its weights are the oracle's BM25 weight
(python/zcgvs_tools/build_lexical.py:143-154), and its layout is the reference builder's (postings
of a term ascending by document, one per document)."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from zcgvs_tools import lexical


@pytest.mark.parametrize("chunk", [700, 4096])
def test_synthetic_index_equals_the_list_builder(chunk):
    n, vocab, seed = 3000, 500, 9
    index = lexical.synthetic_index(n, vocab, seed=seed, chunk_docs=chunk)
    # the same token stream, drawn document chunk by document chunk
    rng = np.random.default_rng(seed)
    lengths = rng.poisson(200.0, size=n)
    sampler = lexical._ZipfSampler(vocab, 1.1)
    docs = []
    for d0 in range(0, n, chunk):
        counts = lengths[d0:d0 + chunk]
        flat = sampler.draw(rng.random(int(counts.sum())))
        docs += np.split(flat, np.cumsum(counts)[:-1])
    ref = lexical.build_bm25(docs, vocab)
    for key in ("offsets", "posting_docs", "posting_weights"):
        assert np.array_equal(index[key], ref[key]), key
    assert index["average_doc_length"] == ref["average_doc_length"]


def test_synthetic_index_layout_and_weights():
    n, vocab = 20_000, 3000
    index = lexical.synthetic_index(n, vocab, seed=4, with_counts=True)
    offsets, docs, weights, tf = index["offsets"], index["posting_docs"], index["posting_weights"], index["tf"]
    lengths = index["lengths"]
    assert offsets[0] == 0 and offsets[-1] == docs.size == weights.size == tf.size
    assert np.all(np.diff(offsets) >= 0)
    # strictly ascending documents inside every term: one posting per (term, document)
    term_of = np.repeat(np.arange(vocab), np.diff(offsets))
    same_term = term_of[1:] == term_of[:-1]
    assert np.all(docs[1:][same_term] > docs[:-1][same_term])
    # term counts add up to the document lengths, and avgdl is their mean
    assert np.array_equal(np.bincount(docs, weights=tf, minlength=n).astype(np.int64), lengths)
    assert index["average_doc_length"] == float(lengths.mean())
    # every sampled weight is the oracle's BM25 weight of its (df, tf, length)
    df = np.diff(offsets)
    pick = np.random.default_rng(1).choice(docs.size, 400, replace=False)
    for p in pick:
        expected = oracle.bm25_weight(n, int(df[term_of[p]]), int(tf[p]), float(lengths[docs[p]]),
                                      index["average_doc_length"], 1.2, 0.75)
        assert weights[p] == np.float32(expected)


def test_zipf_sampler_equals_the_plain_inverse_cdf():
    u = np.random.default_rng(3).random(200_000)
    u[:3] = [0.0, 1.0 - 2.0 ** -53, 0.5]
    for vocab, s in ((30_000, 1.1), (1000, 0.5), (7, 2.0)):
        ranks = np.arange(1, vocab + 1, dtype=np.float64)
        cdf = np.cumsum(ranks ** -s)
        cdf /= cdf[-1]
        expected = np.minimum(np.searchsorted(cdf, u, side="right"), vocab - 1)
        assert np.array_equal(lexical._ZipfSampler(vocab, s).draw(u), expected)


def test_synthetic_queries_are_distinct_terms():
    terms = lexical.synthetic_queries(16, 8, 30_000, seed=11)
    assert terms.shape == (16, 8)
    assert all(len(set(row.tolist())) == 8 for row in terms)
    assert terms.min() >= 0 and terms.max() < 30_000
