"""Batched binary (Hamming) searches, the matrix-core scan, against the CPU oracle: ids and
scores bit-exact under the lowest-index tie-break.

Batches of 4 or more queries over 512- or 1024-dim sign-packed rows take the MFMA scans: up to 64
queries the stream kernel, once per set of 32, and more the tile kernel. The cases cover both row
sizes on both kernels, partial query groups and sets (17, 33, 100), a batch over two launches (130),
k from 1 to 1000 (Hamming scores tie massively at the k-th place), a partial last tile, queries
whose bits are all clear or all set, and duplicated rows."""

import numpy as np
import pytest

import oracle
from helpers import assert_topk_equivalent, normalized

pytestmark = pytest.mark.gpu


def search(capi, words, dim, queries, k):
    n = words.shape[0]
    store = capi.store_desc(capi.DeviceArray.from_host(words), n, dim, capi.BINARY)
    desc = capi.search_desc(store, capi.DeviceArray.from_host(queries), queries.shape[0], k)
    idx, val, flags = capi.search(desc)
    assert not flags.any(), "candidate overflow on a random corpus"
    return idx, val


@pytest.mark.parametrize("n,dim,batch,k", [
    (70_001, 512, 4, 10),
    (70_001, 512, 33, 100),
    (70_001, 512, 100, 10),      # the tile kernel at 512 bits
    (70_001, 1024, 17, 1),
    (120_007, 1024, 32, 10),
    (120_007, 1024, 100, 100),
    (60_013, 1024, 130, 10),
    (60_013, 1024, 32, 1000),
])
def test_batched_hamming_bit_exact(gpu, n, dim, batch, k):
    capi = gpu
    corpus = normalized(n, dim, 300 + batch)
    queries = normalized(batch, dim, 400 + batch)
    words = oracle.pack_binary(corpus)
    idx, val = search(capi, words, dim, queries, k)
    ref = oracle.scores_hamming(words, oracle.pack_binary(queries), dim)
    assert_topk_equivalent(idx, val, ref, k)


def test_batched_hamming_extreme_queries_and_duplicates(gpu):
    capi = gpu
    n, dim, k = 50_000, 1024, 64
    base = normalized(700, dim, 11)
    corpus = base[np.arange(n) % 700]  # 700 classes of identical rows
    queries = normalized(8, dim, 12)
    queries[0] = 1.0   # every bit set
    queries[1] = -1.0  # every bit clear
    queries[2] = -queries[3]  # complementary pair
    words = oracle.pack_binary(corpus)
    idx, val = search(capi, words, dim, queries, k)
    ref = oracle.scores_hamming(words, oracle.pack_binary(queries), dim)
    assert_topk_equivalent(idx, val, ref, k)
