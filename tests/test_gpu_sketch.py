"""The sketch-planned search against the oracle.

A per-vector int8 search on the matrix cores over a large corpus runs a sketch launch (every
stride-th 64-row block; per row half of a workgroup, the best score of each query), takes the
j-th best of those scores as a speculative threshold, scans the whole corpus once keeping the keys
at or above it, and flags a query whose candidate buffers overflowed or which found fewer than k
keys. Flagged queries are scanned again over the whole corpus by the matrix-core scan with a
threshold that is a certain lower bound (the rerun), and their selection comes from that. Every
path must give the oracle's top-k bit for bit: the speculative path itself, the fallback when the
threshold was too high (ZCGVS_SEARCH_TEST_HIGH_THRESHOLD), the rerun after overflowing candidate
buffers (ZCGVS_SEARCH_TEST_TINY_SEGMENTS), the last resort after an overflowing rerun
(ZCGVS_SEARCH_TEST_TINY_RERUN) or for every query (ZCGVS_SEARCH_FORCE_EXACT_PASS), with
an allow-mask, and with more than one launch of 256 queries.

A binary (Hamming) search of at most 32 queries runs the same plan in the streaming binary scan
(8 sketch slots per workgroup, one per pair of wavefronts); Hamming scores tie massively, so the
threshold admits every row at the threshold's distance."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from helpers import assert_topk_equivalent, normalized

pytestmark = pytest.mark.gpu

N, DIM, BATCH, K = 1_000_000, 256, 256, 100


@pytest.fixture(scope="module")
def corpus(gpu):
    capi = gpu
    codes, scales = oracle.quantize_rows_i8(normalized(N, DIM, 91))
    queries = normalized(300, DIM, 92)
    return dict(codes=codes, scales=scales, queries=queries,
                d_codes=capi.DeviceArray.from_host(codes), d_scales=capi.DeviceArray.from_host(scales),
                d_queries=capi.DeviceArray.from_host(queries[:BATCH]),
                d_queries_300=capi.DeviceArray.from_host(queries))


def _desc(capi, c, batch=BATCH, k=K, flags=0, mask=None):
    store = capi.store_desc(c["d_codes"], N, DIM, capi.I8, 1.0, c["d_scales"])
    queries = c["d_queries"] if batch == BATCH else c["d_queries_300"]
    return capi.search_desc(store, queries, batch, k, capi.COSINE, int8_mode=capi.INT8_PER_VECTOR,
                            mask=mask, flags=flags)


def _exact_scores(c, idx, val, batch, mask=None):
    # every query: each returned score is the oracle's score of that id, bit for bit
    qcodes, qscales = oracle.quantize_rows_i8(c["queries"][:batch])
    for b in range(batch):
        rows = idx[b]
        assert len(set(rows.tolist())) == rows.size, f"query {b}: repeated id"
        exact = oracle.scores_i8i8(c["codes"][rows], c["scales"][rows], qcodes[b:b + 1], qscales[b:b + 1],
                                   None if mask is None else mask[rows])[0]
        assert np.array_equal(val[b], exact), f"query {b}: scores differ from the oracle's"


def _ordered_keys(scores):
    """ordered32(score) << 32 as the kernels key a score (-0.0 as +0.0; -inf, an empty slot, as 0)."""
    scores = np.asarray(scores, dtype=np.float32)
    bits = np.where(scores == 0, np.float32(0), scores).view(np.uint32).astype(np.uint64)
    ordered = np.where(bits & 0x80000000, ~bits & 0xFFFFFFFF, bits | 0x80000000)
    return np.where(np.isneginf(scores), 0, ordered).astype(np.uint64) << np.uint64(32)


def _search_with_state(capi, desc):
    size = capi.search_workspace_bytes(desc)
    workspace = capi.DeviceArray(size, np.uint8)
    idx = capi.DeviceArray((desc.batch, desc.k), np.int32)
    val = capi.DeviceArray((desc.batch, desc.k), np.float32)
    capi.search_topk(desc, workspace, size, idx, val)
    capi.synchronize()
    flags = np.empty(desc.batch, dtype=np.uint32)
    capi.call("zcgvs_memcpy_d2h", flags.ctypes.data, capi.search_overflow_flags(desc, workspace), flags.nbytes, None)
    state = capi.search_sketch_state(desc, workspace)
    return idx.to_host(), val.to_host(), flags, state


def _check_sketch(state, flags, sampled_scores, queries):
    """The thresholds are the rank-th and width-th best slot keys (radix select against a sort),
    and the slots are maxima over disjoint sets of the sampled rows: the i-th best slot score is at
    most the i-th best sampled row score, with equality for i = 1 (sampled_scores: the oracle's
    scores of every sampled row, [len(queries), rows])."""
    keys = _ordered_keys(state["slots"])
    ranked = np.sort(keys, axis=0)[::-1]
    rank, width = state["rank"], state["width"]
    assert 1 <= rank <= width <= keys.shape[0]
    spec = ~flags.astype(bool)
    assert np.array_equal(state["tau"][spec], ranked[rank - 1][spec]), "speculative thresholds differ"
    assert np.array_equal(state["tau_safe"], ranked[width - 1]), "certain thresholds differ"
    for i, q in enumerate(queries):
        slot_best = np.sort(state["slots"][:, q])[::-1]
        rows_best = np.sort(sampled_scores[i])[::-1][:slot_best.size]
        assert slot_best[0] == rows_best[0], f"query {q}: the best slot is not the best sampled row"
        assert np.all(slot_best[:rows_best.size] <= rows_best), f"query {q}: a slot beats the sampled rows"


def _sampled(c, idx, val, sample, k, mask=None):
    qcodes, qscales = oracle.quantize_rows_i8(c["queries"][sample])
    ref = oracle.scores_i8i8(c["codes"], c["scales"], qcodes, qscales, mask)
    assert_topk_equivalent(idx[sample], val[sample], ref, k)


@pytest.fixture(scope="module")
def baseline(gpu, corpus):
    capi = gpu
    desc = _desc(capi, corpus)
    rows = capi.search_phase_rows(desc)
    assert len(rows) == 2 and rows[1] == N, f"not sketch-planned: {rows}"
    idx, val, flags = capi.search(desc)
    return idx, val, flags


def test_speculative_scan_is_exact(corpus, baseline):
    idx, val, flags = baseline
    assert not flags.any(), "a random corpus should not need the fallback"
    _exact_scores(corpus, idx, val, BATCH)
    _sampled(corpus, idx, val, [0, 1, 97, 128, 200, 255], K)


def test_sketch_thresholds(gpu, corpus, baseline):
    # every 8th 64-row block is sampled at 1M rows
    capi = gpu
    idx, val, flags, state = _search_with_state(capi, _desc(capi, corpus))
    assert state is not None and state["slots"].shape[1] == BATCH
    assert np.array_equal(idx, baseline[0]) and np.array_equal(val, baseline[1])
    rows = np.concatenate([np.arange(b * 64, min(b * 64 + 64, N)) for b in range(0, (N + 63) // 64, 8)])
    queries = [0, 101, 255]
    qcodes, qscales = oracle.quantize_rows_i8(corpus["queries"][queries])
    sampled = oracle.scores_i8i8(corpus["codes"][rows], corpus["scales"][rows], qcodes, qscales)
    _check_sketch(state, flags, sampled, queries)


@pytest.mark.parametrize("flag", ["high", "tiny", "force"])
def test_fallback_paths_match(gpu, corpus, baseline, flag):
    capi = gpu
    bits = {"high": capi.SEARCH_TEST_HIGH_THRESHOLD, "tiny": capi.SEARCH_TEST_TINY_SEGMENTS,
            "force": capi.SEARCH_FORCE_EXACT_PASS}[flag]
    idx, val, flags = capi.search(_desc(capi, corpus, flags=bits))
    if flag != "force":
        assert int(np.count_nonzero(flags)) > BATCH // 2, f"{flag}: expected most queries flagged"
    ref_idx, ref_val, _ = baseline
    assert np.array_equal(idx, ref_idx), f"{flag}: ids differ from the speculative path's"
    assert np.array_equal(val, ref_val), f"{flag}: scores differ from the speculative path's"


def test_overflowing_rerun_takes_the_last_resort(gpu, corpus, baseline):
    # two-slot segments in the first attempt and in the rerun: nearly every query is listed, its
    # rerun overflows as well, and recoverKernel recomputes it (one sweep, running list)
    capi = gpu
    bits = capi.SEARCH_TEST_TINY_SEGMENTS | capi.SEARCH_TEST_TINY_RERUN
    idx, val, flags = capi.search(_desc(capi, corpus, flags=bits))
    assert int(np.count_nonzero(flags)) > BATCH // 2
    assert np.array_equal(idx, baseline[0]) and np.array_equal(val, baseline[1])


def test_masked_rerun(gpu, corpus):
    capi = gpu
    mask = (np.random.default_rng(93).random(N) > 0.25).astype(np.uint8)
    d_mask = capi.DeviceArray.from_host(mask)
    results = []
    for bits in (0, capi.SEARCH_TEST_TINY_SEGMENTS, capi.SEARCH_TEST_HIGH_THRESHOLD):
        idx, val, flags = capi.search(_desc(capi, corpus, flags=bits, mask=d_mask))
        assert not mask[idx.ravel()].size or mask[idx.ravel()].all(), "a masked row was returned"
        results.append((idx, val))
    for idx, val in results[1:]:
        assert np.array_equal(idx, results[0][0]) and np.array_equal(val, results[0][1])
    _exact_scores(corpus, results[0][0], results[0][1], BATCH, mask)
    _sampled(corpus, results[0][0], results[0][1], [3, 150], K, mask)


def test_partial_launch_of_queries(gpu, corpus):
    # 40 queries: the launch's wavefronts past the first two hold 8 or no queries; the sketch, the
    # speculative scan and the rerun after tiny segments agree with each other and the oracle
    capi = gpu
    batch, k = 40, 100
    assert len(capi.search_phase_rows(_desc(capi, corpus, batch=batch, k=k))) == 2, "not sketch-planned"
    plain = capi.search(_desc(capi, corpus, batch=batch, k=k))
    assert not plain[2].any()
    for bits in (capi.SEARCH_TEST_TINY_SEGMENTS, capi.SEARCH_TEST_HIGH_THRESHOLD):
        other = capi.search(_desc(capi, corpus, batch=batch, k=k, flags=bits))
        assert int(np.count_nonzero(other[2])) > batch // 2
        assert np.array_equal(plain[0], other[0]) and np.array_equal(plain[1], other[1])
    _exact_scores(corpus, plain[0], plain[1], batch)
    _sampled(corpus, plain[0], plain[1], [0, 31, 32, 39], k)


def test_two_launches_of_queries(gpu, corpus):
    # 300 queries: two launches per scan; with tiny segments all of them are flagged, so the
    # rerun's list spans both launches (entries 256..299 in the second)
    capi = gpu
    batch, k = 300, 50
    plain = capi.search(_desc(capi, corpus, batch=batch, k=k))
    tiny = capi.search(_desc(capi, corpus, batch=batch, k=k, flags=capi.SEARCH_TEST_TINY_SEGMENTS))
    assert int(np.count_nonzero(tiny[2])) > batch // 2
    assert np.array_equal(plain[0], tiny[0]) and np.array_equal(plain[1], tiny[1])
    _sampled(corpus, plain[0], plain[1], [0, 255, 256, 299], k)


BIN_N, BIN_DIM = 2_000_003, 1024


@pytest.fixture(scope="module")
def binary_corpus(gpu):
    capi = gpu
    words = np.random.default_rng(94).integers(0, 2**32, size=(BIN_N, BIN_DIM // 32), dtype=np.uint32)
    queries = normalized(64, BIN_DIM, 95)
    return dict(words=words, qwords=oracle.pack_binary(queries), d_words=capi.DeviceArray.from_host(words),
                d_queries=capi.DeviceArray.from_host(queries))


def _binary_desc(capi, c, batch, k, flags=0):
    store = capi.store_desc(c["d_words"], BIN_N, BIN_DIM, capi.BINARY)
    return capi.search_desc(store, c["d_queries"], batch, k, capi.COSINE, flags=flags)


@pytest.mark.parametrize("batch,k", [(32, 100), (20, 1000), (64, 100), (48, 1000)])
def test_binary_sketch_plan(gpu, binary_corpus, batch, k):
    # up to 32 queries one stream launch per phase; 33-64 one sketch launch per set of 32, the full
    # scan on the tile kernel, and reruns of more than 32 flagged queries in two list launches
    capi = gpu
    c = binary_corpus
    desc = _binary_desc(capi, c, batch, k)
    rows = capi.search_phase_rows(desc)
    assert len(rows) == 2 and rows[1] == BIN_N, f"not sketch-planned: {rows}"
    idx, val, flags = capi.search(desc)
    assert not flags.any(), "a random corpus should not need the fallback"
    for name, bits in (("high", capi.SEARCH_TEST_HIGH_THRESHOLD), ("tiny", capi.SEARCH_TEST_TINY_SEGMENTS),
                       ("tiny rerun", capi.SEARCH_TEST_TINY_SEGMENTS | capi.SEARCH_TEST_TINY_RERUN),
                       ("force", capi.SEARCH_FORCE_EXACT_PASS)):
        got_idx, got_val, got_flags = capi.search(_binary_desc(capi, c, batch, k, bits))
        if name != "force":
            assert int(np.count_nonzero(got_flags)) > batch // 2, f"{name}: expected most queries flagged"
        assert np.array_equal(got_idx, idx), f"{name}: ids differ from the speculative path's"
        assert np.array_equal(got_val, val), f"{name}: scores differ from the speculative path's"
    sample = sorted({0, 7, 16, batch // 2 + 3, batch - 1})
    ref = oracle.scores_hamming(c["words"], c["qwords"][sample], BIN_DIM)
    assert_topk_equivalent(idx[sample], val[sample], ref, k)


def test_binary_sketch_thresholds(gpu, binary_corpus):
    # every 4th 384-row block is sampled at 2M rows of 1024 bits
    capi = gpu
    c = binary_corpus
    for batch, k in ((32, 100), (20, 1000)):
        idx, val, flags, state = _search_with_state(capi, _binary_desc(capi, c, batch, k))
        assert state is not None and state["slots"].shape[1] == batch
        rows = np.concatenate([np.arange(b * 384, min(b * 384 + 384, BIN_N))
                               for b in range(0, (BIN_N + 383) // 384, 4)])
        queries = [0, batch - 1]
        sampled = oracle.scores_hamming(c["words"][rows], c["qwords"][queries], BIN_DIM)
        _check_sketch(state, flags, sampled, queries)


def test_binary_512_sketch_plan(gpu):
    # 512-bit rows: 768-row blocks, every 4th one sampled at 3.2M rows; the speculative path, the
    # rerun and the oracle agree bit for bit
    capi = gpu
    n, dim, batch, k = 3_200_001, 512, 24, 100
    words = np.random.default_rng(96).integers(0, 2**32, size=(n, dim // 32), dtype=np.uint32)
    queries = normalized(batch, dim, 97)
    d_words, d_queries = capi.DeviceArray.from_host(words), capi.DeviceArray.from_host(queries)

    def desc(flags=0):
        return capi.search_desc(capi.store_desc(d_words, n, dim, capi.BINARY), d_queries, batch, k, capi.COSINE,
                                flags=flags)

    rows = capi.search_phase_rows(desc())
    assert len(rows) == 2 and rows[1] == n, f"not sketch-planned: {rows}"
    idx, val, flags = capi.search(desc())
    assert not flags.any()
    tiny = capi.search(desc(capi.SEARCH_TEST_TINY_SEGMENTS))
    assert int(np.count_nonzero(tiny[2])) > batch // 2
    assert np.array_equal(tiny[0], idx) and np.array_equal(tiny[1], val)
    sample = [0, 11, batch - 1]
    ref = oracle.scores_hamming(words, oracle.pack_binary(queries)[sample], dim)
    assert_topk_equivalent(idx[sample], val[sample], ref, k)
