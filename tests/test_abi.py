"""CPU-side checks of the C ABI: the library loads, exports every symbol include/zcgvs_hip.h
declares, and its host-side argument checks (src/search/searcher.cpp:91-135, topk.cu:146-153,
similarity.cu:356-358) answer without touching a GPU."""

import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    header = (ROOT / "include" / "zcgvs_hip.h").read_text()
    pattern = r"^(?:const\s+)?[a-z_0-9]+\**\s+\**(zcgvs_[a-z0-9_]+)\s*\("
    return sorted(set(re.findall(pattern, header, flags=re.MULTILINE)))


def test_library_exports_every_declared_symbol(capi):
    lib = capi.library()
    names = declared_symbols()
    assert len(names) >= 50
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(capi.exported_symbols()) == set(names)


def test_version_and_sizing_helpers(capi):
    lib = capi.library()
    assert lib.zcgvs_version().decode().startswith("zcgvs-hip")
    assert lib.zcgvs_topk_max_k() == 1024
    assert lib.zcgvs_topk_tile_size() == 1024
    assert lib.zcgvs_similarity_query_tile() == 8
    assert lib.zcgvs_topk_block_count(5000) == 5
    assert capi.topk_scratch_elements(5000, 100) >= 5 * 100
    assert lib.zcgvs_similarity_shared_bytes(capi.F32, 384, 11) == 8 * 384 * 4
    assert lib.zcgvs_similarity_shared_bytes(capi.BINARY, 384, 3) == 3 * 12 * 4
    assert lib.zcgvs_rescore_shared_bytes(384) == 384 * 4
    # the lexical slice table: one count per term and 4096-document boundary, plus the end
    assert capi.lexical_slice_table_bytes(30_000, 1_000_000) == 30_000 * (245 + 1) * 4
    assert capi.lexical_slice_table_bytes(7, 4096) == 7 * 2 * 4
    assert capi.lexical_slice_table_bytes(7, 4097) == 7 * 3 * 4
    assert capi.lexical_slice_table_bytes(0, 100) == 0
    assert capi.lexical_slice_table_bytes(7, 0) == 0
    assert capi.lexical_slice_table_bytes(7, 2**31) == 0


def test_empty_work_returns_ok_without_a_gpu(capi):
    # launchers with nothing to do return before touching the device
    capi.launch_similarity(None, capi.F32, 1.0, 0, 384, None, 1, None, 0, None)
    capi.launch_topk(None, 0, 10, 1, None, None, None, None, None, None)
    capi.launch_bm25(None, None, None, None, 0, 100, None)


def test_argument_errors_without_a_gpu(capi):
    with pytest.raises(ValueError, match="exceeds per-tile capacity"):
        capi.launch_topk(1, 5000, 2000, 1, 1, 1, 1, 1, 1, 1)
    with pytest.raises(ValueError, match="exceeds candidate count"):
        capi.launch_topk(1, 50, 100, 1, 1, 1, 1, 1, 1, 1)
    with pytest.raises(ValueError, match="float32, float16 or int8"):
        capi.launch_gather_rescore(1, capi.BINARY, 1.0, 10, 32, 1, 1, 1, 1, 0, 1)
    with pytest.raises(ValueError, match="unknown storage dtype"):
        capi.launch_similarity(1, 9, 1.0, 10, 32, 1, 1, None, 0, 1)
    with pytest.raises(ValueError, match="cosine and dot only"):
        capi.launch_similarity_i8i8(1, 1, 10, 32, 1, 1, 1, None, capi.L2, 1)


def _desc(capi, **kw):
    corpus = capi.store_desc(kw.pop("data", 1 << 20), kw.pop("n", 1000), kw.pop("dim", 64),
                             kw.pop("dtype", capi.F32), 1.0, kw.pop("row_scales", None))
    batch = kw.pop("batch", 2)
    k = kw.pop("k", 10)
    return capi.search_desc(corpus, 1 << 20, batch, k, **kw)


@pytest.mark.parametrize("kw,error,match", [
    (dict(k=0), ValueError, "k must be positive"),
    (dict(k=1001), ValueError, "exceeds corpus size"),
    (dict(n=5000, k=1025), ValueError, "exceeds kernel capacity"),
    (dict(batch=0), ValueError, "batch must be positive"),
    (dict(n=2**31), RuntimeError, "exceeds the supported document count"),
    (dict(metric=7), ValueError, "unknown metric"),
    (dict(dtype=2, int8_mode=1), ValueError, "row scales"),
    (dict(dtype=2, int8_mode=1, row_scales=256, metric=2), ValueError, "cosine and dot only"),
    (dict(rescore_candidates=5), ValueError, "at least k"),
    (dict(rescore_candidates=2000), ValueError, "exceeds corpus size"),
    (dict(n=5000, rescore_candidates=2000), ValueError, "exceeds kernel capacity"),
])
def test_search_validation_without_a_gpu(capi, kw, error, match):
    if "rescore_candidates" in kw:
        kw["rescore"] = capi.store_desc(1 << 21, kw.get("n", 1000), 64, capi.F32)
    with pytest.raises(error, match=match):
        capi.search_workspace_bytes(_desc(capi, **kw))


def test_search_validation_rescore_store(capi):
    with pytest.raises(ValueError, match="must not be binary"):
        capi.search_workspace_bytes(_desc(capi, rescore=capi.store_desc(1 << 21, 1000, 64, capi.BINARY),
                                          rescore_candidates=100))
    with pytest.raises(ValueError, match="fewer documents"):
        capi.search_workspace_bytes(_desc(capi, rescore=capi.store_desc(1 << 21, 999, 64, capi.F32),
                                          rescore_candidates=100))
    with pytest.raises(ValueError, match="lexical index holds fewer"):
        capi.search_workspace_bytes(_desc(capi, query_terms=1 << 22, lexical_stride=4, lex_offsets=1,
                                          lex_docs=1, lex_weights=1, lex_doc_count=10,
                                          lex_vocab_size=100))


def test_lexical_slice_table_validation(capi):
    lexical = dict(query_terms=1 << 22, lexical_stride=4, lex_offsets=1, lex_docs=1, lex_weights=1,
                   lex_vocab_size=100, lex_slice_table=1 << 23)
    with pytest.raises(ValueError, match="slice table needs ZCGVS_SEARCH_SORTED_POSTINGS"):
        capi.search_workspace_bytes(_desc(capi, lex_doc_count=1000, **lexical))
    with pytest.raises(ValueError, match="at most 2\\^31 - 1 documents"):
        capi.search_workspace_bytes(_desc(capi, lex_doc_count=2**31, flags=capi.SEARCH_SORTED_POSTINGS,
                                          **lexical))
    assert capi.search_workspace_bytes(_desc(capi, lex_doc_count=1000, flags=capi.SEARCH_SORTED_POSTINGS,
                                             **lexical)) > 0
    with pytest.raises(ValueError, match="empty index"):
        capi.build_lexical_slice_table(1, 1, 0, 1000, 1)
    with pytest.raises(ValueError, match="null device pointer"):
        capi.build_lexical_slice_table(None, 1, 10, 1000, 1)


def test_workspace_sizes(capi):
    # the per-vector int8 configuration: 10M x 768, 256 queries, k = 100
    size = capi.search_workspace_bytes(_desc(capi, n=10_000_000, dim=768, dtype=capi.I8, batch=256,
                                             k=100, int8_mode=1, row_scales=256))
    assert 0 < size < 1 << 30


def test_descriptors_keep_their_buffers_alive(capi):
    # A descriptor stores raw device addresses. The buffers passed to the descriptor builders
    # must stay referenced by the descriptor, or a temporary DeviceArray would be freed
    # (hipFree) before the kernels that read it run.
    import gc
    import weakref

    class Owner:  # stands in for a DeviceArray: any object with a device address
        def __init__(self, address):
            self.address = address

        def __int__(self):
            return self.address

    refs = []

    def make(address):
        owner = Owner(address)
        refs.append(weakref.ref(owner))
        return owner

    corpus = capi.store_desc(make(1 << 20), 100, 64, capi.F32, 1.0, make(1 << 21))
    rescore = capi.store_desc(make(1 << 22), 100, 64, capi.F16)
    desc = capi.search_desc(corpus, make(1 << 23), 1, 10, rescore=rescore, rescore_candidates=20,
                            mask=make(1 << 24), query_terms=make(1 << 25), lex_offsets=make(1 << 26),
                            lex_docs=make(1 << 27), lex_weights=make(1 << 28))
    del corpus, rescore
    gc.collect()
    assert all(r() is not None for r in refs), "a descriptor dropped a buffer it points at"
    assert desc.corpus.data == 1 << 20 and desc.rescore.data == 1 << 22
    del desc
    gc.collect()
    assert all(r() is None for r in refs)


@pytest.mark.parametrize("n,batch,k,stride", [
    (10_000_000, 256, 100, 32),     # the per-vector int8 10M x 768 configuration
    (1_000_000, 256, 100, 8),       # a smaller corpus samples every 8th block (>= 4 per workgroup)
    (1_000_003, 64, 100, 8),        # ragged tail block
])
def test_sketch_plan_samples_then_scans_everything(capi, n, batch, k, stride):
    # A sketch-planned search (per-vector int8 on the matrix cores, large corpus): a sketch
    # phase over every stride-th 64-row block, then one threshold scan of the whole corpus.
    kw = dict(n=n, dim=768, dtype=2, batch=batch, k=k, int8_mode=1, row_scales=1 << 24)
    rows = capi.search_phase_rows(_desc(capi, **kw))
    blocks = (n + 63) // 64
    sampled = (blocks + stride - 1) // stride
    last_sampled = (blocks - 1) % stride == 0
    assert rows == [sampled * 64 - ((blocks * 64 - n) if last_sampled else 0), n]


@pytest.mark.parametrize("n,batch,k,stride,sketched", [
    (50_000_000, 32, 1000, 64, True),   # the binary 50M x 1024 configuration's Hamming stage
    (2_000_003, 20, 100, 4, True),      # every 4th 384-row block, ragged tail
    (50_000_000, 64, 1000, 64, True),   # two sets of 32: sketch launches per set
    (50_000_000, 128, 1000, 64, True),  # more than 64: sketched set by set, the full scan on the tile kernel
    (1_000_000, 32, 100, 0, False),     # under 4 sampled blocks per workgroup: threshold phases
])
def test_binary_sketch_plan(capi, n, batch, k, stride, sketched):
    # A binary search takes the sketch plan (the streaming kernel's sketch launches, one per set of
    # 32 queries) with 384-row blocks of 1024-bit rows, when every workgroup sees 4 sampled blocks.
    rows = capi.search_phase_rows(_desc(capi, n=n, dim=1024, dtype=capi.BINARY, batch=batch, k=k))
    if sketched:
        blocks = (n + 383) // 384
        sampled = (blocks + stride - 1) // stride
        last_sampled = (blocks - 1) % stride == 0
        assert rows == [sampled * 384 - ((blocks * 384 - n) if last_sampled else 0), n]
    else:
        assert len(rows) >= 3 and sum(rows) == n


@pytest.mark.parametrize("n,dtype,int8_mode,batch,k", [
    (100_000, 2, 1, 256, 100),      # per-vector int8 MFMA path below the sketch plan's size
    (1_000_000, 0, 0, 64, 10),      # float32 VALU path
    (123_457, 1, 0, 5, 40),         # ragged tail block
])
def test_phase_rows_cover_the_corpus_once(capi, n, dtype, int8_mode, batch, k):
    kw = dict(n=n, dim=768 if dtype == 2 else 384, dtype=dtype, batch=batch, k=k)
    if int8_mode:
        kw.update(int8_mode=1, row_scales=1 << 24)
    rows = capi.search_phase_rows(_desc(capi, **kw))
    assert len(rows) >= 2
    assert sum(rows) == n  # the phases partition the corpus
    assert all(r > 0 for r in rows)


@pytest.mark.parametrize("n,dtype,int8_mode,batch,k", [
    (123_457, 1, 0, 3, 10),         # float16, three queries
    (1_000_000, 0, 0, 1, 32),       # float32
    (10_000_000, 2, 1, 4, 100),     # per-vector int8 below the MFMA batch, merged in groups
    (50_000_000, 3, 0, 1, 1000),    # binary, the widest selection the merges take
])
def test_small_batches_scan_in_one_pass(capi, n, dtype, int8_mode, batch, k):
    kw = dict(n=n, dim=768 if dtype == 2 else 384, dtype=dtype, batch=batch, k=k)
    if int8_mode:
        kw.update(int8_mode=1, row_scales=1 << 24)
    assert capi.search_phase_rows(_desc(capi, **kw)) == [n]


@pytest.mark.parametrize("with_roctx", [False, True])
def test_trace_ranges_compile_in_and_out(tmp_path, with_roctx):
    # include/zcgvs/core/trace_range.hpp: empty ranges by default, roctx push/pop with
    # ZCGVS_WITH_ROCTX (the counterpart of the reference's NVTX ranges)
    import shutil
    import subprocess
    if shutil.which("g++") is None:
        pytest.skip("no host C++ compiler")
    source = tmp_path / "ranges.cpp"
    source.write_text('#include "zcgvs/core/trace_range.hpp"\nint f() { ZCGVS_TRACE_RANGE("zcgvs::test"); return 1; }\n')
    flags = ["-DZCGVS_WITH_ROCTX", "-I/opt/rocm/include"] if with_roctx else []
    if with_roctx and not Path("/opt/rocm/include/rocprofiler-sdk-roctx/roctx.h").exists():
        pytest.skip("roctx header not installed")
    result = subprocess.run(["g++", "-std=c++17", "-fsyntax-only", f"-I{ROOT / 'include'}", *flags, str(source)],
                            capture_output=True, text=True)
    assert result.returncode == 0, result.stderr


def test_name_helpers_follow_the_reference(tmp_path):
    # metricFromName / scalarTypeFromName keep the reference's aliases and defaults
    # (include/zcgvs/core/metric.hpp:26-34, scalar_type.hpp:56-67: unknown names fall back to
    # cosine / float32); the *Strict variants reject unknown names instead.
    import shutil
    import subprocess
    if shutil.which("g++") is None:
        pytest.skip("no host C++ compiler")
    source = tmp_path / "names.cpp"
    source.write_text(r"""
#include <cstdio>
#include <stdexcept>
#include "zcgvs/core/metric.hpp"
#include "zcgvs/core/scalar_type.hpp"
using namespace zcgvs;
static int failures = 0;
#define CHECK(x) do { if (!(x)) { std::printf("failed: %s\n", #x); ++failures; } } while (0)
template <typename F> static bool throws(F f) { try { f(); } catch (const std::invalid_argument&) { return true; } return false; }
int main() {
    CHECK(metricFromName("dot") == Metric::DotProduct);
    CHECK(metricFromName("dotproduct") == Metric::DotProduct);
    CHECK(metricFromName("ip") == Metric::DotProduct);
    CHECK(metricFromName("l2") == Metric::L2);
    CHECK(metricFromName("euclidean") == Metric::L2);
    CHECK(metricFromName("cosine") == Metric::Cosine);
    CHECK(metricFromName("dot_product") == Metric::Cosine);
    CHECK(metricFromName("") == Metric::Cosine);
    CHECK(metricFromNameStrict("ip") == Metric::DotProduct);
    CHECK(metricFromNameStrict("cosine") == Metric::Cosine);
    CHECK(throws([] { metricFromNameStrict("cosin"); }));
    CHECK(scalarTypeFromName("float16") == ScalarType::Float16);
    CHECK(scalarTypeFromName("fp16") == ScalarType::Float16);
    CHECK(scalarTypeFromName("half") == ScalarType::Float16);
    CHECK(scalarTypeFromName("int8") == ScalarType::Int8);
    CHECK(scalarTypeFromName("i8") == ScalarType::Int8);
    CHECK(scalarTypeFromName("binary") == ScalarType::Binary);
    CHECK(scalarTypeFromName("bin") == ScalarType::Binary);
    CHECK(scalarTypeFromName("b1") == ScalarType::Binary);
    CHECK(scalarTypeFromName("float32") == ScalarType::Float32);
    CHECK(scalarTypeFromName("whatever") == ScalarType::Float32);
    CHECK(scalarTypeFromNameStrict("f32") == ScalarType::Float32);
    CHECK(scalarTypeFromNameStrict("b1") == ScalarType::Binary);
    CHECK(throws([] { scalarTypeFromNameStrict("int4"); }));
    CHECK(std::string(metricName(metricFromName("ip"))) == "dot");
    CHECK(std::string(scalarName(scalarTypeFromName("half"))) == "float16");
    return failures == 0 ? 0 : 1;
}
""")
    exe = tmp_path / "names"
    built = subprocess.run(["g++", "-std=c++17", f"-I{ROOT / 'include'}", str(source), "-o", str(exe)],
                           capture_output=True, text=True)
    assert built.returncode == 0, built.stderr
    ran = subprocess.run([str(exe)], capture_output=True, text=True)
    assert ran.returncode == 0, ran.stdout
