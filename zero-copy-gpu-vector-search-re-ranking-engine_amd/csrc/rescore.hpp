// Internal interfaces between the fused search and the rescore / lexical / conversion kernels.
#pragma once

#include "common.hpp"

namespace zcgvs_hip {

// Exact score of the corpus row named by each candidate key ([batch, candidate_count] selection
// keys; key 0 = no candidate) against float32 query q, written back as (score, corpus id) keys
// (0 for "no candidate").
int launchRescoreKeys(const void* corpus, int dtype, float scale, int doc_count, int dim,
                      const float* queries, int batch, const std::uint64_t* candidate_keys,
                      int candidate_count, int metric, std::uint64_t* out_keys,
                      hipStream_t stream);

// BM25 over the CSR index for [batch, term_stride] term slots into lexical [batch, doc_count]
// (every entry written), and the per-query maximum max(0, max_i lexical) into lexical_max
// [batch]. With `bounds` (lexicalBoundsBytes of scratch; each term's postings ascending by
// document, one per document) the postings are read in document-range slices, whose bounds come
// from `slice_table` (zcgvs_build_lexical_slice_table of an index of index_doc_count documents)
// when it is not null; with null bounds the postings are scattered slot by slot, in any order.
std::size_t lexicalBoundsBytes(int batch, int term_stride, int doc_count);
int launchLexicalScores(const std::int64_t* offsets, const int* docs, const float* weights,
                        int vocab_size, const int* query_terms, int term_stride, int batch,
                        int doc_count, float* lexical, float* lexical_max, std::int64_t* bounds,
                        const std::uint32_t* slice_table, std::int64_t index_doc_count,
                        hipStream_t stream);

// Per-row int8 quantization used for the queries of the per-vector int8 mode.
int launchQuantizeRows(const float* src, int rows, int dim, std::int8_t* dst, float* scales,
                       hipStream_t stream);

}  // namespace zcgvs_hip
