// LexicalIndex: ZCVL load/save with CSR validation (src/data/lexical_index.cpp:14-71).
#include "zcgvs/data/lexical_index.hpp"

#include <fstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "zcgvs/data/binary_format.hpp"

namespace zcgvs {

namespace {

// Offsets start at 0, never decrease and end at nnz; every posting names a document in range.
// Returns whether every term's postings are strictly ascending by document (the layout the
// reference's builder writes, which the device BM25 stage reads in document-range slices).
bool validateCsr(const std::int64_t* offsets, const int* docs, int vocab_size, std::int64_t nnz,
                 std::int64_t doc_count) {
    if (offsets[0] != 0 || offsets[vocab_size] != nnz) {
        throw std::runtime_error("zcgvs: lexical index CSR offsets are inconsistent with nnz");
    }
    for (int t = 0; t < vocab_size; ++t) {
        if (offsets[t + 1] < offsets[t]) {
            throw std::runtime_error("zcgvs: lexical index CSR offsets are not ascending");
        }
    }
    for (std::int64_t i = 0; i < nnz; ++i) {
        if (docs[i] < 0 || docs[i] >= doc_count) {
            throw std::runtime_error("zcgvs: lexical index posting names a document out of range");
        }
    }
    bool sorted = true;
    for (int t = 0; t < vocab_size && sorted; ++t) {
        for (std::int64_t i = offsets[t] + 1; i < offsets[t + 1]; ++i) {
            if (docs[i] <= docs[i - 1]) {
                sorted = false;
                break;
            }
        }
    }
    return sorted;
}

void upload(const void* host, void* device, std::size_t bytes) {
    if (bytes > 0) {
        check(zcgvs_memcpy_h2d(device, host, bytes, nullptr));
    }
}

}  // namespace

LexicalIndex LexicalIndex::fromHostCsr(const std::int64_t* offsets, const int* docs, const float* weights,
                                       std::int64_t doc_count, int vocab_size, float k1, float b,
                                       float average_doc_length) {
    if (offsets == nullptr || doc_count <= 0 || vocab_size <= 0) {
        throw std::invalid_argument("zcgvs: lexical index needs documents, a vocabulary and offsets");
    }
    const std::int64_t nnz = offsets[vocab_size];
    if (nnz < 0 || (nnz > 0 && (docs == nullptr || weights == nullptr))) {
        throw std::invalid_argument("zcgvs: lexical index postings are missing");
    }
    const bool sorted = validateCsr(offsets, docs, vocab_size, nnz, doc_count);
    LexicalIndex index;
    index.sorted_postings_ = sorted;
    index.doc_count_ = doc_count;
    index.vocab_size_ = vocab_size;
    index.posting_count_ = nnz;
    index.k1_ = k1;
    index.b_ = b;
    index.average_doc_length_ = average_doc_length;
    index.offsets_.allocate(static_cast<std::size_t>(vocab_size) + 1);
    upload(offsets, index.offsets_.data(), index.offsets_.bytes());
    if (nnz > 0) {
        index.posting_docs_.allocate(static_cast<std::size_t>(nnz));
        index.posting_weights_.allocate(static_cast<std::size_t>(nnz));
        upload(docs, index.posting_docs_.data(), index.posting_docs_.bytes());
        upload(weights, index.posting_weights_.data(), index.posting_weights_.bytes());
    }
    // Sorted postings get the slice table the device BM25 stage reads its slice bounds from.
    const std::size_t table_bytes = zcgvs_lexical_slice_table_bytes(vocab_size, doc_count);
    if (sorted && nnz > 0 && table_bytes > 0) {
        index.slice_table_.allocate(table_bytes / sizeof(std::uint32_t));
        check(zcgvs_build_lexical_slice_table(index.offsets_.data(), index.posting_docs_.data(), vocab_size,
                                              doc_count, index.slice_table_.data(), nullptr));
    }
    check(zcgvs_device_synchronize());
    return index;
}

LexicalIndex LexicalIndex::loadFromFile(const std::string& path) {
    std::ifstream in(path, std::ios::binary);
    if (!in) {
        throw std::runtime_error("zcgvs: cannot open lexical index '" + path + "'");
    }
    FormatReader reader(in);
    reader.magic(format::kLexicalMagic);
    const auto version = reader.value<std::uint32_t>();
    if (version != format::kLexicalVersion) {
        throw std::runtime_error("zcgvs: unsupported lexical index version " + std::to_string(version));
    }
    const auto doc_count = reader.value<std::int64_t>();
    const auto vocab_size = reader.value<std::int32_t>();
    const auto nnz = reader.value<std::int64_t>();
    const auto k1 = reader.value<float>();
    const auto b = reader.value<float>();
    const auto avgdl = reader.value<float>();
    if (doc_count <= 0 || vocab_size <= 0 || nnz < 0) {
        throw std::runtime_error("zcgvs: lexical index header describes an empty index");
    }
    std::vector<std::int64_t> offsets(static_cast<std::size_t>(vocab_size) + 1);
    reader.bytes(offsets.data(), offsets.size() * sizeof(std::int64_t));
    if (offsets.front() != 0 || offsets.back() != nnz) {
        throw std::runtime_error("zcgvs: lexical index CSR offsets are inconsistent with nnz");
    }
    std::vector<int> docs(static_cast<std::size_t>(nnz));
    std::vector<float> weights(static_cast<std::size_t>(nnz));
    reader.bytes(docs.data(), docs.size() * sizeof(int));
    reader.bytes(weights.data(), weights.size() * sizeof(float));
    return fromHostCsr(offsets.data(), docs.data(), weights.data(), doc_count, vocab_size, k1, b, avgdl);
}

void LexicalIndex::saveToFile(const std::string& path) const {
    std::ofstream out(path, std::ios::binary);
    if (!out) {
        throw std::runtime_error("zcgvs: cannot create lexical index '" + path + "'");
    }
    std::vector<std::int64_t> offsets(static_cast<std::size_t>(vocab_size_) + 1);
    std::vector<int> docs(static_cast<std::size_t>(posting_count_));
    std::vector<float> weights(static_cast<std::size_t>(posting_count_));
    offsets_.copyToHost(offsets.data(), offsets.size(), nullptr);
    if (posting_count_ > 0) {
        posting_docs_.copyToHost(docs.data(), docs.size(), nullptr);
        posting_weights_.copyToHost(weights.data(), weights.size(), nullptr);
    }
    check(zcgvs_device_synchronize());
    FormatWriter writer(out);
    writer.bytes(format::kLexicalMagic, 4);
    writer.value<std::uint32_t>(format::kLexicalVersion);
    writer.value<std::int64_t>(doc_count_);
    writer.value<std::int32_t>(vocab_size_);
    writer.value<std::int64_t>(posting_count_);
    writer.value<float>(k1_);
    writer.value<float>(b_);
    writer.value<float>(average_doc_length_);
    writer.bytes(offsets.data(), offsets.size() * sizeof(std::int64_t));
    writer.bytes(docs.data(), docs.size() * sizeof(int));
    writer.bytes(weights.data(), weights.size() * sizeof(float));
}

}  // namespace zcgvs
