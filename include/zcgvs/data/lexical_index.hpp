// Device-resident CSR inverted index over term ids (include/zcgvs/data/lexical_index.hpp). Each
// posting weight is the full BM25 contribution of its (term, document) pair, so query-time
// scoring is a scatter-add.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>

#include "zcgvs/core/device_buffer.hpp"

namespace zcgvs {

class LexicalIndex {
public:
    LexicalIndex() = default;

    static LexicalIndex loadFromFile(const std::string& path);

    // From host CSR arrays (offsets [vocab_size + 1], docs/weights [offsets[vocab_size]]),
    // validated like a file.
    static LexicalIndex fromHostCsr(const std::int64_t* offsets, const int* docs, const float* weights,
                                    std::int64_t doc_count, int vocab_size, float k1, float b,
                                    float average_doc_length);

    void saveToFile(const std::string& path) const;

    const std::int64_t* deviceOffsets() const { return offsets_.data(); }
    const int* devicePostingDocs() const { return posting_docs_.data(); }
    const float* devicePostingWeights() const { return posting_weights_.data(); }

    std::int64_t docCount() const { return doc_count_; }
    std::int64_t postingCount() const { return posting_count_; }
    int vocabSize() const { return vocab_size_; }
    float k1() const { return k1_; }
    float b() const { return b_; }
    float averageDocLength() const { return average_doc_length_; }
    // Every term's postings strictly ascending by document (checked at load).
    bool postingsSorted() const { return sorted_postings_; }
    // Per-term posting counts below every 4096-document boundary (zcgvs_build_lexical_slice_table),
    // built at load for sorted postings; null otherwise.
    const std::uint32_t* deviceSliceTable() const { return slice_table_.data(); }
    std::size_t deviceBytes() const {
        return offsets_.bytes() + posting_docs_.bytes() + posting_weights_.bytes() + slice_table_.bytes();
    }

private:
    DeviceBuffer<std::int64_t> offsets_;
    DeviceBuffer<int> posting_docs_;
    DeviceBuffer<float> posting_weights_;
    DeviceBuffer<std::uint32_t> slice_table_;
    std::int64_t doc_count_ = 0;
    std::int64_t posting_count_ = 0;
    int vocab_size_ = 0;
    float k1_ = 1.2f;
    float b_ = 0.75f;
    float average_doc_length_ = 0.0f;
    bool sorted_postings_ = true;
};

}  // namespace zcgvs
