// Embeddings plus per-document ids and passages (include/zcgvs/data/corpus.hpp).
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "zcgvs/data/embedding_store.hpp"

namespace zcgvs {

class Corpus {
public:
    // An empty metadata path gives each document its decimal index as id and an empty passage.
    static Corpus load(const std::string& embeddings_path, const std::string& metadata_path);
    static Corpus fromStore(EmbeddingStore store, std::vector<std::string> ids,
                            std::vector<std::string> texts);

    static void saveMetadata(const std::string& path, const std::vector<std::string>& ids,
                             const std::vector<std::string>& texts);

    const EmbeddingStore& embeddings() const { return embeddings_; }
    std::int64_t size() const { return static_cast<std::int64_t>(doc_ids_.size()); }
    int dim() const { return embeddings_.dim(); }
    const std::string& docId(int index) const { return doc_ids_.at(static_cast<std::size_t>(index)); }
    const std::string& text(int index) const { return texts_.at(static_cast<std::size_t>(index)); }

    void addDocuments(const std::vector<std::string>& ids, const std::vector<std::string>& texts,
                      const float* host_float32, std::int64_t add_count, zcgvs_stream_t stream);

private:
    EmbeddingStore embeddings_;
    std::vector<std::string> doc_ids_;
    std::vector<std::string> texts_;
};

}  // namespace zcgvs
