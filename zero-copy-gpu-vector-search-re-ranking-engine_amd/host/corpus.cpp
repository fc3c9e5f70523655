// Corpus: embeddings + ZCVM metadata (src/data/corpus.cpp).
#include "zcgvs/data/corpus.hpp"

#include <fstream>
#include <stdexcept>
#include <string>

#include "zcgvs/data/binary_format.hpp"

namespace zcgvs {

namespace {

void readMetadata(const std::string& path, std::int64_t expected, std::vector<std::string>& ids,
                  std::vector<std::string>& texts) {
    std::ifstream in(path, std::ios::binary);
    if (!in) {
        throw std::runtime_error("zcgvs: cannot open metadata file '" + path + "'");
    }
    FormatReader reader(in);
    reader.magic(format::kMetadataMagic);
    const auto version = reader.value<std::uint32_t>();
    if (version != format::kMetadataVersion) {
        throw std::runtime_error("zcgvs: unsupported metadata version " + std::to_string(version));
    }
    const auto count = reader.value<std::int64_t>();
    if (count != expected) {
        throw std::runtime_error("zcgvs: metadata doc count does not match embeddings");
    }
    ids.reserve(static_cast<std::size_t>(count));
    texts.reserve(static_cast<std::size_t>(count));
    for (std::int64_t i = 0; i < count; ++i) {
        ids.push_back(reader.text(reader.value<std::uint32_t>()));
        texts.push_back(reader.text(reader.value<std::uint32_t>()));
    }
}

}  // namespace

Corpus Corpus::load(const std::string& embeddings_path, const std::string& metadata_path) {
    Corpus corpus;
    corpus.embeddings_ = EmbeddingStore::loadFromFile(embeddings_path);
    const std::int64_t n = corpus.embeddings_.docCount();
    if (metadata_path.empty()) {
        corpus.doc_ids_.reserve(static_cast<std::size_t>(n));
        for (std::int64_t i = 0; i < n; ++i) {
            corpus.doc_ids_.push_back(std::to_string(i));
        }
        corpus.texts_.assign(static_cast<std::size_t>(n), std::string());
    } else {
        readMetadata(metadata_path, n, corpus.doc_ids_, corpus.texts_);
    }
    return corpus;
}

Corpus Corpus::fromStore(EmbeddingStore store, std::vector<std::string> ids, std::vector<std::string> texts) {
    const auto n = static_cast<std::size_t>(store.docCount());
    if (ids.empty()) {
        for (std::size_t i = 0; i < n; ++i) {
            ids.push_back(std::to_string(i));
        }
    }
    if (texts.empty()) {
        texts.assign(n, std::string());
    }
    if (ids.size() != n || texts.size() != n) {
        throw std::invalid_argument("zcgvs: ids and texts must have one entry per document");
    }
    Corpus corpus;
    corpus.embeddings_ = std::move(store);
    corpus.doc_ids_ = std::move(ids);
    corpus.texts_ = std::move(texts);
    return corpus;
}

void Corpus::saveMetadata(const std::string& path, const std::vector<std::string>& ids,
                          const std::vector<std::string>& texts) {
    if (ids.size() != texts.size()) {
        throw std::invalid_argument("zcgvs: ids and texts must have equal length");
    }
    std::ofstream out(path, std::ios::binary);
    if (!out) {
        throw std::runtime_error("zcgvs: cannot create metadata file '" + path + "'");
    }
    FormatWriter writer(out);
    writer.bytes(format::kMetadataMagic, 4);
    writer.value<std::uint32_t>(format::kMetadataVersion);
    writer.value<std::int64_t>(static_cast<std::int64_t>(ids.size()));
    for (std::size_t i = 0; i < ids.size(); ++i) {
        writer.text(ids[i]);
        writer.text(texts[i]);
    }
}

void Corpus::addDocuments(const std::vector<std::string>& ids, const std::vector<std::string>& texts,
                          const float* host_float32, std::int64_t add_count, zcgvs_stream_t stream) {
    if (ids.size() != texts.size() || static_cast<std::int64_t>(ids.size()) != add_count) {
        throw std::runtime_error("zcgvs: addDocuments received mismatched id/text/vector counts");
    }
    if (add_count <= 0) {
        return;
    }
    embeddings_.append(host_float32, add_count, stream);
    doc_ids_.insert(doc_ids_.end(), ids.begin(), ids.end());
    texts_.insert(texts_.end(), texts.begin(), texts.end());
}

}  // namespace zcgvs
