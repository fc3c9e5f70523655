// Plugin seam for text queries (the role of include/zcgvs/embed/query_embedder.hpp): turns a
// query into a dim-long float32 vector, and optionally into the term ids the lexical index uses.
#pragma once

#include <string>
#include <vector>

namespace zcgvs {

class QueryEmbedder {
public:
    virtual ~QueryEmbedder() = default;
    virtual std::vector<float> embed(const std::string& text) const = 0;
    // Term ids for the hybrid stage (deduplicated by the engine); empty when not supported.
    virtual std::vector<int> lexicalTerms(const std::string& /*text*/) const { return {}; }
};

}  // namespace zcgvs
