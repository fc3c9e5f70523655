// Results and timings (include/zcgvs/engine/search_hit.hpp, search_response.hpp).
#pragma once

#include <string>
#include <vector>

namespace zcgvs {

struct SearchHit {
    std::string doc_id;
    std::string text;
    float similarity = 0.0f;
    float rerank_score = 0.0f;
    int corpus_index = -1;
};

struct Candidate {
    std::string doc_id;
    float score = 0.0f;
    int corpus_index = -1;
};

// Host stages are wall clock; search_gpu_ms comes from events bracketing the device pipeline.
struct SearchTiming {
    double tokenize_ms = 0.0;
    double embed_ms = 0.0;
    double search_gpu_ms = 0.0;
    double copy_ms = 0.0;
    double rerank_ms = 0.0;
    double total_ms = 0.0;
    int batch = 1;
    bool graph_replay = false;
};

struct SearchResponse {
    std::vector<SearchHit> hits;
    SearchTiming timing;
};

struct BatchSearchResponse {
    std::vector<std::vector<SearchHit>> results;
    SearchTiming timing;
};

}  // namespace zcgvs
