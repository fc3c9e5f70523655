// Per-request knobs (include/zcgvs/engine/search_options.hpp); sentinel values fall back to the
// EngineConfig.
#pragma once

#include <vector>

#include "zcgvs/core/metric.hpp"
#include "zcgvs/search/search_params.hpp"

namespace zcgvs {

struct SearchOptions {
    int top_k = 0;       // <= 0: EngineConfig::default_top_k
    int candidates = 0;  // <= 0: EngineConfig::default_candidates
    bool use_config_metric = true;
    Metric metric = Metric::Cosine;
    std::vector<int> allow;       // corpus indices the search is restricted to; empty = all
    int rescore_candidates = -1;  // < 0: EngineConfig::rescore_candidates
    float dense_weight = -1.0f;   // < 0: EngineConfig::dense_weight
    bool hybrid = false;
    bool rerank = true;
    bool use_config_backend = true;
    SimilarityBackend backend = SimilarityBackend::Custom;
    bool use_config_graphs = true;
    bool use_graph = false;
};

}  // namespace zcgvs
