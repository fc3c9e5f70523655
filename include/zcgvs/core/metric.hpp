// Similarity metrics (include/zcgvs/core/metric.hpp:8-12). The numeric codes are part of the
// reference's ABI and configuration files.
#pragma once

#include <cstdint>
#include <stdexcept>
#include <string>

namespace zcgvs {

enum class Metric : std::int32_t {
    Cosine = 0,
    DotProduct = 1,
    L2 = 2,
};

inline const char* metricName(Metric metric) {
    switch (metric) {
        case Metric::Cosine: return "cosine";
        case Metric::DotProduct: return "dot";
        case Metric::L2: return "l2";
    }
    return "unknown";
}

// The reference's lenient parser (include/zcgvs/core/metric.hpp:26-34): "dot", "dotproduct" and
// "ip" name the dot product, "l2" and "euclidean" the L2 distance; every other name, "cosine"
// included, is cosine.
inline Metric metricFromName(const std::string& name) {
    if (name == "dot" || name == "dotproduct" || name == "ip") return Metric::DotProduct;
    if (name == "l2" || name == "euclidean") return Metric::L2;
    return Metric::Cosine;
}

// A strict parser for callers that must reject typos: the names metricFromName accepts, plus
// "cosine", and std::invalid_argument for anything else.
inline Metric metricFromNameStrict(const std::string& name) {
    if (name == "cosine") return Metric::Cosine;
    if (name == "dot" || name == "dotproduct" || name == "ip" || name == "l2" || name == "euclidean") {
        return metricFromName(name);
    }
    throw std::invalid_argument("zcgvs: unknown metric '" + name + "'");
}

}  // namespace zcgvs
