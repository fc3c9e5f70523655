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

inline Metric metricFromName(const std::string& name) {
    if (name == "cosine") return Metric::Cosine;
    if (name == "dot" || name == "dot_product") return Metric::DotProduct;
    if (name == "l2") return Metric::L2;
    throw std::invalid_argument("zcgvs: unknown metric '" + name + "'");
}

}  // namespace zcgvs
