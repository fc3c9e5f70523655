// Flattened [batch, k] selection copied back to the host (include/zcgvs/search/
// search_result.hpp:10-19). An index of -1 marks a padding slot (fewer than k usable documents).
#pragma once

#include <cstddef>
#include <vector>

namespace zcgvs {

struct HostTopK {
    std::vector<int> indices;
    std::vector<float> scores;
    int batch = 0;
    int k = 0;

    std::size_t offset(int query) const {
        return static_cast<std::size_t>(query) * static_cast<std::size_t>(k);
    }
};

}  // namespace zcgvs
