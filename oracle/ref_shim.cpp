// extern "C" entry points over the reference's own CPU path, tests/cpp/cpu_reference.hpp, which
// this file includes from the reference checkout (see Makefile). Used only to check the oracle
// restatement and, optionally, as the CPU baseline. TEST INFRASTRUCTURE ONLY.
#include <cstdint>
#include <vector>

#include "cpu_reference.hpp"

extern "C" {

// tests/cpp/cpu_reference.hpp:12-24
void ref_cosine_similarity(const float* corpus, int doc_count, int dim, const float* query,
                           float* out) {
    const std::vector<float> c(corpus, corpus + static_cast<std::size_t>(doc_count) * dim);
    const std::vector<float> q(query, query + dim);
    const std::vector<float> s = zcgvs::testing::cpuCosineSimilarity(c, doc_count, dim, q);
    for (int i = 0; i < doc_count; ++i) {
        out[i] = s[static_cast<std::size_t>(i)];
    }
}

// tests/cpp/cpu_reference.hpp:26-34
void ref_topk_indices(const float* scores, int count, int k, int* out) {
    const std::vector<float> s(scores, scores + count);
    const std::vector<int> idx = zcgvs::testing::cpuTopKIndices(s, k);
    for (int i = 0; i < k; ++i) {
        out[i] = idx[static_cast<std::size_t>(i)];
    }
}

// tests/cpp/cpu_reference.hpp:36-49 (one row)
void ref_l2_normalize(float* values, int dim) {
    std::vector<float> v(values, values + dim);
    zcgvs::testing::l2Normalize(v, 0, dim);
    for (int j = 0; j < dim; ++j) {
        values[j] = v[static_cast<std::size_t>(j)];
    }
}

// tests/cpp/cpu_reference.hpp:51-62
void ref_quantize_dequantize_i8(const float* values, int count, float scale, float* out) {
    const std::vector<float> v(values, values + count);
    const std::vector<float> r = zcgvs::testing::cpuQuantizeDequantizeInt8(v, scale);
    for (int i = 0; i < count; ++i) {
        out[i] = r[static_cast<std::size_t>(i)];
    }
}

// tests/cpp/cpu_reference.hpp:64-78
void ref_pack_binary(const float* matrix, int rows, int dim, std::uint32_t* out) {
    const std::vector<float> m(matrix, matrix + static_cast<std::size_t>(rows) * dim);
    const std::vector<std::uint32_t> p = zcgvs::testing::cpuPackBinary(m, rows, dim);
    for (std::size_t i = 0; i < p.size(); ++i) {
        out[i] = p[i];
    }
}

// tests/cpp/cpu_reference.hpp:80-90
int ref_hamming(const std::uint32_t* a, const std::uint32_t* b, int words) {
    return zcgvs::testing::cpuHamming(a, b, words);
}

}  // extern "C"
