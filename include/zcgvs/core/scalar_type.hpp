// Storage precisions of a corpus (include/zcgvs/core/scalar_type.hpp:12-40). The codes are the
// ZCVE file's dtype field.
#pragma once

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

namespace zcgvs {

enum class ScalarType : std::int32_t {
    Float32 = 0,
    Float16 = 1,
    Int8 = 2,
    Binary = 3,
};

// 32-bit words of one sign-packed row: bit b of word w is dimension 32 w + b.
inline std::size_t binaryWords(int dim) { return static_cast<std::size_t>((dim + 31) / 32); }

inline std::size_t rowBytes(ScalarType type, int dim) {
    switch (type) {
        case ScalarType::Float32: return static_cast<std::size_t>(dim) * 4;
        case ScalarType::Float16: return static_cast<std::size_t>(dim) * 2;
        case ScalarType::Int8: return static_cast<std::size_t>(dim);
        case ScalarType::Binary: return binaryWords(dim) * 4;
    }
    throw std::invalid_argument("zcgvs: unknown scalar type");
}

inline bool isQuantized(ScalarType type) {
    return type == ScalarType::Int8 || type == ScalarType::Binary;
}

inline const char* scalarName(ScalarType type) {
    switch (type) {
        case ScalarType::Float32: return "float32";
        case ScalarType::Float16: return "float16";
        case ScalarType::Int8: return "int8";
        case ScalarType::Binary: return "binary";
    }
    return "unknown";
}

inline ScalarType scalarTypeFromCode(std::int32_t code) {
    if (code < 0 || code > 3) {
        throw std::runtime_error("zcgvs: unsupported embedding dtype code " + std::to_string(code));
    }
    return static_cast<ScalarType>(code);
}

}  // namespace zcgvs
