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

// The reference's lenient parser (include/zcgvs/core/scalar_type.hpp:56-67): "float16", "fp16"
// and "half" name Float16, "int8" and "i8" Int8, "binary", "bin" and "b1" Binary; every other
// name is Float32.
inline ScalarType scalarTypeFromName(const std::string& name) {
    if (name == "float16" || name == "fp16" || name == "half") return ScalarType::Float16;
    if (name == "int8" || name == "i8") return ScalarType::Int8;
    if (name == "binary" || name == "bin" || name == "b1") return ScalarType::Binary;
    return ScalarType::Float32;
}

// A strict parser: the names scalarTypeFromName accepts, plus "float32", "fp32" and "f32", and
// std::invalid_argument for anything else.
inline ScalarType scalarTypeFromNameStrict(const std::string& name) {
    if (name == "float32" || name == "fp32" || name == "f32") return ScalarType::Float32;
    const ScalarType type = scalarTypeFromName(name);
    if (type == ScalarType::Float32) {
        throw std::invalid_argument("zcgvs: unknown scalar type '" + name + "'");
    }
    return type;
}

// The ZCVE header's dtype code (include/zcgvs/data/binary_format.hpp), rejecting unknown codes.
inline ScalarType scalarTypeFromCode(std::int32_t code) {
    if (code < 0 || code > 3) {
        throw std::runtime_error("zcgvs: unsupported embedding dtype code " + std::to_string(code));
    }
    return static_cast<ScalarType>(code);
}

}  // namespace zcgvs
