// The device-resident corpus matrix (include/zcgvs/data/embedding_store.hpp): rows at the file's
// precision, uploaded once and never per query. Adds the per-row int8 scale array the per-vector
// int8 mode needs (s_r = max|x_r| / 127, codes rint(x * (1 / s_r)) clamped to +-127).
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>

#include "zcgvs/core/device_buffer.hpp"
#include "zcgvs/core/scalar_type.hpp"

namespace zcgvs {

class EmbeddingStore {
public:
    EmbeddingStore() = default;

    // ZCVE v1/v2 (and v3 with per-row scales). The rows stream through pinned staging in
    // fixed-size chunks, so the host never holds the whole matrix.
    static EmbeddingStore loadFromFile(const std::string& path);

    // Builds a store from a host float32 matrix, converting on the device (src/data/
    // embedding_store.cpp:87-132): fp16 by round-to-nearest-even, int8 with the matrix-wide
    // `scale` (1.0 when not positive), binary by sign packing.
    static EmbeddingStore fromHostMatrix(const float* host_float32, std::int64_t doc_count, int dim,
                                         ScalarType dtype, float scale, bool normalized);

    // int8 rows with one scale per row (the per-vector mode), quantized on the device.
    static EmbeddingStore fromHostMatrixPerRow(const float* host_float32, std::int64_t doc_count,
                                               int dim, bool normalized);

    // Writes the store as ZCVE (version 2, or 3 when it carries per-row scales).
    void saveToFile(const std::string& path) const;

    const void* deviceData() const { return rows_.data(); }
    std::int64_t docCount() const { return doc_count_; }
    int dim() const { return dim_; }
    bool normalized() const { return normalized_; }
    ScalarType dtype() const { return dtype_; }
    float scale() const { return scale_; }
    std::int64_t capacity() const { return capacity_; }
    std::size_t deviceBytes() const { return rows_.bytes() + row_scales_.bytes(); }
    std::size_t rowStride() const { return rowBytes(dtype_, dim_); }
    bool hasRowScales() const { return per_row_; }
    const float* deviceRowScales() const { return per_row_ ? row_scales_.data() : nullptr; }

    // Appends float32 rows converted to the store's precision; the row buffer grows
    // geometrically (src/data/embedding_store.cpp:134-192). Synchronizes `stream`.
    void append(const float* host_float32, std::int64_t add_count, zcgvs_stream_t stream);

private:
    void reserve(std::int64_t docs, zcgvs_stream_t stream);
    void convertRows(const float* host_float32, std::int64_t first, std::int64_t count,
                     zcgvs_stream_t stream);

    DeviceBuffer<std::uint8_t> rows_;
    DeviceBuffer<float> row_scales_;
    std::int64_t doc_count_ = 0;
    std::int64_t capacity_ = 0;
    int dim_ = 0;
    bool normalized_ = false;
    bool per_row_ = false;
    ScalarType dtype_ = ScalarType::Float32;
    float scale_ = 1.0f;
};

}  // namespace zcgvs
