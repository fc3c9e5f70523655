// EmbeddingStore: file load/save, device-side conversion and geometric append
// (src/data/embedding_store.cpp).
#include "zcgvs/data/embedding_store.hpp"

#include <algorithm>
#include <fstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "zcgvs/core/hip_stream.hpp"
#include "zcgvs/data/binary_format.hpp"

namespace zcgvs {

namespace {

constexpr std::size_t kStageBytes = 64u << 20;  // host->device staging chunk

// Streams `total` bytes from `reader` into device memory at `dst` through two pinned chunks, so
// reading chunk i + 1 from the file overlaps the copy of chunk i.
void streamToDevice(FormatReader& reader, std::uint8_t* dst, std::size_t total) {
    if (total == 0) {
        return;
    }
    HipStream stream;
    PinnedBuffer<std::uint8_t> pinned[2];
    HipEvent copied[2];
    const std::size_t chunk = std::min(kStageBytes, total);
    pinned[0].allocate(chunk);
    pinned[1].allocate(chunk);
    std::size_t index = 0;
    for (std::size_t offset = 0; offset < total; offset += chunk, ++index) {
        const int slot = static_cast<int>(index % 2);
        if (index >= 2) {
            copied[slot].synchronize();  // the copy out of this chunk has finished
        }
        const std::size_t count = std::min(chunk, total - offset);
        reader.bytes(pinned[slot].data(), count);
        check(zcgvs_memcpy_h2d(dst + offset, pinned[slot].data(), count, stream.get()));
        copied[slot].record(stream.get());
    }
    stream.synchronize();
}

void readBack(const void* device, void* host, std::size_t bytes) {
    if (bytes > 0) {
        check(zcgvs_memcpy_d2h(host, device, bytes, nullptr));
        check(zcgvs_device_synchronize());
    }
}

}  // namespace

EmbeddingStore EmbeddingStore::loadFromFile(const std::string& path) {
    std::ifstream in(path, std::ios::binary);
    if (!in) {
        throw std::runtime_error("zcgvs: cannot open embedding file '" + path + "'");
    }
    FormatReader reader(in);
    reader.magic(format::kEmbeddingMagic);
    const auto version = reader.value<std::uint32_t>();
    if (version == 0 || version > format::kEmbeddingRowScaleVersion) {
        throw std::runtime_error("zcgvs: unsupported embedding file version " + std::to_string(version));
    }
    const auto flags = reader.value<std::uint32_t>();
    const auto doc_count = reader.value<std::int64_t>();
    const auto dim = reader.value<std::int32_t>();
    const auto dtype_code = reader.value<std::int32_t>();
    if (doc_count <= 0 || dim <= 0) {
        throw std::runtime_error("zcgvs: embedding file reports an empty matrix");
    }

    EmbeddingStore store;
    store.dim_ = dim;
    store.dtype_ = scalarTypeFromCode(dtype_code);
    store.normalized_ = (flags & format::kFlagNormalized) != 0;
    const std::size_t stride = store.rowStride();
    if (version >= 2) {
        store.scale_ = reader.value<float>();
        const auto recorded = reader.value<std::int32_t>();
        if (recorded <= 0 || static_cast<std::size_t>(recorded) != stride) {
            throw std::runtime_error("zcgvs: embedding row stride does not match dtype and dim");
        }
    } else if (isQuantized(store.dtype_)) {
        throw std::runtime_error("zcgvs: quantized embeddings require file version 2");
    }
    store.per_row_ = version >= 3 && (flags & format::kFlagRowScales) != 0;
    if (store.per_row_ && store.dtype_ != ScalarType::Int8) {
        throw std::runtime_error("zcgvs: per-row scales are defined for int8 rows only");
    }
    // A short file is rejected before any device memory is taken for it.
    const std::size_t payload = static_cast<std::size_t>(doc_count) * stride +
                                (store.per_row_ ? static_cast<std::size_t>(doc_count) * sizeof(float) : 0);
    const std::streampos here = in.tellg();
    in.seekg(0, std::ios::end);
    const std::streamoff available = in.tellg() - here;
    in.seekg(here);
    if (available < 0 || static_cast<std::size_t>(available) < payload) {
        throw std::runtime_error("zcgvs binary: unexpected end of stream");
    }

    store.rows_.allocate(static_cast<std::size_t>(doc_count) * stride);
    streamToDevice(reader, store.rows_.data(), static_cast<std::size_t>(doc_count) * stride);
    if (store.per_row_) {
        store.row_scales_.allocate(static_cast<std::size_t>(doc_count));
        streamToDevice(reader, reinterpret_cast<std::uint8_t*>(store.row_scales_.data()),
                       static_cast<std::size_t>(doc_count) * sizeof(float));
    }
    store.doc_count_ = doc_count;
    store.capacity_ = doc_count;
    return store;
}

void EmbeddingStore::saveToFile(const std::string& path) const {
    std::ofstream out(path, std::ios::binary);
    if (!out) {
        throw std::runtime_error("zcgvs: cannot create embedding file '" + path + "'");
    }
    FormatWriter writer(out);
    writer.bytes(format::kEmbeddingMagic, 4);
    writer.value<std::uint32_t>(per_row_ ? format::kEmbeddingRowScaleVersion : format::kEmbeddingVersion);
    writer.value<std::uint32_t>((normalized_ ? format::kFlagNormalized : 0u) |
                                (per_row_ ? format::kFlagRowScales : 0u));
    writer.value<std::int64_t>(doc_count_);
    writer.value<std::int32_t>(dim_);
    writer.value<std::int32_t>(static_cast<std::int32_t>(dtype_));
    writer.value<float>(scale_);
    writer.value<std::int32_t>(static_cast<std::int32_t>(rowStride()));
    const std::size_t chunk_rows = std::max<std::size_t>(1, kStageBytes / rowStride());
    std::vector<std::uint8_t> host;
    for (std::int64_t first = 0; first < doc_count_; first += static_cast<std::int64_t>(chunk_rows)) {
        const std::size_t rows = std::min<std::size_t>(chunk_rows, static_cast<std::size_t>(doc_count_ - first));
        host.resize(rows * rowStride());
        readBack(rows_.data() + static_cast<std::size_t>(first) * rowStride(), host.data(), host.size());
        writer.bytes(host.data(), host.size());
    }
    if (per_row_) {
        std::vector<float> scales(static_cast<std::size_t>(doc_count_));
        readBack(row_scales_.data(), scales.data(), scales.size() * sizeof(float));
        writer.bytes(scales.data(), scales.size() * sizeof(float));
    }
}

void EmbeddingStore::reserve(std::int64_t docs, zcgvs_stream_t stream) {
    if (capacity_ >= docs) {
        return;
    }
    const std::int64_t grown = std::max(docs, capacity_ * 2);
    DeviceBuffer<std::uint8_t> rows(static_cast<std::size_t>(grown) * rowStride());
    if (doc_count_ > 0) {
        check(zcgvs_memcpy_d2d(rows.data(), rows_.data(), static_cast<std::size_t>(doc_count_) * rowStride(), stream));
    }
    DeviceBuffer<float> scales;
    if (per_row_) {
        scales.allocate(static_cast<std::size_t>(grown));
        if (doc_count_ > 0) {
            check(zcgvs_memcpy_d2d(scales.data(), row_scales_.data(),
                                   static_cast<std::size_t>(doc_count_) * sizeof(float), stream));
        }
    }
    check(zcgvs_stream_synchronize(stream));
    rows_ = std::move(rows);
    if (per_row_) {
        row_scales_ = std::move(scales);
    }
    capacity_ = grown;
}

// Rows [first, first + count) from host float32, converted on the device in bounded chunks.
void EmbeddingStore::convertRows(const float* host, std::int64_t first, std::int64_t count,
                                 zcgvs_stream_t stream) {
    const std::size_t row_floats = static_cast<std::size_t>(dim_);
    const std::int64_t chunk_rows =
        std::max<std::int64_t>(1, static_cast<std::int64_t>(kStageBytes / (row_floats * sizeof(float))));
    DeviceBuffer<float> staging;
    if (dtype_ != ScalarType::Float32) {
        staging.allocate(static_cast<std::size_t>(std::min(chunk_rows, count)) * row_floats);
    }
    for (std::int64_t done = 0; done < count; done += chunk_rows) {
        const std::int64_t rows = std::min(chunk_rows, count - done);
        const std::size_t elements = static_cast<std::size_t>(rows) * row_floats;
        const float* src = host + static_cast<std::size_t>(done) * row_floats;
        std::uint8_t* dst = rows_.data() + static_cast<std::size_t>(first + done) * rowStride();
        if (dtype_ == ScalarType::Float32) {
            check(zcgvs_memcpy_h2d(dst, src, elements * sizeof(float), stream));
            continue;
        }
        check(zcgvs_memcpy_h2d(staging.data(), src, elements * sizeof(float), stream));
        switch (dtype_) {
            case ScalarType::Float16:
                check(zcgvs_launch_convert_f32_to_f16(staging.data(), dst, elements, stream));
                break;
            case ScalarType::Int8:
                if (per_row_) {
                    check(zcgvs_launch_quantize_rows_i8(staging.data(), static_cast<int>(rows), dim_,
                                                        reinterpret_cast<std::int8_t*>(dst),
                                                        row_scales_.data() + first + done, stream));
                } else {
                    check(zcgvs_launch_convert_f32_to_i8(staging.data(), dst, elements, scale_, stream));
                }
                break;
            case ScalarType::Binary:
                check(zcgvs_launch_pack_binary(staging.data(), dst, static_cast<int>(rows), dim_, stream));
                break;
            default:
                throw std::invalid_argument("zcgvs: unsupported storage dtype");
        }
        // the staging chunk is reused by the next iteration
        check(zcgvs_stream_synchronize(stream));
    }
    check(zcgvs_stream_synchronize(stream));
}

EmbeddingStore EmbeddingStore::fromHostMatrix(const float* host_float32, std::int64_t doc_count, int dim,
                                              ScalarType dtype, float scale, bool normalized) {
    if (host_float32 == nullptr || doc_count <= 0 || dim <= 0) {
        throw std::invalid_argument("zcgvs: fromHostMatrix requires a non-empty matrix");
    }
    EmbeddingStore store;
    store.dim_ = dim;
    store.dtype_ = dtype;
    store.normalized_ = normalized;
    store.scale_ = (dtype == ScalarType::Int8 && scale > 0.0f) ? scale : 1.0f;
    store.rows_.allocate(static_cast<std::size_t>(doc_count) * store.rowStride());
    store.capacity_ = doc_count;
    HipStream stream;
    store.convertRows(host_float32, 0, doc_count, stream.get());
    store.doc_count_ = doc_count;
    return store;
}

EmbeddingStore EmbeddingStore::fromHostMatrixPerRow(const float* host_float32, std::int64_t doc_count,
                                                    int dim, bool normalized) {
    if (host_float32 == nullptr || doc_count <= 0 || dim <= 0) {
        throw std::invalid_argument("zcgvs: fromHostMatrix requires a non-empty matrix");
    }
    EmbeddingStore store;
    store.dim_ = dim;
    store.dtype_ = ScalarType::Int8;
    store.normalized_ = normalized;
    store.per_row_ = true;
    store.rows_.allocate(static_cast<std::size_t>(doc_count) * store.rowStride());
    store.row_scales_.allocate(static_cast<std::size_t>(doc_count));
    store.capacity_ = doc_count;
    HipStream stream;
    store.convertRows(host_float32, 0, doc_count, stream.get());
    store.doc_count_ = doc_count;
    return store;
}

void EmbeddingStore::append(const float* host_float32, std::int64_t add_count, zcgvs_stream_t stream) {
    if (add_count <= 0) {
        return;
    }
    if (dim_ <= 0) {
        throw std::runtime_error("zcgvs: append requires an initialized store");
    }
    if (host_float32 == nullptr) {
        throw std::invalid_argument("zcgvs: append requires host rows");
    }
    reserve(doc_count_ + add_count, stream);
    convertRows(host_float32, doc_count_, add_count, stream);
    doc_count_ += add_count;
}

}  // namespace zcgvs
