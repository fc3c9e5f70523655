// On-disk layouts of the reference's artifacts (include/zcgvs/data/binary_format.hpp:12-62),
// little-endian, kept byte-compatible so files written by the reference's Python tools load here
// and files written here load there (version 3 excepted, below).
//
//   ZCVE embeddings  magic 'ZCVE', u32 version, u32 flags (bit 0: rows L2-normalized),
//                    i64 doc_count, i32 dim, i32 dtype (0 f32, 1 f16, 2 int8, 3 binary),
//                    version >= 2: f32 scale (matrix-wide int8 scale), i32 row_stride,
//                    then doc_count * row_stride bytes of rows.
//                    version 3 (this build's extension): flags bit 1 marks int8 rows with a
//                    per-row scale each; doc_count f32 scales follow the rows.
//   ZCVM metadata    magic 'ZCVM', u32 version 1, i64 doc_count, then per document
//                    u32 id_len, id bytes, u32 text_len, text bytes (UTF-8).
//   ZCVL lexical     magic 'ZCVL', u32 version 1, i64 doc_count, i32 vocab_size, i64 nnz,
//                    f32 k1, f32 b, f32 avg_doc_len, (vocab_size + 1) i64 term offsets,
//                    nnz i32 posting docs, nnz f32 posting weights (full BM25 contribution).
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <istream>
#include <ostream>
#include <stdexcept>
#include <string>

namespace zcgvs {

namespace format {

inline constexpr char kEmbeddingMagic[4] = {'Z', 'C', 'V', 'E'};
inline constexpr char kMetadataMagic[4] = {'Z', 'C', 'V', 'M'};
inline constexpr char kLexicalMagic[4] = {'Z', 'C', 'V', 'L'};

inline constexpr std::uint32_t kEmbeddingVersion = 2;        // what the reference writes
inline constexpr std::uint32_t kEmbeddingRowScaleVersion = 3;
inline constexpr std::uint32_t kMetadataVersion = 1;
inline constexpr std::uint32_t kLexicalVersion = 1;

inline constexpr std::uint32_t kFlagNormalized = 1u << 0;
inline constexpr std::uint32_t kFlagRowScales = 1u << 1;

}  // namespace format

// Sequential little-endian reads with end-of-stream detection.
class FormatReader {
public:
    explicit FormatReader(std::istream& in) : in_(in) {}

    void bytes(void* out, std::size_t count) {
        in_.read(static_cast<char*>(out), static_cast<std::streamsize>(count));
        if (static_cast<std::size_t>(in_.gcount()) != count) {
            throw std::runtime_error("zcgvs binary: unexpected end of stream");
        }
    }

    template <typename T>
    T value() {
        T out{};
        bytes(&out, sizeof(T));
        return out;
    }

    std::string text(std::size_t length) {
        std::string out(length, '\0');
        if (length > 0) {
            bytes(&out[0], length);
        }
        return out;
    }

    void magic(const char (&expected)[4]) {
        char seen[4];
        bytes(seen, sizeof(seen));
        if (std::memcmp(seen, expected, sizeof(seen)) != 0) {
            throw std::runtime_error("zcgvs binary: magic mismatch");
        }
    }

private:
    std::istream& in_;
};

class FormatWriter {
public:
    explicit FormatWriter(std::ostream& out) : out_(out) {}

    void bytes(const void* data, std::size_t count) {
        out_.write(static_cast<const char*>(data), static_cast<std::streamsize>(count));
        if (!out_) {
            throw std::runtime_error("zcgvs binary: write failed");
        }
    }

    template <typename T>
    void value(T v) {
        bytes(&v, sizeof(T));
    }

    void text(const std::string& s) {
        value<std::uint32_t>(static_cast<std::uint32_t>(s.size()));
        bytes(s.data(), s.size());
    }

private:
    std::ostream& out_;
};

}  // namespace zcgvs
