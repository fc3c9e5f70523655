// Shared device helpers and the status/error plumbing of the C ABI.
//
// Selection key. Every top-k in this library orders 64-bit keys
//     key = (ordered32(score) << 32) | (0xFFFFFFFF - index)
// so that a larger key is a better hit: a higher score first and, among equal scores, the lower
// corpus index first. That is the order std::stable_sort by descending score over ascending
// indices produces (tests/cpp/cpu_reference.hpp:26-34). ordered32 maps float bits to an unsigned
// integer with the same order as the float values; -0.0 is mapped like +0.0 (the comparison
// `a > b` of the reference treats them as equal) and NaN maps to 0, below every other score.
// Keys are unique for distinct indices, so every merge of partial selections is associative and
// deterministic. Key 0 means "no element" (it would need index 0xFFFFFFFF and a NaN score).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "zcgvs_hip.h"

namespace zcgvs_hip {

// --------------------------------------------------------------------------------------------
// Host-side status plumbing
// --------------------------------------------------------------------------------------------
int setError(int status, const std::string& message);
int clearError();
int hipFailure(hipError_t error, const char* what, const char* file, int line);

#define ZCGVS_HIP_RETURN(expr)                                                   \
    do {                                                                         \
        const hipError_t zcgvs_status_ = (expr);                                 \
        if (zcgvs_status_ != hipSuccess) {                                       \
            return ::zcgvs_hip::hipFailure(zcgvs_status_, #expr, __FILE__, __LINE__); \
        }                                                                        \
    } while (0)

#define ZCGVS_LAUNCH_CHECK(what) ZCGVS_HIP_RETURN(hipGetLastError())

inline hipStream_t toStream(zcgvs_stream_t stream) { return reinterpret_cast<hipStream_t>(stream); }

inline bool aligned16(const void* pointer) {
    return (reinterpret_cast<std::uintptr_t>(pointer) & 15u) == 0;
}

__host__ __device__ inline std::size_t binaryWords(int dim) { return static_cast<std::size_t>((dim + 31) / 32); }

__host__ __device__ inline std::size_t rowBytes(int dtype, int dim) {
    switch (dtype) {
        case ZCGVS_DTYPE_F16:
            return static_cast<std::size_t>(dim) * 2;
        case ZCGVS_DTYPE_I8:
            return static_cast<std::size_t>(dim);
        case ZCGVS_DTYPE_BINARY:
            return binaryWords(dim) * 4;
        default:
            return static_cast<std::size_t>(dim) * 4;
    }
}

inline bool validDtype(int dtype) { return dtype >= ZCGVS_DTYPE_F32 && dtype <= ZCGVS_DTYPE_BINARY; }
inline bool validMetric(int metric) { return metric >= ZCGVS_METRIC_COSINE && metric <= ZCGVS_METRIC_L2; }

// Number of compute units of the current device (cached per device).
int deviceComputeUnits();

// Looks up the current device's address of the no-allocation entry point's static scratch
// array (once per device; later calls return at once), so that no lookup happens inside a
// graph capture: zcgvs_graph_begin_capture calls it before the capture starts.
int prepareStaticScratch();

// --------------------------------------------------------------------------------------------
// Device helpers
// --------------------------------------------------------------------------------------------
constexpr int kWave = 64;
constexpr float kMaskedScore = -3.402823466e+38f;  // -FLT_MAX, the reference's masked score

__device__ __forceinline__ std::uint32_t orderedBits(float value) {
    if (value != value) {
        return 0u;  // NaN ranks below everything
    }
    std::uint32_t bits = __float_as_uint(value);
    if (value == 0.0f) {
        bits = 0u;  // -0.0 ranks equal to +0.0
    }
    return (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
}

__device__ __forceinline__ float scoreFromOrdered(std::uint32_t ordered) {
    const std::uint32_t bits = (ordered & 0x80000000u) ? (ordered & 0x7FFFFFFFu) : ~ordered;
    return __uint_as_float(bits);
}

__device__ __forceinline__ std::uint64_t makeKey(float score, std::uint32_t index) {
    return (static_cast<std::uint64_t>(orderedBits(score)) << 32) |
           static_cast<std::uint64_t>(0xFFFFFFFFu - index);
}

__device__ __forceinline__ int keyIndex(std::uint64_t key) {
    return static_cast<int>(0xFFFFFFFFu - static_cast<std::uint32_t>(key));
}

__device__ __forceinline__ float keyScore(std::uint64_t key) {
    return scoreFromOrdered(static_cast<std::uint32_t>(key >> 32));
}

// Writes a selected key as the (index, score) pair of the reference's output; the "no element"
// key becomes the reference's padding pair (-1, -FLT_MAX) (src/cuda/topk.cu:49-50).
__device__ __forceinline__ void writeHit(std::uint64_t key, int* index_out, float* score_out) {
    if (key == 0ull) {
        *index_out = -1;
        *score_out = kMaskedScore;
    } else {
        *index_out = keyIndex(key);
        *score_out = keyScore(key);
    }
}

template <typename T>
__device__ __forceinline__ T waveXor(T value, int mask) {
    return __shfl_xor(value, mask, kWave);
}

// Reduction of a 64-bit value over the 64 lanes of a wavefront with an associative, commutative
// `op`; every lane gets the result. Inside each row of 16 lanes the partners come from
// data-parallel moves (quad permutes, half-row and row mirrors), then a swizzle joins the rows of
// each 32-lane half and a permute joins the halves.
template <typename Op>
__device__ __forceinline__ std::uint64_t waveReduce64(std::uint64_t value, Op op) {
    auto partner = [](std::uint64_t v, auto move) {
        const int lo = move(static_cast<int>(static_cast<std::uint32_t>(v)));
        const int hi = move(static_cast<int>(static_cast<std::uint32_t>(v >> 32)));
        return (static_cast<std::uint64_t>(static_cast<std::uint32_t>(hi)) << 32) | static_cast<std::uint32_t>(lo);
    };
    value = op(value, partner(value, [](int x) { return __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false); }));
    value = op(value, partner(value, [](int x) { return __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false); }));
    value = op(value, partner(value, [](int x) { return __builtin_amdgcn_update_dpp(0, x, 0x141, 0xF, 0xF, false); }));
    value = op(value, partner(value, [](int x) { return __builtin_amdgcn_update_dpp(0, x, 0x140, 0xF, 0xF, false); }));
    value = op(value, partner(value, [](int x) { return __builtin_amdgcn_ds_swizzle(x, 0x401F); }));
    value = op(value, partner(value, [](int x) { return __shfl_xor(x, 32, kWave); }));
    return value;
}

}  // namespace zcgvs_hip
