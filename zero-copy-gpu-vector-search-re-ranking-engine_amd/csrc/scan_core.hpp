// Row-scoring building blocks shared by the materialized scan (zcgvs_launch_similarity) and the
// fused scan-and-select kernels.
//
// Layout. A corpus row of `chunks` 16-byte chunks is read by a group of L consecutive lanes of a
// 64-wide wavefront; lane g of the group reads chunks g, g+L, g+2L, ... so each load instruction
// of the wave fetches 64/L rows x (L x 16 B) contiguous segments. L is chosen so that a lane reads
// at most four chunks per row (eight in the fused VALU scan). The per-lane partial sums are
// combined inside the group by groupSum, which leaves the row's sum in every lane of the group.
//
// Arithmetic follows include/zcgvs/cuda/decode.cuh:22-42: the stored value is widened to float32
// (int8 values are multiplied by the matrix-wide scale first), dot/cosine accumulate q * x and L2
// accumulates (q - x)^2 and is negated at the end. Accumulation uses fused multiply-add in a
// different order than the sequential CPU loop, so float scores agree to rounding, not bitwise.
#pragma once

#include <hip/hip_fp16.h>

#include "common.hpp"

namespace zcgvs_hip {

constexpr int kQueryTile = 8;     // queries co-resident per pass (include/zcgvs/cuda/decode.cuh:20)
constexpr int kScanThreads = 256;  // 4 wavefronts

__host__ __device__ constexpr int elementsPerChunk(int dtype) {
    return dtype == ZCGVS_DTYPE_F32 ? 4 : dtype == ZCGVS_DTYPE_F16 ? 8 : 16;
}

template <int kDtype>
struct ChunkTraits;

template <>
struct ChunkTraits<ZCGVS_DTYPE_F32> {
    static constexpr int kElems = 4;
    __device__ static __forceinline__ void decode(const uint4& raw, float, float (&v)[4]) {
        v[0] = __uint_as_float(raw.x);
        v[1] = __uint_as_float(raw.y);
        v[2] = __uint_as_float(raw.z);
        v[3] = __uint_as_float(raw.w);
    }
};

template <>
struct ChunkTraits<ZCGVS_DTYPE_F16> {
    static constexpr int kElems = 8;
    __device__ static __forceinline__ void decode(const uint4& raw, float, float (&v)[8]) {
        const std::uint32_t words[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            __half_raw lo;
            __half_raw hi;
            lo.x = static_cast<unsigned short>(words[i] & 0xFFFFu);
            hi.x = static_cast<unsigned short>(words[i] >> 16);
            v[2 * i] = __half2float(__half(lo));
            v[2 * i + 1] = __half2float(__half(hi));
        }
    }
};

template <>
struct ChunkTraits<ZCGVS_DTYPE_I8> {
    static constexpr int kElems = 16;
    __device__ static __forceinline__ void decode(const uint4& raw, float scale, float (&v)[16]) {
        const std::uint32_t words[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int w = static_cast<int>(words[i]);
            v[4 * i + 0] = static_cast<float>((w << 24) >> 24) * scale;
            v[4 * i + 1] = static_cast<float>((w << 16) >> 24) * scale;
            v[4 * i + 2] = static_cast<float>((w << 8) >> 24) * scale;
            v[4 * i + 3] = static_cast<float>(w >> 24) * scale;
        }
    }
};

__device__ __forceinline__ uint4 loadChunk(const std::uint8_t* pointer) {
    return *reinterpret_cast<const uint4*>(pointer);
}

// Streaming load that does not keep the line in the caches (the corpus is read exactly once).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 loadChunkStreaming(const std::uint8_t* pointer) {
    const u32x4 raw = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(pointer));
    return make_uint4(raw.x, raw.y, raw.z, raw.w);
}

// Partner value for step `step` of groupSum: inside a row of 16 lanes the data-parallel
// primitives pair lane i with i ^ 1, i ^ 2 (quad permutes), 7 - i within each half-row and 15 - i
// within the row (mirrors); every pairing joins two groups that already hold their own sums, so
// after the step each lane holds the sum of the union. Across rows a swizzle (xor 16 inside 32
// lanes) and a permute (xor 32) follow.
template <int kStep>
__device__ __forceinline__ int groupPartner(int bits) {
    if constexpr (kStep == 0) {
        return __builtin_amdgcn_update_dpp(0, bits, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    } else if constexpr (kStep == 1) {
        return __builtin_amdgcn_update_dpp(0, bits, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    } else if constexpr (kStep == 2) {
        return __builtin_amdgcn_update_dpp(0, bits, 0x141, 0xF, 0xF, false);  // row_half_mirror
    } else if constexpr (kStep == 3) {
        return __builtin_amdgcn_update_dpp(0, bits, 0x140, 0xF, 0xF, false);  // row_mirror
    } else if constexpr (kStep == 4) {
        return __builtin_amdgcn_ds_swizzle(bits, 0x401F);  // xor 16 within 32 lanes
    } else {
        return __shfl_xor(bits, 32, kWave);
    }
}

template <typename T>
__device__ __forceinline__ int asBits(T value) {
    if constexpr (sizeof(T) == 4 && !__is_integral(T)) {
        return __float_as_int(value);
    } else {
        return static_cast<int>(value);
    }
}

template <typename T>
__device__ __forceinline__ T fromBits(int bits) {
    if constexpr (sizeof(T) == 4 && !__is_integral(T)) {
        return __int_as_float(bits);
    } else {
        return static_cast<T>(bits);
    }
}

// Sum over the L lanes of a group (L a power of two <= 64, groups aligned to L); every lane of
// the group gets the same total.
template <int L, typename T>
__device__ __forceinline__ T groupSum(T value) {
    static_assert(sizeof(T) == 4, "32-bit values");
    if constexpr (L >= 2) {
        value += fromBits<T>(groupPartner<0>(asBits(value)));
    }
    if constexpr (L >= 4) {
        value += fromBits<T>(groupPartner<1>(asBits(value)));
    }
    if constexpr (L >= 8) {
        value += fromBits<T>(groupPartner<2>(asBits(value)));
    }
    if constexpr (L >= 16) {
        value += fromBits<T>(groupPartner<3>(asBits(value)));
    }
    if constexpr (L >= 32) {
        value += fromBits<T>(groupPartner<4>(asBits(value)));
    }
    if constexpr (L >= 64) {
        value += fromBits<T>(groupPartner<5>(asBits(value)));
    }
    return value;
}

// Lanes per row for a row of `chunks` 16-byte chunks: the smallest power of two giving each
// lane at most `per_lane` chunks, capped at a full wavefront, and at least min_lanes (or as
// many as the row has chunks), so one load instruction reads whole cache lines of a row.
inline int lanesPerRow(int chunks, int per_lane = 4, int min_lanes = 1) {
    int lanes = 1;
    while (lanes < kWave && ((chunks + lanes - 1) / lanes > per_lane || (lanes < min_lanes && lanes < chunks))) {
        lanes <<= 1;
    }
    return lanes;
}

}  // namespace zcgvs_hip
