// Index-side conversions (src/cuda/convert.cu:17-53, 55-93), the per-row int8 quantizer of the
// per-vector mode, and the on-device synthetic generator.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.hpp"
#include "rescore.hpp"

namespace zcgvs_hip {

namespace {

constexpr int kConvertThreads = 256;
constexpr std::size_t kMaxConvertBlocks = 65535;

unsigned convertBlocks(std::size_t count) {
    return static_cast<unsigned>(
        std::max<std::size_t>(1, std::min(kMaxConvertBlocks, (count + kConvertThreads - 1) / kConvertThreads)));
}

__global__ void convertF32ToF16Kernel(const float* __restrict__ src, __half* __restrict__ dst,
                                      std::size_t count) {
    const std::size_t stride = static_cast<std::size_t>(gridDim.x) * blockDim.x;
    for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
         i < count; i += stride) {
        dst[i] = __float2half_rn(src[i]);
    }
}

// q = clamp(rint(x * inverse_scale), -127, 127): round half to even, like nearbyint in
// tests/cpp/cpu_reference.hpp:51-62.
__device__ __forceinline__ std::int8_t quantize(float x, float inverse_scale) {
    const float scaled = rintf(x * inverse_scale);
    return static_cast<std::int8_t>(fminf(fmaxf(scaled, -127.0f), 127.0f));
}

__global__ void convertF32ToI8Kernel(const float* __restrict__ src, std::int8_t* __restrict__ dst,
                                     std::size_t count, float inverse_scale) {
    const std::size_t stride = static_cast<std::size_t>(gridDim.x) * blockDim.x;
    for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
         i < count; i += stride) {
        dst[i] = quantize(src[i], inverse_scale);
    }
}

// Word w of a row: bit b set iff x[32w + b] >= 0 (so -0.0 sets it and NaN does not); dimensions
// past dim stay zero.
__global__ void packBinaryKernel(const float* __restrict__ src, std::uint32_t* __restrict__ dst,
                                 int rows, int dim, int words) {
    const std::size_t total = static_cast<std::size_t>(rows) * words;
    const std::size_t stride = static_cast<std::size_t>(gridDim.x) * blockDim.x;
    for (std::size_t index = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
         index < total; index += stride) {
        const std::size_t row = index / static_cast<std::size_t>(words);
        const int word = static_cast<int>(index - row * static_cast<std::size_t>(words));
        const float* values = src + row * static_cast<std::size_t>(dim);
        std::uint32_t bits = 0u;
        const int base = word * 32;
        const int limit = min(32, dim - base);
        for (int b = 0; b < limit; ++b) {
            if (values[base + b] >= 0.0f) {
                bits |= 1u << b;
            }
        }
        dst[index] = bits;
    }
}

// One wavefront per row: s = max|x| / 127 (1 for an all-zero row), then the quantizer above with
// the reciprocal 1/s.
__global__ __launch_bounds__(256) void quantizeRowsKernel(const float* __restrict__ src, int rows,
                                                          int dim, std::int8_t* __restrict__ dst,
                                                          float* __restrict__ scales) {
    const int lane = threadIdx.x & (kWave - 1);
    const long long row = static_cast<long long>(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
    if (row >= rows) {
        return;
    }
    const float* values = src + static_cast<std::size_t>(row) * dim;
    float peak = 0.0f;
    for (int j = lane; j < dim; j += kWave) {
        peak = fmaxf(peak, fabsf(values[j]));
    }
#pragma unroll
    for (int offset = kWave / 2; offset > 0; offset >>= 1) {
        peak = fmaxf(peak, waveXor(peak, offset));
    }
    const float scale = peak > 0.0f ? peak / 127.0f : 1.0f;
    const float inverse = 1.0f / scale;
    std::int8_t* out = dst + static_cast<std::size_t>(row) * dim;
    for (int j = lane; j < dim; j += kWave) {
        out[j] = quantize(values[j], inverse);
    }
    if (lane == 0) {
        scales[row] = scale;
    }
}

// ---- synthetic data ------------------------------------------------------------------------
__device__ __forceinline__ std::uint64_t splitmix64(std::uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// Uniform double in (0, 1) from the top 53 bits.
__device__ __forceinline__ double unitOpen(std::uint64_t bits) {
    return (static_cast<double>(bits >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}

// One wavefront per row: element pair p of row r comes from splitmix64 of
// (seed, r, p); Box-Muller in double; rounded to float; the row is divided by its float32 norm
// (squares summed by the wavefront's tree reduction).
__global__ __launch_bounds__(256) void generateKernel(float* __restrict__ out, long long rows,
                                                      int dim, std::uint64_t seed,
                                                      long long row_offset) {
    const int lane = threadIdx.x & (kWave - 1);
    const long long local = static_cast<long long>(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
    if (local >= rows) {
        return;
    }
    const std::uint64_t row = static_cast<std::uint64_t>(local + row_offset);
    const std::uint64_t row_seed = splitmix64(seed ^ splitmix64(row));
    float* values = out + static_cast<std::size_t>(local) * dim;
    const int pairs = (dim + 1) / 2;
    float sum = 0.0f;
    for (int p = lane; p < pairs; p += kWave) {
        const std::uint64_t a = splitmix64(row_seed + 2ull * static_cast<std::uint64_t>(p));
        const std::uint64_t b = splitmix64(row_seed + 2ull * static_cast<std::uint64_t>(p) + 1ull);
        const double radius = sqrt(-2.0 * log(unitOpen(a)));
        const double angle = 6.283185307179586 * unitOpen(b);
        const float x0 = static_cast<float>(radius * cos(angle));
        const float x1 = static_cast<float>(radius * sin(angle));
        values[2 * p] = x0;
        sum = fmaf(x0, x0, sum);
        if (2 * p + 1 < dim) {
            values[2 * p + 1] = x1;
            sum = fmaf(x1, x1, sum);
        }
    }
#pragma unroll
    for (int offset = kWave / 2; offset > 0; offset >>= 1) {
        sum += waveXor(sum, offset);
    }
    const float norm = sqrtf(sum);
    if (norm > 0.0f) {
        for (int j = lane; j < dim; j += kWave) {
            values[j] = values[j] / norm;
        }
    }
}

}  // namespace

int launchQuantizeRows(const float* src, int rows, int dim, std::int8_t* dst, float* scales,
                       hipStream_t stream) {
    const unsigned blocks = static_cast<unsigned>((rows + 3) / 4);
    quantizeRowsKernel<<<blocks, 256, 0, stream>>>(src, rows, dim, dst, scales);
    ZCGVS_LAUNCH_CHECK("quantize rows");
    return ZCGVS_OK;
}

}  // namespace zcgvs_hip

using namespace zcgvs_hip;

extern "C" {

int zcgvs_launch_convert_f32_to_f16(const float* d_src, void* d_dst_half, std::size_t count,
                                    zcgvs_stream_t stream) {
    if (count == 0) {
        return clearError();
    }
    if (d_src == nullptr || d_dst_half == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs convert: null device pointer");
    }
    convertF32ToF16Kernel<<<convertBlocks(count), kConvertThreads, 0, toStream(stream)>>>(
        d_src, static_cast<__half*>(d_dst_half), count);
    ZCGVS_LAUNCH_CHECK("convert f16");
    return clearError();
}

int zcgvs_launch_convert_f32_to_i8(const float* d_src, void* d_dst_int8, std::size_t count,
                                   float scale, zcgvs_stream_t stream) {
    if (count == 0) {
        return clearError();
    }
    if (d_src == nullptr || d_dst_int8 == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs convert: null device pointer");
    }
    const float inverse_scale = (scale > 0.0f) ? (1.0f / scale) : 0.0f;
    convertF32ToI8Kernel<<<convertBlocks(count), kConvertThreads, 0, toStream(stream)>>>(
        d_src, static_cast<std::int8_t*>(d_dst_int8), count, inverse_scale);
    ZCGVS_LAUNCH_CHECK("convert i8");
    return clearError();
}

int zcgvs_launch_pack_binary(const float* d_src, void* d_dst_words, int rows, int dim,
                             zcgvs_stream_t stream) {
    if (rows <= 0 || dim <= 0) {
        return clearError();
    }
    if (d_src == nullptr || d_dst_words == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs pack: null device pointer");
    }
    const int words = static_cast<int>(binaryWords(dim));
    packBinaryKernel<<<convertBlocks(static_cast<std::size_t>(rows) * words), kConvertThreads, 0,
                       toStream(stream)>>>(d_src, static_cast<std::uint32_t*>(d_dst_words), rows,
                                           dim, words);
    ZCGVS_LAUNCH_CHECK("pack binary");
    return clearError();
}

int zcgvs_launch_quantize_rows_i8(const float* d_src, int rows, int dim, std::int8_t* d_dst,
                                  float* d_scales, zcgvs_stream_t stream) {
    if (rows <= 0 || dim <= 0) {
        return clearError();
    }
    if (d_src == nullptr || d_dst == nullptr || d_scales == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs quantize: null device pointer");
    }
    const int status = launchQuantizeRows(d_src, rows, dim, d_dst, d_scales, toStream(stream));
    return status == ZCGVS_OK ? clearError() : status;
}

int zcgvs_generate_normalized(float* d_out, std::int64_t rows, int dim, std::uint64_t seed,
                              std::int64_t row_offset, zcgvs_stream_t stream) {
    if (rows <= 0 || dim <= 0) {
        return clearError();
    }
    if (d_out == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs generate: null device pointer");
    }
    const long long blocks = (rows + 3) / 4;
    if (blocks > 0x7FFFFFFFLL) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs generate: too many rows per call");
    }
    generateKernel<<<static_cast<unsigned>(blocks), 256, 0, toStream(stream)>>>(
        d_out, rows, dim, seed, row_offset);
    ZCGVS_LAUNCH_CHECK("generate");
    return clearError();
}

}  // extern "C"
