// Measured HBM rates of the device (zcgvs_measure_hbm_bandwidth): the achievable counterpart of
// the nominal peak the reference derives from the memory clock and bus width
// (include/zcgvs/core/cuda_context.hpp:20-23) and prints every scan's GB/s against
// (apps/bench_kernels.cu:133-143).
//
// Two streaming kernels over buffers far larger than the last-level cache: a read that folds
// every 16-byte chunk into a per-thread xor (one word per workgroup is written, so the loads
// cannot be dropped) and a copy. Both use nontemporal 16-byte accesses, eight in flight per
// thread per iteration, in two access orders (each workgroup reading contiguous 32 KiB spans,
// or each thread's loads spread over the grid); each order is launched at a few grid sizes and
// the best timed launch counts.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.hpp"

namespace zcgvs_hip {

namespace {

typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));

constexpr int kProbeThreads = 256;
constexpr int kProbeUnroll = 8;

// Chunk index of load u of this thread in span `span`: with kBlocked, a workgroup's kProbeUnroll
// loads cover one contiguous span of kProbeUnroll * kProbeThreads chunks (each wavefront reads
// 1 KiB runs of one 32 KiB span); otherwise the loads of one thread stride the whole grid apart.
template <bool kBlocked>
__device__ inline std::size_t probeIndex(std::size_t span, int u) {
    if (kBlocked) {
        return (span * gridDim.x + blockIdx.x) * (kProbeUnroll * kProbeThreads) +
               static_cast<std::size_t>(u) * kProbeThreads + threadIdx.x;
    }
    return span * (static_cast<std::size_t>(gridDim.x) * kProbeThreads * kProbeUnroll) +
           static_cast<std::size_t>(u) * gridDim.x * kProbeThreads +
           static_cast<std::size_t>(blockIdx.x) * kProbeThreads + threadIdx.x;
}

template <bool kBlocked>
__global__ __launch_bounds__(kProbeThreads) void probeReadKernel(const u32x4v* __restrict__ src,
                                                                 std::size_t chunks,
                                                                 std::uint32_t* __restrict__ sink) {
    // every span is whole: the grid reads spans [0, spans) of kProbeUnroll * grid threads chunks
    const std::size_t per_span = static_cast<std::size_t>(gridDim.x) * kProbeThreads * kProbeUnroll;
    const std::size_t spans = chunks / per_span;
    u32x4v acc = {0u, 0u, 0u, 0u};
    for (std::size_t span = 0; span < spans; ++span) {
        u32x4v v[kProbeUnroll];
#pragma unroll
        for (int u = 0; u < kProbeUnroll; ++u) {
            v[u] = __builtin_nontemporal_load(src + probeIndex<kBlocked>(span, u));
        }
#pragma unroll
        for (int u = 0; u < kProbeUnroll; ++u) {
            acc ^= v[u];
        }
    }
    for (std::size_t i = spans * per_span + static_cast<std::size_t>(blockIdx.x) * kProbeThreads + threadIdx.x;
         i < chunks; i += static_cast<std::size_t>(gridDim.x) * kProbeThreads) {
        acc ^= __builtin_nontemporal_load(src + i);
    }
    std::uint32_t word = acc.x ^ acc.y ^ acc.z ^ acc.w;
#pragma unroll
    for (int offset = kWave / 2; offset > 0; offset >>= 1) {
        word ^= waveXor(word, offset);
    }
    __shared__ std::uint32_t partial[kProbeThreads / kWave];
    if ((threadIdx.x & (kWave - 1)) == 0) {
        partial[threadIdx.x / kWave] = word;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        std::uint32_t all = 0u;
        for (int w = 0; w < kProbeThreads / kWave; ++w) {
            all ^= partial[w];
        }
        sink[blockIdx.x] = all;
    }
}

template <bool kBlocked>
__global__ __launch_bounds__(kProbeThreads) void probeCopyKernel(const u32x4v* __restrict__ src,
                                                                 u32x4v* __restrict__ dst,
                                                                 std::size_t chunks) {
    const std::size_t per_span = static_cast<std::size_t>(gridDim.x) * kProbeThreads * kProbeUnroll;
    const std::size_t spans = chunks / per_span;
    for (std::size_t span = 0; span < spans; ++span) {
        u32x4v v[kProbeUnroll];
#pragma unroll
        for (int u = 0; u < kProbeUnroll; ++u) {
            v[u] = __builtin_nontemporal_load(src + probeIndex<kBlocked>(span, u));
        }
#pragma unroll
        for (int u = 0; u < kProbeUnroll; ++u) {
            __builtin_nontemporal_store(v[u], dst + probeIndex<kBlocked>(span, u));
        }
    }
    for (std::size_t i = spans * per_span + static_cast<std::size_t>(blockIdx.x) * kProbeThreads + threadIdx.x;
         i < chunks; i += static_cast<std::size_t>(gridDim.x) * kProbeThreads) {
        __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
    }
}

__global__ void probeFillKernel(u32x4v* __restrict__ dst, std::size_t chunks) {
    const std::size_t stride = static_cast<std::size_t>(gridDim.x) * blockDim.x;
    for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < chunks;
         i += stride) {
        const std::uint32_t x = static_cast<std::uint32_t>(i) * 2654435761u;
        dst[i] = u32x4v{x, x ^ 1u, x ^ 2u, x ^ 3u};
    }
}

// Frees the probe's buffers and events on every exit path.
struct ProbeResources {
    void* src = nullptr;
    void* dst = nullptr;
    void* sink = nullptr;
    hipStream_t stream = nullptr;
    hipEvent_t begin = nullptr;
    hipEvent_t end = nullptr;
    ~ProbeResources() {
        if (stream != nullptr) {
            (void)hipStreamSynchronize(stream);
        }
        if (begin != nullptr) (void)hipEventDestroy(begin);
        if (end != nullptr) (void)hipEventDestroy(end);
        if (stream != nullptr) (void)hipStreamDestroy(stream);
        if (src != nullptr) (void)hipFree(src);
        if (dst != nullptr) (void)hipFree(dst);
        if (sink != nullptr) (void)hipFree(sink);
    }
};

}  // namespace

}  // namespace zcgvs_hip

using namespace zcgvs_hip;

extern "C" {

int zcgvs_measure_hbm_bandwidth(std::size_t bytes, int iterations, double* read_gbs, double* copy_gbs) {
    if (read_gbs == nullptr || copy_gbs == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: bandwidth outputs must not be null");
    }
    if (bytes < (64u << 20) || iterations <= 0) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT,
                        "zcgvs: the bandwidth probe needs at least 64 MiB and one iteration");
    }
    *read_gbs = 0.0;
    *copy_gbs = 0.0;
    const std::size_t chunks = bytes / 16;
    const std::size_t used = chunks * 16;
    const int units = deviceComputeUnits();
    const int grids[3] = {4 * units, 8 * units, 16 * units};
    ProbeResources r;
    ZCGVS_HIP_RETURN(hipMalloc(&r.src, used));
    ZCGVS_HIP_RETURN(hipMalloc(&r.dst, used));
    ZCGVS_HIP_RETURN(hipMalloc(&r.sink, static_cast<std::size_t>(16 * units) * sizeof(std::uint32_t)));
    ZCGVS_HIP_RETURN(hipStreamCreateWithFlags(&r.stream, hipStreamNonBlocking));
    ZCGVS_HIP_RETURN(hipEventCreate(&r.begin));
    ZCGVS_HIP_RETURN(hipEventCreate(&r.end));
    auto* src = static_cast<u32x4v*>(r.src);
    auto* dst = static_cast<u32x4v*>(r.dst);
    probeFillKernel<<<4 * units, 256, 0, r.stream>>>(src, chunks);
    ZCGVS_LAUNCH_CHECK("probe fill");
    probeFillKernel<<<4 * units, 256, 0, r.stream>>>(dst, chunks);
    ZCGVS_LAUNCH_CHECK("probe fill");
    double best_read = 0.0;
    double best_copy = 0.0;
    // one timed launch of `launch` per iteration after a warm-up; the best rate counts
    auto timeBest = [&](auto&& launch, double bytes_moved, double* best) -> int {
        for (int it = 0; it <= iterations; ++it) {  // the first launch of each shape is a warm-up
            ZCGVS_HIP_RETURN(hipEventRecord(r.begin, r.stream));
            launch();
            ZCGVS_LAUNCH_CHECK("bandwidth probe");
            ZCGVS_HIP_RETURN(hipEventRecord(r.end, r.stream));
            ZCGVS_HIP_RETURN(hipEventSynchronize(r.end));
            float ms = 0.0f;
            ZCGVS_HIP_RETURN(hipEventElapsedTime(&ms, r.begin, r.end));
            if (it > 0 && ms > 0.0f) {
                *best = std::max(*best, bytes_moved / (ms * 1e-3) / 1e9);
            }
        }
        return ZCGVS_OK;
    };
    auto* sink = static_cast<std::uint32_t*>(r.sink);
    const double once = static_cast<double>(used);
    for (int g : grids) {
        int status = timeBest([&] { probeReadKernel<false><<<g, kProbeThreads, 0, r.stream>>>(src, chunks, sink); },
                              once, &best_read);
        if (status == ZCGVS_OK) {
            status = timeBest([&] { probeReadKernel<true><<<g, kProbeThreads, 0, r.stream>>>(src, chunks, sink); },
                              once, &best_read);
        }
        if (status == ZCGVS_OK) {
            status = timeBest([&] { probeCopyKernel<false><<<g, kProbeThreads, 0, r.stream>>>(src, dst, chunks); },
                              2.0 * once, &best_copy);
        }
        if (status == ZCGVS_OK) {
            status = timeBest([&] { probeCopyKernel<true><<<g, kProbeThreads, 0, r.stream>>>(src, dst, chunks); },
                              2.0 * once, &best_copy);
        }
        if (status != ZCGVS_OK) {
            return status;
        }
    }
    *read_gbs = best_read;
    *copy_gbs = best_copy;
    return clearError();
}

}  // extern "C"
