// Thin HIP runtime layer of the C ABI: errors, device queries, memory, streams, events, graphs.
// The C++17 host (Searcher, stores, Engine) reaches the GPU only through these functions and the
// launchers, in place of include/zcgvs/core/{cuda_check,cuda_context,device_buffer,
// pinned_buffer,cuda_stream}.hpp of the reference.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "common.hpp"

namespace zcgvs_hip {

namespace {
thread_local std::string t_last_error;
}

int setError(int status, const std::string& message) {
    t_last_error = message;
    return status;
}

int clearError() {
    t_last_error.clear();
    return ZCGVS_OK;
}

int hipFailure(hipError_t error, const char* what, const char* file, int line) {
    char buffer[512];
    std::snprintf(buffer, sizeof(buffer), "zcgvs HIP error %s (%s) at %s:%d: %s",
                  hipGetErrorName(error), hipGetErrorString(error), file, line, what);
    return setError(ZCGVS_ERR_HIP, buffer);
}

int deviceComputeUnits() {
    static std::mutex mutex;
    static std::vector<int> cache;
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) {
        return 256;
    }
    std::lock_guard<std::mutex> lock(mutex);
    if (static_cast<int>(cache.size()) <= device) {
        cache.resize(static_cast<std::size_t>(device) + 1, 0);
    }
    if (cache[static_cast<std::size_t>(device)] == 0) {
        int units = 0;
        if (hipDeviceGetAttribute(&units, hipDeviceAttributeMultiprocessorCount, device) !=
                hipSuccess ||
            units <= 0) {
            units = 256;
        }
        cache[static_cast<std::size_t>(device)] = units;
    }
    return cache[static_cast<std::size_t>(device)];
}

namespace {

__global__ void fillU32Kernel(std::uint32_t* __restrict__ dst, std::uint32_t value,
                              std::size_t count) {
    const std::size_t stride = static_cast<std::size_t>(gridDim.x) * blockDim.x;
    for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
         i < count; i += stride) {
        dst[i] = value;
    }
}

}  // namespace

}  // namespace zcgvs_hip

using namespace zcgvs_hip;

extern "C" {

const char* zcgvs_last_error(void) { return t_last_error.c_str(); }

const char* zcgvs_version(void) { return "zcgvs-hip 0.1.0 gfx950"; }

int zcgvs_device_count(int* count) {
    if (count == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: count must not be null");
    }
    ZCGVS_HIP_RETURN(hipGetDeviceCount(count));
    return clearError();
}

int zcgvs_set_device(int device) {
    ZCGVS_HIP_RETURN(hipSetDevice(device));
    return clearError();
}

int zcgvs_get_device(int* device) {
    if (device == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: device must not be null");
    }
    ZCGVS_HIP_RETURN(hipGetDevice(device));
    return clearError();
}

int zcgvs_device_query(int device, zcgvs_device_info* out) {
    if (out == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: info must not be null");
    }
    hipDeviceProp_t props;
    ZCGVS_HIP_RETURN(hipGetDeviceProperties(&props, device));
    std::memset(out, 0, sizeof(*out));
    std::snprintf(out->name, sizeof(out->name), "%s", props.name);
    std::snprintf(out->arch, sizeof(out->arch), "%s", props.gcnArchName);
    out->total_memory = props.totalGlobalMem;
    out->compute_units = props.multiProcessorCount;
    out->clock_khz = props.clockRate;
    out->memory_clock_khz = props.memoryClockRate;
    out->memory_bus_width = props.memoryBusWidth;
    out->l2_cache_bytes = props.l2CacheSize;
    out->major = props.major;
    out->minor = props.minor;
    out->peak_bandwidth_gbs =
        2.0 * static_cast<double>(props.memoryClockRate) * 1e3 *
        (static_cast<double>(props.memoryBusWidth) / 8.0) / 1e9;
    return clearError();
}

int zcgvs_device_synchronize(void) {
    ZCGVS_HIP_RETURN(hipDeviceSynchronize());
    return clearError();
}

int zcgvs_malloc(void** ptr, std::size_t bytes) {
    if (ptr == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: ptr must not be null");
    }
    *ptr = nullptr;
    if (bytes == 0) {
        return clearError();
    }
    ZCGVS_HIP_RETURN(hipMalloc(ptr, bytes));
    return clearError();
}

int zcgvs_free(void* ptr) {
    if (ptr != nullptr) {
        ZCGVS_HIP_RETURN(hipFree(ptr));
    }
    return clearError();
}

int zcgvs_host_alloc(void** ptr, std::size_t bytes) {
    if (ptr == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: ptr must not be null");
    }
    *ptr = nullptr;
    if (bytes == 0) {
        return clearError();
    }
    ZCGVS_HIP_RETURN(hipHostMalloc(ptr, bytes, hipHostMallocDefault));
    return clearError();
}

int zcgvs_host_free(void* ptr) {
    if (ptr != nullptr) {
        ZCGVS_HIP_RETURN(hipHostFree(ptr));
    }
    return clearError();
}

int zcgvs_memcpy_h2d(void* dst, const void* src, std::size_t bytes, zcgvs_stream_t stream) {
    if (bytes == 0) {
        return clearError();
    }
    ZCGVS_HIP_RETURN(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, toStream(stream)));
    return clearError();
}

int zcgvs_memcpy_d2h(void* dst, const void* src, std::size_t bytes, zcgvs_stream_t stream) {
    if (bytes == 0) {
        return clearError();
    }
    ZCGVS_HIP_RETURN(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, toStream(stream)));
    return clearError();
}

int zcgvs_memcpy_d2d(void* dst, const void* src, std::size_t bytes, zcgvs_stream_t stream) {
    if (bytes == 0) {
        return clearError();
    }
    ZCGVS_HIP_RETURN(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, toStream(stream)));
    return clearError();
}

int zcgvs_memset(void* dst, int value, std::size_t bytes, zcgvs_stream_t stream) {
    if (bytes == 0) {
        return clearError();
    }
    ZCGVS_HIP_RETURN(hipMemsetAsync(dst, value, bytes, toStream(stream)));
    return clearError();
}

int zcgvs_fill_u32(void* dst, std::uint32_t value, std::size_t count, zcgvs_stream_t stream) {
    if (count == 0) {
        return clearError();
    }
    if (dst == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: fill destination is null");
    }
    std::size_t blocks = (count + 255) / 256;
    if (blocks > 8192) {
        blocks = 8192;
    }
    fillU32Kernel<<<static_cast<unsigned>(blocks), 256, 0, toStream(stream)>>>(
        static_cast<std::uint32_t*>(dst), value, count);
    ZCGVS_LAUNCH_CHECK("fill");
    return clearError();
}

int zcgvs_stream_create(zcgvs_stream_t* stream) {
    if (stream == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: stream must not be null");
    }
    hipStream_t created = nullptr;
    // Default priority only: streams of different priorities are not used anywhere here.
    ZCGVS_HIP_RETURN(hipStreamCreateWithFlags(&created, hipStreamNonBlocking));
    *stream = created;
    return clearError();
}

int zcgvs_stream_destroy(zcgvs_stream_t stream) {
    if (stream != nullptr) {
        ZCGVS_HIP_RETURN(hipStreamDestroy(toStream(stream)));
    }
    return clearError();
}

int zcgvs_stream_synchronize(zcgvs_stream_t stream) {
    ZCGVS_HIP_RETURN(hipStreamSynchronize(toStream(stream)));
    return clearError();
}

int zcgvs_event_create(zcgvs_event_t* event) {
    if (event == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: event must not be null");
    }
    hipEvent_t created = nullptr;
    ZCGVS_HIP_RETURN(hipEventCreate(&created));
    *event = created;
    return clearError();
}

int zcgvs_event_destroy(zcgvs_event_t event) {
    if (event != nullptr) {
        ZCGVS_HIP_RETURN(hipEventDestroy(reinterpret_cast<hipEvent_t>(event)));
    }
    return clearError();
}

int zcgvs_event_record(zcgvs_event_t event, zcgvs_stream_t stream) {
    ZCGVS_HIP_RETURN(hipEventRecord(reinterpret_cast<hipEvent_t>(event), toStream(stream)));
    return clearError();
}

int zcgvs_event_synchronize(zcgvs_event_t event) {
    ZCGVS_HIP_RETURN(hipEventSynchronize(reinterpret_cast<hipEvent_t>(event)));
    return clearError();
}

int zcgvs_event_elapsed_ms(float* ms, zcgvs_event_t start, zcgvs_event_t end) {
    if (ms == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: ms must not be null");
    }
    ZCGVS_HIP_RETURN(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start),
                                         reinterpret_cast<hipEvent_t>(end)));
    return clearError();
}

int zcgvs_graph_begin_capture(zcgvs_stream_t stream) {
    if (stream == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT,
                        "zcgvs: graph capture needs a created (non-null) stream");
    }
    // the static scratch of zcgvs_search_topk_noalloc is looked up now, outside the capture
    const int status = prepareStaticScratch();
    if (status != ZCGVS_OK) {
        return status;
    }
    ZCGVS_HIP_RETURN(hipStreamBeginCapture(toStream(stream), hipStreamCaptureModeThreadLocal));
    return clearError();
}

int zcgvs_graph_end_capture(zcgvs_stream_t stream, zcgvs_graph_t* graph) {
    if (graph == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: graph must not be null");
    }
    *graph = nullptr;
    hipGraph_t captured = nullptr;
    ZCGVS_HIP_RETURN(hipStreamEndCapture(toStream(stream), &captured));
    hipGraphExec_t exec = nullptr;
    const hipError_t status = hipGraphInstantiate(&exec, captured, nullptr, nullptr, 0);
    (void)hipGraphDestroy(captured);
    ZCGVS_HIP_RETURN(status);
    *graph = exec;
    return clearError();
}

int zcgvs_graph_launch(zcgvs_graph_t graph, zcgvs_stream_t stream) {
    if (graph == nullptr) {
        return setError(ZCGVS_ERR_INVALID_ARGUMENT, "zcgvs: graph must not be null");
    }
    ZCGVS_HIP_RETURN(hipGraphLaunch(reinterpret_cast<hipGraphExec_t>(graph), toStream(stream)));
    return clearError();
}

int zcgvs_graph_destroy(zcgvs_graph_t graph) {
    if (graph != nullptr) {
        ZCGVS_HIP_RETURN(hipGraphExecDestroy(reinterpret_cast<hipGraphExec_t>(graph)));
    }
    return clearError();
}

}  // extern "C"
