// An owned, non-blocking HIP stream at the default priority (the role of
// include/zcgvs/core/cuda_stream.hpp), and the device selection/query helpers of
// src/core/cuda_context.cpp.
#pragma once

#include <cstddef>
#include <string>

#include "zcgvs/core/error.hpp"

namespace zcgvs {

class HipStream {
public:
    HipStream() { check(zcgvs_stream_create(&stream_)); }
    ~HipStream() {
        if (stream_ != nullptr) {
            zcgvs_stream_destroy(stream_);
        }
    }
    HipStream(const HipStream&) = delete;
    HipStream& operator=(const HipStream&) = delete;

    zcgvs_stream_t get() const { return stream_; }
    void synchronize() const { check(zcgvs_stream_synchronize(stream_)); }

private:
    zcgvs_stream_t stream_ = nullptr;
};

class HipEvent {
public:
    HipEvent() { check(zcgvs_event_create(&event_)); }
    ~HipEvent() {
        if (event_ != nullptr) {
            zcgvs_event_destroy(event_);
        }
    }
    HipEvent(const HipEvent&) = delete;
    HipEvent& operator=(const HipEvent&) = delete;

    zcgvs_event_t get() const { return event_; }
    void record(zcgvs_stream_t stream) const { check(zcgvs_event_record(event_, stream)); }
    void synchronize() const { check(zcgvs_event_synchronize(event_)); }
    // Milliseconds from `start` to this event (both recorded and complete).
    float elapsedSince(const HipEvent& start) const {
        float ms = 0.0f;
        check(zcgvs_event_elapsed_ms(&ms, start.event_, event_));
        return ms;
    }

private:
    zcgvs_event_t event_ = nullptr;
};

struct DeviceInfo {
    std::string name;
    std::string arch;
    std::size_t total_memory = 0;
    int compute_units = 0;
    int compute_major = 0;
    int compute_minor = 0;
    double peak_bandwidth_gbs = 0.0;
};

inline int deviceCount() {
    int count = 0;
    check(zcgvs_device_count(&count));
    return count;
}

inline void setDevice(int device) { check(zcgvs_set_device(device)); }

inline DeviceInfo queryDevice(int device) {
    zcgvs_device_info raw{};
    check(zcgvs_device_query(device, &raw));
    DeviceInfo info;
    info.name = raw.name;
    info.arch = raw.arch;
    info.total_memory = raw.total_memory;
    info.compute_units = raw.compute_units;
    info.compute_major = raw.major;
    info.compute_minor = raw.minor;
    info.peak_bandwidth_gbs = raw.peak_bandwidth_gbs;
    return info;
}

}  // namespace zcgvs
